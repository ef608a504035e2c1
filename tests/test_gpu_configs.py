"""GPU parity at the full shapes of the benchmark configurations.

The bench runs exactly these paths (C1: a batch-32 Prefill into the cache and the cost-balanced split;
C3: 64 ragged prompts drawn on the device, stored by Prefill.store_only, uniform runs of 28 tiles
with two waves per workgroup and the golden-ratio scatter; C2: the 4 x 8192-token attention launch with
an exact head; C4: the 28-layer Qwen2-7B architecture through TriAttention).  Each test holds the GPU
to the oracle on the same bits: the sequences or rows it checks are copied to the host.

Bar: attention outputs (fp32) within 2e-3 max-abs and 1e-3 mean-abs of the oracle; bf16 outputs (C4)
may also carry half a bf16 ulp; exact (bf16) heads against float64 attention with a max-abs bar of
2e-3 or fp32 attention's own error on the same rows, whichever is larger.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, assert_close_bf16, compare_codes, run_prefill, sample_tokens
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import Prefill
from triattention_amd.maps import from_bands
from triattention_amd.synthetic import bits

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def exact_rows(q, k, v, rows, scale):
    """Causal attention of query rows ``rows`` of q [Hq,T,128] over k, v [Hk,T,128] (bf16, CPU), in float64
    and in float32: ([n,128], [n,128]) for rows given as (q-head, token)."""
    g = q.shape[0] // k.shape[0]
    out64, out32 = [], []
    for h, i in rows:
        for dt, out in ((torch.float64, out64), (torch.float32, out32)):
            qi = q[h, i].to(dt)
            kk, vv = k[h // g, :i + 1].to(dt), v[h // g, :i + 1].to(dt)
            w = torch.softmax((kk @ qi) * scale, dim=0)
            out.append((w @ vv).numpy())
    return np.stack(out64), np.stack(out32)


def decode_exact_rows(qd, keys, values, heads, scale):
    """One-token attention of q-heads ``heads`` of qd [Hq,128] over keys / values [Hk,L,128] in float64 and
    float32."""
    g = qd.shape[0] // keys.shape[0]
    res = []
    for dt in (torch.float64, torch.float32):
        rows = []
        for h in heads:
            w = torch.softmax((keys[h // g].to(dt) @ qd[h].to(dt)) * scale, dim=0)
            rows.append((w @ values[h // g].to(dt)).numpy())
        res.append(np.stack(rows))
    return res


def test_config1_full_decode(module):
    """C1 (B32, Hq 24 / Hk 8, prompt 4096, 25% INT8 / 75% INT4): the batch-32 Prefill fills the cache, the
    cost-balanced partition splits it, and 8 sequences at steps 0 and 1 match the oracle."""
    print("\n[parity] C1 full: B32 Hq24/Hk8 prompt 4096 (host draw)", flush=True)
    c1 = S.config1()
    assert "i8" in c1["kinds"] and "i4" in c1["kinds"]
    dev = torch.device("cuda")
    batch, hq, hk, prompt = 32, 24, 8, c1["prompt"]
    q = torch.cat([s["q"] for s in c1["seqs"]]).to(dev)
    k = torch.cat([s["k"] for s in c1["seqs"]]).to(dev)
    v = torch.cat([s["v"] for s in c1["seqs"]]).to(dev)
    bands = c1["bands"]
    cache = DecodeCache(module, max_tail=256)
    cache.out_dtype = torch.float32
    Prefill(module, from_bands({"0": bands.tolist()}), cache)(0, q, k, v, SCALE)
    torch.cuda.synchronize()
    del q, k, v
    e = cache.layers[0]
    assert e["bounds"] is not None, "C1 takes the cost-balanced partition"
    check = [0, 4, 9, 13, 18, 22, 27, 31]
    codes = {b: O.prefill_codes(None, bits(c1["seqs"][b]["k"][0]), bits(c1["seqs"][b]["v"][0]), bands.numpy(),
                                decode_cache=True) for b in check}
    ktail = np.zeros((batch, hk, 256, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    g = S.gen(4243)
    for step in range(2):
        if step == 0:
            qd, kd, vd = c1["q"], c1["k"], c1["v"]
        else:
            qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
        print(f"[parity] C1 step {step}", flush=True)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), SCALE).cpu().numpy()
        for b in check:
            ref = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), SCALE, ktail[b],
                           vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"C1 step {step} sequence {b}")
        ktail[:, :, step] = bits(kd[:, :, 0])
        vtail[:, :, step] = bits(vd[:, :, 0])
        cache.advance()


def test_config3_full_ragged_decode(module):
    """C3 (64 ragged prompts, log-uniform in [512, 32768], Hq 32 / Hk 8): the bench's device draw and
    store_only path, uniform runs of 28 tiles, two waves per workgroup; the shortest, the longest and three
    middle sequences match the oracle at steps 0 and 1."""
    lengths = S.config3_lengths()
    kinds, bands = S.config3_map()
    hq, hk, batch = 32, 8, len(lengths)
    print(f"\n[parity] C3 full: {batch} ragged prompts, {sum(lengths)} tokens (device draw)", flush=True)
    dev = torch.device("cuda")
    gdev = torch.Generator(device=dev).manual_seed(1003)
    cache = DecodeCache(module, max_tail=256)
    cache.ragged = True
    cache.out_dtype = torch.float32
    pre = Prefill(module, from_bands({"0": bands.tolist()}), cache)
    by_len = sorted(range(batch), key=lambda b: lengths[b])
    check = sorted({by_len[0], by_len[-1], by_len[16], by_len[32], by_len[48]})
    host = {}
    for b, n in enumerate(lengths):
        k = S.outlier_tensor_device(gdev, 1, hk, n)
        v = S.outlier_tensor_device(gdev, 1, hk, n)
        pre.store_only(0, k, v, hq)
        if b in check:
            host[b] = (k[0].cpu(), v[0].cpu())
    torch.cuda.synchronize()
    e = cache.layers[0]
    assert e["bounds"] is None and e["per"] == 28, (e["per"], "C3 runs uniform splits of 28 tiles")
    listed = DecodeCache._task_items(e).size
    assert 4 * module.device_cus() < listed <= 8 * module.device_cus(), \
        "C3: more splits than one resident wave per SIMD, in one-wave workgroups"
    codes = {b: O.prefill_codes(None, bits(host[b][0]), bits(host[b][1]), bands.numpy(), decode_cache=True)
             for b in check}
    ktail = np.zeros((batch, hk, 256, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    for step in range(2):
        qd, kd, vd = (S.outlier_tensor_device(gdev, batch, hq, 1), S.outlier_tensor_device(gdev, batch, hk, 1),
                      S.outlier_tensor_device(gdev, batch, hk, 1))
        print(f"[parity] C3 step {step}", flush=True)
        out = cache(0, qd, kd, vd, SCALE).cpu().numpy()
        qd, kd, vd = qd.cpu(), kd.cpu(), vd.cpu()
        for b in check:
            ref = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), lengths[b], cache.split_of(0, b), SCALE,
                           ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"C3 step {step} sequence {b} (prompt {lengths[b]})")
        ktail[:, :, step] = bits(kd[:, :, 0])
        vtail[:, :, step] = bits(vd[:, :, 0])
        cache.advance()


def test_ragged_decode_shared_prefill_equal_tile_counts(module):
    """One Prefill executor feeds a ragged cache with prompts whose tile counts repeat (100 / 110 / 64 /
    120 tokens: 2, 2, 1 and 2 tiles).  The executor reuses its scale and statistics buffers for equal
    shapes; every sequence must still decode with its own."""
    print("\n[parity] ragged decode, one Prefill, prompts 100/110/64/120", flush=True)
    hq, hk, max_tail = 8, 2, 4
    from triattention_amd.synthetic import INF
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                         dtype=torch.int32)
    cache = DecodeCache(module, max_tail=max_tail)
    cache.ragged = True
    cache.out_dtype = torch.float32
    pre = Prefill(module, from_bands({"0": bands.tolist()}), cache, out_dtype=torch.float32)
    prompts = [100, 110, 64, 120]
    dev = torch.device("cuda")
    codes = []
    for i, n in enumerate(prompts):
        g = S.gen(8200 + i)
        q, k, v = S.outlier_tensor(g, 1, hq, n), S.outlier_tensor(g, 1, hk, n), S.outlier_tensor(g, 1, hk, n)
        pre(0, q.to(dev), k.to(dev), v.to(dev), SCALE)
        codes.append(O.prefill_codes(None, bits(k[0]), bits(v[0]), bands.numpy(), decode_cache=True))
    g = S.gen(8300)
    ktail = np.zeros((len(prompts), hk, max_tail, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    for step in range(2):
        qd, kd, vd = (S.outlier_tensor(g, len(prompts), hq, 1), S.outlier_tensor(g, len(prompts), hk, 1),
                      S.outlier_tensor(g, len(prompts), hk, 1))
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), SCALE).cpu().numpy()
        for b, n in enumerate(prompts):
            ref = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), n, cache.split_of(0, b), SCALE, ktail[b],
                           vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"step {step} sequence {b} (prompt {n})")
            ktail[b, :, step] = bits(kd[b, :, 0])
            vtail[b, :, step] = bits(vd[b, :, 0])
        cache.advance()


def test_config2_full_sampled_rows(module):
    """C2 (B4, Hq 28 / Hk 4, T 8192, log-uniform channel scales, KV heads INT8 / INT4 / bf16): every code,
    scale and record of every sequence bit-exact; sampled rows of every q-head (first and last tiles, the
    middle, random) against the oracle (quantized heads) or float64 attention (the exact head)."""
    print("\n[parity] C2 full: B4 Hq28/Hk4 T8192 (host draw)", flush=True)
    c = S.config2()
    kinds = c["kinds"]
    assert "i8" in kinds and "i4" in kinds and "bf16" in kinds, kinds
    batch, hq, hk, t = 4, 28, 4, 8192
    bf16_kv = [h for h, kind in enumerate(kinds) if kind == "bf16"]
    out, ops, _ = run_prefill(module, c["q"], c["k"], c["v"], c["bands"], c["scale"], bf16_kv=bf16_kv)
    out = out.numpy()
    g = hq // hk
    rng = np.random.default_rng(1202)
    for b in range(batch):
        print(f"[parity] C2 sequence {b}: codes and sampled rows", flush=True)
        codes = O.prefill_codes(bits(c["q"][b]), bits(c["k"][b]), bits(c["v"][b]), c["bands"].numpy())
        compare_codes(ops, codes, b, batch, hq, hk, t)
        rows = [(h, i) for h in range(hq) for i in sample_tokens(t, rng)]
        quant = [(h, i) for h, i in rows if h // g not in bf16_kv]
        exact = [(h, i) for h, i in rows if h // g in bf16_kv]
        ref, tol = O.prefill_rows(codes, c["bands"].numpy(), hq, hk, t, c["scale"], [h * t + i for h, i in quant],
                                  tol=True)
        got = np.stack([out[b, h, i] for h, i in quant])
        assert_close(got, ref, what=f"C2 sequence {b} quantized heads ({len(quant)} rows)", tol=tol)
        r64, r32 = exact_rows(c["q"][b], c["k"][b], c["v"][b], exact, c["scale"])
        bar = max(2e-3, float(np.abs(r32 - r64).max()))
        got = np.stack([out[b, h, i] for h, i in exact])
        assert_close(got, r64, max_abs=bar, what=f"C2 sequence {b} exact heads ({len(exact)} rows)")


class _Recorder:
    """Forwards to a Prefill / DecodeCache and keeps the inputs and output of one layer's calls."""

    def __init__(self, inner, layer):
        self.inner, self.layer, self.calls = inner, layer, []

    def __getattr__(self, name):
        return getattr(self.inner, name)

    def __call__(self, layer, q, k, v, scale):
        out = self.inner(layer, q, k, v, scale)
        if layer == self.layer:
            self.calls.append((q.cpu(), k.cpu(), v.cpu(), out.float().cpu(), scale))
        return out


def test_config4_full_shape_generation(module):
    """C4 (random-init Qwen2-7B architecture: 28 layers, hidden 3584, Hq 28 / Hk 4, FFN 18944, vocab 152064,
    4096-token prompt, per-(layer, KV head) INT8 / INT4 / bf16 map): three greedy tokens through
    TriAttention.  Properties: finite logits, every layer stored, each cache head's kept-tile count as its
    map gives it.  Parity: one layer holding all three head kinds, its prompt call (sampled rows) and
    its first two decode calls, against the oracle (quantized heads) and float64 attention (exact heads)."""
    transformers = pytest.importorskip("transformers")
    from triattention_amd.models import TriAttention
    kw, ids, bands, bf16, kinds = S.config4()
    layer = next(l for l in range(28) if set(kinds[l].tolist()) == {0, 1, 2})
    print(f"\n[parity] C4 full shape: 28-layer Qwen2-7B random init, prompt 4096, checked layer {layer}", flush=True)
    dev = torch.device("cuda")
    torch.manual_seed(1004)
    with torch.device(dev):
        model = transformers.Qwen2ForCausalLM(transformers.Qwen2Config(**kw)).to(torch.bfloat16).eval()
    tri = TriAttention(model, from_bands(bands, model, bf16=bf16), max_new_tokens=4, module=module)
    tri.prefill = _Recorder(tri.prefill, layer)
    tri.decode_cache = _Recorder(tri.decode_cache, layer)
    steps = 3
    with torch.inference_mode():
        tokens = tri.generate(ids.to(dev), steps, eos=set())
    torch.cuda.synchronize()
    assert len(tokens) == steps and all(0 <= t < 152064 for t in tokens)
    cache = tri.decode_cache.inner
    assert all(cache.stored(l) for l in range(28))
    t = ids.shape[1]
    tiles = (t + 63) // 64
    for l in (0, layer, 27):
        # INT8 (INF, INF), INT4 (1, INF) and bf16 KV heads all keep every prompt tile; INT4 heads hold 4-bit
        # keys on all tiles but the sink and the last
        e = cache.layers[l]
        assert (e["count"].cpu() == tiles).all(), (l, e["count"].cpu().tolist())
        is4 = ((e["kinfo"].cpu()[0, :, :tiles] >> 8) & 1).sum(1).tolist()
        assert is4 == [tiles - 2 if int(kinds[l, h]) == 1 else 0 for h in range(4)], (l, is4)
    (q, k, v, out, scale), = tri.prefill.calls
    b = np.asarray(bands[str(layer)], np.int32)
    exact_kv = bf16[str(layer)]
    g = 7
    rng = np.random.default_rng(1404)
    rows = [(h, i) for h in range(28) for i in sample_tokens(t, rng, extra=2)]
    quant = [(h, i) for h, i in rows if h // g not in exact_kv]
    exact = [(h, i) for h, i in rows if h // g in exact_kv]
    codes = O.prefill_codes(bits(q[0]), bits(k[0]), bits(v[0]), b, decode_cache=True)
    ref, tol = O.prefill_rows(codes, b, 28, 4, t, scale, [h * t + i for h, i in quant], tol=True)
    assert_close_bf16(np.stack([out[0, h, i].numpy() for h, i in quant]), ref, what=f"C4 layer {layer} prefill",
                      tol=tol)
    r64, r32 = exact_rows(q[0], k[0], v[0], exact, scale)
    bar = max(2e-3, float(np.abs(r32 - r64).max()))
    assert_close_bf16(np.stack([out[0, h, i].numpy() for h, i in exact]), r64, max_abs=bar,
                      what=f"C4 layer {layer} prefill exact heads")
    quant_q = [h for h in range(28) if h // g not in exact_kv]
    exact_q = [h for h in range(28) if h // g in exact_kv]
    ktail = np.zeros((4, 4, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    keys, values = k[0].clone(), v[0].clone()
    split = cache.split_of(layer, 0)
    for step, (qd, kd, vd, od, _) in enumerate(tri.decode_cache.calls[:2]):
        refd = O.decode(codes, b, bits(qd[0, :, 0]), t, split, scale, ktail, vtail, bits(kd[0, :, 0]),
                        bits(vd[0, :, 0]), step)
        assert_close_bf16(od[0, quant_q, 0].numpy(), refd[quant_q], what=f"C4 layer {layer} decode step {step}")
        keys, values = torch.cat([keys, kd[0]], 1), torch.cat([values, vd[0]], 1)
        d64, d32 = decode_exact_rows(qd[0, :, 0], keys, values, exact_q, scale)
        bar = max(2e-3, float(np.abs(d32 - d64).max()))
        assert_close_bf16(od[0, exact_q, 0].numpy(), d64, max_abs=bar, what=f"C4 layer {layer} decode step {step} exact")
        ktail[:, step] = bits(kd[0, :, 0])
        vtail[:, step] = bits(vd[0, :, 0])
