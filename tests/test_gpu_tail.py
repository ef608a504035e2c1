"""Tail growth (extension) on the GPU.

The reference's tail holds max_tail generated tokens and then overwrites its last slot
(common_device.cuh:384).  With growth, a full tail's oldest 64 tokens become a new tile of the cache
(tri_tail_spill).  Checked here:
  * the spill kernel against its host restatement, bit for bit (records, scales, metadata, task table,
    tails, tail base), over ragged stores, room that doubles and exact heads;
  * decode outputs against the oracle's GrowingTail over 2,000 steps with max_tail 256 (quantized heads,
    same bar as the other decode tests) and float64 attention over every raw key (exact heads);
  * a 2,000-token HF generation with max_tail 256, every decode call against the oracle;
  * graph replay, room doubling and the eager path give the same tokens."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from cache_host import HostCacheModule
from helpers import assert_close, assert_close_bf16, run_prefill
from test_gpu_parity import _attend64, small
from triattention_amd import models as M
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import I8, Prefill
from triattention_amd.maps import from_bands
from triattention_amd.synthetic import INF, bits

pytestmark = pytest.mark.gpu

BANDS = [[INF, INF], [1, 1], [0, INF], [0, 3], [0, 0], [0, 0], [2, 5], [1, INF]]
ARRAYS = ("entry", "kinfo", "slot", "count", "fmt", "prompt", "xslot", "ka", "ka4", "k8", "k4", "kx", "vx", "tail_k",
          "tail_v")


class TeeCache(DecodeCache):
    """A GPU decode cache whose stores are replayed, on host copies of their sources, into ``host``."""

    def __init__(self, module, host, max_tail, grow_tail):
        super().__init__(module, max_tail, grow_tail=grow_tail)
        self.host = host

    def store(self, layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv=(), kx=None, vx=None):
        cpu = lambda x: None if x is None else x.cpu()
        self.host.store(layer, prompt, cpu(kp), cpu(ka), cpu(kstat), cpu(vstat), {c: cpu(p) for c, p in packed.items()},
                        codes, bands, cpu(k4), cpu(ka4), exact_kv, cpu(kx), cpu(vx))
        super().store(layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv, kx, vx)


def _host_step(cache, kd, vd):
    """The host cache's side of one decode step: growth check, spill, the merge's tail append, advance."""
    e = cache._grow_step(0)
    cache._spill_plan(e).run()
    held = int(cache.step[0]) - int(e["store"].arrays["tail_base"][0])
    slot = min(cache.max_tail - 1, held)
    e["tail_k"][:, :, slot] = kd
    e["tail_v"][:, :, slot] = vd
    cache.advance()


def _compare(gpu, host, what):
    for name in ARRAYS:
        a, b = gpu.get(name), host.get(name)
        assert (a is None) == (b is None), (what, name)
        if a is not None:
            assert a.shape == b.shape, (what, name, a.shape, b.shape)
            assert torch.equal(a.cpu().view(torch.uint8), b.view(torch.uint8)), (what, name)
    assert torch.equal(gpu["v"][I8].cpu(), host["v"][I8]), (what, "v8")
    assert torch.equal(gpu["store"].arrays["tail_base"].cpu(), host["store"].arrays["tail_base"]), (what, "tail base")
    g, h = gpu["store"].arrays["grow"][:gpu["batch"]].cpu(), host["store"].arrays["grow"][:host["batch"]]
    assert torch.equal(g[..., :3], h[..., :3]), (what, "grow")


def _compare_tasks(module, e, what):
    """The task table the spills updated against one built afresh from the metadata they wrote: equal in
    every lane's offsets, flags and K scales, the work item (lane 0) and the entry count (lane 1)."""
    table, n = e["tasks"]
    items = torch.from_numpy(DecodeCache._task_items(e)).to(table.device)
    fresh, n2 = module.decode_tasks(e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"], e["slot"],
                                    e["per"], e["bounds"], items)
    assert n == n2
    a, b = table.view(n, 512).cpu(), fresh.view(n, 512).cpu()
    ints_a, ints_b = a[:, :256].view(n, 64, 4), b[:, :256].view(n, 64, 4)
    assert torch.equal(ints_a[:, :, :3], ints_b[:, :, :3]), what
    assert torch.equal(ints_a[:, :2, 3], ints_b[:, :2, 3]), what
    assert torch.equal(a[:, 256:], b[:, 256:]), what


@pytest.mark.parametrize("bf16_kv", [[], [1]])
def test_tail_spill_kernel_equals_host_restatement(module, bf16_kv):
    hq, hk, max_tail = 8, 4, 64
    print(f"\n[tail] spill kernel vs host restatement, exact KV heads {bf16_kv}", flush=True)
    host = DecodeCache(HostCacheModule(), max_tail=max_tail, grow_tail=64)
    host.ragged = True
    cache = TeeCache(module, host, max_tail, 64)
    cache.ragged = True
    fn = from_bands({"0": BANDS}, bf16={"0": bf16_kv} if bf16_kv else None)
    pre = Prefill(module, fn, cache, out_dtype=torch.float32)
    dev = torch.device("cuda")
    for i, (prompt, batch) in enumerate(((130, 2), (64, 1), (700, 1))):
        q, k, v = small(9700 + i, batch, hq, hk, prompt)
        pre(0, q.to(dev), k.to(dev), v.to(dev), 128 ** -0.5)
    rows = 4
    g = S.gen(9800)
    for t in range(64 * 5 + 30):
        qd, kd, vd = S.outlier_tensor(g, rows, hq, 1), S.outlier_tensor(g, rows, hk, 1), S.outlier_tensor(g, rows, hk, 1)
        cache(0, qd.to(dev), kd.to(dev), vd.to(dev), 128 ** -0.5)
        cache.advance()
        _host_step(host, kd[:, :, 0], vd[:, :, 0])
        if t % 64 == 1 or t == 64 * 5 + 29:
            torch.cuda.synchronize()
            _compare(cache.layers[0], host.layers[0], f"after step {t}")
            if not bf16_kv:
                _compare_tasks(module, cache.layers[0], f"tasks after step {t}")
    assert cache.layers[0]["store"].tb == 64 * 5 and cache.layers[0]["store"].grow_tiles == 8


def test_a_spill_without_room_for_one_head_changes_nothing(module):
    """tri_tail_spill spills for every (sequence, KV head) or for none: with the V record array cut at
    one head's first growth slot, the launch on a full tail leaves the tails, the tail base, the
    metadata and the records as they were; the same launch over the whole array then spills."""
    hq, hk, max_tail = 8, 4, 64
    print("\n[tail] spill without room for one head", flush=True)
    cache = DecodeCache(module, max_tail=max_tail, grow_tail=64)
    pre = Prefill(module, from_bands({"0": BANDS}), cache, out_dtype=torch.float32)
    dev = torch.device("cuda")
    q, k, v = small(9900, 2, hq, hk, 130)
    pre(0, q.to(dev), k.to(dev), v.to(dev), 128 ** -0.5)
    g = S.gen(9901)
    for _ in range(max_tail):
        qd, kd, vd = S.outlier_tensor(g, 2, hq, 1), S.outlier_tensor(g, 2, hk, 1), S.outlier_tensor(g, 2, hk, 1)
        cache(0, qd.to(dev), kd.to(dev), vd.to(dev), 128 ** -0.5)
        cache.advance()
    e = cache.layers[0]
    st, a, rows = e["store"], e["store"].arrays, e["batch"]
    torch.cuda.synchronize()
    assert int(cache.step[0]) == max_tail and int(a["tail_base"][0]) == 0  # full: the next launch spills
    dst = dict(entry=e["entry"], kinfo=e["kinfo"], slot=e["slot"], count=e["count"], count0=a["count0"][:rows],
               fmt=e["fmt"], xslot=e["xslot"], ka=e["ka"], ka4=e["ka4"], kstat=e["kstat"], vstat=e["vstat"],
               k8=e["k8"], k4=e["k4"], v8=e["v"][I8], kx=e["kx"], vx=e["vx"])
    grow = a["grow"][:rows].cpu()
    kept = grow[:, :, 0] >= 0
    assert kept.sum() > 1
    short = int(grow[:, :, 2][kept].max())  # that head's first growth slot is past the cut array
    tasks = e.get("tasks") if cache.tasks else None
    launch = lambda d: module.plan_tail_spill(cache.step, a["tail_base"], e["tail_k"], e["tail_v"], a["grow"][:rows],
                                              st.grow_tiles, e["prompt"], d, tasks)
    names = ("entry", "kinfo", "slot", "count", "fmt", "ka", "k8", "tail_k", "tail_v")
    before = {n: e[n].clone() for n in names}
    before["v8"], before["tail_base"] = dst["v8"].clone(), a["tail_base"].clone()
    if tasks is not None:
        before["tasks"] = tasks[0].clone()
    now = lambda n: dst["v8"] if n == "v8" else a["tail_base"] if n == "tail_base" else \
        tasks[0] if n == "tasks" else e[n]
    launch(dict(dst, v8=dst["v8"][:short])).run()
    torch.cuda.synchronize()
    for n, x in before.items():
        assert torch.equal(now(n), x), f"{n} changed by a spill without room"
    launch(dst).run()
    torch.cuda.synchronize()
    assert a["tail_base"].tolist() == [64, 0]  # (a 64-slot tail has no rows left to move up)
    assert torch.equal(e["count"][kept.to(dev)], before["count"][kept.to(dev)] + 1)


def _decode_run(module, prompts, bf16_kv, steps, max_tail, seed, check_every):
    hq, hk = 8, 4
    bands = torch.tensor(BANDS, dtype=torch.int32)
    cache = DecodeCache(module, max_tail=max_tail, grow_tail=steps)
    cache.ragged = len(prompts) > 1
    cache.out_dtype = torch.float32
    dev = torch.device("cuda")
    seqs, raw = [], []
    for i, (prompt, batch) in enumerate(prompts):
        q, k, v = small(seed + i, batch, hq, hk, prompt)
        run_prefill(module, q, k, v, bands, 128 ** -0.5, decode_cache=cache, bf16_kv=bf16_kv)
        for b in range(batch):
            codes = O.prefill_codes(None, bits(k[b]), bits(v[b]), bands.numpy(), decode_cache=True)
            seqs.append(O.GrowingTail(codes, bands.numpy(), prompt, max_tail))
            kr, vr = torch.zeros(hk, prompt + steps, 128), torch.zeros(hk, prompt + steps, 128)
            kr[:, :prompt], vr[:, :prompt] = k[b].float(), v[b].float()
            raw.append((kr, vr, prompt))
    rows = len(seqs)
    exact_q = [h for h in range(hq) if h // 2 in bf16_kv]
    quant_q = [h for h in range(hq) if h // 2 not in bf16_kv]
    g = S.gen(seed + 50)
    checked = 0
    for t in range(steps):
        qd, kd, vd = S.outlier_tensor(g, rows, hq, 1), S.outlier_tensor(g, rows, hk, 1), S.outlier_tensor(g, rows, hk, 1)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), 128 ** -0.5)
        held = seqs[0].held
        check = t % check_every == 0 or held >= max_tail - 1 or t == steps - 1
        if check:
            out = out.cpu().numpy()
        for b in range(rows):
            ref = seqs[b].step(bits(qd[b, :, 0]), bits(kd[b, :, 0]), bits(vd[b, :, 0]), cache.split_of(0, b),
                               128 ** -0.5, compute=check)
            kr, vr, p = raw[b]
            kr[:, p + t], vr[:, p + t] = kd[b, :, 0].float(), vd[b, :, 0].float()
            if check:
                assert_close(out[b, quant_q, 0], ref[quant_q], what=f"quantized heads step {t} seq {b}")
                if exact_q:
                    r64, r32 = _attend64(qd[b, :, 0], kr[:, :p + t + 1], vr[:, :p + t + 1], 128 ** -0.5)
                    bar = max(2e-3, float(np.abs(r32[exact_q] - r64[exact_q]).max()))
                    assert_close(out[b, exact_q, 0], r64[exact_q], max_abs=bar, what=f"exact heads step {t} seq {b}")
        checked += check
        cache.advance()
    st = cache.layers[0]["store"]
    assert st.tb == 64 * len(seqs[0].grown) > 0
    return checked


@pytest.mark.parametrize("prompts,bf16_kv", [([(300, 2)], []), ([(100, 1), (700, 1)], [1])])
def test_decode_with_tail_growth_matches_the_oracle(module, prompts, bf16_kv):
    print(f"\n[tail] decode 2000 steps, max_tail 256, prompts {prompts}, exact {bf16_kv}", flush=True)
    checked = _decode_run(module, prompts, bf16_kv, 2000, 256, 9900 + len(bf16_kv), 9)
    assert checked > 200


def tiny_qwen2(device):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                                   rope_theta=1e6, tie_word_embeddings=False)
    torch.manual_seed(11)
    return transformers.Qwen2ForCausalLM(cfg).to(torch.bfloat16).to(device).eval()


class Recorder:
    def __init__(self, inner):
        self.inner, self.calls = inner, []

    def __getattr__(self, name):
        return getattr(self.inner, name)

    def __call__(self, layer, q, k, v, scale):
        out = self.inner(layer, q, k, v, scale)
        self.calls.append((layer, q.cpu(), k.cpu(), v.cpu(), out.float().cpu(), scale))
        return out


MODEL_BANDS = {"0": [[INF, INF], [0, INF], [1, INF], [1, INF]], "1": [[2, 4], [1, 3], [INF, INF], [INF, INF]]}


def test_generate_2000_tokens_with_max_tail_256_matches_the_oracle(module):
    """A 2,000-token greedy generation through TriAttention with max_tail 256: every decode call of both
    layers against the oracle's GrowingTail (quantized heads) and float64 attention over the raw prompt
    and generated keys (exact heads)."""
    print("\n[tail] HF Qwen2 generate 2000 tokens, max_tail 256", flush=True)
    dev = torch.device("cuda")
    model = tiny_qwen2(dev)
    bf16 = {"1": [1]}
    steps, prompt = 2000, 200
    tri = M.TriAttention(model, from_bands(MODEL_BANDS, model, bf16=bf16), max_new_tokens=steps, module=module,
                         max_tail=256)
    tri.prefill = Recorder(tri.prefill)
    tri.decode_cache = Recorder(tri.decode_cache)
    ids = torch.randint(256, (1, prompt), generator=torch.Generator().manual_seed(12)).to(dev)
    tokens = tri.generate(ids, steps, eos=set())
    assert len(tokens) == steps
    pre, dec = tri.prefill.calls, tri.decode_cache.calls
    assert [c[0] for c in dec] == [0, 1] * steps
    cache = tri.decode_cache.inner
    for layer in (0, 1):
        _, q0, k0, v0, _, scale = pre[layer]
        b = np.asarray(MODEL_BANDS[str(layer)], np.int32)
        codes = O.prefill_codes(None, bits(k0[0]), bits(v0[0]), b, decode_cache=True)
        seq = O.GrowingTail(codes, b, prompt, 256)
        split = cache.split_of(layer, 0)
        exact_q = [h for h in range(4) if h // 2 in bf16.get(str(layer), [])]
        quant_q = [h for h in range(4) if h // 2 not in bf16.get(str(layer), [])]
        keys, values = k0[0].float(), v0[0].float()
        for step, (_, q, k, v, out, _) in enumerate(c for c in dec if c[0] == layer):
            ref = seq.step(bits(q[0, :, 0]), bits(k[0, :, 0]), bits(v[0, :, 0]), split, scale)
            assert_close_bf16(out[0, quant_q, 0].numpy(), ref[quant_q], what=f"decode layer {layer} step {step}")
            keys, values = torch.cat([keys, k[0].float()], 1), torch.cat([values, v[0].float()], 1)
            if exact_q and (step % 7 == 0 or step == steps - 1):
                r64, r32 = _attend64(q[0, :, 0], keys, values, scale)
                bar = max(2e-3, float(np.abs(r32[exact_q] - r64[exact_q]).max()))
                assert_close_bf16(out[0, exact_q, 0].numpy(), r64[exact_q], max_abs=bar,
                                  what=f"decode layer {layer} step {step} exact")
        assert len(seq.grown) == (steps - 1 - 256) // 64 + 1


def test_graph_replay_and_room_doubling_give_the_eager_tokens(module):
    """700 tokens with max_tail 128: eager with room for every tile taken from the tail, eager with room
    for one tile (doubled five times), and graph replay with room for one tile (each doubling runs one
    step eagerly and captures again) generate the same tokens."""
    print("\n[tail] HF Qwen2 generate 700 tokens, max_tail 128: eager / doubling / graph", flush=True)
    dev = torch.device("cuda")
    model = tiny_qwen2(dev)
    ids = torch.randint(256, (1, 150), generator=torch.Generator().manual_seed(13)).to(dev)
    runs = []
    for graph, room in ((False, None), (False, 64), (True, 64), (True, None)):
        tri = M.TriAttention(model, from_bands(MODEL_BANDS, model, bf16={"1": [1]}), max_new_tokens=700,
                             module=module, max_tail=128)
        if room is not None:
            tri.decode_cache.grow_tail = room
        runs.append(tri.generate(ids, 700, eos=set(), graph=graph))
        torch.cuda.synchronize()
        st = tri.decode_cache.layers[0]["store"]
        assert st.tb == 64 * ((700 - 1 - 128) // 64 + 1)
        if room is not None:
            assert st.grow_tiles == 16
    assert runs[0] == runs[1] == runs[2] == runs[3]
