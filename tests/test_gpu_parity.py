"""GPU parity: the gfx950 kernels through the C ABI against the CPU oracle.

Bar: quantized codes, scales and statistics bit-exact; attention outputs (fp32)
within 2e-3 max-abs and 1e-3 mean-abs of the oracle.  Exact (bf16) heads are held
to float64 attention over the same bf16 inputs: mean-abs 1e-3, max-abs 2e-3 or
torch fp32 SDPA's own max-abs error on those inputs, whichever is larger.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, compare_codes, exact_max_abs_bar, exact_reference, oracle_prefill, run_prefill
from triattention_amd import synthetic as S
from triattention_amd.kernels import records as R
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import Prefill
from triattention_amd.maps import from_bands
from triattention_amd.synthetic import INF, bits

pytestmark = pytest.mark.gpu


def small(seed, batch, hq, hk, t):
    g = S.gen(seed)
    return (S.outlier_tensor(g, batch, hq, t), S.outlier_tensor(g, batch, hk, t), S.outlier_tensor(g, batch, hk, t))


MIXED = [[INF, INF], [INF, INF], [INF, INF], [1, INF], [1, INF], [1, INF]]


@pytest.mark.parametrize("t", [1, 63, 64, 65, 200])
def test_codes_and_output_small(module, t):
    print(f"\n[parity] small prefill t={t}", flush=True)
    q, k, v = small(2000 + t, 1, 6, 2, t)
    bands = torch.tensor(MIXED, dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    compare_codes(ops, codes[0], 0, 1, 6, 2, t)
    assert_close(out.numpy(), ref, what=f"prefill t={t}", tol=tol)


def test_statistics_past_one_load_batch(module):
    """K/V statistics of chains longer than one batch of token loads, with a remainder: T = 2500 gives
    the 64 block chains 39 or 40 tokens each (one full batch of 32, then the rest), bit-exact codes and
    statistics against the oracle, outputs within the parity bar."""
    print("\n[parity] prefill t=2500 (statistics over two load batches)", flush=True)
    q, k, v = small(2600, 1, 4, 2, 2500)
    bands = torch.tensor(MIXED[:2] + MIXED[3:5], dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    compare_codes(ops, codes[0], 0, 1, 4, 2, 2500)
    assert_close(out.numpy(), ref, what="prefill t=2500", tol=tol)


def test_zero_query_and_key_rows(module):
    """All-zero query rows (scale 0, so every score of the row is 0 and masked keys give 0 * -inf) and
    all-zero key rows: outputs finite and within the parity bar, codes bit-exact."""
    print("\n[parity] prefill t=150 with zero query / key rows", flush=True)
    q, k, v = small(2500, 1, 6, 2, 150)
    q[0, :, [0, 5, 64, 149]] = 0
    q[0, 2, 70:90] = 0
    k[0, 1, [3, 64, 100]] = 0
    bands = torch.tensor(MIXED, dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    compare_codes(ops, codes[0], 0, 1, 6, 2, 150)
    assert_close(out.numpy(), ref, what="prefill with zero rows", tol=tol)


def test_batch_and_band_variety(module):
    print("\n[parity] batch=2 t=333 assorted bands", flush=True)
    q, k, v = small(3000, 2, 8, 2, 333)
    bands = torch.tensor([[INF, INF], [1, INF], [2, 4], [3, 3], [1, 2], [2, INF], [1, 1], [4, 5]], dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    for b in range(2):
        compare_codes(ops, codes[b], b, 2, 8, 2, 333)
    assert_close(out.numpy(), ref, what="prefill batch 2", tol=tol)


def test_config0_prefill(module):
    print("\n[parity] config 0 (B1 Hq24 Hk8 T1024, 50/50 INT8/INT4)", flush=True)
    c = S.config0()
    out, ops, _ = run_prefill(module, c["q"], c["k"], c["v"], c["bands"], c["scale"])
    ref, codes, tol = oracle_prefill(c["q"], c["k"], c["v"], c["bands"], c["scale"])
    compare_codes(ops, codes[0], 0, 1, 24, 8, 1024)
    mx, mn = assert_close(out.numpy(), ref, what="config 0", tol=tol)
    print(f"config0 max abs {mx:.3e} mean abs {mn:.3e}")


def test_bf16_output_within_one_ulp(module):
    print("\n[parity] bf16 output rounding", flush=True)
    q, k, v = small(4000, 1, 6, 2, 200)
    bands = torch.tensor(MIXED, dtype=torch.int32)
    out16, _, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5, out_dtype=torch.bfloat16)
    ref, _, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    r = torch.from_numpy(ref).to(torch.bfloat16).float()
    # one bf16 ulp, plus the exp2-rounding bound where a probability may round either way
    ulp = torch.abs(r).clamp(min=1e-30).log2().floor().exp2() * 2.0 ** -7 + torch.from_numpy(tol)
    assert bool((torch.abs(out16 - r) <= ulp + 1e-30).all())


def _decode_case(module, prompt, bands, batch=1, steps=3, max_tail=8, seed=5000, hq=6, hk=2, per=None, tasks=True):
    print(f"\n[parity] decode prompt={prompt} batch={batch} steps={steps} per={per} tasks={tasks}", flush=True)
    q, k, v = small(seed, batch, hq, hk, prompt)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    cache.per = per
    cache.tasks = tasks
    _, ops, pre = run_prefill(module, q, k, v, bands, scale, decode_cache=cache)
    ref_codes = [O.prefill_codes(bits(q[b]), bits(k[b]), bits(v[b]), bands.numpy(), decode_cache=True)
                 for b in range(batch)]
    e = cache.layers[0]
    kept = (e["ka"], e["kstat"], e["vstat"], e["ka4"])  # the copies the cache keeps
    for b in range(batch):
        compare_codes(ops, ref_codes[b], b, batch, hq, hk, prompt, kept=kept)
    g = S.gen(seed + 1)
    ktail = np.zeros((batch, hk, max_tail, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    dev = torch.device("cuda")
    for step in range(steps):
        qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        for b in range(batch):
            ref = O.decode(ref_codes[b], bands.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale,
                           ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"decode step {step} seq {b}")
            prior = min(step, max_tail - 1)
            ktail[b, :, prior] = bits(kd[b, :, 0])
            vtail[b, :, prior] = bits(vd[b, :, 0])
        cache.advance()


def test_decode_mixed(module):
    bands = torch.tensor(MIXED, dtype=torch.int32)
    _decode_case(module, 300, bands)


def test_decode_bands_and_tail_overflow(module):
    bands = torch.tensor([[2, 4], [1, INF], [INF, INF], [3, 6], [1, 1], [2, 2]], dtype=torch.int32)
    _decode_case(module, 1500, bands, batch=2, steps=5, max_tail=3, seed=5100)


@pytest.mark.parametrize("per", [1, 3, 64])
def test_decode_uniform_split(module, per):
    """The reference's split (runs of `per` tiles, no partition) through the same kernel."""
    bands = torch.tensor([[2, 4], [1, INF], [INF, INF], [3, 6], [1, 1], [2, 2]], dtype=torch.int32)
    _decode_case(module, 1500, bands, batch=2, steps=2, max_tail=3, seed=5150, per=per)


@pytest.mark.parametrize("hq,hk,per", [(24, 8, 1), (24, 8, 2), (24, 8, 3), (32, 8, 2), (16, 2, 3), (8, 8, 2)])
def test_decode_two_waves_per_workgroup(module, hq, hk, per):
    """A grid larger than the resident one-wave workgroups (8 per CU) runs two waves per workgroup,
    taking a split's tiles alternately: per 1 leaves the second wave without tiles, per 3 gives the
    waves 2 and 1.  Groups 3 and 1 (DUP layout, packed 4-bit Q in registers), 4 (DUP, packed Q read
    from LDS) and 8 (two row blocks); mixed INT8/INT4/skipped tiles."""
    g = hq // hk
    kinds = [[INF, INF], [1, INF], [2, 5], [3, INF]]
    bands = torch.tensor([kinds[h % 4] for h in range(hk) for _ in range(g)], dtype=torch.int32)
    prompt = 600
    splits = -(-10 // per)
    batch = (9 * module.device_cus()) // (splits * hk) + 1
    _decode_case(module, prompt, bands, batch=batch, steps=2, max_tail=4, seed=5300 + 10 * g + per, hq=hq, hk=hk,
                 per=per)


@pytest.mark.parametrize("per", [1, 3])
def test_decode_two_waves_per_workgroup_without_task_table(module, per):
    """The gather path (no task table: each split finds its entries in the cache's metadata) with a grid
    larger than the resident one-wave workgroups, so two waves per workgroup."""
    hq, hk = 24, 8
    kinds = [[INF, INF], [1, INF], [2, 5], [0, INF]]
    bands = torch.tensor([kinds[h % 4] for h in range(hk) for _ in range(hq // hk)], dtype=torch.int32)
    splits = -(-10 // per)
    batch = (9 * module.device_cus()) // (splits * hk) + 1
    _decode_case(module, 600, bands, batch=batch, steps=2, max_tail=4, seed=5500 + per, hq=hq, hk=hk, per=per,
                 tasks=False)


def test_decode_short_prompt(module):
    bands = torch.tensor(MIXED, dtype=torch.int32)
    _decode_case(module, 40, bands, steps=2, seed=5200)


@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2), (8, 1), (7, 1)])
def test_decode_group_sizes(module, hq, hk):
    g = hq // hk
    kinds = [[INF, INF], [1, INF], [2, 5], [3, INF], [1, 1], [INF, INF], [1, INF], [2, 2]]
    bands = torch.tensor([kinds[h % len(kinds)] for h in range(hq)], dtype=torch.int32)
    _decode_case(module, 777, bands, batch=2, steps=2, max_tail=4, seed=5300 + g, hq=hq, hk=hk)


def test_decode_long_tail(module):
    """Twenty steps with a 24-slot tail: the merge's unrolled tail loops and the tail overwrite."""
    bands = torch.tensor([[INF, INF], [1, INF], [2, 6], [1, INF], [INF, INF], [3, 3]], dtype=torch.int32)
    _decode_case(module, 500, bands, batch=2, steps=20, max_tail=24, seed=5400)


def test_decode_full_1024_token_tail(module):
    """The largest tail the merge holds (max_tail 1024): steps 1021-1025 over a tail pre-filled with
    random bf16 rows, the last three overwriting slot 1023 as the reference does."""
    print("\n[parity] decode with a 1024-token tail (steps 1021-1025)", flush=True)
    hq, hk, batch, prompt, max_tail = 8, 2, 2, 300, 1024
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                         dtype=torch.int32)
    q, k, v = small(5600, batch, hq, hk, prompt)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, bands, scale, decode_cache=cache)
    codes = [O.prefill_codes(bits(q[b]), bits(k[b]), bits(v[b]), bands.numpy(), decode_cache=True)
             for b in range(batch)]
    e = cache.layers[0]
    g = S.gen(5601)
    e["tail_k"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_k"].device))
    e["tail_v"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_v"].device))
    ktail, vtail = bits(e["tail_k"].cpu()).copy(), bits(e["tail_v"].cpu()).copy()
    cache.step.fill_(1021)
    dev = torch.device("cuda")
    for step in range(1021, 1026):
        qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        prior = min(step, max_tail - 1)
        for b in range(batch):
            ref = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale, ktail[b],
                           vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"step {step} seq {b}")
            ktail[b, :, prior] = bits(kd[b, :, 0])
            vtail[b, :, prior] = bits(vd[b, :, 0])
        cache.advance()
    assert np.array_equal(bits(e["tail_k"].cpu()), ktail) and np.array_equal(bits(e["tail_v"].cpu()), vtail)


def test_decode_entries_without_v_format_flags(module):
    """Without the task table, the split kernel gathers its splits from the metadata rows; entry words
    without the V-format flags (the reference's plain tile indices) make it read fmt as well.  Both give
    the task table's outputs bit for bit."""
    from triattention_amd.kernels.decode import ENTRY_TILE
    print("\n[parity] decode with plain tile indices in the entry table", flush=True)
    hq, hk, prompt = 8, 2, 1100
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                         dtype=torch.int32)
    q, k, v = small(5700, 2, hq, hk, prompt)
    cache = DecodeCache(module, max_tail=4)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, bands, 128 ** -0.5, decode_cache=cache)
    g = S.gen(5701)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, 2, hq, 1).to(dev), S.outlier_tensor(g, 2, hk, 1).to(dev),
                  S.outlier_tensor(g, 2, hk, 1).to(dev))
    tasks = cache(0, qd, kd, vd, 128 ** -0.5).cpu()
    e = cache.layers[0]
    assert "tasks" in e
    for key in [key for key in e if isinstance(key, tuple) and key[0] == "plan"]:
        del e[key]
    cache.tasks = False
    flagged = cache(0, qd, kd, vd, 128 ** -0.5).cpu()
    assert torch.equal(tasks.view(torch.int32), flagged.view(torch.int32))
    for key in [key for key in e if isinstance(key, tuple) and key[0] == "plan"]:
        del e[key]
    assert bool((e["entry"] != (e["entry"] & ENTRY_TILE)).any())
    e["entry"].bitwise_and_(ENTRY_TILE)
    plain = cache(0, qd, kd, vd, 128 ** -0.5).cpu()
    assert torch.equal(tasks.view(torch.int32), plain.view(torch.int32))


def test_timed_split_launch_matches_untimed(module):
    """tri_decode_partials_timed (the split-KV kernel launched with its own start/stop events) followed
    by the merge gives the untimed decode's outputs bit for bit, and the events hold a positive time."""
    print("\n[parity] timed split-KV launch", flush=True)
    hq, hk, prompt = 6, 2, 700
    bands = torch.tensor(MIXED, dtype=torch.int32)
    q, k, v = small(5800, 2, hq, hk, prompt)
    cache = DecodeCache(module, max_tail=4)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, bands, 128 ** -0.5, decode_cache=cache)
    g = S.gen(5801)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, 2, hq, 1).to(dev), S.outlier_tensor(g, 2, hk, 1).to(dev),
                  S.outlier_tensor(g, 2, hk, 1).to(dev))
    untimed = cache(0, qd, kd, vd, 128 ** -0.5).cpu()
    out = torch.empty((2, hq, 1, 128), dtype=torch.float32, device=dev)
    plan = cache.plan(0, qd, kd, out, 128 ** -0.5)
    stream = torch.cuda.current_stream()
    events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    for e in events:
        e.record(stream)
    plan.run(qd, kd, vd, out, 1, events=events)
    plan.run(qd, kd, vd, out, 2, short_tail=cache.short_tail(0, hq))  # the merge form the untimed call took
    torch.cuda.synchronize()
    assert torch.equal(untimed.view(torch.int32), out.cpu().view(torch.int32))
    assert events[0].elapsed_time(events[1]) > 0.0
    with pytest.raises(RuntimeError):
        plan.run(qd, kd, vd, out, 3, events=events)


def test_ragged_decode_batch(module):
    """Ragged cache: four prompts of different lengths stored by separate Prefill calls, served by one
    decode launch per step; every sequence matches the oracle."""
    print("\n[parity] ragged decode, prompts 100/700/64/2000", flush=True)
    hq, hk, max_tail, steps = 8, 2, 4, 3
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                         dtype=torch.int32)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.ragged = True
    cache.out_dtype = torch.float32
    prompts = [100, 700, 64, 2000]
    codes = []
    for i, n in enumerate(prompts):
        q, k, v = small(8000 + i, 1, hq, hk, n)
        run_prefill(module, q, k, v, bands, scale, decode_cache=cache)
        codes.append(O.prefill_codes(bits(q[0]), bits(k[0]), bits(v[0]), bands.numpy(), decode_cache=True))
    e = cache.layers[0]
    assert e["batch"] == len(prompts)
    g = S.gen(8100)
    ktail = np.zeros((len(prompts), hk, max_tail, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    dev = torch.device("cuda")
    for step in range(steps):
        qd, kd, vd = (S.outlier_tensor(g, len(prompts), hq, 1), S.outlier_tensor(g, len(prompts), hk, 1),
                      S.outlier_tensor(g, len(prompts), hk, 1))
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        for b, n in enumerate(prompts):
            ref = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), n, cache.split_of(0, b), scale, ktail[b],
                           vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(out[b, :, 0], ref, what=f"ragged step {step} seq {b} (prompt {n})")
            ktail[b, :, step] = bits(kd[b, :, 0])
            vtail[b, :, step] = bits(vd[b, :, 0])
        cache.advance()


def test_store_only_builds_the_same_cache(module):
    """Prefill.store_only (no attention launch) stores the same records and metadata as a full Prefill
    call, and decode returns identical bits from either cache."""
    print("\n[parity] store_only vs Prefill cache", flush=True)
    hq, hk, t = 6, 3, 333
    q, k, v = small(8500, 2, hq, hk, t)
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [2, 2]], dtype=torch.int32)
    dev = torch.device("cuda")
    caches = []
    for full in (True, False):
        cache = DecodeCache(module, max_tail=4)
        pre = Prefill(module, from_bands({"0": bands.tolist()}, bf16={"0": [1]}), cache)
        if full:
            pre(0, q.to(dev), k.to(dev), v.to(dev), 128 ** -0.5)
        else:
            pre.store_only(0, k.to(dev), v.to(dev), hq)
        caches.append(cache)
    a, b = (c.layers[0] for c in caches)
    for key in ("k8", "k4", "ka", "ka4", "kstat", "vstat", "entry", "kinfo", "count", "slot", "fmt", "xslot", "kx",
                "vx"):
        assert torch.equal(a[key], b[key]), key
    for code in a["v"]:
        assert torch.equal(a["v"][code], b["v"][code])
    g = S.gen(8600)
    qd, kd, vd = (S.outlier_tensor(g, 2, hq, 1).to(dev), S.outlier_tensor(g, 2, hk, 1).to(dev),
                  S.outlier_tensor(g, 2, hk, 1).to(dev))
    outs = [c(0, qd, kd, vd, 128 ** -0.5) for c in caches]
    assert torch.equal(outs[0], outs[1])


def _attend64(q, keys, values, scale):
    """float64 and float32 attention of one query per head over explicit key/value lists:
    q [Hq,128], keys/values [Hk,L,128] (GQA groups adjacent)."""
    g = q.shape[0] // keys.shape[0]
    outs = []
    for dt in (torch.float64, torch.float32):
        k = keys.to(dt).repeat_interleave(g, 0)
        v = values.to(dt).repeat_interleave(g, 0)
        w = torch.softmax(torch.einsum("hd,hld->hl", q.to(dt), k) * scale, dim=-1)
        outs.append(torch.einsum("hl,hld->hd", w, v).numpy())
    return outs


@pytest.mark.parametrize("prompt,bf16_kv,batch", [(300, [1], 2), (64, [0, 2], 1), (1500, [2], 2), (200, [0, 1, 2], 2)])
def test_decode_with_exact_heads(module, prompt, bf16_kv, batch):
    """Maps with bf16 KV heads through Prefill + DecodeCache: quantized heads match the oracle, exact heads
    match float64 attention over the raw bf16 prompt and tail."""
    print(f"\n[parity] decode with exact heads prompt={prompt} kv={bf16_kv} batch={batch}", flush=True)
    hq, hk, steps, max_tail = 6, 3, 4, 8
    q, k, v = small(7000 + prompt, batch, hq, hk, prompt)
    bands = torch.tensor([[2, 4], [1, INF], [INF, INF], [1, 1], [3, 6], [2, 2]], dtype=torch.int32)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, bands, scale, decode_cache=cache, bf16_kv=bf16_kv)
    ref_codes = [O.prefill_codes(bits(q[b]), bits(k[b]), bits(v[b]), bands.numpy(), decode_cache=True)
                 for b in range(batch)]
    g = S.gen(7100 + prompt)
    ktail = np.zeros((batch, hk, max_tail, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    keys, values = k.clone(), v.clone()
    exact_q = [h for h in range(hq) if h // 2 in bf16_kv]
    quant_q = [h for h in range(hq) if h // 2 not in bf16_kv]
    dev = torch.device("cuda")
    for step in range(steps):
        qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        keys, values = torch.cat([keys, kd], 2), torch.cat([values, vd], 2)
        for b in range(batch):
            if quant_q:
                ref = O.decode(ref_codes[b], bands.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale,
                               ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
                assert_close(out[b, quant_q, 0], ref[quant_q], what=f"quantized heads step {step} seq {b}")
            r64, r32 = _attend64(qd[b, :, 0], keys[b], values[b], scale)
            bar = max(2e-3, float(np.abs(r32[exact_q] - r64[exact_q]).max()))
            assert_close(out[b, exact_q, 0], r64[exact_q], max_abs=bar, what=f"exact heads step {step} seq {b}")
            ktail[b, :, step] = bits(kd[b, :, 0])
            vtail[b, :, step] = bits(vd[b, :, 0])
        cache.advance()


@pytest.mark.parametrize("t,bf16_kv", [(37, [1]), (64, [1]), (333, [1]), (200, [0, 2]), (129, [0, 1, 2])])
def test_exact_bf16_heads_in_the_same_launch(module, t, bf16_kv):
    """KV heads kept bf16: their q-heads match float64 attention on the raw operands, the others the oracle."""
    print(f"\n[parity] exact bf16 heads t={t} kv={bf16_kv}", flush=True)
    q, k, v = small(6000 + t, 2, 6, 3, t)
    bands = torch.tensor([[INF, INF], [INF, INF], [1, INF], [1, INF], [2, 3], [2, 3]], dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5, bf16_kv=bf16_kv)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    ex = exact_reference(q, k, v, 128 ** -0.5)
    exact_q = [h for h in range(6) if h // 2 in bf16_kv]
    quant = [h for h in range(6) if h // 2 not in bf16_kv]
    if quant:
        assert_close(out.numpy()[:, quant], ref[:, quant], what="quantized heads", tol=tol[:, quant])
    bar = exact_max_abs_bar(q, k, v, 128 ** -0.5, exact_q, ex)
    assert_close(out.numpy()[:, exact_q], ex[:, exact_q], max_abs=bar, what="exact heads")


def test_attention_with_and_without_v8_sums(module):
    """The P V products of INT8/INT4 tiles start from pack_v's -127 * sum(V8) (the Prefill path) or from
    two MFMAs against a constant operand (the reference-shaped call without sums), and INT4 key tiles read
    prepare_qk's expanded K4 records (the Prefill path) or expand the packed ones: the same integers, so
    the outputs of all four forms are bit-identical, and they match the oracle.  The expanded records
    are 16 times the K4 codes in the K8 layout, bit for bit."""
    print("\n[parity] attention with and without V8 sums and expanded K4 records", flush=True)
    q, k, v = small(3500, 2, 8, 2, 777)
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                         dtype=torch.int32)
    out, ops, pre = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    assert ops["v8sum"] is not None and ops["k4x"] is not None
    # the expanded records: K4 codes in the K8 layout, as bytes of 16 * code
    k4 = R.unpack_k4(ops["k4"].cpu().numpy())
    k4x = R.unpack_k8(ops["k4x"].cpu().numpy())
    assert k4.shape == k4x.shape == (2 * 2 * 13, 64, 128)
    np.testing.assert_array_equal(k4x.astype(np.int32), 16 * k4.astype(np.int32))
    table = next(iter(pre.tables.values()))
    pk = ops["packed"]
    for sums, wide in ((None, None), (ops["v8sum"], None), (None, ops["k4x"])):
        plain = torch.empty_like(out).cuda()
        module.attention(table.order, table.bands, None, None, pk[1], pk[2], pk[3], ops["vstat"], ops["q8"],
                         ops["kp"], ops["qa"], ops["ka"], ops["q4"], ops["k4"], ops["qa4"], ops["ka4"], plain,
                         128 ** -0.5, v8sum=sums, k4x=wide)
        torch.cuda.synchronize()
        assert torch.equal(out, plain.cpu()), (sums is not None, wide is not None)
    ref, _, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    assert_close(out.numpy(), ref, what="prefill with V8 sums", tol=tol)


NO_INT8 = [[0, INF], [0, 3], [0, 1], [0, 0], [1, INF], [INF, INF]]


@pytest.mark.parametrize("t", [200, 333])
def test_bands_without_int8_tiles(module, t):
    """w8 = 0: the INT4 list reaches the query tile itself, which the reference masks as the last entry
    of its pass (prefill_sm80.cu:328-329) after the fp16 pass has already visited it; t = 333 also masks
    keys past t in that tile.  All four kernel forms (V8 sums or not, expanded K4 records or not) give
    the same outputs, within the parity bar of the oracle."""
    print(f"\n[parity] prefill t={t} with w8 = 0 bands", flush=True)
    q, k, v = small(3600 + t, 1, 6, 2, t)
    bands = torch.tensor(NO_INT8, dtype=torch.int32)
    out, ops, pre = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    table = next(iter(pre.tables.values()))
    pk = ops["packed"]
    for sums, wide in ((None, None), (ops["v8sum"], None), (None, ops["k4x"])):
        plain = torch.empty_like(out).cuda()
        module.attention(table.order, table.bands, None, None, pk[1], pk[2], pk[3], ops["vstat"], ops["q8"],
                         ops["kp"], ops["qa"], ops["ka"], ops["q4"], ops["k4"], ops["qa4"], ops["ka4"], plain,
                         128 ** -0.5, v8sum=sums, k4x=wide)
        torch.cuda.synchronize()
        assert torch.equal(out, plain.cpu()), (sums is not None, wide is not None)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    compare_codes(ops, codes[0], 0, 1, 6, 2, t)
    assert_close(out.numpy(), ref, what=f"prefill w8 = 0 t={t}", tol=tol)


ODD_BANDS = [[4, 2], [0, 2], [5, 5], [0, 0]]


def test_unusual_bands(module):
    """Bands whose lists degenerate: w4 < w8 (no INT4 tiles), [0, 2] (one or two INT4 tiles ending at the
    query tile), [5, 5] (INT8 only) and [0, 0] (the two fp16 tiles only), batch 2, t = 257 (the last
    query tile holds one row); prefill and three decode steps against the oracle."""
    print("\n[parity] prefill t=257 batch 2 with unusual bands", flush=True)
    q, k, v = small(3700, 2, 4, 2, 257)
    bands = torch.tensor(ODD_BANDS, dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    for b in range(2):
        compare_codes(ops, codes[b], b, 2, 4, 2, 257)
    assert_close(out.numpy(), ref, what="prefill unusual bands", tol=tol)
    _decode_case(module, 257, bands, batch=2, steps=3, seed=5270, hq=4, hk=2)


@pytest.mark.parametrize("hq,hk,t", [(4, 4, 256), (8, 8, 130), (16, 2, 512)])
def test_prefill_group_sizes(module, hq, hk, t):
    """One q-head per KV head (the launch sequence's XCD rounds with groups of one: 4 x 4 query tiles
    fill two rounds of 8; 8 x 3 do not) and groups of 8, every band kind."""
    print(f"\n[parity] prefill hq {hq} hk {hk} t {t}", flush=True)
    q, k, v = small(3800 + hq + t, 1, hq, hk, t)
    kinds = [[INF, INF], [1, INF], [2, 4], [0, 3]]
    bands = torch.tensor([kinds[h % 4] for h in range(hq)], dtype=torch.int32)
    out, ops, _ = run_prefill(module, q, k, v, bands, 128 ** -0.5)
    ref, codes, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    compare_codes(ops, codes[0], 0, 1, hq, hk, t)
    assert_close(out.numpy(), ref, what=f"prefill hq {hq} hk {hk}", tol=tol)


def test_decode_bands_without_int8_tiles(module):
    """The decode side of w8 = 0 bands: the newest prompt tile is INT4 (or skipped for [0, 0])."""
    _decode_case(module, 333, torch.tensor(NO_INT8, dtype=torch.int32), steps=2, seed=5260)


def test_config2_shape_slice(module):
    """Config 2 recipe (Hq 28 / Hk 4, log-uniform channel scales, one bf16 KV head) at T = 1024, batch 1."""
    print("\n[parity] config 2 slice (B1 T1024)", flush=True)
    c = S.config2(batch=1, t=1024)
    bf16_kv = [h for h, kind in enumerate(c["kinds"]) if kind == "bf16"]
    out, ops, _ = run_prefill(module, c["q"], c["k"], c["v"], c["bands"], c["scale"], bf16_kv=bf16_kv)
    ref, codes, tol = oracle_prefill(c["q"], c["k"], c["v"], c["bands"], c["scale"])
    ex = exact_reference(c["q"], c["k"], c["v"], c["scale"])
    g = 7
    exact_q = [h for h in range(28) if h // g in bf16_kv]
    quant_q = [h for h in range(28) if h // g not in bf16_kv]
    compare_codes(ops, codes[0], 0, 1, 28, 4, 1024)
    assert_close(out.numpy()[:, quant_q], ref[:, quant_q], what="config 2 quantized heads", tol=tol[:, quant_q])
    bar = exact_max_abs_bar(c["q"], c["k"], c["v"], c["scale"], exact_q, ex)
    mx, _ = assert_close(out.numpy()[:, exact_q], ex[:, exact_q], max_abs=bar, what="config 2 exact heads")
    print(f"config2 exact heads: max abs {mx:.3e}, bar {bar:.3e} (fp32 SDPA vs float64)")


def test_shared_scratch_executors(module):
    """Calibration's pattern (calibrate.py:44-64): many Prefill executors with different uniform bands
    share one scratch dict and run one after another on the same layer inputs.  Each must match the
    oracle for its own bands, and return exactly what an executor with its own scratch returns."""
    print("\n[parity] shared-scratch Prefill executors", flush=True)
    from triattention_amd.maps import uniform
    hq, hk, t = 6, 2, 300
    qh, kh, vh = small(6100, 1, hq, hk, t)
    dev = torch.device("cuda")
    q, k, v = qh.to(dev), kh.to(dev), vh.to(dev)
    # a slice of calibrate.py:14-19's grid: sink/diagonal only, short and long INT8 bands, INT4 bands, all INT8
    configs = [(1, 1), (1, 2), (2, 8), (INF, INF), (1, INF), (4, 4), (16, INF), (2, 2048)]
    shared = {}
    outs = []
    for w8, w4 in configs:
        pre = Prefill(module, uniform(w8, w4), out_dtype=torch.float32)
        pre.buffers = shared
        outs.append(pre(0, q, k, v, 128 ** -0.5).clone())
    for (w8, w4), got in zip(configs, outs):
        bands = torch.tensor([[w8, w4]] * hq, dtype=torch.int32)
        ref, _, tol = oracle_prefill(qh, kh, vh, bands, 128 ** -0.5)
        assert_close(got.cpu().numpy(), ref, what=f"executor ({w8}, {w4}) with shared scratch", tol=tol)
    # fresh executors with their own scratch return the same bits
    for (w8, w4), first in zip(configs, outs):
        alone = Prefill(module, uniform(w8, w4), out_dtype=torch.float32)(0, q, k, v, 128 ** -0.5)
        assert torch.equal(first, alone), (w8, w4)
