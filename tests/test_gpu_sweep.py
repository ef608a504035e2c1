"""GPU parity over seeded random shapes: prefill codes bit-exact and outputs within the parity bar,
then a few decode steps against the oracle, for shapes the fixed cases do not pin -- every GQA group
size 1..8, prompt lengths around tile edges and in between, random (w8, w4) band pairs (w4 below w8
included), batches of 1-3, tails from 1 slot (every step overwrites it) to longer than the steps, and
uniform splits of 1..7 tiles or the cache's own partition; and ragged caches, prompts of different
lengths (sequences of 1 token included) stored one Prefill call at a time and decoded together; and
caches with tail growth and exact (bf16) KV heads over a few hundred steps (two to four spills of the
tail into the cache), quantized heads against the oracle's GrowingTail, exact heads against float64
attention over every raw key; and prefill with random exact (bf16) KV heads and a bf16 or fp32 output,
quantized heads against the oracle, exact heads against float64 attention.

Bar: as in test_gpu_parity (fp32 outputs within 2e-3 max-abs, 1e-3 mean-abs of the oracle)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O
from helpers import (assert_close, assert_close_bf16, compare_codes, exact_max_abs_bar, exact_reference, oracle_prefill,
                     run_prefill)
from test_gpu_parity import _attend64
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.synthetic import INF, bits

pytestmark = pytest.mark.gpu

# TRI_SWEEP_SCALE=n runs n times as many cases of each kind (the extra cases draw new seeds)
SCALE = max(1, int(os.environ.get("TRI_SWEEP_SCALE", "1")))
CASES = 40 * SCALE
RAGGED_CASES = 12 * SCALE
GROWTH_CASES = 8 * SCALE
EXACT_CASES = 12 * SCALE


def draw(i):
    """Case i: shape, bands and decode settings drawn from a generator seeded by i."""
    r = np.random.default_rng(9100 + i)
    g = int(r.integers(1, 9))
    hk = int(r.integers(1, 4 if g > 4 else 5))
    batch = int(r.integers(1, 4))
    if r.random() < 0.5:
        t = int(64 * r.integers(1, 8) + r.integers(-1, 2))
    else:
        t = int(r.integers(1, 520))
    choices8, choices4 = [1, 2, 3, 5, INF], [1, 2, 4, 7, INF]
    bands = [[int(r.choice(choices8)), int(r.choice(choices4))] for _ in range(g * hk)]
    return dict(g=g, hk=hk, hq=g * hk, batch=batch, t=t, bands=bands, steps=int(r.integers(1, 4)),
                max_tail=int(r.choice([1, 2, 5, 16])), per=[None, 1, 2, 7][int(r.integers(0, 4))])


@pytest.mark.parametrize("i", range(CASES))
def test_random_shape_prefill_and_decode(module, i):
    c = draw(i)
    hq, hk, batch, t = c["hq"], c["hk"], c["batch"], c["t"]
    print(f"\n[sweep] case {i}: batch={batch} hq={hq} hk={hk} t={t} bands={c['bands']} steps={c['steps']} "
          f"max_tail={c['max_tail']} per={c['per']}", flush=True)
    gen = S.gen(9200 + i)
    q, k, v = S.outlier_tensor(gen, batch, hq, t), S.outlier_tensor(gen, batch, hk, t), S.outlier_tensor(gen, batch, hk, t)
    bands = torch.tensor(c["bands"], dtype=torch.int32)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=c["max_tail"])
    cache.out_dtype = torch.float32
    cache.per = c["per"]
    out, ops, _ = run_prefill(module, q, k, v, bands, scale, decode_cache=cache)
    # (with a decode cache the V statistics are the prompt's own even where the prefill itself needs
    # no quantized V, common_host.cuh:39: the oracle is asked for the same)
    ref, _, tol = oracle_prefill(q, k, v, bands, scale, decode_cache=True)
    assert_close(out.numpy(), ref, what=f"case {i} prefill", tol=tol)
    codes = [O.prefill_codes(bits(q[b]), bits(k[b]), bits(v[b]), bands.numpy(), decode_cache=True)
             for b in range(batch)]
    e = cache.layers[0]
    kept = (e["ka"], e["kstat"], e["vstat"], e["ka4"])
    for b in range(batch):
        compare_codes(ops, codes[b], b, batch, hq, hk, t, kept=kept)
    ktail = np.zeros((batch, hk, c["max_tail"], 128), np.uint16)
    vtail = np.zeros_like(ktail)
    dev = torch.device("cuda")
    for step in range(c["steps"]):
        qd, kd, vd = S.outlier_tensor(gen, batch, hq, 1), S.outlier_tensor(gen, batch, hk, 1), S.outlier_tensor(gen, batch, hk, 1)
        got = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        for b in range(batch):
            want = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), t, cache.split_of(0, b), scale,
                            ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(got[b, :, 0], want, what=f"case {i} decode step {step} seq {b}")
            prior = min(step, c["max_tail"] - 1)
            ktail[b, :, prior] = bits(kd[b, :, 0])
            vtail[b, :, prior] = bits(vd[b, :, 0])
        cache.advance()


@pytest.mark.parametrize("i", range(RAGGED_CASES))
def test_random_ragged_cache_decode(module, i):
    r = np.random.default_rng(9500 + i)
    c = draw(100 + i)
    hq, hk, max_tail = c["hq"], c["hk"], c["max_tail"]
    prompts = [int(r.choice([1, 2, 63, 64, 65])) if r.random() < 0.3 else int(r.integers(1, 900))
               for _ in range(int(r.integers(2, 6)))]
    print(f"\n[sweep] ragged case {i}: prompts={prompts} hq={hq} hk={hk} bands={c['bands']} steps={c['steps']} "
          f"max_tail={max_tail} per={c['per']}", flush=True)
    bands = torch.tensor(c["bands"], dtype=torch.int32)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.ragged = True
    cache.out_dtype = torch.float32
    cache.per = c["per"]
    gen = S.gen(9600 + i)
    codes = []
    for n in prompts:
        q, k, v = S.outlier_tensor(gen, 1, hq, n), S.outlier_tensor(gen, 1, hk, n), S.outlier_tensor(gen, 1, hk, n)
        run_prefill(module, q, k, v, bands, scale, decode_cache=cache)
        codes.append(O.prefill_codes(bits(q[0]), bits(k[0]), bits(v[0]), bands.numpy(), decode_cache=True))
    nb = len(prompts)
    ktail = np.zeros((nb, hk, max_tail, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    dev = torch.device("cuda")
    for step in range(c["steps"]):
        qd, kd, vd = S.outlier_tensor(gen, nb, hq, 1), S.outlier_tensor(gen, nb, hk, 1), S.outlier_tensor(gen, nb, hk, 1)
        got = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale).float().cpu().numpy()
        for b, n in enumerate(prompts):
            want = O.decode(codes[b], bands.numpy(), bits(qd[b, :, 0]), n, cache.split_of(0, b), scale, ktail[b],
                            vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step)
            assert_close(got[b, :, 0], want, what=f"ragged case {i} step {step} seq {b} (prompt {n})")
            prior = min(step, max_tail - 1)
            ktail[b, :, prior] = bits(kd[b, :, 0])
            vtail[b, :, prior] = bits(vd[b, :, 0])
        cache.advance()


@pytest.mark.parametrize("i", range(GROWTH_CASES))
def test_random_tail_growth_with_exact_heads(module, i):
    r = np.random.default_rng(9700 + i)
    c = draw(200 + i)
    g = c["g"]
    hk = max(2, c["hk"])
    hq = g * hk
    bands = torch.tensor((c["bands"] * 2)[:hq], dtype=torch.int32)
    bf16_kv = sorted(int(h) for h in r.choice(hk, size=int(r.integers(0, hk)), replace=False))
    max_tail = int(r.choice([64, 65, 100, 128]))
    steps = int(r.integers(2 * max_tail + 10, 4 * max_tail + 20))
    prompts = [int(r.integers(1, 700)) for _ in range(int(r.integers(1, 4)))]
    print(f"\n[sweep] growth case {i}: prompts={prompts} hq={hq} hk={hk} exact={bf16_kv} max_tail={max_tail} "
          f"steps={steps}", flush=True)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail, grow_tail=steps)
    cache.ragged = len(prompts) > 1
    cache.out_dtype = torch.float32
    gen = S.gen(9800 + i)
    seqs, raw = [], []
    for n in prompts:
        q, k, v = S.outlier_tensor(gen, 1, hq, n), S.outlier_tensor(gen, 1, hk, n), S.outlier_tensor(gen, 1, hk, n)
        run_prefill(module, q, k, v, bands, scale, decode_cache=cache, bf16_kv=bf16_kv)
        codes = O.prefill_codes(None, bits(k[0]), bits(v[0]), bands.numpy(), decode_cache=True)
        seqs.append(O.GrowingTail(codes, bands.numpy(), n, max_tail))
        kr, vr = torch.zeros(hk, n + steps, 128), torch.zeros(hk, n + steps, 128)
        kr[:, :n], vr[:, :n] = k[0].float(), v[0].float()
        raw.append((kr, vr, n))
    exact_q = [h for h in range(hq) if h // g in bf16_kv]
    quant_q = [h for h in range(hq) if h // g not in bf16_kv]
    dev = torch.device("cuda")
    nb = len(prompts)
    for t in range(steps):
        qd, kd, vd = S.outlier_tensor(gen, nb, hq, 1), S.outlier_tensor(gen, nb, hk, 1), S.outlier_tensor(gen, nb, hk, 1)
        out = cache(0, qd.to(dev), kd.to(dev), vd.to(dev), scale)
        check = t % 23 == 0 or seqs[0].held >= max_tail - 1 or t == steps - 1
        if check:
            out = out.cpu().numpy()
        for b in range(nb):
            want = seqs[b].step(bits(qd[b, :, 0]), bits(kd[b, :, 0]), bits(vd[b, :, 0]), cache.split_of(0, b), scale,
                                compute=check)
            kr, vr, p = raw[b]
            kr[:, p + t], vr[:, p + t] = kd[b, :, 0].float(), vd[b, :, 0].float()
            if check:
                if quant_q:
                    assert_close(out[b, quant_q, 0], want[quant_q], what=f"growth case {i} step {t} seq {b} quantized")
                if exact_q:
                    r64, r32 = _attend64(qd[b, :, 0], kr[:, :p + t + 1], vr[:, :p + t + 1], scale)
                    bar = max(2e-3, float(np.abs(r32[exact_q] - r64[exact_q]).max()))
                    assert_close(out[b, exact_q, 0], r64[exact_q], max_abs=bar,
                                 what=f"growth case {i} step {t} seq {b} exact")
        cache.advance()
    assert cache.layers[0]["store"].tb >= 64


@pytest.mark.parametrize("i", range(EXACT_CASES))
def test_random_prefill_with_exact_heads(module, i):
    r = np.random.default_rng(9900 + i)
    c = draw(300 + i)
    g, hk, batch = c["g"], max(2, c["hk"]), c["batch"]
    hq = g * hk
    t = int(r.integers(1, 1500))
    bands = torch.tensor((c["bands"] * 2)[:hq], dtype=torch.int32)
    bf16_kv = sorted(int(h) for h in r.choice(hk, size=int(r.integers(1, hk + 1)), replace=False))
    out_dtype = torch.bfloat16 if r.random() < 0.5 else torch.float32
    print(f"\n[sweep] exact case {i}: batch={batch} hq={hq} hk={hk} t={t} exact={bf16_kv} out={out_dtype}", flush=True)
    gen = S.gen(9950 + i)
    q, k, v = S.outlier_tensor(gen, batch, hq, t), S.outlier_tensor(gen, batch, hk, t), S.outlier_tensor(gen, batch, hk, t)
    scale = 128 ** -0.5
    out, _, _ = run_prefill(module, q, k, v, bands, scale, out_dtype=out_dtype, bf16_kv=bf16_kv)
    out = out.numpy()
    exact_q = [h for h in range(hq) if h // g in bf16_kv]
    quant_q = [h for h in range(hq) if h // g not in bf16_kv]
    close = assert_close_bf16 if out_dtype == torch.bfloat16 else assert_close
    if quant_q:
        ref, _, tol = oracle_prefill(q, k, v, bands, scale)
        close(out[:, quant_q], ref[:, quant_q], what=f"exact case {i} quantized heads", tol=tol[:, quant_q])
    ex = exact_reference(q, k, v, scale)
    bar = exact_max_abs_bar(q, k, v, scale, exact_q, ex)
    close(out[:, exact_q], ex[:, exact_q], max_abs=bar, what=f"exact case {i} exact heads")
