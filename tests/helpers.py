"""Shared helpers of the parity tests: run the product path and the oracle on the same inputs."""
from __future__ import annotations

import numpy as np
import torch

import oracle as O
from triattention_amd.kernels import records as R
from triattention_amd.kernels.prefill import F16, I4, I8, Prefill
from triattention_amd.maps import from_bands
from triattention_amd.synthetic import bits

# attention-output tolerance of the parity gate (fp32 outputs vs the oracle)
MAX_ABS, MEAN_ABS = 2e-3, 1e-3


def bands_fn_of(bands: torch.Tensor, bf16_kv=None):
    table = {"0": bands.tolist()}
    return from_bands(table, bf16={"0": list(bf16_kv)} if bf16_kv else None)


def exact_reference(q, k, v, scale):
    """Causal attention of [B,Hq,T,128] bf16 inputs in float64 on the CPU (torch SDPA math): the
    mathematically exact result the bf16 heads are held to."""
    g = q.shape[1] // k.shape[1]
    kf = k.double().repeat_interleave(g, 1)
    vf = v.double().repeat_interleave(g, 1)
    return torch.nn.functional.scaled_dot_product_attention(q.double(), kf, vf, is_causal=True, scale=scale).numpy()


def exact_max_abs_bar(q, k, v, scale, heads, ref64):
    """Max-abs bar for exact (bf16) heads: 2e-3, or torch's own fp32 SDPA error against the float64
    result on the same inputs if that is larger (outputs of magnitude ~100 put fp32 SDPA itself
    above 2e-3).  The exact heads must be at least as accurate as fp32 SDPA."""
    g = q.shape[1] // k.shape[1]
    f32 = torch.nn.functional.scaled_dot_product_attention(
        q.float(), k.float().repeat_interleave(g, 1), v.float().repeat_interleave(g, 1), is_causal=True,
        scale=scale).numpy()
    return max(MAX_ABS, float(np.abs(f32[:, heads] - ref64[:, heads]).max()))


def run_prefill(module, q, k, v, bands, scale, decode_cache=None, out_dtype=torch.float32, bf16_kv=None):
    """Prefill on the GPU through the host operator; returns (out cpu, operand views)."""
    pre = Prefill(module, bands_fn_of(bands, bf16_kv), decode_cache, out_dtype=out_dtype)
    dev = torch.device("cuda")
    out = pre(0, q.to(dev), k.to(dev), v.to(dev), scale)
    torch.cuda.synchronize()
    ops = next(iter(pre.views.values()))
    return out.float().cpu(), ops, pre


def u32(a):
    return np.ascontiguousarray(a).view(np.uint32)


def compare_codes(ops, codes, b, batch, hq, hk, t, kept=None):
    """Assert bit equality of every GPU operand of sequence b with the oracle's."""
    tiles = (t + 63) // 64
    cpu = lambda x: x.detach().cpu().numpy()
    np.testing.assert_array_equal(cpu(ops["q8"])[b], codes["q8"])
    np.testing.assert_array_equal(u32(cpu(ops["qa"]).reshape(batch, hq * t)[b]), u32(codes["qa"]))
    if codes["q4"] is not None:
        np.testing.assert_array_equal(cpu(ops["q4"]).reshape(batch, hq, t, 64)[b], codes["q4"])
        np.testing.assert_array_equal(u32(cpu(ops["qa4"]).reshape(batch, hq * t)[b]), u32(codes["qa4"]))
    ka, kstat, vstat, ka4 = (ops["ka"], ops["kstat"], ops["vstat"], ops["ka4"]) if kept is None else kept
    np.testing.assert_array_equal(u32(cpu(kstat).reshape(batch, hk, 3, 128)[b]), u32(codes["kstat"]))
    np.testing.assert_array_equal(u32(cpu(vstat).reshape(batch, hk, 3, 128)[b]), u32(codes["vstat"]))
    np.testing.assert_array_equal(u32(cpu(ka).reshape(batch, hk, tiles, 4)[b]), u32(codes["ka"]))
    recs = cpu(ops["kp"]).reshape(batch, hk * tiles, 2048)[b]
    np.testing.assert_array_equal(R.unpack_k8(recs).reshape(hk, tiles * 64, 128), codes["k8"])
    if codes["k4"] is not None:
        np.testing.assert_array_equal(u32(cpu(ka4).reshape(batch, hk, tiles, 4)[b]), u32(codes["ka4"]))
        recs4 = cpu(ops["k4"]).reshape(batch, hk * tiles, 1024)[b]
        np.testing.assert_array_equal(R.unpack_k4(recs4).reshape(hk, tiles * 64, 128), codes["k4"])
    packed = ops["packed"]
    v16 = cpu(packed[F16]).reshape(batch, hk * tiles, 4096)[b]
    np.testing.assert_array_equal(R.unpack_v16(v16).reshape(hk, tiles * 64, 128), codes["v16"])
    if codes["v8"] is not None:
        v8 = cpu(packed[I8]).reshape(batch, hk * tiles, 2048)[b]
        np.testing.assert_array_equal(R.unpack_v8(v8).reshape(hk, tiles * 64, 128), codes["v8"])
    if codes["v4"] is not None:
        v4 = cpu(packed[I4]).reshape(batch, hk * tiles, 1024)[b]
        np.testing.assert_array_equal(R.unpack_v4(v4).reshape(hk, tiles * 64, 128), codes["v4"])


def oracle_prefill(q, k, v, bands, scale, decode_cache=False):
    """Per-sequence oracle outputs [B, Hq, T, 128], codes, and the per-element exp2-rounding bound
    [B, Hq, T, 128] that the prefill comparisons add to their bar: where a two-ulp change of a per-score
    exp2 (the kernels' hardware exp2, as the reference's ex2.approx) rounds a P level or an fp16
    probability to its neighbour, the output may move by up to that much; elsewhere it is 0."""
    outs, codes, tols = [], [], []
    for b in range(q.shape[0]):
        o, c, tl = O.prefill(bits(q[b]), bits(k[b]), bits(v[b]), bands.numpy(), scale, decode_cache=decode_cache,
                             tol=True)
        outs.append(o)
        codes.append(c)
        tols.append(tl)
    return np.stack(outs), codes, np.stack(tols)


# The prefill's exp2-rounding allowance (oracle_prefill's per-element bound ``tol``, zero for most
# elements): it may be present on at most TOL_FRAC_CAP of a check's elements, and at most RELY_FRAC_CAP
# of them (at least RELY_MIN) may actually need it, i.e. sit above the flat max-abs bar.
# Whatever the bound, no element may exceed the flat bar by more than USED_CAP (the largest excess
# measured over every prefill check of the GPU suite is 1.2e-3; over the 1,898 prefill checks of the
# sweep at TRI_SWEEP_SCALE=40, 4 exceed 1e-2, the largest by 4.35e-2, all inside their per-element
# bound).
TOL_FRAC_CAP = 0.05
RELY_FRAC_CAP = 1e-3
RELY_MIN = 2
USED_CAP = 1e-2


def sample_tokens(t, rng, extra=4):
    """Query rows sampled from a long prompt: the first and last tiles' edges, the middle, and ``extra``
    random rows."""
    fixed = [0, 1, 63, 64, 65, t // 2 - 1, t // 2, t - 1]
    return sorted(set([i for i in fixed if 0 <= i < t] + rng.integers(0, t, extra).tolist()))


def tol_budget(err, tol, max_abs, what):
    """Checks and reports how large and how common the exp2-rounding allowance of one prefill check is."""
    tol = np.asarray(tol, np.float64)
    assert np.isfinite(tol).all(), f"{what}: the exp2-rounding bound is not finite"
    frac = float((tol > 0).mean())
    rely = err > max_abs
    n_rely = int(rely.sum())
    used = float((err - max_abs)[rely].max()) if n_rely else 0.0
    print(f"[tol] {what}: bound on {frac:.3%} of {tol.size} elements (largest {float(tol.max()):.2e}); "
          f"{n_rely} elements above the flat bar use it (largest excess {used:.2e})", flush=True)
    assert frac <= TOL_FRAC_CAP, f"{what}: exp2-rounding bound on {frac:.2%} of the elements (cap {TOL_FRAC_CAP:.0%})"
    assert n_rely <= max(RELY_MIN, RELY_FRAC_CAP * tol.size), \
        f"{what}: {n_rely} of {tol.size} elements need the exp2-rounding allowance (cap {RELY_FRAC_CAP:.1%})"
    assert used <= USED_CAP, f"{what}: an element exceeds the flat bar by {used:.2e} (cap {USED_CAP:.0e})"


def assert_close_bf16(gpu, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what="", tol=None):
    """assert_close for a bf16 output: each element may also be off by the half ulp of bf16 rounding,
    at most |ref| * 2**-8 (8 significand bits)."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    allowed = max_abs + np.abs(ref) * 2.0 ** -8 + (0.0 if tol is None else np.asarray(tol, np.float64))
    assert np.isfinite(gpu).all(), f"{what}: non-finite output"
    if tol is not None:
        tol_budget(err, tol, max_abs + np.abs(ref) * 2.0 ** -8, what)
    worst = float((err - allowed).max())
    assert worst <= 0 and err.mean() <= mean_abs + float(np.abs(ref).mean()) * 2.0 ** -9, \
        f"{what}: max abs {err.max():.3e}, worst excess over the bf16 bar {worst:.3e}, mean abs {err.mean():.3e}"
    return float(err.max()), float(err.mean())


def assert_close(gpu, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what="", tol=None):
    """Max-abs and mean-abs bars; ``tol`` (prefill outputs: oracle_prefill's exp2-rounding bound) is
    added to the max-abs bar element by element."""
    err = np.abs(np.asarray(gpu, np.float64) - np.asarray(ref, np.float64))
    assert np.isfinite(np.asarray(gpu)).all(), f"{what}: non-finite output"
    if tol is not None:
        tol_budget(err, tol, max_abs, what)
    over = err - max_abs - (0.0 if tol is None else np.asarray(tol, np.float64))
    assert over.max() <= 0 and err.mean() <= mean_abs, \
        f"{what}: max abs {err.max():.3e} (<= {max_abs} + exp2-rounding bound), worst excess {over.max():.3e}, " \
        f"mean abs {err.mean():.3e} (<= {mean_abs})"
    return float(err.max()), float(err.mean())
