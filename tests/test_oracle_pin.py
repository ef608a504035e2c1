"""The oracle's quantized-P attention pinned at the parity scale (no GPU).

``tests/tilewise.py`` evaluates the reference's rules (prefill_sm80.cu:244-487,
common_device.cuh:178-469) tile by tile in float64, independently of the C
oracle.  Against it, for every visited tile of every checked row or q-head:
the visit order, the running max (0.5 fp32 ulp), base (1.1 ulp), bq (3 ulp),
every P level and fp16 probability that is not within the fp32 evaluation's
error of a rounding boundary (exactly), and the output (2e-5 relative to the
row's magnitude).  The planted-mistake tests show that each plausible slip in
the P rules (dropped margin or its relative term, dropped +0.5, wrong dither
byte or none, bq over the wrong level count, missing INT4-V restore, one slope
for all key groups) fails these checks.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import tilewise as TW
from triattention_amd import synthetic as S
from triattention_amd.synthetic import INF, bits

SCALE = 128 ** -0.5
OUT_REL = 2e-5


def _inputs(seed, hq, hk, t):
    g = S.gen(seed)
    return (S.outlier_tensor(g, 1, hq, t)[0], S.outlier_tensor(g, 1, hk, t)[0], S.outlier_tensor(g, 1, hk, t)[0])


PREFILL_CASES = [
    # (seed, hq, hk, t, bands): sink/diagonal F16, INT8 and INT4 bands, partial last tile
    (61, 4, 2, 200, [[INF, INF], [1, INF], [2, 3], [1, 1]]),
    (62, 6, 2, 330, [[2, 4], [3, INF], [1, 2], [INF, INF], [1, INF], [4, 5]]),
]


def pin_prefill_rows(case, rows):
    seed, hq, hk, t, bands = case
    q, k, v = _inputs(seed, hq, hk, t)
    bands = np.array(bands, np.int32)
    codes = O.prefill_codes(bits(q), bits(k), bits(v), bands)
    sml = O.sm_log2(SCALE)
    compared = ambig = 0
    for qh, i in rows:
        tr = O.prefill_trace(codes, bands, hq, hk, t, SCALE, qh, i)
        out64, c, a = TW.prefill_row(codes, bands, hq, hk, t, sml, qh, i, tr)
        err = float(np.abs(tr["out"] - out64).max())
        TW.check(err <= OUT_REL * max(1.0, float(np.abs(out64).max())), f"row ({qh},{i}): output off by {err:.3e}")
        compared += c
        ambig += a
    return compared, ambig, codes


def _rows(case, stride):
    _, hq, _, t, _ = case
    return [(qh, i) for qh in range(hq) for i in range(0, t, stride)] + [(qh, t - 1) for qh in range(hq)]


@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_quantized_p_rules_tile_by_tile(case):
    compared, ambig, codes = pin_prefill_rows(case, _rows(case, 2))
    assert compared > 5000
    assert ambig <= 0.05 * compared, (ambig, compared)


def test_prefill_trace_row_equals_the_full_call_and_the_row_subset():
    """The traced row, the row-subset entry and the whole-layer call compute the same bits."""
    seed, hq, hk, t, bands = PREFILL_CASES[1]
    q, k, v = _inputs(seed, hq, hk, t)
    bands = np.array(bands, np.int32)
    codes = O.prefill_codes(bits(q), bits(k), bits(v), bands)
    full = O.prefill_attention(codes, bands, hq, hk, t, SCALE)
    rows = [(0, 0), (1, 63), (2, 64), (3, 200), (5, t - 1)]
    sub = O.prefill_rows(codes, bands, hq, hk, t, SCALE, [qh * t + i for qh, i in rows])
    for n, (qh, i) in enumerate(rows):
        tr = O.prefill_trace(codes, bands, hq, hk, t, SCALE, qh, i)
        assert np.array_equal(tr["out"].view(np.uint32), full[qh, i].view(np.uint32))
        assert np.array_equal(sub[n].view(np.uint32), full[qh, i].view(np.uint32))


DECODE_BANDS = np.array([[INF, INF], [INF, INF], [1, INF], [3, 6], [2, 2], [1, 1]], np.int32)


def _decode_setup(seed=63, prompt=1400, hq=6, hk=2, steps=3, max_tail=8):
    q, k, v = _inputs(seed, hq, hk, prompt)
    codes = O.prefill_codes(bits(q), bits(k), bits(v), DECODE_BANDS, decode_cache=True)
    g = S.gen(seed + 1)
    qd = bits(S.outlier_tensor(g, 1, hq, 1)[0, :, 0])
    kt = bits(S.outlier_tensor(g, 1, hk, max_tail)[0])
    vt = bits(S.outlier_tensor(g, 1, hk, max_tail)[0])
    kd, vd = bits(S.outlier_tensor(g, 1, hk, 1)[0, :, 0]), bits(S.outlier_tensor(g, 1, hk, 1)[0, :, 0])
    return codes, qd, kt, vt, kd, vd


def _uniform_splits(heads, per):
    maxn = max(1, max(len(h["tiles"]) for h in heads))
    splits = max(1, -(-maxn // per))
    return lambda kh: [(min(s * per, len(heads[kh]["tiles"])), min(s * per + per, len(heads[kh]["tiles"])))
                       for s in range(splits)]


def pin_decode(split, step):
    prompt, hq, hk, max_tail = 1400, 6, 2, 8
    codes, qd, kt, vt, kd, vd = _decode_setup(prompt=prompt, hq=hq, hk=hk, max_tail=max_tail)
    heads, _ = TW.decode_metadata(DECODE_BANDS, hq, hk, prompt)
    if np.ndim(split) == 0:
        splits_of = _uniform_splits(heads, int(split))
    else:
        splits_of = lambda kh: [(int(a), int(b)) for a, b in zip(split[kh][:-1], split[kh][1:])]
    sml = O.sm_log2(SCALE)
    compared = ambig = 0
    full = O.decode(codes, DECODE_BANDS, qd, prompt, split, SCALE, kt, vt, kd, vd, step)
    for qh in range(hq):
        tr = O.decode_trace(codes, DECODE_BANDS, qd, prompt, split, SCALE, kt, vt, kd, vd, step, qh)
        assert np.array_equal(tr["out"].view(np.uint32), full[qh].view(np.uint32))
        out64, c, a = TW.decode_head(codes, DECODE_BANDS, hq, hk, prompt, sml, qd, splits_of, kt, vt, kd, vd, step,
                                     max_tail, qh, tr)
        err = float(np.abs(tr["out"] - out64).max())
        TW.check(err <= OUT_REL * max(1.0, float(np.abs(out64).max())), f"head {qh}: output off by {err:.3e}")
        compared += c
        ambig += a
    return compared, ambig


@pytest.mark.parametrize("split, step", [(3, 0), (64, 5), ("bounds", 2), (1, 9)])
def test_decode_dithered_p_rules_tile_by_tile(split, step):
    if split == "bounds":
        # a caller's partition: uneven runs and an empty split per head
        prompt, hq, hk = 1400, 6, 2
        heads, _ = TW.decode_metadata(DECODE_BANDS, hq, hk, prompt)
        n = [len(h["tiles"]) for h in heads]
        split = np.array([[0, 2, 2, 9, n[0]], [0, 1, n[1] // 2, n[1], n[1]]], np.int32)
    compared, ambig = pin_decode(split, step)
    assert compared > 4000
    assert ambig <= 0.05 * compared, (ambig, compared)


PREFILL_MUTATIONS = ["no_margin", "no_half", "no_rel_margin", "bq_levels", "slope_group"]
DECODE_MUTATIONS = ["no_margin", "dither_byte", "no_rel_margin", "bq_levels", "v4_restore", "no_dither", "slope_group"]


@pytest.fixture
def planted():
    yield O.set_mutation
    O.set_mutation(0)


@pytest.mark.parametrize("name", PREFILL_MUTATIONS)
def test_planted_prefill_mistake_fails_the_pin(planted, name):
    planted(O.MUTATIONS[name])
    case = PREFILL_CASES[0]
    with pytest.raises(TW.Mismatch):
        pin_prefill_rows(case, _rows(case, 7))


@pytest.mark.parametrize("name", DECODE_MUTATIONS)
def test_planted_decode_mistake_fails_the_pin(planted, name):
    planted(O.MUTATIONS[name])
    with pytest.raises(TW.Mismatch):
        pin_decode(3, 2)


@pytest.mark.parametrize("seed,t", [(91, 700), (92, 333), (93, 129)])
def test_exp2_rounding_bound_covers_both_neighbours(seed, t):
    """The per-element bound the GPU prefill comparisons add to 2e-3: where a two-ulp change of a
    per-score exp2 rounds a P level or an fp16 probability to its neighbour, the output may move by at
    most ``tol``.  Pinned by moving every per-score exp2 two ulps up, then down (planted in the
    oracle): each run stays within tol of the unmoved output, and the bound is tight where it is
    not zero (some element moves by more than half its bound)."""
    hq, hk = 8, 2
    q, k, v = _inputs(seed, hq, hk, t)
    bands = np.array([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]], np.int32)
    out, codes, tol = O.prefill(bits(q), bits(k), bits(v), bands, SCALE, tol=True)
    assert np.isfinite(tol).all() and (tol >= 0).all()
    assert (tol > 0).any(), "the case should hold ambiguous probabilities"
    assert (tol == 0).mean() > 0.5, "most outputs are determined exactly"
    ratio = 0.0
    for name in ("exp_up", "exp_down"):
        O.set_mutation(O.MUTATIONS[name])
        try:
            moved = O.prefill_attention(codes, bands, hq, hk, t, SCALE)
        finally:
            O.set_mutation(0)
        diff = np.abs(moved.astype(np.float64) - out)
        slack = 1e-6 * (1.0 + np.abs(out))  # fp32 roundings of the unmoved terms
        assert (diff <= tol + slack).all(), f"{name}: max excess {(diff - tol - slack).max():.3e}"
        assert (diff[tol == 0] <= slack[tol == 0]).all()
        ratio = max(ratio, float((diff[tol > 0] / tol[tol > 0]).max()))
    assert ratio > 0.5, f"bound not tight: largest move {ratio:.2f} of it"
