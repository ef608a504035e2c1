"""Tile-wise float64 evaluation of the quantized-P attention rules (test infrastructure).

An independent restatement, in numpy float64, of what the reference defines for
one prefill query row and for one decode q-head, written from the reference
source rather than from the C oracle:

  * band lists and visit order: prefill_sm80.cu:279-286 (F16 [0] or [0, qb],
    INT8 lo8..qb-1, INT4 lo4..qb-w8) and :460-465 (F16, then INT8, then INT4);
    only the visit of tile qb is masked (:455-457, :188-192);
  * scores in log2 units, slope RN(RN(qa*sm_log2)*ka_group): :297-298, :244-253;
  * per tile: row max, m' = max(m, tile), alpha = 2^(m - m') (:335-344);
  * F16 tiles: p = fp16(2^(s - m')), denom += sum p, acc += sum p * V16 (:358-383);
  * INT8 / INT4 tiles: base = tile + 0.75 * slope_max + |tile| * 2.4e-7
    (:255-257, :386-391), bq = 2^(base - m') / 255, P = floor(RN_{2^-8}(255 *
    2^(s - base) + 0.5)) (:78, :392-403), denom += bq * sum P, acc += bq * sum P * v8;
  * epilogue: out = acc / denom * scale_c + mean_c (:466-487);
  * decode (common_device.cuh:178-371, :373-469, kernels/decode.py:24-67): kept
    tiles per KV head by the group's states, each q-head scoring only its own,
    P = floor(RN_{2^-8}(levels * 2^(s - base) + (dot & 0xff) / 256)) with
    levels 255 (INT8 V) or 15 (INT4 V), INT4 V weighted by bq * 127 / 7, split
    partials (m, l, o) merged by log-sum-exp with the exact bf16 tail.

Every quantity is float64 except the fp32 values the reference itself defines
as fp32 inputs to the rules (the Q and K scale products).  Where the fp32
evaluation that the reference performs can land on either side of a rounding
boundary of the P quantizer, the level is "ambiguous" and is taken from the
oracle's record; every other level must agree exactly.
"""
from __future__ import annotations

import numpy as np

BN, D = 64, 128
MAGIC = 12582912.0  # 1.5 * 2^23, the reference's integer-to-float offset (prefill_sm80.cu:27)
FLT_MAX = float(np.finfo(np.float32).max)
U24 = 2.0 ** -24


def f32(x):
    return np.float32(x)


def ulp32(x):
    return np.spacing(np.abs(np.float32(x))).astype(np.float64)


def band_lists(w8: int, w4: int, qb: int):
    """(tile, kind) in visit order; kind 0 F16, 1 INT8, 2 INT4."""
    f16 = [0] if qb == 0 else [0, qb]
    lo8 = max(1, qb - w8 + 1)
    lo4 = max(1, qb - w4 + 1)
    return ([(j, 0) for j in f16] + [(j, 1) for j in range(lo8, qb)] +
            [(j, 2) for j in range(lo4, qb - w8 + 1)])


def unpack_q4(packed_row):
    b = packed_row.astype(np.int64)
    c = np.empty(D, np.int64)
    c[0::2] = ((b & 15) ^ 8) - 8
    c[1::2] = ((b >> 4) ^ 8) - 8
    return c


def levels_of(e_scaled, c):
    """floor(RN_{2^-8}(x + c)) for x = levels * 2^(s - base) (float64) and an offset c on the 2^-8 grid."""
    return np.floor((np.rint(e_scaled * 256.0) + np.rint(c * 256.0)) / 256.0).astype(np.int64)


def ambiguous(e_scaled, c, delta):
    """True where x + c lies within delta (absolute) of a point at which the 2^-8 rounding moves the
    floor: n - 2^-9 for integer n."""
    y = e_scaled + c
    frac = (y + 2.0 ** -9) - np.floor(y + 2.0 ** -9)
    dist = np.minimum(frac, 1.0 - frac)
    return dist <= delta + 2.0 ** -40


def fp16_ambiguous(p64, rel):
    """True where p64 lies within rel * p64 of a midpoint between adjacent fp16 values."""
    p16 = p64.astype(np.float16).astype(np.float64)
    nxt = np.nextafter(p64.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    prv = np.nextafter(p64.astype(np.float16), np.float16(0)).astype(np.float64)
    mid_up, mid_dn = (p16 + nxt) / 2, (p16 + prv) / 2
    d = np.minimum(np.abs(p64 - mid_up), np.abs(p64 - mid_dn))
    return d <= rel * np.abs(p64) + 2.0 ** -40


class Mismatch(AssertionError):
    pass


def check(cond, what):
    if not bool(np.all(cond)):
        raise Mismatch(what)


@np.errstate(over="ignore", invalid="ignore")
def prefill_row(codes, bands, hq, hk, t, sml, qh, i, trace):
    """Evaluate row (qh, i) in float64 and hold the oracle's record ``trace`` (prefill_trace) to it.
    Returns (float64 output, number of P levels compared, number ambiguous)."""
    g = hq // hk
    kh = qh // g
    qb = i // BN
    w8, w4 = int(bands[qh][0]), int(bands[qh][1])
    visits = band_lists(w8, w4, qb)
    check(len(visits) == len(trace["col"]), f"row ({qh},{i}): {len(trace['col'])} tiles visited, expected {len(visits)}")
    check(np.array_equal(trace["col"], [c for c, _ in visits]) and np.array_equal(trace["kind"], [k for _, k in visits]),
          f"row ({qh},{i}): visit order")
    row = qh * t + i
    qs8 = f32(f32(codes["qa"][row]) * sml)
    qs4 = f32(f32(codes["qa4"][row]) * sml) if codes["q4"] is not None else f32(0)
    q8 = codes["q8"][qh, i].astype(np.int64)
    q4 = unpack_q4(codes["q4"][qh, i]) if codes["q4"] is not None else None
    vmean, vscale = codes["vstat"][kh, 0].astype(np.float64), codes["vstat"][kh, 1].astype(np.float64)
    m, denom = -FLT_MAX, 0.0
    acc = np.zeros(D)
    compared = ambig = 0
    for e, (col, kind) in enumerate(visits):
        four = kind == 2
        keys = col * BN + np.arange(BN)
        valid = np.ones(BN, bool) if col != qb else (keys <= i) & (keys < t)
        kc = (codes["k4"] if four else codes["k8"])[kh, col * BN:(col + 1) * BN].astype(np.int64)
        dots = kc @ (q4 if four else q8)
        ks = (codes["ka4"] if four else codes["ka"])[kh, col]
        qs = qs4 if four else qs8
        slope = np.array([f32(qs * f32(ks[grp])) for grp in range(4)], np.float64)[np.arange(BN) // 16]
        s = slope * dots
        tile = float(s[valid].max()) if valid.any() else -np.inf
        m_new = max(m, tile)
        alpha = float(np.exp2(m - m_new))
        check(abs(float(trace["m"][e]) - m_new) <= 0.5 * ulp32(m_new), f"row ({qh},{i}) tile {col}: running max")
        m_o = float(trace["m"][e])
        if kind == 0:
            # fp16 probabilities relative to the running max
            # the reference's argument fma(slope, dot + 2^23*1.5, fma(-slope, 2^23*1.5, -m)): the inner fma
            # rounds once at the magnitude of slope * 1.5 * 2^23, the outer once at the result's
            arg_err = U24 * (np.abs(slope * MAGIC + m_o) + np.abs(s - m_o))
            # That error (~2^-12 relative at C0-like scales) exceeds half an fp16 step, so an fp16
            # probability is pinned to its float64 value within the two, and the recurrence below
            # takes the oracle's fp16 values.
            p64 = np.where(valid, np.exp2(s - m_o), 0.0)
            p_o = trace["p"][e].astype(np.uint16).view(np.float16).astype(np.float64)
            half16 = np.spacing(p64.astype(np.float16)).astype(np.float64) / 2
            bound = p64 * (np.log(2) * arg_err + 2 * U24) * 1.01 + half16 + 2.0 ** -26
            check(np.abs(p_o - p64) <= bound, f"row ({qh},{i}) tile {col}: fp16 probabilities")
            p = p_o
            v = codes["v16"][kh, col * BN:(col + 1) * BN].view(np.float16).astype(np.float64)
            denom = denom * alpha + p.sum()
            acc = acc * alpha + p @ v
        else:
            ksmax = f32(qs * f32(max(ks)))
            base = tile if tile > -np.inf else m_new
            base = base + 0.75 * float(ksmax) + abs(base) * 2.4e-7
            check(abs(float(trace["base"][e]) - base) <= 1.1 * ulp32(base), f"row ({qh},{i}) tile {col}: base")
            base_o = float(trace["base"][e])
            # (the exp2 of per-tile factors clamps its argument at -125: the reference's flush-to-zero
            # exp2 returns 0 there, the kernels and the oracle 2^-125; either is negligible)
            bq = float(np.exp2(max(base_o - m_o, -125.0))) / 255.0
            check(abs(float(trace["bq"][e]) - bq) <= 3 * ulp32(bq), f"row ({qh},{i}) tile {col}: bq")
            # levels from the oracle's base (checked above), so that only the P rule itself is compared
            x = np.where(valid, 255.0 * np.exp2(s - base_o), 0.0)
            # INT4: fma(slope, dot, -base), one rounding; INT8: the magic-offset form, two (as above)
            if four:
                arg_err = U24 * np.abs(s - base_o)
            else:
                arg_err = U24 * (np.abs(slope * MAGIC + base_o) + np.abs(s - base_o))
            amb = valid & ambiguous(x, 0.5, x * (np.log(2) * arg_err + 2 * U24))
            lev = levels_of(x, 0.5)
            p_o = trace["p"][e].astype(np.int64)
            check(np.array_equal(lev[~amb], p_o[~amb]), f"row ({qh},{i}) tile {col}: P levels "
                                                         f"{lev[~amb][lev[~amb] != p_o[~amb]][:4]} vs "
                                                         f"{p_o[~amb][lev[~amb] != p_o[~amb]][:4]}")
            P = np.where(amb, p_o, lev).astype(np.float64)
            compared += int(valid.sum())
            ambig += int(amb.sum())
            # the float64 recurrence from its own base and bq, with the levels compared above
            base64 = base
            bq64 = float(np.exp2(base64 - m_new)) / 255.0
            v8 = codes["v8"][kh, col * BN:(col + 1) * BN].astype(np.float64)
            denom = denom * alpha + bq64 * P.sum()
            acc = acc * alpha + bq64 * (P @ v8)
        m = m_new
    out = acc / denom * vscale + vmean if denom > 0 else vmean.copy()
    return out, compared, ambig


def decode_metadata(bands, hq, hk, prompt):
    """Per KV head: kept tiles (ascending), their K width (group maximum of the states) and, per q-head,
    whether the head owns the tile (kernels/decode.py:27-36)."""
    g = hq // hk
    tiles = (prompt + BN - 1) // BN

    def state(w8, w4, j):
        d = tiles - 1 - j
        return 8 if (j == 0 or d < w8) else (4 if d < w4 else 0)

    heads = []
    for kh in range(hk):
        st = np.array([[state(int(bands[kh * g + r][0]), int(bands[kh * g + r][1]), j) for j in range(tiles)]
                       for r in range(g)])
        kv = st.max(0)
        kept = np.nonzero(kv > 0)[0]
        heads.append(dict(tiles=kept, width=kv[kept], own=st[:, kept] > 0))
    return heads, tiles


@np.errstate(over="ignore", invalid="ignore")
def decode_head(codes, bands, hq, hk, prompt, sml, q_bits, splits_of, ktail_bits, vtail_bits, kcur_bits, vcur_bits,
                step, max_tail, qh, trace):
    """Evaluate one decode q-head in float64 and hold the oracle's record to it.  ``splits_of`` maps the
    KV head to its list of (first, last) entry ranges.  Returns (float64 output, compared, ambiguous)."""
    g = hq // hk
    kh = qh // g
    heads, tiles = decode_metadata(bands, hq, hk, prompt)
    h = heads[kh]
    bf = lambda b: (np.asarray(b, np.uint32) << 16).view(np.float32).astype(np.float64)
    # in-kernel Q quantization (common_device.cuh:291-315): rotated row, INT8 / INT4 codes, fp32 scales
    import oracle as O
    y = O.rotate(bf(q_bits[qh]).astype(np.float32)[None])[0]
    mq = f32(np.abs(y).max())
    if mq > 0:
        q8 = np.rint(y * f32(f32(127) / mq)).astype(np.int64)
        q4 = np.rint(y * f32(f32(7) / mq)).astype(np.int64)
        qsc, qsc4 = f32(f32(mq / f32(127)) * sml), f32(f32(mq / f32(7)) * sml)
    else:
        q8 = q4 = np.zeros(D, np.int64)
        qsc = qsc4 = f32(np.finfo(np.float32).tiny)
    q4 = ((q4 & 15) ^ 8) - 8
    vmean, vscale = codes["vstat"][kh, 0].astype(np.float64), codes["vstat"][kh, 1].astype(np.float64)
    kmean = codes["kstat"][kh, 0].astype(np.float64)
    compared = ambig = 0
    e_trace = 0
    parts = []
    for si, (first, last) in enumerate(splits_of(kh)):
        m, den = -FLT_MAX, 0.0
        acc = np.zeros(D)
        for e in range(first, last):
            j = int(h["tiles"][e])
            four = int(h["width"][e]) == 4
            vfmt8 = (tiles - 1 - j < 16) or j == 0
            levels = 255.0 if vfmt8 else 15.0
            check(int(trace["col"][e_trace]) == j and int(trace["split"][e_trace]) == si and
                  int(trace["kind"][e_trace]) == ((4 if four else 8) | (1 if vfmt8 else 2) << 4),
                  f"head {qh} entry {e}: tile, split or kind")
            keys = j * BN + np.arange(BN)
            valid = bool(h["own"][qh % g, e]) & (keys < prompt)
            kc = (codes["k4"] if four else codes["k8"])[kh, j * BN:(j + 1) * BN].astype(np.int64)
            dots = kc @ (q4 if four else q8)
            ks = (codes["ka4"] if four else codes["ka"])[kh, j]
            qs = qsc4 if four else qsc
            slope = np.array([f32(qs * f32(ks[grp])) for grp in range(4)], np.float64)[np.arange(BN) // 16]
            s = slope * dots
            tile = float(s[valid].max()) if valid.any() else -np.inf
            m_new = max(m, tile)
            alpha = float(np.exp2(m - m_new))
            check(abs(float(trace["m"][e_trace]) - m_new) <= 0.5 * ulp32(m_new), f"head {qh} tile {j}: running max")
            any_ = tile > -np.inf
            base = tile if any_ else m_new
            base = base + 0.75 * float(f32(qs * f32(max(ks)))) + abs(base) * 2.4e-7
            check(abs(float(trace["base"][e_trace]) - base) <= 1.1 * ulp32(base), f"head {qh} tile {j}: base")
            base_o = float(trace["base"][e_trace])
            m_o = float(trace["m"][e_trace])
            bq = float(np.exp2(max(base_o - m_o, -125.0))) / levels if any_ else 0.0
            check(abs(float(trace["bq"][e_trace]) - bq) <= 3 * ulp32(bq), f"head {qh} tile {j}: bq")
            x = np.where(valid, levels * np.exp2(s - base_o), 0.0)
            dither = np.where(valid, (dots & 0xFF) / 256.0, 0.0)
            # INT4: fma(slope, dot, -base); INT8: fma(slope, dot + 2^23*1.5, RN(RN(-slope * 2^23*1.5) - base)),
            # which rounds at the magnitude of slope * 1.5 * 2^23 twice
            if four:
                arg_err = U24 * np.abs(s - base_o)
            else:
                arg_err = U24 * (np.abs(slope) * MAGIC + np.abs(slope * MAGIC + base_o) + np.abs(s - base_o))
            amb = valid & ambiguous(x, dither, x * (np.log(2) * arg_err + 2 * U24))
            lev = levels_of(x, dither)
            p_o = trace["p"][e_trace].astype(np.int64)
            check(np.array_equal(lev[~amb], p_o[~amb]), f"head {qh} tile {j}: P levels")
            P = np.where(amb, p_o, lev).astype(np.float64)
            compared += int(np.sum(valid))
            ambig += int(amb.sum())
            bq64 = float(np.exp2(base - m_new)) / levels if any_ else 0.0
            restore = bq64 if vfmt8 else bq64 * 127.0 / 7.0
            vc = (codes["v8"] if vfmt8 else codes["v4"])[kh, j * BN:(j + 1) * BN].astype(np.float64)
            den = den * alpha + bq64 * P.sum()
            acc = acc * alpha + restore * (P @ vc)
            m = m_new
            e_trace += 1
        parts.append((m, den, acc))
    check(e_trace == len(trace["col"]), f"head {qh}: {len(trace['col'])} tiles visited, expected {e_trace}")
    for si, (m, den, acc) in enumerate(parts):
        check(abs(float(trace["pm"][si]) - m) <= 0.5 * ulp32(m), f"head {qh} split {si}: m")
    # merge with the exact bf16 tail (common_device.cuh:373-469)
    prior = min(step, max_tail - 1)
    qv = bf(q_bits[qh])
    tk = [bf(ktail_bits[kh, t]) for t in range(prior)] + [bf(kcur_bits[kh])]
    tv = [bf(vtail_bits[kh, t]) for t in range(prior)] + [bf(vcur_bits[kh])]
    ts = np.array([float(qv @ (k - kmean)) * float(sml) for k in tk])
    M = max([p[0] for p in parts] + list(ts))
    w = np.array([np.exp2(p[0] - M) for p in parts])
    l_ = sum(wi * p[1] for wi, p in zip(w, parts))
    o_ = sum(wi * p[2] for wi, p in zip(w, parts))
    et = np.exp2(ts - M)
    out = (o_ * vscale + l_ * vmean + et @ np.array(tv)) / (l_ + et.sum())
    return out, compared, ambig
