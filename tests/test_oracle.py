"""Pins of the CPU oracle against what the mathematics fixes (no GPU).

Each check is chosen so that a plausible mistake in the restatement (dropped
term, wrong sign or index, transposed operand, wrong rounding order) fails it:
float64 references, closed forms, independent numpy restatements with explicit
fp32 rounding, and invariants.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from triattention_amd import synthetic as S
from triattention_amd.synthetic import INF, bits

SIGNS = [0x9A3B5E71, 0x2C6D8F13, 0xE41B7A95, 0x5F02C3D8]
C = np.float32(0.08838834764831845)


def ulp_err(y, ref):
    y = np.asarray(y, np.float64)
    sp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(y - ref) / sp


# ------------------------------------------------------------------ exp2
def test_texp2_faithful_over_domain():
    rng = np.random.default_rng(0)
    x = np.concatenate([-rng.uniform(0, 125, 1_000_000), -rng.uniform(0, 1, 500_000),
                        -np.exp(rng.uniform(-30, 0, 200_000))]).astype(np.float32)
    y = O.texp2(x)
    ref = np.exp2(x.astype(np.float64))
    assert ulp_err(y, ref).max() <= 1.0


# exp2f of S. L. Moshier's Cephes Math Library (single precision): 2^x = 1 + x P(x) on [-0.5, 0.5],
# P's coefficients from the highest degree down, as published (decimal)
CEPHES_EXP2F_P = (1.535336188319500e-4, 1.339887440266574e-3, 9.618437357674640e-3, 5.550332471162809e-2,
                  2.402264791363012e-1, 6.931472028550421e-1)


def test_texp2_is_the_cephes_polynomial():
    """texp2's 2^f is the Cephes exp2f polynomial with its coefficients rounded to binary32, evaluated by
    fma in Horner order: the oracle's values equal that evaluation (fma emulated in float64, exact
    products; a double rounding may move a result by one ulp) on a dense sample of f in [-0.5, 0.5]."""
    f = np.linspace(-0.5, 0.5, 200_001).astype(np.float32)
    c = [np.float32(x) for x in CEPHES_EXP2F_P] + [np.float32(1.0)]
    p = np.full_like(f, c[0])
    for k in c[1:]:
        p = (p.astype(np.float64) * f.astype(np.float64) + np.float64(k)).astype(np.float32)
    y = O.texp2(f)
    diff = np.abs(y.view(np.int32).astype(np.int64) - p.view(np.int32).astype(np.int64))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.999
    # a different polynomial of the same degree (the Taylor coefficients ln2^k / k!) is told apart
    t = [np.float32(np.log(2) ** k / math.factorial(k)) for k in range(6, -1, -1)]
    q = np.full_like(f, t[0])
    for k in t[1:]:
        q = (q.astype(np.float64) * f.astype(np.float64) + np.float64(k)).astype(np.float32)
    assert (q != y).mean() > 0.1


def test_texp2_special_values():
    ks = np.arange(0, 126, dtype=np.float32)
    assert np.array_equal(O.texp2(-ks), np.ldexp(np.float32(1), -ks.astype(int)).astype(np.float32))
    assert O.texp2(np.float32([0.0]))[0] == 1.0
    lo = np.float32(2.0 ** -125)
    assert np.all(O.texp2(np.float32([-np.inf, -200.0, -125.0])) == lo)


def test_texp2_gpu_form_equals_rint_ldexp_form():
    """The kernels add n = rint(x) to the exponent field via the 1.5*2^23 shifter; a dense sample of
    every float pattern in [-200, 127] (stride 997) plus the specials must give identical bits."""
    pos = np.arange(0, np.float32(127.0).view(np.uint32) + 1, 997, dtype=np.uint32)
    neg = np.arange(0, np.float32(200.0).view(np.uint32) + 1, 997, dtype=np.uint32) | np.uint32(0x80000000)
    x = np.concatenate([pos, neg]).view(np.float32)
    x = np.concatenate([x, np.float32([-np.inf, np.inf, np.nan, -125.0, -124.5, -0.5, 0.5, 126.5, -0.0])])
    a, b = O.texp2(x).view(np.uint32), O.texp2_shifter(x).view(np.uint32)
    assert np.array_equal(a, b), x[a != b][:5]


# -------------------------------------------------------------- rotation
def walsh(i, j):
    return -1.0 if bin(i & j).count("1") % 2 else 1.0


def sign(c):
    return -1.0 if (SIGNS[c >> 5] >> (c & 31)) & 1 else 1.0


def test_rotation_basis_is_signed_scaled_walsh():
    m = O.rotate(np.eye(128, dtype=np.float32))  # row j = R e_j
    expect = np.array([[sign(j) * walsh(i, j) for i in range(128)] for j in range(128)], np.float64) * float(C)
    assert np.array_equal(m.astype(np.float64), expect.astype(np.float32).astype(np.float64))
    assert sum(bin(s).count("1") for s in SIGNS) == 66  # 66 sign-flipped channels


def test_rotation_orthogonal_and_odd():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    y = O.rotate(x)
    m = O.rotate(np.eye(128, dtype=np.float32)).astype(np.float64)
    assert np.abs(m @ m.T - np.eye(128)).max() < 1e-6
    assert np.array_equal(O.rotate(-x), -y)
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


def numpy_rotate(x):
    """Independent restatement: sign flip, butterflies over bits 0..6 with fp32 rounding per stage, scale."""
    s = np.array([sign(c) for c in range(128)], np.float32)
    y = (x * s).astype(np.float32)
    for bit in range(7):
        h = 1 << bit
        y = y.reshape(-1, 128 // (2 * h), 2, h)
        lo, hi = y[:, :, 0, :].copy(), y[:, :, 1, :].copy()
        y[:, :, 0, :] = (lo + hi).astype(np.float32)
        y[:, :, 1, :] = (lo - hi).astype(np.float32)
        y = y.reshape(-1, 128)
    return (y * C).astype(np.float32)


def test_rotation_bit_exact_vs_numpy_stage_order():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((256, 128)) * np.where(rng.random(128) < 0.03, 20, 1)).astype(np.float32)
    assert np.array_equal(O.rotate(x), numpy_rotate(x))


# ------------------------------------------------------------ quantizers
def rand_bf16(shape, seed):
    g = S.gen(seed)
    return S.outlier_tensor(g, 1, shape[0], shape[1])[0]


def test_quantize_q_invariants_and_numpy_restatement():
    x = rand_bf16((3, 70), 10)
    xb = bits(x)
    q8, qa, q4, qa4 = O.quantize_q(xb, int4=True)
    y = numpy_rotate(x.float().numpy().reshape(-1, 128))
    m = np.abs(y).max(1)
    inv = (np.float32(127) / m).astype(np.float32)
    codes = np.rint((y * inv[:, None]).astype(np.float32)).astype(np.int8)
    assert np.array_equal(q8.reshape(-1, 128), codes)
    assert np.array_equal(qa, (m / np.float32(127)).astype(np.float32))
    assert np.abs(q8).max() == 127 and (np.abs(q8.reshape(-1, 128)).max(1) == 127).all()
    inv4 = (np.float32(7) / m).astype(np.float32)
    c4 = np.rint((y * inv4[:, None]).astype(np.float32)).astype(np.int64)
    assert c4.min() >= -7 and c4.max() <= 7
    packed = ((c4[:, 0::2] & 15) | ((c4[:, 1::2] & 15) << 4)).astype(np.uint8)
    assert np.array_equal(q4.reshape(-1, 64), packed)
    assert np.array_equal(qa4, (m / np.float32(7)).astype(np.float32))
    assert (np.abs(y - codes * qa[:, None]) <= qa[:, None] * 0.5 * (1 + 1e-5)).all()


def test_quantize_q_zero_row():
    z = np.zeros((1, 2, 128), np.uint16)
    q8, qa, q4, qa4 = O.quantize_q(z, int4=True)
    assert not q8.any() and not qa.any() and not q4.any() and not qa4.any()


def test_stats_block_order_exact():
    x = rand_bf16((2, 333), 11)
    partial, stat = O.stats(bits(x))
    xf = x.float().numpy()  # [H, T, 128]
    h, t, _ = xf.shape
    sums = np.zeros((h, 64, 128), np.float32)
    for b in range(64):
        s = np.zeros((h, 128), np.float32)
        for tk in range(b, t, 64):
            s = (s + xf[:, tk]).astype(np.float32)
        sums[:, b] = s
    assert np.array_equal(partial[:, :, 0], sums)
    tot = np.zeros((h, 128), np.float32)
    for b in range(64):
        tot = (tot + sums[:, b]).astype(np.float32)
    mean = (tot / np.float32(t)).astype(np.float32)
    assert np.array_equal(stat[:, 0], mean)
    assert np.allclose(stat[:, 0], xf.astype(np.float64).mean(1), rtol=1e-5, atol=1e-6)
    rng_ = np.maximum(xf.max(1) - mean, mean - xf.min(1)).astype(np.float32)
    assert np.array_equal(stat[:, 1], (rng_ / np.float32(127)).astype(np.float32))
    assert np.array_equal(stat[:, 2], (np.float32(1) / stat[:, 1]).astype(np.float32))
    _, ident = O.stats(bits(x), identity=True)
    assert (ident[:, 0] == 0).all() and (ident[:, 1] == 1).all() and (ident[:, 2] == 1).all()


@pytest.mark.parametrize("t", [1, 63, 64, 65, 200])
def test_quantize_k_invariants(t):
    x = rand_bf16((2, t), 20 + t)
    _, kstat = O.stats(bits(x))
    k8, ka, k4, ka4 = O.quantize_k(bits(x), kstat, int4=True)
    tiles = (t + 63) // 64
    y = numpy_rotate((x.float().numpy() - kstat[:, 0][:, None, :]).astype(np.float32).reshape(-1, 128))
    y = y.reshape(2, t, 128)
    yp = np.zeros((2, tiles * 64, 128), np.float32)
    yp[:, :t] = y
    g = yp.reshape(2, tiles, 4, 16 * 128)
    cm = np.abs(g).max(-1)
    assert np.array_equal(ka, np.where(cm > 0, cm / np.float32(127), np.float32(1)).astype(np.float32))
    inv = np.where(cm > 0, np.float32(127) / np.where(cm > 0, cm, 1), 0).astype(np.float32)
    codes = np.rint((g * inv[..., None]).astype(np.float32)).astype(np.int8).reshape(2, tiles * 64, 128)
    assert np.array_equal(k8, codes)
    assert not k8[:, t:].any() and not k4[:, t:].any()
    assert k4.min() >= -7 and k4.max() <= 7
    nz = cm > 0
    assert (np.abs(k8.reshape(2, tiles, 4, -1)).max(-1)[nz] == 127).all()
    assert (np.abs(k4.reshape(2, tiles, 4, -1)).max(-1)[nz] == 7).all()


def test_pack_v_matches_numpy_conversions():
    x = rand_bf16((2, 150), 30)
    _, vstat = O.stats(bits(x))
    v16, v8, v4 = O.pack_v(bits(x), vstat)
    vn = ((x.float().numpy() - vstat[:, 0][:, None]).astype(np.float32) * vstat[:, 2][:, None]).astype(np.float32)
    full = np.zeros((2, 192, 128), np.float32)
    full[:, :150] = vn
    assert np.array_equal(v16, full.astype(np.float16).view(np.uint16))
    assert np.array_equal(v8, np.clip(np.rint(full), -127, 127).astype(np.int8))
    assert np.array_equal(v4, np.clip(np.rint((full * np.float32(7 / 127)).astype(np.float32)), -7, 7).astype(np.int8))
    assert np.abs(vn).max() <= 127.01


# ------------------------------------------------------------ band lists
@pytest.mark.parametrize("w8,w4", [(INF, INF), (1, INF), (2, 4), (3, 3), (1, 1), (5, 9), (2, INF)])
def test_band_lists_brute_force(w8, w4):
    for qb in range(0, 14):
        got = O.band_tiles(w8, w4, qb)
        f16 = [(0, 0)] + ([(qb, 0)] if qb > 0 else [])
        i8 = [(j, 1) for j in range(1, qb) if qb - j < w8]
        q4 = [(j, 2) for j in range(1, qb) if w8 <= qb - j < w4]
        assert got == f16 + i8 + q4


# ------------------------------------------------------------- attention
def dequant_reference(codes, bands, t, scale, hq, hk):
    """float64 softmax attention over the oracle's own dequantized operands, per visited tile kind."""
    sml = float(O.sm_log2(scale))
    g = hq // hk
    out = np.zeros((hq, t, 128))
    f16 = lambda a: a.view(np.float16).astype(np.float64)
    for h in range(hq):
        kh = h // g
        for i in range(t):
            ws, vs = [], []
            for col, kind in O.band_tiles(*bands[h], i // 64):
                keys = np.arange(col * 64, min(col * 64 + 64, i + 1))
                if kind == 2:
                    b = codes["q4"][h, i].astype(np.int64)
                    qc = np.empty(128, np.int64)
                    qc[0::2], qc[1::2] = ((b & 15) ^ 8) - 8, ((b >> 4) ^ 8) - 8
                    dots = codes["k4"][kh, keys].astype(np.int64) @ qc
                    s = codes["qa4"][h * t + i] * codes["ka4"][kh, col, (keys - col * 64) // 16] * dots
                else:
                    dots = codes["k8"][kh, keys].astype(np.int64) @ codes["q8"][h, i].astype(np.int64)
                    s = codes["qa"][h * t + i] * codes["ka"][kh, col, (keys - col * 64) // 16] * dots
                ws.append(s.astype(np.float64) * sml)
                vs.append(f16(codes["v16"][kh, keys]) if kind == 0 else codes["v8"][kh, keys].astype(np.float64))
            w = np.concatenate(ws)
            p = np.exp2(w - w.max())
            o = p @ np.concatenate(vs) / p.sum()
            out[h, i] = o * codes["vstat"][kh, 1] + codes["vstat"][kh, 0]
    return out


def test_prefill_close_to_dequantized_float64():
    g = S.gen(40)
    hq, hk, t = 4, 2, 150
    q, k, v = (S.outlier_tensor(g, 1, hq, t)[0], S.outlier_tensor(g, 1, hk, t)[0], S.outlier_tensor(g, 1, hk, t)[0])
    bands = np.array([[INF, INF], [1, INF], [2, 3], [1, 1]], np.int32)
    out, codes = O.prefill(bits(q), bits(k), bits(v), bands, 128 ** -0.5)
    ref = dequant_reference(codes, bands, t, 128 ** -0.5, hq, hk)
    err = np.abs(out - ref)
    # P is quantized to 8 bits per tile: small mean error, bounded worst case
    assert err.mean() < 5e-3 and err.max() < 1.0
    # rows of the first tile use fp16 probabilities only
    assert err[:, :64].max() < 0.05


def test_prefill_uniform_attention_when_q_is_zero():
    g = S.gen(41)
    hq, hk, t = 2, 1, 200
    q = torch.zeros(hq, t, 128, dtype=torch.bfloat16)
    k, v = S.outlier_tensor(g, 1, hk, t)[0], S.outlier_tensor(g, 1, hk, t)[0]
    bands = np.array([[INF, INF], [1, INF]], np.int32)
    out, codes = O.prefill(bits(q), bits(k), bits(v), bands, 128 ** -0.5)
    f16 = codes["v16"][0].view(np.float16).astype(np.float64)
    v8 = codes["v8"][0].astype(np.float64)
    for h in range(hq):
        for i in [0, 63, 64, 130, 199]:
            vals = []
            for col, kind in O.band_tiles(*bands[h], i // 64):
                keys = np.arange(col * 64, min(col * 64 + 64, i + 1))
                vals.append(f16[keys] if kind == 0 else v8[keys])
            ref = np.concatenate(vals).mean(0) * codes["vstat"][0, 1] + codes["vstat"][0, 0]
            assert np.abs(out[h, i] - ref).max() < 1e-3


def test_prefill_constant_v_returns_the_constant():
    g = S.gen(42)
    hq, hk, t = 2, 1, 130
    q, k = S.outlier_tensor(g, 1, hq, t)[0], S.outlier_tensor(g, 1, hk, t)[0]
    row = torch.randn(128, generator=g).to(torch.bfloat16)
    v = row[None, None, :].expand(hk, t, 128).contiguous()
    bands = np.array([[INF, INF], [1, INF]], np.int32)
    out, _ = O.prefill(bits(q), bits(k), bits(v), bands, 128 ** -0.5)
    assert np.abs(out - row.float().numpy()[None, None, :]).max() < 1e-5


# ---------------------------------------------------------------- decode
def _decode_setup(seed, prompt, bands, hq=4, hk=2):
    g = S.gen(seed)
    q, k, v = (S.outlier_tensor(g, 1, hq, prompt)[0], S.outlier_tensor(g, 1, hk, prompt)[0],
               S.outlier_tensor(g, 1, hk, prompt)[0])
    codes = O.prefill_codes(bits(q), bits(k), bits(v), bands, decode_cache=True)
    qd, kd, vd = (S.outlier_tensor(g, 1, hq, 1)[0, :, 0], S.outlier_tensor(g, 1, hk, 1)[0, :, 0],
                  S.outlier_tensor(g, 1, hk, 1)[0, :, 0])
    return codes, qd, kd, vd


def test_decode_split_invariance():
    bands = np.array([[INF, INF], [1, INF], [2, 5], [1, 1]], np.int32)
    codes, qd, kd, vd = _decode_setup(50, 900, bands)
    z = np.zeros((2, 4, 128), np.uint16)
    outs = [O.decode(codes, bands, bits(qd), 900, per, 128 ** -0.5, z, z, bits(kd), bits(vd), 0) for per in (1, 3, 100)]
    assert np.abs(outs[0] - outs[2]).max() < 1e-4 and np.abs(outs[1] - outs[2]).max() < 1e-4


def test_decode_bounds_reproduce_the_uniform_split():
    """Bounds [0, per, 2 per, ..., count] per head give the uniform split's bits; a different partition
    moves the output only by the partials' rounding."""
    bands = np.array([[INF, INF], [1, INF], [2, 5], [1, 1]], np.int32)
    prompt = 900
    codes, qd, kd, vd = _decode_setup(52, prompt, bands)
    z = np.zeros((2, 4, 128), np.uint16)
    run = lambda split: O.decode(codes, bands, bits(qd), prompt, split, 128 ** -0.5, z, z, bits(kd), bits(vd), 0)
    tiles = (prompt + 63) // 64
    count = [sum(max(O.decode_state(*bands[2 * h + r], tiles, j) for r in range(2)) > 0 for j in range(tiles))
             for h in range(2)]
    maxn = max(count)
    for per in (1, 3, 5, 64):
        splits = -(-maxn // per)
        bounds = np.array([[min(c, s * per) for s in range(splits + 1)] for c in count], np.int32)
        assert np.array_equal(run(bounds).view(np.uint32), run(per).view(np.uint32)), per
    # uneven runs, an empty split and the tail-heavy last split
    odd = np.array([[0, 2, 2, 9, count[0], count[0]], [0, 1, 7, 8, 10, count[1]]], np.int32)
    assert np.abs(run(odd) - run(100)).max() < 1e-4


def test_decode_close_to_dequantized_float64():
    """Decode keeps the tiles of each head's band, INT8/INT4 K by group maximum,
    INT8/INT4 V by recency, and the exact bf16 current token."""
    bands = np.array([[INF, INF], [INF, INF], [1, INF], [3, 6]], np.int32)
    prompt, hq, hk = 1300, 4, 2
    codes, qd, kd, vd = _decode_setup(51, prompt, bands)
    z = np.zeros((hk, 4, 128), np.uint16)
    out = O.decode(codes, bands, bits(qd), prompt, 2, 128 ** -0.5, z, z, bits(kd), bits(vd), 0)
    sml = float(O.sm_log2(128 ** -0.5))
    tiles = (prompt + 63) // 64
    g = hq // hk
    rot = O.rotate(qd.float().numpy())
    for h in range(hq):
        kh = h // g
        states = [[O.decode_state(*bands[kh * g + r], tiles, j) for j in range(tiles)] for r in range(g)]
        m = np.abs(rot[h]).max()
        q8 = np.rint((rot[h] * np.float32(np.float32(127) / m)).astype(np.float32))
        q4 = np.rint((rot[h] * np.float32(np.float32(7) / m)).astype(np.float32))
        ws, vs = [], []
        for j in range(tiles):
            own = states[h % g][j]
            kv = max(states[r][j] for r in range(g))
            if own == 0:
                continue
            keys = np.arange(j * 64, min(j * 64 + 64, prompt))
            if kv == 4:
                s = (m / 7) * codes["ka4"][kh, j, (keys - j * 64) // 16] * (codes["k4"][kh, keys] @ q4)
            else:
                s = (m / 127) * codes["ka"][kh, j, (keys - j * 64) // 16] * (codes["k8"][kh, keys] @ q8)
            vcode = codes["v8"] if O.lib().ora_decode_vfmt(tiles, j) == 1 else codes["v4"] * (127 / 7)
            ws.append(s * sml)
            vs.append(vcode[kh, keys].astype(np.float64) * codes["vstat"][kh, 1] + codes["vstat"][kh, 0])
        ts = float(qd[h].float().numpy() @ (kd[kh].float().numpy() - codes["kstat"][kh, 0])) * sml
        w = np.concatenate(ws + [[ts]])
        vv = np.concatenate(vs + [vd[kh].float().numpy()[None]])
        p = np.exp2(w - w.max())
        ref = p @ vv / p.sum()
        err = np.abs(out[h] - ref)
        assert err.mean() < 0.05 and err.max() < 2.0, (h, err.mean(), err.max())


def test_decode_tail_only_is_exact_attention_over_tail():
    """A head whose band keeps only the sink tile still sees the whole bf16 tail."""
    bands = np.array([[0, 0], [0, 0]], np.int32)
    hq, hk, prompt = 2, 1, 200
    codes, qd, kd, vd = _decode_setup(52, prompt, bands, hq=hq, hk=hk)
    g = S.gen(53)
    steps = 5
    kt = S.outlier_tensor(g, 1, hk, steps)[0]
    vt = S.outlier_tensor(g, 1, hk, steps)[0]
    ktail = np.zeros((hk, 8, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    ktail[:, :steps] = bits(kt)
    vtail[:, :steps] = bits(vt)
    out = O.decode(codes, bands, bits(qd), prompt, 4, 128 ** -0.5, ktail, vtail, bits(kd), bits(vd), steps)
    assert np.isfinite(out).all()
    # removing the sink tile's influence: compare against the quantized sink + exact tail in float64
    sml = float(O.sm_log2(128 ** -0.5))
    for h in range(hq):
        keys_t = np.concatenate([kt[0].float().numpy(), kd.float().numpy()])
        vals_t = np.concatenate([vt[0].float().numpy(), vd.float().numpy()])
        ts = (keys_t - codes["kstat"][0, 0]) @ qd[h].float().numpy() * sml
        rot = O.rotate(qd[h].float().numpy())
        m = np.abs(rot).max()
        q8 = np.rint((rot * np.float32(np.float32(127) / m)).astype(np.float32))
        s = (m / 127) * codes["ka"][0, 0, np.arange(64) // 16] * (codes["k8"][0, :64] @ q8) * sml
        w = np.concatenate([s, ts])
        vv = np.concatenate([codes["v8"][0, :64].astype(np.float64) * codes["vstat"][0, 1] + codes["vstat"][0, 0],
                             vals_t])
        p = np.exp2(w - w.max())
        ref = p @ vv / p.sum()
        assert np.abs(out[h] - ref).max() < 1.0 and np.abs(out[h] - ref).mean() < 0.05
