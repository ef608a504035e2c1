"""CPU oracle for TriAttention's quantized attention path (TEST INFRASTRUCTURE).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker: the product path in
``triattention_amd`` never routes through it.

The arithmetic lives in ``triatt_oracle.c`` (a restatement of the reference's
CUDA kernels, each function citing the reference lines it follows); this
module loads the gcc-built library with ctypes and exposes numpy-level
helpers.  bf16 tensors are passed as their raw uint16 bit patterns.

Host-side logic restated here in Python (closed-form integer code):
  * ``formats_for`` / ``identity_v``  -- kernels/prefill.py:20-26, :79-82, :91-93 and
    cuda/common_host.cuh:39 (which V records a Prefill call requests).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libtriatt_oracle.so"
INF = 1 << 20
D = 128
BN = 64


def build() -> Path:
    """Compile the C oracle with its Makefile (gcc, no fast-math)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        I, I64, F = ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.ora_texp2.restype = F
        L.ora_texp2.argtypes = [F]
        L.ora_texp2_batch.argtypes = [P, P, I64]
        L.ora_texp2_shifter_batch.argtypes = [P, P, I64]
        L.ora_rotate128.argtypes = [P]
        L.ora_f32_to_f16.restype = ctypes.c_uint16
        L.ora_f32_to_f16.argtypes = [F]
        L.ora_quantize_q.argtypes = [P, I64, I64, I, I, P, P, P, P]
        L.ora_stats.argtypes = [P, I64, I64, I, I, I, P, P]
        L.ora_quantize_k.argtypes = [P, I64, I64, I, I, P, P, P, P, P]
        L.ora_pack_v.argtypes = [P, I64, I64, I, I, P, P, P, P]
        L.ora_band_tiles.restype = I
        L.ora_band_tiles.argtypes = [I, I, I, P, P]
        L.ora_prefill.argtypes = [I, I, I, P, F, P, P, P, P, P, P, P, P, P, P, P, P, P, I]
        L.ora_decode_state.restype = I
        L.ora_decode_state.argtypes = [I, I, I, I]
        L.ora_decode_vfmt.restype = I
        L.ora_decode_vfmt.argtypes = [I, I]
        L.ora_decode.argtypes = [I, I, I, P, I, F, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I64, P, I, I, P]
        L.ora_num_threads.restype = I
        L.ora_set_mutation.argtypes = [I]
        L.ora_prefill_rows.argtypes = [I, I, I, P, F, P, P, P, P, P, P, P, P, P, P, P, P, I64, P, P, I]
        L.ora_prefill_trace.restype = I
        L.ora_prefill_trace.argtypes = [I, I, I, P, F, P, P, P, P, P, P, P, P, P, P, P, I, I, I, P, P, P, P, P, P, P]
        L.ora_decode_trace.restype = I
        L.ora_decode_trace.argtypes = [I, I, I, P, I, F, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I64, P, I, I,
                                       I, I, P, P, P, P, P, P, P, P, P, P, P]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def sm_log2(scale: float) -> np.float32:
    """f32(scale * log2 e), computed in double first (common_host.cuh:65)."""
    return np.float32(scale * 1.4426950408889634)


# ----------------------------------------------------------------- elementwise
def texp2(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().ora_texp2_batch(_p(x), _p(y), x.size)
    return y


def texp2_shifter(x):
    """texp2 in the GPU kernels' form (shifter + exponent-field add); equal to texp2 by construction."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().ora_texp2_shifter_batch(_p(x), _p(y), x.size)
    return y


def rotate(x):
    """Rotate every 128-vector of ``x`` (float32, last dim 128)."""
    x = _c(x, np.float32).copy()
    flat = x.reshape(-1, D)
    for i in range(flat.shape[0]):
        lib().ora_rotate128(_p(flat[i]))
    return x


def f32_to_f16_bits(x):
    x = _c(x, np.float32)
    f = np.vectorize(lambda v: lib().ora_f32_to_f16(float(v)), otypes=[np.uint16])
    return f(x)


# ------------------------------------------------------------------ quantizers
def quantize_q(q_bits, int4: bool):
    """q_bits uint16 [H, T, 128] -> q8 int8 [H,T,128], qa f32 [H*T], q4 u8 [H,T,64], qa4."""
    q = _c(q_bits, np.uint16)
    h, t, _ = q.shape
    q8 = np.empty((h, t, D), np.int8)
    qa = np.empty(h * t, np.float32)
    q4 = np.empty((h, t, D // 2), np.uint8) if int4 else None
    qa4 = np.empty(h * t, np.float32) if int4 else None
    lib().ora_quantize_q(_p(q), t * D, D, h, t, _p(q8), _p(qa), _p(q4), _p(qa4))
    return q8, qa, q4, qa4


def stats(x_bits, identity: bool = False):
    """-> partial f32 [H,64,3,128], stat f32 [H,3,128] (mean, scale, 1/scale)."""
    x = _c(x_bits, np.uint16)
    h, t, _ = x.shape
    partial = np.empty((h, 64, 3, D), np.float32)
    stat = np.empty((h, 3, D), np.float32)
    lib().ora_stats(_p(x), t * D, D, h, t, int(identity), _p(partial), _p(stat))
    return partial, stat


def quantize_k(k_bits, kstat, int4: bool):
    """-> k8 int8 [H, tiles*64, 128], ka f32 [H, tiles, 4], k4 int8 (signed codes) or None, ka4."""
    k = _c(k_bits, np.uint16)
    h, t, _ = k.shape
    tiles = (t + BN - 1) // BN
    kstat = _c(kstat, np.float32)
    k8 = np.empty((h, tiles * BN, D), np.int8)
    ka = np.empty((h, tiles, 4), np.float32)
    k4 = np.empty((h, tiles * BN, D), np.int8) if int4 else None
    ka4 = np.empty((h, tiles, 4), np.float32) if int4 else None
    lib().ora_quantize_k(_p(k), t * D, D, h, t, _p(kstat), _p(k8), _p(ka), _p(k4), _p(ka4))
    return k8, ka, k4, ka4


def pack_v(v_bits, vstat, want16=True, want8=True, want4=True):
    """-> v16 uint16 fp16 bits, v8 int8, v4 int8 (signed codes), each [H, tiles*64, 128] or None."""
    v = _c(v_bits, np.uint16)
    h, t, _ = v.shape
    tiles = (t + BN - 1) // BN
    vstat = _c(vstat, np.float32)
    shape = (h, tiles * BN, D)
    v16 = np.empty(shape, np.uint16) if want16 else None
    v8 = np.empty(shape, np.int8) if want8 else None
    v4 = np.empty(shape, np.int8) if want4 else None
    lib().ora_pack_v(_p(v), t * D, D, h, t, _p(vstat), _p(v16), _p(v8), _p(v4))
    return v16, v8, v4


# ------------------------------------------------------------- host-side logic
F16, I8, I4, Q4 = 1, 2, 3, 4


def band_tiles(w8: int, w4: int, qb: int):
    """Visit-order (tile, kind) list; kind 0=F16, 1=I8, 2=Q4 (prefill_sm80.cu:280-286, :460-465)."""
    cols = np.empty(4096, np.int32)
    kind = np.empty(4096, np.int32)
    n = lib().ora_band_tiles(int(w8), int(w4), int(qb), _p(cols), _p(kind))
    return list(zip(cols[:n].tolist(), kind[:n].tolist()))


def formats_for(bands, rows: int):
    """Formats a Prefill call needs from its band table (kernels/prefill.py:20-26)."""
    b = np.asarray(bands, dtype=np.int64).reshape(-1, 2)
    w8, w4 = b[:, :1], b[:, 1:]
    qb = np.arange(rows)[None, :]
    n8 = np.clip(qb - np.maximum(qb - w8 + 1, 1), 0, None)
    n4 = np.clip(qb - w8 - np.maximum(qb - w4 + 1, 1) + 1, 0, None)
    f = {F16}
    if (n8 > 0).any():
        f.add(I8)
    if (n4 > 0).any():
        f.add(Q4)
    return f


def decode_vcodes(rows: int):
    """V format per tile for the decode cache (kernels/decode.py:17-22)."""
    j = np.arange(rows)
    return np.where((rows - 1 - j < 16) | (j == 0), I8, I4)


# --------------------------------------------------------------------- prefill
def prefill_codes(q_bits, k_bits, v_bits, bands, decode_cache: bool = False):
    """The operand preparation of one Prefill call (kernels/prefill.py:87-101):
    which formats exist, the V identity rule, and every code/scale array.
    ``q_bits`` may be None (the Q codes are then omitted: a decode needs only K and V)."""
    t = k_bits.shape[1]
    rows = (t + BN - 1) // BN
    formats = formats_for(bands, rows)
    int4 = Q4 in formats
    if decode_cache:
        formats |= set(decode_vcodes(rows).tolist())
    want8 = I8 in formats or int4
    want4 = I4 in formats
    q8, qa, q4, qa4 = quantize_q(q_bits, int4) if q_bits is not None else (None,) * 4
    _, kstat = stats(k_bits)
    k8, ka, k4, ka4 = quantize_k(k_bits, kstat, int4)
    identity = not want8 and not want4
    _, vstat = stats(v_bits, identity=identity)
    v16, v8, v4 = pack_v(v_bits, vstat, True, want8, want4)
    return dict(q8=q8, qa=qa, q4=q4, qa4=qa4, kstat=kstat, k8=k8, ka=ka, k4=k4, ka4=ka4, vstat=vstat,
                v16=v16, v8=v8, v4=v4, int4=int4, formats=formats, identity=identity)


def prefill_attention(codes, bands, hq: int, hk: int, t: int, scale: float, threads: int = 0, tol: bool = False):
    """fp32 output [Hq, T, 128] of the banded quantized attention (prefill_sm80.cu:259-488).

    With ``tol``, also the per-element bound of how far the output moves where a two-ulp change of a
    per-score exp2 rounds a P level or an fp16 probability to its neighbour (the kernels' hardware
    exp2, like the reference's ex2.approx, may land on either side): returns (out, tol)."""
    b = _c(bands, np.int32).reshape(hq, 2)
    out = np.empty((hq, t, D), np.float32)
    bound = np.empty((hq, t, D), np.float32) if tol else None
    v8 = codes["v8"] if codes["v8"] is not None else np.zeros((1,), np.int8)
    lib().ora_prefill(hq, hk, t, _p(b), sm_log2(scale), _p(codes["q8"]), _p(codes["qa"]), _p(codes["q4"]),
                      _p(codes["qa4"]), _p(codes["k8"]), _p(codes["ka"]), _p(codes["k4"]), _p(codes["ka4"]),
                      _p(codes["v16"]), _p(v8), _p(codes["vstat"]), _p(out), _p(bound), int(threads))
    return (out, bound) if tol else out


def _prefill_operands(codes, bands, hq, scale):
    b = _c(bands, np.int32).reshape(hq, 2)
    v8 = codes["v8"] if codes["v8"] is not None else np.zeros((1,), np.int8)
    return (_p(b), sm_log2(scale), _p(codes["q8"]), _p(codes["qa"]), _p(codes["q4"]), _p(codes["qa4"]),
            _p(codes["k8"]), _p(codes["ka"]), _p(codes["k4"]), _p(codes["ka4"]), _p(codes["v16"]), _p(v8),
            _p(codes["vstat"])), (b, v8)


def prefill_rows(codes, bands, hq: int, hk: int, t: int, scale: float, rows, threads: int = 0, tol: bool = False):
    """Rows ``rows`` (flat q-head * t + token indices) of ``prefill_attention``'s output, [len(rows), 128]
    (with ``tol``: (out, tol) as for prefill_attention)."""
    rows = _c(rows, np.int64).reshape(-1)
    out = np.empty((rows.size, D), np.float32)
    bound = np.empty((rows.size, D), np.float32) if tol else None
    args, keep = _prefill_operands(codes, bands, hq, scale)
    lib().ora_prefill_rows(hq, hk, t, *args, _p(rows), rows.size, _p(out), _p(bound), int(threads))
    return (out, bound) if tol else out


def prefill_trace(codes, bands, hq: int, hk: int, t: int, scale: float, qh: int, i: int):
    """One output row with its per-tile record: dict(col, kind, m, base, bq, p [tiles, 64], out)."""
    cap = (t + BN - 1) // BN + 2
    col, kind = np.zeros(cap, np.int32), np.zeros(cap, np.int32)
    m, base, bq = np.zeros(cap, np.float32), np.zeros(cap, np.float32), np.zeros(cap, np.float32)
    p = np.zeros((cap, BN), np.int32)
    out = np.zeros(D, np.float32)
    args, keep = _prefill_operands(codes, bands, hq, scale)
    n = lib().ora_prefill_trace(hq, hk, t, *args, int(qh), int(i), cap, _p(col), _p(kind), _p(m), _p(base), _p(bq),
                                _p(p), _p(out))
    return dict(col=col[:n], kind=kind[:n], m=m[:n], base=base[:n], bq=bq[:n], p=p[:n], out=out)


def set_mutation(value: int) -> None:
    """Plant one of the oracle's test mistakes (0 = none); only the tests of the oracle's pins use it."""
    lib().ora_set_mutation(int(value))


MUTATIONS = dict(no_margin=1, no_half=2, dither_byte=3, no_rel_margin=4, bq_levels=5, v4_restore=6, no_dither=7,
                 slope_group=8, grown_mask=9, grown_state=10, exp_up=11, exp_down=12)


def prefill(q_bits, k_bits, v_bits, bands, scale: float, decode_cache: bool = False, threads: int = 0,
            tol: bool = False):
    """Whole Prefill call of one sequence: codes plus fp32 attention output (with ``tol``: output,
    codes and the exp2-rounding bound of prefill_attention)."""
    hq, t, _ = q_bits.shape
    hk = k_bits.shape[0]
    codes = prefill_codes(q_bits, k_bits, v_bits, bands, decode_cache)
    if tol:
        out, bound = prefill_attention(codes, bands, hq, hk, t, scale, threads, tol=True)
        return out, codes, bound
    return prefill_attention(codes, bands, hq, hk, t, scale, threads), codes


# ---------------------------------------------------------------------- decode
def decode_state(w8, w4, tiles, j):
    return lib().ora_decode_state(int(w8), int(w4), int(tiles), int(j))


def _operands(codes, grown):
    """The decode's code arrays: the prompt's, followed per KV head by the tiles taken from the tail
    (``grown``: tail_tile dicts, oldest first), and the tiles per head in them."""
    hk = codes["kstat"].shape[0]
    tiles = codes["k8"].shape[1] // BN
    grown = list(grown or [])
    if not grown:
        ops = {n: codes[n] for n in ("k8", "ka", "k4", "ka4", "v8", "v4")}
        return ops, tiles
    n = len(grown)
    cat = lambda name, prompt_part: np.ascontiguousarray(
        np.concatenate([prompt_part] + [t[name] for t in grown], axis=1))
    zeros = lambda: np.zeros((hk, tiles * BN, D), np.int8)
    ones = lambda: np.ones((hk, tiles, 4), np.float32)
    ops = dict(k8=cat("k8", codes["k8"]), ka=cat("ka", codes["ka"]),
               k4=cat("k4", codes["k4"] if codes["k4"] is not None else zeros()),
               ka4=cat("ka4", codes["ka4"] if codes["ka4"] is not None else ones()),
               v8=cat("v8", codes["v8"] if codes["v8"] is not None else zeros()),
               v4=np.concatenate([codes["v4"] if codes["v4"] is not None else zeros(),
                                  np.zeros((hk, n * BN, D), np.int8)], axis=1))
    return ops, tiles + n


def decode(codes, bands, q_bits, prompt: int, per, scale: float, ktail, vtail, kcur, vcur, step: int, grown=None):
    """fp32 output [Hq, 128] of one decode step of one sequence.

    ``codes`` holds the prompt's prefill operands (k8/ka/k4/ka4/v8/v4/kstat/vstat);
    q_bits [Hq,128], ktail/vtail [Hk,max_tail,128], kcur/vcur [Hk,128] are uint16 bf16 bits.
    ``per`` is the uniform split size (common_host.cuh:55), or an int [Hk, splits+1] array of
    per-head split bounds (the product's balanced partition, an extension).  ``step`` is the number
    of tokens the tail holds before this one.  ``grown`` (extension): the tiles taken from a full tail
    so far (tail_tile results, oldest first), which follow the prompt's tiles.
    """
    if np.ndim(per) == 0:
        bounds, nsplit, per = None, 0, int(per)
    else:
        bounds = _c(per, np.int32)
        nsplit, per = bounds.shape[1] - 1, 1
    hq = q_bits.shape[0]
    hk = codes["kstat"].shape[0]
    b = _c(bands, np.int32).reshape(hq, 2)
    out = np.empty((hq, D), np.float32)
    ktail = _c(ktail, np.uint16)
    vtail = _c(vtail, np.uint16)
    ops, ctiles = _operands(codes, grown)
    dummy = np.zeros((1,), np.int8)
    v4 = ops["v4"] if ops["v4"] is not None else dummy
    v8 = ops["v8"] if ops["v8"] is not None else dummy
    lib().ora_decode(hq, hk, int(prompt), _p(b), int(per), sm_log2(scale), _p(_c(q_bits, np.uint16)),
                     _p(ops["k8"]), _p(ops["ka"]), _p(ops["k4"]), _p(ops["ka4"]), _p(v8), _p(v4),
                     _p(codes["vstat"]), _p(codes["kstat"]), _p(ktail), _p(vtail), int(ktail.shape[1]),
                     _p(_c(kcur, np.uint16)), _p(_c(vcur, np.uint16)), int(step),
                     None if bounds is None else _p(bounds), int(nsplit), int(ctiles), _p(out))
    return out


def decode_trace(codes, bands, q_bits, prompt: int, per, scale: float, ktail, vtail, kcur, vcur, step: int,
                 qh: int, grown=None):
    """``decode`` for q-head ``qh`` with its record: per kept tile (split order) col, kind (K width 8/4 |
    V format << 4), split, m, base, bq, p [tiles, 64]; the split partials pm, pl, po [splits, 128]; out."""
    if np.ndim(per) == 0:
        bounds, nsplit, per = None, 0, int(per)
        splits = None
    else:
        bounds = _c(per, np.int32)
        nsplit, per = bounds.shape[1] - 1, 1
        splits = nsplit
    hq = q_bits.shape[0]
    b = _c(bands, np.int32).reshape(hq, 2)
    ops, ctiles = _operands(codes, grown)
    cap = max(1, ctiles)
    if splits is None:
        splits = max(1, -(-ctiles // per))
    col, kind, split = np.zeros(cap, np.int32), np.zeros(cap, np.int32), np.zeros(cap, np.int32)
    m, base, bq = np.zeros(cap, np.float32), np.zeros(cap, np.float32), np.zeros(cap, np.float32)
    p = np.zeros((cap, BN), np.int32)
    pm, pl, po = np.zeros(splits, np.float32), np.zeros(splits, np.float32), np.zeros((splits, D), np.float32)
    out = np.zeros(D, np.float32)
    ktail, vtail = _c(ktail, np.uint16), _c(vtail, np.uint16)
    dummy = np.zeros((1,), np.int8)
    v4 = ops["v4"] if ops["v4"] is not None else dummy
    v8 = ops["v8"] if ops["v8"] is not None else dummy
    q = _c(q_bits, np.uint16)
    kc, vc = _c(kcur, np.uint16), _c(vcur, np.uint16)
    n = lib().ora_decode_trace(hq, codes["kstat"].shape[0], int(prompt), _p(b), int(per), sm_log2(scale), _p(q),
                               _p(ops["k8"]), _p(ops["ka"]), _p(ops["k4"]), _p(ops["ka4"]), _p(v8), _p(v4),
                               _p(codes["vstat"]), _p(codes["kstat"]), _p(ktail), _p(vtail), int(ktail.shape[1]),
                               _p(kc), _p(vc), int(step), None if bounds is None else _p(bounds), int(nsplit),
                               int(ctiles), int(qh), cap, _p(col), _p(kind), _p(split), _p(m), _p(base), _p(bq),
                               _p(p), _p(pm), _p(pl), _p(po), _p(out))
    return dict(col=col[:n], kind=kind[:n], split=split[:n], m=m[:n], base=base[:n], bq=bq[:n], p=p[:n], pm=pm,
                pl=pl, po=po, out=out)


# ------------------------------------------------------------- tail growth
def tail_tile(k_bits, v_bits, kstat, vstat):
    """Codes of one tile taken from a full tail (extension): the 64 oldest tail rows k_bits / v_bits
    [Hk, 64, 128] (uint16 bf16 bits) quantized with the prompt's statistics, as the prompt's tiles
    are (INT8 and INT4 K with group scales, INT8 V)."""
    k8, ka, k4, ka4 = quantize_k(k_bits, kstat, True)
    _, v8, _ = pack_v(v_bits, vstat, want16=False, want8=True, want4=False)
    return dict(k8=k8, ka=ka, k4=k4, ka4=ka4, v8=v8)


class GrowingTail:
    """Decode of one sequence with tail growth (extension; the reference overwrites the tail's last
    slot once it holds max_tail tokens, common_device.cuh:384).  Before a step whose tail is full,
    its 64 oldest rows become a tile of the cache (tail_tile) and the rest move up by 64 slots; the
    step then attends over the prompt's tiles, the tiles taken so far and the tail, and appends its
    own k / v to the tail."""

    def __init__(self, codes, bands, prompt: int, max_tail: int):
        hk = codes["kstat"].shape[0]
        self.codes, self.bands, self.prompt, self.max_tail = codes, bands, int(prompt), int(max_tail)
        self.ktail = np.zeros((hk, max_tail, D), np.uint16)
        self.vtail = np.zeros((hk, max_tail, D), np.uint16)
        self.held = 0
        self.grown = []

    def step(self, q_bits, kcur, vcur, per, scale: float, compute: bool = True):
        """The fp32 output [Hq, 128] of one step (q_bits [Hq,128], kcur / vcur [Hk,128] bf16 bits); with
        ``compute`` False only the state moves on (None is returned)."""
        if self.max_tail >= BN and self.held >= self.max_tail:
            self.grown.append(tail_tile(self.ktail[:, :BN], self.vtail[:, :BN], self.codes["kstat"],
                                        self.codes["vstat"]))
            self.ktail[:, :self.max_tail - BN] = self.ktail[:, BN:].copy()
            self.vtail[:, :self.max_tail - BN] = self.vtail[:, BN:].copy()
            self.held -= BN
        out = decode(self.codes, self.bands, q_bits, self.prompt, per, scale, self.ktail, self.vtail, kcur, vcur,
                     self.held, grown=self.grown) if compute else None
        slot = min(self.held, self.max_tail - 1)
        self.ktail[:, slot] = _c(kcur, np.uint16)
        self.vtail[:, slot] = _c(vcur, np.uint16)
        self.held = slot + 1
        return out


def num_threads() -> int:
    return lib().ora_num_threads()
