"""Loader and torch-facing binding of the gfx950 kernel library.

Replaces triattention/kernels/extension.py (which JIT-built the CUDA sources
with nvcc).  Here the kernels are prebuilt in-tree by ``build()`` into
``triattention_amd/_lib/libtriattention_amd.so`` (hipcc, gfx950) and loaded with
ctypes.  ``load_extension()`` returns a module object whose five ops keep the
names, argument order and in-place semantics of the reference's pybind module
(cuda/common_host.cuh:96-102); tensors are handed to the C ABI
(include/triattention_amd.h) as device pointers with sizes and strides, and
every op runs on the current torch stream.  Argument errors raise
RuntimeError, as TORCH_CHECK did in the reference.

Extensions over the reference signatures (batch = 1 is exactly the reference):
  * a leading batch dimension on every tensor;
  * ``attention`` also accepts an fp32 ``out`` (parity testing);
  * ``attention`` computes the q-heads flagged in ``exact`` as exact bf16
    attention over records written by ``pack_exact`` (maps that keep some KV
    heads unquantized);
  * ``decode`` takes ragged batches: ``prompt`` may be a device int32 tensor of
    per-sequence lengths, with per-sequence metadata rows.
"""
from __future__ import annotations

import ctypes
import functools
import subprocess
import weakref
from pathlib import Path

import torch

PACKAGE = Path(__file__).resolve().parent.parent
CSRC = PACKAGE / "csrc"
LIBRARY = PACKAGE / "_lib" / "libtriattention_amd.so"
D = 128
STAT_BLOCKS = 64
K8_WORDS, K4_WORDS, V16_WORDS, V8_WORDS, V4_WORDS = 2048, 1024, 4096, 2048, 1024

EXPORTS = ("tri_last_error", "tri_prepare_qk", "tri_pack_v", "tri_attention", "tri_pack_exact", "tri_decode",
           "tri_decode_partials", "tri_decode_merge", "tri_decode_short_tail", "tri_decode_merge_short_tail",
           "tri_decode_partials_timed", "tri_decode_noalloc",
           "tri_decode_tasks", "tri_cache_store", "tri_tail_spill", "tri_decode_occupancy", "tri_device_cus",
           "tri_stream_read", "tri_issue_probe", "tri_prefill_pairs")
KX_BYTES = 16384
TASK_WORDS = 512  # int32 words of the decode task table per (sequence, KV head, split)


def build(arch: str = "gfx950") -> Path:
    """Compile every HIP kernel of the package into the in-tree shared library."""
    subprocess.run(["make", "-s", "-C", str(CSRC), f"ARCH={arch}"], check=True)
    return LIBRARY


def load_library() -> ctypes.CDLL:
    """dlopen the kernel library and declare its C ABI (no GPU needed)."""
    if not LIBRARY.exists():
        raise RuntimeError(f"TriAttention kernel library missing: {LIBRARY} (run triattention_amd.kernels.extension.build())")
    lib = ctypes.CDLL(str(LIBRARY))
    P, I, I64, D_ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
    lib.tri_last_error.restype = ctypes.c_char_p
    lib.tri_last_error.argtypes = []
    lib.tri_prepare_qk.argtypes = [P, I64, I64, I64, P, I64, I64, I64, I, I, I, I,
                                   P, P, P, P, P, P, P, P, P, P, P, P]
    lib.tri_pack_v.argtypes = [P, I64, I64, I64, I, I, I, P, P, P, P, P, P, P]
    lib.tri_attention.argtypes = [P, I, P, I, I, I, I, P, P, P, P, P, P, P, P, P, P, P, P, I, I64, I64, I64, D_,
                                  P, P, I64, I64, I64, P, P, I, P, P, P]
    lib.tri_pack_exact.argtypes = [P, I64, I64, I64, P, I64, I64, I64, I, I, I, I, P, I, P, P, P]
    decode_args = [P, I64, I64, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I,
                   P, P, I64, I64, P, P, I, I64, I64, P, P, P, P, I, I, I, I, I, I, I64, I64, I64, I64,
                   P, P, P, I64, P, I, P, I, P, D_, P]
    for name in ("tri_decode", "tri_decode_partials", "tri_decode_merge", "tri_decode_short_tail",
                 "tri_decode_merge_short_tail"):
        getattr(lib, name).argtypes = decode_args
    lib.tri_decode_partials_timed.argtypes = decode_args + [P, P]
    # tri_decode without pm / pl / po (arguments 31-33 of tri_decode)
    lib.tri_decode_noalloc.argtypes = decode_args[:31] + decode_args[34:]
    lib.tri_decode_tasks.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P, I, P, I, P, P]
    lib.tri_cache_store.argtypes = [P, P, I, I, I, I, I, I, P, P, P, P, P, P, P, P, P, P, I, I, I, I, P, P, P, P, P, P,
                                    P, P, P, P, P, P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, P, I64, I64,
                                    P]
    lib.tri_tail_spill.argtypes = [P, P, P, P, I64, I64, I64, I, I, I, I, I, P, I, P, P, P, P, P, P, P, P, P, P, P,
                                   P, P, I64, P, I64, P, I64, P, P, I64, P, I, P]
    lib.tri_decode_occupancy.argtypes = [ctypes.POINTER(ctypes.c_int)]
    lib.tri_device_cus.argtypes = [ctypes.POINTER(ctypes.c_int)]
    lib.tri_stream_read.argtypes = [P, I64, I, I, I, P, P]
    lib.tri_issue_probe.argtypes = [I, I, I, P, P]
    lib.tri_prefill_pairs.argtypes = [I]
    for name in EXPORTS:
        if name != "tri_last_error":
            getattr(lib, name).restype = ctypes.c_int
    return lib


def arch() -> str:
    if not torch.cuda.is_available():
        raise RuntimeError("TriAttention requires an AMD Instinct GPU (ROCm); none is visible.")
    name = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if name != "gfx950":
        raise RuntimeError(f"TriAttention kernels are built for gfx950 (MI355X); found {name}.")
    return name


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Module:
    """The op set of the reference's extension module, on the gfx950 kernels."""

    PLAN_CACHE = 256  # decode plans kept for callers of the reference-shaped ``decode`` (one per layer)

    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib
        self._plans = {}

    def _call(self, fn, *args):
        if fn(*args) != 0:
            raise RuntimeError(self.lib.tri_last_error().decode())

    @staticmethod
    def _stream(device) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)

    # -------------------------------------------------------------- prepare_qk
    def prepare_qk(self, q, k, q8, qa, kp, ka, partial, kstat, q4=None, qa4=None, k4p=None, ka4=None, k4x=None):
        """Per-token INT8 (and INT4) Q and centred per-block INT8 (and INT4) K operands.

        Extension: ``k4x`` (uint32, as many words as ``kp``, with the INT4 buffers) receives the K4 records
        expanded to 16 * code bytes in the K8 layout, which ``attention(..., k4x=...)`` reads."""
        _check(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 4 and q.size(3) == D and q.stride(3) == 1 and
               k.dtype == torch.bfloat16 and k.dim() == 4 and k.size(0) == q.size(0) and k.size(2) == q.size(2) and
               k.size(3) == D and k.stride(3) == 1, "BF16 Q/K [B,H,T,128] with contiguous features")
        b, hq, t, _ = q.shape
        hk = k.size(1)
        tiles = (t + 63) // 64
        _check(q8.numel() == b * hq * t * D and qa.numel() == b * hq * t and kp.numel() == b * hk * tiles * K8_WORDS and
               ka.numel() == b * hk * tiles * 4 and partial.numel() >= b * hk * STAT_BLOCKS * 3 * D and
               kstat.numel() == b * hk * 3 * D, "Q/K buffers")
        int4 = q4 is not None
        _check(int4 == (qa4 is not None) == (k4p is not None) == (ka4 is not None) and
               (not int4 or (q4.numel() == b * hq * t * D // 2 and qa4.numel() == b * hq * t and
                             k4p.numel() == b * hk * tiles * K4_WORDS and ka4.numel() == b * hk * tiles * 4)),
               "INT4 Q/K buffers (all or none)")
        _check(k4x is None or (int4 and k4x.dtype == torch.uint32 and k4x.is_contiguous() and
                               k4x.numel() == b * hk * tiles * K8_WORDS), "expanded K4 records (with the INT4 buffers)")
        with torch.cuda.device(q.device):
            self._call(self.lib.tri_prepare_qk, _ptr(q), q.stride(0), q.stride(1), q.stride(2), _ptr(k), k.stride(0),
                       k.stride(1), k.stride(2), b, hq, hk, t, _ptr(q8), _ptr(qa), _ptr(kp), _ptr(ka), _ptr(partial),
                       _ptr(kstat), _ptr(q4), _ptr(qa4), _ptr(k4p), _ptr(ka4), _ptr(k4x), self._stream(q.device))

    # ------------------------------------------------------------------ pack_v
    def pack_v(self, v, partial, vstat, v16p=None, v8p=None, v4p=None, v8sum=None):
        """Normalised BF16 V' into FP16/INT8/INT4 PV operands.

        Extension: ``v8sum`` (int32 [B*Hkv*tiles*128], with ``v8p``) receives -127 times each channel's
        sum of each tile's V8 codes, which ``attention(..., v8sum=...)`` starts its P V products from."""
        _check(v.is_cuda and v.dtype == torch.bfloat16 and v.dim() == 4 and v.size(3) == D and v.stride(3) == 1,
               "BF16 V [B,Hkv,T,128]")
        b, hk, t, _ = v.shape
        tiles = (t + 63) // 64
        _check(partial.numel() >= b * hk * STAT_BLOCKS * 3 * D and vstat.numel() == b * hk * 3 * D,
               "V statistics buffers")
        for x, words in ((v16p, V16_WORDS), (v8p, V8_WORDS), (v4p, V4_WORDS)):
            _check(x is None or (x.dtype == torch.uint32 and x.is_contiguous() and x.numel() == b * hk * tiles * words),
                   "packed V size")
        _check(v8sum is None or (v8p is not None and _v8sum_ok(v8sum, b * hk * tiles)), "V8 sums")
        with torch.cuda.device(v.device):
            self._call(self.lib.tri_pack_v, _ptr(v), v.stride(0), v.stride(1), v.stride(2), b, hk, t, _ptr(partial),
                       _ptr(vstat), _ptr(v16p), _ptr(v8p), _ptr(v4p), _ptr(v8sum), self._stream(v.device))

    # --------------------------------------------------------------- attention
    def attention(self, order, bands, groups, entries, v16p, v8p, v4p, vstat, q8, k8p, qa8, ka8, q4, k4p, qa4, ka4,
                  out, scale, exact=None, q=None, kx=None, vx=None, nx=0, v8sum=None, k4x=None):
        """Banded causal attention: per key tile skip / INT8 QK x FP16 or INT8 PV / INT4 QK x INT8 PV.

        Extension: ``exact`` (int32 [Hq] on the device, 0 or 1 + record slot
        of the q-head's KV head) with the raw bf16 ``q`` [B,Hq,T,128] and the
        ``kx``/``vx`` records of ``pack_exact`` computes the flagged q-heads as
        exact causal attention on the unquantized operands.  ``v8sum``: what
        ``pack_v(..., v8sum=...)`` wrote for ``v8p`` (the same result, fewer MFMAs).  ``k4x``: what
        ``prepare_qk(..., k4x=...)`` wrote for ``k4p`` (the same result, fewer VALU instructions)."""
        _check(q8.dtype == torch.int8 and q8.dim() == 4 and q8.size(3) == D and q8.is_contiguous(), "Q8 [B,Hq,T,128]")
        b, h, t, _ = q8.shape
        hk = vstat.numel() // (b * 3 * D)
        tiles = (t + 63) // 64
        _check(tiles <= 2048, "at most 131072 tokens")
        _check(hk > 0 and h % hk == 0 and order.dtype == torch.int32 and order.numel() == h * tiles, "CTA order")
        _check(groups is None and entries is None,
               "task-table attention (groups/entries) is not provided; pass bands [Hq,2]")
        _check(bands is not None and bands.dtype == torch.int32 and bands.is_contiguous() and bands.numel() == h * 2,
               "bands [Hq,2] or task tables")
        _check((q4 is None) == (k4p is None) == (qa4 is None) == (ka4 is None), "INT4 Q/K operands (all or none)")
        _check(v16p is not None and v16p.numel() == b * hk * tiles * V16_WORDS, "packed V16")
        _check(v8p is not None or (q4 is None and _only_f16(bands, tiles)), "packed V8 required by INT8/INT4 bands")
        _check(out.dim() == 4 and tuple(out.shape) == (b, h, t, D) and out.stride(3) == 1 and
               out.dtype in (torch.float32, torch.bfloat16, torch.float16), "output [B,Hq,T,128]")
        dt = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[out.dtype]
        if exact is not None:
            _check(exact.dtype == torch.int32 and exact.numel() == h and exact.is_cuda and
                   q is not None and q.dtype == torch.bfloat16 and tuple(q.shape) == (b, h, t, D) and
                   q.stride(3) == 1, "exact heads: flags [Hq] and bf16 q [B,Hq,T,128]")
            _check(1 <= nx <= hk and kx is not None and vx is not None and
                   kx.numel() * kx.element_size() >= b * nx * tiles * KX_BYTES and
                   vx.numel() * vx.element_size() >= b * nx * tiles * KX_BYTES, "exact heads: KX/VX records")
        _check(v8sum is None or (v8p is not None and _v8sum_ok(v8sum, b * hk * tiles)), "V8 sums")
        _check(k4x is None or (q4 is not None and k4x.dtype == torch.uint32 and k4x.is_contiguous() and
                               k4x.numel() == b * hk * tiles * K8_WORDS), "expanded K4 records (with the INT4 operands)")
        qs = q.stride() if exact is not None else (0, 0, 0)
        with torch.cuda.device(q8.device):
            self._call(self.lib.tri_attention, _ptr(order), order.numel(), _ptr(bands), b, h, hk, t, _ptr(v16p),
                       _ptr(v8p), _ptr(vstat), _ptr(q8), _ptr(k8p), _ptr(qa8), _ptr(ka8), _ptr(q4), _ptr(k4p),
                       _ptr(qa4), _ptr(ka4), _ptr(out), dt, out.stride(0), out.stride(1), out.stride(2),
                       float(scale), _ptr(exact), _ptr(q if exact is not None else None), qs[0], qs[1], qs[2],
                       _ptr(kx if exact is not None else None), _ptr(vx if exact is not None else None),
                       int(nx) if exact is not None else 0, _ptr(v8sum), _ptr(k4x), self._stream(q8.device))
        return out

    def pack_exact(self, k, v, exact, nx, kx, vx):
        """bf16 K/V of the exact KV heads -> KX/VX records [B][nx][tiles] (16 KiB each; extension)."""
        _check(k.dtype == v.dtype == torch.bfloat16 and k.dim() == 4 and k.shape == v.shape and k.size(3) == D and
               k.stride(3) == 1 and v.stride(3) == 1, "K/V bf16 [B,Hk,T,128]")
        b, hk, t, _ = k.shape
        h = exact.numel()
        tiles = (t + 63) // 64
        _check(exact.dtype == torch.int32 and exact.is_cuda and h % hk == 0, "exact flags [Hq]")
        _check(1 <= nx <= hk and kx.numel() * kx.element_size() >= b * nx * tiles * KX_BYTES and
               vx.numel() * vx.element_size() >= b * nx * tiles * KX_BYTES, "KX/VX records [B][nx][tiles]")
        with torch.cuda.device(k.device):
            self._call(self.lib.tri_pack_exact, _ptr(k), *k.stride()[:3], _ptr(v), *v.stride()[:3], b, h, hk, t,
                       _ptr(exact), int(nx), _ptr(kx), _ptr(vx), self._stream(k.device))

    # ------------------------------------------------------------------ decode
    def decode(self, q, k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8, v4, vstat, kstat, ktail, vtail, kcur,
               vcur, step, out, pm, pl, po, prompt, per, scale, phase=3, xslot=None, kxc=None, vxc=None, bounds=None):
        """Single-token decode over the quantized cache plus the bf16 tail.

        ``phase`` (extension): 3 runs both kernels, 1 only the split-KV kernel,
        2 only the merge (for per-kernel timing).  ``xslot`` (extension, int32
        [B,Hk], -1 = quantized head) with the KX/VX record arrays ``kxc``/``vxc``
        makes the listed KV heads attend exactly over their bf16 prompt.  ``bounds``
        (extension, int32 [B,Hk,splits+1]) replaces the uniform split of ``per`` tiles
        by the given partition of each head's kept tiles."""
        # A caller of the reference's op (decode.py:76-79) passes the same cache tensors at every step, with
        # new q / k / v / out: the validated plan is kept per cache (tensor identities, shapes and strides,
        # prompt, per, scale), so a step costs one launch call, not a re-validation and a prompt tensor.
        cache_args = (k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8, v4, vstat, kstat, ktail, vtail, step,
                      pm, pl, po, xslot, kxc, vxc, bounds)
        key = (tuple(None if t is None else (t.data_ptr(), _geometry(t)) for t in cache_args),
               prompt.data_ptr() if isinstance(prompt, torch.Tensor) else int(prompt), int(per), float(scale),
               _geometry(q), _geometry(kcur), _geometry(vcur), _geometry(out))
        plan = self._plans.pop(key, None)
        if plan is not None and any(ref() is None for ref in plan.weak):
            plan = None  # a tensor of that cache was freed (its address may be reused)
        if plan is None:
            plan = self.plan_decode(q, k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8, v4, vstat, kstat,
                                    ktail, vtail, kcur, vcur, step, out, pm, pl, po, prompt, per, scale, xslot, kxc,
                                    vxc, bounds)
            # the caller owns the cache: the kept plan holds it weakly (and its own prompt tensor strongly),
            # so dropping a cache frees it
            plan.weak = tuple(weakref.ref(t) for t in cache_args if t is not None)
            plan.keep = tuple(t for t in plan.keep if t is not None and not any(t is c for c in cache_args))
        self._plans[key] = plan  # most recently used last
        while len(self._plans) > self.PLAN_CACHE:
            self._plans.pop(next(iter(self._plans)))
        plan.run(q, kcur, vcur, out, phase)
        return out

    def plan_decode(self, q, k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8, v4, vstat, kstat, ktail, vtail,
                    kcur, vcur, step, out, pm, pl, po, prompt, per, scale, xslot=None, kxc=None, vxc=None,
                    bounds=None, tasks=None, tail_base=None):
        """Validate and marshal every argument of ``decode`` once (extension).  The returned
        plan's ``run(q, kcur, vcur, out, phase)`` launches with new q / k / v / out tensors of the
        planned shapes and strides and the same cache, at a few microseconds of host time.
        ``tasks``: (table, listed splits) as ``decode_tasks`` returns it for this cache and split, or None;
        the caller keeps the partials of the splits it leaves out empty.  ``tail_base``: the int64
        tokens ``tail_spill`` has moved from the tail into the cache (the tail then holds step - tail_base
        tokens), or None for the reference's tail."""
        _check(q.dtype == torch.bfloat16 and q.dim() == 4 and q.size(2) == 1 and q.size(3) == D and q.stride(3) == 1,
               "q [B,Hq,1,128]")
        b, hq = q.size(0), q.size(1)
        hk = kstat.numel() // (b * 3 * D)
        max_tail = ktail.size(2)
        maxn = entry.size(-1)
        _check(hk > 0 and hq % hk == 0 and hq // hk <= 8 and max_tail <= 1024, "decode geometry")
        if isinstance(prompt, torch.Tensor):
            prompt_t = prompt
        else:
            prompt_t = torch.full((b,), int(prompt), dtype=torch.int32, device=q.device)
        tiles_max = fmt.numel() // b
        if bounds is not None:
            _check(bounds.dtype == torch.int32 and bounds.is_cuda and bounds.dim() == 3 and
                   tuple(bounds.shape[:2]) == (b, hk) and bounds.size(2) >= 2 and bounds.is_contiguous(),
                   "decode: bounds int32 [B,Hk,splits+1]")
            splits = bounds.size(2) - 1
        else:
            _check(1 <= int(per) <= 64, "decode: per (tiles per split) must be in [1, 64]")
            splits = max(1, -(-maxn // int(per)))
        if xslot is not None:
            _check(xslot.dtype == torch.int32 and xslot.is_cuda and xslot.numel() == b * hk and kxc is not None and
                   vxc is not None and kxc.numel() * kxc.element_size() % KX_BYTES == 0 and
                   kxc.numel() * kxc.element_size() == vxc.numel() * vxc.element_size(), "exact heads: xslot / KX / VX")
        _check(_geometry(vcur) == _geometry(kcur), "decode: k and v of the new token must have the same shape and strides")
        # the merge kernel writes out, ktail and vtail at sequence / head offsets and reads kcur / vcur
        # the same way: every one of them must span the whole [B, H, ., 128] it addresses
        _check(kcur.dtype == torch.bfloat16 and kcur.dim() == 4 and tuple(kcur.shape) == (b, hk, 1, D),
               "decode: k / v of the new token must be bf16 [B,Hk,1,128]")
        _check(ktail.dtype == torch.bfloat16 and ktail.dim() == 4 and tuple(ktail.shape) == (b, hk, max_tail, D) and
               ktail.stride(3) == 1 and _geometry(vtail) == _geometry(ktail),
               "decode: tails must be bf16 [B,Hk,max_tail,128], K and V alike")
        _check(out.dim() == 4 and tuple(out.shape) == (b, hq, 1, D), "decode: out must be [B,Hq,1,128]")
        _check(prompt_t.numel() == b and prompt_t.dtype == torch.int32, "decode: one int32 prompt length per sequence")
        _check(fmt.numel() % b == 0 and tiles_max >= 1, "decode: fmt [B, tiles]")
        _check(pm.dtype == pl.dtype == po.dtype == torch.float32 and pm.numel() >= b * hq * splits and
               pl.numel() >= b * hq * splits and po.numel() >= b * hq * splits * D,
               "decode: split partials pm / pl [B*Hq*splits], po [B*Hq*splits*128] (fp32)")
        _check(ka.dtype == torch.float32 and (ka4 is None or ka4.dtype == torch.float32) and
               vstat.dtype == kstat.dtype == torch.float32 and vstat.numel() == b * hk * 3 * D,
               "decode: K scales and statistics (fp32)")
        _check(step.dtype == torch.int64 and step.numel() >= 1 and
               entry.dtype == torch.int32 and kinfo.dtype == torch.int32 and count.dtype == torch.int32 and
               slot.dtype == torch.int32 and fmt.dtype == torch.int32 and
               entry.numel() == b * hk * maxn and kinfo.numel() == entry.numel() and slot.numel() == entry.numel() and
               count.numel() == b * hk and ka.numel() == b * hk * tiles_max * 4 and
               k8c.dim() == 2 and k8c.size(1) == K8_WORDS and v8.dim() == 2 and v8.size(1) == V8_WORDS and
               v4.dim() == 2 and v4.size(1) == V4_WORDS and (k4c is None) == (ka4 is None) and
               (k4c is None or (k4c.dim() == 2 and k4c.size(1) == K4_WORDS and ka4.numel() == ka.numel())) and
               out.dtype in (torch.bfloat16, torch.float32) and out.stride(3) == 1,
               "decode geometry/buffers")
        for name, t in (("q", q), ("k", kcur), ("tail", ktail), ("out", out), ("step", step), ("prompt", prompt_t),
                        ("entry", entry), ("kinfo", kinfo), ("slot", slot), ("count", count), ("fmt", fmt),
                        ("ka", ka), ("ka4", ka4), ("vstat", vstat), ("kstat", kstat), ("pm", pm), ("pl", pl),
                        ("po", po), ("k8", k8c), ("k4", k4c), ("v8", v8), ("v4", v4)):
            contiguous = name in ("q", "k", "tail", "out") or t is None or t.is_contiguous()
            _check(t is None or (t.is_cuda and t.device == q.device and contiguous),
                   f"decode: {name} must be a{'' if name in ('q', 'k', 'tail', 'out') else ' contiguous'} tensor "
                   f"on q's device")
        _check(tail_base is None or (tail_base.dtype == torch.int64 and tail_base.is_cuda and
                                     tail_base.device == q.device and tail_base.numel() >= 1),
               "decode: tail_base int64 on q's device")
        table, n_tasks = tasks if tasks is not None else (None, 0)
        if table is not None:
            _check(table.dtype == torch.int32 and table.is_cuda and table.is_contiguous() and
                   1 <= n_tasks <= b * hk * splits and table.numel() == n_tasks * TASK_WORDS,
                   "decode: task table int32 [n_tasks*512], at most one task per split")
        kc = kcur.view(b, hk, -1, D) if kcur.dim() == 4 else kcur
        args = [0, q.stride(0), q.stride(1), _ptr(k8c), _ptr(k4c), _ptr(ka),
                _ptr(ka4), _ptr(entry), _ptr(kinfo), _ptr(count), _ptr(fmt), _ptr(slot), _ptr(v8), _ptr(v4),
                _ptr(vstat), _ptr(kstat), _ptr(ktail), _ptr(vtail), ktail.stride(0), ktail.stride(1),
                ktail.stride(2), max_tail, 0, 0, kc.stride(0), kc.stride(1), _ptr(step),
                0, 0 if out.dtype == torch.float32 else 1, out.stride(0), out.stride(1), _ptr(pm),
                _ptr(pl), _ptr(po), _ptr(prompt_t), b, hq, hk, maxn, int(per), tiles_max, k8c.size(0),
                0 if k4c is None else k4c.size(0), v8.size(0), v4.size(0), _ptr(xslot), _ptr(kxc),
                _ptr(vxc), 0 if kxc is None else kxc.numel() * kxc.element_size() // KX_BYTES, _ptr(bounds),
                splits if bounds is not None else 0, _ptr(table), int(n_tasks), _ptr(tail_base), float(scale), 0]
        keep = (k8c, k4c, ka, ka4, entry, kinfo, count, fmt, slot, v8, v4, vstat, kstat, ktail, vtail, step, pm, pl,
                po, prompt_t, xslot, kxc, vxc, bounds, table, tail_base)
        return DecodePlan(self, args, q, kcur, out, keep)

    def decode_tasks(self, ka, ka4, entry, kinfo, count, fmt, slot, per, bounds=None, items=None):
        """The split kernel's task table for a decode cache and its split (extension): (int32
        [n*512], n) for the work items ``items`` (int32 on the device; None: every split)."""
        b, hk, maxn = entry.shape
        tiles_max = fmt.numel() // b
        splits = bounds.size(2) - 1 if bounds is not None else max(1, -(-maxn // int(per)))
        _check(entry.dtype == kinfo.dtype == slot.dtype == count.dtype == fmt.dtype == torch.int32 and
               kinfo.shape == entry.shape and slot.shape == entry.shape and count.numel() == b * hk and
               ka.numel() == b * hk * tiles_max * 4 and (ka4 is None or ka4.numel() == ka.numel()),
               "decode_tasks: cache metadata")
        n = b * hk * splits if items is None else items.numel()
        _check(items is None or (items.dtype == torch.int32 and items.is_cuda and 1 <= n <= b * hk * splits),
               "decode_tasks: items int32 on the device, at most one per split")
        table = torch.empty(n * TASK_WORDS, dtype=torch.int32, device=entry.device)
        with torch.cuda.device(entry.device):
            self._call(self.lib.tri_decode_tasks, _ptr(ka), _ptr(ka4), _ptr(entry), _ptr(kinfo), _ptr(count),
                       _ptr(fmt), _ptr(slot), b, hk, maxn, int(per), tiles_max, _ptr(bounds),
                       splits if bounds is not None else 0, _ptr(items), n if items is not None else 0, _ptr(table),
                       self._stream(entry.device))
        return table, n

    def cache_store(self, bands, exact, t, kp, k4p, ka, ka4, kstat, vstat, v8p, v4p, kx, vx, nx, row0, dst, used,
                    cap, xstride=None):
        """Append one Prefill call's batch to a decode cache on the device (extension; the reference
        assembles its cache on the host, kernels/decode.py:24-67).  Sources as ``store`` receives them;
        ``dst`` the cache's arrays (entry / kinfo / slot [rows][hk][maxn], count, fmt, prompt, xslot, ka,
        ka4, kstat, vstat, compacted k8 / k4 / v8 / v4 records and kx / vx bytes), ``used`` / ``cap`` the
        records in use and held per kind (k8, k4, v8, v4, x), sequence rows from ``row0``.  ``xstride``:
        KX / VX records per (sequence, exact head) in the cache (default: the prompt's tiles)."""
        b, hk = vstat.shape[0], vstat.shape[1]
        hq = bands.shape[0]
        rows, maxn = dst["entry"].shape[0], dst["entry"].shape[2]
        tiles_max = dst["fmt"].shape[1]
        tiles = (t + 63) // 64
        xstride = tiles if xstride is None else int(xstride)
        _check(xstride >= tiles, "cache_store: xstride below the prompt's tiles")
        _check(bands.dtype == torch.int32 and bands.is_cuda and bands.is_contiguous() and bands.dim() == 2 and
               bands.size(1) == 2, "cache_store: bands int32 [Hq,2] on the device")
        _check(exact is None or (exact.dtype == torch.int32 and exact.is_cuda and exact.numel() == hk),
               "cache_store: exact flags int32 [Hk] on the device")
        _check(kp.numel() * kp.element_size() >= b * hk * tiles * K8_WORDS * 4 and
               v8p.numel() * v8p.element_size() >= b * hk * tiles * V8_WORDS * 4 and
               (k4p is None or k4p.numel() * k4p.element_size() >= b * hk * tiles * K4_WORDS * 4) and
               (v4p is None or v4p.numel() * v4p.element_size() >= b * hk * tiles * V4_WORDS * 4) and
               ka.numel() >= b * hk * tiles * 4 and (ka4 is None or ka4.numel() >= b * hk * tiles * 4) and
               kstat.numel() == b * hk * 3 * D and vstat.numel() == b * hk * 3 * D,
               "cache_store: source records and scales [B,Hk,tiles]")
        _check(exact is None or (kx is not None and vx is not None and
                                 kx.numel() * kx.element_size() >= b * nx * tiles * KX_BYTES and
                                 vx.numel() * vx.element_size() >= b * nx * tiles * KX_BYTES),
               "cache_store: KX/VX records of the exact heads")
        for name in ("entry", "kinfo", "slot"):
            _check(tuple(dst[name].shape) == (rows, hk, maxn) and dst[name].dtype == torch.int32, f"cache_store: {name}")
        _check(tuple(dst["ka"].shape) == (rows, hk, tiles_max, 4) and
               (dst["ka4"] is None or tuple(dst["ka4"].shape) == (rows, hk, tiles_max, 4)) and
               tuple(dst["count"].shape) == (rows, hk) and dst["prompt"].numel() == rows and
               tuple(dst["kstat"].shape) == (rows, hk, 3, D) and tuple(dst["vstat"].shape) == (rows, hk, 3, D) and
               (dst["xslot"] is None or tuple(dst["xslot"].shape) == (rows, hk)), "cache_store: cache rows")
        for kind, words in (("k8", K8_WORDS), ("k4", K4_WORDS), ("v8", V8_WORDS), ("v4", V4_WORDS)):
            x = dst[kind]
            _check((x is None and cap[kind] == 0) or (x is not None and x.shape[0] >= cap[kind] and x.shape[1] == words),
                   f"cache_store: {kind} record array")
        _check(dst["kx"] is None or dst["kx"].numel() >= cap["x"] * KX_BYTES, "cache_store: KX/VX record arrays")
        p = _ptr
        with torch.cuda.device(vstat.device):
            self._call(self.lib.tri_cache_store, p(bands), p(exact), b, hq, hk, int(t), int(nx), xstride, p(kp), p(k4p),
                       p(ka),
                       p(ka4), p(kstat), p(vstat), p(v8p), p(v4p), p(kx), p(vx), int(row0), rows, maxn, tiles_max,
                       p(dst["entry"]), p(dst["kinfo"]), p(dst["slot"]), p(dst["count"]), p(dst["fmt"]),
                       p(dst["prompt"]), p(dst["xslot"]), p(dst["ka"]), p(dst["ka4"]), p(dst["kstat"]),
                       p(dst["vstat"]), p(dst["k8"]), used["k8"], cap["k8"], p(dst["k4"]), used["k4"], cap["k4"],
                       p(dst["v8"]), used["v8"], cap["v8"], p(dst["v4"]), used["v4"], cap["v4"], p(dst["kx"]),
                       p(dst["vx"]), used["x"], cap["x"], self._stream(vstat.device))

    def plan_tail_spill(self, step, tail_base, ktail, vtail, grow, cap, prompt, dst, tasks=None):
        """Validate and marshal one layer's ``tail_spill`` launch (extension; the reference clamps its
        tail, common_device.cuh:384).  ``dst``: the cache arrays as ``cache_store`` takes them (entry /
        kinfo / slot, count, fmt, xslot, ka, ka4, kstat, vstat, k8 / k4 / v8 records, kx / vx bytes);
        ``grow`` int32 [rows, hk, 4]; ``cap`` spilled tiles per head the arrays hold; ``tasks`` the
        decode's (table, n) or None; ``dst["count0"]`` each head's entry count at the store.  A spill
        happens for every (sequence, KV head) or, when any lacks room, for none.  The plan's ``run()``
        launches on the current stream."""
        rows, hk, maxn = dst["entry"].shape
        tiles_max = dst["fmt"].shape[1]
        max_tail = ktail.size(2)
        _check(step.dtype == tail_base.dtype == torch.int64 and tail_base.numel() == 2 and step.is_cuda and
               tail_base.is_cuda, "tail_spill: step int64 and tail_base int64 [2] on the device")
        _check(ktail.dtype == torch.bfloat16 and ktail.dim() == 4 and tuple(ktail.shape[:2]) == (rows, hk) and
               ktail.size(3) == D and ktail.stride(3) == 1 and _geometry(vtail) == _geometry(ktail),
               "tail_spill: tails bf16 [rows,Hk,max_tail,128], K and V alike")
        _check(64 <= max_tail <= 1024, "tail_spill: max_tail must be in [64, 1024]")
        _check(grow.dtype == torch.int32 and grow.is_contiguous() and tuple(grow.shape) == (rows, hk, 4),
               "tail_spill: grow int32 [rows,Hk,4]")
        _check(prompt.dtype == torch.int32 and prompt.numel() == rows and int(cap) >= 0, "tail_spill: prompt / cap")
        for name in ("kinfo", "slot"):
            _check(tuple(dst[name].shape) == (rows, hk, maxn), f"tail_spill: {name}")
        _check(dst["count0"].dtype == torch.int32 and dst["count0"].is_contiguous() and
               tuple(dst["count0"].shape) == (rows, hk), "tail_spill: count0 int32 [rows,Hk]")
        _check(tuple(dst["ka"].shape) == (rows, hk, tiles_max, 4) and tuple(dst["count"].shape) == (rows, hk) and
               (dst["ka4"] is None or tuple(dst["ka4"].shape) == (rows, hk, tiles_max, 4)) and
               tuple(dst["kstat"].shape) == (rows, hk, 3, D) and tuple(dst["vstat"].shape) == (rows, hk, 3, D) and
               (dst["xslot"] is None or tuple(dst["xslot"].shape) == (rows, hk)), "tail_spill: cache rows")
        for kind, words in (("k8", K8_WORDS), ("k4", K4_WORDS), ("v8", V8_WORDS)):
            x = dst[kind]
            _check(x is None or (x.dim() == 2 and x.shape[1] == words), f"tail_spill: {kind} record array")
        table, n_tasks = tasks if tasks is not None else (None, 0)
        xb = lambda x: 0 if x is None else x.numel() * x.element_size() // KX_BYTES
        p = _ptr
        args = [p(step), p(tail_base), p(ktail), p(vtail), ktail.stride(0), ktail.stride(1), ktail.stride(2),
                max_tail, rows, hk, maxn, tiles_max, p(grow), int(cap), p(prompt), p(dst["xslot"]), p(dst["entry"]),
                p(dst["kinfo"]), p(dst["slot"]), p(dst["count"]), p(dst["count0"]), p(dst["fmt"]), p(dst["ka"]),
                p(dst["ka4"]),
                p(dst["kstat"]), p(dst["vstat"]), p(dst["k8"]), dst["k8"].shape[0], p(dst["k4"]),
                0 if dst["k4"] is None else dst["k4"].shape[0], p(dst["v8"]), dst["v8"].shape[0],
                p(dst["kx"] if dst["xslot"] is not None else None), p(dst["vx"] if dst["xslot"] is not None else None),
                xb(dst["kx"]) if dst["xslot"] is not None else 0, p(table), int(n_tasks), 0]
        keep = (step, tail_base, ktail, vtail, grow, prompt, table, dict(dst))
        return SpillPlan(self, args, ktail.device, keep)

    def decode_occupancy(self) -> int:
        """Resident decode workgroups per compute unit."""
        n = ctypes.c_int(0)
        self._call(self.lib.tri_decode_occupancy, ctypes.byref(n))
        return int(n.value)

    def device_cus(self) -> int:
        n = ctypes.c_int(0)
        self._call(self.lib.tri_device_cus, ctypes.byref(n))
        return int(n.value)

    def prefill_pairs(self, mode: int) -> None:
        """tri_prefill_pairs: attention's launch form for this process (0 by launch size, 1 two-wave
        workgroups, 2 four-wave workgroups whose wave pairs split the key tiles)."""
        self._call(self.lib.tri_prefill_pairs, int(mode))

    def issue_probe(self, mode: int, waves_per_simd: int, iters: int):
        """tri_issue_probe: per wave (shader-clock cycles, 100 MHz ticks), int64 [waves, 2] on the CPU."""
        dev = torch.device("cuda", torch.cuda.current_device())
        waves = self.device_cus() * 4 * waves_per_simd
        out = torch.zeros(2 * waves, dtype=torch.int64, device=dev)
        with torch.cuda.device(dev):
            self._call(self.lib.tri_issue_probe, mode, waves_per_simd, iters, _ptr(out), self._stream(dev))
        torch.cuda.synchronize()
        return out.view(waves, 2).cpu()

    def stream_read(self, buf, waves: int, waves_per_group: int, depth: int, sink) -> None:
        """Measurement aid (no reference counterpart): read every 8 KiB record of the device buffer
        ``buf`` with no compute, ``depth`` records in flight per wave (tri_stream_read)."""
        records = buf.numel() * buf.element_size() // 8192
        self._call(self.lib.tri_stream_read, buf.data_ptr(), records, waves, waves_per_group, depth,
                   sink.data_ptr(), self._stream(buf.device))


def _geometry(t):
    """What a launch depends on: shape, dtype, device and the strides of the dimensions of extent > 1
    (a stride over a dimension of extent 1 is never applied)."""
    return tuple(t.shape), tuple(s if n > 1 else None for n, s in zip(t.shape, t.stride())), t.dtype, t.device


class DecodePlan:
    """A validated, marshalled ``decode`` call; ``run`` swaps in the per-step tensors."""

    Q, QSB, QSH, KC, VC, KSB, KSH, OUT, STREAM = 0, 1, 2, 22, 23, 24, 25, 27, 55

    def __init__(self, module, args, q, kcur, out, keep):
        self.module, self.args, self.keep = module, args, keep
        self.qgeom, self.cgeom, self.ogeom = _geometry(q), _geometry(kcur), _geometry(out)
        self.device = q.device
        lib = module.lib
        self.fns = {3: lib.tri_decode, 1: lib.tri_decode_partials, 2: lib.tri_decode_merge}
        self.short_fns = {3: lib.tri_decode_short_tail, 1: lib.tri_decode_partials, 2: lib.tri_decode_merge_short_tail}

    def run(self, q, kcur, vcur, out, phase=3, events=None, short_tail=False):
        """Launch ``phase`` (3: both kernels, 1: the split-KV kernel, 2: the merge).  ``events`` (phase 1
        only): a pair of recorded torch.cuda.Event objects that the split-KV kernel's launch records as
        its own start and stop (``tri_decode_partials_timed``).  ``short_tail``: the merge as one wave
        per (sequence, q-head), the faster form while the tail holds at most 64 tokens (any tail gives a
        correct result)."""
        if _geometry(q) != self.qgeom or _geometry(kcur) != self.cgeom or _geometry(vcur) != self.cgeom or \
                _geometry(out) != self.ogeom:
            raise RuntimeError("decode plan: q / k / v / out differ in shape, strides, dtype or device from the plan")
        a = self.args
        a[self.Q], a[self.KC], a[self.VC], a[self.OUT] = q.data_ptr(), kcur.data_ptr(), vcur.data_ptr(), out.data_ptr()
        index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        a[self.STREAM] = torch.cuda.current_stream(index).cuda_stream
        fn, extra = (self.short_fns if short_tail else self.fns)[phase], ()
        if events is not None:
            if phase != 1:
                raise RuntimeError("decode plan: events time the split-KV kernel (phase 1) only")
            fn, extra = self.module.lib.tri_decode_partials_timed, tuple(e.cuda_event for e in events)
        if torch.cuda.current_device() != index:
            with torch.cuda.device(index):
                self.module._call(fn, *a, *extra)
        else:
            self.module._call(fn, *a, *extra)
        return out


class SpillPlan:
    """A validated, marshalled ``tail_spill`` launch for one layer's decode cache."""

    def __init__(self, module, args, device, keep):
        self.module, self.args, self.device, self.keep = module, args, device, keep

    def run(self):
        index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.args[-1] = torch.cuda.current_stream(index).cuda_stream  # (the stream is the last argument)
        if torch.cuda.current_device() != index:
            with torch.cuda.device(index):
                self.module._call(self.module.lib.tri_tail_spill, *self.args)
        else:
            self.module._call(self.module.lib.tri_tail_spill, *self.args)


def _v8sum_ok(x, tiles_all):
    """int32 V8 sums of ``tiles_all`` (sequence, KV head, tile) records, 128 per tile, 16-byte aligned."""
    return (x.dtype == torch.int32 and x.is_contiguous() and x.numel() == tiles_all * D and
            x.data_ptr() % 16 == 0)


def _only_f16(bands, tiles: int) -> bool:
    b = bands.detach().to("cpu", torch.int64).view(-1, 2)
    qb = torch.arange(tiles)[None, :]
    w8, w4 = b[:, :1], b[:, 1:]
    n8 = (qb - torch.clamp(qb - w8 + 1, min=1)).clamp(min=0)
    n4 = (qb - w8 - torch.clamp(qb - w4 + 1, min=1) + 1).clamp(min=0)
    return not bool((n8 > 0).any() or (n4 > 0).any())


@functools.cache
def load_extension() -> Module:
    """The gfx950 op module; raises RuntimeError without a gfx950 GPU or without the built library."""
    arch()
    return Module(load_library())
