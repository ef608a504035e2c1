"""Prefill host operator: band table, scratch pool and the op sequence
``prepare_qk -> pack_v -> attention -> store``.

Mirrors triattention/kernels/prefill.py (BandTable :10-28, Prefill :31-108)
with the same names, call signature and buffer-sharing contract, extended to a
leading batch dimension ([B, H, T, 128]; B = 1 is the reference behaviour).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

SKIP, F16, I8, I4, Q4 = 0, 1, 2, 3, 4
WORDS = {F16: 4096, I8: 2048, I4: 1024}
KX_BYTES = 16384  # bf16 K (or V) record of one tile of an exact KV head


def tile_counts(bands: torch.Tensor, rows: int):
    """Per (q-head, query tile) counts of INT8-QK and INT4-QK key tiles (prefill_sm80.cu:280-286)."""
    b = torch.as_tensor(bands, dtype=torch.int64).cpu().view(-1, 2)
    w8, w4 = b[:, :1], b[:, 1:]
    qb = torch.arange(rows)[None, :]
    n8 = (qb - torch.clamp(qb - w8 + 1, min=1)).clamp(min=0)
    n4 = (qb - w8 - torch.clamp(qb - w4 + 1, min=1) + 1).clamp(min=0)
    return n8, n4


@dataclass
class BandTable:
    order: torch.Tensor
    bands: torch.Tensor
    formats: frozenset
    host: torch.Tensor

    @classmethod
    def build(cls, bands, rows, kv_heads, device):
        """Workgroup order and the V formats a band table needs.

        Order: KV head by KV head, query tiles from the last (longest) to the
        first, the q-heads of the GQA group adjacent, so that the group's
        workgroups read the same K/V tiles close together in time
        (kernels/prefill.py:24-25).
        """
        host = torch.as_tensor(bands, dtype=torch.int64).cpu().view(-1, 2)
        heads = host.shape[0]
        group = heads // kv_heads
        qhead = torch.arange(heads).view(kv_heads, 1, group)
        qtile = torch.arange(rows - 1, -1, -1).view(1, rows, 1)
        order = (qhead * rows + qtile).reshape(-1)
        n8, n4 = tile_counts(host, rows)
        formats = {F16}
        if bool((n8 > 0).any()):
            formats.add(I8)
        if bool((n4 > 0).any()):
            formats.add(Q4)
        host32 = host.to(torch.int32).contiguous()
        return cls(order.to(torch.int32).to(device), host32.to(device), frozenset(formats), host32)


@dataclass(frozen=True)
class Layout:
    """Shape of one Prefill call: everything its scratch buffers depend on."""
    batch: int
    hq: int
    hk: int
    t: int
    int4: bool           # INT4 Q/K operands exist (some band has INT4 key tiles)
    formats: frozenset   # V record formats the call writes

    @property
    def tiles(self):
        return (self.t + 63) // 64


# The scratch of a Prefill call, one row per buffer: the name it is pooled under (Prefill.buffers, which
# executors may share), its element count and dtype for a layout, and whether the layout needs it.
# Word counts per (KV head, tile) are the reference's record sizes (decode.py:7-8).
SCRATCH = (
    ("q8", lambda L: L.batch * L.hq * L.t * 128, torch.int8, lambda L: True),
    ("qa", lambda L: L.batch * L.hq * L.t, torch.float32, lambda L: True),
    ("k", lambda L: L.batch * L.hk * L.tiles * 2048, torch.uint32, lambda L: True),
    ("ka", lambda L: L.batch * L.hk * L.tiles * 4, torch.float32, lambda L: True),
    ("partial", lambda L: L.batch * L.hk * 64 * 3 * 128, torch.float32, lambda L: True),
    ("kstat", lambda L: L.batch * L.hk * 3 * 128, torch.float32, lambda L: True),
    ("vstat", lambda L: L.batch * L.hk * 3 * 128, torch.float32, lambda L: True),
    ("q4", lambda L: L.batch * L.hq * L.t * 64, torch.uint8, lambda L: L.int4),
    ("qa4", lambda L: L.batch * L.hq * L.t, torch.float32, lambda L: L.int4),
    ("k4", lambda L: L.batch * L.hk * L.tiles * 1024, torch.uint32, lambda L: L.int4),
    ("ka4", lambda L: L.batch * L.hk * L.tiles * 4, torch.float32, lambda L: L.int4),
    # the K4 records expanded to 16 * code bytes in the K8 layout (extension: INT4 key tiles read these)
    ("k4x", lambda L: L.batch * L.hk * L.tiles * 2048, torch.uint32, lambda L: L.int4),
    # V records: FP16 always; INT8 for INT8 bands and for every INT4 band (INT4 key tiles pair with
    # INT8 V, prefill_sm80.cu:462-465); INT4 when the decode cache asks for it
    (f"v{F16}", lambda L: L.batch * L.hk * L.tiles * WORDS[F16], torch.uint32, lambda L: F16 in L.formats),
    (f"v{I8}", lambda L: L.batch * L.hk * L.tiles * WORDS[I8], torch.uint32, lambda L: I8 in L.formats or L.int4),
    (f"v{I4}", lambda L: L.batch * L.hk * L.tiles * WORDS[I4], torch.uint32, lambda L: I4 in L.formats),
    # -127 * each channel's sum of every INT8 V record (extension: the P V products start from it)
    ("v8sum", lambda L: L.batch * L.hk * L.tiles * 128, torch.int32, lambda L: I8 in L.formats or L.int4),
)


class Prefill:
    """Callable ``prefill(layer, q, k, v, scale) -> out`` for HF attention hooks.

    q [B, Hq, T, 128], k/v [B, Hk, T, 128] bf16 -> out [B, Hq, T, 128] with
    token-major strides (kernels/prefill.py:102).  ``out_dtype`` (an extension)
    selects fp32 output for parity testing; the default is q's dtype.  Maps
    whose ``bands_fn.bf16(layer)`` lists KV heads (the map's optional "bf16"
    key) get exact attention for those heads' q-heads in the same launch.

    Scratch lives in ``buffers`` (name -> flat device tensor, grown on demand), which executors may
    share (calibrate.py:44-48 assigns one dict to all of them); ``views`` caches each layout's typed
    views of it.  A decode cache copies what it keeps at ``store`` time, so the scratch is free for
    the next call as soon as the call's launches are queued.
    """

    def __init__(self, module, bands_fn, decode_cache=None, out_dtype=None):
        self.module, self.bands_fn, self.decode_cache = module, bands_fn, decode_cache
        self.out_dtype = out_dtype
        self.tables, self.buffers, self.views = {}, {}, {}
        self.exact_flags = {}
        self.records = None

    def exact(self, layer, heads, kv_heads, device):
        """(int32 [Hq] device flags, nx) for the KV heads the map keeps in bf16, or (None, 0).

        A flagged q-head holds 1 + the record slot of its KV head (slots in
        increasing KV-head order); unflagged q-heads hold 0."""
        bf16 = getattr(self.bands_fn, "bf16", None)
        kv = sorted(set(int(h) for h in bf16(layer))) if bf16 is not None else []
        if not kv:
            return None, 0
        if not all(0 <= h < kv_heads for h in kv):
            raise ValueError(f"bf16 KV heads {kv} out of range for {kv_heads} KV heads")
        key = (layer, heads, device)
        if key not in self.exact_flags:
            group = heads // kv_heads
            flags = torch.zeros(heads, dtype=torch.int32)
            for slot, h in enumerate(kv):
                flags[h * group:(h + 1) * group] = slot + 1
            self.exact_flags[key] = flags.to(device), len(kv)
        return self.exact_flags[key]

    def exact_records(self, nbytes, device):
        """KX/VX record buffers of the exact heads (grown on demand, reused across calls)."""
        cur = self.records
        if cur is None or cur[0].numel() < nbytes or cur[0].device != device:
            cur = self.records = (torch.empty(nbytes, dtype=torch.uint8, device=device),
                                  torch.empty(nbytes, dtype=torch.uint8, device=device))
        return cur[0][:nbytes], cur[1][:nbytes]

    def table(self, layer, heads, kv_heads, rows, device):
        """The band table of (layer, heads, rows); maps marked ``layer_independent`` share one per shape."""
        per_layer = not getattr(self.bands_fn, "layer_independent", False)
        key = (layer if per_layer else None, heads, rows)
        found = self.tables.get(key)
        if found is None:
            found = self.tables[key] = BandTable.build(self.bands_fn(layer, heads), rows, kv_heads, device)
        return found

    def operands(self, layout, device):
        """Typed views of the pooled scratch for ``layout`` (None for buffers the layout does not need).
        A pool buffer too small or of another dtype or device is replaced, which invalidates every
        cached view."""
        found = self.views.get((layout, device))
        if found is not None:
            return found
        ops = {}
        for name, count, dtype, needed in SCRATCH:
            if not needed(layout):
                ops[name] = None
                continue
            n = count(layout)
            pool = self.buffers.get(name)
            if pool is None or pool.numel() < n or pool.dtype != dtype or pool.device != device:
                pool = self.buffers[name] = torch.empty(n, dtype=dtype, device=device)
                self.views.clear()
            ops[name] = pool[:n]
        ops["q8"] = ops["q8"].view(layout.batch, layout.hq, layout.t, 128)
        ops["vstat"] = ops["vstat"].view(layout.batch, layout.hk, 3, 128)
        ops["kp"] = ops.pop("k")
        ops["packed"] = {code: ops.pop(f"v{code}") for code in (F16, I8, I4)}
        self.views[(layout, device)] = ops
        return ops

    def __call__(self, layer, q, k, v, scale):
        return self._run(layer, q, k, v, scale, attend=True)

    def store_only(self, layer, k, v, heads):
        """Extension: quantize, pack and store K/V of a ``heads``-q-head layer into the decode
        cache without computing the prompt's attention (the cache is all a caller needs when
        the prompt outputs are not used).  Q's codes are computed from a zero Q and discarded."""
        if self.decode_cache is None:
            raise ValueError("store_only needs a decode cache")
        batch, _, t, d = k.shape
        q = torch.zeros((1, 1, 1, d), dtype=k.dtype, device=k.device).expand(batch, heads, t, d)
        self._run(layer, q, k, v, None, attend=False)

    def _run(self, layer, q, k, v, scale, attend):
        """The reference's op sequence (kernels/prefill.py:87-108): quantize Q/K, pack V, attend,
        then hand the records to the decode cache."""
        batch, hq, t, _ = q.shape
        hk, rows, device = k.shape[1], (t + 63) // 64, q.device
        table = self.table(layer, hq, hk, rows, device)
        decode = self.decode_cache.codes(rows) if self.decode_cache is not None else None
        formats = table.formats | decode[1] if decode is not None else table.formats
        layout = Layout(batch, hq, hk, t, Q4 in table.formats, frozenset(formats))
        ops = self.operands(layout, device)
        packed = ops["packed"]
        k4x = ops["k4x"] if attend else None  # (only the prompt's attention reads the expanded records)
        self.module.prepare_qk(q, k, ops["q8"], ops["qa"], ops["kp"], ops["ka"], ops["partial"], ops["kstat"],
                               ops["q4"], ops["qa4"], ops["k4"], ops["ka4"], k4x=k4x)
        v8sum = ops["v8sum"] if attend else None  # (only the prompt's attention reads the sums)
        self.module.pack_v(v, ops["partial"], ops["vstat"], packed[F16], packed[I8], packed[I4], v8sum=v8sum)
        exact, nx = self.exact(layer, hq, hk, device)
        kx = vx = None
        if exact is not None:
            kx, vx = self.exact_records(batch * nx * rows * KX_BYTES, device)
            self.module.pack_exact(k, v, exact, nx, kx, vx)
        out = None
        if attend:
            dtype = self.out_dtype or q.dtype
            out = torch.empty((batch, t, hq, 128), dtype=dtype, device=device).transpose(1, 2)
            extra = {} if exact is None else dict(exact=exact, q=q, kx=kx, vx=vx, nx=nx)
            self.module.attention(table.order, table.bands, None, None, packed[F16], packed[I8], packed[I4],
                                  ops["vstat"], ops["q8"], ops["kp"], ops["qa"], ops["ka"], ops["q4"], ops["k4"],
                                  ops["qa4"], ops["ka4"], out, scale, v8sum=v8sum, k4x=k4x, **extra)
        if decode is not None:
            exact_kv = sorted(set(int(h) for h in self.bands_fn.bf16(layer))) if exact is not None else []
            self.decode_cache.store(layer, t, ops["kp"], ops["ka"], ops["kstat"], ops["vstat"], packed, decode[0],
                                    table.host, ops["k4"], ops["ka4"], exact_kv, kx, vx)
        return out
