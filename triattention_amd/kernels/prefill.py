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


class Prefill:
    """Callable ``prefill(layer, q, k, v, scale) -> out`` for HF attention hooks.

    q [B, Hq, T, 128], k/v [B, Hk, T, 128] bf16 -> out [B, Hq, T, 128] with
    token-major strides (kernels/prefill.py:102).  ``out_dtype`` (an extension)
    selects fp32 output for parity testing; the default is q's dtype.  Maps
    whose ``bands_fn.bf16(layer)`` lists KV heads (the map's optional "bf16"
    key) get exact attention for those heads' q-heads in the same launch.
    """

    def __init__(self, module, bands_fn, decode_cache=None, out_dtype=None):
        self.module, self.bands_fn, self.decode_cache = module, bands_fn, decode_cache
        self.out_dtype = out_dtype
        self.tables, self.buffers, self.views, self.layer_buffers = {}, {}, {}, {}
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
        key = (None if getattr(self.bands_fn, "layer_independent", False) else layer, heads, rows)
        if key not in self.tables:
            self.tables[key] = BandTable.build(self.bands_fn(layer, heads), rows, kv_heads, device)
        return self.tables[key]

    def buffer(self, name, numel, dtype, device):
        current = self.buffers.get(name)
        if current is None or current.numel() < numel or current.dtype != dtype or current.device != device:
            current = self.buffers[name] = torch.empty(numel, dtype=dtype, device=device)
            self.views.clear()
        return current[:numel]

    def kept(self, layer, batch, hk, rows, int4, device):
        """Per-layer scale/statistics buffers that the decode cache keeps (kernels/prefill.py:49-58)."""
        key = (layer, batch, hk, rows, int4)
        if key not in self.layer_buffers:
            self.layer_buffers[key] = (
                torch.empty(batch * hk * rows * 4, dtype=torch.float32, device=device),
                torch.empty(batch * hk * 3 * 128, dtype=torch.float32, device=device),
                torch.empty((batch, hk, 3, 128), dtype=torch.float32, device=device),
                torch.empty(batch * hk * rows * 4, dtype=torch.float32, device=device) if int4 else None,
            )
        return self.layer_buffers[key]

    def operands(self, batch, hq, hk, t, int4, formats, device):
        key = (batch, hq, hk, t, int4, formats, device)
        if key in self.views:
            return self.views[key]
        rows = (t + 63) // 64
        buf = lambda name, n, dtype: self.buffer(name, n, dtype, device)
        ops = dict(
            q8=buf("q8", batch * hq * t * 128, torch.int8).view(batch, hq, t, 128),
            qa=buf("qa", batch * hq * t, torch.float32),
            kp=buf("k", batch * hk * rows * 2048, torch.uint32),
            ka=buf("ka", batch * hk * rows * 4, torch.float32),
            partial=buf("partial", batch * hk * 64 * 3 * 128, torch.float32),
            kstat=buf("kstat", batch * hk * 3 * 128, torch.float32),
            vstat=buf("vstat", batch * hk * 3 * 128, torch.float32).view(batch, hk, 3, 128),
            q4=buf("q4", batch * hq * t * 64, torch.uint8) if int4 else None,
            qa4=buf("qa4", batch * hq * t, torch.float32) if int4 else None,
            k4=buf("k4", batch * hk * rows * 1024, torch.uint32) if int4 else None,
            ka4=buf("ka4", batch * hk * rows * 4, torch.float32) if int4 else None,
        )
        packed = {code: buf(f"v{code}", batch * hk * rows * words, torch.uint32) if code in formats else None
                  for code, words in WORDS.items()}
        if int4 and packed[I8] is None:
            packed[I8] = buf(f"v{I8}", batch * hk * rows * 2048, torch.uint32)
        ops["packed"] = packed
        self.views[key] = ops
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
        batch, hq, t, _ = q.shape
        hk, rows, device = k.shape[1], (t + 63) // 64, q.device
        table = self.table(layer, hq, hk, rows, device)
        int4 = Q4 in table.formats
        decode = self.decode_cache.codes(rows) if self.decode_cache is not None else None
        formats = table.formats | decode[1] if decode is not None else table.formats
        ops = self.operands(batch, hq, hk, t, int4, formats, device)
        ka, kstat, vstat, ka4 = ops["ka"], ops["kstat"], ops["vstat"], ops["ka4"]
        if decode is not None:
            ka, kstat, vstat, ka4 = self.kept(layer, batch, hk, rows, int4, device)
        packed = ops["packed"]
        self.module.prepare_qk(q, k, ops["q8"], ops["qa"], ops["kp"], ka, ops["partial"], kstat,
                               ops["q4"], ops["qa4"], ops["k4"], ka4)
        self.module.pack_v(v, ops["partial"], vstat, packed[F16], packed[I8], packed[I4])
        exact, nx = self.exact(layer, hq, hk, device)
        if exact is not None:
            kx, vx = self.exact_records(batch * nx * rows * KX_BYTES, device)
            self.module.pack_exact(k, v, exact, nx, kx, vx)
        out = None
        if attend:
            dtype = self.out_dtype or q.dtype
            out = torch.empty((batch, t, hq, 128), dtype=dtype, device=device).transpose(1, 2)
            if exact is None:
                self.module.attention(table.order, table.bands, None, None, packed[F16], packed[I8], packed[I4],
                                      vstat, ops["q8"], ops["kp"], ops["qa"], ka, ops["q4"], ops["k4"], ops["qa4"],
                                      ka4, out, scale)
            else:
                self.module.attention(table.order, table.bands, None, None, packed[F16], packed[I8], packed[I4],
                                      vstat, ops["q8"], ops["kp"], ops["qa"], ka, ops["q4"], ops["k4"], ops["qa4"],
                                      ka4, out, scale, exact=exact, q=q, kx=kx, vx=vx, nx=nx)
        if decode is not None:
            exact_kv = sorted(set(int(h) for h in self.bands_fn.bf16(layer))) if exact is not None else []
            self.decode_cache.store(layer, t, ops["kp"], ka, kstat, vstat, packed, decode[0], table.host,
                                    ops["k4"], ka4, exact_kv, *(self.records if exact is not None else (None, None)))
        return out
