"""Decode cache: the quantized prompt records that survive each q-head's band,
compacted per KV head, plus a bf16 tail for the generated tokens.

Mirrors triattention/kernels/decode.py (codes :17-22, store :24-67,
__call__ :69-80, advance/stored :82-86).  The metadata rules are the
reference's: per tile and q-head a state 8 / 4 / 0 from the band, the K
precision of a (KV head, tile) is the maximum over its GQA group, each q-head
attends only its own kept tiles (rowmask), and the V format is INT8 for the
sink tile and the last NEAR_V8 tiles, INT4 elsewhere.

Extension: exact (bf16) KV heads (the map's optional "bf16" key) keep every
prompt tile as bf16 KX/VX records and attend exactly; the same launch serves
both kinds of head.

Extension: batches.  One ``store`` holds the B sequences of one Prefill call;
with ``ragged = True`` successive ``store`` calls for a layer append their
sequences (e.g. one Prefill per prompt of a different length), and the decode
op then serves the whole ragged batch in one launch.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .extension import _geometry
from .prefill import I4, I8

WORDS = {I8: 2048, I4: 1024}
K8_WORDS, K4_WORDS = 2048, 1024
KX_BYTES = 16384
NEAR_V8 = 16
SPLITS_PER_CU = 4  # decode workgroups per CU that the split partition targets
# Split-kernel time per kept tile by record kind (hundredths of a us; C1, one wave per SIMD, per-workgroup
# timestamps): 133 for INT4 K and INT4 V, +20 for INT8 K, +43 for INT8 V (its 8 KiB record and P.V);
# exact bf16 tiles (16 KiB K + 16 KiB V) are priced at 2.5x an INT4/INT4 tile.
TILE_COST, K8_COST, V8_COST, EXACT_COST = 133, 20, 43, 333
BALANCE_TILES = 16  # kept tiles per slot up to which the split partition is balanced by cost
# entry words: bits 0-28 the tile index (decode.py:36); extension: bit 30 marks that bit 29 holds
# the tile's V format (1 = INT8 V), which spares the decode kernel a dependent load of fmt
ENTRY_TILE, ENTRY_V8, ENTRY_VFMT = (1 << 29) - 1, 1 << 29, 1 << 30


def tile_states(bands: torch.Tensor, tiles: int) -> torch.Tensor:
    """state[h, j]: 8 (INT8 K), 4 (INT4 K) or 0 (skipped) for q-head h, tile j (decode.py:27-30)."""
    b = torch.as_tensor(bands, dtype=torch.int64).cpu().view(-1, 2)
    j = torch.arange(tiles)
    w8, w4, d = b[:, :1], b[:, 1:], (tiles - 1) - j[None, :]
    return torch.where((j[None, :] == 0) | (d < w8), 8, torch.where(d < w4, 4, 0))


def sequence_metadata(bands, tiles: int, hk: int, vcodes: torch.Tensor, exact_kv=()):
    """Kept-tile lists and slots of one sequence (host, int64), as decode.py:27-53.

    Extension: KV heads in ``exact_kv`` keep every tile (count = tiles, entry
    j = j) and select no quantized record; the kernel reads their bf16 KX/VX
    records instead."""
    state = tile_states(bands, tiles)
    hq = state.shape[0]
    state = state.view(hk, hq // hk, tiles)
    exact = torch.zeros(hk, dtype=torch.bool)
    exact[list(exact_kv)] = True
    state[exact] = 8
    kv = state.amax(1)
    rowmask = ((state > 0).to(torch.int64) << torch.arange(state.shape[1])[None, :, None]).sum(1)
    count = (kv > 0).sum(1)
    maxn = max(1, int(count.max()))
    order = torch.argsort((kv == 0).to(torch.int8), dim=1, stable=True)[:, :maxn]
    valid = torch.arange(maxn)[None, :] < count[:, None]
    kprec = kv.gather(1, order)
    quant = valid & ~exact[:, None]
    is4 = (kprec == 4) & quant
    is8 = (kprec == 8) & quant
    rows = torch.arange(hk)[:, None] * tiles + order
    ragged = lambda select: torch.cumsum(select.flatten(), 0).view(hk, maxn) - 1
    kslot = torch.where(is4, ragged(is4), torch.where(is8, ragged(is8), 0))
    kbase = torch.where(valid, (rowmask.gather(1, order) & 0xFF) | (is4.to(torch.int64) << 8), 0)
    vcode = vcodes[order]
    vslot = torch.zeros((hk, maxn), dtype=torch.int64)
    vsel = {}
    for code in (I8, I4):
        select = quant & (vcode == code)
        vslot = torch.where(select, ragged(select), vslot)
        vsel[code] = select
    return dict(count=count, maxn=maxn, order=order, valid=valid, is4=is4, is8=is8, rows=rows, kslot=kslot,
                kbase=kbase, vslot=vslot, vcode=vcode, vsel=vsel, exact=exact)


def entry_costs(meta) -> np.ndarray:
    """Cost of each kept entry of one sequence [Hk, maxn] (float64, 0 past the count): the split
    kernel's measured time per tile of its kind (TILE_COST, plus K8_COST for INT8 K and V8_COST for
    INT8 V; EXACT_COST for an exact head's tile)."""
    exact = meta["exact"].numpy()[:, None]
    quant = TILE_COST + np.where(meta["is4"].numpy(), 0, K8_COST) + np.where(meta["vcode"].numpy() == I8, V8_COST, 0)
    return np.where(meta["valid"].numpy(), np.where(exact, EXACT_COST, quant), 0).astype(np.float64)


def split_bounds(costs: np.ndarray, valid: np.ndarray, n: np.ndarray) -> np.ndarray:
    """Entry bounds [Hk, max(n) + 1] cutting head h's kept entries into n[h] runs of near-equal cost:
    entry e joins the run that holds the midpoint of its cost interval.  Bounds past n[h] equal the
    count, so those splits are empty."""
    cum = costs.cumsum(1)
    mid = cum - costs / 2
    s = np.arange(int(n.max()) + 1, dtype=np.float64)[None, :]
    nf = n.astype(np.float64)[:, None]
    thr = cum[:, -1:] * np.minimum(s, nf) / nf
    return ((mid[:, None, :] < thr[:, :, None]) & valid[:, None, :]).sum(-1)


def balanced_partition(metas, batches, slots: int):
    """Per-sequence split bounds [Hk, splits + 1] (int32 tensors) for each metadata in ``metas`` (one
    per group of sequences of equal length, ``batches`` sequences each), and the common split count.

    Extension (the reference splits every head into runs of one tile count, decode.py:54-55): the
    split kernel streams each split's records at about the same rate per wave, so its time is set
    by the largest split.  Heads are cut by cost (the measured time of each tile's kind) into
    n_h = ceil(cost_h / t) runs of near-equal cost, with the smallest target t whose split count
    fits ``slots`` resident workgroups, at most 64 entries per split."""
    costs = [entry_costs(m) for m in metas]
    heads = [c.sum(1) for c in costs]
    floors = [np.maximum((m["count"].numpy() + 63) // 64, 1) for m in metas]
    h_all, f_all = np.concatenate(heads), np.concatenate(floors).astype(np.float64)
    w_all = np.concatenate([np.full(len(h), b, np.float64) for h, b in zip(heads, batches)])
    items = lambda t: float((w_all * np.maximum(np.ceil(h_all / t), f_all)).sum())
    lo, hi = max(float(c.max()) for c in costs), float(h_all.max()) + 1.0
    if items(hi) <= slots:
        for _ in range(60):
            mid = (lo + hi) / 2
            lo, hi = (lo, mid) if items(mid) <= slots else (mid, hi)
    out = []
    for m, c, h, f in zip(metas, costs, heads, floors):
        n = np.maximum(np.ceil(h / hi).astype(np.int64), f)
        valid = m["valid"].numpy()
        while True:
            b = split_bounds(c, valid, n)
            over = (np.diff(b, axis=1) > 64).any(1)
            if not over.any():
                break
            n = n + over
        out.append(b)
    splits = max(b.shape[1] - 1 for b in out)
    pad = lambda b: np.concatenate([b, np.repeat(b[:, -1:], splits + 1 - b.shape[1], 1)], 1)
    return [torch.from_numpy(pad(b).astype(np.int32)) for b in out], splits


class DecodeCache:
    def __init__(self, module, max_tail=256):
        self.module, self.max_tail = module, max_tail
        self.layers, self.formats, self.step = {}, {}, None
        self.ragged = False
        self.out_dtype = None
        self.meta_cache = {}
        self.wave = None
        # None: the balanced split partition; an int: the reference's uniform split of `per` tiles
        self.per = None

    def codes(self, rows):
        if rows not in self.formats:
            j = torch.arange(rows)
            codes = torch.where((rows - 1 - j < NEAR_V8) | (j == 0), I8, I4)
            self.formats[rows] = codes, frozenset(codes.unique().tolist())
        return self.formats[rows]

    def store(self, layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv=(), kx=None,
              vx=None):
        """Keep one Prefill call's records (decode.py:24-67).  Extension: ``exact_kv``
        lists the KV heads kept in bf16, whose KX/VX records ``kx``/``vx``
        ([B][len(exact_kv)][tiles], tri_pack_exact layout) are copied whole."""
        tiles = (prompt + 63) // 64
        batch = vstat.shape[0]
        hk, device = vstat.shape[1], ka.device
        exact_kv = sorted(set(int(h) for h in exact_kv))
        meta, dev = self._metadata(bands, tiles, hk, codes, exact_kv, device)
        nbytes = batch * len(exact_kv) * tiles * KX_BYTES
        # record indices of every sequence of the batch, sequence-major, built on the device
        seq = torch.arange(batch, dtype=torch.int64, device=device)[:, None] * (hk * tiles)
        pick = lambda kind: (seq + dev["pick"][kind][None, :]).flatten()
        group = dict(prompt=prompt, batch=batch, hk=hk, tiles=tiles, meta=meta, dev=dev,
                     n8=int(meta["is8"].sum()), n4=int(meta["is4"].sum()),
                     nv={code: int(meta["vsel"][code].sum()) for code in (I8, I4)},
                     k8=kp.view(batch * hk * tiles, K8_WORDS).index_select(0, pick("k8")),
                     k4=(k4.view(batch * hk * tiles, K4_WORDS).index_select(0, pick("k4"))
                         if bool(meta["is4"].any()) else None),
                     v={code: (packed[code].view(batch * hk * tiles, WORDS[code]).index_select(0, pick(code))
                               if bool(meta["vsel"][code].any()) else None) for code in (I8, I4)},
                     # copies, not views: the Prefill reuses these buffers for its next call with the
                     # same shape, and a ragged cache re-reads every stored group
                     ka=ka.view(batch, hk, tiles, 4).clone(),
                     ka4=ka4.view(batch, hk, tiles, 4).clone() if ka4 is not None else None,
                     kstat=kstat.view(batch, hk, 3, 128).clone(), vstat=vstat.view(batch, hk, 3, 128).clone(),
                     exact=exact_kv,
                     kx=kx.reshape(-1)[:nbytes].clone() if exact_kv else None,
                     vx=vx.reshape(-1)[:nbytes].clone() if exact_kv else None)
        if self.step is None:
            self.step = torch.zeros(1, dtype=torch.int64, device=device)
        self.step.zero_()
        entry = self.layers.get(layer)
        groups = entry["groups"] + [group] if (self.ragged and entry is not None) else [group]
        self.layers[layer] = self._assemble(groups, device)

    def _metadata(self, bands, tiles, hk, codes, exact_kv, device):
        """One sequence's metadata (host, closed-form integer code) and its device copy, cached per
        (bands, tiles, KV heads, exact heads, device): every sequence of the same length shares it."""
        b = torch.as_tensor(bands, dtype=torch.int32).cpu()
        key = (b.numpy().tobytes(), tiles, hk, tuple(exact_kv), str(device))
        hit = self.meta_cache.get(key)
        if hit is None:
            meta = sequence_metadata(b, tiles, hk, codes, exact_kv)
            to = lambda x: x.to(device)
            dev = dict(valid=to(meta["valid"]), order=to(meta["order"]), is4=to(meta["is4"]),
                       kslot=to(meta["kslot"]), kbase=to(meta["kbase"]), vcode=to(meta["vcode"]),
                       vslot=to(meta["vslot"]), count=to(meta["count"]), fmt=to(codes.to(torch.int64) - 1),
                       pick={kind: to(meta["rows"][select]) for kind, select in
                             (("k8", meta["is8"]), ("k4", meta["is4"]), (I8, meta["vsel"][I8]),
                              (I4, meta["vsel"][I4]))})
            hit = self.meta_cache[key] = (meta, dev)
        return hit

    def _assemble(self, groups, device):
        """Batched metadata and concatenated records over every stored sequence: a few device
        operations per group (a store's sequences share one length), none per sequence."""
        hk = groups[0]["hk"]
        total = sum(g["batch"] for g in groups)
        tiles_max = max(g["tiles"] for g in groups)
        maxn = max(g["meta"]["maxn"] for g in groups)
        i64 = dict(dtype=torch.int64, device=device)
        entry = torch.zeros((total, hk, maxn), **i64)
        kinfo = torch.zeros_like(entry)
        slot = torch.zeros_like(entry)
        count = torch.zeros((total, hk), **i64)
        fmt = torch.ones((total, tiles_max), **i64)
        prompt = torch.zeros(total, **i64)
        has4 = any(g["k4"] is not None for g in groups)
        ka = torch.ones((total, hk, tiles_max, 4), dtype=torch.float32, device=device)
        ka4 = torch.ones_like(ka) if has4 else None
        kstat = torch.empty((total, hk, 3, 128), dtype=torch.float32, device=device)
        vstat = torch.empty_like(kstat)
        k8s, k4s, v8s, v4s, kxs, vxs = [], [], [], [], [], []
        xslot = torch.full((total, hk), -1, **i64)
        o8 = o4 = ov8 = ov4 = ox = 0
        row = 0
        for g in groups:
            d, n, b, tiles = g["dev"], g["meta"]["maxn"], g["batch"], g["tiles"]
            rows = slice(row, row + b)
            sq = torch.arange(b, **i64)
            s3 = sq[:, None, None]
            entry[rows, :, :n] = torch.where(d["valid"], d["order"] | ENTRY_VFMT | (d["vcode"] == I8).to(torch.int64) << 29, 0)
            ks = torch.where(d["is4"], d["kslot"] + o4 + s3 * g["n4"], d["kslot"] + o8 + s3 * g["n8"])
            kinfo[rows, :, :n] = torch.where(d["valid"], d["kbase"] | (ks << 9), 0)
            vs = torch.where(d["vcode"] == I4, d["vslot"] + ov4 + s3 * g["nv"][I4], d["vslot"] + ov8 + s3 * g["nv"][I8])
            slot[rows, :, :n] = torch.where(d["valid"], vs, 0)
            count[rows] = d["count"]
            fmt[rows, :tiles] = d["fmt"]
            prompt[rows] = g["prompt"]
            for xs, h in enumerate(g["exact"]):
                xslot[rows, h] = ox + (sq * len(g["exact"]) + xs) * tiles
            ka[rows, :, :tiles] = g["ka"]
            if g["ka4"] is not None and ka4 is not None:
                ka4[rows, :, :tiles] = g["ka4"]
            kstat[rows] = g["kstat"]
            vstat[rows] = g["vstat"]
            k8s.append(g["k8"])
            if g["k4"] is not None:
                k4s.append(g["k4"])
            if g["v"][I8] is not None:
                v8s.append(g["v"][I8])
            if g["v"][I4] is not None:
                v4s.append(g["v"][I4])
            if g["exact"]:
                kxs.append(g["kx"])
                vxs.append(g["vx"])
                ox += b * len(g["exact"]) * tiles
            o8 += b * g["n8"]
            o4 += b * g["n4"]
            ov8 += b * g["nv"][I8]
            ov4 += b * g["nv"][I4]
            row += b
        cat = lambda parts, words: (torch.cat(parts) if sum(p.shape[0] for p in parts) else
                                    torch.zeros((1, words), dtype=torch.uint32, device=device))
        if self.wave is None:
            cus = self.module.device_cus() if hasattr(self.module, "device_cus") else \
                torch.cuda.get_device_properties(device).multi_processor_count
            self.wave = cus * max(1, min(self.module.decode_occupancy(), SPLITS_PER_CU))
        # Split partition, from the host metadata (no device sync).
        # - Up to BALANCE_TILES kept tiles per slot (one wave of SPLITS_PER_CU workgroups per CU;
        #   C1: 16384 tiles on 1024 slots): every SIMD runs one split, so the kernel lasts as
        #   long as its costliest split, and balanced_partition cuts the heads by cost (C1:
        #   36.9 us vs 39.6 us for runs of 16 tiles).
        # - Above that (C3: 48.8k tiles), runs of `per` tiles, as the reference splits
        #   (decode.py:54-55), over one wave of slots with every average head in at least 3
        #   splits: the dispatcher then balances the waves itself, and no partition tried did
        #   better (C3, two waves per workgroup: 121.5 us at 32 tiles per split, 127-128 at 24 or
        #   36, 129 at 16, 134 at 64; balanced over 4096-8192 slots 138-168 us).
        # - self.per set: always runs of that many tiles.  At most 64 tiles per split.
        kept = sum(g["batch"] * int(g["meta"]["count"].sum()) for g in groups)
        if self.per is None and kept <= BALANCE_TILES * self.wave:
            parts, splits = balanced_partition([g["meta"] for g in groups], [g["batch"] for g in groups], self.wave)
            bounds_host = torch.cat([p[None].expand(g["batch"], -1, -1) for p, g in zip(parts, groups)])
            per = int(bounds_host.diff(dim=2).max())
            bounds = bounds_host.to(device)
        else:
            mean = kept / max(1, total * hk)
            per = self.per or min(64, max(1, min(-(-kept // self.wave), math.ceil(mean / 3))))
            bounds_host = bounds = None
            splits = max(1, -(-maxn // per))
        to = lambda x: x.to(torch.int32).to(device)
        tail_k = torch.zeros((total, hk, self.max_tail, 128), dtype=torch.bfloat16, device=device)
        return dict(groups=groups, prompt=to(prompt), maxn=maxn, per=per, splits=splits, bounds=bounds,
                    bounds_host=None if bounds_host is None else bounds_host.numpy(), fmt=to(fmt), slot=to(slot),
                    entry=to(entry),
                    kinfo=to(kinfo), count=to(count), k8=cat(k8s, K8_WORDS), k4=cat(k4s, K4_WORDS) if has4 else None,
                    ka=ka, ka4=ka4, kstat=kstat, vstat=vstat, v={I8: cat(v8s, WORDS[I8]), I4: cat(v4s, WORDS[I4])},
                    tail_k=tail_k, tail_v=torch.zeros_like(tail_k), batch=total, tiles_max=tiles_max,
                    xslot=to(xslot) if kxs else None, kx=torch.cat(kxs) if kxs else None,
                    vx=torch.cat(vxs) if vxs else None)

    def __call__(self, layer, q, k, v, scale):
        e = self.layers[layer]
        hq = q.shape[1]
        splits = e["splits"]
        key = ("partials", hq)
        if key not in e:
            n = e["batch"] * hq * splits
            e[key] = (torch.empty(n, device=q.device), torch.empty(n, device=q.device),
                      torch.empty(n * 128, device=q.device))
        dtype = self.out_dtype or q.dtype
        out = torch.empty(q.shape, dtype=dtype, device=q.device)
        self.plan(layer, q, k, out, scale).run(q, k, v, out)
        return out

    def plan(self, layer, q, k, out, scale):
        """The layer's validated decode call for q / k (and v) / out of these shapes (built once, then reused)."""
        e = self.layers[layer]
        key = ("plan", _geometry(q), _geometry(k), _geometry(out), float(scale))
        if key not in e:
            hq = q.shape[1]
            e[key] = self.module.plan_decode(
                q, e["k8"], e["k4"], e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"], e["slot"],
                e["v"][I8], e["v"][I4], e["vstat"], e["kstat"], e["tail_k"], e["tail_v"], k, k, self.step, out,
                *e[("partials", hq)], e["prompt"], e["per"], scale, e["xslot"], e["kx"], e["vx"], e["bounds"])
        return e[key]

    def split_of(self, layer, b):
        """The split argument of the oracle's decode for sequence b of the layer: its bounds
        [Hk, splits + 1], or the uniform `per`."""
        e = self.layers[layer]
        return e["per"] if e["bounds_host"] is None else e["bounds_host"][b]

    def advance(self):
        self.step.add_(1)

    def stored(self, layer):
        return layer in self.layers
