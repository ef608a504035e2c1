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

Extension: tail growth (``grow_tail`` > 0).  The reference's tail holds
max_tail generated tokens and then overwrites its last slot
(common_device.cuh:384).  Here each layer's decode step first launches
``tail_spill``: when the tail is full, its oldest 64 tokens become a new tile
of the cache (quantized with the prompt's statistics, classified as the newest
tile) and the tail moves up by 64 slots.  The store reserves room for
``grow_tail`` tokens of such tiles per (sequence, KV head); the decode's
partition gets growth splits that fill as tiles arrive, so every launch's
arguments stay the same until the room runs out (a captured step replays
unchanged), and the cache then doubles the room.
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
BN = 64  # tokens per tile (and per move of a full tail into the cache)


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


def growth_kinds(bands, hk: int, exact_kv=()):
    """Per KV head, how a tile taken from a full tail is kept (extension): kind 8 / 4 (K precision),
    1 (exact head) or 0 (no q-head keeps it), and its kinfo bits (rowmask | INT4 K << 8).  The tile is
    classified as the newest tile of the cache, d = 0 in decode.py:27-33: state 8 for a q-head with
    w8 > 0, else 4 with w4 > 0, else 0."""
    b = torch.as_tensor(bands, dtype=torch.int64).cpu().view(-1, 2).numpy()
    g = b.shape[0] // hk
    state = np.where(b[:, 0] > 0, 8, np.where(b[:, 1] > 0, 4, 0)).reshape(hk, g)
    kind = state.max(1)
    mask = ((state > 0).astype(np.int64) << np.arange(g)[None, :]).sum(1)
    info = np.where(kind > 0, (mask & 0xFF) | ((kind == 4).astype(np.int64) << 8), -1)
    for h in exact_kv:
        kind[h], info[h] = 1, (1 << g) - 1
    return kind.astype(np.int64), info.astype(np.int32)


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


class _LayerStore:
    """A layer's decode-cache arrays on the device, with room to append sequences: per-sequence rows
    (metadata [rows][hk][maxn], scales [rows][hk][tiles_max][4], statistics, bf16 tails) and the
    compacted record arrays.  ``n`` counts the records in use, ``cap`` what each array holds.  Growing
    copies what is stored (amortised by doubling in ragged mode); nothing stored is recomputed."""

    RECORD = dict(k8=(K8_WORDS, torch.uint32), k4=(K4_WORDS, torch.uint32), v8=(WORDS[I8], torch.uint32),
                  v4=(WORDS[I4], torch.uint32))

    def __init__(self, hk, max_tail, device):
        self.hk, self.max_tail, self.device = hk, max_tail, device
        self.rows = self.maxn = self.tiles_max = 0
        self.n = dict(k8=0, k4=0, v8=0, v4=0, x=0)
        self.cap = dict(rows=0, k8=0, k4=0, v8=0, v4=0, x=0)
        self.arrays = {name: None for name in ("entry", "kinfo", "slot", "count", "fmt", "prompt", "xslot", "ka",
                                               "ka4", "kstat", "vstat", "tail_k", "tail_v", "k8", "k4", "v8", "v4",
                                               "kx", "vx", "grow", "count0")}
        self.groups = []
        # tail growth: tiles of room per (sequence, KV head), and the host's mirror of the device's
        # tail base (tokens moved from the tail into the cache since the store)
        self.grow_tiles = 0
        self.tb = 0
        self.arrays["tail_base"] = torch.zeros(2, dtype=torch.int64, device=device)

    def _regrow(self, name, shape, fill, dtype):
        """Array ``name`` at ``shape``, filled with ``fill`` and holding the old contents in its corner."""
        old = self.arrays[name]
        if old is not None and tuple(old.shape) == tuple(shape):
            return
        new = torch.full(shape, fill, dtype=dtype, device=self.device) if fill is not None else \
            torch.zeros(shape, dtype=dtype, device=self.device)
        if old is not None:
            new[tuple(slice(0, min(o, n)) for o, n in zip(old.shape, shape))] = \
                old[tuple(slice(0, min(o, n)) for o, n in zip(old.shape, shape))]
        self.arrays[name] = new

    def reserve(self, rows, maxn, tiles_max, records, int4, exact, ragged):
        """Make room for ``rows`` sequences with metadata rows of ``maxn`` entries over ``tiles_max``
        tiles and ``records`` (per kind) records."""
        grow = (lambda need, cap: max(need, 2 * cap) if need > cap else cap) if ragged else \
            (lambda need, cap: max(need, cap))
        cap_rows = grow(rows, self.cap["rows"])
        relayout = cap_rows != self.cap["rows"] or maxn != self.maxn or tiles_max != self.tiles_max
        self.cap["rows"], self.maxn, self.tiles_max = cap_rows, maxn, tiles_max
        hk, i32, f32 = self.hk, torch.int32, torch.float32
        if relayout:
            for name in ("entry", "kinfo", "slot"):
                self._regrow(name, (cap_rows, hk, maxn), 0, i32)
            self._regrow("count", (cap_rows, hk), 0, i32)
            self._regrow("fmt", (cap_rows, tiles_max), 1, i32)
            self._regrow("prompt", (cap_rows,), 0, i32)
            self._regrow("ka", (cap_rows, hk, tiles_max, 4), 1.0, f32)
            self._regrow("kstat", (cap_rows, hk, 3, 128), 0.0, f32)
            self._regrow("vstat", (cap_rows, hk, 3, 128), 0.0, f32)
            for name in ("tail_k", "tail_v"):
                self._regrow(name, (cap_rows, hk, self.max_tail, 128), 0.0, torch.bfloat16)
            self._regrow("grow", (cap_rows, hk, 4), -1, i32)
            self._regrow("count0", (cap_rows, hk), 0, i32)
        if (int4 or self.arrays["ka4"] is not None) and (relayout or self.arrays["ka4"] is None):
            self._regrow("ka4", (cap_rows, hk, tiles_max, 4), 1.0, f32)
        if (exact or self.arrays["xslot"] is not None) and (relayout or self.arrays["xslot"] is None):
            self._regrow("xslot", (cap_rows, hk), -1, i32)
        for kind, (words, dtype) in self.RECORD.items():
            # the decode op takes non-empty K8 / V8 / V4 arrays: at least one (zero) record each
            need = max(records[kind], 1 if kind != "k4" else 0)
            if kind == "k4" and not int4 and self.arrays["k4"] is None:
                continue
            cap = grow(max(need, 1), self.cap[kind])
            if cap != self.cap[kind] or self.arrays[kind] is None:
                self._regrow(kind, (cap, words), None, dtype)
                self.cap[kind] = cap
        if exact or self.arrays["kx"] is not None:
            cap = grow(max(records["x"], 1), self.cap["x"])
            if cap != self.cap["x"] or self.arrays["kx"] is None:
                self._regrow("kx", (cap * KX_BYTES,), None, torch.uint8)
                self._regrow("vx", (cap * KX_BYTES,), None, torch.uint8)
                self.cap["x"] = cap


class DecodeCache:
    def __init__(self, module, max_tail=256, grow_tail=0):
        self.module, self.max_tail = module, max_tail
        self.layers, self.formats, self.step = {}, {}, None
        self.ragged = False
        self.out_dtype = None
        self.meta_cache = {}
        self.wave = None
        # None: the balanced split partition; an int: the reference's uniform split of `per` tiles
        self.per = None
        # the split kernel reads its splits from a task table built once per cache layout (False: it
        # gathers them from the metadata rows, as the reference's kernel does)
        self.tasks = True
        # tail growth (extension): tokens of room per (sequence, KV head) for tiles taken from a full
        # tail (0: the reference's clamped tail)
        if grow_tail and max_tail < BN:
            raise ValueError(f"tail growth moves {BN} tokens at a time: max_tail must be at least {BN}")
        self.grow_tail = int(grow_tail)
        # host mirror of the device step (the tail base of each layer is mirrored in its store), the
        # layers called since the last advance, and graph capture bookkeeping
        self.host_step = 0
        self._called = set()
        self.capturing = False
        self._capture_set = set()

    def codes(self, rows):
        if rows not in self.formats:
            j = torch.arange(rows)
            codes = torch.where((rows - 1 - j < NEAR_V8) | (j == 0), I8, I4)
            self.formats[rows] = codes, frozenset(codes.unique().tolist())
        return self.formats[rows]

    def store(self, layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv=(), kx=None,
              vx=None):
        """Keep one Prefill call's records (decode.py:24-67).

        One device launch (``cache_store``) classifies the prompt's tiles, writes the batch's metadata
        rows and copies the kept records, scales and statistics into the layer's own arrays, so the
        Prefill may reuse every buffer it passed here.  With ``ragged = True`` the batch is appended
        after the layer's earlier sequences (arrays grow geometrically; earlier rows are never
        rebuilt); otherwise it replaces them.  Extension: ``exact_kv`` lists the KV heads kept in
        bf16, whose KX/VX records ``kx``/``vx`` ([B][len(exact_kv)][tiles], tri_pack_exact layout)
        are copied whole."""
        tiles = (prompt + 63) // 64
        batch = vstat.shape[0]
        hk, device = vstat.shape[1], ka.device
        exact_kv = sorted(set(int(h) for h in exact_kv))
        meta, dev = self._metadata(bands, tiles, hk, codes, exact_kv, device)
        hq = dev["bands"].shape[0]
        entry = self.layers.get(layer)
        st = entry["store"] if (self.ragged and entry is not None) else _LayerStore(hk, self.max_tail, device)
        if st.hk != hk:
            raise ValueError(f"decode cache layer {layer}: {hk} KV heads after {st.hk}")
        if self.grow_tail and not st.grow_tiles:
            st.grow_tiles = -(-self.grow_tail // BN)
        G = st.grow_tiles
        kind, info = growth_kinds(bands, hk, exact_kv) if G else (np.zeros(hk, np.int64), np.full(hk, -1, np.int32))
        nx = len(exact_kv)
        xstride = tiles + G
        seq = dict(k8=int(meta["is8"].sum()), k4=int(meta["is4"].sum()), v8=int(meta["vsel"][I8].sum()),
                   v4=int(meta["vsel"][I4].sum()), x=nx * xstride)
        # growth room per sequence: G records per KV head of each kind (V always INT8)
        room = dict(k8=int((kind == 8).sum()) * G, k4=int((kind == 4).sum()) * G,
                    v8=int(((kind == 8) | (kind == 4)).sum()) * G, v4=0, x=0)
        row0 = st.rows
        int4 = k4 is not None or ka4 is not None or bool(room["k4"])
        st.reserve(row0 + batch, max(st.maxn, meta["maxn"] + G), max(st.tiles_max, tiles + G),
                   {k: st.n[k] + batch * (seq[k] + room[k]) for k in seq}, int4, bool(exact_kv), ragged=self.ragged)
        used = dict(st.n)
        self.module.cache_store(dev["bands"], dev["exact"], prompt, kp, k4, ka, ka4, kstat, vstat, packed[I8],
                                packed.get(I4), kx, vx, nx, row0, st.arrays, used, st.cap, xstride=xstride)
        a = st.arrays
        if G:
            # growth regions after the batch's prompt records: sequence s, head h of kind K takes G records
            # from base_K + (s * heads_K + rank of h among them) * G
            grow = np.full((batch, hk, 4), -1, np.int32)
            grow[:, :, 0] = info[None, :]
            for rec, sel in (("k8", kind == 8), ("k4", kind == 4)):
                heads = np.flatnonzero(sel)
                base = st.n[rec] + batch * seq[rec]
                for r, h in enumerate(heads):
                    grow[:, h, 1] = base + (np.arange(batch) * len(heads) + r) * G
            vheads = np.flatnonzero((kind == 8) | (kind == 4))
            vbase = st.n["v8"] + batch * seq["v8"]
            for r, h in enumerate(vheads):
                grow[:, h, 2] = vbase + (np.arange(batch) * len(vheads) + r) * G
            a["grow"][row0:row0 + batch].copy_(torch.from_numpy(grow))
        a["count0"][row0:row0 + batch].copy_(a["count"][row0:row0 + batch])
        if self.ragged and row0:
            a["count"][:row0].copy_(a["count0"][:row0])  # the earlier rows' tiles taken from their tails go
        st.rows += batch
        for k in seq:
            st.n[k] += batch * (seq[k] + room[k])
        st.groups.append(dict(prompt=prompt, batch=batch, hk=hk, tiles=tiles, meta=meta, exact=exact_kv, row0=row0,
                              kind=kind, xstride=xstride, ox=used["x"]))
        if self.step is None:
            self.step = torch.zeros(1, dtype=torch.int64, device=device)
        self.step.zero_()
        self.host_step = 0
        st.tb = 0
        a["tail_base"].zero_()
        a["tail_k"][:st.rows].zero_()
        a["tail_v"][:st.rows].zero_()
        self.layers[layer] = self._assemble(st)

    def _metadata(self, bands, tiles, hk, codes, exact_kv, device):
        """One sequence's metadata (host, closed-form integer code: the record counts that size the
        cache's arrays and the entry costs of the split partition) with the device copies the store
        launch reads, cached per (bands, tiles, KV heads, exact heads, device): every sequence of the
        same length shares it."""
        b = torch.as_tensor(bands, dtype=torch.int32).cpu().contiguous()
        key = (b.numpy().tobytes(), tiles, hk, tuple(exact_kv), str(device))
        hit = self.meta_cache.get(key)
        if hit is None:
            meta = sequence_metadata(b, tiles, hk, codes, exact_kv)
            flags = torch.full((hk,), -1, dtype=torch.int32)
            for xs, h in enumerate(exact_kv):
                flags[h] = xs
            dev = dict(bands=b.to(device), exact=flags.to(device) if exact_kv else None)
            hit = self.meta_cache[key] = (meta, dev)
        return hit

    def _assemble(self, st):
        """The layer entry the decode op reads: views of the store's arrays over its sequences, and the
        split partition over every stored group (host metadata, no device sync)."""
        groups, device = st.groups, st.device
        a, rows = st.arrays, st.rows
        if self.wave is None:
            cus = self.module.device_cus() if hasattr(self.module, "device_cus") else \
                torch.cuda.get_device_properties(device).multi_processor_count
            self.wave = cus * max(1, min(self.module.decode_occupancy(), SPLITS_PER_CU))
        # Split partition, from the host metadata (no device sync).
        # - Up to BALANCE_TILES kept tiles per slot (one wave of SPLITS_PER_CU workgroups per CU;
        #   C1: 16384 tiles on 1024 slots): every SIMD runs one split, so the kernel lasts as
        #   long as its costliest split, and balanced_partition cuts the heads by cost (C1:
        #   36.9 us vs 39.6 us for runs of 16 tiles).
        # - Above that (C3: 49.1k tiles), runs of `per` tiles, as the reference splits
        #   (decode.py:54-55), over one wave of slots with every average head in about 3.5
        #   splits: the dispatcher then balances the waves itself, and no partition tried did
        #   better (C3, two waves per workgroup, listed splits, median of 3 rounds on one box:
        #   102.1 us at 28 tiles per split, 103.2 at 30, 104.4 at 32, 105.2 at 26, 106.7 at 24,
        #   108.2 at 36; balanced over 4096-8192 slots 138-168 us in an earlier build).
        # - self.per set: always runs of that many tiles.  At most 64 tiles per split.
        kept = sum(g["batch"] * int(g["meta"]["count"].sum()) for g in groups)
        if self.per is None and kept <= BALANCE_TILES * self.wave:
            parts, splits = balanced_partition([g["meta"] for g in groups], [g["batch"] for g in groups], self.wave)
            bounds_host = torch.cat([p[None].expand(g["batch"], -1, -1) for p, g in zip(parts, groups)])
            per = int(bounds_host.diff(dim=2).max())
            bounds = bounds_host.to(device)
        else:
            mean = kept / max(1, rows * st.hk)
            per = self.per or min(64, max(1, min(-(-kept // self.wave), math.ceil(mean / 3.5))))
            bounds_host = bounds = None
            splits = max(1, -(-st.maxn // per))
        if st.grow_tiles:
            # tail growth: growth splits of 64 entries after each head's prompt entries (split_range
            # clamps them to the head's count, which grows as tiles arrive)
            counts = torch.from_numpy(np.concatenate(
                [np.repeat(g["meta"]["count"].numpy()[None], g["batch"], 0) for g in groups]).astype(np.int32))
            if bounds_host is None:
                runs = -(-int(counts.max()) // per)
                bounds_host = torch.minimum(torch.arange(runs + 1, dtype=torch.int32)[None, None, :] * per,
                                            counts[:, :, None])
            extra = torch.minimum(torch.arange(1, -(-st.grow_tiles // 64) + 1, dtype=torch.int32) * 64,
                                  torch.tensor(st.grow_tiles, dtype=torch.int32))
            bounds_host = torch.cat([bounds_host, counts[:, :, None] + extra[None, None, :]], 2).contiguous()
            splits = bounds_host.shape[2] - 1
            per = int(bounds_host.diff(dim=2).max())
            bounds = bounds_host.to(device)
        some = lambda name, n: a[name][:max(1, n)]
        has_x = any(g["exact"] for g in groups)
        return dict(groups=groups, store=st, prompt=a["prompt"][:rows], maxn=st.maxn, per=per, splits=splits,
                    bounds=bounds, bounds_host=None if bounds_host is None else bounds_host.numpy(),
                    fmt=a["fmt"][:rows], slot=a["slot"][:rows], entry=a["entry"][:rows], kinfo=a["kinfo"][:rows],
                    count=a["count"][:rows], k8=some("k8", st.n["k8"]),
                    k4=some("k4", st.n["k4"]) if a["k4"] is not None else None, ka=a["ka"][:rows],
                    ka4=a["ka4"][:rows] if a["ka4"] is not None else None, kstat=a["kstat"][:rows],
                    vstat=a["vstat"][:rows], v={I8: some("v8", st.n["v8"]), I4: some("v4", st.n["v4"])},
                    tail_k=a["tail_k"][:rows], tail_v=a["tail_v"][:rows], batch=rows, tiles_max=st.tiles_max,
                    xslot=a["xslot"][:rows] if has_x else None,
                    kx=a["kx"][:st.n["x"] * KX_BYTES] if has_x else None,
                    vx=a["vx"][:st.n["x"] * KX_BYTES] if has_x else None,
                    grow_splits=-(-st.grow_tiles // 64) if st.grow_tiles else 0)

    def _grow_step(self, layer):
        """Tail growth bookkeeping before a decode step of ``layer``: when the tail is full and the room
        for tiles taken from it is used up, the room doubles (a new layer entry).  Returns the entry."""
        e = self.layers[layer]
        st = e["store"]
        if st.grow_tiles:
            if self.capturing:
                self._capture_set.add(layer)
            else:
                if self.host_step - st.tb >= self.max_tail and st.tb // BN >= st.grow_tiles:
                    self._extend(st)
                    e = self.layers[layer] = self._assemble(st)
                self._called.add(layer)
        return e

    def __call__(self, layer, q, k, v, scale):
        e = self._grow_step(layer)
        st = e["store"]
        dtype = self.out_dtype or q.dtype
        out = torch.empty(q.shape, dtype=dtype, device=q.device)
        plan = self.plan(layer, q, k, out, scale)
        if st.grow_tiles:
            self._spill_plan(e).run()
        plan.run(q, k, v, out, short_tail=self.short_tail(layer, q.shape[1]))
        return out

    # the merge runs as one wave per (sequence, q-head) while the tail holds at most SHORT_TAIL tokens on a
    # grid of at least SHORT_WIDE (sequence, q-head) workgroups per CU (the rule of tri_decode's merge)
    SHORT_TAIL = 16
    SHORT_WIDE = 2

    def tail_tokens(self, layer):
        """Tokens the merge of ``layer``'s next decode step reads from its tail (host mirror): the
        step's own token and those before it, past the tokens moved into the cache (after this step's
        spill, if it finds the tail full with room left), at most max_tail."""
        st = self.layers[layer]["store"]
        tb = st.tb if st.grow_tiles else 0
        if st.grow_tiles and self.host_step - tb >= self.max_tail and tb // BN < st.grow_tiles:
            tb += BN
        return min(self.max_tail - 1, max(0, self.host_step - tb)) + 1

    def short_tail(self, layer, hq):
        """Whether ``layer``'s next merge (hq q-heads) launches the one-wave kernel: tail_tokens at most
        SHORT_TAIL on a grid of at least SHORT_WIDE (sequence, q-head) workgroups per CU, the rule by
        which tri_decode's merge picks its form on the device, so that an eager step gives the bits a
        replayed graph gives.  A step being captured launches tri_decode's merge, which makes the choice
        itself at every replay (a captured one-wave launch would keep that form at later, longer tails)."""
        if self.capturing:
            return False
        if self.layers[layer]["batch"] * hq < self.SHORT_WIDE * self.module.device_cus():
            return False
        return self.tail_tokens(layer) <= self.SHORT_TAIL

    def plan(self, layer, q, k, out, scale):
        """The layer's validated decode call for q / k (and v) / out of these shapes (built once, then reused)."""
        e = self.layers[layer]
        key = ("partials", q.shape[1])
        if key not in e:
            # every slot starts as the empty partial: splits that hold no kept tile are left out of the
            # launch (the task table lists the others) and keep it
            n = e["batch"] * q.shape[1] * e["splits"]
            e[key] = (torch.full((n,), -3.4028234663852886e38, device=q.device), torch.zeros(n, device=q.device),
                      torch.zeros(n * 128, device=q.device))
        key = ("plan", _geometry(q), _geometry(k), _geometry(out), float(scale))
        if key not in e:
            hq = q.shape[1]
            if self.tasks and e["xslot"] is None and "tasks" not in e and hasattr(self.module, "decode_tasks"):
                items_host = self._task_items(e)
                items = torch.from_numpy(items_host).to(q.device)
                e["tasks"] = self.module.decode_tasks(e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"],
                                                      e["slot"], e["per"], e["bounds"], items)
                if e["grow_splits"]:
                    # task row of each head's first growth split (a head's growth splits are empty at the
                    # store, so they are listed last, consecutively, in item order)
                    first = np.arange(e["batch"] * e["store"].hk, dtype=np.int64) * e["splits"] + \
                        (e["splits"] - e["grow_splits"])
                    where = np.full(int(items_host.max()) + 1, -1, np.int64)
                    where[items_host] = np.arange(items_host.size)
                    rows = where[first].astype(np.int32)
                    e["store"].arrays["grow"][:e["batch"], :, 3].copy_(
                        torch.from_numpy(rows.reshape(e["batch"], e["store"].hk)))
            e[key] = self.module.plan_decode(
                q, e["k8"], e["k4"], e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"], e["slot"],
                e["v"][I8], e["v"][I4], e["vstat"], e["kstat"], e["tail_k"], e["tail_v"], k, k, self.step, out,
                *e[("partials", hq)], e["prompt"], e["per"], scale, e["xslot"], e["kx"], e["vx"], e["bounds"],
                e.get("tasks") if self.tasks else None,
                tail_base=e["store"].arrays["tail_base"] if e["grow_splits"] else None)
        return e[key]

    def _spill_plan(self, e):
        """The layer's tail_spill launch (tail growth), built once per cache layout."""
        if "spill" not in e:
            st, a, rows = e["store"], e["store"].arrays, e["batch"]
            if "tasks" not in e or not self.tasks:
                a["grow"][:rows, :, 3].fill_(-1)
            dst = dict(entry=e["entry"], kinfo=e["kinfo"], slot=e["slot"], count=e["count"],
                       count0=a["count0"][:rows], fmt=e["fmt"],
                       xslot=e["xslot"], ka=e["ka"], ka4=e["ka4"], kstat=e["kstat"], vstat=e["vstat"], k8=e["k8"],
                       k4=e["k4"], v8=e["v"][I8], kx=e["kx"], vx=e["vx"])
            e["spill"] = self.module.plan_tail_spill(self.step, a["tail_base"], e["tail_k"], e["tail_v"],
                                                     a["grow"][:rows], st.grow_tiles, e["prompt"], dst,
                                                     e.get("tasks") if self.tasks else None)
        return e["spill"]

    def _extend(self, st):
        """Double the room for tiles taken from the tail (when a full tail finds it used up): each
        (sequence, KV head) gets a new run of records twice as long, the tiles already taken move to its
        start (records and metadata), and the metadata rows, scales and exact-head records grow to fit."""
        g0, g1 = st.grow_tiles, 2 * st.grow_tiles
        n = st.tb // BN  # tiles taken so far (all sequences alike)
        a = st.arrays
        rows, hk = st.rows, st.hk
        room = dict(k8=0, k4=0, v8=0, v4=0, x=0)
        for g in st.groups:
            room["k8"] += g["batch"] * int((g["kind"] == 8).sum()) * g1
            room["k4"] += g["batch"] * int((g["kind"] == 4).sum()) * g1
            room["v8"] += g["batch"] * int(((g["kind"] == 8) | (g["kind"] == 4)).sum()) * g1
        st.reserve(rows, st.maxn + g1 - g0, st.tiles_max + g1 - g0, {k: st.n[k] + room[k] for k in room},
                   a["k4"] is not None, a["kx"] is not None, ragged=self.ragged)
        grow = a["grow"][:rows].cpu().numpy()
        count0 = a["count0"][:rows].cpu().numpy()
        new = grow.copy()
        moves = {"k8": ([], []), "k4": ([], []), "v8": ([], [])}
        meta_idx, kinfo_val, slot_val = [], [], []
        base = dict(st.n)
        for r in range(rows):
            for h in range(hk):
                info, gk, gv = int(grow[r, h, 0]), int(grow[r, h, 1]), int(grow[r, h, 2])
                if info < 0 or gk < 0:
                    continue
                rec = "k4" if (info >> 8) & 1 else "k8"
                new[r, h, 1], new[r, h, 2] = base[rec], base["v8"]
                moves[rec][0].extend(range(gk, gk + n))
                moves[rec][1].extend(range(base[rec], base[rec] + n))
                moves["v8"][0].extend(range(gv, gv + n))
                moves["v8"][1].extend(range(base["v8"], base["v8"] + n))
                for i in range(n):
                    meta_idx.append((r, h, int(count0[r, h]) + i))
                    kinfo_val.append((info & 0x1FF) | ((base[rec] + i) << 9))
                    slot_val.append(base["v8"] + i)
                base[rec] += g1
                base["v8"] += g1
        for rec, (src, dst) in moves.items():
            if src:
                arr = a[rec].view(torch.int32)  # (no indexed copies on uint32 tensors)
                arr[torch.tensor(dst, device=arr.device)] = arr[torch.tensor(src, device=arr.device)]
        if meta_idx:
            idx = torch.tensor(meta_idx, dtype=torch.int64).T.to(a["kinfo"].device)
            a["kinfo"][idx[0], idx[1], idx[2]] = torch.tensor(kinfo_val, dtype=torch.int32, device=idx.device)
            a["slot"][idx[0], idx[1], idx[2]] = torch.tensor(slot_val, dtype=torch.int32, device=idx.device)
        a["grow"][:rows].copy_(torch.from_numpy(new))
        for k in room:
            st.n[k] += room[k]
        if a["kx"] is not None and any(g["exact"] for g in st.groups):
            # exact heads address tile j at xslot + j: give each (sequence, exact head) a longer run
            kx, vx = a["kx"].view(-1, KX_BYTES), a["vx"].view(-1, KX_BYTES)
            total = sum(g["batch"] * len(g["exact"]) * (g["xstride"] + g1 - g0) for g in st.groups)
            nkx = torch.zeros((max(1, total), KX_BYTES), dtype=torch.uint8, device=kx.device)
            nvx = torch.zeros_like(nkx)
            xslot = a["xslot"][:rows].cpu().numpy()
            off = 0
            for g in st.groups:
                nx, xs0 = len(g["exact"]), g["xstride"]
                xs1 = xs0 + g1 - g0
                for s in range(g["batch"]):
                    for i, h in enumerate(g["exact"]):
                        old = g["ox"] + (s * nx + i) * xs0
                        dst = off + (s * nx + i) * xs1
                        nkx[dst:dst + xs0] = kx[old:old + xs0]
                        nvx[dst:dst + xs0] = vx[old:old + xs0]
                        xslot[g["row0"] + s, h] = dst
                g["ox"], g["xstride"] = off, xs1
                off += g["batch"] * nx * xs1
            a["kx"], a["vx"] = nkx.view(-1), nvx.view(-1)
            a["xslot"][:rows].copy_(torch.from_numpy(xslot))
            st.n["x"] = st.cap["x"] = max(1, total)
        st.grow_tiles = g1

    @staticmethod
    def _task_items(e):
        """Work items ((sequence * Hk + head) * splits + split) of the splits that hold kept tiles (and every
        growth split), from the host metadata: a split of the balanced partition is empty when its bounds
        coincide, one of the uniform runs when it starts past its head's count.  Ordered costliest first
        (the split kernel's measured time per tile kind, entry_costs; ties by item): the kernel deals the
        listed splits to the XCDs round-robin in this order, so the long splits start first and every XCD
        gets its share of each cost."""
        groups = e["groups"]
        counts = np.concatenate([np.repeat(g["meta"]["count"].numpy()[None], g["batch"], 0) for g in groups])
        per_group = [entry_costs(g["meta"]) for g in groups]
        width = max(c.shape[1] for c in per_group)
        costs = np.concatenate([np.repeat(np.pad(c, ((0, 0), (0, width - c.shape[1])))[None], g["batch"], 0)
                                for c, g in zip(per_group, groups)])
        cum = np.concatenate([np.zeros(costs.shape[:2] + (1,)), costs.cumsum(2)], 2)
        if e["bounds_host"] is not None:
            b = np.minimum(e["bounds_host"], counts[:, :, None])
            nonempty = e["bounds_host"][:, :, 1:] > e["bounds_host"][:, :, :-1]
        else:
            first = np.arange(e["splits"])[None, None, :] * e["per"]
            nonempty = first < counts[:, :, None]
            b = np.minimum(np.concatenate([first, first[:, :, -1:] + e["per"]], 2), counts[:, :, None])
        b = np.minimum(b, width)
        split_cost = np.take_along_axis(cum, b[:, :, 1:], 2) - np.take_along_axis(cum, b[:, :, :-1], 2)
        items = np.flatnonzero(nonempty.reshape(-1)).astype(np.int32)
        if not items.size:
            return np.zeros(1, np.int32)
        order = np.lexsort((items, -split_cost.reshape(-1)[items]))
        return items[order]

    def split_of(self, layer, b):
        """The split argument of the oracle's decode for sequence b of the layer: its bounds
        [Hk, splits + 1], or the uniform `per`."""
        e = self.layers[layer]
        return e["per"] if e["bounds_host"] is None else e["bounds_host"][b]

    def advance(self):
        self.step.add_(1)
        if not self.capturing:
            self._mirror(self._called)
            self._called = set()

    def _mirror(self, layers):
        """Host mirror of one step: the device's tail base of each layer in ``layers`` moves by 64 when
        that step found its tail full with room left (tail_spill's rule), and the step counter by one."""
        for layer in layers:
            st = self.layers[layer]["store"]
            if st.grow_tiles and self.host_step - st.tb >= self.max_tail and st.tb // BN < st.grow_tiles:
                st.tb += BN
        self.host_step += 1

    # ---- graph capture of decode steps (extension): the launches of a step stay the same while no
    # layer has to grow its room for tiles taken from the tail
    def begin_capture(self):
        self.capturing = True
        self._capture_set = set()

    def end_capture(self):
        self.capturing = False

    def graph_ready(self) -> bool:
        """Whether a captured step can replay now: no captured layer finds its tail full with its room
        used up (that step must run eagerly, which grows the room, and the step be captured again)."""
        for layer in self._capture_set:
            st = self.layers[layer]["store"]
            if st.grow_tiles and self.host_step - st.tb >= self.max_tail and st.tb // BN >= st.grow_tiles:
                return False
        return True

    def replayed(self):
        """Record one replay of a captured step (the host mirror of its spills and step advance)."""
        self._mirror(self._capture_set)

    def stored(self, layer):
        return layer in self.layers
