"""Host restatements of the decode-cache launches (test infrastructure).

``host_cache_store`` fills a cache's arrays as ``tri_cache_store`` documents it, from the host metadata
``sequence_metadata`` (kernels/decode.py:27-53, pinned by brute-force enumeration in test_host.py), with
plain loops over sequences, KV heads and entries.  ``HostSpill`` restates ``tri_tail_spill`` (tail growth)
the same way, quantizing with the oracle's tail_tile.  The CPU tests run DecodeCache on them; the GPU tests
hold the kernels to them bit for bit."""
from __future__ import annotations

import numpy as np
import torch

import oracle as O
from triattention_amd.kernels import records as R
from triattention_amd.kernels.decode import ENTRY_VFMT, ENTRY_V8, NEAR_V8, sequence_metadata
from triattention_amd.kernels.prefill import I4, I8

WORDS = dict(k8=2048, k4=1024, v8=2048, v4=1024)
KX = 16384


def host_cache_store(bands, exact, t, kp, k4p, ka, ka4, kstat, vstat, v8p, v4p, kx, vx, nx, row0, dst, used, cap,
                     xstride=None):
    tiles = (t + 63) // 64
    xstride = tiles if xstride is None else xstride
    b, hk = vstat.shape[0], vstat.shape[1]
    exact_kv = [] if exact is None else [h for h in range(hk) if int(exact[h]) >= 0]
    j = torch.arange(tiles)
    vcodes = torch.where((tiles - 1 - j < NEAR_V8) | (j == 0), I8, I4)
    m = sequence_metadata(bands.cpu(), tiles, hk, vcodes, exact_kv)
    per = dict(k8=int(m["is8"].sum()), k4=int(m["is4"].sum()), v8=int(m["vsel"][I8].sum()),
               v4=int(m["vsel"][I4].sum()))
    src = {kind: (x.reshape(-1, WORDS[kind]) if x is not None else None)
           for kind, x in (("k8", kp), ("k4", k4p), ("v8", v8p), ("v4", v4p))}
    kas, ka4s = ka.reshape(b, hk, tiles, 4), ka4.reshape(b, hk, tiles, 4) if ka4 is not None else None
    for s in range(b):
        row = row0 + s
        dst["prompt"][row] = t
        dst["fmt"][row] = 1
        dst["fmt"][row, :tiles] = (vcodes - 1).to(torch.int32)
        for kh in range(hk):
            cnt = int(m["count"][kh])
            dst["count"][row, kh] = cnt
            for name in ("entry", "kinfo", "slot"):
                dst[name][row, kh] = 0
            rec = (s * hk + kh) * tiles
            for e in range(cnt):
                jj = int(m["order"][kh, e])
                vi8 = int(vcodes[jj]) == I8
                dst["entry"][row, kh, e] = jj | ENTRY_VFMT | (ENTRY_V8 if vi8 else 0)
                is4, is8 = bool(m["is4"][kh, e]), bool(m["is8"][kh, e])
                kind = "k4" if is4 else "k8"
                ks = used[kind] + s * per[kind] + int(m["kslot"][kh, e]) if (is4 or is8) else 0
                dst["kinfo"][row, kh, e] = int(m["kbase"][kh, e]) | (ks << 9)
                if is4 or is8:
                    vkind = "v8" if vi8 else "v4"
                    vs = used[vkind] + s * per[vkind] + int(m["vslot"][kh, e])
                    dst["slot"][row, kh, e] = vs
                    if ks < cap[kind]:
                        dst[kind][ks] = src[kind][rec + jj]
                    if vs < cap[vkind]:
                        dst[vkind][vs] = src[vkind][rec + jj]
            dst["ka"][row, kh] = 1.0
            dst["ka"][row, kh, :tiles] = kas[s, kh]
            if dst["ka4"] is not None:
                dst["ka4"][row, kh] = 1.0
                if ka4s is not None:
                    dst["ka4"][row, kh, :tiles] = ka4s[s, kh]
            dst["kstat"][row, kh] = kstat.reshape(b, hk, 3, 128)[s, kh]
            dst["vstat"][row, kh] = vstat.reshape(b, hk, 3, 128)[s, kh]
            if dst["xslot"] is not None:
                dst["xslot"][row, kh] = -1
            if kh in exact_kv:
                xs = exact_kv.index(kh)
                x0 = used["x"] + (s * nx + xs) * xstride
                dst["xslot"][row, kh] = x0
                n = tiles * KX
                first = (s * nx + xs) * tiles * KX
                dst["kx"][x0 * KX:x0 * KX + n] = kx.reshape(-1)[first:first + n]
                dst["vx"][x0 * KX:x0 * KX + n] = vx.reshape(-1)[first:first + n]


class HostCacheModule:
    """The module calls DecodeCache makes, on the host: four CUs, two resident decode workgroups per
    CU, and ``cache_store`` restated by ``host_cache_store``."""

    def device_cus(self):
        return 4

    def decode_occupancy(self):
        return 2

    def cache_store(self, *args, xstride=None):
        host_cache_store(*args, xstride=xstride)

    def plan_tail_spill(self, step, tail_base, ktail, vtail, grow, cap, prompt, dst, tasks=None):
        return HostSpill(step, tail_base, ktail, vtail, grow, cap, prompt, dst, tasks)


def pack_kx(k_bits, v_bits):
    """KX and VX records (16 KiB each, the layout tri_pack_exact documents) of one 64-key tile of bf16 bits
    [64, 128] (uint16)."""
    k = np.asarray(k_bits, np.uint16).reshape(64, 128)
    v = np.asarray(v_bits, np.uint16).reshape(64, 128)
    kx = np.zeros(8192, np.uint16)
    key, f0 = np.meshgrid(np.arange(64), np.arange(0, 128, 8), indexing="ij")
    off = (key >> 5) * 4096 + (f0 >> 4) * 512 + (((f0 >> 3) & 1) * 32 + (key & 31)) * 8  # uint16 units
    for e in range(8):
        kx[(off + e).ravel()] = k[key.ravel(), (f0 + e).ravel()]
    vx = np.zeros(8192, np.uint16)
    c = np.arange(1024)
    F, L = c >> 6, c & 63
    kb, cb, khalf, h = F >> 3, (F >> 1) & 3, F & 1, L >> 5
    ch = cb * 32 + (L & 31)
    for e in range(8):
        vx[c * 8 + e] = v[kb * 32 + 16 * khalf + 8 * (e >> 2) + 4 * h + (e & 3), ch]
    return kx.view(np.uint8), vx.view(np.uint8)


class HostSpill:
    """tri_tail_spill on host tensors, as its header documents it: when the tail is full and room is left,
    the oldest 64 rows of every (sequence, KV head) become tile ceil(prompt / 64) + tail_base / 64, the
    tail moves up by 64 and tail_base grows by 64; when any (sequence, KV head) lacks room for the tile,
    nothing changes."""

    def __init__(self, step, tail_base, ktail, vtail, grow, cap, prompt, dst, tasks):
        self.step, self.tail_base, self.ktail, self.vtail = step, tail_base, ktail, vtail
        self.grow, self.cap, self.prompt, self.dst, self.tasks = grow, int(cap), prompt, dst, tasks

    def has_room(self, k):
        """Room for spilled tile k in every (sequence, KV head), as the header states the rule."""
        d = self.dst
        rows, hk, maxn = d["entry"].shape
        tiles_max = d["fmt"].shape[1]
        n = {kind: 0 if d[kind] is None else d[kind].shape[0] for kind in ("k8", "k4", "v8")}
        n_kx = 0 if d["kx"] is None else d["kx"].numel() // 16384
        for row in range(rows):
            j = (int(self.prompt[row]) + 63) // 64 + k
            for kh in range(hk):
                if j >= tiles_max or int(d["count0"][row, kh]) + k >= maxn:
                    return False
                info, gk, gv, _ = (int(x) for x in self.grow[row, kh])
                x0 = int(d["xslot"][row, kh]) if d["xslot"] is not None else -1
                if x0 >= 0:
                    if x0 + j >= n_kx:
                        return False
                elif info >= 0:
                    is4 = (info >> 8) & 1
                    if gk + k >= n["k4" if is4 else "k8"] or gv + k >= n["v8"] or (is4 and d["ka4"] is None):
                        return False
        return True

    def run(self):
        d = self.dst
        rows, hk, maxn = d["entry"].shape
        tiles_max = d["fmt"].shape[1]
        max_tail = self.ktail.shape[2]
        tb = int(self.tail_base[0])
        if int(self.step[0]) - tb < max_tail or tb // 64 >= self.cap:
            return
        k = tb // 64
        if not self.has_room(k):
            return
        kbits = self.ktail.view(torch.int16).numpy().view(np.uint16)
        vbits = self.vtail.view(torch.int16).numpy().view(np.uint16)
        for row in range(rows):
            j = (int(self.prompt[row]) + 63) // 64 + k
            if j >= tiles_max:
                continue
            for kh in range(hk):
                info, gk, gv, tr = (int(x) for x in self.grow[row, kh])
                e = int(d["count"][row, kh])
                if e >= maxn:
                    continue
                if kh == 0:
                    d["fmt"][row, j] = 1
                x0 = int(d["xslot"][row, kh]) if d["xslot"] is not None else -1
                if x0 >= 0:
                    kx, vx = pack_kx(kbits[row, kh, :64], vbits[row, kh, :64])
                    rec = x0 + j
                    d["kx"][rec * 16384:(rec + 1) * 16384] = torch.from_numpy(kx.copy())
                    d["vx"][rec * 16384:(rec + 1) * 16384] = torch.from_numpy(vx.copy())
                    d["entry"][row, kh, e] = j | ENTRY_VFMT | ENTRY_V8
                    d["kinfo"][row, kh, e] = info & 0xFF
                    d["slot"][row, kh, e] = 0
                    d["count"][row, kh] = e + 1
                    continue
                if info < 0:
                    continue
                is4 = (info >> 8) & 1
                ks, vs = gk + k, gv + k
                kstat = d["kstat"][row, kh].numpy()[None]
                vstat = d["vstat"][row, kh].numpy()[None]
                t = O.tail_tile(kbits[row, kh, :64][None], vbits[row, kh, :64][None], kstat, vstat)
                if is4:
                    d["k4"][ks] = torch.from_numpy(R.pack_k4(t["k4"][0]).view(np.uint32).reshape(-1).copy())
                    d["ka4"][row, kh, j] = torch.from_numpy(t["ka4"][0, 0])
                    scales = t["ka4"][0, 0]
                else:
                    d["k8"][ks] = torch.from_numpy(R.pack_k8(t["k8"][0]).view(np.uint32).reshape(-1).copy())
                    d["ka"][row, kh, j] = torch.from_numpy(t["ka"][0, 0])
                    scales = t["ka"][0, 0]
                d["v8"][vs] = torch.from_numpy(R.pack_v8(t["v8"][0]).view(np.uint32).reshape(-1).copy())
                d["entry"][row, kh, e] = j | ENTRY_VFMT | ENTRY_V8
                d["kinfo"][row, kh, e] = (info & 0x1FF) | (ks << 9)
                d["slot"][row, kh, e] = vs
                d["count"][row, kh] = e + 1
                if self.tasks is not None and tr >= 0:
                    table, n = self.tasks
                    row_t = tr + k // 64
                    if row_t < n:
                        lane = k % 64
                        w = table[row_t * 512:(row_t + 1) * 512]
                        w[4 * lane] = ks
                        w[4 * lane + 1] = vs
                        w[4 * lane + 2] = (info & 0x1FF) | (1 << 9) | (j << 10)
                        if lane > 0:
                            w[4 * lane + 3] = lane + 1
                        w[7] = lane + 1
                        w.view(torch.float32)[256 + 4 * lane:256 + 4 * lane + 4] = torch.from_numpy(scales)
        self.ktail[:, :, :max_tail - 64] = self.ktail[:, :, 64:].clone()
        self.vtail[:, :, :max_tail - 64] = self.vtail[:, :, 64:].clone()
        self.tail_base[0] = tb + 64
