"""Host restatement of the decode-cache store launch (test infrastructure).

``host_cache_store`` fills a cache's arrays as ``tri_cache_store`` documents it, from the host metadata
``sequence_metadata`` (kernels/decode.py:27-53, pinned by brute-force enumeration in test_host.py), with
plain loops over sequences, KV heads and entries.  The CPU tests run DecodeCache on it; the GPU tests
hold the kernel to it bit for bit."""
from __future__ import annotations

import torch

from triattention_amd.kernels.decode import ENTRY_VFMT, ENTRY_V8, NEAR_V8, sequence_metadata
from triattention_amd.kernels.prefill import I4, I8

WORDS = dict(k8=2048, k4=1024, v8=2048, v4=1024)
KX = 16384


def host_cache_store(bands, exact, t, kp, k4p, ka, ka4, kstat, vstat, v8p, v4p, kx, vx, nx, row0, dst, used, cap):
    tiles = (t + 63) // 64
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
                x0 = used["x"] + (s * nx + xs) * tiles
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

    def cache_store(self, *args):
        host_cache_store(*args)
