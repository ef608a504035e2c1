"""The device-side decode-cache build (tri_cache_store) against its host restatement, bit for bit.

Each Prefill call's store goes to the GPU cache and, with the same source buffers copied to the host, to
a host cache whose module restates the launch from ``sequence_metadata`` (tests/cache_host.py).  Every
array the decode op reads must be equal: metadata rows, prompt lengths, V formats, scales, statistics,
the compacted records and the exact heads' records; over ragged appends that grow every array, prompts
of equal tile counts, a batched call, INT4 and INT8 heads and exact (bf16) heads."""
from __future__ import annotations

import pytest
import torch

from cache_host import HostCacheModule
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import Prefill
from triattention_amd.maps import from_bands
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu


class TeeCache(DecodeCache):
    """A GPU decode cache whose every store is replayed, on host copies of its sources, into ``host``."""

    def __init__(self, module, host, max_tail):
        super().__init__(module, max_tail)
        self.host = host

    def store(self, layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv=(), kx=None, vx=None):
        cpu = lambda x: None if x is None else x.cpu()
        self.host.store(layer, prompt, cpu(kp), cpu(ka), cpu(kstat), cpu(vstat), {c: cpu(p) for c, p in packed.items()},
                        codes, bands, cpu(k4), cpu(ka4), exact_kv, cpu(kx), cpu(vx))
        super().store(layer, prompt, kp, ka, kstat, vstat, packed, codes, bands, k4, ka4, exact_kv, kx, vx)


ARRAYS = ("entry", "kinfo", "slot", "count", "fmt", "prompt", "xslot", "ka", "ka4", "kstat", "vstat", "k8", "k4",
          "kx", "vx")


def _compare(gpu, host, what):
    for name in ARRAYS:
        a, b = gpu.get(name), host.get(name)
        assert (a is None) == (b is None), (what, name)
        if a is not None:
            assert a.shape == b.shape, (what, name, a.shape, b.shape)
            assert torch.equal(a.cpu().view(torch.uint8), b.view(torch.uint8)), (what, name)
    for code in gpu["v"]:
        assert torch.equal(gpu["v"][code].cpu(), host["v"][code]), (what, "v", code)


@pytest.mark.parametrize("bf16_kv", [[], [1]])
def test_device_cache_build_equals_host_restatement(module, bf16_kv):
    hq, hk = 8, 2
    bands = [[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [1, INF], [1, INF]]
    print(f"\n[cache] device cache build vs host, exact KV heads {bf16_kv}", flush=True)
    host = DecodeCache(HostCacheModule(), max_tail=4)
    host.ragged = True
    cache = TeeCache(module, host, max_tail=4)
    cache.ragged = True
    fn = from_bands({"0": bands}, bf16={"0": bf16_kv} if bf16_kv else None)
    pre = Prefill(module, fn, cache, out_dtype=torch.float32)
    dev = torch.device("cuda")
    # ragged appends: equal tile counts (100 / 110), one tile, a batch of three, long prompts that grow
    # the metadata rows and the scale arrays, then short ones again
    for i, (prompt, batch) in enumerate(((100, 1), (110, 1), (64, 1), (300, 3), (2000, 1), (1500, 2), (130, 1))):
        g = S.gen(9300 + i)
        q, k, v = S.outlier_tensor(g, batch, hq, prompt), S.outlier_tensor(g, batch, hk, prompt), \
            S.outlier_tensor(g, batch, hk, prompt)
        pre(0, q.to(dev), k.to(dev), v.to(dev), 128 ** -0.5)
        torch.cuda.synchronize()
        _compare(cache.layers[0], host.layers[0], f"after store {i} (prompt {prompt}, batch {batch})")
    assert cache.layers[0]["batch"] == 10
