"""tri_decode_noalloc, the decode entry point that allocates nothing (its split partials live in a
scratch array inside the library), against tri_decode with caller buffers: the same kernels on the
same cache must give the same bits.  Two calls in a row, the second smaller than the first, so the
second runs on a scratch that still holds the first call's partials."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import run_prefill
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5
BANDS = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2], [INF, INF], [2, 2]],
                     dtype=torch.int32)


def _cache(module, seed, batch, prompt, max_tail=8):
    g = S.gen(seed)
    q, k, v = S.outlier_tensor(g, batch, 8, prompt), S.outlier_tensor(g, batch, 2, prompt), S.outlier_tensor(g, batch, 2, prompt)
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, BANDS, SCALE, decode_cache=cache)
    return cache


def _args(plan, q, kcur, vcur, out):
    """The plan's tri_decode arguments with this step's tensors and the current stream."""
    a = list(plan.args)
    a[plan.Q], a[plan.KC], a[plan.VC], a[plan.OUT] = q.data_ptr(), kcur.data_ptr(), vcur.data_ptr(), out.data_ptr()
    a[plan.STREAM] = torch.cuda.current_stream().cuda_stream
    return a


def _compare(module, cache, seed):
    e = cache.layers[0]
    batch = e["batch"]
    g = S.gen(seed)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, batch, 8, 1).to(dev), S.outlier_tensor(g, batch, 2, 1).to(dev),
                  S.outlier_tensor(g, batch, 2, 1).to(dev))
    ref = cache(0, qd, kd, vd, SCALE)  # tri_decode with the cache's own partial buffers
    got = torch.full_like(ref, float("nan"))
    plan = cache.plan(0, qd, kd, got, SCALE)
    a = _args(plan, qd, kd, vd, got)
    del a[31:34]  # tri_decode_noalloc takes no pm / pl / po
    rc = module.lib.tri_decode_noalloc(*a)
    assert rc == 0, module.lib.tri_last_error().decode()
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), float((got - ref).abs().max())
    return batch * 8 * e["splits"]


def test_noalloc_decode_equals_decode_with_caller_buffers(module):
    print("\n[noalloc] batch 4 prompt 700, then batch 1 prompt 130", flush=True)
    big = _cache(module, 9100, 4, 700)
    small = _cache(module, 9101, 1, 130)
    n_big = _compare(module, big, 9200)
    n_small = _compare(module, small, 9201)
    assert n_small < n_big
    big.advance()
    # a further step of the larger cache after the smaller call (its tail now holds a token)
    _compare(module, big, 9202)
