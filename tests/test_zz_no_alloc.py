"""tri_decode_noalloc, the decode entry point that allocates nothing (its split partials live in a
scratch array inside the library), against tri_decode with caller buffers: the same kernels on the
same cache must give the same bits.  Two calls in a row, the second smaller than the first, so the
second runs on a scratch that still holds the first call's partials; with the task table and with the
reference's gather, and with an exact (bf16) KV head.  A call on a second stream while the first
stream's call is still pending is refused."""
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


def _cache(module, seed, batch, prompt, max_tail=8, tasks=True, bf16_kv=None):
    g = S.gen(seed)
    q, k, v = S.outlier_tensor(g, batch, 8, prompt), S.outlier_tensor(g, batch, 2, prompt), S.outlier_tensor(g, batch, 2, prompt)
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    cache.tasks = tasks
    run_prefill(module, q, k, v, BANDS, SCALE, decode_cache=cache, bf16_kv=bf16_kv)
    return cache


def _args(plan, q, kcur, vcur, out, stream=None):
    """The plan's tri_decode_noalloc arguments (no pm / pl / po) with this step's tensors and a stream
    (the current one by default)."""
    a = list(plan.args)
    a[plan.Q], a[plan.KC], a[plan.VC], a[plan.OUT] = q.data_ptr(), kcur.data_ptr(), vcur.data_ptr(), out.data_ptr()
    a[plan.STREAM] = (stream or torch.cuda.current_stream()).cuda_stream
    del a[31:34]
    return a


def _compare(module, cache, seed):
    e = cache.layers[0]
    batch = e["batch"]
    g = S.gen(seed)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, batch, 8, 1).to(dev), S.outlier_tensor(g, batch, 2, 1).to(dev),
                  S.outlier_tensor(g, batch, 2, 1).to(dev))
    # tri_decode (split kernel and its merge, as tri_decode_noalloc launches them) with the
    # cache's own partial buffers
    ref = torch.full((batch, 8, 1, 128), float("nan"), device=dev)
    plan = cache.plan(0, qd, kd, ref, SCALE)
    plan.run(qd, kd, vd, ref)
    got = torch.full_like(ref, float("nan"))
    rc = module.lib.tri_decode_noalloc(*_args(plan, qd, kd, vd, got))
    assert rc == 0, module.lib.tri_last_error().decode()
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), float((got - ref).abs().max())
    return batch * 8 * e["splits"]


@pytest.mark.parametrize("tasks,bf16_kv", [(True, None), (False, None), (True, [1])])
def test_noalloc_decode_equals_decode_with_caller_buffers(module, tasks, bf16_kv):
    print(f"\n[noalloc] tasks {tasks} bf16_kv {bf16_kv}: batch 4 prompt 700, then batch 1 prompt 130", flush=True)
    big = _cache(module, 9100, 4, 700, tasks=tasks, bf16_kv=bf16_kv)
    small = _cache(module, 9101, 1, 130, tasks=tasks, bf16_kv=bf16_kv)
    n_big = _compare(module, big, 9200)
    n_small = _compare(module, small, 9201)
    assert n_small < n_big
    big.advance()
    # a further step of the larger cache after the smaller call (its tail now holds a token)
    _compare(module, big, 9202)


def test_noalloc_refuses_a_second_stream_while_the_first_is_pending(module):
    print("\n[noalloc] two streams: batch 2 prompt 300", flush=True)
    cache = _cache(module, 9300, 2, 300)
    g = S.gen(9301)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, 2, 8, 1).to(dev), S.outlier_tensor(g, 2, 2, 1).to(dev),
                  S.outlier_tensor(g, 2, 2, 1).to(dev))
    ref = torch.full((2, 8, 1, 128), float("nan"), device=dev)
    plan = cache.plan(0, qd, kd, ref, SCALE)
    plan.run(qd, kd, vd, ref)  # tri_decode: its merge, as tri_decode_noalloc
    torch.cuda.synchronize()
    got_a, got_b = torch.full_like(ref, float("nan")), torch.full_like(ref, float("nan"))
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    x = torch.randn(8192, 8192, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        for _ in range(40):  # tens of milliseconds of queued work ahead of the call on stream A
            y = x @ x
        assert module.lib.tri_decode_noalloc(*_args(plan, qd, kd, vd, got_a, sa)) == 0
    # stream A's call is still queued behind its GEMMs: a call on stream B must not touch the scratch
    assert module.lib.tri_decode_noalloc(*_args(plan, qd, kd, vd, got_b, sb)) == 1
    assert b"another stream" in module.lib.tri_last_error()
    sa.synchronize()
    assert module.lib.tri_decode_noalloc(*_args(plan, qd, kd, vd, got_b, sb)) == 0
    sb.synchronize()
    del y
    for got in (got_a, got_b):
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), float((got - ref).abs().max())
