"""The reference-shaped ``decode`` op as the reference's DecodeCache calls it (decode.py:76-79): one
sequence, the cache's tensors, an int prompt length, an int ``per`` and fresh q / k / v / out each step.
It must return what this repository's DecodeCache returns on the same cache, and keep one validated plan
per cache across steps (no re-validation, no per-call prompt tensor)."""
from __future__ import annotations

import pytest
import torch

from helpers import run_prefill
from test_gpu_parity import small
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import I4, I8
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu


def test_reference_shaped_decode_reuses_its_plan(module):
    print("\n[dropin] reference-shaped decode calls, prompt 700, per 3", flush=True)
    hq, hk, prompt, scale = 6, 3, 700, 128 ** -0.5
    bands = torch.tensor([[INF, INF], [1, 1], [0, INF], [0, 3], [2, 5], [1, INF]], dtype=torch.int32)
    q, k, v = small(9970, 1, hq, hk, prompt)
    ours = DecodeCache(module, max_tail=16)
    ours.per, ours.tasks = 3, False  # the reference's uniform split and gather
    run_prefill(module, q, k, v, bands, scale, decode_cache=ours, out_dtype=torch.bfloat16)
    e = ours.layers[0]
    dev = torch.device("cuda")
    # the reference's own buffers for the same cache: its tails, step counter and split partials
    tail_k, tail_v = torch.zeros_like(e["tail_k"]), torch.zeros_like(e["tail_v"])
    step = torch.zeros(1, dtype=torch.int64, device=dev)
    splits = e["splits"]
    partials = (torch.empty(hq * splits, device=dev), torch.empty(hq * splits, device=dev),
                torch.empty(hq * splits * 128, device=dev))
    g = torch.Generator().manual_seed(9971)
    module._plans.clear()
    plans = []
    for t in range(4):
        qd = torch.randn(1, hq, 1, 128, generator=g).to(torch.bfloat16).to(dev)
        kd = torch.randn(1, hk, 1, 128, generator=g).to(torch.bfloat16).to(dev)
        vd = torch.randn(1, hk, 1, 128, generator=g).to(torch.bfloat16).to(dev)
        want = ours(0, qd, kd, vd, scale)
        ours.advance()
        out = torch.empty_like(qd)
        module.decode(qd, e["k8"], e["k4"], e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"],
                      e["slot"], e["v"][I8], e["v"][I4], e["vstat"], e["kstat"], tail_k, tail_v, kd, vd, step, out,
                      *partials, prompt, e["per"], scale)
        step.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want.cpu()), f"step {t}"
        assert len(module._plans) == 1
        plans.append(next(iter(module._plans.values())))
    assert all(p is plans[0] for p in plans)
    # a different cache (its own tails) gets its own plan; dropping it lets its plan go stale
    other_k, other_v = torch.zeros_like(tail_k), torch.zeros_like(tail_v)
    module.decode(qd, e["k8"], e["k4"], e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], e["fmt"], e["slot"],
                  e["v"][I8], e["v"][I4], e["vstat"], e["kstat"], other_k, other_v, kd, vd, step,
                  torch.empty_like(qd), *partials, prompt, e["per"], scale)
    assert len(module._plans) == 2
    stale = list(module._plans.values())[-1]
    assert all(ref() is not None for ref in stale.weak)
    del other_k, other_v
    assert any(ref() is None for ref in stale.weak)
