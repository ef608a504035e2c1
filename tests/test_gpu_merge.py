"""The two forms of the decode merge against the oracle, over tail lengths and split counts.

The one-wave merge (tri_decode_short_tail, taken while the tail holds at most 64 tokens) follows the
reference's merge order exactly (32-lane butterfly tail scores, split sums in four interleaved
groups, tail tokens one after another), as the oracle does: given the oracle's own split partials
(written into the cache's partial buffers, then the merge launched alone), its fp32 output must equal
the oracle's bit for bit.  tri_decode's merge chooses its form on the device from the tail's length
(the one-wave form up to 64 tokens, four waves beyond), so that a captured graph, replayed at steps
with longer and longer tails, gives the bits of the eager steps: up to 64 tokens its output equals
the one-wave form's bit for bit.  Whole decode steps (split kernel and merge) of both launches keep
the 2e-3 / 1e-3 bar (the split kernel's partials agree with the oracle's to fp32 rounding).  Tails
past 64 tokens and split counts past 16 (and 64) run the one-wave form's loops."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, bits, run_prefill
from triattention_amd import synthetic as S
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu
BANDS = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1], [3, INF], [1, 2]], dtype=torch.int32)


@pytest.mark.parametrize("tail,per,prompt", [(1, None, 300), (2, None, 300), (63, None, 700), (64, 1, 1500),
                                             (65, 2, 1500), (130, 1, 64 * 70 + 5), (200, 3, 900)])
def test_merge_forms_against_the_oracle(module, tail, per, prompt):
    hq, hk, batch, max_tail = 6, 2, 2, 256
    print(f"\n[merge] tail {tail} per {per} prompt {prompt}", flush=True)
    g = S.gen(7000 + tail)
    q, k, v = S.outlier_tensor(g, batch, hq, prompt), S.outlier_tensor(g, batch, hk, prompt), S.outlier_tensor(g, batch, hk, prompt)
    scale = 128 ** -0.5
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    cache.per = per
    run_prefill(module, q, k, v, BANDS, scale, decode_cache=cache)
    codes = [O.prefill_codes(bits(q[b]), bits(k[b]), bits(v[b]), BANDS.numpy(), decode_cache=True)
             for b in range(batch)]
    e = cache.layers[0]
    splits = e["splits"]
    e["tail_k"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_k"].device))
    e["tail_v"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_v"].device))
    ktail, vtail = bits(e["tail_k"].cpu()).copy(), bits(e["tail_v"].cpu()).copy()
    step = tail - 1  # the merge reads `step` tail rows and this step's token
    cache.step.fill_(step)
    cache.host_step = step
    assert cache.tail_tokens(0) == tail and cache.short_tail(0) == (tail <= 64)
    dev = torch.device("cuda")
    qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
    traces = [[O.decode_trace(codes[b], BANDS.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale,
                              ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step, h)
               for h in range(hq)] for b in range(batch)]
    refs = [np.stack([traces[b][h]["out"] for h in range(hq)]) for b in range(batch)]
    forms = {}
    for short in (True, False):
        out = torch.full((batch, hq, 1, 128), float("nan"), device=dev)
        plan = cache.plan(0, qd.to(dev), kd.to(dev), out, scale)
        plan.run(qd.to(dev), kd.to(dev), vd.to(dev), out, short_tail=short)
        torch.cuda.synchronize()
        got = forms[short] = out.cpu().numpy()
        for b in range(batch):
            assert_close(got[b, :, 0], refs[b], what=f"decode step, {'one-wave' if short else 'device-chosen'} "
                                                      f"merge, seq {b}, splits {splits}")
    if tail <= 64:  # the device chose the one-wave form: the same bits
        assert np.array_equal(forms[True].view(np.uint32), forms[False].view(np.uint32))
    # the merge alone on the oracle's split partials: the one-wave form is the reference's order
    pm, pl, po = e[("partials", hq)]
    pm_h, pl_h, po_h = pm.cpu().numpy(), pl.cpu().numpy(), po.cpu().numpy().reshape(-1, 128)
    for b in range(batch):
        for h in range(hq):
            t = traces[b][h]
            n = min(splits, t["pm"].size)
            assert not t["pl"][n:].any()  # splits past the cache's are empty
            row = (b * hq + h) * splits
            pm_h[row:row + n], pl_h[row:row + n], po_h[row:row + n] = t["pm"][:n], t["pl"][:n], t["po"][:n]
            pm_h[row + n:row + splits], pl_h[row + n:row + splits], po_h[row + n:row + splits] = -3.4028235e38, 0, 0
    pm.copy_(torch.from_numpy(pm_h))
    pl.copy_(torch.from_numpy(pl_h))
    po.copy_(torch.from_numpy(po_h.reshape(-1)))
    for short in (True, False) if tail <= 64 else (True,):
        out = torch.full((batch, hq, 1, 128), float("nan"), device=dev)
        plan = cache.plan(0, qd.to(dev), kd.to(dev), out, scale)
        plan.run(qd.to(dev), kd.to(dev), vd.to(dev), out, 2, short_tail=short)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for b in range(batch):
            assert np.array_equal(got[b, :, 0].view(np.uint32), refs[b].view(np.uint32)), \
                (f"{'one-wave' if short else 'device-chosen'} merge on the oracle's partials, seq {b}: "
                 f"max abs {np.abs(got[b, :, 0] - refs[b]).max():.3e}")
    # both forms appended this step's token to the tail at the same slot
    ktail[:, :, step] = bits(kd[:, :, 0])
    vtail[:, :, step] = bits(vd[:, :, 0])
    assert np.array_equal(bits(e["tail_k"].cpu()), ktail) and np.array_equal(bits(e["tail_v"].cpu()), vtail)
