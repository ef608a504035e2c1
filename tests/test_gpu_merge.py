"""The two forms of the decode merge against the oracle, over tail lengths and split counts.

The one-wave merge (tri_decode_short_tail, taken while the tail holds at most 64 tokens) follows the
reference's merge order exactly (32-lane butterfly tail scores, split sums in four interleaved
groups, tail tokens one after another), as the oracle does: given the oracle's own split partials
(written into the cache's partial buffers, then the merge launched alone), its fp32 output must equal
the oracle's bit for bit.  tri_decode's merge chooses its form on the device (the one-wave form while
the tail holds at most 16 tokens on a grid of at least 2 (sequence, q-head) workgroups per CU, four
waves otherwise), so that a captured graph, replayed at steps with longer and longer tails, gives the
bits of the eager steps: on such a grid and tail its output equals the one-wave kernel's bit for bit
(test_device_chosen_merge_on_a_wide_grid).  Whole decode steps (split kernel and merge) of both
launches keep the 2e-3 / 1e-3 bar (the split kernel's partials agree with the oracle's to fp32
rounding).  Tails past 64 tokens and split counts past 16 (and 64) run the one-wave form's loops."""
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
    # (12 workgroups: too few for the one-wave form on the device or in the host's eager choice)
    assert cache.tail_tokens(0) == tail and not cache.short_tail(0, hq)
    dev = torch.device("cuda")
    qd, kd, vd = S.outlier_tensor(g, batch, hq, 1), S.outlier_tensor(g, batch, hk, 1), S.outlier_tensor(g, batch, hk, 1)
    traces = [[O.decode_trace(codes[b], BANDS.numpy(), bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale,
                              ktail[b], vtail[b], bits(kd[b, :, 0]), bits(vd[b, :, 0]), step, h)
               for h in range(hq)] for b in range(batch)]
    refs = [np.stack([traces[b][h]["out"] for h in range(hq)]) for b in range(batch)]
    for short in (True, False):
        out = torch.full((batch, hq, 1, 128), float("nan"), device=dev)
        plan = cache.plan(0, qd.to(dev), kd.to(dev), out, scale)
        plan.run(qd.to(dev), kd.to(dev), vd.to(dev), out, short_tail=short)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for b in range(batch):
            assert_close(got[b, :, 0], refs[b], what=f"decode step, {'one-wave' if short else 'device-chosen'} "
                                                      f"merge, seq {b}, splits {splits}")
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
    out = torch.full((batch, hq, 1, 128), float("nan"), device=dev)
    plan = cache.plan(0, qd.to(dev), kd.to(dev), out, scale)
    plan.run(qd.to(dev), kd.to(dev), vd.to(dev), out, 2, short_tail=True)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(batch):
        assert np.array_equal(got[b, :, 0].view(np.uint32), refs[b].view(np.uint32)), \
            f"one-wave merge on the oracle's partials, seq {b}: max abs {np.abs(got[b, :, 0] - refs[b]).max():.3e}"
    # both forms appended this step's token to the tail at the same slot
    ktail[:, :, step] = bits(kd[:, :, 0])
    vtail[:, :, step] = bits(vd[:, :, 0])
    assert np.array_equal(bits(e["tail_k"].cpu()), ktail) and np.array_equal(bits(e["tail_v"].cpu()), vtail)


@pytest.mark.parametrize("tail", [1, 16, 17])
def test_device_chosen_merge_on_a_wide_grid(module, tail):
    """On a grid of at least 2 (sequence, q-head) workgroups per CU, tri_decode's merge takes the one-wave
    form on the device while the tail holds at most 16 tokens, with the one-wave kernel's bits (so an
    eager step, which launches that kernel, and a graph replay agree), and four waves beyond; the host's
    eager choice follows the same rule."""
    hq, hk, prompt, max_tail = 32, 8, 200, 64
    batch = -(-2 * module.device_cus() // hq)
    print(f"\n[merge] device-chosen form, batch {batch} x hq {hq}, tail {tail}", flush=True)
    g = S.gen(7100 + tail)
    bands = torch.tensor([[INF, INF], [1, INF], [2, 5], [1, 1]] * 8, dtype=torch.int32)
    q, k, v = S.outlier_tensor(g, batch, hq, prompt), S.outlier_tensor(g, batch, hk, prompt), S.outlier_tensor(g, batch, hk, prompt)
    cache = DecodeCache(module, max_tail=max_tail)
    cache.out_dtype = torch.float32
    run_prefill(module, q, k, v, bands, 128 ** -0.5, decode_cache=cache)
    e = cache.layers[0]
    e["tail_k"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_k"].device))
    e["tail_v"].copy_(S.outlier_tensor(g, batch, hk, max_tail).to(e["tail_v"].device))
    cache.step.fill_(tail - 1)
    cache.host_step = tail - 1
    assert cache.tail_tokens(0) == tail and cache.short_tail(0, hq) == (tail <= 16)
    dev = torch.device("cuda")
    qd, kd, vd = (S.outlier_tensor(g, batch, hq, 1).to(dev), S.outlier_tensor(g, batch, hk, 1).to(dev),
                  S.outlier_tensor(g, batch, hk, 1).to(dev))
    outs = {}
    for short in (True, False):
        out = torch.full((batch, hq, 1, 128), float("nan"), device=dev)
        plan = cache.plan(0, qd, kd, out, 128 ** -0.5)
        plan.run(qd, kd, vd, out, short_tail=short)
        torch.cuda.synchronize()
        outs[short] = out.cpu()
    assert torch.isfinite(outs[False]).all()
    same = torch.equal(outs[True].view(torch.int32), outs[False].view(torch.int32))
    if tail <= 16:
        assert same, "the device-chosen merge left the one-wave form's bits"
    else:  # four waves: a different summation order, within the decode bar of the one-wave form
        assert not same
        assert_close(outs[False].numpy(), outs[True].numpy(), what=f"four-wave against one-wave merge, tail {tail}")
