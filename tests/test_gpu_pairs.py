"""GPU parity of attention's two launch forms (tri_prefill_pairs).

Launches of at most two workgroups per CU (short prompts) give each workgroup four waves: two pairs
over the same 64 query rows, pair 0 with the F16 tiles and the start of the quantized tile list, pair 1
with the rest, merged through LDS before the output.  Larger launches keep two-wave workgroups.  The
same inputs go through both forms here, forced: each is held to the oracle with the parity bar
(2e-3 max-abs plus the exp2-rounding bound, 1e-3 mean-abs), and the two to each other within 1e-4
(they take the same P levels and fp16 probabilities and differ only in the fp32 summation order of
the two parts and in the reference maximum each part's scale factors are relative to).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, exact_max_abs_bar, exact_reference, oracle_prefill, run_prefill
from triattention_amd import synthetic as S
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu

FORMS_AGREE = 1e-4


def small(seed, batch, hq, hk, t):
    g = S.gen(seed)
    return (S.outlier_tensor(g, batch, hq, t), S.outlier_tensor(g, batch, hk, t), S.outlier_tensor(g, batch, hk, t))


@pytest.fixture
def forms(module):
    """Runs fn under each forced launch form and restores the size-based choice afterwards."""
    def run(fn):
        outs = {}
        try:
            for mode in (1, 2):
                module.prefill_pairs(mode)
                outs[mode] = fn()
        finally:
            module.prefill_pairs(0)
        return outs
    return run


MIXED = [[INF, INF], [INF, INF], [INF, INF], [1, INF], [1, INF], [1, INF]]
VARIED = [[INF, INF], [1, INF], [2, 4], [3, 3], [1, 2], [2, INF], [1, 1], [4, 5]]
NO_INT8 = [[0, INF], [0, 3], [0, 1], [0, 0], [1, INF], [INF, INF]]
ODD = [[4, 2], [0, 2], [5, 5], [0, 0]]


@pytest.mark.parametrize("t,batch,hq,hk,bands,seed", [
    (1, 1, 6, 2, MIXED, 9001), (63, 1, 6, 2, MIXED, 9002), (65, 1, 6, 2, MIXED, 9003),
    (200, 1, 6, 2, MIXED, 9004), (333, 2, 8, 2, VARIED, 9005), (777, 1, 8, 2, VARIED, 9006),
    (200, 1, 6, 2, NO_INT8, 9007), (333, 1, 6, 2, NO_INT8, 9008), (257, 2, 4, 2, ODD, 9009)])
def test_both_forms_match_the_oracle(module, forms, t, batch, hq, hk, bands, seed):
    print(f"\n[pairs] t={t} batch={batch} hq={hq} hk={hk} seed={seed}", flush=True)
    q, k, v = small(seed, batch, hq, hk, t)
    bt = torch.tensor(bands, dtype=torch.int32)
    outs = forms(lambda: run_prefill(module, q, k, v, bt, 128 ** -0.5)[0].numpy())
    ref, _, tol = oracle_prefill(q, k, v, bt, 128 ** -0.5)
    for mode, out in outs.items():
        assert_close(out, ref, what=f"form {mode} t={t}", tol=tol)
    d = float(np.abs(outs[1] - outs[2]).max())
    print(f"forms differ by {d:.2e}")
    assert d <= FORMS_AGREE, d


def test_exact_heads_in_both_forms(module, forms):
    """bf16 KV heads run on pair 0 of a four-wave workgroup (pair 1 passes the same barriers)."""
    print("\n[pairs] exact bf16 heads t=333", flush=True)
    q, k, v = small(9100, 2, 6, 3, 333)
    bands = torch.tensor([[INF, INF], [INF, INF], [1, INF], [1, INF], [2, 3], [2, 3]], dtype=torch.int32)
    outs = forms(lambda: run_prefill(module, q, k, v, bands, 128 ** -0.5, bf16_kv=[1])[0].numpy())
    ref, _, tol = oracle_prefill(q, k, v, bands, 128 ** -0.5)
    ex = exact_reference(q, k, v, 128 ** -0.5)
    bar = exact_max_abs_bar(q, k, v, 128 ** -0.5, [2, 3], ex)
    for mode, out in outs.items():
        quant = [0, 1, 4, 5]
        assert_close(out[:, quant], ref[:, quant], what=f"form {mode} quantized heads", tol=tol[:, quant])
        assert_close(out[:, [2, 3]], ex[:, [2, 3]], max_abs=bar, what=f"form {mode} exact heads")
    # the exact heads run the same code in both forms: bit-identical
    assert np.array_equal(outs[1][:, [2, 3]], outs[2][:, [2, 3]])


def test_four_wave_form_with_and_without_v8_sums(module, forms):
    """Under the four-wave form the reference-shaped call (no V8 sums, packed K4 records) and the Prefill
    path's (sums, expanded records) give bit-identical outputs, as under the two-wave form."""
    print("\n[pairs] four-wave form, V8 sums and expanded K4 records", flush=True)
    q, k, v = small(9200, 2, 8, 2, 777)
    bands = torch.tensor(VARIED, dtype=torch.int32)
    try:
        module.prefill_pairs(2)
        out, ops, pre = run_prefill(module, q, k, v, bands, 128 ** -0.5)
        table = next(iter(pre.tables.values()))
        pk = ops["packed"]
        for sums, wide in ((None, None), (ops["v8sum"], None), (None, ops["k4x"])):
            plain = torch.empty_like(out).cuda()
            module.attention(table.order, table.bands, None, None, pk[1], pk[2], pk[3], ops["vstat"], ops["q8"],
                             ops["kp"], ops["qa"], ops["ka"], ops["q4"], ops["k4"], ops["qa4"], ops["ka4"], plain,
                             128 ** -0.5, v8sum=sums, k4x=wide)
            torch.cuda.synchronize()
            assert torch.equal(out, plain.cpu()), (sums is not None, wide is not None)
    finally:
        module.prefill_pairs(0)


def test_config0_in_both_forms(module, forms):
    """Config 0 (its launch takes the four-wave form by size) forced into each form."""
    print("\n[pairs] config 0 in both forms", flush=True)
    c = S.config0()
    outs = forms(lambda: run_prefill(module, c["q"], c["k"], c["v"], c["bands"], c["scale"])[0].numpy())
    ref, _, tol = oracle_prefill(c["q"], c["k"], c["v"], c["bands"], c["scale"])
    for mode, out in outs.items():
        assert_close(out, ref, what=f"config 0 form {mode}", tol=tol)
    d = float(np.abs(outs[1] - outs[2]).max())
    print(f"config 0 forms differ by {d:.2e}")
    assert d <= FORMS_AGREE, d


def test_prefill_pairs_rejects_unknown_modes(module):
    with pytest.raises(RuntimeError, match="mode must be 0, 1 or 2"):
        module.prefill_pairs(3)
