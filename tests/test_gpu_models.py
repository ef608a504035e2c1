"""End-to-end parity of the HF integration on the GPU: a small random-init Qwen2 generates through
``TriAttention``; every attention call it makes (prompt prefill per layer, then one decode call per
layer and generated token) is checked against the oracle on that call's own inputs.

Quantized q-heads are held to the oracle (prefill and decode restatements, the decode tail holding the
generated tokens' bf16 K/V), exact (bf16) q-heads to float64 attention over the raw operands.  The model
runs in bf16, so each output element may also carry bf16 rounding (half an ulp, |ref| * 2**-8)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close_bf16, exact_max_abs_bar, exact_reference
from test_gpu_parity import _attend64
from triattention_amd import models as M
from triattention_amd.maps import INF, from_bands
from triattention_amd.synthetic import bits

transformers = pytest.importorskip("transformers")
pytestmark = pytest.mark.gpu


class Recorder:
    """Forwards to a Prefill / DecodeCache and keeps (layer, q, k, v, out) of each call on the CPU."""

    def __init__(self, inner):
        self.inner, self.calls = inner, []

    def __getattr__(self, name):
        return getattr(self.inner, name)

    def __call__(self, layer, q, k, v, scale):
        out = self.inner(layer, q, k, v, scale)
        self.calls.append((layer, q.cpu(), k.cpu(), v.cpu(), out.float().cpu(), scale))
        return out


def tiny_qwen2(device):
    cfg = transformers.Qwen2Config(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                                   rope_theta=1e6, tie_word_embeddings=False)
    torch.manual_seed(11)
    return transformers.Qwen2ForCausalLM(cfg).to(torch.bfloat16).to(device).eval()


def test_generate_through_the_kernels_matches_the_oracle(module):
    print("\n[parity] HF Qwen2 (2 layers, Hq 4 / Hk 2) generate: prompt 200, 6 tokens", flush=True)
    dev = torch.device("cuda")
    model = tiny_qwen2(dev)
    bands = {"0": [[INF, INF], [INF, INF], [1, INF], [1, INF]], "1": [[2, 4], [1, 3], [INF, INF], [INF, INF]]}
    bf16 = {"1": [1]}
    steps, prompt = 6, 200
    tri = M.TriAttention(model, from_bands(bands, model, bf16=bf16), max_new_tokens=steps, module=module)
    tri.prefill = Recorder(tri.prefill)
    tri.decode_cache = Recorder(tri.decode_cache)
    ids = torch.randint(256, (1, prompt), generator=torch.Generator().manual_seed(12)).to(dev)
    tokens = tri.generate(ids, steps, eos=set())
    assert len(tokens) == steps and all(0 <= t < 256 for t in tokens)
    pre, dec = tri.prefill.calls, tri.decode_cache.calls
    assert [c[0] for c in pre] == [0, 1]
    assert [c[0] for c in dec] == [0, 1] * steps
    for layer, q, k, v, out, scale in pre:
        b = np.asarray(bands[str(layer)], np.int32)
        exact_kv = bf16.get(str(layer), [])
        exact_q = [h for h in range(4) if h // 2 in exact_kv]
        quant_q = [h for h in range(4) if h // 2 not in exact_kv]
        assert q.shape == (1, 4, prompt, 128) and out.shape == (1, 4, prompt, 128)
        ref, _, tol = O.prefill(bits(q[0]), bits(k[0]), bits(v[0]), b, scale, decode_cache=True, tol=True)
        assert_close_bf16(out[0, quant_q].numpy(), ref[quant_q], what=f"prefill layer {layer} quantized heads",
                          tol=tol[quant_q])
        if exact_q:
            ex = exact_reference(q, k, v, scale)
            bar = exact_max_abs_bar(q, k, v, scale, exact_q, ex)
            assert_close_bf16(out[:, exact_q].numpy(), ex[:, exact_q], max_abs=bar, what=f"prefill layer {layer} exact")
    for layer in (0, 1):
        _, q0, k0, v0, _, scale = pre[layer]
        b = np.asarray(bands[str(layer)], np.int32)
        codes = O.prefill_codes(bits(q0[0]), bits(k0[0]), bits(v0[0]), b, decode_cache=True)
        split = tri.decode_cache.inner.split_of(layer, 0)
        exact_kv = bf16.get(str(layer), [])
        exact_q = [h for h in range(4) if h // 2 in exact_kv]
        quant_q = [h for h in range(4) if h // 2 not in exact_kv]
        ktail = np.zeros((2, steps, 128), np.uint16)
        vtail = np.zeros_like(ktail)
        keys, values = k0[0].float(), v0[0].float()
        for step, (_, q, k, v, out, _) in enumerate(c for c in dec if c[0] == layer):
            ref = O.decode(codes, b, bits(q[0, :, 0]), prompt, split, scale, ktail, vtail, bits(k[0, :, 0]),
                           bits(v[0, :, 0]), step)
            assert_close_bf16(out[0, quant_q, 0].numpy(), ref[quant_q], what=f"decode layer {layer} step {step}")
            keys, values = torch.cat([keys, k[0].float()], 1), torch.cat([values, v[0].float()], 1)
            if exact_q:
                r64, r32 = _attend64(q[0, :, 0], keys, values, scale)
                bar = max(2e-3, float(np.abs(r32[exact_q] - r64[exact_q]).max()))
                assert_close_bf16(out[0, exact_q, 0].numpy(), r64[exact_q], max_abs=bar,
                             what=f"decode layer {layer} step {step} exact")
            ktail[:, step] = bits(k[0, :, 0])
            vtail[:, step] = bits(v[0, :, 0])


def test_exact_attention_matches_float64(module):
    print("\n[parity] exact_attention B2 Hq 6 / Hk 2 T 150", flush=True)
    g = torch.Generator().manual_seed(21)
    q = torch.randn(2, 6, 150, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 2, 150, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 2, 150, 128, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    out = M.exact_attention(q.to(dev), k.to(dev), v.to(dev), 128 ** -0.5).float().cpu().numpy()
    ex = exact_reference(q, k, v, 128 ** -0.5)
    bar = exact_max_abs_bar(q, k, v, 128 ** -0.5, list(range(6)), ex)
    assert_close_bf16(out, ex, max_abs=bar, what="exact_attention")


def test_graph_replay_generates_the_eager_tokens(module):
    """generate(graph=True) replays one captured one-token forward per token; with the same kernels
    and arguments it must give exactly the eager tokens (checked over 12 replays, with the eager run
    and synchronisations in between)."""
    print("\n[parity] HF Qwen2 generate: HIP graph replay vs eager", flush=True)
    dev = torch.device("cuda")
    model = tiny_qwen2(dev)
    bands = {"0": [[INF, INF], [INF, INF], [1, INF], [1, INF]], "1": [[2, 4], [1, 3], [INF, INF], [INF, INF]]}
    ids = torch.randint(256, (1, 150), generator=torch.Generator().manual_seed(13)).to(dev)
    runs = []
    for graph in (False, True, False, True):
        tri = M.TriAttention(model, from_bands(bands, model, bf16={"1": [1]}), max_new_tokens=14, module=module)
        runs.append(tri.generate(ids, 14, eos=set(), graph=graph))
        torch.cuda.synchronize()
    assert runs[0] == runs[1] == runs[2] == runs[3], runs
