"""Host logic of the HF integration (triattention_amd.models), on the CPU.

The attention hook and the prefill/decode dispatch of ``TriAttention`` are
checked with stand-ins for ``Prefill`` and ``DecodeCache`` that compute exact
attention in float32 (prompt stored by the prefill stand-in, generated tokens
appended by the decode stand-in).  Greedy generation through the hook must then
give the tokens of the model's own attention with its KV cache."""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from triattention_amd import models as M  # noqa: E402
from triattention_amd.maps import INF, from_bands  # noqa: E402


def tiny_qwen2(layers=2, heads=4, kv_heads=2, vocab=97, seed=0):
    cfg = transformers.Qwen2Config(vocab_size=vocab, hidden_size=heads * 128, intermediate_size=256,
                                   num_hidden_layers=layers, num_attention_heads=heads,
                                   num_key_value_heads=kv_heads, max_position_embeddings=1024,
                                   rope_theta=1e6, tie_word_embeddings=False)
    torch.manual_seed(seed)
    model = transformers.Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():  # larger weights than the N(0, 0.02) default, so the greedy tokens vary
        for p in model.parameters():
            p.mul_(8.0)
    return model


def sdpa(q, k, v, scale):
    g = q.shape[1] // k.shape[1]
    return torch.nn.functional.scaled_dot_product_attention(
        q.float(), k.float().repeat_interleave(g, 1), v.float().repeat_interleave(g, 1),
        is_causal=q.shape[2] > 1, scale=scale).to(q.dtype)


class FakePrefill:
    def __init__(self, cache):
        self.cache, self.calls = cache, []

    def __call__(self, layer, q, k, v, scale):
        self.calls.append((layer, tuple(q.shape), tuple(k.shape)))
        self.cache.kv[layer] = (k.clone(), v.clone())
        return sdpa(q, k, v, scale)


class FakeDecodeCache:
    def __init__(self):
        self.kv, self.calls, self.steps = {}, [], 0

    def stored(self, layer):
        return layer in self.kv

    def __call__(self, layer, q, k, v, scale):
        self.calls.append((layer, self.steps, tuple(q.shape)))
        pk, pv = self.kv[layer]
        self.kv[layer] = (torch.cat([pk, k], 2), torch.cat([pv, v], 2))
        return sdpa(q, *self.kv[layer], scale)

    def advance(self):
        self.steps += 1


def test_generate_dispatches_prompt_to_prefill_and_tokens_to_decode():
    model = tiny_qwen2()
    bands = {str(l): [[INF, INF]] * 4 for l in range(2)}
    tri = M.TriAttention(model, from_bands(bands, model), max_new_tokens=5, module=object())
    cache = FakeDecodeCache()
    tri.decode_cache, tri.prefill = cache, FakePrefill(cache)
    torch.manual_seed(1)
    ids = torch.randint(97, (1, 37))
    tokens = tri.generate(ids, 5, eos=set())
    assert len(tokens) == 5
    assert tri.prefill.calls == [(0, (1, 4, 37, 128), (1, 2, 37, 128)), (1, (1, 4, 37, 128), (1, 2, 37, 128))]
    # every generated token after the first runs one decode call per layer, then advances the step
    assert cache.calls == [(layer, step, (1, 4, 1, 128)) for step in range(5) for layer in range(2)]
    assert cache.steps == 5
    # the same greedy tokens as the model's own attention with its KV cache
    model.set_attn_implementation("sdpa")
    ref = model.generate(ids, max_new_tokens=5, do_sample=False, eos_token_id=None, pad_token_id=0)
    assert tokens == ref[0, 37:].tolist()


def test_generate_stops_before_an_eos_token():
    model = tiny_qwen2(seed=3)
    tri = M.TriAttention(model, from_bands({str(l): [[INF, INF]] * 4 for l in range(2)}), max_new_tokens=8,
                         module=object())
    cache = FakeDecodeCache()
    tri.decode_cache, tri.prefill = cache, FakePrefill(cache)
    ids = torch.randint(97, (1, 20), generator=torch.Generator().manual_seed(4))
    full = tri.generate(ids, 8, eos=set())
    stop = full[3]
    cache2 = FakeDecodeCache()
    tri.decode_cache, tri.prefill = cache2, FakePrefill(cache2)
    cut = tri.generate(ids, 8, eos={stop})
    assert cut == full[:full.index(stop)]


def test_use_attention_output_layout():
    """The hook returns [B, T, H, D] (the transpose of the attention function's [B, H, T, D])."""
    model = tiny_qwen2(layers=1)
    seen = []

    def fn(mod, q, k, v, scaling):
        seen.append((mod.layer_idx, tuple(q.shape), scaling))
        return sdpa(q, k, v, scaling)

    M.use_attention(model, "probe", fn)
    ids = torch.randint(97, (1, 9), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=False).logits
    assert seen == [(0, (1, 4, 9, 128), 128 ** -0.5)]
    model.set_attn_implementation("sdpa")
    with torch.no_grad():
        ref = model(input_ids=ids, use_cache=False).logits
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


def test_map_must_match_the_model():
    model = tiny_qwen2(layers=2)
    with pytest.raises(ValueError):
        from_bands({"0": [[INF, INF]] * 4}, model)
    with pytest.raises(ValueError):
        from_bands({str(l): [[INF, INF]] * 3 for l in range(2)}, model)


def test_all_exact_bands_fn():
    fn = M._AllExact(4)
    assert fn.bf16(7) == [0, 1, 2, 3]
    assert fn(0, 12).shape == (12, 2)


def _save_local_checkpoint(tmp_path, model_type="qwen2"):
    """A tiny bf16 checkpoint plus a word-level tokenizer with a chat template, saved to a directory."""
    from tokenizers import Tokenizer, models, pre_tokenizers

    model = tiny_qwen2(layers=1)
    model.generation_config.eos_token_id = [3, 5]
    model.to(torch.bfloat16).save_pretrained(tmp_path)
    vocab = {w: i for i, w in enumerate(["<unk>", "<s>", "hello", "</s>", "world", "<|im_end|>"])}
    raw = Tokenizer(models.WordLevel(vocab, unk_token="<unk>"))
    raw.pre_tokenizer = pre_tokenizers.Whitespace()
    tok = transformers.PreTrainedTokenizerFast(tokenizer_object=raw, unk_token="<unk>", bos_token="<s>",
                                               eos_token="</s>")
    tok.chat_template = ("{% for m in messages %}<{{ m.role }}> {{ m.content }} {% endfor %}"
                         "{% if add_generation_prompt %}<assistant> {{ date_string }}{% endif %}")
    tok.save_pretrained(tmp_path)
    return model


def test_loaders_read_a_local_checkpoint(tmp_path):
    saved = _save_local_checkpoint(tmp_path)
    tok = M.load_tokenizer(tmp_path)
    model = M.load_model(tmp_path, device="cpu")
    assert model.dtype == torch.bfloat16 and not model.training
    # qwen2 checkpoints get the reference's YaRN long-context RoPE (models.py:23-27)
    rope = model.config.rope_parameters
    assert rope["rope_type"] == "yarn" and rope["factor"] == 4.0
    assert rope["original_max_position_embeddings"] == 32768 and rope["rope_theta"] == 1e6
    assert model.config.max_position_embeddings == 4 * 32768
    for a, b in zip(saved.state_dict().values(), model.state_dict().values()):
        assert torch.equal(a, b)
    assert M.render_prompt(tok, "hello world") == "<user> hello world <assistant> 30 Jul 2026"
    # the tokenizer's end id (3) and the generation config's list [3, 5]
    assert M.eos_ids(tok, model) == {3, 5}


def test_loaders_refuse_anything_but_a_local_directory(tmp_path):
    for name in ("Qwen/Qwen2-7B-Instruct", tmp_path / "missing"):
        with pytest.raises(FileNotFoundError, match="not a local model directory"):
            M.load_model(name, device="cpu")
        with pytest.raises(FileNotFoundError, match="not a local model directory"):
            M.load_tokenizer(name)
