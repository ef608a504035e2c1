"""Hugging Face integration: the attention hook, prefill/decode dispatch and
greedy generation on the gfx950 kernels.

Mirrors the attention half of triattention/models.py (exact_attention :45-47,
use_attention :50-55, TriAttention :58-85) with the same names, arguments and
behaviour:

* a model's attention calls go to ``Prefill`` for a prompt and to
  ``DecodeCache`` for a one-token query of a layer whose prompt is stored;
* ``generate`` runs the model without the HF KV cache (the decode cache holds
  the quantized prompt and the bf16 tail of generated tokens) and returns the
  greedy tokens, stopping at an end-of-sequence id.

``exact_attention`` (the reference's bf16 baseline, SDPA flash there) runs the
exact-head path of this library's prefill kernel: every KV head listed as
bf16, so each q-head attends causally over the unquantized bf16 operands with
fp32 accumulation.

Extensions: ``TriAttention`` accepts a map path or a ``bands_fn`` (as built by
``triattention_amd.maps``), an optional ``module`` (the loaded extension) and
an optional ``max_tail``: with more new tokens than the tail holds (the
reference's tail is max_new_tokens long, and its kernels cap it at 1024), the
decode cache grows, taking the oldest 64 tail tokens into a new quantized tile
whenever the tail is full.

Checkpoint and tokenizer loading, the chat prompt and end-of-sequence ids
(``load_tokenizer``, ``load_model``, ``render_prompt``, ``eos_ids``;
models.py:16-42) behave as the reference's, with one policy of this build:
they read local directories only (``local_files_only``) and refuse anything
else with a clear error, so a model name never turns into a download.  Any HF
causal LM whose attention modules call the registered attention function can
be handed to ``TriAttention``, however it was loaded.
"""
from __future__ import annotations

import os

import torch

from .kernels.decode import DecodeCache
from .kernels.extension import load_extension
from .kernels.prefill import Prefill
from .maps import INF, load_map, preset


def _local_dir(path):
    """``path`` as a local checkpoint directory; anything else (a hub model name) is refused."""
    path = os.fspath(path)
    if not os.path.isdir(path):
        raise FileNotFoundError(f"{path!r} is not a local model directory (this build never downloads a model "
                                f"or tokenizer; pass the path of a saved checkpoint)")
    return path


def load_tokenizer(path):
    """The checkpoint's tokenizer (models.py:16-18).  Mistral-3 checkpoints load with
    ``fix_mistral_regex``, as the reference asks of them."""
    from transformers import AutoConfig, AutoTokenizer

    path = _local_dir(path)
    kind = AutoConfig.from_pretrained(path, local_files_only=True).model_type
    extra = {"fix_mistral_regex": True} if kind == "mistral3" else {}
    return AutoTokenizer.from_pretrained(path, local_files_only=True, **extra)


def _long_context(config):
    """Qwen2 checkpoints run with YaRN RoPE scaling, 4x their 32,768-token window (models.py:23-27)."""
    if config.model_type != "qwen2":
        return config
    config.rope_parameters = {"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768,
                              "rope_theta": config.rope_parameters["rope_theta"]}
    config.max_position_embeddings = 32768 * 4
    return config


def load_model(path, device="cuda"):
    """A bf16 checkpoint in eval mode on ``device`` (models.py:21-31): causal LMs through
    ``AutoModelForCausalLM``, checkpoints with a vision tower through ``AutoModelForImageTextToText``.
    Extension: ``device`` (the reference always moves the model to the current GPU)."""
    import transformers

    path = _local_dir(path)
    config = _long_context(transformers.AutoConfig.from_pretrained(path, local_files_only=True))
    auto = (transformers.AutoModelForImageTextToText if getattr(config, "vision_config", None) is not None
            else transformers.AutoModelForCausalLM)
    model = auto.from_pretrained(path, config=config, dtype=torch.bfloat16, local_files_only=True)
    return model.to(device).eval()


def render_prompt(tokenizer, prompt):
    """One user turn through the tokenizer's chat template, ready for the assistant's reply, with the
    reference's fixed date string (models.py:34-36)."""
    messages = [{"role": "user", "content": prompt}]
    return tokenizer.apply_chat_template(messages, tokenize=False, add_generation_prompt=True,
                                         date_string="30 Jul 2026")


def eos_ids(tokenizer, model):
    """Every id that ends generation: the tokenizer's end-of-sequence id(s) together with the model's
    generation config's (models.py:39-41)."""
    found = set()
    for ids in (tokenizer.eos_token_id, model.generation_config.eos_token_id):
        if ids is None:
            continue
        found.update(ids if isinstance(ids, (list, tuple, set)) else [ids])
    return found


class _AllExact:
    """bands_fn that keeps every KV head bf16 (the bands themselves are then unused)."""

    layer_independent = True

    def __init__(self, kv_heads):
        self.kv_heads = kv_heads

    def __call__(self, layer, heads):
        return torch.tensor([[INF, INF]] * heads, dtype=torch.int32)

    def bf16(self, layer):
        return list(range(self.kv_heads))


_exact = {}


def exact_attention(query, key, value, scaling):
    """Exact causal GQA attention, [B, Hq, T, 128] bf16 -> [B, Hq, T, 128] (models.py:45-47).

    Runs the prefill kernel with every KV head exact: bf16 operands, fp32 scores,
    softmax and accumulation."""
    kv_heads = key.shape[1]
    runner = _exact.get(kv_heads)
    if runner is None:
        runner = _exact[kv_heads] = Prefill(load_extension(), _AllExact(kv_heads))
    return runner(0, query, key, value, scaling)


def use_attention(model, name, fn):
    """Register ``fn(module, q, k, v, scaling) -> [B, H, T, D]`` as attention implementation ``name``
    and switch ``model`` to it (models.py:50-55)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    def attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        return fn(module, query, key, value, scaling).transpose(1, 2).contiguous(), None

    ALL_ATTENTION_FUNCTIONS[name] = attention
    model.set_attn_implementation(name)


class TriAttention:
    """Quantized attention for a HF model: prompt through ``Prefill``, generated tokens through
    ``DecodeCache`` (models.py:58-85)."""

    def __init__(self, model, qk_map=None, max_new_tokens=256, module=None, max_tail=None):
        self.model = model
        module = module if module is not None else load_extension()
        # the reference sizes the tail for every new token (max_tail = max_new_tokens); past the tail's
        # 1024-token cap, or with a shorter max_tail, the cache grows instead
        max_tail = min(max_new_tokens, 1024) if max_tail is None else int(max_tail)
        grow = max_new_tokens - max_tail + 64 if max_new_tokens > max_tail else 0
        self.decode_cache = DecodeCache(module, max_tail=max_tail, grow_tail=grow)
        bands_fn = qk_map if callable(qk_map) else load_map(qk_map or preset(model), model)
        self.prefill = Prefill(module, bands_fn, self.decode_cache)

        def attention(mod, query, key, value, scaling):
            if query.shape[2] == 1 and self.decode_cache.stored(mod.layer_idx):
                return self.decode_cache(mod.layer_idx, query, key, value, scaling)
            return self.prefill(mod.layer_idx, query, key, value, scaling)

        use_attention(model, "triattention", attention)

    @torch.inference_mode()
    def generate(self, ids, max_new_tokens, eos, graph=False):
        """Greedy tokens after the prompt ``ids`` [1, T], at most ``max_new_tokens``, stopping before an id
        in ``eos`` (models.py:72-85).

        Extension: ``graph=True`` runs the first generated token's forward eagerly, captures the
        one-token forward (every layer's projections, decode kernels and the step advance) in a
        HIP graph, and replays it for the following tokens with the token id and position written
        into the graph's input buffers.  Same kernels and arguments, so the same tokens."""
        out = self.model(input_ids=ids, use_cache=False, logits_to_keep=1)
        tokens = []
        step = None
        cache = self.decode_cache
        for i in range(max_new_tokens):
            token = int(out.logits[0, -1].argmax())
            if token in eos:
                break
            tokens.append(token)
            # (a step at which a layer's tail is full and its room for tiles taken from the tail used
            # up runs eagerly, which grows the room, and the step is captured again)
            if step is not None and cache.graph_ready():
                step.ids.fill_(token)
                step.position.fill_(ids.shape[1] + i)
                out = step.replay()
                cache.replayed()
                continue
            position = torch.tensor([[ids.shape[1] + i]], device=ids.device)
            out = self.model(input_ids=torch.tensor([[token]], device=ids.device), position_ids=position,
                             use_cache=False)
            self.decode_cache.advance()
            if graph:
                step = _GraphStep(self.model, self.decode_cache, ids.device)
        return tokens


class _GraphStep:
    """The one-token forward plus the decode step advance, captured once and replayed."""

    def __init__(self, model, cache, device):
        self.ids = torch.zeros((1, 1), dtype=torch.long, device=device)
        self.position = torch.zeros((1, 1), dtype=torch.long, device=device)
        # one untimed forward on a side stream first, as graph capture requires of libraries that
        # set up state lazily; it writes the tail slot of the coming step, which the first replay
        # rewrites, and does not advance the step
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            model(input_ids=self.ids, position_ids=self.position, use_cache=False)
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        cache.begin_capture()
        try:
            with torch.cuda.graph(self.graph):
                self.out = model(input_ids=self.ids, position_ids=self.position, use_cache=False)
                cache.advance()
        finally:
            cache.end_capture()

    def replay(self):
        self.graph.replay()
        return self.out
