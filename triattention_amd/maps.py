"""Per-head distance-band maps (format ``triattention-map-v1``).

Mirrors triattention/maps.py:13-41: ``load_map`` / ``from_bands`` / ``uniform``
/ ``preset`` return a ``bands_fn(layer, heads) -> int32 [heads, 2]`` of
``(w8, w4)`` in 64-token tiles; ``INF = 1 << 20`` marks an unbounded band.

Extension (ignored by v1 readers, which read only ``"bands"``): an optional
``"bf16": {"<layer>": [kv_head, ...]}`` key lists KV heads whose attention is
computed exactly on the unquantized bf16 operands.  ``bands_fn.bf16(layer)``
returns that list (empty when absent).
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

INF = 1 << 20
DATA = Path(__file__).resolve().parent / "data"
PRESETS = {"llama": "llama-3.2-3b-instruct", "qwen2": "qwen2-7b-instruct", "mistral3": "ministral-3-8b-instruct-2512"}


def preset(model):
    name = PRESETS.get(model.config.model_type)
    if name is None:
        raise ValueError(f"no bundled map for model type {model.config.model_type!r}; pass --map")
    return DATA / f"{name}.json"


def load_map(path, model=None):
    data = json.loads(Path(path).read_text())
    return from_bands(data["bands"], model, bf16=data.get("bf16"))


def from_bands(bands, model=None, bf16=None):
    if model is not None:
        text = getattr(model.config, "text_config", model.config)
        if len(bands) != text.num_hidden_layers or len(bands["0"]) != text.num_attention_heads:
            raise ValueError("the map does not match the model's layers and heads")

    def bands_fn(layer, heads):
        return torch.tensor(bands[str(layer)], dtype=torch.int32)

    bands_fn.bf16 = lambda layer: list((bf16 or {}).get(str(layer), []))
    return bands_fn


def uniform(w8, w4):
    def bands_fn(layer, heads):
        return torch.tensor([[w8, w4]] * heads, dtype=torch.int32)

    bands_fn.layer_independent = True
    bands_fn.bf16 = lambda layer: []
    return bands_fn


def save_map(path, bands, bf16=None, **header):
    """Write a map v1 file (select.py:76-78 layout), with the optional bf16 key."""
    data = dict(format="triattention-map-v1", **header, bands={str(k): [list(map(int, b)) for b in v]
                                                               for k, v in bands.items()})
    if bf16:
        data["bf16"] = {str(k): [int(h) for h in v] for k, v in bf16.items()}
    Path(path).write_text(json.dumps(data, separators=(",", ":")) + "\n")
