"""Seeded synthetic inputs of the benchmark configurations.

Inputs are generated on the CPU in fp32 with a ``torch.Generator`` seeded per
configuration, outliers applied, cast to bf16, and only then copied to the
device, so CPU and GPU runs see identical bits.

  C0  prefill B1, Hq24/Hk8, T1024: N(0,1), 4 random channels per (tensor, head) x20;
      bands: a seeded half of the KV heads INT8 (INF, INF), the rest INT4 (1, INF).
  C1  decode B32, Hq24/Hk8, prompt 4096: K/V as C0, 25% INT8 / 75% INT4 KV heads.
  C2  prefill B4, Hq28/Hk4, T8192: per (tensor, head, channel) scale exp(U(0, ln 30));
      one seeded KV head bf16; of the others, in a seeded order, one INT8, one INT4 and the
      rest INT8 or INT4 with p = 0.5.
  C3  ragged decode B64, Hq32/Hk8: prompt lengths round(exp(U(ln 512, ln 32768))),
      per-KV-head Bernoulli(0.5) INT8 / INT4.  At full size its prompt K/V are drawn on
      the device (``outlier_tensor_device``); the parity tests copy those draws to the host.
  C4  random-init Qwen2-7B architecture (``config4``): 4096 random prompt ids, a seeded
      per-(layer, KV head) draw over INT8 / INT4 / bf16.
"""
from __future__ import annotations

import math

import torch

INF = 1 << 20
INT8_BAND = (INF, INF)
INT4_BAND = (1, INF)


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def outlier_tensor(g: torch.Generator, batch: int, heads: int, t: int, d: int = 128, factor: float = 20.0,
                   channels: int = 4) -> torch.Tensor:
    x = torch.randn(batch, heads, t, d, generator=g)
    for b in range(batch):
        for h in range(heads):
            idx = torch.randperm(d, generator=g)[:channels]
            x[b, h, :, idx] *= factor
    return x.to(torch.bfloat16)


def loguniform_scaled_tensor(g: torch.Generator, batch: int, heads: int, t: int, d: int = 128,
                             hi: float = 30.0) -> torch.Tensor:
    x = torch.randn(batch, heads, t, d, generator=g)
    scale = torch.exp(torch.rand(batch, heads, 1, d, generator=g) * math.log(hi))
    return (x * scale).to(torch.bfloat16)


def kv_head_bands(kinds, group: int) -> torch.Tensor:
    """Per q-head (w8, w4) from a per-KV-head kind list ('i8' / 'i4' / 'bf16')."""
    rows = []
    for kind in kinds:
        band = INT4_BAND if kind == "i4" else INT8_BAND
        rows += [band] * group
    return torch.tensor(rows, dtype=torch.int32)


def split_kinds(g: torch.Generator, hk: int, n8: int):
    perm = torch.randperm(hk, generator=g).tolist()
    kinds = ["i4"] * hk
    for h in perm[:n8]:
        kinds[h] = "i8"
    return kinds


def config0(seed: int = 1000, t: int = 1024, hq: int = 24, hk: int = 8):
    g = gen(seed)
    q = outlier_tensor(g, 1, hq, t)
    k = outlier_tensor(g, 1, hk, t)
    v = outlier_tensor(g, 1, hk, t)
    kinds = split_kinds(g, hk, hk // 2)
    return dict(q=q, k=k, v=v, kinds=kinds, bands=kv_head_bands(kinds, hq // hk), scale=128 ** -0.5)


def config1(seed: int = 1001, batch: int = 32, prompt: int = 4096, hq: int = 24, hk: int = 8):
    g = gen(seed)
    kinds = split_kinds(g, hk, hk // 4)
    seqs = []
    for b in range(batch):
        gb = gen(seed + b + 1)
        seqs.append(dict(q=outlier_tensor(gb, 1, hq, prompt), k=outlier_tensor(gb, 1, hk, prompt),
                         v=outlier_tensor(gb, 1, hk, prompt)))
    qd = outlier_tensor(g, batch, hq, 1)
    kd = outlier_tensor(g, batch, hk, 1)
    vd = outlier_tensor(g, batch, hk, 1)
    return dict(seqs=seqs, kinds=kinds, bands=kv_head_bands(kinds, hq // hk), q=qd, k=kd, v=vd,
                prompt=prompt, scale=128 ** -0.5)


def config2(seed: int = 1002, batch: int = 4, t: int = 8192, hq: int = 28, hk: int = 4):
    g = gen(seed)
    q = loguniform_scaled_tensor(g, batch, hq, t)
    k = loguniform_scaled_tensor(g, batch, hk, t)
    v = loguniform_scaled_tensor(g, batch, hk, t)
    bf16_head = int(torch.randint(hk, (1,), generator=g))
    # the other KV heads split 50/50 between INT8 and INT4: a seeded order of them, the first INT8, the
    # second INT4 (so both kinds always occur), any further ones Bernoulli(0.5)
    rest = [h for h in range(hk) if h != bf16_head]
    rest = [rest[i] for i in torch.randperm(len(rest), generator=g).tolist()]
    kinds = ["bf16"] * hk
    for n, h in enumerate(rest):
        kinds[h] = "i8" if n == 0 else "i4" if n == 1 else ("i8" if float(torch.rand(1, generator=g)) < 0.5 else "i4")
    return dict(q=q, k=k, v=v, kinds=kinds, bands=kv_head_bands(kinds, hq // hk), scale=128 ** -0.5)


def config3_lengths(seed: int = 1003, batch: int = 64, lo: int = 512, hi: int = 32768):
    g = gen(seed)
    u = torch.rand(batch, generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(x) * (math.log(hi) - math.log(lo))))) for x in u]


def outlier_tensor_device(g: torch.Generator, batch: int, heads: int, t: int, d: int = 128,
                          factor: float = 20.0, channels: int = 4) -> torch.Tensor:
    """``outlier_tensor``'s distribution drawn on the generator's device (for full-size
    configurations whose host generation would take minutes; bits differ from the host draw)."""
    x = torch.randn(batch, heads, t, d, generator=g, device=g.device)
    idx = torch.rand(batch, heads, d, generator=g, device=g.device).argsort(-1)[..., :channels]
    mult = torch.ones(batch, heads, d, device=g.device).scatter_(-1, idx, factor)
    return (x * mult[:, :, None, :]).to(torch.bfloat16)


def config3_map(seed: int = 1003, hq: int = 32, hk: int = 8):
    """Per-KV-head INT8 / INT4 kinds of config 3 and the q-head bands they give."""
    g = gen(seed + 7)
    kinds = ["i8" if float(torch.rand(1, generator=g)) < 0.5 else "i4" for _ in range(hk)]
    return kinds, kv_head_bands(kinds, hq // hk)


def config3(seed: int = 1003, batch: int = 64, hq: int = 32, hk: int = 8, lengths=None):
    lengths = lengths or config3_lengths(seed, batch)
    g = gen(seed + 7)
    kinds = ["i8" if float(torch.rand(1, generator=g)) < 0.5 else "i4" for _ in range(hk)]
    seqs = []
    for b, n in enumerate(lengths):
        gb = gen(seed + 100 + b)
        seqs.append(dict(q=outlier_tensor(gb, 1, hq, n), k=outlier_tensor(gb, 1, hk, n),
                         v=outlier_tensor(gb, 1, hk, n)))
    qd = outlier_tensor(g, len(lengths), hq, 1)
    kd = outlier_tensor(g, len(lengths), hk, 1)
    vd = outlier_tensor(g, len(lengths), hk, 1)
    return dict(seqs=seqs, lengths=lengths, kinds=kinds, bands=kv_head_bands(kinds, hq // hk), q=qd, k=kd, v=vd,
                scale=128 ** -0.5)


def bits(x: torch.Tensor):
    """uint16 numpy view of a bf16 CPU tensor."""
    import numpy as np
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def config4(seed: int = 1004, prompt: int = 4096):
    """C4 model configuration (keyword arguments of transformers.Qwen2Config), prompt ids [1, prompt], and
    the map: per (layer, KV head) a uniform draw over INT8 / INT4 / bf16 -> (bands by layer, bf16 KV heads
    by layer, kinds [28, 4] with 0 INT8, 1 INT4, 2 bf16)."""
    cfg = dict(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
               num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=32768, rope_theta=1e6,
               initializer_range=0.02, tie_word_embeddings=False)
    g = gen(seed)
    ids = torch.randint(152064, (1, prompt), generator=g)
    kinds = torch.randint(3, (28, 4), generator=g)
    band = {0: [INF, INF], 1: [1, INF], 2: [INF, INF]}
    bands = {str(l): [band[int(kinds[l, h // 7])] for h in range(28)] for l in range(28)}
    bf16 = {str(l): [h for h in range(4) if int(kinds[l, h]) == 2] for l in range(28)}
    return cfg, ids, bands, bf16, kinds
