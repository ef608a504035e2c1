"""Golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py from the pinned oracle).

CPU: the oracle and the product's host-side band logic reproduce the stored arrays exactly.
GPU: the kernels reproduce the stored codes and scales bit for bit and the stored outputs within the
parity tolerance (2e-3 max-abs / 1e-3 mean-abs)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, compare_codes, run_prefill
from triattention_amd.kernels.decode import DecodeCache, tile_states
from triattention_amd.kernels.prefill import tile_counts

GOLDEN = Path(__file__).resolve().parent / "golden"
TS = (1, 63, 64, 65, 200)
CODE_KEYS = ("q8", "qa", "q4", "qa4", "k8", "ka", "k4", "ka4", "kstat", "vstat", "v16", "v8", "v4")


def load(name):
    return dict(np.load(GOLDEN / name, allow_pickle=False))


def bf16(bits_u16, batch=True):
    t = torch.from_numpy(np.ascontiguousarray(bits_u16).view(np.int16)).view(torch.bfloat16)
    return t[None] if batch else t


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


# --------------------------------------------------------------------------- CPU
def test_rotation_vectors():
    g = load("rotation.npz")
    same(O.rotate(np.eye(128, dtype=np.float32)), g["basis"])
    same(O.rotate(g["x"]), g["rx"])


@pytest.mark.parametrize("t", TS)
def test_oracle_codes(t):
    g = load(f"codes_T{t}.npz")
    c = O.prefill_codes(g["q"], g["k"], g["v"], g["bands"], decode_cache=True)
    for key in CODE_KEYS:
        if key in g:
            same(c[key], g[key])
        else:
            assert c[key] is None, key


def test_oracle_prefill_output():
    g, inp = load("prefill_T200.npz"), load("codes_T200.npz")
    c = O.prefill_codes(inp["q"], inp["k"], inp["v"], g["bands"], decode_cache=True)
    same(O.prefill_attention(c, g["bands"], 6, 2, 200, float(g["scale"])), g["out"])


@pytest.mark.parametrize("prompt", (64, 300))
def test_oracle_decode_outputs(prompt):
    g = load(f"decode_L{prompt}.npz")
    c = O.prefill_codes(g["q"], g["k"], g["v"], g["bands"], decode_cache=True)
    ktail = np.zeros((2, int(g["max_tail"]), 128), np.uint16)
    vtail = np.zeros_like(ktail)
    for step in range(g["out"].shape[0]):
        out = O.decode(c, g["bands"], g["qd"][step], prompt, int(g["per"]), float(g["scale"]), ktail, vtail,
                       g["kd"][step], g["vd"][step], step)
        same(out, g["out"][step])
        ktail[:, step], vtail[:, step] = g["kd"][step], g["vd"][step]


def test_band_visits_and_states():
    g = load("bands.npz")
    rows, bands = int(g["rows"]), g["bands"]
    i = 0
    for w8, w4 in bands:
        for qb in range(rows):
            lo, hi = g["offsets"][i], g["offsets"][i + 1]
            visits = O.band_tiles(w8, w4, qb)
            assert [c for c, _ in visits] == g["cols"][lo:hi].tolist()
            assert [k for _, k in visits] == g["kinds"][lo:hi].tolist()
            i += 1
    for h, (w8, w4) in enumerate(bands):
        assert [O.decode_state(w8, w4, rows, j) for j in range(rows)] == g["state"][h].tolist()


def test_host_band_logic_matches_the_fixtures():
    """The product's own host restatements (Prefill.tile_counts, DecodeCache tile_states) agree with the
    stored visit kinds and decode states."""
    g = load("bands.npz")
    rows = int(g["rows"])
    n8, n4 = tile_counts(torch.from_numpy(g["bands"]), rows)
    states = tile_states(torch.from_numpy(g["bands"]), rows)
    i = 0
    for h in range(len(g["bands"])):
        for qb in range(rows):
            kinds = g["kinds"][g["offsets"][i]:g["offsets"][i + 1]]
            assert int((kinds == 1).sum()) == int(n8[h, qb]) and int((kinds == 2).sum()) == int(n4[h, qb])
            i += 1
    assert states.tolist() == g["state"].tolist()


# --------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("t", TS)
def test_kernel_codes_match_golden(module, t):
    print(f"\n[golden] codes T={t}", flush=True)
    g = load(f"codes_T{t}.npz")
    codes = {key: g.get(key) for key in CODE_KEYS}
    cache = DecodeCache(module, max_tail=8)
    out, ops, pre = run_prefill(module, bf16(g["q"]), bf16(g["k"]), bf16(g["v"]), torch.from_numpy(g["bands"]),
                                128 ** -0.5, decode_cache=cache)
    e = cache.layers[0]
    compare_codes(ops, codes, 0, 1, 6, 2, t, kept=(e["ka"], e["kstat"], e["vstat"], e["ka4"]))
    if t == 200:
        assert_close(out[0].numpy(), load("prefill_T200.npz")["out"], what="prefill T200 vs golden")


@pytest.mark.gpu
@pytest.mark.parametrize("prompt", (64, 300))
def test_kernel_decode_matches_golden(module, prompt):
    print(f"\n[golden] decode L={prompt}", flush=True)
    g = load(f"decode_L{prompt}.npz")
    dev = torch.device("cuda")
    cache = DecodeCache(module, max_tail=int(g["max_tail"]))
    cache.out_dtype = torch.float32
    run_prefill(module, bf16(g["q"]), bf16(g["k"]), bf16(g["v"]), torch.from_numpy(g["bands"]), float(g["scale"]),
                decode_cache=cache)
    for step in range(g["out"].shape[0]):
        qd = bf16(g["qd"][step])[:, :, None].to(dev)
        kd = bf16(g["kd"][step])[:, :, None].to(dev)
        vd = bf16(g["vd"][step])[:, :, None].to(dev)
        out = cache(0, qd, kd, vd, float(g["scale"])).float().cpu().numpy()
        assert_close(out[0, :, 0], g["out"][step], what=f"decode L{prompt} step {step} vs golden")
        cache.advance()
