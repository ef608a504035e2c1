"""Writes the golden vectors of tests/golden/ from the CPU oracle (run from the repository root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors or known-answer tests for this path (its
kernels are CUDA only), so these fixtures are the oracle's outputs on seeded
inputs, pinned once the oracle itself was pinned against closed forms and
float64 references (tests/test_oracle.py).  They freeze that result: a later
change to the oracle or to the kernels that moves any code, scale or output is
caught against the stored arrays.

Contents (inputs are stored as bf16 bit patterns, so no RNG is re-run):
  rotation.npz  R e_i for the 128 basis vectors and R x for 8 seeded vectors
  codes_T{t}.npz  Q/K/V codes, scales and statistics, Hq 6 / Hk 2 (g 3), mixed bands
  prefill_T200.npz  prefill output (fp32) for the inputs of codes_T200.npz
  decode_L{l}.npz  decode outputs (fp32) at steps 0..3 after a prompt of length l
  bands.npz  per (band, query tile) the visit order of key tiles with their kind (F16 / INT8 /
             INT4 QK), and the decode tile states
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402
from triattention_amd import synthetic as S  # noqa: E402
from triattention_amd.synthetic import INF, bits  # noqa: E402

HQ, HK = 6, 2
BANDS = np.array([[INF, INF], [1, INF], [2, 3], [1, 1], [3, INF], [2, 2]], np.int32)
SCALE = 128 ** -0.5
TS = (1, 63, 64, 65, 200)
PROMPTS = (64, 300)
STEPS = 4
MAX_TAIL = 8
PER = 2


def inputs(seed, t):
    g = S.gen(seed)
    q = S.outlier_tensor(g, 1, HQ, t)[0]
    k = S.outlier_tensor(g, 1, HK, t)[0]
    v = S.outlier_tensor(g, 1, HK, t)[0]
    return bits(q), bits(k), bits(v)


def main():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    np.savez_compressed(HERE / "rotation.npz", basis=O.rotate(np.eye(128, dtype=np.float32)), x=x, rx=O.rotate(x))
    for t in TS:
        q, k, v = inputs(9000 + t, t)
        c = O.prefill_codes(q, k, v, BANDS, decode_cache=True)
        arrays = {name: c[name] for name in ("q8", "qa", "q4", "qa4", "k8", "ka", "k4", "ka4", "kstat", "vstat",
                                              "v16", "v8", "v4") if c[name] is not None}
        np.savez_compressed(HERE / f"codes_T{t}.npz", q=q, k=k, v=v, bands=BANDS, **arrays)
        if t == 200:
            out = O.prefill_attention(c, BANDS, HQ, HK, t, SCALE)
            np.savez_compressed(HERE / "prefill_T200.npz", bands=BANDS, scale=SCALE, out=out)  # inputs: codes_T200
    for prompt in PROMPTS:
        q, k, v = inputs(9500 + prompt, prompt)
        c = O.prefill_codes(q, k, v, BANDS, decode_cache=True)
        g = S.gen(9600 + prompt)
        qd = bits(S.outlier_tensor(g, 1, HQ, STEPS)[0].transpose(0, 1).contiguous())  # [steps, Hq, 128]
        kd = bits(S.outlier_tensor(g, 1, HK, STEPS)[0].transpose(0, 1).contiguous())
        vd = bits(S.outlier_tensor(g, 1, HK, STEPS)[0].transpose(0, 1).contiguous())
        ktail = np.zeros((HK, MAX_TAIL, 128), np.uint16)
        vtail = np.zeros_like(ktail)
        outs = []
        for step in range(STEPS):
            outs.append(O.decode(c, BANDS, qd[step], prompt, PER, SCALE, ktail, vtail, kd[step], vd[step], step))
            ktail[:, step], vtail[:, step] = kd[step], vd[step]
        np.savez_compressed(HERE / f"decode_L{prompt}.npz", q=q, k=k, v=v, bands=BANDS, scale=SCALE, per=PER,
                            max_tail=MAX_TAIL, qd=qd, kd=kd, vd=vd, out=np.stack(outs))
    rows = 40
    band_set = np.array([[1, 1], [1, INF], [INF, INF], [2, 3], [3, 9], [5, 5], [4, 17], [16, 40]], np.int32)
    cols, kinds, offsets = [], [], [0]
    for w8, w4 in band_set:
        for qb in range(rows):
            visits = O.band_tiles(w8, w4, qb)
            cols += [c for c, _ in visits]
            kinds += [kd for _, kd in visits]
            offsets.append(len(cols))
    state = np.array([[O.decode_state(w8, w4, rows, j) for j in range(rows)] for w8, w4 in band_set], np.int64)
    np.savez_compressed(HERE / "bands.npz", bands=band_set, rows=rows, cols=np.array(cols, np.int32),
                        kinds=np.array(kinds, np.int8), offsets=np.array(offsets, np.int64), state=state)
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    torch.set_num_threads(1)
    main()
