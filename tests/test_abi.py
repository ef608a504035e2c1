"""The C-ABI library loads and exports every symbol include/triattention_amd.h declares (no GPU calls)."""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

from triattention_amd.kernels.extension import EXPORTS, LIBRARY, load_library

ROOT = Path(__file__).resolve().parent.parent


def header_symbols():
    text = (ROOT / "include" / "triattention_amd.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(tri_\w+)\(", text, re.M)))


def test_library_exports_header_symbols():
    lib = load_library()
    syms = header_symbols()
    assert len(syms) >= 8
    for name in syms:
        assert hasattr(lib, name), name
    assert set(syms) == set(EXPORTS)


def test_validation_errors_need_no_gpu():
    lib = load_library()
    rc = lib.tri_prepare_qk(*([None] + [0] * 3 + [None] + [0] * 3 + [1, 1, 1, 1] + [None] * 12))
    assert rc != 0 and b"null buffer" in lib.tri_last_error()
    blocks = None
    assert lib.tri_decode_occupancy(blocks) != 0 and b"null output" in lib.tri_last_error()


def test_exact_head_validation_needs_no_gpu():
    lib = load_library()
    fake = ctypes.c_void_p(4096)  # aligned, never dereferenced: validation fails before any launch
    rc = lib.tri_pack_exact(None, 0, 0, 0, None, 0, 0, 0, 1, 4, 2, 64, None, 1, None, None, None)
    assert rc != 0 and b"pack_exact: null buffer" in lib.tri_last_error()
    rc = lib.tri_pack_exact(fake, 0, 0, 0, fake, 0, 0, 0, 1, 4, 2, 64, fake, 3, fake, fake, None)
    assert rc != 0 and b"nx must be in [1, hk]" in lib.tri_last_error()
    rc = lib.tri_pack_exact(fake, 0, 0, 12, fake, 0, 0, 128, 1, 4, 2, 64, fake, 1, fake, fake, None)
    assert rc != 0 and b"16-byte aligned" in lib.tri_last_error()
    # attention with exact heads but no records
    rc = lib.tri_attention(fake, 4, fake, 1, 4, 2, 64, fake, fake, fake, fake, fake, fake, fake, None, None, None, None,
                           fake, 0, 0, 0, 0, 0.125, fake, fake, 0, 0, 0, fake, fake, 0, None, None, None)
    assert rc != 0 and b"KX/VX records" in lib.tri_last_error()
    # V8 sums without the V8 records they sum (pack_v and attention)
    rc = lib.tri_pack_v(fake, 0, 0, 128, 1, 2, 64, fake, fake, fake, None, None, fake, None)
    assert rc != 0 and b"V8 sums need the V8 records" in lib.tri_last_error()
    rc = lib.tri_attention(fake, 4, fake, 1, 4, 2, 64, fake, None, fake, fake, fake, fake, fake, None, None, None, None,
                           fake, 0, 0, 0, 0, 0.125, None, None, 0, 0, 0, None, None, 0, fake, None, None)
    assert rc != 0 and b"V8 sums need the V8 records" in lib.tri_last_error()
    # expanded K4 records without the INT4 operands (prepare_qk and attention)
    rc = lib.tri_prepare_qk(fake, 0, 0, 128, fake, 0, 0, 128, 1, 2, 2, 64, fake, fake, fake, fake, fake, fake,
                            None, None, None, None, fake, None)
    assert rc != 0 and b"expanded K4 records need the INT4 buffers" in lib.tri_last_error()
    rc = lib.tri_attention(fake, 4, fake, 1, 4, 2, 64, fake, fake, fake, fake, fake, fake, fake, None, None, None, None,
                           fake, 0, 0, 0, 0, 0.125, None, None, 0, 0, 0, None, None, 0, None, fake, None)
    assert rc != 0 and b"expanded K4 records need the INT4 operands" in lib.tri_last_error()


def _decode_args(fake, per=8, kcur=None, tst=128):
    """tri_decode arguments with every buffer a fake aligned pointer (validation fails before any launch)."""
    kc = kcur if kcur is not None else fake
    return [fake, 24 * 128, 128, fake, None, fake, None, fake, fake, fake, fake, fake, fake, fake, fake, fake,
            fake, fake, 8 * 256 * 128, 256 * tst, tst, 256, kc, kc, 8 * 128, 128, fake, fake, 1, 24 * 128, 128,
            fake, fake, fake, fake, 1, 24, 8, 64, per, 64, 16, 0, 4, 4, None, None, None, 0, None, 0, None, 0,
            None, 0.088, None]


def test_decode_validation_needs_no_gpu():
    lib = load_library()
    fake = ctypes.c_void_p(4096)
    assert lib.tri_decode(*_decode_args(fake, per=65)) != 0
    assert b"in [1, 64]" in lib.tri_last_error()
    assert lib.tri_decode(*_decode_args(fake, kcur=ctypes.c_void_p(4096 + 8))) != 0
    assert b"16-byte aligned rows" in lib.tri_last_error()
    assert lib.tri_decode(*_decode_args(fake, tst=100)) != 0
    assert b"tail buffers must be 16-byte aligned" in lib.tri_last_error()


def test_oracle_library_loads():
    import oracle as O
    assert O.lib().ora_texp2(ctypes.c_float(0.0)) == 1.0


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_noalloc_decode_rejects_partials_beyond_its_scratch():
    """batch x q-heads x splits partials beyond the library's scratch are refused before any device
    work (64 x 32 x 64 = 131072 > 48395)."""
    lib = load_library()
    fake = ctypes.c_void_p(4096)
    args = list(_decode_args(fake, per=1))
    del args[31:34]
    # batch, hq, hk, maxn, per sit right after prompt (index 31 once pm / pl / po are gone)
    args[32], args[33], args[34], args[35], args[36] = 64, 32, 8, 64, 1
    assert lib.tri_decode_noalloc(*args) != 0
    assert b"exceed" in lib.tri_last_error() and b"48395" in lib.tri_last_error()


def test_tail_spill_validation_needs_no_gpu():
    """tri_tail_spill refuses tails shorter than one tile, misaligned tails and missing buffers before
    any device work."""
    lib = load_library()
    fake = ctypes.c_void_p(4096)

    def args(max_tail=256, tst=128, grow=fake):
        return [fake, fake, fake, fake, 8 * max_tail * tst, max_tail * tst, tst, max_tail, 2, 8, 64, 64, grow, 4,
                fake, None, fake, fake, fake, fake, fake, fake, fake, None, fake, fake, fake, 16, None, 0, fake, 16,
                None, None, 0, None, 0, None]
    assert lib.tri_tail_spill(*args(max_tail=32)) != 0
    assert b"max_tail must be in [64, 1024]" in lib.tri_last_error()
    assert lib.tri_tail_spill(*args(tst=100)) != 0
    assert b"16-byte aligned rows" in lib.tri_last_error()
    assert lib.tri_tail_spill(*args(grow=None)) != 0
    assert b"null buffer" in lib.tri_last_error()
