"""Host-side logic without a GPU: band table, decode metadata, maps, record codec."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import oracle as O
from triattention_amd import maps
from triattention_amd.kernels import records as R
from triattention_amd.kernels.decode import ENTRY_TILE, ENTRY_V8, ENTRY_VFMT, DecodeCache, sequence_metadata, tile_states
from triattention_amd.kernels.prefill import F16, I4, I8, Q4, BandTable
from triattention_amd.synthetic import INF


def test_band_table_order_and_formats():
    bands = torch.tensor([[INF, INF], [1, INF], [2, 4], [3, 3], [1, 1], [2, INF]], dtype=torch.int32)
    rows, hk = 7, 2
    t = BandTable.build(bands, rows, hk, "cpu")
    expect = [qh * rows + qb for kv in range(hk) for qb in reversed(range(rows)) for qh in range(kv * 3, kv * 3 + 3)]
    assert t.order.tolist() == expect
    assert t.formats == frozenset(O.formats_for(bands.numpy(), rows))
    assert BandTable.build(torch.tensor([[INF, INF]] * 2, dtype=torch.int32), 2, 1, "cpu").formats == {F16}
    assert BandTable.build(torch.tensor([[1, INF]] * 2, dtype=torch.int32), 3, 1, "cpu").formats == {F16, Q4}


def brute_metadata(bands, tiles, hk, vcodes):
    """Enumeration restatement of decode.py:27-53 for one sequence."""
    hq = len(bands)
    g = hq // hk
    out = []
    c8 = c4 = 0
    v8 = v4 = 0
    per_head = []
    for kh in range(hk):
        kept = []
        for j in range(tiles):
            st = [O.decode_state(*bands[kh * g + r], tiles, j) for r in range(g)]
            if max(st) > 0:
                kept.append((j, max(st), sum(1 << r for r in range(g) if st[r] > 0)))
        per_head.append(kept)
    for kh in range(hk):
        rows = []
        for j, kv, mask in per_head[kh]:
            if kv == 4:
                ks, c4 = c4, c4 + 1
            else:
                ks, c8 = c8, c8 + 1
            if vcodes[j] == I8:
                vs, v8 = v8, v8 + 1
            else:
                vs, v4 = v4, v4 + 1
            rows.append((j, mask | ((kv == 4) << 8) | (ks << 9), vs))
        out.append(rows)
    return out


@pytest.mark.parametrize("bands", [
    [[INF, INF], [1, INF], [2, 4], [3, 3], [1, 1], [2, INF]],
    [[2, 4], [2, 4], [2, 4], [1, 2], [1, 2], [1, 2]],
    [[0, 0], [1, 1], [5, 5], [1, 3], [INF, INF], [2, 2]],
])
def test_decode_metadata_enumeration(bands):
    tiles, hk = 5, 2
    vcodes = torch.where((tiles - 1 - torch.arange(tiles) < 16) | (torch.arange(tiles) == 0), I8, I4)
    vcodes = torch.tensor([I8, I4, I4, I8, I8])  # exercise both V formats
    m = sequence_metadata(torch.tensor(bands), tiles, hk, vcodes)
    ref = brute_metadata(bands, tiles, hk, vcodes.tolist())
    for kh in range(hk):
        n = int(m["count"][kh])
        assert n == len(ref[kh])
        for e, (j, kinfo, vs) in enumerate(ref[kh]):
            assert int(m["order"][kh, e]) == j
            assert int(m["kbase"][kh, e] | (m["kslot"][kh, e] << 9)) == kinfo
            assert int(m["vslot"][kh, e]) == vs


def test_tile_states_closed_form():
    s = tile_states(torch.tensor([[2, 4], [INF, INF], [1, INF], [0, 0]]), 6)
    assert s.tolist() == [[8, 0, 4, 4, 8, 8], [8] * 6, [8, 4, 4, 4, 4, 8], [8, 0, 0, 0, 0, 0]]


from cache_host import HostCacheModule as FakeModule  # noqa: E402


def test_balanced_partition_is_a_valid_cost_balanced_split():
    """Bounds start at 0, end at the count, never decrease, hold at most 64 entries per split, fit the
    slot budget, and cut C1-like heads (INT8 or INT4 K, INT8 V on the sink and last 16 tiles) into
    splits within 10% of the mean cost at two workgroups per SIMD."""
    from triattention_amd.kernels.decode import balanced_partition, entry_costs
    rng = np.random.default_rng(3)
    cache = DecodeCache(None)
    hk = 8
    for tiles, slots, batch in ((64, 2048, 32), (64, 1024, 32), (7, 64, 3), (512, 300, 2), (1, 16, 1)):
        w8 = rng.choice([1, 2, INF], size=3 * hk)
        bands = torch.tensor([[int(a), INF] for a in w8], dtype=torch.int32)
        meta = sequence_metadata(bands, tiles, hk, cache.codes(tiles)[0])
        (b,), splits = balanced_partition([meta], [batch], slots)
        assert b.shape == (hk, splits + 1) and b.dtype == torch.int32
        assert (b[:, 0] == 0).all() and (b[:, -1] == meta["count"]).all()
        sizes = b.diff(dim=1)
        assert (sizes >= 0).all() and (sizes <= 64).all()
        n = (sizes > 0).sum(1)
        floor = int(torch.clamp((meta["count"] + 63) // 64, min=1).sum())
        assert batch * int(n.sum()) <= max(slots, batch * floor)
        if tiles == 64 and slots == 2048:
            c = torch.from_numpy(entry_costs(meta))
            cum = torch.cat([torch.zeros(hk, 1, dtype=torch.float64), c.cumsum(1)], 1)
            part = (cum.gather(1, b[:, 1:].long()) - cum.gather(1, b[:, :-1].long()))[sizes > 0]
            assert float(part.max()) <= 1.1 * float(part.mean())
    # a head far costlier than the rest still gets runs of at most 64 entries
    meta = sequence_metadata(torch.tensor([[INF, INF]] * 4, dtype=torch.int32), 300, 2,
                             cache.codes(300)[0], exact_kv=[1])
    (b,), _ = balanced_partition([meta], [1], 4)
    assert (b.diff(dim=1) <= 64).all() and (b[:, -1] == meta["count"]).all()


def test_ragged_cache_assembly_slots_are_consistent():
    cache = DecodeCache(FakeModule(), max_tail=8)
    cache.ragged = True
    hk, bands = 2, torch.tensor([[INF, INF], [1, INF], [2, 4], [1, 1]], dtype=torch.int32)
    rng = torch.Generator().manual_seed(0)
    seen = []
    for prompt, batch in ((100, 2), (700, 1), (64, 3)):
        tiles = (prompt + 63) // 64
        kp = torch.randint(0, 2 ** 31, (batch * hk * tiles * 2048,), generator=rng).to(torch.uint32)
        k4 = torch.randint(0, 2 ** 31, (batch * hk * tiles * 1024,), generator=rng).to(torch.uint32)
        packed = {F16: None, I8: torch.randint(0, 2 ** 31, (batch * hk * tiles * 2048,), generator=rng).to(torch.uint32),
                  I4: torch.randint(0, 2 ** 31, (batch * hk * tiles * 1024,), generator=rng).to(torch.uint32)}
        ka = torch.rand(batch * hk * tiles * 4, generator=rng)
        ka4 = torch.rand(batch * hk * tiles * 4, generator=rng)
        stat = torch.rand(batch, hk, 3, 128, generator=rng)
        codes, _ = cache.codes(tiles)
        cache.store(0, prompt, kp, ka, stat.clone(), stat.clone(), packed, codes, bands, k4, ka4)
        seen.append((prompt, batch, kp.view(batch, hk, tiles, 2048), k4.view(batch, hk, tiles, 1024),
                     packed[I8].view(batch, hk, tiles, 2048), packed[I4].view(batch, hk, tiles, 1024)))
    e = cache.layers[0]
    assert e["batch"] == 6 and e["prompt"].tolist() == [100, 100, 700, 64, 64, 64]
    # every kept entry points at the record of its own sequence, head and tile
    row = 0
    for prompt, batch, k8, k4, v8, v4 in seen:
        for s in range(batch):
            for kh in range(hk):
                for n in range(int(e["count"][row, kh])):
                    word = int(e["entry"][row, kh, n])
                    j = word & ENTRY_TILE
                    # the V format travels in the entry word too, and agrees with fmt
                    assert word & ENTRY_VFMT and bool(word & ENTRY_V8) == (int(e["fmt"][row, j]) == 1)
                    info = int(e["kinfo"][row, kh, n])
                    src, dst = (k4, e["k4"]) if (info >> 8) & 1 else (k8, e["k8"])
                    assert torch.equal(dst[info >> 9], src[s, kh, j])
                    vsrc, vdst = (v8, e["v"][I8]) if int(e["fmt"][row, j]) == 1 else (v4, e["v"][I4])
                    assert torch.equal(vdst[int(e["slot"][row, kh, n])], vsrc[s, kh, j])
            row += 1


def test_split_rule_balances_one_wave_and_runs_uniform_above():
    """Up to BALANCE_TILES kept tiles per slot the cache holds a balanced partition (bounds cover every
    kept entry); above it, uniform runs of `per` tiles and no bounds; cache.per forces the uniform
    split."""
    from triattention_amd.kernels.decode import BALANCE_TILES
    hk, bands = 2, torch.tensor([[INF, INF], [1, INF], [2, 4], [1, 1]], dtype=torch.int32)
    prompt, batch = 3000, 2
    tiles = (prompt + 63) // 64
    z32 = lambda n: torch.zeros(n, dtype=torch.int32).to(torch.uint32)
    for wave, per, balanced in ((1024, None, True), (2, None, False), (1024, 5, False)):
        cache = DecodeCache(FakeModule(), max_tail=8)
        cache.wave, cache.per = wave, per
        codes, _ = cache.codes(tiles)
        packed = {F16: None, I8: z32(batch * hk * tiles * 2048), I4: z32(batch * hk * tiles * 1024)}
        stat = torch.zeros(batch, hk, 3, 128)
        cache.store(0, prompt, z32(batch * hk * tiles * 2048), torch.ones(batch * hk * tiles * 4), stat.clone(),
                    stat.clone(), packed, codes, bands, z32(batch * hk * tiles * 1024), torch.ones(batch * hk * tiles * 4))
        e = cache.layers[0]
        kept = int(e["count"].sum())
        assert (kept <= BALANCE_TILES * wave and per is None) == balanced
        if balanced:
            b = e["bounds_host"]
            assert b.shape == (batch, hk, e["splits"] + 1)
            assert (b[:, :, 0] == 0).all() and (b[:, :, -1] == e["count"].numpy()).all()
            assert np.array_equal(cache.split_of(0, 1), b[1])
        else:
            assert e["bounds"] is None and e["splits"] == -(-e["maxn"] // e["per"])
            assert cache.split_of(0, 0) == e["per"] and (per is None or e["per"] == per)


def test_exact_heads_in_a_ragged_cache():
    """bf16 KV heads keep every tile, select no quantized record, and xslot points at their own KX records."""
    cache = DecodeCache(FakeModule(), max_tail=8)
    cache.ragged = True
    hk, bands = 3, torch.tensor([[2, 4], [1, INF], [INF, INF], [1, 1], [3, 3], [1, 2]], dtype=torch.int32)
    exact_kv = [0, 2]
    rng = torch.Generator().manual_seed(1)
    seen = []
    for prompt, batch in ((300, 2), (64, 1)):
        tiles = (prompt + 63) // 64
        kp = torch.randint(0, 2 ** 31, (batch * hk * tiles * 2048,), generator=rng).to(torch.uint32)
        k4 = torch.randint(0, 2 ** 31, (batch * hk * tiles * 1024,), generator=rng).to(torch.uint32)
        packed = {F16: None, I8: torch.randint(0, 2 ** 31, (batch * hk * tiles * 2048,), generator=rng).to(torch.uint32),
                  I4: torch.randint(0, 2 ** 31, (batch * hk * tiles * 1024,), generator=rng).to(torch.uint32)}
        ka = torch.rand(batch * hk * tiles * 4, generator=rng)
        stat = torch.rand(batch, hk, 3, 128, generator=rng)
        kx = torch.randint(0, 256, (batch * 2 * tiles * 16384 + 999,), generator=rng).to(torch.uint8)
        vx = torch.randint(0, 256, kx.shape, generator=rng).to(torch.uint8)
        codes, _ = cache.codes(tiles)
        cache.store(0, prompt, kp, ka, stat.clone(), stat.clone(), packed, codes, bands, k4, ka.clone(), exact_kv,
                    kx, vx)
        seen.append((prompt, batch, tiles, kx[:batch * 2 * tiles * 16384].view(batch, 2, tiles, 16384),
                     vx[:batch * 2 * tiles * 16384].view(batch, 2, tiles, 16384)))
    e = cache.layers[0]
    kxs, vxs = e["kx"].view(-1, 16384), e["vx"].view(-1, 16384)
    row = 0
    for prompt, batch, tiles, kx, vx in seen:
        for s in range(batch):
            assert int(e["xslot"][row, 1]) == -1
            for slot, h in enumerate(exact_kv):
                assert int(e["count"][row, h]) == tiles
                assert (e["entry"][row, h, :tiles] & ENTRY_TILE).tolist() == list(range(tiles))
                x0 = int(e["xslot"][row, h])
                for j in range(tiles):
                    assert torch.equal(kxs[x0 + j], kx[s, slot, j]) and torch.equal(vxs[x0 + j], vx[s, slot, j])
            row += 1
    # only KV head 1 selects quantized records
    n8 = sum(int(sequence_metadata(bands, (p + 63) // 64, hk, cache.codes((p + 63) // 64)[0], exact_kv)["is8"].sum()) * b
             for p, b, *_ in seen)
    assert e["k8"].shape[0] == n8


def test_maps_bundled_and_extension(tmp_path):
    for name in maps.PRESETS.values():
        data = json.loads((maps.DATA / f"{name}.json").read_text())
        assert data["format"] == "triattention-map-v1"
        fn = maps.load_map(maps.DATA / f"{name}.json")
        b = fn(0, len(data["bands"]["0"]))
        assert b.dtype == torch.int32 and b.shape[1] == 2 and fn.bf16(0) == []

    class Cfg:
        num_hidden_layers, num_attention_heads = 2, 3

    class Model:
        config = Cfg()

    bands = {"0": [[1, 2]] * 3, "1": [[INF, INF]] * 3}
    maps.from_bands(bands, Model())
    with pytest.raises(ValueError):
        maps.from_bands({"0": [[1, 2]] * 3}, Model())
    p = tmp_path / "m.json"
    maps.save_map(p, bands, bf16={1: [0]}, model_type="qwen2")
    fn = maps.load_map(p)
    assert fn(1, 3).tolist() == [[INF, INF]] * 3 and fn.bf16(1) == [0] and fn.bf16(0) == []
    u = maps.uniform(4, 8)
    assert u(0, 5).tolist() == [[4, 8]] * 5 and u.layer_independent


def test_record_codec_round_trip_and_layout():
    rng = np.random.default_rng(0)
    codes = rng.integers(-127, 128, (3, 64, 128)).astype(np.int8)
    assert np.array_equal(R.unpack_k8(R.pack_k8(codes)), codes)
    assert np.array_equal(R.unpack_v8(R.pack_v8(codes)), codes)
    c4 = rng.integers(-7, 8, (3, 64, 128)).astype(np.int8)
    assert np.array_equal(R.unpack_k4(R.pack_k4(c4)), c4)
    assert np.array_equal(R.unpack_v4(R.pack_v4(c4)), c4)
    h = rng.integers(0, 65535, (2, 64, 128)).astype(np.uint16)
    assert np.array_equal(R.unpack_v16(R.pack_v16(h)), h)
    # layout pins: K8 byte of (key 37, feature 90); V8 byte of (key 13, channel 70)
    rec = R.pack_k8(codes[:1]).reshape(-1)
    kb, kk, ks, f = 1, 5, 2, 90 - 64
    assert rec[(kb * 4 + ks) * 1024 + (kk + 32 * (f // 16)) * 16 + f % 16] == codes[0, 37, 90].view(np.uint8)
    rec = R.pack_v8(codes[:1]).reshape(-1)
    key, ch = 13, 70
    kb, w = key // 32, key % 32
    p = 4 * (w // 8) + w % 4
    L = (ch % 32) + 32 * ((w % 8) // 4)
    assert rec[((ch // 32) * 2 + kb) * 1024 + L * 16 + p] == codes[0, 13, 70].view(np.uint8)


def test_every_head_exact_keeps_one_placeholder_record_per_kind():
    """A layer whose KV heads are all bf16 selects no quantized record; each record array the kernel
    takes is then a single zero record (the kernel needs non-empty arrays and never reads it)."""
    cache = DecodeCache(FakeModule(), max_tail=4)
    hk, prompt, batch = 2, 130, 1
    tiles = (prompt + 63) // 64
    bands = torch.tensor([[INF, INF]] * 4, dtype=torch.int32)
    kp = torch.zeros(batch * hk * tiles * 2048, dtype=torch.uint32)
    packed = {F16: None, I8: torch.zeros(batch * hk * tiles * 2048, dtype=torch.uint32), I4: None}
    ka = torch.ones(batch * hk * tiles * 4)
    stat = torch.zeros(batch, hk, 3, 128)
    kx = torch.zeros(batch * hk * tiles * 16384, dtype=torch.uint8)
    codes, _ = cache.codes(tiles)
    cache.store(0, prompt, kp, ka, stat, stat.clone(), packed, codes, bands, None, None, [0, 1], kx, kx.clone())
    e = cache.layers[0]
    assert e["k8"].shape == (1, 2048) and not e["k8"].to(torch.int64).any()
    assert e["v"][I8].shape == (1, 2048) and e["v"][I4].shape == (1, 1024)
    assert e["xslot"].tolist() == [[0, tiles]]
    assert e["count"].tolist() == [[tiles, tiles]]


def test_ragged_store_keeps_each_groups_scales_and_statistics():
    """A Prefill hands the cache the same scale/statistics buffers for every call of one shape
    (two prompts of 150 and 190 tokens both have 3 tiles).  Each stored group must keep the values
    it was given, not whatever a later call wrote into the shared buffers."""
    cache = DecodeCache(FakeModule(), max_tail=8)
    cache.ragged = True
    hk, bands = 2, torch.tensor([[1, INF], [1, INF], [2, 4], [1, 1]], dtype=torch.int32)
    tiles, batch = 3, 1
    z32 = lambda n: torch.zeros(n, dtype=torch.int32).to(torch.uint32)
    ka, ka4 = torch.empty(batch * hk * tiles * 4), torch.empty(batch * hk * tiles * 4)
    kstat, vstat = torch.empty(batch * hk * 3 * 128), torch.empty(batch, hk, 3, 128)
    codes, _ = cache.codes(tiles)
    for prompt in (150, 190):
        for buf in (ka, ka4, kstat, vstat):
            buf.fill_(float(prompt))  # "statistics" of this prompt, written into the shared buffers
        packed = {F16: None, I8: z32(batch * hk * tiles * 2048), I4: z32(batch * hk * tiles * 1024)}
        cache.store(0, prompt, z32(batch * hk * tiles * 2048), ka, kstat, vstat, packed, codes, bands,
                    z32(batch * hk * tiles * 1024), ka4)
    e = cache.layers[0]
    for row, prompt in enumerate((150, 190)):
        for name in ("ka", "ka4", "kstat", "vstat"):
            assert bool((e[name][row] == float(prompt)).all()), (name, row)


def _decode_plan_tensors(b=2, hq=4, hk=2, maxn=3, tiles=3, max_tail=8, splits=2):
    i32 = lambda *s: torch.zeros(*s, dtype=torch.int32)
    f32 = lambda *s: torch.zeros(*s, dtype=torch.float32)
    bf = lambda *s: torch.zeros(*s, dtype=torch.bfloat16)
    u32 = lambda *s: torch.zeros(*s, dtype=torch.int32).to(torch.uint32)
    return dict(q=bf(b, hq, 1, 128), k8c=u32(4, 2048), k4c=u32(4, 1024), ka=f32(b * hk * tiles * 4),
                ka4=f32(b * hk * tiles * 4), entry=i32(b, hk, maxn), kinfo=i32(b, hk, maxn), count=i32(b, hk),
                fmt=i32(b, tiles), slot=i32(b, hk, maxn), v8=u32(4, 2048), v4=u32(4, 1024), vstat=f32(b, hk, 3, 128),
                kstat=f32(b, hk, 3, 128), ktail=bf(b, hk, max_tail, 128), vtail=bf(b, hk, max_tail, 128),
                kcur=bf(b, hk, 1, 128), vcur=bf(b, hk, 1, 128), step=torch.zeros(1, dtype=torch.int64),
                out=f32(b, hq, 1, 128), pm=f32(b * hq * splits), pl=f32(b * hq * splits),
                po=f32(b * hq * splits * 128), prompt=i32(b), per=2, scale=128 ** -0.5)


@pytest.mark.parametrize("bad, message", [
    (dict(out=torch.zeros(1, 4, 1, 128)), "out must be"),
    (dict(kcur=torch.zeros(2, 1, 1, 128, dtype=torch.bfloat16), vcur=torch.zeros(2, 1, 1, 128, dtype=torch.bfloat16)),
     "new token must be bf16"),
    (dict(kcur=torch.zeros(2, 2, 1, 128), vcur=torch.zeros(2, 2, 1, 128)), "new token must be bf16"),
    (dict(ktail=torch.zeros(2, 2, 4, 128, dtype=torch.bfloat16)), "tails must be"),
    (dict(vtail=torch.zeros(2, 2, 8, 128)), "tails must be"),
    (dict(vtail=torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16)[:, :, ::2]), "tails must be"),
    (dict(pl=torch.zeros(3)), "split partials"),
    (dict(po=torch.zeros(8)), "split partials"),
    (dict(fmt=torch.zeros(5, dtype=torch.int32)), "fmt"),
    (dict(prompt=torch.zeros(3, dtype=torch.int32)), "prompt length"),
    (dict(count=torch.zeros(2, 3, dtype=torch.int32)), "decode geometry/buffers"),
    (dict(step=torch.zeros(1, dtype=torch.int32)), "decode geometry/buffers"),
    ({}, "on q's device"),  # every shape right: the CPU tensors themselves are refused
])
def test_plan_decode_rejects_mismatched_buffers(bad, message):
    """The merge kernel writes out / ktail / vtail and reads kcur / vcur at sequence and head offsets
    derived from q's shape, so the plan refuses any of them that does not span that shape."""
    from triattention_amd.kernels.extension import Module, load_library
    args = _decode_plan_tensors()
    args.update(bad)
    with pytest.raises(RuntimeError, match=message):
        Module(load_library()).plan_decode(**args)
