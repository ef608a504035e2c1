"""Tail growth (extension) without a GPU: the oracle's restatement pinned against a longer prompt, and the
decode cache's bookkeeping (growth regions, room doubling, exact heads, ragged stores) driven through the
host restatement of tri_tail_spill.

The reference's tail holds max_tail generated tokens and then overwrites its last slot
(common_device.cuh:384); with growth, a full tail's oldest 64 tokens become a new tile of the cache,
quantized with the prompt's statistics and classified as the newest tile."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from cache_host import HostCacheModule, pack_kx
from triattention_amd import synthetic as S
from triattention_amd.kernels import records as R
from triattention_amd.kernels.decode import ENTRY_TILE, DecodeCache, growth_kinds, tile_states
from triattention_amd.kernels.prefill import F16, I4, I8
from triattention_amd.synthetic import INF


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _split_codes(codes, tiles):
    """The first ``tiles`` tiles of a prompt's codes, and its later tiles as tail_tile dicts."""
    cut = lambda a, lo, hi, per: None if a is None else np.ascontiguousarray(a[:, lo * per:hi * per])
    total = codes["k8"].shape[1] // 64
    head = dict(codes)
    for name, per in (("k8", 64), ("k4", 64), ("v8", 64), ("v4", 64), ("ka", 1), ("ka4", 1)):
        head[name] = cut(codes[name], 0, tiles, per)
    grown = [dict(k8=cut(codes["k8"], j, j + 1, 64), ka=cut(codes["ka"], j, j + 1, 1),
                  k4=cut(codes["k4"], j, j + 1, 64), ka4=cut(codes["ka4"], j, j + 1, 1),
                  v8=cut(codes["v8"], j, j + 1, 64)) for j in range(tiles, total)]
    return head, grown


@pytest.mark.parametrize("mutation", [None, "grown_mask", "grown_state"])
def test_grown_tiles_decode_as_a_longer_prompt(mutation):
    """With bands whose tile states do not depend on the distance from the end (every tile INT8; the
    sink INT8 and the rest INT4; the sink alone) and at most 16 tiles (every V INT8), a cache of prompt P
    (a multiple of 64) plus tiles taken from the tail equals the cache of the prompt P + 64 n, when both
    are quantized with the same statistics.  tail_tile of the later rows is those tiles' prefill codes.
    Planted mistakes (tail tiles masked like prompt tiles; classified against the prompt's tile count)
    break the equality."""
    hq, hk, p, n = 6, 3, 192, 2
    bands = np.array([[INF, INF], [INF, INF], [0, INF], [0, INF], [0, 0], [0, INF]], np.int32)
    g = S.gen(4401)
    q = S.outlier_tensor(g, 1, hq, 1)[0, :, 0]
    k, v = S.outlier_tensor(g, 1, hk, p + 64 * n)[0], S.outlier_tensor(g, 1, hk, p + 64 * n)[0]
    kt, vt = S.outlier_tensor(g, 1, hk, 24)[0], S.outlier_tensor(g, 1, hk, 24)[0]
    kc, vc = S.outlier_tensor(g, 1, hk, 1)[0, :, 0], S.outlier_tensor(g, 1, hk, 1)[0, :, 0]
    codes = O.prefill_codes(None, bits(k), bits(v), bands, decode_cache=True)
    assert codes["k4"] is not None and codes["v4"] is None
    head, grown = _split_codes(codes, p // 64)
    for j, t in enumerate(grown):
        rows = slice(p + 64 * j, p + 64 * (j + 1))
        mine = O.tail_tile(bits(k[:, rows]), bits(v[:, rows]), codes["kstat"], codes["vstat"])
        for name in ("k8", "ka", "k4", "ka4", "v8"):
            assert np.array_equal(mine[name], t[name]), name
    ktail = np.zeros((hk, 32, 128), np.uint16)
    vtail = np.zeros_like(ktail)
    ktail[:, :24], vtail[:, :24] = bits(kt), bits(vt)
    scale = 128 ** -0.5
    want = O.decode(codes, bands, bits(q), p + 64 * n, 1, scale, ktail, vtail, bits(kc), bits(vc), 24)
    try:
        if mutation:
            O.set_mutation(O.MUTATIONS[mutation])
        got = O.decode(head, bands, bits(q), p, 1, scale, ktail, vtail, bits(kc), bits(vc), 24, grown=grown)
    finally:
        O.set_mutation(0)
    if mutation is None:
        assert np.array_equal(got, want)
    else:
        assert not np.allclose(got, want, atol=1e-3)


def test_growth_kinds_are_the_newest_tile_states():
    """growth_kinds gives, per KV head, the group's maximum state and rowmask of the newest tile of a cache
    one tile longer than any prompt (tile_states at d = 0, j > 0); exact heads keep the tile whole."""
    bands = torch.tensor([[INF, INF], [1, INF], [0, INF], [0, 3], [0, 0], [0, 0], [2, 5], [0, 0]], dtype=torch.int32)
    kind, info = growth_kinds(bands, 4, exact_kv=[3])
    st = tile_states(bands, 9)[:, 8].view(4, 2)
    for h in range(3):
        kv = int(st[h].max())
        assert kind[h] == kv
        mask = sum(1 << r for r in range(2) if int(st[h, r]) > 0)
        assert info[h] == (-1 if kv == 0 else mask | ((kv == 4) << 8))
    assert kind[2] == 0 and info[2] == -1
    assert kind[3] == 1 and info[3] == 0b11


def _store(cache, prompt, batch, hk, bands, exact_kv, k, v):
    """One Prefill call's store with real codes of the given K/V (so that the statistics are real)."""
    tiles = (prompt + 63) // 64
    kp, k4, ka, ka4, v8, v4, kst, vst, kxs, vxs = ([] for _ in range(10))
    for s in range(batch):
        c = O.prefill_codes(None, bits(k[s, :, :prompt]), bits(v[s, :, :prompt]), bands.numpy(), decode_cache=True)
        kp.append(R.pack_k8(c["k8"].reshape(-1, 64, 128)).view(np.uint32))
        k4.append(R.pack_k4(c["k4"].reshape(-1, 64, 128)).view(np.uint32) if c["k4"] is not None else
                  np.zeros((hk * tiles, 1024), np.uint32))
        ka.append(c["ka"].reshape(-1))
        ka4.append(c["ka4"].reshape(-1) if c["ka4"] is not None else np.ones(hk * tiles * 4, np.float32))
        v8.append(R.pack_v8(c["v8"].reshape(-1, 64, 128)).view(np.uint32))
        v4.append(R.pack_v4(c["v4"].reshape(-1, 64, 128)).view(np.uint32) if c["v4"] is not None else
                  np.zeros((hk * tiles, 1024), np.uint32))
        kst.append(c["kstat"])
        vst.append(c["vstat"])
        for h in exact_kv:
            for j in range(tiles):
                kb = np.zeros((64, 128), np.uint16)
                vb = np.zeros((64, 128), np.uint16)
                n = min(64, prompt - 64 * j)
                kb[:n], vb[:n] = bits(k[s, h, 64 * j:64 * j + n]), bits(v[s, h, 64 * j:64 * j + n])
                a, b = pack_kx(kb, vb)
                kxs.append(a)
                vxs.append(b)
    cat = lambda xs, dt: torch.from_numpy(np.concatenate([np.asarray(x).reshape(-1) for x in xs]).astype(dt))
    u32 = lambda xs: torch.from_numpy(
        np.ascontiguousarray(np.concatenate([x.reshape(-1) for x in xs])).view(np.int32)).view(torch.uint32)
    packed = {F16: None, I8: u32(v8), I4: u32(v4)}
    codes, _ = cache.codes(tiles)
    kx = cat(kxs, np.uint8) if exact_kv else None
    vx = cat(vxs, np.uint8) if exact_kv else None
    cache.store(0, prompt, u32(kp), cat(ka, np.float32), torch.from_numpy(np.stack(kst)),
                torch.from_numpy(np.stack(vst)), packed, codes, bands, u32(k4), cat(ka4, np.float32), exact_kv,
                kx, vx)


def _step(cache, kd, vd):
    """One decode step's tail bookkeeping on the host: the growth check and spill, then the merge's tail
    append of the new k / v at slot min(max_tail - 1, step - tail_base), then the step advance."""
    e = cache._grow_step(0)
    cache._spill_plan(e).run()
    a = e["store"].arrays
    held = int(cache.step[0]) - int(a["tail_base"][0])
    slot = min(cache.max_tail - 1, held)
    e["tail_k"][:, :, slot] = kd
    e["tail_v"][:, :, slot] = vd
    cache.advance()
    assert cache.host_step == int(cache.step[0]) and e["store"].tb == int(a["tail_base"][0])


@pytest.mark.parametrize("exact_kv", [(), (2,)])
def test_cache_growth_bookkeeping_against_the_oracle(exact_kv):
    """Ragged stores, room for one tile (grow_tail 64) that doubles twice, INT8 / INT4 / dropped / exact
    KV heads: after 64 * 6 + 100 steps with max_tail 64, every (sequence, KV head) lists its prompt
    entries and then one entry per tile taken from the tail (tiles ceil(prompt / 64) + i, INT8 V), whose
    K / V records and scales are the oracle's tail_tile of generated tokens 64 i .. 64 i + 63, and the
    tail holds the tokens after them; exact heads hold the tiles as KX / VX records."""
    hq, hk, max_tail = 8, 4, 64
    bands = torch.tensor([[INF, INF], [1, 1], [0, INF], [0, 3], [0, 0], [0, 0], [2, 5], [1, INF]],
                         dtype=torch.int32)
    cache = DecodeCache(HostCacheModule(), max_tail=max_tail, grow_tail=64)
    cache.ragged = True
    g = S.gen(4500 + len(exact_kv))
    prompts = [(130, 2), (64, 1)]
    kv = []
    for prompt, batch in prompts:
        k, v = S.outlier_tensor(g, batch, hk, prompt), S.outlier_tensor(g, batch, hk, prompt)
        _store(cache, prompt, batch, hk, bands, exact_kv, k, v)
        kv.append((k, v))
    kinds, infos = growth_kinds(bands, hk, exact_kv)
    steps = 64 * 6 + 100
    rows = sum(b for _, b in prompts)
    gen_k = S.outlier_tensor(g, rows, hk, steps)
    gen_v = S.outlier_tensor(g, rows, hk, steps)
    for t in range(steps):
        _step(cache, gen_k[:, :, t], gen_v[:, :, t])
    e = cache.layers[0]
    st = e["store"]
    spilled = st.tb // 64
    assert spilled == (steps - 1 - max_tail) // 64 + 1 == 7 and st.grow_tiles == 8
    held = steps - 64 * spilled
    assert torch.equal(e["tail_k"][:, :, :held], gen_k[:, :, 64 * spilled:])
    row = 0
    for (prompt, batch), (k, v) in zip(prompts, kv):
        tiles = (prompt + 63) // 64
        for s in range(batch):
            for h in range(hk):
                c = O.prefill_codes(None, bits(k[s, h:h + 1]), bits(v[s, h:h + 1]), bands.numpy()[2 * h:2 * h + 2],
                                    decode_cache=True)
                c0 = int(e["store"].arrays["count0"][row, h])
                n_want = c0 + (spilled if kinds[h] else 0)
                assert int(e["count"][row, h]) == n_want
                for i in range(spilled if kinds[h] else 0):
                    j = tiles + i
                    word = int(e["entry"][row, h, c0 + i])
                    assert word & ENTRY_TILE == j
                    rk, rv = bits(gen_k[row, h, 64 * i:64 * (i + 1)]), bits(gen_v[row, h, 64 * i:64 * (i + 1)])
                    if kinds[h] == 1:
                        x0 = int(e["xslot"][row, h])
                        kx, vx = pack_kx(rk, rv)
                        assert np.array_equal(e["kx"][(x0 + j) * 16384:(x0 + j + 1) * 16384].numpy(), kx)
                        assert np.array_equal(e["vx"][(x0 + j) * 16384:(x0 + j + 1) * 16384].numpy(), vx)
                        continue
                    t = O.tail_tile(rk[None], rv[None], c["kstat"], c["vstat"])
                    info = int(e["kinfo"][row, h, c0 + i])
                    assert info & 0x1FF == infos[h]
                    if (info >> 8) & 1:
                        rec = e["k4"][info >> 9].numpy().view(np.uint8)
                        assert np.array_equal(R.unpack_k4(rec)[0], t["k4"][0])
                        assert np.array_equal(e["ka4"][row, h, j].numpy(), t["ka4"][0, 0])
                    else:
                        rec = e["k8"][info >> 9].numpy().view(np.uint8)
                        assert np.array_equal(R.unpack_k8(rec)[0], t["k8"][0])
                        assert np.array_equal(e["ka"][row, h, j].numpy(), t["ka"][0, 0])
                    vrec = e["v"][I8][int(e["slot"][row, h, c0 + i])].numpy().view(np.uint8)
                    assert np.array_equal(R.unpack_v8(vrec)[0], t["v8"][0])
                    assert int(e["fmt"][row, j]) == 1
            row += 1
    # the partition holds the growth splits after each head's prompt entries, 64 entries each
    b = e["bounds_host"]
    assert e["grow_splits"] == 1 and np.array_equal(b[:, :, -1] - b[:, :, -2], np.full(b.shape[:2], 8))


def test_growing_tail_oracle_moves_64_tokens_when_full():
    """GrowingTail: a step that finds max_tail tokens in the tail first takes the oldest 64 into a tile;
    the tail then holds the later tokens in order, and the step attends over all of them."""
    hq, hk, max_tail, prompt = 4, 2, 64, 70
    bands = np.array([[INF, INF], [0, INF], [1, 1], [0, 0]], np.int32)
    g = S.gen(4600)
    k, v = S.outlier_tensor(g, 1, hk, prompt)[0], S.outlier_tensor(g, 1, hk, prompt)[0]
    codes = O.prefill_codes(None, bits(k), bits(v), bands, decode_cache=True)
    seq = O.GrowingTail(codes, bands, prompt, max_tail)
    gk, gv = S.outlier_tensor(g, 1, hk, 200)[0], S.outlier_tensor(g, 1, hk, 200)[0]
    q = S.outlier_tensor(g, 1, hq, 1)[0, :, 0]
    for t in range(200):
        seq.step(bits(q), bits(gk[:, t]), bits(gv[:, t]), 1, 128 ** -0.5)
        n = 0 if t < max_tail else (t - max_tail) // 64 + 1
        assert len(seq.grown) == n and seq.held == t + 1 - 64 * n
        assert np.array_equal(seq.ktail[:, :seq.held], bits(gk[:, 64 * n:t + 1]))
