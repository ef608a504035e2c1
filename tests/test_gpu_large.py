"""Record arrays beyond 2 GiB: the decode kernels address every record through its own 64-bit base, so a
cache whose records sit past byte 2^31 of their arrays decodes exactly as the same cache at the start of
small arrays (bit-equal outputs; the gather path, the task table, and exact heads)."""
from __future__ import annotations

import pytest
import torch

from helpers import run_prefill
from test_gpu_parity import small
from triattention_amd.kernels.decode import DecodeCache
from triattention_amd.kernels.prefill import I4, I8
from triattention_amd.synthetic import INF

pytestmark = pytest.mark.gpu

BANDS = [[INF, INF], [1, 1], [0, INF], [0, 3], [2, 5], [1, INF]]


def _far(small_arr, slots, dev):
    """The records of ``small_arr`` at slots ``slots`` .. of an array that holds slots + n records."""
    n, words = small_arr.shape
    big = torch.zeros((slots + n, words), dtype=torch.int32, device=dev)
    big[slots:] = small_arr.view(torch.int32)
    return big.view(torch.uint32)


@pytest.mark.parametrize("bf16_kv,tasks", [([], True), ([], False), ([1], False)])
def test_records_past_2_gib_decode_bit_equal(module, bf16_kv, tasks):
    hq, hk, prompt, batch = 6, 3, 700, 2
    print(f"\n[large] records past 2 GiB, exact {bf16_kv}, task table {tasks}", flush=True)
    q, k, v = small(9950, batch, hq, hk, prompt)
    bands = torch.tensor(BANDS, dtype=torch.int32)
    cache = DecodeCache(module, max_tail=64)
    cache.out_dtype = torch.float32
    cache.tasks = tasks
    run_prefill(module, q, k, v, bands, 128 ** -0.5, decode_cache=cache, bf16_kv=bf16_kv)
    e = cache.layers[0]
    dev = torch.device("cuda")
    # slot offsets that put every record past byte 2^31 (K8 / V8 8 KiB, K4 / V4 4 KiB, KX / VX 16 KiB)
    o8, o4 = (1 << 31) // 8192 + 7, (1 << 31) // 4096 + 5
    k8 = _far(e["k8"], o8, dev)
    v8 = _far(e["v"][I8], o8, dev)
    v4 = _far(e["v"][I4], o4, dev)
    k4 = _far(e["k4"], o4, dev) if e["k4"] is not None else None
    assert k8.numel() * 4 > (1 << 31) and v4.numel() * 4 > (1 << 31)
    kinfo, slot = e["kinfo"].clone(), e["slot"].clone()
    is4 = ((kinfo >> 8) & 1).bool()
    kinfo = kinfo + torch.where(is4, o4, o8).to(torch.int32) * 512
    fmt = e["fmt"]
    tiles = e["entry"] & ((1 << 29) - 1)
    vfmt = torch.gather(fmt[:, None, :].expand(-1, hk, -1), 2, tiles.long().clamp(max=fmt.shape[1] - 1))
    valid = torch.arange(e["entry"].shape[2], device=dev)[None, None, :] < e["count"][:, :, None]
    slot = torch.where(valid, slot + torch.where(vfmt == 1, o8, o4).to(torch.int32), slot)
    kinfo = torch.where(valid, kinfo, e["kinfo"])
    kx = vx = xslot = None
    if e["xslot"] is not None:
        ox = (1 << 31) // 16384 + 3
        kx = torch.zeros(ox * 16384 + e["kx"].numel(), dtype=torch.uint8, device=dev)
        vx = torch.zeros_like(kx)
        kx[ox * 16384:], vx[ox * 16384:] = e["kx"], e["vx"]
        xslot = torch.where(e["xslot"] >= 0, e["xslot"] + ox, e["xslot"])
    g = torch.Generator().manual_seed(9951)
    qd = torch.randn(batch, hq, 1, 128, generator=g).to(torch.bfloat16).to(dev)
    kd = torch.randn(batch, hk, 1, 128, generator=g).to(torch.bfloat16).to(dev)
    vd = torch.randn(batch, hk, 1, 128, generator=g).to(torch.bfloat16).to(dev)
    outs = []
    for far in (False, True):
        splits = e["splits"]
        n = batch * hq * splits
        pm, pl, po = (torch.full((n,), -3.4028234663852886e38, device=dev), torch.zeros(n, device=dev),
                      torch.zeros(n * 128, device=dev))
        tk, tv = e["tail_k"].clone(), e["tail_v"].clone()
        step = torch.zeros(1, dtype=torch.int64, device=dev)
        args = (k8, k4, e["ka"], e["ka4"], e["entry"], kinfo, e["count"], fmt, slot, v8, v4) if far else \
            (e["k8"], e["k4"], e["ka"], e["ka4"], e["entry"], e["kinfo"], e["count"], fmt, e["slot"], e["v"][I8],
             e["v"][I4])
        table = None
        if tasks and e["xslot"] is None:
            items = torch.from_numpy(DecodeCache._task_items(e)).to(dev)
            table = module.decode_tasks(args[2], args[3], args[4], args[5], args[6], args[7], args[8], e["per"],
                                        e["bounds"], items)
        out = torch.empty((batch, hq, 1, 128), dtype=torch.float32, device=dev)
        plan = module.plan_decode(qd, *args, e["vstat"], e["kstat"], tk, tv, kd, vd, step, out, pm, pl, po,
                                  e["prompt"], e["per"], 128 ** -0.5, xslot if far else e["xslot"],
                                  kx if far else e["kx"], vx if far else e["vx"], e["bounds"], table)
        plan.run(qd, kd, vd, out)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
