"""Benchmark of the quantized attention path on one MI355X.

Headline ("C1"): one decode op of 32 sequences,
Llama-3.2-3B attention shape (24 q-heads / 8 KV heads, head_dim 128), prompt
4096 held in the quantized cache, 25% INT8 / 75% INT4 KV heads, one new bf16
token per sequence.  ``value`` = algorithmic HBM bytes of the step / step time
(GB/s); the step is the split-KV decode kernel plus the merge kernel, inputs
resident in HBM; one token runs the decode op of each of the 28 layers of
Llama-3.2-3B, every layer with its own cache, so the records stream from HBM
rather than from the 256 MB Infinity Cache.  Also
reported: model tokens/s (batch over one token of all 28 layers' decode ops;
the per-op rate is named layer_op_tokens_per_s), the decode kernel's roofline
(HIP events that the kernel's own launch records, inside the timed region), the CPU oracle timed
on a bounded sample, prefill attention TOPS on configs[0] and configs[2] (C0, C2),
and the ragged decode of configs[3] (C3).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill] [--no-c3]
       python bench.py --c4   (configs[4]: end-to-end greedy generation, one JSON line of its own)
       python bench.py --calibrate   (the calibration sweep's Prefill executors sharing scratch)
       python bench.py --copy-probe   (a plain 256 MiB device copy, five times: the
       known-size kernel that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)

``roofline.traffic`` is the decode kernel's HBM bytes per launch measured with
those counters; it is read from profiles/decode_kernel_C1_traffic.md, which
holds the commands, the raw counter values and the hash of the kernel sources
they were taken on (null, with a note, when that file is absent or the hash
differs from the sources here).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
K8, K4, V8, V4 = 8192, 4096, 8192, 4096


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may use (OMP_NUM_THREADS caps it where
    the host shares its cores)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap)) if cap and cap.isdigit() else n)


def decode_record_bytes(cache_entry):
    """Algorithmic record bytes of one decode step: for every kept (sequence, KV head, tile),
    its K record (8 or 4 KiB), its V record (8 or 4 KiB) and 16 B of group scales."""
    import torch
    e = cache_entry
    kinfo = e["kinfo"].cpu().to(torch.int64)
    count = e["count"].cpu().to(torch.int64)
    entry = e["entry"].cpu().to(torch.int64) & ((1 << 29) - 1)  # the tile index (bits 0-28)
    fmt = e["fmt"].cpu().to(torch.int64)
    b, hk, maxn = kinfo.shape
    valid = torch.arange(maxn)[None, None, :] < count[:, :, None]
    is4 = ((kinfo >> 8) & 1).bool()
    kbytes = torch.where(is4, K4, K8)
    vf = torch.gather(fmt[:, None, :].expand(b, hk, fmt.shape[1]), 2, entry)
    vbytes = torch.where(vf == 1, V8, V4)
    return int(((kbytes + vbytes + 16) * valid).sum()), int(valid.sum())


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_kernel_C1_traffic.md"
COPY_PROBE_BYTES = 256 << 20
# Ministral-8B, whose shape configs[3] names, has 36 decoder layers
C3_LAYERS = 36
# layers (each with a cache of its own, ~490 MB) in the C3 token replayed as a HIP graph
C3_GRAPH_LAYERS = 4
# record bytes (K/V records and K group scales) one C1 decode launch reads: 16,384 kept tiles
C1_RECORD_BYTES = 170_655_744


# the sources the split-KV decode kernel is compiled from: a counter summary taken on other sources
# no longer describes the kernel that runs
TRAFFIC_SOURCES = (ROOT / "triattention_amd" / "csrc" / "decode.hip", ROOT / "triattention_amd" / "csrc" / "common.h")


def source_hash(files):
    """First 16 hex digits of the SHA-256 of ``files``' bytes, in order."""
    import hashlib
    h = hashlib.sha256()
    for f in files:
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def decode_source_hash():
    """The decode kernel's sources (decode.hip, then common.h), hashed as ``source_hash``."""
    return source_hash(TRAFFIC_SOURCES)


# the prefill kernel's sources, and the counter summary whose per-tile figures the C2 line carries
PREFILL_SOURCES = (ROOT / "triattention_amd" / "csrc" / "prefill.hip", ROOT / "triattention_amd" / "csrc" / "common.h")
PREFILL_PROFILE = ROOT / "profiles" / "prefill_counters_C2.md"
PREFILL_FIELDS = ("simd_cycles_per_tile_wave", "valu_per_tile_wave", "mfma_per_tile_wave",
                  "transcendental_per_tile_wave", "mfma_busy_fraction", "mfma_coexec_fraction")


def prefill_source_hash():
    """The prefill kernel's sources (prefill.hip, then common.h), hashed as ``source_hash``."""
    return source_hash(PREFILL_SOURCES)


def profile_fields(path, keys):
    """``key: value`` lines of a committed summary, for the listed keys."""
    fields = {}
    if path.exists():
        for line in path.read_text().splitlines():
            if ":" in line and line.split(":", 1)[0] in keys:
                key, val = line.split(":", 1)
                fields[key] = val.strip()
    return fields


def prefill_counters():
    """(per-tile counter figures of the C2 mix, note) from the committed counter summary, or None when it
    was taken on other prefill sources than the ones built here."""
    fields = profile_fields(PREFILL_PROFILE, PREFILL_FIELDS + ("kernel_source_sha16",))
    here = prefill_source_hash()
    if fields.get("kernel_source_sha16") != here:
        return None, (f"counter summary taken on prefill kernel sources {fields.get('kernel_source_sha16')}, "
                      f"these are {here}: not reported")
    return ({k: float(fields[k]) for k in PREFILL_FIELDS if k in fields},
            f"rocprofv3 counters of the C2 mix per 64-key tile of one wave, {PREFILL_PROFILE.name} "
            f"(kernel sources {here})")


def measured_traffic():
    """(HBM bytes per decode_kernel launch, note) from the committed counter summary.  The bytes are
    None when the summary is missing or was taken on other kernel sources than the ones built here
    (its kernel_source_sha16 line against decode_source_hash()), so a stale counter is never
    reported as current."""
    if not TRAFFIC_PROFILE.exists():
        return None, "no counter summary"
    fields = {}
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if ":" in line and line.split(":", 1)[0] in ("traffic_bytes_per_launch", "kernel_source_sha16"):
            key, val = line.split(":", 1)
            fields[key] = val.strip()
    here = decode_source_hash()
    if fields.get("kernel_source_sha16") != here:
        return None, (f"counter summary taken on decode kernel sources {fields.get('kernel_source_sha16')}, "
                      f"these are {here}: not reported")
    if "traffic_bytes_per_launch" not in fields:
        return None, "no traffic line in the counter summary"
    return int(fields["traffic_bytes_per_launch"]), (f"FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated, "
                                                     f"{TRAFFIC_PROFILE.name} (kernel sources {here})")


MERGE_FORM = "auto"  # --merge-form: "device" launches tri_decode's merge, which picks its form itself


def short_merge(cache, layer, hq):
    """Whether the decode op of ``layer`` launches the one-wave merge kernel (the cache's choice by tail
    length and grid size), rather than tri_decode's merge, which picks the same form on the device
    (--merge-form device: the launch a graph captured by the model path replays)."""
    return MERGE_FORM == "auto" and cache.short_tail(layer, hq)


def kernel_events(n, stream):
    """n (start, stop) HIP event pairs for the split-KV kernel: the launch records them as the kernel's
    own start and stop (hipExtLaunchKernel through tri_decode_partials_timed), so the timed loop holds
    no event commands of its own.  Each event is recorded once here so that it exists."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for pair in evs:
        for e in pair:
            e.record(stream)
    torch.cuda.synchronize()
    return evs


def copy_probe():
    import torch
    n = COPY_PROBE_BYTES // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"copy probe: 5 x torch.neg over {COPY_PROBE_BYTES} B in, {COPY_PROBE_BYTES} B out", flush=True)


# launch shapes of the streaming-read probe (waves, waves per workgroup, records in flight per wave)
STREAM_SHAPES = ((1024, 1, 1), (1024, 1, 2), (1024, 1, 3), (2048, 1, 2), (2048, 2, 2), (4096, 4, 1), (4096, 4, 2),
                 (8192, 4, 2))
STREAM_SHAPES_DEFAULT = ((1024, 1, 3), (2048, 2, 2), (4096, 4, 2), (8192, 4, 2))
# more waves, for launches of many more bytes (used where every wave gets at least two records per slot)
STREAM_SHAPES_LARGE = ((16384, 4, 2), (32768, 4, 2))


def stream_ceiling(module, dev, nbytes, layers, shapes, reps=5, verbose=False):
    """The device's streaming-read ceiling for a launch that reads ``nbytes``: tri_stream_read (no
    compute, 16-byte loads per lane, contiguous 8 KiB records per wave) over ``layers`` buffers of
    that size in turn, so that, as in the decode bench, each launch reads from HBM rather than the
    256 MB Infinity Cache.  Returns the best (us per launch, GB/s, shape) over ``shapes``."""
    import torch
    records = nbytes // 8192
    bufs = [torch.empty(records * 8192, dtype=torch.uint8, device=dev) for _ in range(layers)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    best = None
    for shape in shapes:
        for b in bufs:
            module.stream_read(b, *shape, sink)
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for b in bufs:
                module.stream_read(b, *shape, sink)
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / layers)
        us = min(times)
        gbs = records * 8192 / (us * 1e-6) / 1e9
        if verbose:
            print(f"stream read: {shape[0]:5d} waves, {shape[1]} per workgroup, {shape[2]} in flight: "
                  f"{us:7.2f} us per launch, {gbs:7.1f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak)", flush=True)
        if best is None or us < best[0]:
            best = (us, gbs, shape)
    del bufs
    return best


def read_ceiling(args):
    """--read-ceiling: the streaming-read probe over every shape, at the C1 decode launch's bytes, or
    at each byte count of --ceiling-bytes (the buffers rotate over at least 4.8 GB, so every launch
    reads HBM rather than the 256 MB Infinity Cache)."""
    import torch
    from triattention_amd.kernels.extension import load_extension
    module = load_extension()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    mat = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 1.5:
        mat = (mat @ mat).clamp_(-1.0, 1.0)
        torch.cuda.synchronize()
    del mat
    sizes = [int(x) for x in args.ceiling_bytes.split(",")] if args.ceiling_bytes else [C1_RECORD_BYTES]
    for nbytes in sizes:
        buffers = args.layers if nbytes == C1_RECORD_BYTES else max(2, -(-4_800_000_000 // nbytes))
        shapes = STREAM_SHAPES + tuple(s for s in STREAM_SHAPES_LARGE if nbytes >= s[0] * 2 * 8192 * s[2])
        print(f"== {nbytes} B per launch, {buffers} buffers", flush=True)
        us, gbs, shape = stream_ceiling(module, dev, nbytes, buffers, shapes, verbose=True)
        print(json.dumps({"stream_ceiling": {"bytes": nbytes, "buffers": buffers, "us": round(us, 2),
                                             "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                                             "shape": list(shape)}}), flush=True)


ISSUE_MODES = {0: ("32 v_fma_f32", 32), 1: ("8 v_exp_f32", 8), 2: ("24 v_fma_f32 + 8 v_exp_f32", 32),
               3: ("4 v_mfma_i32_32x32x32_i8", 4), 4: ("4 v_mfma_f32_32x32x16_bf16", 4),
               5: ("4 i8 MFMA + 64 v_fma_f32, one wave", 68),
               6: ("first wave of a SIMD 4 i8 MFMA, the others 32 v_fma_f32", None),
               7: ("4 i8 MFMA + 96 v_fma_f32, spread", 100), 8: ("4 i8 MFMA + 96 v_fma_f32, MFMAs first", 100),
               9: ("as 8, then a barrier", 100), 10: ("as 9, fma after the MFMA results", 100),
               11: ("as 10, odd waves half an iteration behind", 100), 12: ("as 7, then a barrier", 100),
               13: ("tile-shaped: 16 MFMA + 128 fma, then 200 fma + 32 exp, every wave in step", 376),
               14: ("as 13, odd waves of a SIMD in the other half", 376)}


def issue_probe(args):
    """--issue-probe: SIMD cycles per instruction of the attention tiles' instruction kinds at 1-4 waves
    per SIMD (tri_issue_probe; shader-clock cycles from s_memtime).  A SIMD's time is its slowest wave's,
    its work every instruction its waves issued; the median over the device's SIMDs is reported."""
    import torch
    from triattention_amd.kernels.extension import load_extension
    module = load_extension()
    torch.cuda.set_device(0)
    iters = 4096
    rows = []
    wanted = {int(m) for m in args.issue_modes.split(",")} if args.issue_modes else set(ISSUE_MODES)
    for mode, (what, per_iter) in ISSUE_MODES.items():
        if mode not in wanted:
            continue
        for w in range(1, 5):
            if mode == 6 and w < 2:
                continue
            module.issue_probe(mode, w, 64)  # (warm-up launch)
            r = module.issue_probe(mode, w, iters)
            cyc, ticks = r[:, 0].double(), r[:, 1].double()
            ghz = float(statistics.median((cyc / ticks * 0.1).tolist()))
            per_wg = 4 * w
            wg = cyc.view(-1, per_wg)  # [CUs, waves of the workgroup]; wave i on SIMD i % 4
            simd_time = wg.view(-1, w, 4).amax(dim=1)  # [CUs, 4]
            if mode == 6:
                mfma_rate = iters * 4 / simd_time  # MFMAs per cycle: one MFMA wave per SIMD
                valu_rate = iters * 32 * (w - 1) / simd_time
                row = {"mode": mode, "what": what, "waves_per_simd": w, "clock_ghz": round(ghz, 3),
                       "mfma_cycles_each": round(float(1 / mfma_rate.median()), 2),
                       "fma_cycles_each": round(float(1 / valu_rate.median()), 2)}
            else:
                cpi = simd_time / (iters * per_iter * w)
                row = {"mode": mode, "what": what, "waves_per_simd": w, "clock_ghz": round(ghz, 3),
                       "simd_cycles_per_instruction": round(float(cpi.median()), 2)}
            rows.append(row)
            print(json.dumps(row), flush=True)
    print(json.dumps({"issue_probe": rows}), flush=True)


def graph_steps(run_token, tokens, stream):
    """ms per token of ``run_token`` (one token's launches: every layer's decode op and the step
    advance) captured once as a HIP graph and replayed ``tokens`` times, as the model path replays
    its one-token forward: no host time between the kernels."""
    import torch
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run_token()
    for _ in range(3):
        graph.replay()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    g0.record(stream)
    for _ in range(tokens):
        graph.replay()
    g1.record(stream)
    torch.cuda.synchronize()
    return g0.elapsed_time(g1) / tokens


def c3_decode(module, dev, stream, args, S, DecodeCache, Prefill, from_bands):
    """one ragged decode step of 64 sequences (Hq 32 / Hk 8) whose prompts of
    log-uniform length in [512, 32768] sit in one quantized cache.  The prompts' K/V are drawn
    on the device and stored with Prefill.store_only (quantize + pack, no prompt attention);
    C3_GRAPH_LAYERS layers each hold a cache of their own with the same prompts.  The timed region is
    their decode ops (split-KV kernel + merge) in turn, the step advancing once per token, launched
    from Python as a serving loop would (the split kernel timed by its launch's events); beside it the
    same token replayed as a HIP graph (the graph's launch cost spread over its layers, as in the
    model)."""
    import torch
    lengths = S.config3_lengths()
    kinds, bands = S.config3_map()
    hq, hk = 32, 8
    log(f"C3: storing {len(lengths)} ragged prompts ({sum(lengths)} tokens)")
    gdev = torch.Generator(device=dev).manual_seed(1003)
    kvs = []
    for n in lengths:
        k = S.outlier_tensor_device(gdev, 1, hk, n)
        kvs.append((k, S.outlier_tensor_device(gdev, 1, hk, n)))
    # the cache build: one store_only per prompt (quantize K, pack V, and the device-side store that
    # classifies the tiles and appends the records), timed twice, the second on a warm allocator
    for rep in range(2):
        cache = DecodeCache(module, max_tail=256)
        cache.ragged = True
        if args.c3_per:
            cache.per = args.c3_per  # (measurement aid: runs of this many tiles instead of the default)
        pre = Prefill(module, from_bands({str(layer): bands.tolist() for layer in range(C3_GRAPH_LAYERS)}), cache)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        b0.record(stream)
        for k, v in kvs:
            pre.store_only(0, k, v, hq)
        b1.record(stream)
        torch.cuda.synchronize()
        build_wall_ms = (time.perf_counter() - t0) * 1e3
        build_gpu_ms = b0.elapsed_time(b1)
    for layer in range(1, C3_GRAPH_LAYERS):  # the graph token's other layers (untimed)
        for k, v in kvs:
            pre.store_only(layer, k, v, hq)
    torch.cuda.synchronize()
    del pre, kvs
    log(f"C3 cache build: {build_wall_ms:.1f} ms wall, {build_gpu_ms:.1f} ms on the GPU")
    e = cache.layers[0]
    rec_bytes, kept = decode_record_bytes(e)
    batch = len(lengths)
    steps, warmup = max(5, args.steps // 2), max(2, args.warmup // 2)
    toks = [(S.outlier_tensor_device(gdev, batch, hq, 1), S.outlier_tensor_device(gdev, batch, hk, 1),
             S.outlier_tensor_device(gdev, batch, hk, 1)) for _ in range(steps + warmup)]
    log(f"C3 cache: {kept} kept tiles, {rec_bytes} record bytes/step, per={e['per']}, maxn={e['maxn']}")
    for i in range(warmup):
        for layer in range(C3_GRAPH_LAYERS):
            cache(layer, *toks[i], 128 ** -0.5)
        cache.advance()
    out = torch.empty((batch, hq, 1, 128), dtype=torch.bfloat16, device=dev)
    plans = [cache.plan(layer, toks[0][0], toks[0][1], out, 128 ** -0.5) for layer in range(C3_GRAPH_LAYERS)]
    # step i is layer i % C3_GRAPH_LAYERS's decode op, the step advancing after the last layer: the
    # layers' caches (~2 GB together) exceed the 256 MB Infinity Cache, so every op reads HBM
    evs = kernel_events(steps, stream)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        qd, kd, vd = toks[warmup + i]
        layer = i % C3_GRAPH_LAYERS
        plans[layer].run(qd, kd, vd, out, 1, events=evs[i])
        plans[layer].run(qd, kd, vd, out, 2, short_tail=short_merge(cache, layer, hq))
        if layer == C3_GRAPH_LAYERS - 1:
            cache.advance()
    end.record(stream)
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / steps
    dec_ms = statistics.fmean(ev[0].elapsed_time(ev[1]) for ev in evs)

    def token():
        qd, kd, vd = toks[warmup]
        for layer in range(C3_GRAPH_LAYERS):
            plans[layer].run(qd, kd, vd, out, short_tail=short_merge(cache, layer, hq))
        cache.advance()
    graph_ms = graph_steps(token, steps, stream) / C3_GRAPH_LAYERS
    ms = eager_ms
    log(f"C3 decode step {ms * 1e3:.1f} us eager, {graph_ms * 1e3:.1f} us per layer from a {C3_GRAPH_LAYERS}-layer "
        f"HIP graph (split-KV kernel {dec_ms * 1e3:.1f} us)")
    return {"workload": "C3 ragged decode: batch 64, Hq 32 / Hk 8, prompts log-uniform in [512, 32768] "
                        f"(total {sum(lengths)} tokens), KV heads {kinds}",
            "data": "synthetic, drawn on the device (seeded torch.Generator on cuda)",
            "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 5),
            "graph_ms_per_step": round(graph_ms, 5),
            "step_launch": f"per decode op of a {C3_GRAPH_LAYERS}-layer token (each layer its own cache of the "
                           "same prompts, ~2 GB together): eager (the split-KV kernel, the merge and the step "
                           "advance launched from Python); graph_ms_per_step: the token replayed as a HIP graph",
            "record_bytes_per_step": rec_bytes, "kept_tiles": kept,
            "decode_kv_gbs": round(rec_bytes / (ms * 1e-3) / 1e9, 2),
            "cache_build_ms": {"wall": round(build_wall_ms, 2), "gpu": round(build_gpu_ms, 2),
                               "what": "64 Prefill.store_only calls: quantize, pack and the device-side store"},
            "split_kernel_us": round(dec_ms * 1e3, 2),
            "split_kernel_gbs": round(rec_bytes / (dec_ms * 1e-3) / 1e9, 2),
            "frac_hbm_peak": round(rec_bytes / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "layer_op_tokens_per_s": round(batch / (ms * 1e-3), 1),
            "model_tokens_per_s": {"value": round(batch / (C3_LAYERS * graph_ms * 1e-3), 1), "layers": C3_LAYERS,
                                   "what": f"batch / ({C3_LAYERS} x the replayed step per layer): the attention "
                                           "part of a Ministral-8B decode step, every layer taken as costly as "
                                           f"the {C3_GRAPH_LAYERS} measured (extrapolated)"}}


def c4_config():
    """C4 model, prompt and map: random-init Qwen2-7B shape, 4096 random
    prompt ids, a seeded per-(layer, KV head) draw over INT8 / INT4 / bf16."""
    import transformers

    from triattention_amd import synthetic as S
    from triattention_amd.maps import from_bands

    kw, ids, bands, bf16, kinds = S.config4()
    cfg = transformers.Qwen2Config(**kw)
    mixed = from_bands(bands, bf16=bf16)
    exact = from_bands(bands, bf16={str(l): [0, 1, 2, 3] for l in range(28)})
    share = {name: float((kinds == i).float().mean()) for i, name in enumerate(("int8", "int4", "bf16"))}
    return cfg, ids, mixed, exact, share


def c4_runs(which=("mixed", "mixed_eager", "all_bf16"), reps=2):
    """C4: greedy generation of 256 tokens after a 4096-token prompt through TriAttention on the model
    of configs[4], per run: "mixed" (the map, the one-token forward replayed as a HIP graph),
    "mixed_eager" (the same without the graph), "all_bf16" (every KV head exact, graph).  The last of
    ``reps`` repetitions is reported (the first also builds the per-layer plans and buffers)."""
    import torch
    import transformers

    from triattention_amd.models import TriAttention, _GraphStep

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg, ids, mixed, exact, share = c4_config()
    log("C4: random-init Qwen2-7B (bf16, N(0, 0.02)) on the GPU")
    torch.manual_seed(1004)
    with torch.device(dev):
        model = transformers.Qwen2ForCausalLM(cfg).to(torch.bfloat16).eval()
    ids = ids.to(dev)
    new = 256
    runs = {}
    maps = {"mixed": (mixed, True), "mixed_eager": (mixed, False), "all_bf16": (exact, True)}
    for name in which:
        fn, graph = maps[name]
        tri = TriAttention(model, fn, max_new_tokens=new)
        for rep in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with torch.inference_mode():
                out = model(input_ids=ids, use_cache=False, logits_to_keep=1)
                torch.cuda.synchronize()
            t1 = time.perf_counter()
            # TriAttention.generate's loop after the prompt (the prompt forward is timed above)
            with torch.inference_mode():
                tokens, step = [], None
                for i in range(new):
                    tokens.append(int(out.logits[0, -1].argmax()))
                    if i == new - 1:
                        break
                    if step is not None and tri.decode_cache.graph_ready():
                        step.ids.fill_(tokens[-1])
                        step.position.fill_(ids.shape[1] + i)
                        out = step.replay()
                        tri.decode_cache.replayed()
                        continue
                    position = torch.tensor([[ids.shape[1] + i]], device=dev)
                    out = model(input_ids=torch.tensor([[tokens[-1]]], device=dev), position_ids=position,
                                use_cache=False)
                    tri.decode_cache.advance()
                    if graph:
                        step = _GraphStep(model, tri.decode_cache, dev)
            t2 = time.perf_counter()
        runs[name] = {"prefill_ms": round((t1 - t0) * 1e3, 2), "decode_s": round(t2 - t1, 4),
                      "decode_tokens_per_s": round((new - 1) / (t2 - t1), 2),
                      "generate_tokens_per_s": round(new / (t2 - t0), 2), "hip_graph": graph,
                      "tokens_head": tokens[:8]}
        log(f"C4 {name}: prefill {runs[name]['prefill_ms']} ms, decode {runs[name]['decode_tokens_per_s']} tokens/s")
        del tri
    if "mixed" in runs and "mixed_eager" in runs:
        assert runs["mixed"]["tokens_head"] == runs["mixed_eager"]["tokens_head"], "graph replay changed the tokens"
    del model
    torch.cuda.empty_cache()
    workload = ("C4 e2e: Qwen2-7B architecture (28 layers, hidden 3584, Hq 28 / Hk 4, FFN 18944, vocab 152064, "
                "rope 1e6), prompt 4096 + 256 greedy steps, batch 1, HF modules without the HF KV cache (the "
                "decode cache holds K/V)")
    return runs, share, new, workload


def c4_e2e(args):
    runs, share, new, workload = c4_runs(tuple(args.c4_runs.split(",")))
    main = runs.get("mixed") or next(iter(runs.values()))
    result = {
        "metric": "C4 end-to-end greedy decode tokens/s (prefill time reported separately)",
        "value": main["decode_tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": new,
        "warmup": 1, "ms_per_step": round(main["decode_s"] / (new - 1) * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 model; int8/int4/bf16 attention per map",
        "data": "synthetic (random-init weights N(0, 0.02), 4096 random prompt ids, seed 1004)",
        "config": {"workload": workload + "; value: the one-token forward replayed as a HIP graph (mixed_eager: "
                               "the same without it)",
                   "map_share": share, "global_batch": 1, "seq_len": 4096, "parallelism": "single GPU"},
        "runs": runs,
    }
    print(json.dumps(result))


def calibration_run():
    """configs-adjacent consumer measurement (calibrate.py:44-64): every distance-band configuration of
    the calibration grid as its own Prefill executor, all sharing one scratch dict, over one
    Qwen2-7B-shape attention layer (B 1, Hq 28 / Hk 4, T 4096).  Returns the sweep's time and sizes."""
    import torch

    from triattention_amd import synthetic as S
    from triattention_amd.kernels.extension import load_extension
    from triattention_amd.kernels.prefill import Prefill
    from triattention_amd.maps import INF, uniform

    w8s = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, INF)
    w4s = (2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, INF)
    grid = [(w8, w4) for w8 in w8s for w4 in sorted({w8, *w4s}) if w4 >= w8 and not (w8 == INF and w4 != INF)]
    dev = torch.device("cuda:0")
    module = load_extension()
    g = torch.Generator(device=dev).manual_seed(1005)
    t = 4096
    q, k, v = (S.outlier_tensor_device(g, 1, 28, t), S.outlier_tensor_device(g, 1, 4, t),
               S.outlier_tensor_device(g, 1, 4, t))
    shared = {}
    executors = []
    for w8, w4 in grid:
        executors.append(Prefill(module, uniform(w8, w4)))
        executors[-1].buffers = shared
    for pre in executors:  # builds every band table and view
        pre(0, q, k, v, 128 ** -0.5)
    torch.cuda.synchronize()
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        for pre in executors:
            pre(0, q, k, v, 128 ** -0.5)
    torch.cuda.synchronize()
    sweep_ms = (time.perf_counter() - t0) / reps * 1e3
    scratch = sum(b.numel() * b.element_size() for b in shared.values())
    log(f"calibration sweep: {len(grid)} executors, {sweep_ms:.1f} ms per sweep, shared scratch {scratch / 2**20:.1f} MiB")
    return {"sweep_ms": round(sweep_ms, 3), "executors": len(grid), "per_executor_ms": round(sweep_ms / len(grid), 4),
            "shared_scratch_bytes": scratch, "reps": reps,
            "workload": f"calibrate.py pattern: {len(grid)} Prefill executors with uniform bands sharing one scratch "
                        "dict, one Qwen2-7B-shape layer (B 1, Hq 28 / Hk 4, T 4096)"}


def calibration_sweep(args):
    r = calibration_run()
    print(json.dumps({
        "metric": "calibration sweep time (all band configurations of one layer, shared scratch)",
        "value": r["sweep_ms"], "unit": "ms", "n_gpus": 1, "steps": r["reps"], "warmup": 1,
        "ms_per_step": r["sweep_ms"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8/int4 codes, fp32 softmax", "data": "synthetic (device-drawn N(0,1) with outlier channels)",
        "config": {"workload": r["workload"], "executors": r["executors"], "per_executor_ms": r["per_executor_ms"],
                   "shared_scratch_bytes": r["shared_scratch_bytes"], "parallelism": "single GPU"}}))


def prefill_only(args):
    """--only prefill / c2: the prefill figures alone (C0 and C2, or the C2 attention launch repeated),
    so that a profiler's trace or counters cover nothing else."""
    import torch

    from triattention_amd import synthetic as S
    from triattention_amd.kernels.extension import load_extension
    from triattention_amd.kernels.prefill import Prefill
    from triattention_amd.maps import from_bands

    module = load_extension()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    cases = [("C0", S.config0, 20)] if args.only == "prefill" else []
    cases.append(("C2", S.config2, 5 if args.only == "prefill" else args.steps))
    out = {}
    for name, make, reps in cases:
        cfg = make()
        if name == "C0":
            cfg["kinds"] = []
        if name == "C2" and args.c2_kind:
            # only the C2 inputs with every KV head of one kind (counter runs of one kind)
            kind = args.c2_kind
            v = dict(cfg, kinds=[kind] * 4, bands=S.kv_head_bands([kind] * 4, 7))
            out[f"C2 all {kind}"] = prefill_case(module, dev, stream, f"C2 all {kind}", v, reps, Prefill, from_bands,
                                                 full_call=False)
            continue
        out[name] = prefill_case(module, dev, stream, name, cfg, reps, Prefill, from_bands, full_call=args.only == "prefill")
        if name == "C2" and args.c2_kinds:
            # the C2 inputs with every KV head of one kind (the per-kind cost of the attention tile)
            for kind in args.c2_kinds.split(","):
                v = dict(cfg, kinds=[kind] * 4, bands=S.kv_head_bands([kind] * 4, 7))
                out[f"C2 all {kind}"] = prefill_case(module, dev, stream, f"C2 all {kind}", v, reps, Prefill,
                                                     from_bands, full_call=False)
    print(json.dumps({"prefill": out}))


def prefill_case(module, dev, stream, name, cfg, reps, Prefill, from_bands, full_call=True):
    """Attention-kernel time (HIP events over ``reps`` launches) and the full Prefill call of one config."""
    import torch
    q0, k0, v0 = cfg["q"].to(dev), cfg["k"].to(dev), cfg["v"].to(dev)
    b, hq0, t, _ = q0.shape
    hk0 = k0.shape[1]
    bf16_kv = [h for h, kind in enumerate(cfg["kinds"]) if kind == "bf16"]
    fn = from_bands({"0": cfg["bands"].tolist()}, bf16={"0": bf16_kv} if bf16_kv else None)
    pre0 = Prefill(module, fn)
    pre0(0, q0, k0, v0, cfg["scale"])
    ops = next(iter(pre0.views.values()))
    table = next(iter(pre0.tables.values()))
    exact, nx = pre0.exact(0, hq0, hk0, dev)
    kx, vx = pre0.records if exact is not None else (None, None)
    outp = torch.empty((b, t, hq0, 128), dtype=torch.bfloat16, device=dev).transpose(1, 2)
    pk = ops["packed"]

    def attn():
        module.attention(table.order, table.bands, None, None, pk[1], pk[2], pk[3], ops["vstat"], ops["q8"],
                         ops["kp"], ops["qa"], ops["ka"], ops["q4"], ops["k4"], ops["qa4"], ops["ka4"], outp,
                         cfg["scale"], exact=exact, q=q0, kx=kx, vx=vx, nx=nx, v8sum=ops["v8sum"], k4x=ops["k4x"])

    # untimed calls until ~0.5 s of this workload has run: the clocks rise under sustained
    # load (C2's first calls are ~17% slower than its tenth)
    t_warm = time.perf_counter()
    n_warm = 0
    while n_warm < 2 or time.perf_counter() - t_warm < 0.5:
        attn()
        torch.cuda.synchronize()
        n_warm += 1
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a0.record(stream)
    for _ in range(reps):
        attn()
    a1.record(stream)
    torch.cuda.synchronize()
    att_ms = a0.elapsed_time(a1) / reps
    full_ms = float("nan")
    if full_call:
        w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0.record(stream)
        for _ in range(reps):
            pre0(0, q0, k0, v0, cfg["scale"])
        w1.record(stream)
        torch.cuda.synchronize()
        full_ms = w0.elapsed_time(w1) / reps
    # every head keeps all causal pairs here (INT8 / INT4 / bf16 bands skip no tiles)
    ops_alg = b * hq0 * 4 * 128 * (t * (t + 1) // 2)
    tops = ops_alg / (att_ms * 1e-3) / 1e12
    # mixed bound: QK of the quantized heads at the int8 peak, their PV and every exact head's QK and PV
    # at the bf16 / fp16 peak (the quantized PV runs on int8 MFMA, but its semantics are a u8 x s8 product
    # that the bf16 peak also prices)
    nq = sum(1 for kind in cfg["kinds"] for _ in range(hq0 // hk0) if kind != "bf16") if cfg["kinds"] else hq0
    per_head = ops_alg / hq0
    mixed_us = (nq * per_head / 2 / (INT8_PEAK_TOPS * 1e12) + nq * per_head / 2 / (BF16_PEAK_TFLOPS * 1e12) +
                (hq0 - nq) * per_head / (BF16_PEAK_TFLOPS * 1e12)) * 1e6
    log(f"prefill {name}: attention {att_ms * 1e3:.1f} us = {tops:.1f} int8-TOPS, full call {full_ms * 1e3:.1f} us")
    return {"attention_us": round(att_ms * 1e3, 2), "prefill_call_us": round(full_ms * 1e3, 2),
            "algorithmic_ops": ops_alg, "int8_tops": round(tops, 2),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "mixed_bound_us": round(mixed_us, 2), "frac_mixed_bound": round(mixed_us / (att_ms * 1e3), 4),
            # prompt tokens through ONE layer's Prefill call per second (not a model's prefill rate)
            "layer_call_prompt_tokens_per_s": round(b * t / (full_ms * 1e-3), 1) if full_call else None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time the streaming-read probe over every launch shape at the C1 launch's bytes instead")
    ap.add_argument("--issue-probe", action="store_true",
                    help="SIMD cycles per instruction of the attention tiles' instruction kinds (tri_issue_probe)")
    ap.add_argument("--issue-modes", default="", help="with --issue-probe: comma-separated modes (default all)")
    ap.add_argument("--ceiling-bytes", default="",
                    help="with --read-ceiling: comma-separated byte counts per launch (default: the C1 launch's)")
    ap.add_argument("--merge-form", choices=("auto", "device"), default="auto",
                    help="decode merge launch: the one-wave kernel while the tail holds at most 64 tokens "
                         "(auto), or always tri_decode's merge, which makes the same choice on the device")
    ap.add_argument("--no-c3", action="store_true")
    ap.add_argument("--c3-per", type=int, default=0, help="C3 cache split runs of this many tiles (measurement aid)")
    ap.add_argument("--layers", type=int, default=28, help="C1 layers (own caches, one decode op each per token)")
    ap.add_argument("--c2-kinds", default="", help="with --only c2: also time the C2 inputs with every KV head of "
                                                   "each listed kind (i8, i4, bf16; comma-separated)")
    ap.add_argument("--c2-kind", default="", help="with --only c2: time only the C2 inputs with every KV head of "
                                                  "this kind (i8, i4 or bf16) instead of the C2 mix")
    ap.add_argument("--no-c4", action="store_true", help="leave out the C4 generation from the default run")
    ap.add_argument("--no-calibrate", action="store_true", help="leave out the calibration sweep from the default run")
    ap.add_argument("--only", choices=("prefill", "c2"),
                    help="run one workload alone and print its figures (for profilers): 'prefill' = C0 and C2, "
                         "'c2' = the C2 attention launch")
    ap.add_argument("--c4", action="store_true", help="run the C4 end-to-end generation instead")
    ap.add_argument("--c4-runs", default="mixed,mixed_eager,all_bf16",
                    help="with --c4: which runs (mixed: the map with the HIP graph, mixed_eager: without it, "
                         "all_bf16: every KV head exact)")
    ap.add_argument("--calibrate", action="store_true", help="time the calibration sweep's Prefill executors instead")
    args = ap.parse_args()
    global MERGE_FORM
    MERGE_FORM = args.merge_form
    if args.copy_probe:
        copy_probe()
        return
    if args.issue_probe:
        issue_probe(args)
        return
    if args.read_ceiling:
        read_ceiling(args)
        return
    if args.c4 and args.gpus == 1:
        c4_e2e(args)
        return
    if args.calibrate and args.gpus == 1:
        calibration_sweep(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    if args.only:
        prefill_only(args)
        return

    import numpy as np
    import torch

    from triattention_amd import synthetic as S
    from triattention_amd.kernels.decode import DecodeCache
    from triattention_amd.kernels.extension import load_extension
    from triattention_amd.kernels.prefill import Prefill
    from triattention_amd.maps import from_bands

    module = load_extension()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    # ------------------------------------------------------------------ C1 setup
    log("generating C1 inputs (32 x 4096 tokens)")
    c1 = S.config1()
    batch, hq, hk, prompt = len(c1["seqs"]), 24, 8, c1["prompt"]
    q = torch.cat([s["q"] for s in c1["seqs"]]).to(dev)
    k = torch.cat([s["k"] for s in c1["seqs"]]).to(dev)
    v = torch.cat([s["v"] for s in c1["seqs"]]).to(dev)
    bands = c1["bands"]
    scale = c1["scale"]
    total_steps = args.warmup + args.steps + 1
    # The 28 layers of Llama-3.2-3B (the shape C1 names), the same prompt in each but every layer
    # with its own record arrays: one token runs every layer's decode op once, so the working set
    # (28 x 171 MB) far exceeds the 256 MB Infinity Cache and each decode op streams its records
    # from HBM, as in the model.  (A single cache re-read every step would be served partly from
    # that cache: 38.4 vs 44.8 us measured.)  The token's HIP graph holds the 28 decode ops and one
    # step advance, as the model's one-token forward does.  Layer 0 runs the full prefill (its
    # decode outputs are checked against the oracle below); the others store the same records.
    layers = args.layers
    cache = DecodeCache(module, max_tail=256)
    pre = Prefill(module, from_bands({str(layer): bands.tolist() for layer in range(layers)}), cache)
    pre(0, q, k, v, scale)
    for layer in range(1, layers):
        pre.store_only(layer, k, v, hq)
    torch.cuda.synchronize()
    del q, k, v, pre
    e = cache.layers[0]
    rec_bytes, kept_tiles = decode_record_bytes(e)
    g = S.gen(4242)
    toks = [(S.outlier_tensor(g, batch, hq, 1).to(dev), S.outlier_tensor(g, batch, hk, 1).to(dev),
             S.outlier_tensor(g, batch, hk, 1).to(dev)) for _ in range(total_steps)]
    log(f"cache: {kept_tiles} kept tiles, {rec_bytes} record bytes/step, per={e['per']}, maxn={e['maxn']}")

    # step 0 output, kept for the parity spot check against the oracle
    out0 = cache(0, *toks[0], scale).float().cpu()
    for layer in range(1, layers):
        cache(layer, *toks[0], scale)
    cache.advance()

    out = torch.empty((batch, hq, 1, 128), dtype=torch.bfloat16, device=dev)
    plans = [cache.plan(layer, toks[0][0], toks[0][1], out, scale) for layer in range(layers)]

    def step(i, ev=None):
        # one decode op of layer i % layers: the split-KV kernel and the merge kernel; the step
        # counter advances once per token, after the last layer
        qd, kd, vd = toks[i % total_steps]
        plan = plans[i % layers]
        short = short_merge(cache, i % layers, hq)
        if ev is None:
            plan.run(qd, kd, vd, out, short_tail=short)
        else:
            plan.run(qd, kd, vd, out, 1, events=ev)
            plan.run(qd, kd, vd, out, 2, short_tail=short)
        if i % layers == layers - 1:
            cache.advance()

    # A GPU that has been idle runs well below its working clocks until it has carried a compute
    # load for about a second: a decode step measured 110 us right after setup and 54.5 us after
    # one second of bf16 GEMMs, steady for the next 30 s, and decode steps alone did not lift it.
    # So before the W warmup steps: ~1.5 s of untimed GEMMs, then ~0.5 s of decode steps.
    log("device warm-up: ~1.5 s of bf16 GEMMs and ~0.5 s of untimed decode steps")
    mat = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 1.5:
        mat = (mat @ mat).clamp_(-1.0, 1.0)
        torch.cuda.synchronize()
    del mat
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.5:
        for j in range(200):
            step(1 + j % layers)
        torch.cuda.synchronize()
    # C1 is one token after the prompt: restart the step counter (the bf16 tail length)
    cache.step.fill_(1)
    cache.host_step = 1
    log(f"warmup {args.warmup} steps")
    for i in range(1, 1 + args.warmup):
        step(i)
    evs = kernel_events(args.steps, stream)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    step0 = int(cache.step.item())
    start.record(stream)
    for i in range(args.steps):
        step(1 + args.warmup + i, evs[i])
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    eager_ms_per_step = total_ms / args.steps
    dec_ms = statistics.fmean(ev[0].elapsed_time(ev[1]) for ev in evs)

    # The step as the model path runs it: one token (every layer's decode op, then the step
    # advance) captured as a HIP graph and replayed, the merge launched as tri_decode's, which picks
    # its form on the device at every replay (as a graph the model path captures does); ms_per_step
    # is per decode op (per layer).
    def token():
        for layer in range(layers):
            plans[layer].run(*toks[(1 + args.warmup + layer) % total_steps], out)
        cache.advance()
    tokens = max(4, -(-args.steps // layers))
    ms_per_step = graph_steps(token, tokens, stream) / layers
    # small algorithmic bytes of a step: q and out (bf16), K mean and V mean/scale per (seq, KV head),
    # and the bf16 K/V tail read by the merge (mean tail length over the timed steps)
    mean_tail = min(256, step0 + args.steps / layers + (tokens + 3) / 2)
    small = batch * hq * 256 * 2 + batch * hk * (3 * 128 * 4) + batch * hk * 2 * 256 * mean_tail
    step_bytes = rec_bytes + small
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = rec_bytes / (dec_ms * 1e-3) / 1e9
    log(f"decode step {ms_per_step * 1e3:.1f} us from a HIP graph, {eager_ms_per_step * 1e3:.1f} us eager "
        f"(split-KV kernel {dec_ms * 1e3:.1f} us)")
    # the same bytes read with no compute, in the probe's best launch shape: what this device streams
    ceil_us, ceil_gbs, ceil_shape = stream_ceiling(module, dev, rec_bytes, layers, STREAM_SHAPES_DEFAULT)
    log(f"streaming-read ceiling for {rec_bytes} B: {ceil_us:.1f} us ({ceil_gbs:.0f} GB/s); the split-KV kernel "
        f"runs at {achieved / ceil_gbs:.3f} of it")

    traffic, traffic_note = measured_traffic()
    result = {
        "metric": "prefill int8 TOPS (% MFMA peak); decode KV GB/s (% HBM peak); tokens/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "eager_ms_per_step": round(eager_ms_per_step, 5),
        "step_launch": "one token (the decode op of each of the 28 layers -- split-KV kernel + merge kernel "
                       "each -- then the step advance) captured as a HIP graph and replayed, as the model path "
                       "runs decode; ms_per_step is per decode op; eager_ms_per_step launches each kernel from "
                       "Python",
        "merge": ("eager steps: the one-wave kernel (tails of at most 16 tokens on a grid of at least 2 "
                  "workgroups per CU: C1's 768 on 256 CUs); graph replays: tri_decode's merge, which makes the "
                  "same choice on the device" if MERGE_FORM == "auto"
                  else "tri_decode's merge, its form chosen on the device (--merge-form device)"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8/int4 codes, fp32 softmax",
        "data": "synthetic (seeded N(0,1) K/V with 4 outlier channels x20 per head, bf16)",
        "config": {"workload": "C1 decode: batch 32, Hq 24 / Hk 8, head_dim 128, prompt 4096 in the quantized "
                               "cache, 25% INT8 / 75% INT4 KV heads, one bf16 token per sequence",
                   "global_batch": batch, "seq_len": prompt, "parallelism": "single GPU"},
        # one decode op serves every sequence's next token for ONE layer; a model token needs all layers
        "layer_op_tokens_per_s": round(batch / (ms_per_step * 1e-3), 1),
        "model_tokens_per_s": {"value": round(batch / (ms_per_step * layers * 1e-3), 1), "layers": layers,
                               "what": f"batch / (one token of all {layers} layers' decode ops in the replayed "
                                       "graph): the attention part of a Llama-3.2-3B decode step, measured"},
        "step_bytes": int(step_bytes),
        "roofline": {"bound": "hbm", "kernel": "decode_kernel", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_note": traffic_note, "algorithmic_bytes": rec_bytes,
                     "avg_us": round(dec_ms * 1e3, 2), "working_set_bytes": layers * rec_bytes},
        "stream_ceiling": {"achieved": round(ceil_gbs, 1), "us": round(ceil_us, 2),
                           "frac": round(ceil_gbs / HBM_PEAK_GBS, 4), "kernel_frac_of_ceiling":
                           round(achieved / ceil_gbs, 4), "shape": list(ceil_shape),
                           "note": "the split-KV kernel's record bytes read by a no-compute probe "
                                   "(tri_stream_read: waves, waves per workgroup, records in flight), "
                                   "best of the listed shapes, from the same rotating buffers"},
    }

    # ------------------------------------------------------------- CPU baseline
    threads = cpu_threads()
    if not args.no_cpu:
        import oracle as O
        from concurrent.futures import ThreadPoolExecutor
        bn = bands.numpy()
        log(f"CPU oracle: K/V codes of the {batch} sequences ({threads} threads)")
        qd, kd, vd = (x.cpu() for x in toks[0])
        zeros = np.zeros((hk, 256, 128), np.uint16)
        # one sequence per task; the oracle's C calls release the GIL, so the pool runs them in parallel
        with ThreadPoolExecutor(threads) as pool:
            codes = list(pool.map(lambda b: O.prefill_codes(None, S.bits(c1["seqs"][b]["k"][0]),
                                                            S.bits(c1["seqs"][b]["v"][0]), bn, decode_cache=True),
                                  range(batch)))
            one = lambda b: O.decode(codes[b], bn, S.bits(qd[b, :, 0]), prompt, cache.split_of(0, b), scale, zeros,
                                     zeros, S.bits(kd[b, :, 0]), S.bits(vd[b, :, 0]), 0)
            times = []
            for rep in range(3):
                t0 = time.perf_counter()
                outs = list(pool.map(one, range(batch)))
                times.append(time.perf_counter() - t0)
        # GPU step-0 output is bf16: compare within one bf16 ulp of the rounded oracle value
        errs = [float((out0[b, :, 0] - torch.from_numpy(outs[b]).to(torch.bfloat16).float()).abs().max())
                for b in range(batch)]
        cpu_step = statistics.median(times)
        result["cpu_baseline"] = {
            "value": round(step_bytes / cpu_step / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the C oracle's decode of all {batch} sequences at step 0 (the whole C1 step, no "
                      f"extrapolation), one sequence per task on {threads} threads, median of 3",
            "ms_per_step": round(cpu_step * 1e3, 2), "layer_op_tokens_per_s": round(batch / cpu_step, 2),
            "host_cpu_count": os.cpu_count()}
        result["parity_spot_check"] = {"sequences": batch, "max_abs_vs_oracle_bf16": max(errs)}

    # ----------------------------------------------------------------- prefill
    if not args.no_prefill:
        log("prefill C0")
        c0 = S.config0()
        c0["kinds"] = []
        r0 = prefill_case(module, dev, stream, "C0", c0, 20, Prefill, from_bands)
        r0["workload"] = "C0 prefill: batch 1, Hq 24 / Hk 8, T 1024, 50/50 INT8/INT4 KV heads"
        if not args.no_cpu:
            import oracle as O
            # the same unit on the host: one whole Prefill call (codes, statistics, records and the
            # attention) of C0 by the C oracle, its attention rows on every thread, median of 3
            times = []
            for rep in range(3):
                t0 = time.perf_counter()
                O.prefill(S.bits(c0["q"][0]), S.bits(c0["k"][0]), S.bits(c0["v"][0]), c0["bands"].numpy(),
                          c0["scale"], threads=threads)
                times.append(time.perf_counter() - t0)
            cpu_ms = statistics.median(times) * 1e3
            result.setdefault("cpu_baseline", {})["prefill_C0"] = {
                "ms_per_call": round(cpu_ms, 2), "layer_call_prompt_tokens_per_s": round(1024 / (cpu_ms * 1e-3), 1),
                "int8_tops": round(r0["algorithmic_ops"] / (cpu_ms * 1e-3) / 1e12, 4), "threads": threads,
                "gpu_speedup_full_call": round(cpu_ms * 1e3 / r0["prefill_call_us"], 1)}
            log(f"CPU oracle C0 prefill: {cpu_ms:.1f} ms per call ({threads} threads)")
        log("prefill C2 (generating 4 x 8192 tokens)")
        c2 = S.config2()
        r2 = prefill_case(module, dev, stream, "C2", c2, 5, Prefill, from_bands)
        r2["workload"] = (f"C2 prefill: batch 4, Hq 28 / Hk 4, T 8192, log-uniform channel scales, KV heads "
                          f"{c2['kinds']}")
        r2["counters"], r2["counters_note"] = prefill_counters()
        result["prefill"] = {"C0": r0, "C2": r2}

    # ------------------------------------------------------- C3 ragged decode
    if not args.no_c3:
        result["c3_decode"] = c3_decode(module, dev, stream, args, S, DecodeCache, Prefill, from_bands)

    # ------------------------------------------- calibration consumer, C4 end to end
    if not args.no_calibrate:
        result["calibration"] = calibration_run()
    if not args.no_c4:
        del cache, plans, toks
        torch.cuda.empty_cache()
        runs, share, new, workload = c4_runs(("mixed",), reps=2)
        result["c4_e2e"] = dict(runs["mixed"], workload=workload + "; the one-token forward replayed as a HIP graph",
                                map_share=share, steps=new)

    print(json.dumps(result))


if __name__ == "__main__":
    main()
