"""Benchmark of the KV data path on one MI355X.

Headline: FP8 swap-out + swap-in of 8,192 tokens (512 random
Qwen3-4B blocks of a 12 GiB BF16 pool with 0.1% +/-40 outliers) through NativeBackend: fused
gather+quantize into staging, copies to pinned host memory on the engine's copy stream, then
copies back and fused dequantize+scatter into 512 fresh random block ids. A step is one out+in; `value` is ms per
step (lower is better). Inputs are resident in HBM when the timed region starts.

Also measured in the same run (extra keys of the JSON line):
  link        pinned hipMemcpyAsync peak each way (the host-link roofline of the swap)
  roofline    the fused quantize kernel: algorithmic bytes / its average duration, from HIP
              events recorded on the stream it runs on around the step's launches repeated
              back to back (no copy beside them), against the 8 TB/s HBM peak
  decode      BASELINE configs[2]: paged decode, batch 32, contexts U[1024, 32768], 36
              layers timed per layer, "unique" KV bytes (decode_bandwidth.py:129-139)
  decode_fp8  configs[3]: the same reading FP8 records, plus batch 1 @ 32,768 and 64 @ 4,096
  decode_graphs  small-batch decode steps (token write + attention, 36 layers) replayed as
              one HIP graph, against the same step launched eagerly; BF16 and FP8 pools
  prefill     paged causal prefill of 2,048-token chunks at the start and at the end of a
              32,768-token context, beside gather + torch flash attention on the same GPU
  overlap     configs[4]: decode steps while 2,048 blocks swap out and back in
  decode_distinct  configs[2] on a ~78 GB pool whose rows share no block
  decode_fp8_distinct  configs[3]'s batch 32 on FP8 records of that pool (the same rows)
  hbm_probe   lk_stream_probe read and copy rates and lk_stream_probe_mix at the FP8 kernels' read/write mixes: the measured HBM ceilings
  swap_bf16   the same 512 blocks swapped raw (gather kernel + DMA), byte-exact
  cpu_baseline  the oracle's C restatement of the FP8 swap arithmetic on all 512 blocks, in
              threads on the host cores; its records are compared with the GPU payload
  cpu_config1  configs[0]: 64 of 4,096 BF16 blocks out and back on the host libraries (the
              reference's own, built from its sources into oracle/_ref, and this package's)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-decode] [--skip-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# Measured HBM bytes per quantize launch over its algorithmic bytes (read + write), from two
# rocprofv3 --pmc passes over this script (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch).
# FETCH_SIZE counts half the bytes read by these kernels: lk_stream_probe's 8 GiB read shows
# as 4 GiB, and its 4 GiB copy as 4 GiB of WRITE_SIZE. Per full 113-record launch:
# 2 x 130,221 + 130,686 KiB measured against 390,636 KiB algorithmic.
QUANTIZE_TRAFFIC_RATIO = 1.0026
L4_FP8_SWAP_MS = 67.0  # the reference's published FP8 swap out+in at 8,192 tokens on an NVIDIA L4 (README.md:27, :115)
QWEN = dict(layers=36, kv_heads=8, query_heads=32, slots=16, head_dim=128)
POOL_BYTES = 12 << 30


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def fill_pool(pool, seed: int, outlier_fraction: float = 0.0) -> None:
    """N(0,1) BF16 plus seeded +/-40 outliers, filled in slices to bound temporaries."""
    import torch

    generator = torch.Generator(device=pool.device).manual_seed(seed)
    for start in range(0, pool.shape[0], 256):
        piece = pool[start : start + 256]
        values = torch.randn(piece.shape, generator=generator, device=pool.device, dtype=torch.float32)
        if outlier_fraction:
            mask = torch.rand(piece.shape, generator=generator, device=pool.device) < outlier_fraction
            signs = torch.where(torch.rand(piece.shape, generator=generator, device=pool.device) < 0.5, -40.0, 40.0)
            values = torch.where(mask, signs, values)
        piece.copy_(values.to(torch.bfloat16))
        del values


def rotating_slots(device, slot_bytes: int, total_bytes: int = 1 << 30) -> list:
    """Staging slots for back-to-back kernel legs, used in turn: together at least 1 GiB (four
    times the 256 MB Infinity Cache), so a slot is long out of the cache when it comes round
    again. Zeroed here, so every byte a launch reads is defined."""
    import torch

    count = max(2, -(-total_bytes // slot_bytes))
    return [torch.zeros(slot_bytes, dtype=torch.uint8, device=device) for _ in range(count)]


def time_launches(stream, launches, bytes_of_each) -> dict:
    """Average duration of a run of kernel launches queued back to back on `stream`, timed by
    one pair of HIP events recorded on that stream around the whole run (an event pair per
    launch would add its own packets to every window). A bounded spin is queued first, so the
    whole run is queued before the stream reaches it: a pause of the host thread cannot fall
    inside the window."""
    import torch

    total_bytes = sum(bytes_of_each)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        spin = getattr(torch.cuda, "_sleep", None)  # torch's test helper: a kernel that spins for n cycles
        if spin is not None:
            spin(200_000_000)
        start.record()
        for launch in launches:
            launch()
        end.record()
    end.synchronize()
    ms = start.elapsed_time(end)
    return {"launches": len(launches), "mean_ms": ms / len(launches), "bytes_per_launch": total_bytes / len(launches),
            "achieved_gbs": total_bytes / (ms * 1e-3) / 1e9}


def measure_link(device, nbytes: int = 512 << 20, repeats: int = 5) -> dict:
    """Pinned-memory hipMemcpyAsync peak each way (torch copies are SDMA copies here)."""
    import torch

    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dev = torch.empty(nbytes, dtype=torch.uint8, device=device)
    out = {}
    stream = torch.cuda.Stream(device=device)
    for name, fn in (("d2h_gbs", lambda: host.copy_(dev, non_blocking=True)), ("h2d_gbs", lambda: dev.copy_(host, non_blocking=True))):
        with torch.cuda.stream(stream):
            fn()
            stream.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(repeats):
                fn()
            end.record()
            end.synchronize()
        out[name] = repeats * nbytes / (start.elapsed_time(end) * 1e-3) / 1e9
    out["bytes"] = nbytes
    return out


def measure_hbm(device, nbytes: int = 8 << 30, repeats: int = 5, launch_bytes: int = 0, launch_repeats: int = 100) -> dict:
    """HBM ceilings measured on this GPU with the library's streaming probes (non-temporal; a
    read moves 4 KiB per wave, a copy or mix 1 KiB per single-wave workgroup, the faster shape
    for each): read-only over 8 GiB, a copy of 4 GiB
    (8 GiB of traffic), and the two traffic mixes of the FP8 record kernels: 8 GiB read and
    4 GiB written (quantize's 2:1), 4 GiB read and 8 GiB written (dequantize's 1:2). Reported
    beside the 8 TB/s specification; rates count bytes read plus bytes written.

    With launch_bytes, the two mixes are also timed at that much traffic per launch (a record
    kernel's launch), launch_repeats launches back to back over consecutive slices of the 8 GiB
    buffers, so that each launch pays the dispatch ramp and drain the record kernels pay and
    reads nothing a cache holds: the like-for-like ceiling for those kernels."""
    import torch

    from layover_amd.kernels import _lib

    lib = _lib.load()
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    src.fill_(1)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _lib.current_stream(device)
    half = nbytes // 2
    out = {}
    for name, run, moved in (
        ("read_gbs", lambda: lib.lk_stream_probe(src.data_ptr(), None, nbytes, sink.data_ptr(), stream), nbytes),
        ("copy_gbs", lambda: lib.lk_stream_probe(src.data_ptr(), dst.data_ptr(), half, sink.data_ptr(), stream), nbytes),
        ("quantize_mix_gbs", lambda: lib.lk_stream_probe_mix(src.data_ptr(), nbytes, dst.data_ptr(), half, stream), nbytes + half),
        ("dequantize_mix_gbs", lambda: lib.lk_stream_probe_mix(src.data_ptr(), half, dst.data_ptr(), nbytes, stream), nbytes + half),
    ):
        _lib.check(run())
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeats):
            _lib.check(run())
        end.record()
        end.synchronize()
        out[name] = repeats * moved / (start.elapsed_time(end) * 1e-3) / 1e9
    if launch_bytes:
        small = launch_bytes // 3 // 4096 * 4096  # the 1 part of a 2:1 or 1:2 mix, whole pages
        slots = nbytes // (2 * small)
        for name, two_to_one in (("quantize_mix_launch_gbs", True), ("dequantize_mix_launch_gbs", False)):
            src_bytes, dst_bytes = (2 * small, small) if two_to_one else (small, 2 * small)

            def launch(i):
                k = i % slots
                _lib.check(lib.lk_stream_probe_mix(src.data_ptr() + k * src_bytes, src_bytes, dst.data_ptr() + k * dst_bytes, dst_bytes, stream))

            for i in range(3):
                launch(i)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for i in range(launch_repeats):
                launch(3 + i)
            end.record()
            end.synchronize()
            out[name] = launch_repeats * 3 * small / (start.elapsed_time(end) * 1e-3) / 1e9
        out["launch_bytes"] = 3 * small
    del src, dst
    torch.cuda.empty_cache()
    return out


def swap_bench(args, device, pool_blocks: int, cache):
    import numpy as np
    import torch

    from layover_amd.kernels.fp8 import Fp8Layout, dequantize_blocks, quantize_blocks
    from layover_amd.kv.transfer import NativeBackend
    from oracle import oracle

    layout = Fp8Layout.from_cache(cache)
    rng = np.random.default_rng(1)
    chosen = rng.permutation(pool_blocks)[: 2 * args.blocks]
    src = [int(i) for i in chosen[: args.blocks]]
    dst = [int(i) for i in chosen[args.blocks :]]

    backend = NativeBackend(device, staging_bytes=args.staging_mib << 20, num_staging=2, ids_capacity=1 << 20)
    backend.prepare(cache, fp8=True)

    def step():
        out = backend.start_out(cache, src, fp8=True)
        out.wait()
        backend.start_in(cache, dst, out.payload).wait()
        return out.payload

    log(f"swap: warmup {args.warmup}")
    for _ in range(args.warmup):
        backend.free(step())

    # Parity on a sample of records: payload bytes vs the oracle's records, restored blocks
    # vs the oracle's dequantization of them.
    payload = step()
    sample = list(range(0, args.blocks, max(1, args.blocks // 4)))[:4]
    bits = cache.pool[torch.tensor([src[i] for i in sample], device=device)].view(torch.int16).cpu().numpy().view(np.uint16)
    expected = oracle.quantize_records(bits, list(range(len(sample))), layout.group_elems, layout.groups_per_block)
    memory = payload.memory.numpy()
    got = np.concatenate([memory[i * layout.record_bytes : (i + 1) * layout.record_bytes] for i in sample])
    restored = cache.pool[torch.tensor([dst[i] for i in sample], device=device)].view(torch.int16).cpu().numpy().view(np.uint16)
    reference = np.zeros_like(bits)
    oracle.dequantize_records(expected, list(range(len(sample))), reference, layout.group_elems, layout.groups_per_block)
    parity = bool(np.array_equal(got, expected) and np.array_equal(restored, reference))
    gpu_records = memory[: args.blocks * layout.record_bytes].copy()  # checked in full against the CPU leg
    # The source blocks as they were quantized (later legs write into the pool).
    source_bits = cache.pool[torch.tensor(src, device=device)].view(torch.int16).cpu().numpy().view(np.uint16).reshape(len(src), -1)
    backend.free(payload)
    if not parity:
        raise SystemExit("FP8 swap is not bit-exact against the oracle: refusing to report a number")

    log(f"swap: timing {args.steps} steps")
    torch.cuda.synchronize()
    start = time.perf_counter()
    out_ms, in_ms = [], []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        out = backend.start_out(cache, src, fp8=True)
        out.wait()
        t1 = time.perf_counter()
        backend.start_in(cache, dst, out.payload).wait()
        t2 = time.perf_counter()
        backend.free(out.payload)
        out_ms.append((t1 - t0) * 1e3)
        in_ms.append((t2 - t1) * 1e3)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    stats = backend.engine.stats()

    # The kernels' own rates: the step's quantize and dequantize launches (the same segments
    # and stream), repeated back to back with no copy to the host beside them. In the steps
    # above a segment's quantize overlaps the previous segment's copy to the host, which the
    # runtime runs as a kernel; that copy holds its CUs' path to memory at the link's pace, so a
    # kernel beside it measures the copy, not itself. Successive launches rotate over staging
    # slots worth 1 GiB, four times the Infinity Cache, so no launch finds the records another
    # just wrote in the cache: both sides of every launch go to HBM.
    log("swap: FP8 kernel leg")
    bytes_of = lambda ids: ids.shape[0] * (2 * layout.block_elems + layout.record_bytes)
    per = backend.engine.staging_bytes // layout.record_bytes
    segments = [(torch.tensor(src[i : i + per], dtype=torch.int32, device=device), torch.tensor(dst[i : i + per], dtype=torch.int32, device=device))
                for i in range(0, len(src), per)]
    stages = rotating_slots(device, backend.engine.staging_bytes)
    quantize_runs, dequantize_runs, sizes = [], [], []
    for repeat in range(args.kernel_repeats):
        for index, (out_ids, in_ids) in enumerate(segments):
            stage = stages[(repeat * len(segments) + index) % len(stages)]
            quantize_runs.append(lambda out_ids=out_ids, stage=stage: quantize_blocks(cache.pool, out_ids, stage, layout))
            dequantize_runs.append(lambda in_ids=in_ids, stage=stage: dequantize_blocks(stage, in_ids, cache.pool, layout))
            sizes.append(bytes_of(out_ids))
    quantize = time_launches(backend.kernel_stream, quantize_runs, sizes)
    dequantize = time_launches(backend.kernel_stream, dequantize_runs, sizes)
    torch.cuda.synchronize()
    del stages
    backend.close()
    record_total = args.blocks * layout.record_bytes
    return {
        "ms_per_step": elapsed * 1e3 / args.steps,
        "out_ms": sorted(out_ms)[len(out_ms) // 2],
        "in_ms": sorted(in_ms)[len(in_ms) // 2],
        "bytes_each_way": record_total,
        "bf16_bytes_each_way": args.blocks * cache.block_bytes,
        "quantize": quantize,
        "dequantize": dequantize,
        "parity_sample_records": len(sample),
        "segments_per_direction": math.ceil(args.blocks / ((args.staging_mib << 20) // layout.record_bytes)),
        "engine_memcpys": stats["memcpys"],
        "source_bits": source_bits,
        "gpu_records": gpu_records,
    }


def bf16_swap_bench(args, device, pool_blocks: int, cache) -> dict:
    """The same 512 blocks swapped as raw BF16 (lt_out_gather / lt_in_scatter: gather kernel,
    DMA per 128 MiB segment, two slots), the reference's 109 ms path on an L4 (README.md:27)."""
    import numpy as np
    import torch

    from layover_amd.kv.transfer import NativeBackend

    rng = np.random.default_rng(1)
    chosen = rng.permutation(pool_blocks)[: 2 * args.blocks]
    src = [int(i) for i in chosen[: args.blocks]]
    dst = [int(i) for i in chosen[args.blocks :]]
    backend = NativeBackend(device, staging_bytes=args.staging_mib << 20, num_staging=2, ids_capacity=1 << 20)
    backend.prepare(cache, fp8=False)
    try:
        def step():
            out = backend.start_out(cache, src)
            out.wait()
            backend.start_in(cache, dst, out.payload).wait()
            return out.payload

        for _ in range(args.warmup):
            backend.free(step())
        payload = step()
        source = cache.pool[torch.tensor(src, device=device)].view(torch.uint8).reshape(-1).cpu().numpy()
        landed = cache.pool[torch.tensor(dst, device=device)].view(torch.uint8).reshape(-1).cpu().numpy()
        parity = bool(np.array_equal(payload.memory.numpy(), source) and np.array_equal(landed, source))
        backend.free(payload)
        if not parity:
            raise SystemExit("BF16 swap is not byte-exact: refusing to report a number")
        out_ms, in_ms = [], []
        torch.cuda.synchronize()
        for _ in range(args.steps):
            t0 = time.perf_counter()
            out = backend.start_out(cache, src)
            out.wait()
            t1 = time.perf_counter()
            backend.start_in(cache, dst, out.payload).wait()
            t2 = time.perf_counter()
            backend.free(out.payload)
            out_ms.append((t1 - t0) * 1e3)
            in_ms.append((t2 - t1) * 1e3)
        stats = backend.engine.stats()
    finally:
        backend.close()
    kernels = bf16_kernel_leg(args, device, cache, src, dst)
    each_way = args.blocks * cache.block_bytes
    total_ms = sum(out_ms) / len(out_ms) + sum(in_ms) / len(in_ms)
    return {
        "ms_per_step": round(total_ms, 3),
        "out_ms": round(sorted(out_ms)[len(out_ms) // 2], 3),
        "in_ms": round(sorted(in_ms)[len(in_ms) // 2], 3),
        "bytes_each_way": each_way,
        "round_trip_gbs": round(2 * each_way / (total_ms * 1e-3) / 1e9, 2),
        "kernels": stats["kernels"],
        "parity": "byte-exact: payload and restored blocks equal the source blocks, all 512",
        "reference_l4_ms": 109.0,
        "kernel_leg": kernels,
    }


def bf16_kernel_leg(args, device, cache, src, dst) -> dict:
    """The BF16 swap's gather and scatter kernels alone (lk_gather_blocks / lk_scatter_blocks,
    the kernels lt_out_gather / lt_in_scatter launch): the step's segments (56 blocks per
    128 MiB slot, 9 x 56 + 8 for 512 blocks) repeated back to back on one stream over rotating
    staging slots (rotating_slots), timed by time_launches. Bytes per block: read + write of
    2,359,296 B. Inside the swap the same launches run between copies on a mostly idle GPU
    and take longer (see the profile)."""
    import torch

    from layover_amd.kernels.blocks import gather_blocks, scatter_blocks

    per_segment = (args.staging_mib << 20) // cache.block_bytes
    slots = rotating_slots(device, per_segment * cache.block_bytes)
    as_ids = lambda ids: torch.tensor(ids, dtype=torch.int32, device=device)
    segments = [(as_ids(src[i : i + per_segment]), as_ids(dst[i : i + per_segment])) for i in range(0, len(src), per_segment)]
    stream = torch.cuda.Stream(device=device)
    result = {"segment_blocks": per_segment, "segments": len(segments), "staging_slots": len(slots)}
    turns = [(o, i, slots[n % len(slots)]) for n, (o, i) in enumerate(segments * args.kernel_repeats)]
    for name, run in (("gather", lambda out_ids, in_ids, slot: gather_blocks(cache.pool, out_ids, slot)),
                      ("scatter", lambda out_ids, in_ids, slot: scatter_blocks(slot, in_ids, cache.pool))):
        launches = [lambda o=o, i=i, slot=slot, run=run: run(o, i, slot) for o, i, slot in turns]
        sizes = [2 * o.numel() * cache.block_bytes for o, _, _ in turns]
        with torch.cuda.stream(stream):
            launches[0]()
        timed = time_launches(stream, launches, sizes)
        result[name] = {"mean_launch_us": round(timed["mean_ms"] * 1e3, 2), "achieved_gbs": round(timed["achieved_gbs"], 1),
                        "frac": round(timed["achieved_gbs"] / HBM_PEAK_GBS, 4), "launches": timed["launches"]}
    torch.cuda.synchronize()
    del slots
    torch.cuda.empty_cache()
    return result


def decode_tables(rng, batch: int, lengths, pool_blocks: int, distinct: bool):
    import numpy as np

    width = max(-(-int(n) // 16) for n in lengths)
    table = np.zeros((batch, width), dtype=np.int32)
    if distinct:
        ids = rng.permutation(pool_blocks)
        at = 0
        for b, n in enumerate(lengths):
            k = -(-int(n) // 16)
            table[b, :k] = ids[at : at + k]
            at += k
    else:
        for b, n in enumerate(lengths):
            k = -(-int(n) // 16)
            table[b, :k] = rng.choice(pool_blocks, k, replace=False)
    return table


def decode_bench(device, pool, lengths, steps: int, warmup: int, seed: int, distinct: bool = False, kv_pool=None, probe: bool = True,
                 pool_blocks: int | None = None):
    """Time 36 single-layer launches per step; bytes are the reference's unique accounting
    (layover_amd.kernels.decode_bytes). `pool` (BF16) may be None when `kv_pool` (FP8 records)
    and `pool_blocks` are given. Rows whose tables list more blocks than the pool holds share
    blocks, and are launched with LK_DECODE_SHARED_BLOCKS, as paged_decode_attention_hip
    decides it; otherwise the tiles are streamed."""
    import numpy as np
    import torch

    from layover_amd.kernels import decode_bytes, hip_decode

    rng = np.random.default_rng(seed)
    batch = len(lengths)
    pool_blocks = pool.shape[0] if pool_blocks is None else pool_blocks
    table = torch.from_numpy(decode_tables(rng, batch, lengths, pool_blocks, distinct)).to(device)
    lens = torch.tensor(lengths, dtype=torch.int32, device=device)
    generator = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch, QWEN["query_heads"], QWEN["head_dim"], generator=generator, device=device).to(torch.bfloat16)
    target = kv_pool if kv_pool is not None else pool
    out = torch.empty_like(q)
    shared = decode_bytes.sequence_blocks(lengths, QWEN["slots"]) > pool_blocks
    shape = hip_decode.decode_shape(q, target, 0, table, QWEN["query_heads"] // QWEN["kv_heads"])
    workspace = torch.empty(hip_decode.workspace_bytes(shape), dtype=torch.uint8, device=device)
    groups = QWEN["query_heads"] // QWEN["kv_heads"]
    for _ in range(warmup):
        for layer in range(QWEN["layers"]):
            hip_decode.run_kernel(q, target, layer, table, lens, groups, out, workspace, shared_blocks=shared)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        for layer in range(QWEN["layers"]):
            hip_decode.run_kernel(q, target, layer, table, lens, groups, out, workspace, shared_blocks=shared)
    end.record()
    end.synchronize()
    per_layer_ms = start.elapsed_time(end) / (steps * QWEN["layers"])
    kv_format = "fp8" if kv_pool is not None else "bf16"
    kv_bytes = (decode_bytes.fp8_record_bytes_per_layer(lengths, decode_bytes.QWEN3_4B) if kv_pool is not None
                else decode_bytes.unique_bytes_per_layer(lengths, decode_bytes.QWEN3_4B, 2))
    launch = decode_bytes.launch_bytes(lengths, decode_bytes.QWEN3_4B, kv_format, 2, table.shape[1])
    result = {
        "batch": batch,
        "per_layer_us": per_layer_ms * 1e3,
        "kv_bytes_per_layer": kv_bytes,
        "launch_bytes": launch,
        "achieved_gbs": launch / (per_layer_ms * 1e-3) / 1e9,
        "frac_of_hbm_peak": launch / (per_layer_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "distinct_blocks": distinct,
        "shared_blocks": shared,
    }
    if not probe:
        return result
    # The same tiles read in the same order with no compute (lk_tile_probe): the ceiling
    # of this access pattern on this pool, which the decode kernel is compared with.
    from layover_amd.kernels import _lib

    lib = _lib.load()
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _lib.current_stream(device)
    storage = kv_pool.records if kv_pool is not None else pool
    shapes = [hip_decode.decode_shape(q, target, layer, table, groups, lens) for layer in range(QWEN["layers"])]
    read_tiles = lambda: [_lib.check(lib.lk_tile_probe(sh, storage.data_ptr(), table.data_ptr(), lens.data_ptr(), sink.data_ptr(), stream))
                          for sh in shapes]
    read_tiles()
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        read_tiles()
    end.record()
    end.synchronize()
    probe_ms = start.elapsed_time(end) / (steps * QWEN["layers"])
    result["tile_probe_us"] = probe_ms * 1e3
    result["tile_probe_gbs"] = kv_bytes / (probe_ms * 1e-3) / 1e9
    result["frac_of_tile_probe"] = probe_ms / per_layer_ms
    return result


def decode_step_events(device, pool, table, lens, q, out, workspace, groups, shared_blocks: bool):
    """Launch one decode step (36 single-layer launches) on the current stream, bracketed by
    timing events; returns the events."""
    import torch

    from layover_amd.kernels import hip_decode

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for layer in range(QWEN["layers"]):
        hip_decode.run_kernel(q, pool, layer, table, lens, groups, out, workspace, shared_blocks=shared_blocks)
    end.record()
    return start, end


def graph_decode_bench(device, cache, fp8_pool, steps: int = 20) -> list:
    """Small-batch decode steps (every layer: write the new token, then paged attention) as
    one HIP graph replay against the same step launched eagerly from Python, on the BF16 pool
    and on the FP8-record pool. Rows use distinct random blocks of the 12 GiB pool."""
    import numpy as np
    import torch

    from layover_amd.kernels import decode_bytes
    from layover_amd.kv.decode_graphs import DecodeAttentionGraphs
    from layover_amd.kv.paged_cache import BlockTable

    runs = []
    for kind, pool in (("bf16", None), ("fp8", fp8_pool)):
        graphs = DecodeAttentionGraphs(cache, QWEN["query_heads"], pool=pool, sizes=(1, 8), max_tokens=32768)
        rng = np.random.default_rng(11)
        free = [b for b in rng.permutation(cache.allocator.num_blocks).tolist() if b not in graphs.scratch_blocks]
        for batch, tokens in ((1, 32768), (8, 4096)):
            need = -(-tokens // 16)
            tables = [BlockTable(free[i * need : (i + 1) * need], tokens) for i in range(batch)]
            q = torch.randn(QWEN["layers"], batch, QWEN["query_heads"], QWEN["head_dim"], device=device).to(torch.bfloat16)
            k = torch.randn(QWEN["layers"], batch, QWEN["kv_heads"], QWEN["head_dim"], device=device).to(torch.bfloat16)
            graphs.run(tables, q, k, k.clone())
            size, width = graphs.size_for(batch), graphs.width_for(tables)
            timings = {}
            for mode, fn in (("graph", lambda: graphs.replay(size, width)), ("eager", lambda: graphs.step_eager(size, width))):
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(steps):
                    fn()
                end.record()
                end.synchronize()
                timings[mode] = start.elapsed_time(end) / steps
            lengths = [tokens] * batch
            kv_bytes = (decode_bytes.fp8_record_bytes_per_layer(lengths, decode_bytes.QWEN3_4B) if kind == "fp8"
                        else decode_bytes.unique_bytes_per_layer(lengths, decode_bytes.QWEN3_4B, 2))
            runs.append({
                "case": f"{kind}_batch{batch}_{tokens}",
                "graph_per_layer_us": round(timings["graph"] * 1e3 / QWEN["layers"], 2),
                "eager_per_layer_us": round(timings["eager"] * 1e3 / QWEN["layers"], 2),
                "graph_kv_gbs": round(kv_bytes / (timings["graph"] * 1e-3 / QWEN["layers"]) / 1e9, 1),
                "graph_frac_of_hbm_peak": round(kv_bytes / (timings["graph"] * 1e-3 / QWEN["layers"]) / 1e9 / HBM_PEAK_GBS, 4),
                "captured_size": size,
                "captured_width": width,
            })
        graphs.release()
        del graphs
        torch.cuda.empty_cache()
    return runs



def prefill_bench(device, layers: int = 36) -> list:
    """Paged causal prefill (Qwen3-4B heads), per layer: a 2,048-token chunk at the start of a
    sequence and at the end of a 32,768-token context, and a 512-token chunk at position 8,192
    (too few row tiles to fill the GPU, so its keys are split). Beside it, the
    reference's GPU path on this GPU (model.py:69-98): gather the history out of the pool,
    then torch's flash attention with the bottom-right causal mask. FLOPs count the causal
    score and value products: 4 x head_dim x visible keys per query row."""
    import torch

    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    runs = []
    for start, tokens in ((0, 2048), (30720, 2048), (8192, 512)):
        end = start + tokens
        blocks = -(-end // 16)
        pool = torch.empty(blocks + 1, 2, layers, QWEN["kv_heads"], 16, QWEN["head_dim"], dtype=torch.bfloat16, device=device)
        fill_pool(pool, seed=13)
        generator = torch.Generator(device=device).manual_seed(14)
        ids = torch.randperm(blocks + 1, generator=generator, device=device)[:blocks].to(torch.int32)
        q = torch.randn(QWEN["query_heads"], tokens, QWEN["head_dim"], generator=generator, device=device).to(torch.bfloat16)
        groups = QWEN["query_heads"] // QWEN["kv_heads"]
        flops = QWEN["query_heads"] * 4 * QWEN["head_dim"] * (tokens * start + tokens * (tokens + 1) // 2)

        def ours(layer):
            return paged_prefill_attention_hip(q, pool, layer, ids, start, groups)

        def gathered(layer):
            k = pool[ids.long(), 0, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :end].repeat_interleave(groups, 0)
            v = pool[ids.long(), 1, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :end].repeat_interleave(groups, 0)
            return torch.ops.aten._scaled_dot_product_flash_attention(q[None], k[None], v[None], 0.0, True)[0][0]

        row = {"case": f"chunk_{tokens}_at_{start}"}
        for name, fn in (("paged_prefill", ours), ("gather_then_torch_flash", gathered)):
            try:
                for layer in range(2):
                    fn(layer)
                torch.cuda.synchronize()
                start_event, end_event = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start_event.record()
                for layer in range(layers):
                    fn(layer)
                end_event.record()
                end_event.synchronize()
                ms = start_event.elapsed_time(end_event) / layers
                row[f"{name}_ms_per_layer"] = round(ms, 3)
                row[f"{name}_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
            except Exception as error:  # torch's flash op may be absent from a build
                row[f"{name}_error"] = repr(error)[:160]
        row["frac_of_bf16_mfma_peak"] = round(row.get("paged_prefill_tflops", 0) / 2500.0, 4)
        # The same chunk over an FP8-resident copy of the pool.
        from layover_amd.kernels.fp8 import Fp8Layout, quantize_blocks
        from layover_amd.kernels.hip_decode import Fp8KVPool

        layout = Fp8Layout.for_pool(pool)
        records = torch.empty(pool.shape[0], layout.record_bytes, dtype=torch.uint8, device=device)
        quantize_blocks(pool, torch.arange(pool.shape[0], dtype=torch.int32, device=device), records.view(-1), layout)
        fp8_pool = Fp8KVPool(records, layers, QWEN["kv_heads"], 16, QWEN["head_dim"])
        for layer in range(2):
            paged_prefill_attention_hip(q, fp8_pool, layer, ids, start, groups)
        torch.cuda.synchronize()
        start_event, end_event = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start_event.record()
        for layer in range(layers):
            paged_prefill_attention_hip(q, fp8_pool, layer, ids, start, groups)
        end_event.record()
        end_event.synchronize()
        ms = start_event.elapsed_time(end_event) / layers
        row["paged_prefill_fp8_pool_ms_per_layer"] = round(ms, 3)
        row["paged_prefill_fp8_pool_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
        runs.append(row)
        del pool, records, fp8_pool
        torch.cuda.empty_cache()
    return runs



def overlap_bench(device, cache, pool_blocks: int, swap_blocks: int = 2048, staging_bytes: int = 128 << 20, num_staging: int = 2) -> dict:
    """decode steps (batch 32, mixed contexts, BF16) on torch's stream
    while an FP8 swap of 2,048 blocks (32,768 tokens) runs on the backend's streams, then the
    swap-in. Decode reads blocks [0, pool - 2048); the swap reads from there and writes into
    the last 2048 blocks, so no decode step reads a block being restored."""
    import numpy as np
    import torch

    from layover_amd.kernels import decode_bytes, hip_decode
    from layover_amd.kv.transfer import NativeBackend

    rng = np.random.default_rng(7)
    decode_region = pool_blocks - swap_blocks
    lengths = [int(n) for n in rng.integers(1024, 32769, size=32)]
    table = torch.from_numpy(decode_tables(rng, 32, lengths, decode_region, False)).to(device)
    lens = torch.tensor(lengths, dtype=torch.int32, device=device)
    q = torch.randn(32, QWEN["query_heads"], QWEN["head_dim"], device=device).to(torch.bfloat16)
    out = torch.empty_like(q)
    groups = QWEN["query_heads"] // QWEN["kv_heads"]
    shape = hip_decode.decode_shape(q, cache.pool, 0, table, groups)
    workspace = torch.empty(hip_decode.workspace_bytes(shape), dtype=torch.uint8, device=device)
    shared = decode_bytes.sequence_blocks(lengths, QWEN["slots"]) > decode_region  # rows drawn from a smaller region share blocks
    step = lambda: decode_step_events(device, cache.pool, table, lens, q, out, workspace, groups, shared)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    solo = [step() for _ in range(5)]
    torch.cuda.synchronize()
    solo_ms = sum(s.elapsed_time(e) for s, e in solo) / len(solo)

    src = [int(i) for i in rng.choice(decode_region, swap_blocks, replace=False)]
    dst = list(range(decode_region, pool_blocks))
    backend = NativeBackend(device, staging_bytes=staging_bytes, num_staging=num_staging, ids_capacity=1 << 20)
    backend.prepare(cache, fp8=True)
    # One untimed swap of the full size, so the pinned payload comes from the engine's host
    # cache in the timed swaps (a first 2.4 GB hipHostMalloc pins pages for tens of ms).
    warm = backend.start_out(cache, src, fp8=True)
    warm.wait()
    backend.start_in(cache, dst, warm.payload).wait()
    backend.free(warm.payload)
    torch.cuda.synchronize()

    def overlapped(start_transfer):
        """Keep two decode steps queued on the compute stream while the transfer runs, and
        poll the ticket every ~0.2 ms, so the transfer's end is timed to that resolution."""
        steps = []
        t0 = time.perf_counter()
        ticket = start_transfer()
        while not ticket.done():
            pending = [e for _, e in steps[-2:] if not e.query()]
            if len(pending) < 2:
                steps.append(step())
            else:
                time.sleep(0.0002)
        elapsed = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
        return ticket, elapsed, steps

    out_ticket, out_ms, out_steps = overlapped(lambda: backend.start_out(cache, src, fp8=True))
    payload = out_ticket.payload
    in_ticket, in_ms, in_steps = overlapped(lambda: backend.start_in(cache, dst, payload))
    torch.cuda.synchronize()
    during_out = [s.elapsed_time(e) for s, e in out_steps]
    during_in = [s.elapsed_time(e) for s, e in in_steps]
    during = during_out + during_in
    backend.free(payload)
    backend.close()
    record = 1_180_800
    kv_bytes = decode_bytes.unique_bytes_per_layer(lengths, decode_bytes.QWEN3_4B, 2) * QWEN["layers"]
    overlap_ms = out_ms + in_ms
    decode_during_ms = sum(during) / max(1, len(during))
    mean = lambda xs: sum(xs) / max(1, len(xs))
    return {
        "decode_step_solo_ms": round(solo_ms, 3),
        "decode_step_during_swap_ms": round(decode_during_ms, 3),
        "decode_inflation_pct": round(100 * (decode_during_ms / solo_ms - 1), 1),
        "decode_inflation_during_swap_out_pct": round(100 * (mean(during_out) / solo_ms - 1), 1),
        "decode_inflation_during_swap_in_pct": round(100 * (mean(during_in) / solo_ms - 1), 1),
        "decode_steps_during_swap": len(during),
        "decode_steps_during_swap_out": len(during_out),
        "decode_steps_during_swap_in": len(during_in),
        "shared_blocks": shared,
        "swap_out_ms": round(out_ms, 2),
        "swap_in_ms": round(in_ms, 2),
        "swap_blocks": swap_blocks,
        "pcie_gbs": round(2 * swap_blocks * record / (overlap_ms * 1e-3) / 1e9, 2),
        "decode_hbm_gbs_during_swap": round(kv_bytes / (decode_during_ms * 1e-3) / 1e9, 1),
    }


def distinct_decode(device, steps: int) -> tuple[dict, dict]:
    """The config-3 decode on a pool with one distinct block per table entry (about 80 GB),
    so no block is read by two sequences: the sensitivity run for the 12 GiB pool's aliasing.
    Then config 4's batch 32 on FP8 records of that pool (about 40 GB more), the same rows."""
    import numpy as np
    import torch

    from layover_amd.kernels.fp8 import Fp8Layout, quantize_blocks
    from layover_amd.kernels.hip_decode import Fp8KVPool

    rng = np.random.default_rng(2)
    lengths = [int(n) for n in rng.integers(1024, 32769, size=32)]
    blocks = sum(-(-n // 16) for n in lengths)
    pool = torch.empty(blocks, 2, QWEN["layers"], QWEN["kv_heads"], 16, QWEN["head_dim"], dtype=torch.bfloat16, device=device)
    fill_pool(pool, seed=5)
    rounded = lambda run: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in run.items()}
    bf16 = decode_bench(device, pool, lengths, steps, 1, seed=3, distinct=True)
    bf16["pool_gb"] = round(pool.numel() * 2 / 1e9, 1)
    layout = Fp8Layout(16 * QWEN["head_dim"], 2 * QWEN["layers"] * QWEN["kv_heads"])
    records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device=device)
    for first in range(0, blocks, 512):
        ids = torch.arange(first, min(blocks, first + 512), dtype=torch.int32, device=device)
        quantize_blocks(pool, ids, records[first:].reshape(-1), layout)
    del pool
    torch.cuda.empty_cache()
    fp8_pool = Fp8KVPool(records, QWEN["layers"], QWEN["kv_heads"], 16, QWEN["head_dim"])
    fp8 = decode_bench(device, None, lengths, steps, 1, seed=3, distinct=True, kv_pool=fp8_pool, pool_blocks=blocks)
    fp8["pool_gb"] = round(records.numel() / 1e9, 1)
    del records, fp8_pool
    torch.cuda.empty_cache()
    return rounded(bf16), rounded(fp8)


def decode_scan(device) -> list:
    """Batch-1 decode at 1,024 ... 131,072 tokens (distinct blocks, BF16 and FP8 records): how
    the per-layer time splits into a fixed cost and a bandwidth part (`--decode-scan`)."""
    import torch

    from layover_amd.config import ModelConfig
    from layover_amd.kernels.fp8 import Fp8Layout, quantize_blocks
    from layover_amd.kernels.hip_decode import Fp8KVPool
    from layover_amd.kv.paged_cache import PagedKVCache

    blocks = 8192 + 64
    cache = PagedKVCache(ModelConfig.qwen3_4b(), blocks, device=device, fill=False)
    fill_pool(cache.pool, seed=0)
    layout = Fp8Layout.from_cache(cache)
    records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device=device)
    for first in range(0, blocks, 512):
        quantize_blocks(cache.pool, torch.arange(first, min(blocks, first + 512), dtype=torch.int32, device=device),
                        records[first:].reshape(-1), layout)
    fp8 = Fp8KVPool(records, QWEN["layers"], QWEN["kv_heads"], QWEN["slots"], QWEN["head_dim"])
    rows = []
    for tokens in (1024, 4096, 16384, 32768, 65536, 131072):
        bf16 = decode_bench(device, cache.pool, [tokens], 20, 2, seed=4, distinct=True)
        f8 = decode_bench(device, cache.pool, [tokens], 20, 2, seed=4, distinct=True, kv_pool=fp8)
        rows.append({"tokens": tokens, "bf16_us": round(bf16["per_layer_us"], 2), "bf16_frac": round(bf16["frac_of_hbm_peak"], 4),
                     "bf16_tile_probe_us": round(bf16["tile_probe_us"], 2), "fp8_us": round(f8["per_layer_us"], 2),
                     "fp8_frac": round(f8["frac_of_hbm_peak"], 4), "fp8_tile_probe_us": round(f8["tile_probe_us"], 2)})
    return rows


def duplex_bench(device, blocks: int = 2048, repeats: int = 3) -> list:
    """One session swapping out while another swaps in (`--duplex`): two backends, one per
    direction, on a 12 GiB Qwen3-4B pool, against the same two transfers one after the
    other. Copies to the host run as runtime blit kernels, copies to the device on the DMA
    engines, so PCIe can carry both directions at once when the streams involved (each
    backend's copy stream and kernel or compute stream, plus torch's) get hardware queues of
    their own; GPU_MAX_HW_QUEUES, as the process was started, is reported beside the result.
    A sample of 64 restored blocks is checked against the swapped-out source bytes (BF16) or
    against a quiet restore of the same payload (FP8). (The pool is never indexed with all
    2,048 ids at once: torch's gather over that many 2.36 MB rows of a 12 GiB pool faulted.)"""
    import numpy as np
    import torch

    from layover_amd.config import ModelConfig
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.paged_cache import PagedKVCache
    from layover_amd.kv.transfer import NativeBackend

    pool_blocks = (12 << 30) // 2_359_296
    cache = PagedKVCache(ModelConfig.qwen3_4b(), pool_blocks, device=device, fill=False)
    fill_pool(cache.pool, seed=0)
    order = np.random.default_rng(1).permutation(pool_blocks)
    leaving = [int(i) for i in order[:blocks]]
    returning = [int(i) for i in order[blocks : 2 * blocks]]
    sample = torch.tensor(returning[:: blocks // 64][:64], device=device)
    outward = NativeBackend(device, staging_bytes=128 << 20, num_staging=2)
    inward = NativeBackend(device, staging_bytes=128 << 20, num_staging=2)
    rows = []
    for fp8 in (True, False):
        for backend in (outward, inward):
            backend.prepare(cache, fp8)
        stored = inward.start_out(cache, returning, fp8)  # the session to restore
        stored.wait()
        expected = cache.pool[sample].clone()
        if fp8:  # what a restore of this payload writes, measured alone
            inward.start_in(cache, returning, stored.payload).wait()
            expected = cache.pool[sample].clone()
        sequential, concurrent = [], []
        for _ in range(repeats + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = outward.start_out(cache, leaving, fp8)
            out.wait()
            inward.start_in(cache, returning, stored.payload).wait()
            t1 = time.perf_counter()
            outward.free(out.payload)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            out = outward.start_out(cache, leaving, fp8)
            restore = inward.start_in(cache, returning, stored.payload)
            out.wait()
            restore.wait()
            t3 = time.perf_counter()
            outward.free(out.payload)
            sequential.append((t1 - t0) * 1e3)
            concurrent.append((t3 - t2) * 1e3)
        exact = bool(torch.equal(cache.pool[sample].view(torch.int16), expected.view(torch.int16)))
        inward.free(stored.payload)
        per_way = blocks * (Fp8Layout.from_cache(cache).record_bytes if fp8 else cache.block_bytes)
        best_seq, best_con = min(sequential[1:]), min(concurrent[1:])
        rows.append({"format": "fp8" if fp8 else "bf16", "blocks_each_way": blocks, "bytes_each_way": per_way,
                     "sequential_ms": round(best_seq, 2), "concurrent_ms": round(best_con, 2),
                     "concurrent_gbs_both_ways": round(2 * per_way / (best_con * 1e-3) / 1e9, 1), "restore_exact": exact})
    outward.close()
    inward.close()
    return rows


def host_cores() -> int:
    return len(os.sched_getaffinity(0))


def cpu_config1(device, blocks_in_pool: int = 4096, moved: int = 64) -> dict:
    """BASELINE configs[0] on the host cores: a 4,096-block Qwen3-4B BF16 pool (9.66 GB of host
    RAM, N(0,1), filled in 64-block slices) gathers 64 random blocks into pinned memory and
    scatters them into 64 other random ids, bit-exact. Timed on the reference's own host
    library (oracle/_ref, built from its sources) when present, and on this package's host
    flavour. The slices are drawn on the GPU (seed 0) and copied down: a NumPy fill of 4.8 G
    values would take longer than the whole bench."""
    import numpy as np
    import torch

    from layover_amd.kv.native import Engine, build_dir
    from oracle import oracle

    block = 2_359_296
    pool = np.empty(blocks_in_pool * block, dtype=np.uint8)
    generator = torch.Generator(device=device).manual_seed(0)
    for first in range(0, blocks_in_pool, 64):
        piece = torch.randn(64 * block // 2, generator=generator, device=device).to(torch.bfloat16)
        pool[first * block : (first + 64) * block] = piece.view(torch.uint8).cpu().numpy()
    rng = np.random.default_rng(0)
    order = rng.permutation(blocks_in_pool)
    src, dst = [int(i) for i in order[:moved]], [int(i) for i in order[moved : 2 * moved]]
    expected = oracle.gather(pool, block, src)
    libraries = {"package": build_dir("host") / "liblayover_transfer.so"}
    if oracle.REFERENCE_LIBRARY.exists():
        libraries["reference"] = oracle.REFERENCE_LIBRARY
    results = {}
    for name, path in libraries.items():
        engine = Engine("host", staging_bytes=128 << 20, ids_capacity=1 << 16, library=path)
        try:
            host = engine.host_alloc(moved * block)
            timings = {"out": [], "in": []}
            exact = True
            for repeat in range(4):  # the first round touches the pages and is not timed
                for i in dst:
                    pool[i * block : (i + 1) * block] = 0
                for leg, call, ids in (("out", engine.out_gather, src), ("in", engine.in_scatter, dst)):
                    t0 = time.perf_counter()
                    transfer = call(pool.ctypes.data, block, ids, host)
                    engine.wait(transfer)
                    elapsed = time.perf_counter() - t0
                    engine.release(transfer)
                    if repeat:
                        timings[leg].append(elapsed)
                exact &= bool(np.array_equal(oracle.gather(pool, block, dst), expected))
            engine.host_free(host)
        finally:
            engine.destroy()
        out_s, in_s = sorted(timings["out"])[1], sorted(timings["in"])[1]
        results[name] = {"out_ms": round(out_s * 1e3, 2), "in_ms": round(in_s * 1e3, 2),
                         "out_gbs": round(moved * block / out_s / 1e9, 2), "in_gbs": round(moved * block / in_s / 1e9, 2),
                         "bit_exact": exact}
    return {
        **results,
        "bytes_each_way": moved * block,
        "pool_blocks": blocks_in_pool,
        "threads": 2,
        "host_cores": host_cores(),
        "sample": f"{moved} of {blocks_in_pool} Qwen3-4B BF16 blocks out, then into {moved} other ids; median of 3 after one untimed round",
    }


def cpu_baseline(layout, bits, gpu_records) -> dict:
    """The CPU leg of the headline workload: the oracle's C restatement of the reference's
    quantizer (fp8.py:86-198) on the same 512 source blocks, quantize then dequantize, split
    over the host cores in threads (the ctypes calls release the GIL). Its records are also
    compared byte for byte with the GPU swap's payload: a full-size parity check."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle import oracle

    threads = min(16, host_cores())
    parts = [part for part in np.array_split(np.arange(len(bits)), threads) if len(part)]

    def leg(part):
        local = np.ascontiguousarray(bits[part])
        ids = np.arange(len(part), dtype=np.int32)
        records = oracle.quantize_records(local, ids, layout.group_elems, layout.groups_per_block)
        restored = np.zeros_like(local)
        oracle.dequantize_records(records, ids, restored, layout.group_elems, layout.groups_per_block)
        return records

    start = time.perf_counter()
    with ThreadPoolExecutor(len(parts)) as pool:
        records = list(pool.map(leg, parts))
    seconds = time.perf_counter() - start
    return {"seconds": seconds, "blocks": len(bits), "threads": len(parts),
            "records_equal_gpu_payload": bool(np.array_equal(np.concatenate(records), gpu_records))}


def calibrate_copy(device, nbytes: int = 1 << 30) -> None:
    """One plain elementwise copy of known size (read nbytes, write nbytes), so hardware
    byte counters (FETCH_SIZE, WRITE_SIZE) of the kernels above can be scaled by what the
    same counters read for a kernel whose traffic is known."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--blocks", type=int, default=512, help="blocks per swap (512 = 8,192 tokens)")
    parser.add_argument("--staging-mib", type=int, default=128)
    parser.add_argument("--decode-steps", type=int, default=5)
    parser.add_argument("--kernel-repeats", type=int, default=20, help="repeats of the step's FP8 kernel launches for the roofline")
    parser.add_argument("--skip-decode", action="store_true")
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--skip-overlap", action="store_true")
    parser.add_argument("--skip-distinct", action="store_true")
    parser.add_argument("--skip-graphs", action="store_true", help="skip the HIP-graph decode steps (rocprofv3 --pmc cannot follow replays)")
    parser.add_argument("--decode-scan", action="store_true", help="run only the batch-1 decode scan over context lengths and print it")
    parser.add_argument("--duplex", action="store_true", help="run only the concurrent swap-out + swap-in measurement and print it")
    parser.add_argument("--overlap-only", action="store_true", help="run only config 5 (decode beside a 2,048-block FP8 swap) and print it")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this KV data path has no multi-GPU step (--gpus {args.gpus} refused)", file=sys.stderr)
        raise SystemExit(2)

    import numpy as np
    import torch

    from layover_amd.config import ModelConfig
    from layover_amd.kernels.fp8 import Fp8Layout, quantize_blocks
    from layover_amd.kernels.hip_decode import Fp8KVPool
    from layover_amd.kv.paged_cache import PagedKVCache

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.decode_scan:
        print(json.dumps({"decode_scan": decode_scan(device)}), flush=True)
        return
    if args.duplex:
        queues = os.environ.get("GPU_MAX_HW_QUEUES", "unset (HIP default 4)")
        print(json.dumps({"swap_duplex": duplex_bench(device), "gpu_max_hw_queues": queues}), flush=True)
        return
    config = ModelConfig.qwen3_4b()
    block_bytes = 2 * config.num_hidden_layers * config.num_key_value_heads * 16 * config.head_dim * 2
    pool_blocks = POOL_BYTES // block_bytes
    log(f"pool: {pool_blocks} blocks of {block_bytes} B (12 GiB), filling")
    cache = PagedKVCache(config, pool_blocks, device=device, fill=False)
    fill_pool(cache.pool, seed=0, outlier_fraction=0.001)
    torch.cuda.synchronize()
    if args.overlap_only:
        log("overlap: decode during a 2,048-block FP8 swap (config 5)")
        print(json.dumps({"overlap": overlap_bench(device, cache, pool_blocks)}), flush=True)
        return

    log("link probe")
    link = measure_link(device)
    swap = swap_bench(args, device, pool_blocks, cache)
    layout = Fp8Layout.from_cache(cache)
    bytes_round_trip = 2 * swap["bytes_each_way"]
    link_peak = 1.0 / (1.0 / link["d2h_gbs"] + 1.0 / link["h2d_gbs"]) * 2  # harmonic: one out then one in
    swap_gbs = bytes_round_trip / (swap["ms_per_step"] * 1e-3) / 1e9
    q = swap["quantize"]

    result = {
        "metric": "FP8 KV swap out+in ms @8192 tok; paged decode attn achieved HBM GB/s",
        "value": round(swap["ms_per_step"], 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(swap["ms_per_step"], 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(swap["ms_per_step"] / L4_FP8_SWAP_MS, 4),
        "dtype": "bf16->fp8e4m3 (RNE codec, bit-exact)",
        "data": "synthetic: N(0,1) BF16 KV + 0.1% +/-40 outliers, seed 0; random-init Qwen3-4B KV shape",
        "config": {
            "workload": "fp8_swap_out_in_8192_tokens",
            "model_kv_shape": "Qwen3-4B (36 layers x K,V x 8 kv heads x 16 slots x 128 dims, bf16)",
            "pool_gib": 12,
            "pool_blocks": pool_blocks,
            "blocks": args.blocks,
            "tokens": args.blocks * 16,
            "staging_mib": args.staging_mib,
            "num_staging": 2,
        },
        "swap": {
            "out_ms": round(swap["out_ms"], 3),
            "in_ms": round(swap["in_ms"], 3),
            "bytes_each_way": swap["bytes_each_way"],
            "round_trip_gbs": round(swap_gbs, 2),
            "frac_of_link_peak": round(swap_gbs / link_peak, 4),
            "parity": f"bit-exact vs oracle on {swap['parity_sample_records']} sampled records and their restored blocks",
            "segments_per_direction": swap["segments_per_direction"],
        },
        "link": {"d2h_gbs": round(link["d2h_gbs"], 2), "h2d_gbs": round(link["h2d_gbs"], 2), "probe_bytes": link["bytes"],
                 "kind": "pinned hipMemcpyAsync, measured in this run"},
        "roofline": {
            "kernel": "quantize_groups_2048 (fused gather + FP8 quantize)",
            "bound": "hbm",
            "achieved": round(q["achieved_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(q["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": round(q["bytes_per_launch"] * QUANTIZE_TRAFFIC_RATIO),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE (x2) and WRITE_SIZE (x1) per dispatch of this command, "
                              f"{QUANTIZE_TRAFFIC_RATIO} x algorithmic bytes; profiles/quantize_dequantize_fp8_swap_qwen3_4b.md",
            "bytes_per_launch": q["bytes_per_launch"],
            "mean_launch_us": round(q["mean_ms"] * 1e3, 2),
            "launches": q["launches"],
        },
        "dequantize_kernel": {"achieved_gbs": round(swap["dequantize"]["achieved_gbs"], 1),
                              "mean_launch_us": round(swap["dequantize"]["mean_ms"] * 1e3, 2),
                              "frac": round(swap["dequantize"]["achieved_gbs"] / HBM_PEAK_GBS, 4)},
    }

    log("swap bf16 (the same 512 blocks, raw)")
    result["swap_bf16"] = bf16_swap_bench(args, device, pool_blocks, cache)

    if not args.skip_decode:
        rng = np.random.default_rng(2)
        mixed = [int(n) for n in rng.integers(1024, 32769, size=32)]
        log("decode bf16 (config 3)")
        decode = decode_bench(device, cache.pool, mixed, args.decode_steps, 1, seed=3)
        # Config 3 as stated: rows drawn from the 12 GiB pool, so they share blocks and some
        # reads are served by the Infinity Cache. The headline `decode` is the distinct-block
        # run below (every byte from DRAM); this one is kept beside it.
        result["decode_aliased"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in decode.items()}
        result["decode_aliased"]["lengths"] = "U[1024, 32768], batch 32, seed 2; rows sampled from the 12 GiB pool (blocks alias across rows)"
        log("decode fp8 records (config 4)")
        records = torch.empty(pool_blocks, layout.record_bytes, dtype=torch.uint8, device=device)
        for first in range(0, pool_blocks, 512):
            ids = torch.arange(first, min(pool_blocks, first + 512), dtype=torch.int32, device=device)
            quantize_blocks(cache.pool, ids, records[first:].reshape(-1), layout)
        fp8_pool = Fp8KVPool(records, config.num_hidden_layers, config.num_key_value_heads, 16, config.head_dim)
        fp8_runs = []
        for name, lengths in (("batch32_mixed_aliased", mixed), ("batch1_32768", [32768]), ("batch64_4096", [4096] * 64)):
            run = decode_bench(device, cache.pool, lengths, args.decode_steps, 1, seed=4, kv_pool=fp8_pool)
            fp8_runs.append({"case": name, **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in run.items()}})
        result["decode_fp8"] = fp8_runs
        if not args.skip_graphs:
            log("decode steps as HIP graph replays (batch 1 and 8)")
            result["decode_graphs"] = graph_decode_bench(device, cache, fp8_pool)
        del records, fp8_pool
        torch.cuda.empty_cache()

    if not args.skip_decode:
        log("paged prefill (2,048-token chunks)")
        result["prefill"] = prefill_bench(device)
    if not args.skip_decode and not args.skip_overlap:
        log("overlap: decode during a 2,048-block FP8 swap (config 5)")
        # Right after the prefill leg's second of matrix-core work, copies to the host run at
        # half rate beside decode for about the next 100 ms (measured on MI355X: the first
        # 2,048-block swap-out 83 ms, every later one 45 ms; a 2 s idle pause removes it), a
        # power-state transient rather than a property of the data path.
        torch.cuda.synchronize()
        time.sleep(2.0)
        result["overlap"] = overlap_bench(device, cache, pool_blocks)
    if not args.skip_decode and not args.skip_distinct:
        log("decode on distinct blocks (~80 GB pool)")
        bf16_distinct, fp8_distinct = distinct_decode(device, args.decode_steps)
        bf16_distinct["lengths"] = "U[1024, 32768], batch 32, seed 2; every table entry a distinct block (no Infinity Cache reuse)"
        result["decode"] = bf16_distinct
        result["decode_fp8"].insert(0, {"case": "batch32_mixed", **fp8_distinct})
    elif "decode_aliased" in result:
        result["decode"] = result["decode_aliased"]

    # Last, so its 12 GiB of buffers come and go after everything timed above.
    log("HBM probe")
    launch_bytes = int(result["roofline"]["bytes_per_launch"]) if "roofline" in result else 0
    result["hbm_probe"] = {k: round(v, 1) for k, v in measure_hbm(device, launch_bytes=launch_bytes).items()}
    result["hbm_probe"]["kind"] = (
        "lk_stream_probe: read 8 GiB; copy 4 GiB (8 GiB of traffic); lk_stream_probe_mix: 8 GiB read + 4 GiB written "
        "(quantize's 2:1), 4 GiB read + 8 GiB written (dequantize's 1:2); *_mix_launch_gbs: the same mixes at one "
        "record launch's traffic per launch (launch_bytes), 100 launches over fresh slices"
    )
    if "roofline" in result:
        # The quantize kernel against the measured ceiling for its own read/write mix, streamed
        # and at its own launch size.
        result["hbm_probe"]["quantize_frac_of_mix"] = round(result["roofline"]["achieved"] / result["hbm_probe"]["quantize_mix_gbs"], 3)
        result["hbm_probe"]["quantize_frac_of_launch_mix"] = round(
            result["roofline"]["achieved"] / result["hbm_probe"]["quantize_mix_launch_gbs"], 3
        )
    if "dequantize_kernel" in result:
        result["hbm_probe"]["dequantize_frac_of_mix"] = round(
            result["dequantize_kernel"]["achieved_gbs"] / result["hbm_probe"]["dequantize_mix_gbs"], 3
        )
        if "dequantize_mix_launch_gbs" in result["hbm_probe"]:
            result["hbm_probe"]["dequantize_frac_of_launch_mix"] = round(
                result["dequantize_kernel"]["achieved_gbs"] / result["hbm_probe"]["dequantize_mix_launch_gbs"], 3
            )

    if not args.skip_cpu:
        log(f"cpu baseline: oracle FP8 quantize+dequantize of all {args.blocks} blocks")
        cpu = cpu_baseline(layout, swap["source_bits"], swap["gpu_records"])
        result["cpu_baseline"] = {
            "value": round(cpu["seconds"] * 1e3, 1),
            "unit": "ms",
            "cores": cpu["threads"],
            "host_cores": host_cores(),
            "kind": "port",
            "sample": f"oracle C quantize+dequantize of all {cpu['blocks']} swapped Qwen3-4B blocks in {cpu['threads']} threads; "
                      "arithmetic only, no host copies",
        }
        result["swap"]["parity_full"] = ("all 512 records bit-exact vs the oracle" if cpu["records_equal_gpu_payload"]
                                         else "MISMATCH against the oracle")
        log("config 1: BF16 gather/scatter on the host libraries, 4,096-block pool")
        result["cpu_config1"] = cpu_config1(device)
    calibrate_copy(device)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
