"""Swap side of the placement cost model, measured through this package's transfer path.

The reference prices keeping, swapping or dropping a paused session's KV from polynomials
fitted by bench/kv_crossover.py (read by layover/agent/cost_model.py:42-95). This module
measures the swap half of that file on MI355X, with the same protocol:
  - one cache sized to exactly `tokens` tokens, every block round-tripped once, out in one
    random permutation of the pool and back into another (kv_crossover.py:187-220), so the
    copy order is unrelated to pool order, as after evictions;
  - BF16 first, then FP8 (whose round trip changes the values), each verified: BF16 bit for
    bit, FP8 within round_trip_bound;
  - each repeat timed with the device synchronized on both sides (kv_crossover.py:77-82),
    leading repeats discarded, medians kept;
  - linear fits with non-negative coefficients, low order first (kv_crossover.py:282-299),
    under the reference's key names: swap_out_s_coef, swap_in_s_coef, fp8_swap_out_s_coef,
    fp8_swap_in_s_coef, with transfer = "native".

Recompute time needs the model's prefill, which this package does not have; `--merge` writes
these swap coefficients into a cost model JSON the reference's own sweep produced, keeping
its recompute_s_coef, so CostModel.from_json(path, transfer="native") loads the result.

    python -m layover_amd.kv.swap_costs --device cuda --out swap_costs
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import time
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np
import torch

from layover_amd.config import ModelConfig
from layover_amd.kernels.fp8 import Fp8Layout, round_trip_within_bound
from layover_amd.kv.paged_cache import PagedKVCache
from layover_amd.kv.transfer import NativeBackend

DEFAULT_TOKENS = [512, 1024, 2048, 4096, 8192, 16384, 32768]
SWAP_KEYS = ("swap_out_s_coef", "swap_in_s_coef", "fp8_swap_out_s_coef", "fp8_swap_in_s_coef")


@dataclass
class Row:
    tokens: int
    blocks: int
    bf16_bytes: int
    fp8_bytes: int
    swap_out_s: float
    swap_in_s: float
    fp8_swap_out_s: float | None
    fp8_swap_in_s: float | None
    cold_pins: int


def sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def timed(device: torch.device, fn) -> float:
    sync(device)
    start = time.perf_counter()
    fn()
    sync(device)
    return time.perf_counter() - start


def permutation(blocks: int, seed: int) -> list[int]:
    return torch.randperm(blocks, generator=torch.Generator().manual_seed(seed)).tolist()


def fit_nonnegative(x: np.ndarray, y: np.ndarray, degree: int) -> list[float]:
    """Least-squares polynomial, low order first, whose coefficients are all >= 0: a term that
    comes out negative is dropped and the rest refitted (kv_crossover.py:282-299). A negative
    term would let the fit call a long context cheap once extrapolated."""
    powers = list(range(degree + 1))
    while True:
        design = np.stack([x.astype(np.float64) ** p for p in powers], axis=1)
        coef = np.linalg.lstsq(design, y.astype(np.float64), rcond=None)[0]
        if (coef >= 0).all() or len(powers) == 1:
            break
        powers.pop(int(np.argmin(coef)))
    result = [0.0] * (degree + 1)
    for power, value in zip(powers, coef):
        result[power] = max(float(value), 0.0)
    return result


def round_trip(backend: NativeBackend, cache: PagedKVCache, fp8: bool, seed: int) -> tuple[float, float]:
    """Every block of the cache out and back once; returns (out seconds, in seconds)."""
    device = cache.device
    blocks = cache.allocator.num_blocks
    source, target = permutation(blocks, seed), permutation(blocks, seed + 1)
    before = cache.pool[torch.tensor(source, device=device)]
    tickets = []

    def out():
        tickets.append(backend.start_out(cache, source, fp8))
        tickets[-1].wait()

    def into():
        backend.start_in(cache, target, tickets[0].payload).wait()

    out_s = timed(device, out)
    in_s = timed(device, into)
    after = cache.pool[torch.tensor(target, device=device)]
    if fp8:
        if not round_trip_within_bound(before, after, Fp8Layout.from_cache(cache).group_elems, ignore_nonfinite=True):
            raise RuntimeError("KV values left the FP8 error bound across the swap round trip")
    elif not torch.equal(before.view(torch.int16), after.view(torch.int16)):
        raise RuntimeError("KV bytes changed across the swap round trip")
    backend.free(tickets[0].payload)
    return out_s, in_s


def measure(cfg: ModelConfig, tokens: int, backend: NativeBackend, device: torch.device, fp8: bool, repeats: int,
            warmup: int, seed: int) -> Row:
    cache = PagedKVCache(cfg, -(-tokens // 16), device, fill=False)
    out_b, in_b, out_f, in_f = [], [], [], []
    pins_at_start = 0
    for i in range(warmup + repeats):
        if i == warmup:
            pins_at_start = backend.pin_stats().get("host_pins", 0)
        generator = torch.Generator(device=device).manual_seed(seed + i)
        cache.pool.copy_(torch.randn(cache.pool.shape, generator=generator, device=device, dtype=torch.float32))
        samples = [round_trip(backend, cache, False, seed + i)]
        if fp8:
            samples.append(round_trip(backend, cache, True, seed + i))
        if i >= warmup:
            out_b.append(samples[0][0])
            in_b.append(samples[0][1])
            if fp8:
                out_f.append(samples[1][0])
                in_f.append(samples[1][1])
    blocks = cache.allocator.num_blocks
    layout = Fp8Layout.from_cache(cache)
    return Row(
        tokens=tokens,
        blocks=blocks,
        bf16_bytes=blocks * cache.block_bytes,
        fp8_bytes=blocks * layout.record_bytes,
        swap_out_s=statistics.median(out_b),
        swap_in_s=statistics.median(in_b),
        fp8_swap_out_s=statistics.median(out_f) if fp8 else None,
        fp8_swap_in_s=statistics.median(in_f) if fp8 else None,
        cold_pins=backend.pin_stats().get("host_pins", 0) - pins_at_start,
    )


def describe(rows: list[Row], args: argparse.Namespace, device: torch.device, backend: NativeBackend, complete: bool) -> dict:
    x = np.array([r.tokens for r in rows])
    fits = {
        "swap_out_s_coef": fit_nonnegative(x, np.array([r.swap_out_s for r in rows]), 1),
        "swap_in_s_coef": fit_nonnegative(x, np.array([r.swap_in_s for r in rows]), 1),
    }
    if args.offload_dtype == "fp8":
        fits["fp8_swap_out_s_coef"] = fit_nonnegative(x, np.array([r.fp8_swap_out_s for r in rows]), 1)
        fits["fp8_swap_in_s_coef"] = fit_nonnegative(x, np.array([r.fp8_swap_in_s for r in rows]), 1)
    pins = backend.pin_stats()
    return {
        "model": args.model,
        "dtype": "bf16",
        "transfer": "native",
        "offload_dtype": args.offload_dtype,
        "device": device.type,
        "device_name": torch.cuda.get_device_name(device) if device.type == "cuda" else "cpu",
        "measured_on_gpu": device.type == "cuda",
        "complete": complete,
        "staging_mib": args.staging_mib,
        "repeats": args.repeats,
        "warmup": args.warmup,
        "cold_pins_in_kept_repeats": sum(r.cold_pins for r in rows),
        "host_pins": pins.get("host_pins", 0),
        "host_pin_gib": pins.get("host_pin_bytes", 0) / 2**30,
        **fits,
        "rows": [asdict(r) for r in rows],
    }


def merge(swap: dict, cost_model: Path) -> dict:
    """A reference cost model JSON with its swap coefficients replaced by these measurements;
    recompute_s_coef and everything else of it kept."""
    if not swap["complete"]:
        raise ValueError("a truncated sweep is never merged into a cost model")
    merged = json.loads(cost_model.read_text())
    for key in SWAP_KEYS:
        if key in swap:
            merged[key] = swap[key]
    merged["transfer"] = "native"
    merged["offload_dtype"] = swap["offload_dtype"]
    merged["measured_on_gpu"] = bool(merged.get("measured_on_gpu")) and swap["measured_on_gpu"]
    merged["swap_device_name"] = swap["device_name"]
    return merged


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--model", default="qwen3_4b", choices=["qwen3_4b", "micro"])
    p.add_argument("--device", default="cuda", choices=["cpu", "cuda"])
    p.add_argument("--offload-dtype", default="fp8", choices=["bf16", "fp8"], help="also measure FP8 offload")
    p.add_argument("--staging-mib", type=int, default=128)
    p.add_argument("--host-cache-mib", type=int, default=8192)
    p.add_argument("--tokens", type=int, nargs="+")
    p.add_argument("--repeats", type=int, default=5)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--out", type=Path, default=Path("results/swap_costs"))
    p.add_argument("--merge", type=Path, help="a cost_model.json from the reference's kv_crossover to update")
    return p.parse_args(argv)


def main(argv=None) -> dict:
    args = parse_args(argv)
    device = torch.device(args.device)
    if device.type == "cuda" and not torch.cuda.is_available():
        raise SystemExit("--device cuda requested but no GPU is available")
    if args.offload_dtype == "fp8" and device.type != "cuda":
        raise SystemExit("FP8 offload runs on the GPU kernels only")
    cfg = ModelConfig.qwen3_4b() if args.model == "qwen3_4b" else ModelConfig.micro()
    tokens = args.tokens or DEFAULT_TOKENS
    backend = NativeBackend(device, staging_bytes=args.staging_mib << 20, host_cache_bytes=args.host_cache_mib << 20)
    # First-use work (staging, streams, FP8 stages) is not what a copy costs.
    idle = PagedKVCache(cfg, 1, device)
    backend.prepare(idle, False)
    if args.offload_dtype == "fp8":
        backend.prepare(idle, True)
    del idle

    args.out.mkdir(parents=True, exist_ok=True)
    partial = args.out / "swap_costs.partial.json"
    rows: list[Row] = []
    for n in tokens:
        rows.append(measure(cfg, n, backend, device, args.offload_dtype == "fp8", args.repeats, args.warmup, args.seed))
        r = rows[-1]
        fp8_text = f"  fp8 out {r.fp8_swap_out_s * 1e3:8.2f} ms in {r.fp8_swap_in_s * 1e3:8.2f} ms" if r.fp8_swap_out_s is not None else ""
        print(f"{n:>6} tokens  {r.bf16_bytes / 2**30:7.3f} GiB  bf16 out {r.swap_out_s * 1e3:8.2f} ms in {r.swap_in_s * 1e3:8.2f} ms{fp8_text}", flush=True)
        with (args.out / "swap_costs.csv").open("w", newline="") as f:
            writer = csv.DictWriter(f, fieldnames=list(asdict(rows[0])))
            writer.writeheader()
            writer.writerows(asdict(row) for row in rows)
        partial.write_text(json.dumps(describe(rows, args, device, backend, False), indent=2) + "\n")
    meta = describe(rows, args, device, backend, True)
    backend.close()
    (args.out / "swap_costs.json").write_text(json.dumps(meta, indent=2) + "\n")
    partial.unlink()
    if args.merge is not None:
        (args.out / "cost_model.json").write_text(json.dumps(merge(meta, args.merge), indent=2) + "\n")
    if meta["cold_pins_in_kept_repeats"]:
        print(f"WARNING: {meta['cold_pins_in_kept_repeats']} host pins inside kept repeats; raise --host-cache-mib", flush=True)
    if not meta["measured_on_gpu"]:
        print("WARNING: not a GPU measurement; do not use these numbers as results.")
    return meta


if __name__ == "__main__":
    main()
