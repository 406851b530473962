"""Swap side of the placement cost model, measured through this package's transfer path.

The reference prices keeping, swapping or dropping a paused session's KV from polynomials
fitted by bench/kv_crossover.py and read by layover/agent/cost_model.py:42-95. This module
measures the swap half on MI355X and writes it under the reference's key names
(swap_out_s_coef, swap_in_s_coef, fp8_swap_out_s_coef, fp8_swap_in_s_coef; transfer =
"native"), seconds = c0 + c1 * tokens. What is measured, per context length:

- a cache of exactly that many tokens, every block swapped out in one random order and back
  into another (as after evictions, copy order unrelated to pool order; the reference's
  protocol, kv_crossover.py:187-220), BF16 and then FP8;
- each direction timed on the host with the device idle on both sides, so host-side costs
  (pinning, launches) count, as they do for a scheduler; leading repeats are discarded and
  the median of the rest kept;
- every round trip checked: BF16 bit for bit, FP8 within round_trip_bound.

The fit is a non-negative least-squares line (a negative term would make a long context look
cheap once extrapolated). Recompute time needs the model's prefill, which this package does
not have: `--merge` writes these coefficients into a cost model JSON from the reference's own
sweep and keeps its recompute_s_coef, so CostModel.from_json(path, transfer="native") loads it.

    python -m layover_amd.kv.swap_costs --device cuda --out swap_costs
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import time
from contextlib import contextmanager
from pathlib import Path

import numpy as np
import torch
from scipy.optimize import nnls

from layover_amd.config import ModelConfig
from layover_amd.kernels.fp8 import Fp8Layout, round_trip_within_bound
from layover_amd.kv.paged_cache import PagedKVCache
from layover_amd.kv.transfer import NativeBackend

DEFAULT_TOKENS = [512, 1024, 2048, 4096, 8192, 16384, 32768]
SWAP_KEYS = ("swap_out_s_coef", "swap_in_s_coef", "fp8_swap_out_s_coef", "fp8_swap_in_s_coef")
ROW_FIELDS = ("tokens", "blocks", "bf16_bytes", "fp8_bytes", "swap_out_s", "swap_in_s", "fp8_swap_out_s", "fp8_swap_in_s", "cold_pins")


def fit_nonnegative(x: np.ndarray, y: np.ndarray, degree: int) -> list[float]:
    """Coefficients (low order first) of the polynomial of `degree` closest to y in least
    squares among those with no negative coefficient (Lawson-Hanson NNLS). Columns are scaled
    to unit norm first: x^0 and x^1 over token counts differ by four orders of magnitude."""
    x = np.asarray(x, dtype=np.float64)
    design = np.stack([x**power for power in range(degree + 1)], axis=1)
    norms = np.linalg.norm(design, axis=0)
    norms[norms == 0] = 1.0
    scaled, _ = nnls(design / norms, np.asarray(y, dtype=np.float64))
    return [float(c) for c in scaled / norms]


class Sweep:
    """Swap timings for one model shape through one NativeBackend."""

    def __init__(self, cfg: ModelConfig, backend: NativeBackend, device: torch.device, with_fp8: bool, repeats: int, warmup: int,
                 seed: int):
        self.cfg, self.backend, self.device = cfg, backend, device
        self.with_fp8, self.repeats, self.warmup, self.seed = with_fp8, repeats, warmup, seed

    @contextmanager
    def _stopwatch(self, into: list[float]):
        """Appends the seconds of the block to `into`, the device drained on both sides."""
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        started = time.perf_counter_ns()
        yield
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        into.append((time.perf_counter_ns() - started) * 1e-9)

    def _orders(self, blocks: int, draw: int) -> tuple[list[int], list[int]]:
        rng = np.random.default_rng([self.seed, draw])
        return rng.permutation(blocks).tolist(), rng.permutation(blocks).tolist()

    def _round_trip(self, cache: PagedKVCache, fp8: bool, draw: int, outs: list[float], ins: list[float]) -> None:
        source, target = self._orders(cache.allocator.num_blocks, draw)
        before = self._rows(cache, source)
        with self._stopwatch(outs):
            offload = self.backend.start_out(cache, source, fp8)
            offload.wait()
        with self._stopwatch(ins):
            self.backend.start_in(cache, target, offload.payload).wait()
        after = self._rows(cache, target)
        self.backend.free(offload.payload)
        group = Fp8Layout.from_cache(cache).group_elems
        for old, new in zip(before, after):
            if fp8 and not round_trip_within_bound(old, new, group, ignore_nonfinite=True):
                raise RuntimeError("KV values left the FP8 error bound across the swap round trip")
            if not fp8 and not torch.equal(old.view(torch.int16), new.view(torch.int16)):
                raise RuntimeError("KV bytes changed across the swap round trip")

    def _rows(self, cache: PagedKVCache, ids: list[int]) -> list[torch.Tensor]:
        """The pool blocks `ids`, gathered 256 at a time: a single torch gather of a whole
        32,768-token context (2,048 blocks, 2.4 G values) is more than its kernels should be
        asked for in one call."""
        return [cache.pool[torch.tensor(ids[i : i + 256], device=self.device)] for i in range(0, len(ids), 256)]

    def row(self, tokens: int) -> dict:
        cache = PagedKVCache(self.cfg, -(-tokens // 16), self.device, fill=False)
        times: dict[tuple[str, str], list[float]] = {(fmt, way): [] for fmt in ("bf16", "fp8") for way in ("out", "in")}
        pins_before_kept = None
        for draw in range(self.warmup + self.repeats):
            kept = draw >= self.warmup
            if kept and pins_before_kept is None:
                pins_before_kept = self.backend.pin_stats().get("host_pins", 0)
            generator = torch.Generator(device=self.device).manual_seed(self.seed + draw)
            cache.pool.copy_(torch.randn(cache.pool.shape, generator=generator, device=self.device, dtype=torch.float32))
            for fmt in ("bf16", "fp8") if self.with_fp8 else ("bf16",):
                sink_out, sink_in = (times[fmt, "out"], times[fmt, "in"]) if kept else ([], [])
                self._round_trip(cache, fmt == "fp8", draw, sink_out, sink_in)
        median = lambda key: statistics.median(times[key]) if times[key] else None  # noqa: E731
        blocks = cache.allocator.num_blocks
        return {
            "tokens": tokens,
            "blocks": blocks,
            "bf16_bytes": blocks * cache.block_bytes,
            "fp8_bytes": blocks * Fp8Layout.from_cache(cache).record_bytes,
            "swap_out_s": median(("bf16", "out")),
            "swap_in_s": median(("bf16", "in")),
            "fp8_swap_out_s": median(("fp8", "out")),
            "fp8_swap_in_s": median(("fp8", "in")),
            "cold_pins": self.backend.pin_stats().get("host_pins", 0) - (pins_before_kept or 0),
        }


def summary(rows: list[dict], args: argparse.Namespace, device: torch.device, backend: NativeBackend, complete: bool) -> dict:
    tokens = np.array([r["tokens"] for r in rows])
    keys = SWAP_KEYS if args.offload_dtype == "fp8" else SWAP_KEYS[:2]
    coefficients = {key: fit_nonnegative(tokens, np.array([r[key.removesuffix("_coef")] for r in rows]), 1) for key in keys}
    pins = backend.pin_stats()
    on_gpu = device.type == "cuda"
    return {
        "model": args.model,
        "dtype": "bf16",
        "transfer": "native",
        "offload_dtype": args.offload_dtype,
        "device_name": torch.cuda.get_device_name(device) if on_gpu else "cpu",
        "measured_on_gpu": on_gpu,
        "complete": complete,
        "staging_mib": args.staging_mib,
        "repeats_kept": args.repeats,
        "repeats_discarded": args.warmup,
        "host_pins_during_kept_repeats": sum(r["cold_pins"] for r in rows),
        "host_pinned_gib": pins.get("host_pin_bytes", 0) / 2**30,
        **coefficients,
        "rows": rows,
    }


def merge(swap: dict, cost_model: Path) -> dict:
    """A reference cost model JSON with its swap coefficients replaced by these measurements,
    recompute_s_coef and everything else of it kept. A truncated sweep is refused, and a CPU
    sweep never turns a GPU cost model into a GPU one."""
    if not swap["complete"]:
        raise ValueError("a truncated sweep is never merged into a cost model")
    merged = json.loads(cost_model.read_text())
    merged.update({key: swap[key] for key in SWAP_KEYS if key in swap})
    merged.update(transfer="native", offload_dtype=swap["offload_dtype"], swap_device_name=swap["device_name"],
                  measured_on_gpu=bool(merged.get("measured_on_gpu")) and swap["measured_on_gpu"])
    return merged


def parse_args(argv=None) -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--model", default="qwen3_4b", choices=["qwen3_4b", "micro"])
    parser.add_argument("--device", default="cuda", choices=["cpu", "cuda"])
    parser.add_argument("--offload-dtype", default="fp8", choices=["bf16", "fp8"], help="fp8 also measures FP8 records")
    parser.add_argument("--staging-mib", type=int, default=128)
    parser.add_argument("--host-cache-mib", type=int, default=8192)
    parser.add_argument("--tokens", type=int, nargs="+", default=DEFAULT_TOKENS)
    parser.add_argument("--repeats", type=int, default=5, help="repeats kept (medians)")
    parser.add_argument("--warmup", type=int, default=1, help="leading repeats discarded")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--out", type=Path, default=Path("results/swap_costs"))
    parser.add_argument("--merge", type=Path, help="a cost_model.json from the reference's kv_crossover to update")
    return parser.parse_args(argv)


def _write_rows(path: Path, rows: list[dict]) -> None:
    with path.open("w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=ROW_FIELDS)
        writer.writeheader()
        writer.writerows(rows)


def main(argv=None) -> dict:
    args = parse_args(argv)
    device = torch.device(args.device)
    if device.type == "cuda" and not torch.cuda.is_available():
        raise SystemExit("--device cuda requested but no GPU is available")
    if args.offload_dtype == "fp8" and device.type != "cuda":
        raise SystemExit("FP8 offload runs on the GPU kernels only")
    cfg = ModelConfig.qwen3_4b() if args.model == "qwen3_4b" else ModelConfig.micro()
    backend = NativeBackend(device, staging_bytes=args.staging_mib << 20, host_cache_bytes=args.host_cache_mib << 20)
    # Staging, streams and FP8 stages made ahead, so no timed copy pays for first use.
    warm = PagedKVCache(cfg, 1, device)
    for fp8 in (False, True) if args.offload_dtype == "fp8" else (False,):
        backend.prepare(warm, fp8)
    del warm

    sweep = Sweep(cfg, backend, device, args.offload_dtype == "fp8", args.repeats, args.warmup, args.seed)
    args.out.mkdir(parents=True, exist_ok=True)
    in_progress = args.out / "swap_costs.partial.json"
    rows: list[dict] = []
    for tokens in args.tokens:
        rows.append(sweep.row(tokens))
        r = rows[-1]
        line = f"{tokens:>6} tokens  {r['bf16_bytes'] / 2**30:7.3f} GiB  bf16 out {r['swap_out_s'] * 1e3:8.2f} ms  in {r['swap_in_s'] * 1e3:8.2f} ms"
        if r["fp8_swap_out_s"] is not None:
            line += f"  fp8 out {r['fp8_swap_out_s'] * 1e3:8.2f} ms  in {r['fp8_swap_in_s'] * 1e3:8.2f} ms"
        print(line, flush=True)
        _write_rows(args.out / "swap_costs.csv", rows)
        in_progress.write_text(json.dumps(summary(rows, args, device, backend, False), indent=2) + "\n")
    result = summary(rows, args, device, backend, True)
    backend.close()
    (args.out / "swap_costs.json").write_text(json.dumps(result, indent=2) + "\n")
    in_progress.unlink()
    if args.merge is not None:
        (args.out / "cost_model.json").write_text(json.dumps(merge(result, args.merge), indent=2) + "\n")
    if result["host_pins_during_kept_repeats"]:
        print(f"note: {result['host_pins_during_kept_repeats']} host pins inside kept repeats; a larger --host-cache-mib avoids them")
    if not result["measured_on_gpu"]:
        print("note: a CPU sweep (host flavour), not a GPU measurement")
    return result


if __name__ == "__main__":
    main()
