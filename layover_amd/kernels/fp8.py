"""FP8 E4M3 records of KV blocks on MI355X.

Drop-in for the reference's layover/kernels/fp8.py call sites: Fp8Layout (fp8.py:58-80),
quantize_blocks / dequantize_blocks (fp8.py:349-384) and the elementwise codec used by its
exhaustive tests (encode_bits_triton / decode_bits_triton, fp8.py:319-329). The arithmetic is
the reference's integer codec (fp8.py:86-137), run as gfx950 HIP kernels
(layover_amd/csrc/fp8_codec.h) through liblayover_kernels.so. Kernels are enqueued on the
current torch stream and return immediately.

There is no CPU implementation of the codec here: a pool that is not on a GPU is refused,
and a missing kernel library raises. (The CPU restatement used to check these kernels is test
infrastructure in oracle/.) group_shifts and round_trip_bound are plain torch on any device:
they price a round trip's error, as the reference's swap measurement does when it verifies an
FP8 swap (bench/kv_crossover.py:213-216).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from layover_amd.kernels import _lib

FP8_NAN = 0x7F
BF16_MAX_FINITE = 0x7F7F
BF16_NAN = 0x7FC0


@dataclass(frozen=True)
class Fp8Layout:
    """Sizes of one stored block, as data then shifts (fp8.py:58-80)."""

    group_elems: int
    groups_per_block: int

    @classmethod
    def from_cache(cls, cache) -> "Fp8Layout":
        cfg = cache.cfg
        return cls(cache.block_tokens * cfg.head_dim, 2 * cfg.num_hidden_layers * cfg.num_key_value_heads)

    @classmethod
    def for_pool(cls, pool: torch.Tensor) -> "Fp8Layout":
        """From a pool shaped [block, 2, layers, kv_heads, slots, dim]."""
        _, kinds, layers, kv_heads, slots, dim = pool.shape
        return cls(slots * dim, kinds * layers * kv_heads)

    @property
    def block_elems(self) -> int:
        return self.group_elems * self.groups_per_block

    @property
    def header_bytes(self) -> int:
        return 2 * self.groups_per_block

    @property
    def record_bytes(self) -> int:
        return self.block_elems + self.header_bytes


def _require_gpu(*tensors: torch.Tensor) -> None:
    for tensor in tensors:
        if tensor.device.type != "cuda":
            raise ValueError(f"the HIP FP8 kernels need GPU tensors, got one on {tensor.device}")
    if len({t.device for t in tensors}) != 1:
        raise ValueError("tensors span devices")


def _check_records(pool: torch.Tensor, ids: torch.Tensor, stage: torch.Tensor, layout: Fp8Layout) -> None:
    if pool.dtype != torch.bfloat16:
        raise ValueError(f"FP8 offload needs a BF16 pool, not {pool.dtype}")
    if ids.dtype != torch.int32 or ids.dim() != 1 or not ids.is_contiguous():
        raise ValueError("ids must be a contiguous 1-D int32 tensor")
    if stage.dtype != torch.uint8 or not stage.is_contiguous():
        raise ValueError("stage must be contiguous uint8")
    if not pool.is_contiguous():
        raise ValueError("the pool must be contiguous")
    if pool.numel() % layout.block_elems:
        raise ValueError(f"a pool of {pool.numel()} values is not whole blocks of {layout.block_elems}")
    if stage.numel() < ids.shape[0] * layout.record_bytes:
        raise ValueError(f"stage of {stage.numel()} bytes cannot hold {ids.shape[0]} records of {layout.record_bytes}")
    _require_gpu(pool, ids, stage)


def quantize_blocks(pool: torch.Tensor, ids: torch.Tensor, stage: torch.Tensor, layout: Fp8Layout, impl: str | None = None) -> None:
    """Write one record per block ids[i] of a BF16 pool to the front of `stage` (fp8.py:349-367).

    ids is int32 on the pool's device; stage is uint8 on the pool's device. Enqueued on the
    current stream."""
    if impl not in (None, "hip"):
        raise ValueError(f"this build has only the 'hip' FP8 implementation, not {impl!r}")
    _check_records(pool, ids, stage, layout)
    if ids.shape[0] == 0:
        return
    lib = _lib.load()
    _lib.check(
        lib.lk_fp8_quantize(pool.data_ptr(), ids.data_ptr(), ids.shape[0], stage.data_ptr(), layout.group_elems,
                            layout.groups_per_block, _lib.current_stream(pool.device))
    )


def dequantize_blocks(stage: torch.Tensor, ids: torch.Tensor, pool: torch.Tensor, layout: Fp8Layout, impl: str | None = None) -> None:
    """Restore the first len(ids) records of `stage` into the pool's blocks `ids` (fp8.py:370-384)."""
    if impl not in (None, "hip"):
        raise ValueError(f"this build has only the 'hip' FP8 implementation, not {impl!r}")
    _check_records(pool, ids, stage, layout)
    if ids.shape[0] == 0:
        return
    lib = _lib.load()
    _lib.check(
        lib.lk_fp8_dequantize(stage.data_ptr(), ids.data_ptr(), ids.shape[0], pool.data_ptr(), layout.group_elems,
                              layout.groups_per_block, _lib.current_stream(pool.device))
    )


def encode_bits_hip(bits: torch.Tensor, shift: int = 0) -> torch.Tensor:
    """BF16 bit patterns (uint16, 1-D, on the GPU) to E4M3 bytes at one shift (fp8.py:319-323)."""
    _require_gpu(bits)
    bits = bits.contiguous()
    out = torch.empty(bits.shape[0], dtype=torch.uint8, device=bits.device)
    _lib.check(_lib.load().lk_fp8_encode(bits.data_ptr(), out.data_ptr(), bits.shape[0], shift, _lib.current_stream(bits.device)))
    return out


def decode_bits_hip(codes: torch.Tensor, shift: int = 0) -> torch.Tensor:
    """E4M3 bytes to BF16 bit patterns (uint16) at one shift (fp8.py:326-329)."""
    _require_gpu(codes)
    codes = codes.contiguous()
    out = torch.empty(codes.shape[0], dtype=torch.uint16, device=codes.device)
    _lib.check(_lib.load().lk_fp8_decode(codes.data_ptr(), out.data_ptr(), codes.shape[0], shift, _lib.current_stream(codes.device)))
    return out


def group_shifts(bits: torch.Tensor) -> torch.Tensor:
    """Per-group shift of BF16 bit patterns shaped [..., group_elems] (fp8.py:86-92): the largest
    raw exponent among finite values with a nonzero exponent field, minus 134; 0 without one."""
    raw = (bits.view(torch.int16).to(torch.int32) >> 7) & 0xFF
    raw = torch.where(raw == 0xFF, torch.zeros_like(raw), raw)
    largest = raw.amax(dim=-1)
    return torch.where(largest > 0, largest - 134, torch.zeros_like(largest))


def round_trip_bound(bits: torch.Tensor, shifts: torch.Tensor | None = None) -> torch.Tensor:
    """Largest absolute error an FP8 round trip may leave on each value, float64, for BF16 bit
    patterns shaped [..., group_elems] (fp8.py:140-152).

    A value whose exponent minus the shift is at least -6 lands on an E4M3 normal, whose 3
    stored bits round to within 1/16 of the value; below that it lands on the subnormal grid of
    spacing 2^(shift-9), so within half of it. Nothing is ever required below 2^-126, the
    smallest BF16 normal, since decoding flushes there."""
    shifts = group_shifts(bits) if shifts is None else shifts
    shifts = shifts.to(torch.int32)[..., None]
    wide = bits.view(torch.int16).to(torch.int32)
    exponent = ((wide >> 7) & 0xFF) - 127
    magnitude = bits.view(torch.bfloat16).to(torch.float64).abs()
    absolute = torch.pow(2.0, (shifts - 10).to(torch.float64)).expand_as(magnitude)
    bound = torch.where(exponent - shifts >= -6, magnitude / 16, absolute)
    return bound.clamp_min(2.0**-126)


def round_trip_within_bound(before: torch.Tensor, after: torch.Tensor, group_elems: int, ignore_nonfinite: bool = False,
                            slice_blocks: int = 16) -> bool:
    """Whether BF16 blocks [block, ...] came back from an FP8 round trip within round_trip_bound
    (fp8.py:155-176). Works a few blocks at a time, on whatever device the tensors are on;
    groups never span blocks, so slicing leaves every shift unchanged. ignore_nonfinite skips
    values that were infinite or NaN before the trip."""
    for start in range(0, before.shape[0], slice_blocks):
        bits = before[start : start + slice_blocks].contiguous().view(torch.uint16).reshape(-1, group_elems)
        values = bits.view(torch.bfloat16).to(torch.float64)
        gap = (after[start : start + slice_blocks].to(torch.float64).reshape(-1, group_elems) - values).abs()
        within = gap <= round_trip_bound(bits)
        if not bool((within[values.isfinite()] if ignore_nonfinite else within).all()):
            return False
    return True
