"""TEST INFRASTRUCTURE ONLY. numpy front end of the C oracle in kv_oracle.c.

Each function names the reference code it restates; the C file holds the arithmetic.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this.
"""

from __future__ import annotations

import ctypes
import subprocess
from ctypes import POINTER, c_double, c_int, c_int32, c_uint8, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_build" / "libkv_oracle.so"
REFERENCE_LIBRARY = HERE / "_ref" / "liblayover_transfer_ref.so"

_lib = None


def build() -> None:
    """Compile the oracle (and the reference host library where the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if Path("/root/reference/native/transfer_host.cc").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        handle.oracle_group_shift.argtypes = [c_void_p, c_uint64]
        handle.oracle_group_shift.restype = c_int32
        handle.oracle_encode.argtypes = [c_uint16, c_int32]
        handle.oracle_encode.restype = c_uint8
        handle.oracle_decode.argtypes = [c_uint8, c_int32]
        handle.oracle_decode.restype = c_uint16
        handle.oracle_encode_array.argtypes = [c_void_p, c_void_p, c_uint64, c_int32]
        handle.oracle_decode_array.argtypes = [c_void_p, c_void_p, c_uint64, c_int32]
        for name in ("oracle_quantize_records", "oracle_dequantize_records"):
            getattr(handle, name).argtypes = [c_void_p, c_void_p, c_uint32, c_void_p, c_uint64, c_uint32]
        for name in ("oracle_gather", "oracle_scatter"):
            getattr(handle, name).argtypes = [c_void_p, c_uint64, c_void_p, c_uint32, c_void_p]
        handle.oracle_decode_attention.argtypes = [
            c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_void_p, c_uint32, c_void_p,
            c_uint32, c_uint32, c_double, c_void_p,
        ]
        handle.oracle_decode_attention.restype = c_int
        _lib = handle
    return _lib


def _ptr(array: np.ndarray) -> int:
    assert array.flags.c_contiguous
    return array.ctypes.data


def group_shifts(bits: np.ndarray) -> np.ndarray:
    """fp8.py:86-92 over uint16 bits shaped [groups, group_elems]."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    groups, elems = bits.shape
    return np.array([lib().oracle_group_shift(_ptr(bits[g]), elems) for g in range(groups)], dtype=np.int32)


def encode(bits: np.ndarray, shift: int) -> np.ndarray:
    """fp8.py:95-116 elementwise at one shift."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(bits.shape, dtype=np.uint8)
    lib().oracle_encode_array(_ptr(bits), _ptr(out), bits.size, shift)
    return out


def decode(codes: np.ndarray, shift: int) -> np.ndarray:
    """fp8.py:119-137 elementwise at one shift."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    out = np.empty(codes.shape, dtype=np.uint16)
    lib().oracle_decode_array(_ptr(codes), _ptr(out), codes.size, shift)
    return out


def record_bytes(group_elems: int, groups_per_block: int) -> int:
    """fp8.py:70-80: block_elems data bytes, then 2 bytes of shift per group."""
    return group_elems * groups_per_block + 2 * groups_per_block


def quantize_records(pool_bits: np.ndarray, ids, group_elems: int, groups_per_block: int) -> np.ndarray:
    """fp8.py:179-187: one record per id, returned as a flat uint8 array."""
    pool_bits = np.ascontiguousarray(pool_bits).view(np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.zeros(len(ids) * record_bytes(group_elems, groups_per_block), dtype=np.uint8)
    lib().oracle_quantize_records(_ptr(pool_bits), _ptr(ids), len(ids), _ptr(out), group_elems, groups_per_block)
    return out


def dequantize_records(stage: np.ndarray, ids, pool_bits: np.ndarray, group_elems: int, groups_per_block: int) -> None:
    """fp8.py:190-198: restore the first len(ids) records into pool blocks ids, in place."""
    assert pool_bits.dtype == np.uint16 and pool_bits.flags.c_contiguous
    stage = np.ascontiguousarray(stage, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    lib().oracle_dequantize_records(_ptr(stage), _ptr(ids), len(ids), _ptr(pool_bits), group_elems, groups_per_block)


def gather(pool: np.ndarray, block_bytes: int, ids) -> np.ndarray:
    """pack.h:56-61 over whole blocks."""
    pool = np.ascontiguousarray(pool).view(np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.empty(len(ids) * block_bytes, dtype=np.uint8)
    lib().oracle_gather(_ptr(pool), block_bytes, _ptr(ids), len(ids), _ptr(out))
    return out


def scatter(pool: np.ndarray, block_bytes: int, ids, data: np.ndarray) -> None:
    """pack.h:63-68 over whole blocks, in place."""
    assert pool.flags.c_contiguous
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    data = np.ascontiguousarray(data).view(np.uint8)
    lib().oracle_scatter(pool.ctypes.data, block_bytes, _ptr(ids), len(ids), _ptr(data))


def append_tokens(records: np.ndarray, layers: int, kv_heads: int, slots: int, head_dim: int, write_blocks, write_slots,
                  layer: int, k_bits: np.ndarray, v_bits: np.ndarray) -> np.ndarray:
    """The FP8-resident pool's decode-time write (no reference counterpart; its BF16 analogue
    is the pool assignment of model.py:139-140), composed only of dequantize_records and
    quantize_records above: the block is dequantized, each touched group gets the new token at
    its write slot and zero after it, the block is quantized again, and only the touched
    groups' codes and shifts are copied back. records uint8 [blocks, record_bytes]; k_bits and
    v_bits uint16 [rows, kv_heads, head_dim]. Returns new records."""
    group_elems, groups_per_block = slots * head_dim, 2 * layers * kv_heads
    block_elems = group_elems * groups_per_block
    out = np.array(records, dtype=np.uint8, copy=True)
    for row, (block, slot) in enumerate(zip(np.asarray(write_blocks).tolist(), np.asarray(write_slots).tolist())):
        bits = np.zeros((1, 2, layers, kv_heads, slots, head_dim), dtype=np.uint16)
        dequantize_records(out[block], [0], bits, group_elems, groups_per_block)
        for kind, fresh in ((0, k_bits), (1, v_bits)):
            bits[0, kind, layer, :, slot, :] = fresh[row]
            bits[0, kind, layer, :, slot + 1 :, :] = 0
        again = quantize_records(bits, [0], group_elems, groups_per_block)
        for kind in (0, 1):
            for head in range(kv_heads):
                g = (kind * layers + layer) * kv_heads + head
                out[block, g * group_elems : (g + 1) * group_elems] = again[g * group_elems : (g + 1) * group_elems]
                out[block, block_elems + 2 * g : block_elems + 2 * g + 2] = again[block_elems + 2 * g : block_elems + 2 * g + 2]
    return out


def decode_attention(q: np.ndarray, pool_bits: np.ndarray, layer: int, table: np.ndarray, lengths: np.ndarray,
                     kv_groups: int, scale: float | None = None) -> np.ndarray:
    """decode_attention.py:9-37 in float64. q [batch, query_heads, dim] (any float dtype, or
    uint16 BF16 bits); pool_bits uint16 [blocks, 2, layers, kv_heads, slots, dim]."""
    if q.dtype == np.uint16:
        q = (q.astype(np.uint32) << 16).view(np.float32)
    q = np.ascontiguousarray(q, dtype=np.float64)
    pool_bits = np.ascontiguousarray(pool_bits).view(np.uint16)
    table = np.ascontiguousarray(table, dtype=np.int32)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    batch, query_heads, dim = q.shape
    _, kinds, layers, kv_heads, slots, pool_dim = pool_bits.shape
    assert kinds == 2 and pool_dim == dim and query_heads == kv_heads * kv_groups
    scale = 1.0 / np.sqrt(dim) if scale is None else scale
    out = np.zeros_like(q)
    status = lib().oracle_decode_attention(
        _ptr(q), _ptr(pool_bits), layers, kv_heads, slots, dim, layer, _ptr(table), table.shape[1], _ptr(lengths),
        batch, query_heads, scale, _ptr(out),
    )
    if status:
        raise ValueError(f"oracle refused the case (status {status})")
    return out


def prefill_attention(q: np.ndarray, pool_bits: np.ndarray, layer: int, block_ids, start: int, kv_groups: int) -> np.ndarray:
    """Causal chunked prefill (model.py:69-98: query t of the chunk sees keys up to start + t),
    composed from decode_attention above: query token t is one decode step of length
    start + t + 1 over the same blocks. q [query_heads, tokens, dim] (float or BF16 bits);
    returns float64 [query_heads, tokens, dim]."""
    heads, tokens, dim = q.shape
    table = np.asarray(block_ids, dtype=np.int32)[None]
    out = np.zeros((heads, tokens, dim), dtype=np.float64)
    for t in range(tokens):
        out[:, t] = decode_attention(q[:, t][None], pool_bits, layer, table, np.array([start + t + 1]), kv_groups)[0]
    return out


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> BF16 bits, rounding to nearest even (NaN becomes 0x7FC0)."""
    wide = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((wide + 0x7FFF + ((wide >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(values, dtype=np.float32))
    rounded[nan] = 0x7FC0
    return rounded


def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
