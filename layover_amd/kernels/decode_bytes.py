"""Bytes one paged-decode launch moves, for the rooflines of the decode kernels.

Restates the reference's accounting (bench/decode_bandwidth.py:125-139, pinned by
tests/test_decode_bandwidth.py:29-41): a row of n tokens reads ceil(n / slots) whole blocks,
the last one whole even when partly empty; "loaded" bytes count each block once per query
head (what the reference's Triton kernel issues, GQA re-reads included); "unique" bytes count
it once per KV head, which is what the HIP kernel reads (one K/V tile feeds every query head
of its group). FP8 records add the two groups' int16 shifts per (block, KV head). The launch
total adds q read, out written (both [batch, query_heads, head_dim]), the table and lengths.
"""

from __future__ import annotations

from dataclasses import dataclass

KV_KINDS = 2
SHIFT_BYTES = 2  # one little-endian int16 per FP8 group


@dataclass(frozen=True)
class KVShape:
    """The head geometry of a paged pool (reference bench/decode_bandwidth.py KVShape)."""

    query_heads: int
    kv_heads: int
    slots: int
    head_dim: int

    @property
    def kv_groups(self) -> int:
        return self.query_heads // self.kv_heads


QWEN3_4B = KVShape(query_heads=32, kv_heads=8, slots=16, head_dim=128)


def sequence_blocks(lengths, slots: int) -> int:
    """Table entries the lengths cover: ceil(n / slots) per row."""
    return sum(-(-int(n) // slots) for n in lengths)


def bytes_loaded_per_layer(lengths, shape: KVShape, element_size: int) -> int:
    """K and V bytes of one layer counted once per query head (the reference's 'loaded')."""
    return sequence_blocks(lengths, shape.slots) * shape.query_heads * KV_KINDS * shape.slots * shape.head_dim * element_size


def unique_bytes_per_layer(lengths, shape: KVShape, element_size: int) -> int:
    """K and V bytes of one layer counted once per KV head (the reference's 'unique')."""
    return bytes_loaded_per_layer(lengths, shape, element_size) // shape.kv_groups


def fp8_record_bytes_per_layer(lengths, shape: KVShape) -> int:
    """Unique bytes of one layer read from FP8 records: per (block, KV head), a K and a V group
    of slots x head_dim E4M3 codes, each with its int16 shift."""
    return sequence_blocks(lengths, shape.slots) * shape.kv_heads * KV_KINDS * (shape.slots * shape.head_dim + SHIFT_BYTES)


def launch_bytes(lengths, shape: KVShape, kv_format: str, q_element_size: int, table_width: int) -> int:
    """Algorithmic bytes of one decode launch: the unique K/V bytes ('bf16' pool, 'f32' pool or
    'fp8' records) plus q read and out written, the [batch, table_width] int32 table and the
    int32 lengths."""
    if kv_format == "fp8":
        kv = fp8_record_bytes_per_layer(lengths, shape)
    else:
        kv = unique_bytes_per_layer(lengths, shape, {"bf16": 2, "f32": 4}[kv_format])
    batch = len(lengths)
    return kv + 2 * batch * shape.query_heads * shape.head_dim * q_element_size + batch * table_width * 4 + batch * 4
