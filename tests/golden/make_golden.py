"""Writes the frozen vectors of tests/golden from the oracle (oracle/kv_oracle.c), on fixed
seeded inputs:

  records_micro.npz  a BF16 pool of a small shape (2 layers, 2 KV heads, 16 slots, 24 dims;
                     special values in one block), the ids swapped out, the FP8 records
                     (fp8.py:58-80 layout) and the pool restored from them into other ids.
  decode_micro.npz   a Qwen3-shaped head (16 slots x 128 dims, GQA 4) with ragged lengths:
                     q, pool, table, lengths and the float64 decode attention output, for the
                     BF16 pool and for the pool's FP8 records (attention over their decoded
                     values).

The inputs are stored, not re-drawn, so the vectors stay fixed whatever numpy's generators
do later. tests/test_golden.py checks that the oracle still gives these outputs (on the CPU)
and that the HIP kernels do (on the GPU). Run from the repository root:

    python3 tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import oracle  # noqa: E402

RECORD_SHAPE = dict(layers=2, kv_heads=2, slots=16, head_dim=24)
RECORD_BLOCKS = 6
DECODE_SHAPE = dict(layers=1, kv_heads=2, slots=16, head_dim=128)
DECODE_GROUPS = 4
DECODE_LAYER = 0
DECODE_LENGTHS = [1, 17, 33]


def pool_bits(rng, blocks, layers, kv_heads, slots, head_dim):
    values = rng.standard_normal((blocks, 2, layers, kv_heads, slots, head_dim), dtype=np.float32)
    values *= np.exp(rng.standard_normal(values.shape, dtype=np.float32))
    return oracle.bf16_bits(values)


def records_micro() -> dict:
    rng = np.random.default_rng(11)
    s = RECORD_SHAPE
    bits = pool_bits(rng, RECORD_BLOCKS, **s)
    flat = bits.reshape(RECORD_BLOCKS, -1)
    flat[2, :8] = [0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC1, 0x7F7F]
    flat[4, 100:104] = [0x4780, 0xC700, 0x3C00, 0x0080]  # a group with a wide exponent spread
    group_elems = s["slots"] * s["head_dim"]
    groups = 2 * s["layers"] * s["kv_heads"]
    ids = np.array([4, 0, 2, 5], dtype=np.int32)
    records = oracle.quantize_records(bits, ids, group_elems, groups)
    target = np.array([1, 3, 0, 2], dtype=np.int32)
    restored = np.zeros_like(bits)
    oracle.dequantize_records(records, target, restored, group_elems, groups)
    return dict(pool=bits, ids=ids, records=records, target_ids=target, restored=restored,
                group_elems=np.int64(group_elems), groups_per_block=np.int64(groups))


def decode_micro() -> dict:
    rng = np.random.default_rng(12)
    s = DECODE_SHAPE
    width = max(-(-n // s["slots"]) for n in DECODE_LENGTHS)
    blocks = len(DECODE_LENGTHS) * width + 1
    bits = oracle.bf16_bits(rng.standard_normal((blocks, 2, s["layers"], s["kv_heads"], s["slots"], s["head_dim"]), dtype=np.float32))
    table = rng.permutation(blocks)[: len(DECODE_LENGTHS) * width].reshape(len(DECODE_LENGTHS), width).astype(np.int32)
    q = oracle.bf16_bits(rng.standard_normal((len(DECODE_LENGTHS), s["kv_heads"] * DECODE_GROUPS, s["head_dim"]), dtype=np.float32))
    lengths = np.array(DECODE_LENGTHS, dtype=np.int32)
    out = oracle.decode_attention(q, bits, DECODE_LAYER, table, lengths, DECODE_GROUPS)

    group_elems = s["slots"] * s["head_dim"]
    groups = 2 * s["layers"] * s["kv_heads"]
    all_ids = np.arange(blocks, dtype=np.int32)
    records = oracle.quantize_records(bits, all_ids, group_elems, groups)
    decoded = np.zeros_like(bits)
    oracle.dequantize_records(records, all_ids, decoded, group_elems, groups)
    out_fp8 = oracle.decode_attention(q, decoded, DECODE_LAYER, table, lengths, DECODE_GROUPS)
    return dict(q=q, pool=bits, table=table, lengths=lengths, out=out, records=records, out_fp8=out_fp8,
                layer=np.int64(DECODE_LAYER), groups=np.int64(DECODE_GROUPS))


def main() -> None:
    oracle.build()
    np.savez_compressed(HERE / "records_micro.npz", **records_micro())
    np.savez_compressed(HERE / "decode_micro.npz", **decode_micro())
    for name in ("records_micro.npz", "decode_micro.npz"):
        print(name, (HERE / name).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
