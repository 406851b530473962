"""The decode byte accounting every decode roofline in bench.py uses, pinned with the reference's
known answers (tests/test_decode_bandwidth.py:29-41) and with counts done by hand."""

import numpy as np

from layover_amd.kernels import decode_bytes as db

QWEN = db.QWEN3_4B


def test_qwen3_4b_block_matches_the_kv_arithmetic():
    # One layer's slice of a block is K + V for 8 KV heads: 2 * 8 * 16 * 128 * 2 B; 36 layers
    # make the 2,359,296-byte block of the reference's pool.
    assert db.unique_bytes_per_layer([16], QWEN, 2) * 36 == 2_359_296
    assert QWEN.kv_groups == 4


def test_bytes_loaded_counts_query_heads_kinds_and_whole_blocks():
    # The reference's cases: 40 tokens is 3 blocks, 1 token is 1 block, 8 KiB per block per
    # query head at BF16, and all 32 query heads load it.
    assert db.bytes_loaded_per_layer([40, 1], QWEN, 2) == 4 * 32 * 8192
    assert db.bytes_loaded_per_layer([32], QWEN, 2) == 2 * 32 * 8192
    assert db.bytes_loaded_per_layer([33], QWEN, 2) == 3 * 32 * 8192


def test_unique_bytes_remove_only_gqa_re_reads():
    loaded = db.bytes_loaded_per_layer([40, 1], QWEN, 2)
    assert db.unique_bytes_per_layer([40, 1], QWEN, 2) == loaded // QWEN.kv_groups == 4 * 8 * 8192


def test_fp8_records_count_codes_and_shifts_per_kv_head():
    # 3 blocks x 8 KV heads x (K, V) x (2,048 codes + a 2-byte shift).
    assert db.fp8_record_bytes_per_layer([40], QWEN) == 3 * 8 * 2 * 2050
    # Half the BF16 bytes plus the shifts, exactly.
    lengths = [1, 16, 17, 32768]
    blocks = db.sequence_blocks(lengths, 16)
    assert db.fp8_record_bytes_per_layer(lengths, QWEN) == db.unique_bytes_per_layer(lengths, QWEN, 2) // 2 + blocks * 8 * 2 * 2


def test_launch_bytes_add_q_out_table_and_lengths():
    # Batch 2, width 3: q and out 2 x 32 x 128 BF16 each, table 6 int32, lengths 2 int32.
    kv = db.unique_bytes_per_layer([40, 1], QWEN, 2)
    assert db.launch_bytes([40, 1], QWEN, "bf16", 2, 3) == kv + 2 * (2 * 32 * 128 * 2) + 6 * 4 + 2 * 4
    assert db.launch_bytes([40, 1], QWEN, "fp8", 4, 3) == db.fp8_record_bytes_per_layer([40, 1], QWEN) + 2 * (2 * 32 * 128 * 4) + 32


def test_the_bench_geometries_by_brute_force():
    # Config 3's lengths (seed 2, the bench's draw): count every (row, block, KV head, kind)
    # tile the kernel reads one by one, against the closed form; about 2.16 GB per layer.
    rng = np.random.default_rng(2)
    lengths = [int(n) for n in rng.integers(1024, 32769, size=32)]
    tiles = 0
    for n in lengths:
        for token0 in range(0, n, 16):
            tiles += 8 * 2  # KV heads x kinds, whole 16-slot tiles
    assert db.unique_bytes_per_layer(lengths, QWEN, 2) == tiles * 16 * 128 * 2
    assert 2.0e9 < tiles * 4096 < 2.3e9
    assert db.fp8_record_bytes_per_layer(lengths, QWEN) == tiles * 2050
    # Config 4's two fixed cases: batch 1 at 32,768 tokens and batch 64 at 4,096.
    assert db.fp8_record_bytes_per_layer([32768], QWEN) == 2048 * 8 * 2 * 2050 == 67_174_400
    assert db.fp8_record_bytes_per_layer([4096] * 64, QWEN) == 537_395_200
