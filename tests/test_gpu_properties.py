"""Property tests of paged decode against the float64 oracle, over drawn shapes.

The first follows the reference's own property test (tests/test_triton_decode.py:335-353):
the same strategy space (1-3 KV heads, GQA 1/2/4, head dims 8-32 including odd ones, 4/7/16
slots, layers 0-2, q gains 0.1-8, BF16 or FP32, 1-4 rows of 1-70 tokens), which here runs
the generic kernel. The second draws the Qwen3 tile shape (16 slots x 128 dims), which runs
the matrix-core kernel, over BF16 pools and FP8 records, 1-40 rows of up to 3,000 tokens.
The third draws FP8 record layouts, alignments and counts for the swap's record kernels.
Draws are derandomized, so every run checks the same cases.
"""

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import oracle

pytestmark = pytest.mark.gpu


def to_gpu_bf16(bits):
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)


def make_case(lengths, kv_heads, groups, head_dim, slots, layers, seed, gain, pool_blocks=None):
    rng = np.random.default_rng(seed)
    width = max(-(-n // slots) for n in lengths)
    blocks = pool_blocks or len(lengths) * width + 2
    pool = oracle.bf16_bits(rng.standard_normal((blocks, 2, layers, kv_heads, slots, head_dim), dtype=np.float32))
    table = np.stack([rng.choice(blocks, width, replace=False) for _ in lengths]).astype(np.int32)
    q = oracle.bf16_bits((gain * rng.standard_normal((len(lengths), kv_heads * groups, head_dim))).astype(np.float32))
    return q, pool, table, np.array(lengths, dtype=np.int32)


def assert_close(out, expected, weighted_abs_v=None):
    """BF16 rounding of the exact answer plus an FP32 allowance (and, for FP8 records, whose
    weights reach the matrix cores as single BF16s, 2^-8 of the attention-weighted mean |v|),
    inside the north-star 2e-2 abs / 1e-2 rel."""
    got = out.double().cpu().numpy()
    allowed = np.abs(expected) * 2.0**-8 + 1e-3
    if weighted_abs_v is not None:
        allowed = allowed + 2.0**-8 * weighted_abs_v
    error = np.abs(got - expected)
    assert np.isfinite(got).all()
    assert (error <= allowed).all(), f"max error {error.max():.3g}"
    assert (error <= 2e-2 + 1e-2 * np.abs(expected)).all()


@settings(max_examples=60, deadline=None, derandomize=True)
@given(
    seed=st.integers(0, 2**16),
    kv_heads=st.sampled_from([1, 2, 3]),
    groups=st.sampled_from([1, 2, 4]),
    head_dim=st.sampled_from([8, 16, 24, 31, 32]),
    slots=st.sampled_from([4, 7, 16]),
    layer=st.integers(0, 2),
    gain=st.sampled_from([0.1, 1.0, 8.0]),
    dtype=st.sampled_from(["float32", "bfloat16"]),
    lengths=st.lists(st.integers(1, 70), min_size=1, max_size=4),
)
def test_decode_matches_the_oracle_over_the_reference_strategy(seed, kv_heads, groups, head_dim, slots, layer, gain, dtype, lengths):
    from layover_amd.kernels import hip_decode

    q, pool, table, lens = make_case(lengths, kv_heads, groups, head_dim, slots, 3, seed, gain)
    expected = oracle.decode_attention(q, pool, layer, table, lens, groups)
    q_gpu, pool_gpu = to_gpu_bf16(q), to_gpu_bf16(pool)
    if dtype == "float32":
        q_gpu, pool_gpu = q_gpu.float(), pool_gpu.float()
    print(f"property case seed {seed} kv {kv_heads} G {groups} dim {head_dim} slots {slots} {dtype} lengths {lengths}", flush=True)
    out = hip_decode.paged_decode_attention_hip(q_gpu, pool_gpu, layer, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), groups)
    assert out.dtype == q_gpu.dtype
    assert_close(out, expected)


@settings(max_examples=40, deadline=None, derandomize=True)
@given(
    seed=st.integers(0, 2**16),
    kv_heads=st.sampled_from([1, 2, 8]),
    groups=st.sampled_from([1, 2, 4, 8]),
    layer=st.integers(0, 2),
    gain=st.sampled_from([0.1, 1.0, 8.0]),
    fp8_pool=st.booleans(),
    lengths=st.lists(st.integers(1, 3000), min_size=1, max_size=40),
)
def test_decode_at_the_qwen_tile_shape_matches_the_oracle(seed, kv_heads, groups, layer, gain, fp8_pool, lengths):
    from layover_amd.kernels import fp8, hip_decode

    layers, slots, head_dim = 3, 16, 128
    q, pool, table, lens = make_case(lengths, kv_heads, groups, head_dim, slots, layers, seed, gain)
    print(f"qwen-shape case seed {seed} kv {kv_heads} G {groups} fp8 {fp8_pool} rows {len(lengths)} longest {max(lengths)}", flush=True)
    q_gpu = to_gpu_bf16(q)
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    weighted = None
    if fp8_pool:
        blocks = pool.shape[0]
        layout = fp8.Fp8Layout(slots * head_dim, 2 * layers * kv_heads)
        records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
        fp8.quantize_blocks(to_gpu_bf16(pool), torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
        target = hip_decode.Fp8KVPool(records, layers, kv_heads, slots, head_dim)
        reference = np.zeros_like(pool)
        oracle.dequantize_records(records.cpu().numpy().reshape(-1), np.arange(blocks, dtype=np.int32), reference, layout.group_elems,
                                  layout.groups_per_block)
        magnitudes = reference.copy()
        magnitudes[:, 1] &= 0x7FFF
        weighted = oracle.decode_attention(q, magnitudes, layer, table, lens, groups)
    else:
        target, reference = to_gpu_bf16(pool), pool
    expected = oracle.decode_attention(q, reference, layer, table, lens, groups)
    out = hip_decode.paged_decode_attention_hip(q_gpu, target, layer, table_gpu, lens_gpu, groups)
    assert_close(out, expected, weighted)


@settings(max_examples=40, deadline=None, derandomize=True)
@given(
    seed=st.integers(0, 2**16),
    layers=st.integers(1, 3),
    kv_heads=st.integers(1, 3),
    slots=st.sampled_from([1, 4, 7, 16]),
    head_dim=st.sampled_from([8, 24, 31, 128]),
    blocks=st.integers(1, 9),
    count=st.integers(0, 12),
    pool_offset=st.sampled_from([0, 1, 8]),
    stage_offset=st.sampled_from([0, 1, 16]),
)
def test_fp8_records_over_drawn_layouts_match_the_oracle(seed, layers, kv_heads, slots, head_dim, blocks, count, pool_offset, stage_offset):
    """Drawn block layouts (group sizes 8 to 2,048 values, odd ones included, so records and
    their shift fields need not be aligned), pools starting 0, 1 or 8 values into their
    allocation and stages 0, 1 or 16 bytes into theirs (the fast kernel only where everything
    is 16-byte aligned), 0-12 records of 1-9 blocks with ids that repeat: records bit-exact
    against the oracle (fp8.py:179-198), stage bytes outside them untouched, and the restore
    bit-exact against the oracle's dequantization into distinct ids."""
    from layover_amd.kernels import fp8

    layout = fp8.Fp8Layout(slots * head_dim, 2 * layers * kv_heads)
    block_elems = layout.block_elems
    print(f"fp8 record case: group {layout.group_elems} x {layout.groups_per_block}, {count} of {blocks}, offsets {pool_offset}/{stage_offset}",
          flush=True)
    rng = np.random.default_rng(seed)
    values = rng.standard_normal(blocks * block_elems, dtype=np.float32) * np.exp(2 * rng.standard_normal(blocks * block_elems, dtype=np.float32))
    values[rng.random(values.size) < 0.002] = 40.0
    bits = oracle.bf16_bits(values)
    bits[: min(6, bits.size)] = [0x0000, 0x8000, 0x0001, 0x7F80, 0x7FC1, 0x7F7F][: min(6, bits.size)]
    total = np.zeros(pool_offset + bits.size, dtype=np.uint16)
    total[pool_offset:] = bits
    pool_total = torch.from_numpy(total.view(np.int16)).cuda().view(torch.bfloat16)
    pool = pool_total[pool_offset:]
    ids = rng.integers(0, blocks, count).astype(np.int32)
    expected = oracle.quantize_records(bits, ids, layout.group_elems, layout.groups_per_block)

    stage_total = torch.full((stage_offset + expected.size + 32,), 0xC3, dtype=torch.uint8, device="cuda")
    stage = stage_total[stage_offset:]
    fp8.quantize_blocks(pool, torch.from_numpy(ids).cuda(), stage, layout)
    got = stage_total.cpu().numpy()
    assert np.array_equal(got[stage_offset : stage_offset + expected.size], expected)
    assert (got[:stage_offset] == 0xC3).all() and (got[stage_offset + expected.size :] == 0xC3).all()

    targets = rng.permutation(blocks)[: min(count, blocks)].astype(np.int32)
    fp8.dequantize_blocks(stage, torch.from_numpy(targets).cuda(), pool, layout)
    reference = bits.copy()
    oracle.dequantize_records(expected, targets, reference, layout.group_elems, layout.groups_per_block)
    got_pool = pool_total.view(torch.int16).cpu().numpy().view(np.uint16)
    assert (got_pool[:pool_offset] == 0).all()
    assert np.array_equal(got_pool[pool_offset:], reference)
