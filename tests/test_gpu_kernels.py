"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI wrappers.

FP8: bit-exact (every BF16 pattern x every shift the computed scale can produce, and whole
records at the Qwen3-4B and micro shapes). Decode: within the north-star tolerance
(2e-2 abs / 1e-2 rel at BF16) of the float64 oracle, and much tighter in practice: the
asserted bound is the BF16 rounding of the exact answer plus a small FP32 allowance.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

QWEN = dict(layers=36, kv_heads=8, slots=16, head_dim=128)


@pytest.fixture(scope="module")
def fp8():
    from layover_amd.kernels import fp8 as module

    return module


@pytest.fixture(scope="module")
def hip_decode():
    from layover_amd.kernels import hip_decode as module

    return module


def test_kernel_library_loads_into_torchs_hip_runtime():
    from layover_amd.kernels import _lib
    from layover_amd.kv.native import hip_runtimes_loaded, load_library

    torch.zeros(1, device="cuda")
    lib = _lib.load()
    assert lib.lk_abi_version() == 3
    assert load_library("hip").lt_flavor() == b"hip"
    assert len(hip_runtimes_loaded()) == 1, hip_runtimes_loaded()


# FP8 codec: every pattern at every shift.

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
ALL_FP8 = np.arange(256, dtype=np.uint32).astype(np.uint8)


def test_encode_is_bit_exact_for_every_pattern_and_every_shift(fp8):
    bits = torch.from_numpy(ALL_BF16.view(np.int16)).cuda().view(torch.uint16)
    for shift in range(-133, 121):
        got = fp8.encode_bits_hip(bits, shift).cpu().numpy()
        expected = oracle.encode(ALL_BF16, shift)
        assert np.array_equal(got, expected), f"shift {shift}: {np.flatnonzero(got != expected)[:8]}"


def test_decode_is_bit_exact_for_every_code_and_every_shift(fp8):
    codes = torch.from_numpy(ALL_FP8).cuda()
    for shift in range(-140, 128):
        got = fp8.decode_bits_hip(codes, shift).cpu().numpy()
        assert np.array_equal(got, oracle.decode(ALL_FP8, shift)), f"shift {shift}"


def make_pool(blocks, layers, kv_heads, slots, head_dim, seed=0, outliers=0.0):
    rng = np.random.default_rng(seed)
    values = rng.standard_normal((blocks, 2, layers, kv_heads, slots, head_dim), dtype=np.float32)
    values *= np.exp(rng.standard_normal(values.shape, dtype=np.float32))
    if outliers:
        mask = rng.random(values.shape) < outliers
        values[mask] = np.where(rng.random(mask.sum()) < 0.5, -40.0, 40.0)
    return oracle.bf16_bits(values)


@pytest.mark.parametrize(
    "shape",
    [dict(QWEN, blocks=24), dict(layers=2, kv_heads=2, slots=16, head_dim=24, blocks=9), dict(layers=1, kv_heads=1, slots=16, head_dim=128, blocks=5)],
    ids=["qwen3_4b", "micro", "one_group_pow2"],
)
def test_records_are_bit_exact_and_restore_bit_exact(fp8, shape):
    blocks = shape.pop("blocks")
    bits = make_pool(blocks, **shape, seed=1, outliers=0.001)
    # Special values in one block: zeros, subnormals, infinities, NaN, the largest finite.
    special = bits.reshape(blocks, -1)
    special[1, :8] = [0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC1, 0x7F7F]
    layout = fp8.Fp8Layout(shape["slots"] * shape["head_dim"], 2 * shape["layers"] * shape["kv_heads"])
    ids = np.random.default_rng(2).permutation(blocks)[: blocks - 2].astype(np.int32)
    expected = oracle.quantize_records(bits, ids, layout.group_elems, layout.groups_per_block)

    pool = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    stage = torch.full((expected.size + 64,), 0xAB, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, torch.from_numpy(ids).cuda(), stage, layout)
    got = stage.cpu().numpy()
    assert np.array_equal(got[: expected.size], expected)
    assert (got[expected.size :] == 0xAB).all()

    target_ids = np.random.default_rng(3).permutation(blocks)[: len(ids)].astype(np.int32)
    restored = torch.zeros_like(pool)
    fp8.dequantize_blocks(stage, torch.from_numpy(target_ids).cuda(), restored, layout)
    reference = np.zeros_like(bits)
    oracle.dequantize_records(expected, target_ids, reference, layout.group_elems, layout.groups_per_block)
    assert np.array_equal(restored.view(torch.int16).cpu().numpy().view(np.uint16), reference)


def crafted_groups(group=2048):
    """Groups that reach every finite BF16 pattern at every shift the computed scale can take:
    for each largest exponent m (shift m - 134), one pinned 2^(m-127) followed by every
    pattern whose exponent is at most m, zero-padded (zeros leave the shift unchanged)."""
    raw = (ALL_BF16 >> 7) & 0xFF
    groups = []
    for m in range(1, 255):
        patterns = ALL_BF16[(raw <= m)]
        per = group - 1
        for start in range(0, patterns.size, per):
            chunk = patterns[start : start + per]
            g = np.zeros(group, dtype=np.uint16)
            g[0] = m << 7
            g[1 : 1 + chunk.size] = chunk
            groups.append(g)
    # Groups with infinities and NaN (the exact fallback), and all-zero / all-subnormal groups.
    for special in ([0x7F80, 0x3F80, 0xBC00], [0xFF80, 0x0001, 0x8005], [0x7FC1, 0x4000], [0x0000], [0x0001, 0x807F, 0x8000]):
        g = np.resize(np.array(special, dtype=np.uint16), group)
        groups.append(g)
    return np.stack(groups)


def test_record_fast_paths_are_bit_exact_for_every_pattern_at_every_shift(fp8):
    groups = crafted_groups()
    per_block = 576
    blocks = -(-groups.shape[0] // per_block)
    bits = np.zeros((blocks * per_block, 2048), dtype=np.uint16)
    bits[: groups.shape[0]] = groups
    bits = bits.reshape(blocks, -1)
    layout = fp8.Fp8Layout(2048, per_block)
    ids = np.arange(blocks, dtype=np.int32)[::-1].copy()
    expected = oracle.quantize_records(bits, ids, layout.group_elems, layout.groups_per_block)
    pool = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    stage = torch.zeros(expected.size, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, torch.from_numpy(ids).cuda(), stage, layout)
    got = stage.cpu().numpy()
    mismatch = np.flatnonzero(got != expected)
    assert mismatch.size == 0, f"{mismatch.size} bytes differ, first at {mismatch[:4]}"
    restored = torch.zeros_like(pool)
    fp8.dequantize_blocks(stage, torch.from_numpy(ids).cuda(), restored, layout)
    reference = np.zeros_like(bits)
    oracle.dequantize_records(expected, ids, reference, layout.group_elems, layout.groups_per_block)
    assert np.array_equal(restored.view(torch.int16).cpu().numpy().view(np.uint16), reference)


def test_dequantize_fast_path_is_bit_exact_for_every_code_at_every_shift(fp8):
    per_block = 576
    layout = fp8.Fp8Layout(2048, per_block)
    shifts = np.arange(-140, 128)
    finite = ALL_FP8[(ALL_FP8 & 0x7F) != 0x7F]
    groups = [np.resize(finite, 2048) for _ in shifts] + [np.resize(ALL_FP8, 2048) for _ in shifts]
    all_shifts = np.concatenate([shifts, shifts]).astype(np.int16)
    blocks = -(-len(groups) // per_block)
    data = np.zeros((blocks * per_block, 2048), dtype=np.uint8)
    data[: len(groups)] = np.stack(groups)
    header = np.zeros(blocks * per_block, dtype=np.int16)
    header[: len(groups)] = all_shifts
    records = np.concatenate([data.reshape(blocks, -1), header.reshape(blocks, per_block).view(np.uint8)], axis=1).reshape(-1)
    ids = np.arange(blocks, dtype=np.int32)
    reference = np.zeros((blocks, layout.block_elems), dtype=np.uint16)
    oracle.dequantize_records(records, ids, reference, layout.group_elems, layout.groups_per_block)
    pool = torch.zeros(blocks, layout.block_elems, dtype=torch.bfloat16, device="cuda")
    fp8.dequantize_blocks(torch.from_numpy(records).cuda(), torch.from_numpy(ids).cuda(), pool, layout)
    got = pool.view(torch.int16).cpu().numpy().view(np.uint16)
    mismatch = np.flatnonzero(got != reference)
    assert mismatch.size == 0, f"{mismatch.size} values differ, first at {mismatch[:4]}"


def test_records_address_past_4_gib(fp8):
    layout = fp8.Fp8Layout(2048, 576)
    block_bytes = 2 * layout.block_elems
    blocks = (5 << 30) // block_bytes + 2
    pool = torch.zeros(blocks, layout.block_elems, dtype=torch.bfloat16, device="cuda")
    source, target = blocks - 1, blocks - 2
    values = make_pool(1, 36, 8, 16, 128, seed=4).reshape(1, -1)
    pool[source] = torch.from_numpy(values.view(np.int16)).cuda().view(torch.bfloat16)[0]
    stage = torch.zeros(layout.record_bytes, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, torch.tensor([source], dtype=torch.int32, device="cuda"), stage, layout)
    expected = oracle.quantize_records(values, [0], layout.group_elems, layout.groups_per_block)
    assert np.array_equal(stage.cpu().numpy(), expected)
    fp8.dequantize_blocks(stage, torch.tensor([target], dtype=torch.int32, device="cuda"), pool, layout)
    reference = np.zeros_like(values)
    oracle.dequantize_records(expected, [0], reference, layout.group_elems, layout.groups_per_block)
    assert np.array_equal(pool[target].view(torch.int16).cpu().numpy().view(np.uint16), reference[0])
    del pool
    torch.cuda.empty_cache()


def test_a_non_bf16_pool_is_refused(fp8):
    layout = fp8.Fp8Layout(384, 8)
    pool = torch.zeros(2, layout.block_elems, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        fp8.quantize_blocks(pool, torch.zeros(1, dtype=torch.int32, device="cuda"), torch.zeros(layout.record_bytes, dtype=torch.uint8, device="cuda"), layout)


# Paged decode.


def decode_case(lengths, layers, kv_heads, slots, head_dim, groups, seed=0, pool_blocks=None, gain=1.0):
    rng = np.random.default_rng(seed)
    width = max(-(-n // slots) for n in lengths)
    blocks = pool_blocks or len(lengths) * width + 3
    pool = oracle.bf16_bits(rng.standard_normal((blocks, 2, layers, kv_heads, slots, head_dim), dtype=np.float32))
    if pool_blocks:
        table = np.stack([rng.choice(blocks, width, replace=False) for _ in lengths]).astype(np.int32)
    else:
        table = rng.permutation(blocks)[: len(lengths) * width].reshape(len(lengths), width).astype(np.int32)
    q = oracle.bf16_bits((gain * rng.standard_normal((len(lengths), kv_heads * groups, head_dim))).astype(np.float32))
    return q, pool, table, np.array(lengths, dtype=np.int32)


def to_gpu_bf16(bits):
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)


def weighted_mean_abs_v(q, pool_bits, layer, table, lengths, groups):
    """Per output, the attention-weighted mean of |v|: the same attention over V with its
    sign bits cleared. A kernel that rounds each weight to BF16 (8 significand bits: relative
    error at most 2^-8, reached for significands just above 1) errs by at most 2^-8 of this."""
    magnitudes = pool_bits.copy()
    magnitudes[:, 1] &= 0x7FFF
    return oracle.decode_attention(q, magnitudes, layer, table, lengths, groups)


def assert_close_to_oracle(out, expected, what="", weight_rounding=None):
    got = out.double().cpu().numpy()
    # BF16 rounding of the exact answer (2^-8 relative) plus an FP32 accumulation allowance;
    # far inside the north-star 2e-2 abs / 1e-2 rel. weight_rounding: the weighted mean of
    # |v| where the kernel feeds the weights to the matrix cores as single BF16s (FP8 pools).
    allowed = np.abs(expected) * 2.0**-8 + 1e-3
    if weight_rounding is not None:
        allowed = allowed + 2.0**-8 * weight_rounding
    error = np.abs(got - expected)
    assert np.isfinite(got).all(), what
    assert (error <= allowed).all(), f"{what}: max error {error.max():.3g} at {np.unravel_index(error.argmax(), error.shape)}"
    assert (error <= 2e-2 + 1e-2 * np.abs(expected)).all()


LENGTHS = {
    "one_token": [1],
    "block_edges": [15, 16, 17, 31, 32, 33],
    "mixed": [1, 16, 17, 47, 48, 80, 3, 64, 700, 2049],
    "long": [5000, 4096],
}


@pytest.mark.parametrize("name", LENGTHS)
@pytest.mark.parametrize("groups", [1, 2, 4, 8])
def test_decode_qwen_shape_matches_the_oracle(hip_decode, name, groups):
    lengths = LENGTHS[name]
    q, pool, table, lens = decode_case(lengths, layers=3, kv_heads=2, slots=16, head_dim=128, groups=groups, seed=groups)
    expected = oracle.decode_attention(q, pool, 1, table, lens, groups)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), to_gpu_bf16(pool), 1, torch.from_numpy(table).cuda(),
                                                torch.from_numpy(lens).cuda(), groups)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    assert_close_to_oracle(out, expected, f"{name} G={groups}")


@pytest.mark.parametrize("head_dim,slots,groups", [(24, 16, 2), (32, 7, 4), (128, 16, 3), (64, 4, 1), (256, 16, 2)])
def test_decode_other_shapes_match_the_oracle(hip_decode, head_dim, slots, groups):
    q, pool, table, lens = decode_case([1, 20, 47, 130], layers=2, kv_heads=3, slots=slots, head_dim=head_dim, groups=groups, seed=5)
    expected = oracle.decode_attention(q, pool, 0, table, lens, groups)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), to_gpu_bf16(pool), 0, torch.from_numpy(table).cuda(),
                                                torch.from_numpy(lens).cuda(), groups)
    assert_close_to_oracle(out, expected, f"D={head_dim} S={slots} G={groups}")


def test_decode_fp32_q_and_pool(hip_decode):
    q, pool, table, lens = decode_case([20, 333], layers=2, kv_heads=2, slots=16, head_dim=128, groups=4, seed=6)
    expected = oracle.decode_attention(q, pool, 1, table, lens, 4)
    qf = to_gpu_bf16(q).float()
    for pool_tensor in (to_gpu_bf16(pool), to_gpu_bf16(pool).float()):
        out = hip_decode.paged_decode_attention_hip(qf, pool_tensor, 1, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), 4)
        assert out.dtype == torch.float32
        error = np.abs(out.double().cpu().numpy() - expected)
        assert error.max() < 1e-4, (pool_tensor.dtype, error.max())


def test_decode_unwritten_slots_cannot_poison_the_result(hip_decode):
    q, pool, table, lens = decode_case([20, 3, 37], layers=2, kv_heads=2, slots=16, head_dim=128, groups=4, seed=7)
    args = lambda p: (to_gpu_bf16(q), to_gpu_bf16(p), 1, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), 4)
    clean = hip_decode.paged_decode_attention_hip(*args(pool))
    for poison in (0x7FC0, 0x7F80, 0xFF80):
        dirty = pool.copy()
        dirty[table[0, 1], :, :, :, 4:] = poison
        dirty[table[1, 0], :, :, :, 3:] = poison
        dirty[table[2, 2], :, :, :, 5:] = poison
        out = hip_decode.paged_decode_attention_hip(*args(dirty))
        assert torch.isfinite(out.float()).all()
        assert torch.equal(out, clean)


def test_decode_large_scores_and_a_moving_maximum(hip_decode):
    q, pool, table, lens = decode_case([300, 64], layers=2, kv_heads=2, slots=16, head_dim=128, groups=4, seed=8, gain=6.0)
    values = oracle.bf16_to_float(pool)
    values[:, 0] *= 6
    values[table[0, -1], 0] *= 3  # a late block with the largest scores
    pool = oracle.bf16_bits(values)
    expected = oracle.decode_attention(q, pool, 1, table, lens, 4)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), to_gpu_bf16(pool), 1, torch.from_numpy(table).cuda(),
                                                torch.from_numpy(lens).cuda(), 4)
    assert_close_to_oracle(out, expected, "large scores")


@pytest.mark.parametrize("layers", [4, 3], ids=["aligned_records", "unaligned_records"])
def test_decode_fp8_pool_matches_the_oracle_on_the_dequantized_pool(fp8, hip_decode, layers):
    kv_heads, slots, head_dim = 2, 16, 128
    q, pool, table, lens = decode_case([1, 17, 500, 1200], layers, kv_heads, slots, head_dim, groups=4, seed=9)
    blocks = pool.shape[0]
    layout = fp8.Fp8Layout(slots * head_dim, 2 * layers * kv_heads)
    records = oracle.quantize_records(pool, np.arange(blocks), layout.group_elems, layout.groups_per_block)
    dequantized = np.zeros_like(pool)
    oracle.dequantize_records(records, np.arange(blocks), dequantized, layout.group_elems, layout.groups_per_block)
    expected = oracle.decode_attention(q, dequantized, 2, table, lens, 4)
    fp8_pool = hip_decode.Fp8KVPool(torch.from_numpy(records.reshape(blocks, -1)).cuda(), layers, kv_heads, slots, head_dim)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), fp8_pool, 2, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), 4)
    # The aligned records run the matrix-core kernel, whose FP8 path rounds the weights to
    # BF16; the unaligned ones the generic FP32 kernel.
    rounding = weighted_mean_abs_v(q, dequantized, 2, table, lens, 4) if layers == 4 else None
    assert_close_to_oracle(out, expected, "fp8 records", weight_rounding=rounding)


@pytest.mark.parametrize("layers", [4, 1], ids=["fast_kernel", "generic_kernel"])
def test_decode_fp8_pool_with_extreme_shifts_uses_the_exact_decode(fp8, hip_decode, layers):
    kv_heads, slots, head_dim = 2, 16, 128
    q, pool, table, lens = decode_case([40], layers, kv_heads, slots, head_dim, groups=2, seed=10)
    values = oracle.bf16_to_float(pool)
    values[:, 0] *= 2.0**-120  # K groups with shifts near -127
    values[:, 1] *= 2.0**-115  # V groups with shifts near -120
    pool = oracle.bf16_bits(values)
    layout = fp8.Fp8Layout(slots * head_dim, 2 * layers * kv_heads)
    blocks = pool.shape[0]
    records = oracle.quantize_records(pool, np.arange(blocks), layout.group_elems, layout.groups_per_block)
    dequantized = np.zeros_like(pool)
    oracle.dequantize_records(records, np.arange(blocks), dequantized, layout.group_elems, layout.groups_per_block)
    q = oracle.bf16_bits(oracle.bf16_to_float(q) * 2.0**118)
    expected = oracle.decode_attention(q, dequantized, layers - 1, table, lens, 2)
    fp8_pool = hip_decode.Fp8KVPool(torch.from_numpy(records.reshape(blocks, -1)).cuda(), layers, kv_heads, slots, head_dim)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), fp8_pool, layers - 1, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), 2)
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all()
    rounding = 2.0**-8 * weighted_mean_abs_v(q, dequantized, layers - 1, table, lens, 2) if layers == 4 else 0.0
    assert (np.abs(got - expected) <= np.abs(expected) * 2.0**-7 + rounding + 2.0**-126).all()


@pytest.mark.parametrize(
    "mutate",
    [
        lambda c: {**c, "lengths": torch.tensor([0, 5], dtype=torch.int32, device="cuda")},
        lambda c: {**c, "lengths": torch.tensor([33, 5], dtype=torch.int32, device="cuda")},
        lambda c: {**c, "table": torch.tensor([[0, 99], [1, 2]], dtype=torch.int32, device="cuda")},
        lambda c: {**c, "table": torch.tensor([[0, -1], [1, 2]], dtype=torch.int32, device="cuda")},
        lambda c: {**c, "layer": 3},
        lambda c: {**c, "groups": 3},
        lambda c: {**c, "q": c["q"][:, :, :-1]},
        lambda c: {**c, "q": c["q"][:1]},
        lambda c: {**c, "pool": c["pool"].transpose(0, 1)},
        lambda c: {**c, "pool": c["pool"][::2]},
        lambda c: {**c, "q": c["q"].double()},
        lambda c: {**c, "pool": c["pool"].double()},
    ],
    ids=["empty_sequence", "longer_than_table", "block_past_pool", "negative_block", "layer_past_pool", "groups_disagree",
         "head_dim_disagrees", "batch_disagrees", "kinds_not_two", "non_contiguous_pool", "q_float64", "pool_float64"],
)
def test_decode_invalid_inputs_are_refused_before_launch(hip_decode, mutate):
    q, pool, table, lens = decode_case([20, 5], layers=3, kv_heads=2, slots=16, head_dim=24, groups=2, seed=41)
    good = dict(q=to_gpu_bf16(q), pool=to_gpu_bf16(pool), table=torch.from_numpy(table).cuda(), lengths=torch.from_numpy(lens).cuda(), layer=1, groups=2)
    bad = mutate(good)
    with pytest.raises(ValueError):
        hip_decode.paged_decode_attention_hip(bad["q"], bad["pool"], bad["layer"], bad["table"], bad["lengths"], bad["groups"])


def test_decode_int64_table_and_non_contiguous_q(hip_decode):
    q, pool, table, lens = decode_case([20, 40], layers=2, kv_heads=2, slots=16, head_dim=128, groups=2, seed=35)
    args = (to_gpu_bf16(pool), 1)
    expected = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), *args, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), 2)
    strided = torch.zeros(2, 8, 128, dtype=torch.bfloat16, device="cuda")
    strided[:, ::2] = to_gpu_bf16(q)
    got = hip_decode.paged_decode_attention_hip(strided[:, ::2], *args, torch.from_numpy(table).long().cuda(), torch.from_numpy(lens).long().cuda(), 2)
    assert torch.equal(got, expected)


def test_decode_block_offsets_past_32_bits(hip_decode):
    layers, kv_heads, slots, head_dim = 36, 2, 16, 128
    stride = 2 * layers * kv_heads * slots * head_dim
    blocks = 2**31 // stride + 8
    pool = torch.zeros(blocks, 2, layers, kv_heads, slots, head_dim, dtype=torch.bfloat16, device="cuda")
    q, small, _, lens = decode_case([40], layers, kv_heads, slots, head_dim, groups=1, seed=40, pool_blocks=3)
    ids = [blocks - 1, blocks - 5, 3]
    pool[torch.tensor(ids, device="cuda")] = to_gpu_bf16(small)
    out = hip_decode.paged_decode_attention_hip(to_gpu_bf16(q), pool, 7, torch.tensor([ids], dtype=torch.int32, device="cuda"),
                                                torch.from_numpy(lens).cuda(), 1)
    expected = oracle.decode_attention(q, small, 7, np.arange(3, dtype=np.int32)[None], lens, 1)
    assert_close_to_oracle(out, expected, "64-bit offsets")
    del pool
    torch.cuda.empty_cache()


@pytest.mark.parametrize("nbytes", [16, 4096, 16 * 1024, 5 * 4096 + 48, 3 << 20])
def test_stream_probe_reads_without_writing_and_copies_exactly(nbytes):
    """lk_stream_probe: a read leaves the sink alone; a copy (partial last chunk included)
    reproduces the source and writes nothing past `bytes`."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    stream = _lib.current_stream(torch.device("cuda"))
    gen = torch.Generator(device="cuda").manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=gen)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    _lib.check(lib.lk_stream_probe(src.data_ptr(), None, nbytes, sink.data_ptr(), stream))
    dst = torch.full((nbytes + 4096,), 0xA5, dtype=torch.uint8, device="cuda")
    _lib.check(lib.lk_stream_probe(src.data_ptr(), dst.data_ptr(), nbytes, sink.data_ptr(), stream))
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 0xA5).all())


@pytest.mark.parametrize("ratio", ["2:1", "1:2"])
def test_stream_probe_mix_moves_the_stated_bytes(ratio):
    """lk_stream_probe_mix: 2:1 writes, as output 8-byte word i, the two halves of input
    16-byte word i XORed; 1:2 writes input 8-byte word i twice as output 16-byte word i. A
    partial last wave writes nothing past dst_bytes, and other ratios are refused."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    stream = _lib.current_stream(torch.device("cuda"))
    words = 37 * 64 + 5
    src_bytes = words * (16 if ratio == "2:1" else 8)
    dst_bytes = src_bytes // 2 if ratio == "2:1" else src_bytes * 2
    src = torch.randint(0, 2**31, (src_bytes // 4,), dtype=torch.int32, device="cuda")
    dst = torch.full((dst_bytes // 4 + 1024,), -7, dtype=torch.int32, device="cuda")
    _lib.check(lib.lk_stream_probe_mix(src.data_ptr(), src_bytes, dst.data_ptr(), dst_bytes, stream))
    torch.cuda.synchronize()
    if ratio == "2:1":
        w = src.view(words, 4).cpu()
        expect = torch.stack([w[:, 0] ^ w[:, 2], w[:, 1] ^ w[:, 3]], dim=1)
    else:
        w = src.view(words, 2).cpu()
        expect = torch.cat([w, w], dim=1)
    assert torch.equal(dst[: dst_bytes // 4].cpu().view_as(expect), expect)
    assert bool((dst[dst_bytes // 4 :] == -7).all())
    with pytest.raises(_lib.KernelError):
        _lib.check(lib.lk_stream_probe_mix(src.data_ptr(), src_bytes, dst.data_ptr(), src_bytes, stream))


@pytest.mark.parametrize("case", ["vector_combine", "unaligned_buffers", "over_64_splits", "over_128_splits"])
def test_decode_combine_paths_match_the_oracle(hip_decode, case):
    """The split merge has a vector form (128-dim heads, at most 128 splits, 16-byte aligned
    workspace and out) and a general one. A 70,000-token row (69 splits) takes the vector
    form's second batch of loads; a workspace 4 bytes off 16-byte alignment and an out 2 bytes
    off, or a 140,000-token row (137 splits), take the general form."""
    lengths = {"over_64_splits": [70000, 3], "over_128_splits": [140000, 3]}.get(case, [5000, 17, 2100])
    q, pool, table, lens = decode_case(lengths, layers=1, kv_heads=2, slots=16, head_dim=128, groups=4, seed=len(case))
    expected = oracle.decode_attention(q, pool, 0, table, lens, 4)
    q_gpu, pool_gpu = to_gpu_bf16(q), to_gpu_bf16(pool)
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    from layover_amd.kernels import _lib

    shape = hip_decode.decode_shape(q_gpu, pool_gpu, 0, table_gpu, 4, lens_gpu)
    need = int(_lib.load().lk_paged_decode_workspace(shape))
    if case == "unaligned_buffers":
        workspace = torch.empty(need + 16, dtype=torch.uint8, device="cuda")[4 : 4 + need]
        out = torch.empty(q_gpu.numel() + 1, dtype=torch.bfloat16, device="cuda")[1:].view(q_gpu.shape)
        assert workspace.data_ptr() % 16 == 4 and out.data_ptr() % 8 == 2
    else:
        workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q_gpu)
    print(f"decode combine {case}: workspace {need} bytes", flush=True)
    hip_decode.run_kernel(q_gpu, pool_gpu, 0, table_gpu, lens_gpu, 4, out, workspace)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, expected, case)


def test_tile_probe_reads_without_writing_and_refuses_other_formats(fp8, hip_decode):
    """lk_tile_probe reads the decode's tiles (a measurement probe) from BF16 and FP8-record
    pools: the sink stays zero, and an FP32 pool is refused before launch."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    q, pool, table, lens = decode_case([40, 700], layers=3, kv_heads=8, slots=16, head_dim=128, groups=4, seed=44)
    q_gpu, pool_gpu = to_gpu_bf16(q), to_gpu_bf16(pool)
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = _lib.current_stream(q_gpu.device)
    shape = hip_decode.decode_shape(q_gpu, pool_gpu, 2, table_gpu, 4, lens_gpu)
    _lib.check(lib.lk_tile_probe(shape, pool_gpu.data_ptr(), table_gpu.data_ptr(), lens_gpu.data_ptr(), sink.data_ptr(), stream))
    layout = fp8.Fp8Layout(16 * 128, 2 * 3 * 8)
    blocks = pool.shape[0]
    records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool_gpu, torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
    fp8_pool = hip_decode.Fp8KVPool(records, 3, 8, 16, 128)
    fp8_shape = hip_decode.decode_shape(q_gpu, fp8_pool, 2, table_gpu, 4, lens_gpu)
    _lib.check(lib.lk_tile_probe(fp8_shape, records.data_ptr(), table_gpu.data_ptr(), lens_gpu.data_ptr(), sink.data_ptr(), stream))
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    wrong = hip_decode.decode_shape(q_gpu.float(), pool_gpu.float(), 2, table_gpu, 4, lens_gpu)
    assert lib.lk_tile_probe(wrong, pool_gpu.data_ptr(), table_gpu.data_ptr(), lens_gpu.data_ptr(), sink.data_ptr(), stream) == _lib.LK_ERR_INVALID


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("q_format", ["bf16", "f32"])
def test_decode_with_one_split_writes_the_output_itself_bit_for_bit(fp8, hip_decode, kv, q_format, monkeypatch):
    """Tables of one split (FP8 records: up to 64 blocks; BF16 on a grid this small: 8-block
    splits, so up to 128 tokens) skip the combine launch: the split kernel writes the output
    with the combine's arithmetic. Outputs equal the two-launch form (LAYOVER_DECODE_COMBINE)
    bit for bit, including a row whose V is all -0.0 (the combine turns -0 into +0) and ragged
    rows of one token, and stay within the oracle's tolerance."""
    from layover_amd.kernels import _lib

    lengths = [1, 16, 17, 1024, 333] if kv == "fp8" else [1, 16, 17, 128, 100]
    q, pool, table, lens = decode_case(lengths, layers=2, kv_heads=2, slots=16, head_dim=128, groups=4, seed=9)
    pool[table[1, 0], 1] = 0x8000  # row 1's only block: every V value -0.0
    q_gpu = to_gpu_bf16(q) if q_format == "bf16" else to_gpu_bf16(q).float()
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    if kv == "bf16":
        target, reference_pool = to_gpu_bf16(pool), pool
    else:
        layout = fp8.Fp8Layout(16 * 128, 2 * 2 * 2)
        blocks = pool.shape[0]
        records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
        fp8.quantize_blocks(to_gpu_bf16(pool), torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
        target = hip_decode.Fp8KVPool(records, 2, 2, 16, 128)
        reference_pool = np.zeros_like(pool)
        oracle.dequantize_records(records.cpu().numpy().reshape(-1), np.arange(blocks, dtype=np.int32), reference_pool, layout.group_elems,
                                  layout.groups_per_block)
    print(f"one-split decode {kv} q {q_format}", flush=True)
    shape = hip_decode.decode_shape(q_gpu, target, 0, table_gpu, 4, lens_gpu)
    assert _lib.load().lk_paged_decode_workspace(shape) == len(lengths) * 8 * 130 * 4  # one split
    for layer in (0, 1):
        direct = hip_decode.paged_decode_attention_hip(q_gpu, target, layer, table_gpu, lens_gpu, 4)
        monkeypatch.setenv("LAYOVER_DECODE_COMBINE", "1")
        combined = hip_decode.paged_decode_attention_hip(q_gpu, target, layer, table_gpu, lens_gpu, 4)
        monkeypatch.delenv("LAYOVER_DECODE_COMBINE")
        torch.cuda.synchronize()
        assert torch.equal(direct.view(torch.int16) if q_format == "bf16" else direct.view(torch.int32),
                           combined.view(torch.int16) if q_format == "bf16" else combined.view(torch.int32)), f"layer {layer}"
        if layer == 1:
            assert (direct[1].float() == 0).all() and not torch.signbit(direct[1].float()).any()
        expected = oracle.decode_attention(q, reference_pool, layer, table, lens, 4)
        weighted = weighted_mean_abs_v(q, reference_pool, layer, table, lens, 4) if kv == "fp8" else None
        assert_close_to_oracle(direct.float(), expected, f"{kv} layer {layer}", weight_rounding=weighted)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("q_format", ["bf16", "f32"])
@pytest.mark.parametrize("grid", ["small", "large"])
def test_streaming_and_cached_tile_loads_agree_bit_for_bit(fp8, hip_decode, kv, q_format, grid):
    """LK_DECODE_SHARED_BLOCKS switches the matrix-core kernel between two forms of its tile
    loads: streaming (K loaded in whole lines and laid out through LDS, non-temporal hints)
    and cached (K loaded in the matrix-core layout directly). The values reaching the matrix
    cores are the same, so outputs are identical, on the 8-wave kernel of small grids and the
    4-wave kernel of large ones (64 rows x 8 KV heads x 2 splits = 1,024 workgroups), with
    ragged lengths and with the fused token write. The small case is also checked against the
    oracle (the streaming form is the default every other decode test runs)."""
    from layover_amd.kernels import _lib

    layers, kv_heads, groups = 2, 8, 4
    if grid == "small":
        lengths = [1, 17, 300, 2049, 777]
        blocks = 5 * 129 + 5
    else:
        rng = np.random.default_rng(5)
        lengths = [int(n) for n in rng.integers(1, 2049, size=64)]
        lengths[0] = 2048
        blocks = 64 * 128 + 8
    gen = torch.Generator(device="cuda").manual_seed(11)
    pool = torch.randn(blocks, 2, layers, kv_heads, 16, 128, generator=gen, device="cuda").to(torch.bfloat16)
    width = max(-(-n // 16) for n in lengths)
    table = torch.randperm(blocks, generator=gen, device="cuda")[: len(lengths) * width].view(len(lengths), width).to(torch.int32)
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    q = torch.randn(len(lengths), kv_heads * groups, 128, generator=gen, device="cuda")
    q = q.to(torch.bfloat16) if q_format == "bf16" else q
    if kv == "bf16":
        target = pool
    else:
        layout = fp8.Fp8Layout(16 * 128, 2 * layers * kv_heads)
        records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
        fp8.quantize_blocks(pool, torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
        target = hip_decode.Fp8KVPool(records, layers, kv_heads, 16, 128)
    shape = hip_decode.decode_shape(q, target, 1, table, groups, lens)
    splits = int(_lib.load().lk_paged_decode_workspace(shape)) // (len(lengths) * kv_heads * groups * 130 * 4)
    if grid == "large":
        assert len(lengths) * splits * kv_heads >= 1024, splits
    print(f"streaming vs cached: {kv} q {q_format} {grid} grid, {splits} splits", flush=True)
    bits = lambda t: t.view(torch.int16) if q_format == "bf16" else t.view(torch.int32)
    outs = {}
    for shared in (False, True):
        out = torch.empty_like(q)
        hip_decode.run_kernel(q, target, 1, table, lens, groups, out, shared_blocks=shared)
        outs[shared] = out
    torch.cuda.synchronize()
    assert torch.equal(bits(outs[False]), bits(outs[True]))
    # The fused write of each row's last token (write position = the last token), both forms,
    # each on its own copy of the pool: pools and outputs equal.
    last = (lens - 1).long()
    write_blocks = table.gather(1, (last // 16).view(-1, 1)).view(-1).contiguous()
    write_slots = (last % 16).to(torch.int32).contiguous()
    k_new = torch.randn(len(lengths), kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    v_new = torch.randn(len(lengths), kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    results = {}
    for shared in (False, True):
        copy = target.clone() if kv == "bf16" else hip_decode.Fp8KVPool(target.records.clone(), layers, kv_heads, 16, 128)
        out = torch.empty_like(q)
        hip_decode.run_kernel_append(q, copy, 1, table, lens, groups, write_blocks, write_slots, k_new, v_new, out, shared_blocks=shared)
        results[shared] = (out, copy if kv == "bf16" else copy.records)
    torch.cuda.synchronize()
    assert torch.equal(bits(results[False][0]), bits(results[True][0]))
    assert torch.equal(results[False][1].view(torch.uint8), results[True][1].view(torch.uint8))
    if grid == "small" and q_format == "bf16":
        q_bits = q.cpu().view(torch.int16).numpy().view(np.uint16)
        if kv == "bf16":
            pool_bits = pool.cpu().view(torch.int16).numpy().view(np.uint16)
        else:
            pool_bits = np.zeros((blocks, 2, layers, kv_heads, 16, 128), dtype=np.uint16)
            oracle.dequantize_records(target.records.cpu().numpy().reshape(-1), np.arange(blocks, dtype=np.int32), pool_bits,
                                      16 * 128, 2 * layers * kv_heads)
        table_np, lens_np = table.cpu().numpy(), lens.cpu().numpy()
        expected = oracle.decode_attention(q_bits, pool_bits, 1, table_np, lens_np, groups)
        weighted = weighted_mean_abs_v(q_bits, pool_bits, 1, table_np, lens_np, groups) if kv == "fp8" else None
        assert_close_to_oracle(outs[False].float(), expected, f"streaming {kv}", weight_rounding=weighted)
