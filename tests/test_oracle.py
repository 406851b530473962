"""Pins the CPU oracle (oracle/kv_oracle.c) before anything is checked against it.

Every check here is independent of the oracle's own formulas: torch's float8_e4m3fn casts
(a library routine), the reference's known answers (tests/test_fp8.py:62-153 of the
reference), the round-trip error bound stated in layover/kernels/fp8.py:25-27, exact
power-of-two scaling done in float64, and decode attention against torch's float64
scaled_dot_product_attention and a pure-Python softmax.
"""

import math

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import oracle

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
ALL_FP8 = np.arange(256, dtype=np.uint32).astype(np.uint8)
SHIFTS = [-133, -117, -40, -7, 0, 5, 40, 119, 120]


def torch_fp8_of_float(values: np.ndarray) -> np.ndarray:
    return torch.from_numpy(values.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()


def fp8_values(codes: np.ndarray) -> np.ndarray:
    return torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).to(torch.float64).numpy()


# Codec against torch at shift 0 (reference test_fp8.py:40-59).


def test_encode_matches_torch_on_every_bf16_pattern():
    encoded = oracle.encode(ALL_BF16, 0)
    values = bf16_values(ALL_BF16)
    nan, inf = np.isnan(values), np.isinf(values)
    too_big = np.abs(np.where(nan, 0, values)) > 464.0
    reference = torch.from_numpy(ALL_BF16.view(np.int16)).view(torch.bfloat16).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    in_range = ~nan & ~inf & ~too_big
    assert in_range.sum() > 30000
    assert np.array_equal(encoded[in_range], reference[in_range])
    assert np.array_equal(encoded[nan], reference[nan])
    sign = ((ALL_BF16 >> 15).astype(np.uint8) << 7)
    assert np.array_equal(encoded[inf | too_big], sign[inf | too_big] | 0x7F)


def test_decode_matches_torch_on_every_fp8_pattern():
    reference = torch.from_numpy(ALL_FP8.copy()).view(torch.float8_e4m3fn).to(torch.bfloat16).view(torch.uint16).numpy()
    assert np.array_equal(oracle.decode(ALL_FP8, 0), reference)


# Codec at every other shift, against exact scaling by powers of two in float64.


@pytest.mark.parametrize("shift", SHIFTS)
def test_encode_at_any_shift_is_torch_rounding_of_the_scaled_value(shift):
    encoded = oracle.encode(ALL_BF16, shift)
    values = bf16_values(ALL_BF16)
    raw = (ALL_BF16 >> 7) & 0xFF
    sign = ((ALL_BF16 >> 15).astype(np.uint8) << 7)
    finite_normal = (raw > 0) & (raw < 255)
    with np.errstate(over="ignore", invalid="ignore"):
        scaled = np.where(finite_normal, values, 0.0) * 2.0 ** (-shift)
    # Below 2**-10 everything rounds to a signed zero; float32 keeps scaled exact above 2**-126.
    small = finite_normal & (np.abs(scaled) < 2.0**-11)
    representable = finite_normal & ~small & (np.abs(scaled) <= 464.0)
    reference = torch_fp8_of_float(np.where(representable, scaled, 0.0))
    assert np.array_equal(encoded[representable], reference[representable])
    assert np.array_equal(encoded[small], sign[small])
    overflow = finite_normal & (np.abs(scaled) > 464.0)
    assert np.array_equal(encoded[overflow], sign[overflow] | 0x7F)
    assert np.array_equal(encoded[raw == 0], sign[raw == 0])
    assert np.array_equal(encoded[raw == 255], sign[raw == 255] | 0x7F)


@pytest.mark.parametrize("shift", SHIFTS)
def test_decode_at_any_shift_is_the_exact_product_or_its_documented_limit(shift):
    decoded = oracle.decode(ALL_FP8, shift)
    values = fp8_values(ALL_FP8)
    magnitude = ALL_FP8 & 0x7F
    nan = magnitude == 0x7F
    assert np.all(decoded[nan] == 0x7FC0)
    product = values * 2.0**shift
    sign = (ALL_FP8 >> 7).astype(np.uint16) << 15
    finite = ~nan
    in_range = finite & (np.abs(product) >= 2.0**-126) & (np.abs(product) < 2.0**128)
    # Every FP8 value times a power of two has at most 4 significant bits: BF16 holds it exactly.
    expected = torch.from_numpy(product[in_range].astype(np.float32)).to(torch.bfloat16).view(torch.uint16).numpy()
    assert np.array_equal(decoded[in_range], expected)
    flushed = finite & (np.abs(product) < 2.0**-126)
    assert np.array_equal(decoded[flushed], sign[flushed])
    saturated = finite & (np.abs(product) >= 2.0**128)
    assert np.array_equal(decoded[saturated], sign[saturated] | 0x7F7F)


# Known answers (reference tests/test_fp8.py:62-153).


def round_trip(bits):
    bits = np.asarray(bits, dtype=np.uint16)
    shift = int(oracle.group_shifts(bits[None])[0])
    return shift, oracle.decode(oracle.encode(bits, shift), shift)


def test_ties_round_to_even():
    bits = oracle.bf16_bits(np.array([1.0625, 1.1875, 3 * 2.0**-10, 2.0**-10], dtype=np.float32))
    decoded = oracle.bf16_to_float(oracle.decode(oracle.encode(bits, 0), 0))
    assert decoded.tolist() == [1.0, 1.25, 2 * 2.0**-9, 0.0]


def test_scale_extends_range():
    bits = oracle.bf16_bits(np.array([6500.0, -3000.0, 1.0], dtype=np.float32))
    shift, restored = round_trip(bits)
    assert shift == 12 - 7
    assert oracle.bf16_to_float(restored)[:2].tolist() == pytest.approx([6500.0, -3000.0], rel=2.0**-4)
    bits = oracle.bf16_bits(np.array([3e-30, 1e-30], dtype=np.float32))
    shift, restored = round_trip(bits)
    assert shift < -100
    assert oracle.bf16_to_float(restored).tolist() == pytest.approx(oracle.bf16_to_float(bits).tolist(), rel=2.0**-4)


def test_top_of_bf16_saturates_instead_of_overflowing():
    shift, restored = round_trip([0x7F7F])
    assert shift == 120 and restored.tolist() == [0x7F7F]


def test_non_finite_values_stay_non_finite_and_do_not_set_the_scale():
    bits = oracle.bf16_bits(np.array([np.inf, -np.inf, np.nan, 1.5, -0.25], dtype=np.float32))
    shift, restored = round_trip(bits)
    after = oracle.bf16_to_float(restored)
    assert np.isnan(after[:3]).all() and shift == -7
    assert after[3:].tolist() == [1.5, -0.25]
    assert oracle.encode(np.array([0x7F80], dtype=np.uint16), 0).tolist() == [0x7F]


def test_zero_and_subnormal_groups_keep_shift_zero_and_their_sign():
    shift, restored = round_trip([0x0000, 0x8000, 0x0001, 0x807F])
    assert shift == 0 and restored.tolist() == [0x0000, 0x8000, 0x0000, 0x8000]


def test_group_shift_ignores_non_finite_and_subnormal_exponents():
    assert oracle.group_shifts(np.array([[0x7F80, 0xFFC0, 0x0001]], dtype=np.uint16)).tolist() == [0]
    assert oracle.group_shifts(np.array([[0x3F80, 0x7F80]], dtype=np.uint16)).tolist() == [-7]
    assert oracle.group_shifts(np.array([[0x0080]], dtype=np.uint16)).tolist() == [1 - 134]


# The stated round-trip error bound (fp8.py:25-27), restated from the docstring.


def assert_within_error(bits, restored, shift):
    before, after = bf16_values(bits), bf16_values(restored)
    raw = (bits.astype(np.int32) >> 7) & 0xFF
    nonfinite = raw == 255
    assert np.isnan(after[nonfinite]).all()
    zero_like = raw == 0
    assert (after[zero_like] == 0).all()
    assert np.array_equal(restored[zero_like] >> 15, bits[zero_like] >> 15)
    normal = ~zero_like & ~nonfinite
    error = np.abs(after[normal] - before[normal])
    scaled_normal = raw[normal] - 127 - shift >= -6
    assert (error[scaled_normal] <= np.abs(before[normal][scaled_normal]) * 2.0**-4).all()
    floor = max(2.0 ** (shift - 10), 2.0**-126)
    assert (error[~scaled_normal] <= floor).all()
    assert np.isfinite(after[normal]).all()


@settings(max_examples=300, deadline=None)
@given(st.lists(st.integers(0, 65535), min_size=1, max_size=128))
def test_round_trip_error_on_arbitrary_bits(patterns):
    bits = np.array(patterns, dtype=np.uint16)
    shift, restored = round_trip(bits)
    assert_within_error(bits, restored, shift)


@settings(max_examples=200, deadline=None)
@given(st.integers(-126, 127), st.lists(st.floats(1.0, 2.0, width=32), min_size=1, max_size=64), st.integers(0, 30))
def test_round_trip_error_across_magnitudes(exponent, significands, spread):
    values = [s * 2.0 ** max(exponent - (i % (spread + 1)), -126) for i, s in enumerate(significands)]
    bits = torch.tensor(values, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    bits = bits[np.isfinite(bf16_values(bits))]
    if bits.size:
        shift, restored = round_trip(bits)
        assert_within_error(bits, restored, shift)


# Records (fp8.py:58-80, :179-198).

QWEN_GROUP, QWEN_GROUPS = 16 * 128, 2 * 36 * 8


def test_record_layout_constants():
    assert QWEN_GROUP * QWEN_GROUPS * 2 == 2_359_296
    assert oracle.record_bytes(QWEN_GROUP, QWEN_GROUPS) == 1_180_800
    assert 2 * QWEN_GROUPS == 1152


def micro_pool(blocks=8, seed=0, group=16 * 24, groups=2 * 2 * 2):
    rng = np.random.default_rng(seed)
    values = rng.standard_normal((blocks, groups * group)) * np.exp(rng.standard_normal((blocks, groups * group)) * 2)
    return oracle.bf16_bits(values.astype(np.float32)).reshape(blocks, groups * group), group, groups


def test_records_hold_each_groups_shift_and_encoding_in_id_order():
    pool, group, groups = micro_pool()
    ids = [5, 0, 3]
    stage = oracle.quantize_records(pool, ids, group, groups)
    record = oracle.record_bytes(group, groups)
    for index, block in enumerate(ids):
        rec = stage[index * record : (index + 1) * record]
        shifts = rec[group * groups :].copy().view(np.int16)
        expected = oracle.group_shifts(pool[block].reshape(groups, group))
        assert np.array_equal(shifts.astype(np.int32), expected)
        for g in range(groups):
            encoded = oracle.encode(pool[block, g * group : (g + 1) * group], int(expected[g]))
            assert np.array_equal(rec[g * group : (g + 1) * group], encoded)


def test_record_round_trip_restores_only_the_target_blocks_within_the_bound():
    pool, group, groups = micro_pool()
    stage = oracle.quantize_records(pool, [1, 2, 3, 4], group, groups)
    target, _, _ = micro_pool(seed=9)
    untouched = target[:6].copy()
    oracle.dequantize_records(stage, [6, 7], target, group, groups)
    assert np.array_equal(target[:6], untouched)
    for source, dest in ((1, 6), (2, 7)):
        for g in range(groups):
            bits = pool[source, g * group : (g + 1) * group]
            shift = int(oracle.group_shifts(bits[None])[0])
            assert_within_error(bits, target[dest, g * group : (g + 1) * group], shift)


def test_gather_and_scatter_are_identities_on_bytes():
    rng = np.random.default_rng(1)
    pool = rng.integers(0, 256, 8 * 4096, dtype=np.uint8)
    host = oracle.gather(pool, 4096, [6, 1, 4])
    assert host.tobytes() == b"".join(pool[i * 4096 : (i + 1) * 4096].tobytes() for i in [6, 1, 4])
    target = np.zeros_like(pool)
    oracle.scatter(target, 4096, [2, 5, 0], host)
    assert target[2 * 4096 : 3 * 4096].tobytes() == pool[6 * 4096 : 7 * 4096].tobytes()
    assert not target[4096 : 2 * 4096].any()


# Decode attention (decode_attention.py:9-37) against independent computations.


def make_case(lengths, kv_heads=2, kv_groups=2, dim=24, slots=16, layers=3, seed=0, gain=1.0):
    rng = np.random.default_rng(seed)
    batch = len(lengths)
    width = max(-(-n // slots) for n in lengths)
    blocks = batch * width + 3
    pool = oracle.bf16_bits(rng.standard_normal((blocks, 2, layers, kv_heads, slots, dim)).astype(np.float32))
    table = rng.permutation(blocks)[: batch * width].reshape(batch, width).astype(np.int32)
    q = oracle.bf16_bits((gain * rng.standard_normal((batch, kv_heads * kv_groups, dim))).astype(np.float32))
    return q, pool, table, np.array(lengths, dtype=np.int32), kv_groups


def sdpa_float64(q, pool, layer, table, lengths, kv_groups):
    qf = torch.from_numpy(oracle.bf16_to_float(q).astype(np.float64))
    pf = torch.from_numpy(oracle.bf16_to_float(pool).astype(np.float64))
    outs = []
    for b in range(q.shape[0]):
        n = int(lengths[b])
        ids = torch.from_numpy(table[b].astype(np.int64))
        keys = pf[ids, 0, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :n].repeat_interleave(kv_groups, 0)
        values = pf[ids, 1, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :n].repeat_interleave(kv_groups, 0)
        outs.append(torch.nn.functional.scaled_dot_product_attention(qf[b][:, None], keys, values)[:, 0])
    return torch.stack(outs).numpy()


@pytest.mark.parametrize("lengths", [[1], [16, 32, 48], [17, 33], [15, 31], [1, 16, 17, 47, 48, 80, 3, 64]])
@pytest.mark.parametrize("groups", [1, 2, 4])
def test_decode_attention_matches_torch_sdpa_in_float64(lengths, groups):
    q, pool, table, lens, groups = make_case(lengths, kv_groups=groups, seed=groups)
    ours = oracle.decode_attention(q, pool, 1, table, lens, groups)
    theirs = sdpa_float64(q, pool, 1, table, lens, groups)
    assert np.abs(ours - theirs).max() < 1e-12


def test_decode_attention_matches_a_pure_python_softmax():
    q, pool, table, lens, groups = make_case([5, 19], kv_heads=1, kv_groups=2, dim=4, slots=4, layers=2, seed=7)
    ours = oracle.decode_attention(q, pool, 0, table, lens, groups)
    qf, pf = oracle.bf16_to_float(q).astype(float), oracle.bf16_to_float(pool).astype(float)
    for b in range(2):
        for h in range(2):
            keys = [pf[table[b, t // 4], 0, 0, 0, t % 4] for t in range(lens[b])]
            vals = [pf[table[b, t // 4], 1, 0, 0, t % 4] for t in range(lens[b])]
            scores = [sum(qf[b, h, d] * k[d] for d in range(4)) / 2.0 for k in keys]
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            expected = [sum(w * v[d] for w, v in zip(weights, vals)) / total for d in range(4)]
            assert ours[b, h] == pytest.approx(expected, rel=1e-12, abs=1e-14)


def test_decode_attention_ignores_whatever_unwritten_slots_hold():
    q, pool, table, lens, groups = make_case([20, 3], seed=37)
    clean = oracle.decode_attention(q, pool, 1, table, lens, groups)
    pool[table[0, 1], :, :, :, 4:] = 0x7FC0
    pool[table[1, 0], :, :, :, 3:] = 0x7F80
    assert np.array_equal(oracle.decode_attention(q, pool, 1, table, lens, groups), clean)


def test_decode_attention_refuses_impossible_lengths():
    q, pool, table, lens, groups = make_case([20])
    with pytest.raises(ValueError):
        oracle.decode_attention(q, pool, 1, table, np.array([0], dtype=np.int32), groups)
    with pytest.raises(ValueError):
        oracle.decode_attention(q, pool, 1, table, np.array([33], dtype=np.int32), groups)
