"""The committed vectors of tests/golden.

fp8_known_answers.json holds the reference's own FP8 known answers (tests/test_fp8.py:62-154)
as data; records_micro.npz and decode_micro.npz are frozen oracle outputs on stored inputs
(tests/golden/make_golden.py). On the CPU the oracle must still give every one of them; on
the GPU the HIP kernels, called through the C ABI, must give the same records and restored
pools bit for bit and the same attention within BF16 rounding.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
KNOWN = json.loads((GOLDEN / "fp8_known_answers.json").read_text())


def load(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def input_bits(case: dict) -> np.ndarray:
    if "bits" in case:
        return np.array(case["bits"], dtype=np.uint16)
    return oracle.bf16_bits(np.array([float(v) for v in case["values"]], dtype=np.float32))


def check_round_trip(case: dict, shift: int, restored: np.ndarray) -> None:
    """The expectations one known-answer case states, whoever computed shift and restored."""
    bits = input_bits(case)
    if "shift" in case:
        assert shift == case["shift"], case["source"]
    if "shift_below" in case:
        assert shift < case["shift_below"], case["source"]
    after = oracle.bf16_to_float(restored)
    if "restored_bits" in case:
        assert restored.tolist() == case["restored_bits"], case["source"]
    if "restored_values" in case:
        assert after.tolist() == case["restored_values"], case["source"]
    if "restored_within" in case:
        spec = case["restored_within"]
        first = spec["first"]
        target = oracle.bf16_to_float(bits)[:first] if spec["of"] == "input" else np.array(spec["of"])
        assert after[:first].tolist() == pytest.approx(target.tolist(), rel=spec["relative"]), case["source"]
    if "restored_nan" in case:
        assert np.isnan(after[case["restored_nan"]]).all(), case["source"]
    if "restored_tail" in case:
        tail = case["restored_tail"]
        assert after[tail["from"]:].tolist() == tail["values"], case["source"]


@pytest.mark.parametrize("case", KNOWN["round_trips"], ids=lambda c: c["source"].split("(")[-1].rstrip(")"))
def test_oracle_gives_the_reference_known_answers(case):
    bits = input_bits(case)
    shift = case["shift"] if case.get("fixed_shift") else int(oracle.group_shifts(bits[None])[0])
    check_round_trip(case, shift, oracle.decode(oracle.encode(bits, shift), shift))


@pytest.mark.parametrize("case", KNOWN["encodes"], ids=lambda c: c["source"].split(" ")[0])
def test_oracle_gives_the_reference_known_codes(case):
    codes = oracle.encode(np.array(case["bits"], dtype=np.uint16), case["shift"])
    assert codes.tolist() == case["codes"]


def test_oracle_still_gives_the_frozen_records():
    g = load("records_micro.npz")
    records = oracle.quantize_records(g["pool"], g["ids"], int(g["group_elems"]), int(g["groups_per_block"]))
    assert np.array_equal(records, g["records"])
    restored = np.zeros_like(g["pool"])
    oracle.dequantize_records(g["records"], g["target_ids"], restored, int(g["group_elems"]), int(g["groups_per_block"]))
    assert np.array_equal(restored, g["restored"])


def test_oracle_still_gives_the_frozen_attention():
    g = load("decode_micro.npz")
    layer, groups = int(g["layer"]), int(g["groups"])
    out = oracle.decode_attention(g["q"], g["pool"], layer, g["table"], g["lengths"], groups)
    assert np.allclose(out, g["out"], rtol=1e-12, atol=1e-12)
    decoded = np.zeros_like(g["pool"])
    ids = np.arange(g["pool"].shape[0], dtype=np.int32)
    group_elems = g["pool"].shape[4] * g["pool"].shape[5]
    groups_per_block = 2 * g["pool"].shape[2] * g["pool"].shape[3]
    oracle.dequantize_records(g["records"], ids, decoded, group_elems, groups_per_block)
    out_fp8 = oracle.decode_attention(g["q"], decoded, layer, g["table"], g["lengths"], groups)
    assert np.allclose(out_fp8, g["out_fp8"], rtol=1e-12, atol=1e-12)


# The HIP kernels against the same vectors.


def gpu_bits(bits: np.ndarray):
    import torch

    return torch.from_numpy(bits.view(np.int16)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("case", KNOWN["round_trips"], ids=lambda c: c["source"].split("(")[-1].rstrip(")"))
def test_record_kernel_gives_the_reference_known_answers(case):
    """The group goes through lk_fp8_quantize / lk_fp8_dequantize as the first group of a
    one-block [2, 1, 1, 16, 128] pool, zeros elsewhere (zeros leave a shift unchanged), so
    the shift is the kernel's own."""
    import torch
    from layover_amd.kernels import fp8

    bits = input_bits(case)
    if case.get("fixed_shift"):
        codes = fp8.encode_bits_hip(gpu_bits(bits).view(torch.uint16), case["shift"])
        restored = fp8.decode_bits_hip(codes, case["shift"]).cpu().numpy().view(np.uint16)
        check_round_trip(case, case["shift"], restored)
        return
    block = np.zeros(2 * 16 * 128, dtype=np.uint16)
    block[: bits.size] = bits
    pool = gpu_bits(block).view(torch.bfloat16).view(1, 2, 1, 1, 16, 128)
    layout = fp8.Fp8Layout(16 * 128, 2)
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    stage = torch.empty(layout.record_bytes, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, ids, stage, layout)
    back = torch.zeros_like(pool)
    fp8.dequantize_blocks(stage, ids, back, layout)
    record = stage.cpu().numpy()
    shift = int(record[layout.block_elems:layout.block_elems + 2].view(np.int16)[0])
    restored = back.view(torch.int16).cpu().numpy().reshape(-1).view(np.uint16)
    check_round_trip(case, shift, restored[: bits.size])
    assert not restored[bits.size:].any()


@pytest.mark.gpu
@pytest.mark.parametrize("case", KNOWN["encodes"], ids=lambda c: c["source"].split(" ")[0])
def test_encode_kernel_gives_the_reference_known_codes(case):
    import torch
    from layover_amd.kernels import fp8

    codes = fp8.encode_bits_hip(gpu_bits(np.array(case["bits"], dtype=np.uint16)).view(torch.uint16), case["shift"])
    assert codes.cpu().numpy().tolist() == case["codes"]


@pytest.mark.gpu
def test_record_kernels_give_the_frozen_records_and_restored_pool():
    import torch
    from layover_amd.kernels import fp8

    g = load("records_micro.npz")
    pool = gpu_bits(g["pool"]).view(torch.bfloat16)
    layout = fp8.Fp8Layout(int(g["group_elems"]), int(g["groups_per_block"]))
    stage = torch.full((g["records"].size + 16,), 0xAB, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, torch.from_numpy(g["ids"]).cuda(), stage, layout)
    got = stage.cpu().numpy()
    assert np.array_equal(got[: g["records"].size], g["records"])
    assert (got[g["records"].size:] == 0xAB).all()
    restored = torch.zeros_like(pool)
    fp8.dequantize_blocks(torch.from_numpy(g["records"]).cuda(), torch.from_numpy(g["target_ids"]).cuda(), restored, layout)
    assert np.array_equal(restored.view(torch.int16).cpu().numpy().view(np.uint16), g["restored"])


def assert_attention_close(out, expected, weighted_abs_v=None):
    got = out.double().cpu().numpy()
    # BF16 rounding of the exact answer plus an FP32 accumulation allowance; for FP8 pools,
    # whose weights go to the matrix cores as single BF16s, 2^-8 of the weighted mean |v|.
    allowed = np.abs(expected) * 2.0**-8 + 1e-3
    if weighted_abs_v is not None:
        allowed = allowed + 2.0**-8 * weighted_abs_v
    assert np.isfinite(got).all()
    assert (np.abs(got - expected) <= allowed).all(), np.abs(got - expected).max()
    assert (np.abs(got - expected) <= 2e-2 + 1e-2 * np.abs(expected)).all()


@pytest.mark.gpu
def test_decode_kernel_gives_the_frozen_attention_on_bf16_and_fp8_pools():
    import torch
    from layover_amd.kernels import hip_decode

    g = load("decode_micro.npz")
    layer, groups = int(g["layer"]), int(g["groups"])
    q = gpu_bits(g["q"]).view(torch.bfloat16)
    table = torch.from_numpy(g["table"]).cuda()
    lengths = torch.from_numpy(g["lengths"]).cuda()
    out = hip_decode.paged_decode_attention_hip(q, gpu_bits(g["pool"]).view(torch.bfloat16), layer, table, lengths, groups)
    assert_attention_close(out, g["out"])

    blocks, _, layers, kv_heads, slots, head_dim = g["pool"].shape
    records = torch.from_numpy(g["records"].reshape(blocks, -1)).cuda()
    pool = hip_decode.Fp8KVPool(records, layers, kv_heads, slots, head_dim)
    out = hip_decode.paged_decode_attention_hip(q, pool, layer, table, lengths, groups)
    decoded = np.zeros_like(g["pool"])
    oracle.dequantize_records(g["records"], np.arange(blocks, dtype=np.int32), decoded, slots * head_dim, 2 * layers * kv_heads)
    magnitudes = decoded.copy()
    magnitudes[:, 1] &= 0x7FFF
    weighted = oracle.decode_attention(g["q"], magnitudes, layer, g["table"], g["lengths"], groups)
    assert_attention_close(out, g["out_fp8"], weighted)
    assert math.isfinite(float(out.float().abs().max()))
