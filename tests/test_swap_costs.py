"""Swap-cost sweep (reference bench/kv_crossover.py's swap half, tests/test_kv_crossover.py) and
the FP8 round-trip bound it verifies with (reference fp8.py:140-176).

The bound is pinned against the oracle's codec: every round trip of the oracle stays inside
it, it is met (exactly on the subnormal grid's ties; at 16/17 of it in the normal regime,
whose largest half step relative to the value is at the tie 1.0625 * 2^e), and a decode at
the wrong shift leaves it."""

import json

import numpy as np
import pytest
import torch

from layover_amd.kernels.fp8 import group_shifts, round_trip_bound, round_trip_within_bound
from layover_amd.kv import swap_costs
from oracle import oracle


def spread_groups(groups=64, elems=384, seed=0):
    """BF16 patterns whose exponents span 40 binades below each group's largest, so both the
    E4M3 normal and subnormal regimes (and BF16 flushes) occur."""
    rng = np.random.default_rng(seed)
    top = rng.integers(20, 235, size=(groups, 1))
    exponent = np.clip(top - rng.integers(0, 40, size=(groups, elems)), 0, 254)
    bits = (rng.integers(0, 2, size=(groups, elems)) << 15) | (exponent << 7) | rng.integers(0, 128, size=(groups, elems))
    return bits.astype(np.uint16)


def oracle_round_trip(bits, shift_offset=0):
    shifts = oracle.group_shifts(bits)
    back = np.stack([oracle.decode(oracle.encode(row, int(s)), int(s) + shift_offset) for row, s in zip(bits, shifts)])
    return shifts, back


def as_torch(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.uint16)


def test_group_shifts_match_the_oracle_including_special_values():
    bits = spread_groups()
    bits[0, :] = 0
    bits[1, :5] = [0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x8000]
    bits[2, :] = 0x0001  # subnormals only: shift 0
    assert np.array_equal(group_shifts(as_torch(bits)).numpy(), oracle.group_shifts(bits))


def test_every_oracle_round_trip_is_inside_the_bound_and_the_bound_is_met():
    bits = spread_groups()
    shifts, back = oracle_round_trip(bits)
    values = oracle.bf16_to_float(bits).astype(np.float64)
    gap = np.abs(oracle.bf16_to_float(back).astype(np.float64) - values)
    bound = round_trip_bound(as_torch(bits)).numpy()
    assert (gap <= bound).all()
    exponent = ((bits >> 7) & 0xFF).astype(np.int64) - 127
    normal = (exponent - shifts[:, None] >= -6) & (exponent > -127)
    ratio = gap / bound
    # Normal regime: the half step 2^(e-4) against |v|/16 is largest at the tie 1.0625 * 2^e.
    assert ratio[normal].max() == pytest.approx(16 / 17, abs=1e-12)
    assert ratio[~normal & (bound > 2.0**-126)].max() == 1.0


def test_a_decode_at_the_wrong_shift_leaves_the_bound():
    bits = spread_groups(seed=1)
    _, back = oracle_round_trip(bits, shift_offset=1)
    before = as_torch(bits).view(torch.bfloat16).reshape(1, -1)
    after = as_torch(back).view(torch.bfloat16).reshape(1, -1)
    assert not round_trip_within_bound(before, after, bits.shape[1])
    _, good = oracle_round_trip(bits)
    assert round_trip_within_bound(before, as_torch(good).view(torch.bfloat16).reshape(1, -1), bits.shape[1])


def test_fit_recovers_a_line_and_stays_nonnegative():
    x = np.array([512, 1024, 2048, 4096, 8192], dtype=np.float64)
    assert swap_costs.fit_nonnegative(x, 1e-3 + 2e-6 * x, 1) == pytest.approx([1e-3, 2e-6])
    # A falling intercept would be negative: it is dropped and the slope refitted.
    coef = swap_costs.fit_nonnegative(x, 3e-6 * x - 1e-3, 1)
    assert coef[0] == 0.0 and coef[1] > 0
    assert swap_costs.fit_nonnegative(x, -x, 1) == [0.0, 0.0]


def test_sweep_on_the_host_flavour_writes_the_reference_keys_and_merges(tmp_path):
    reference_model = tmp_path / "cost_model.json"
    reference_model.write_text(json.dumps({
        "swap_out_s_coef": [9.0, 9.0], "swap_in_s_coef": [9.0, 9.0], "recompute_s_coef": [0.1, 1e-5, 1e-9],
        "measured_on_gpu": True, "transfer": "plain",
    }))
    out = tmp_path / "sweep"
    meta = swap_costs.main(["--device", "cpu", "--model", "micro", "--offload-dtype", "bf16", "--tokens", "64", "200", "512",
                            "--repeats", "2", "--staging-mib", "1", "--host-cache-mib", "64", "--out", str(out),
                            "--merge", str(reference_model)])
    assert meta["complete"] and not meta["measured_on_gpu"] and meta["transfer"] == "native"
    assert [r["tokens"] for r in meta["rows"]] == [64, 200, 512] and meta["rows"][1]["blocks"] == 13
    assert all(c >= 0 for c in meta["swap_out_s_coef"] + meta["swap_in_s_coef"])
    assert "fp8_swap_out_s_coef" not in meta
    assert not (out / "swap_costs.partial.json").exists()
    assert len((out / "swap_costs.csv").read_text().splitlines()) == 4
    merged = json.loads((out / "cost_model.json").read_text())
    assert merged["recompute_s_coef"] == [0.1, 1e-5, 1e-9]
    assert merged["swap_out_s_coef"] == meta["swap_out_s_coef"] and merged["transfer"] == "native"
    assert merged["measured_on_gpu"] is False  # a CPU sweep never makes a cost model a GPU one


def test_a_corrupting_transfer_stops_the_sweep(monkeypatch, tmp_path):
    real = swap_costs.NativeBackend.start_in

    def corrupting(self, cache, blocks, payload):
        payload.memory[3] ^= 1
        return real(self, cache, blocks, payload)

    monkeypatch.setattr(swap_costs.NativeBackend, "start_in", corrupting)
    with pytest.raises(RuntimeError, match="changed"):
        swap_costs.main(["--device", "cpu", "--model", "micro", "--offload-dtype", "bf16", "--tokens", "64", "--repeats", "1",
                         "--warmup", "0", "--staging-mib", "1", "--out", str(tmp_path)])


def test_a_truncated_sweep_is_never_merged():
    with pytest.raises(ValueError, match="truncated"):
        swap_costs.merge({"complete": False}, None)


def test_fp8_needs_the_gpu(tmp_path):
    with pytest.raises(SystemExit):
        swap_costs.main(["--device", "cpu", "--offload-dtype", "fp8", "--out", str(tmp_path)])


@pytest.mark.gpu
def test_gpu_sweep_measures_bf16_and_fp8(tmp_path):
    meta = swap_costs.main(["--tokens", "256", "1024", "--repeats", "1", "--staging-mib", "16", "--host-cache-mib", "512",
                            "--out", str(tmp_path)])
    assert meta["measured_on_gpu"] and meta["complete"]
    for key in swap_costs.SWAP_KEYS:
        assert len(meta[key]) == 2 and min(meta[key]) >= 0
    row = meta["rows"][-1]
    assert row["fp8_bytes"] < row["bf16_bytes"] and row["fp8_swap_out_s"] > 0
