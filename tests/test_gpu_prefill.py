"""Paged causal prefill (lk_paged_prefill) against the float64 oracle, through the C ABI.

Tolerance: the north star's 2e-2 absolute / 1e-2 relative, plus a tighter check that the
error stays within BF16 rounding of the output and of the weights (P enters the matrix cores
as BF16): |err| <= 2^-7 |x| + 4e-3."""

import os

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import oracle

pytestmark = pytest.mark.gpu


def make_pool(blocks, layers, kv_heads, seed, fp8=False):
    from layover_amd.kernels.hip_decode import Fp8KVPool

    rng = np.random.default_rng(seed)
    bits = oracle.bf16_bits(rng.standard_normal((blocks, 2, layers, kv_heads, 16, 128), dtype=np.float32))
    if not fp8:
        return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), bits
    group_elems, groups = 16 * 128, 2 * layers * kv_heads
    records = oracle.quantize_records(bits, list(range(blocks)), group_elems, groups)
    state = np.zeros_like(bits)
    oracle.dequantize_records(records, list(range(blocks)), state, group_elems, groups)
    return Fp8KVPool(torch.from_numpy(records.reshape(blocks, -1)).cuda(), layers, kv_heads, 16, 128), state


def assert_close(got, reference):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - reference)
    assert np.isfinite(got).all()
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(reference)), err.max()
    assert np.all(err <= 2.0**-7 * np.abs(reference) + 4e-3), err.max()


@pytest.mark.parametrize("start,tokens", [(0, 1), (0, 16), (0, 37), (5, 20), (16, 16), (100, 64), (1000, 130), (4090, 7)])
def test_prefill_matches_the_oracle(start, tokens):
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    end = start + tokens
    blocks = -(-end // 16) + 3
    pool, bits = make_pool(blocks, 3, 8, seed=start + tokens)
    rng = np.random.default_rng(tokens)
    block_ids = rng.permutation(blocks)[: -(-end // 16)].astype(np.int32)
    q = torch.randn(32, tokens, 128, device="cuda").to(torch.bfloat16)
    print(f"prefill start={start} tokens={tokens}", flush=True)
    out = paged_prefill_attention_hip(q, pool, 1, torch.from_numpy(block_ids).cuda(), start, 4)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, 1, block_ids, start, 4))


@pytest.mark.parametrize("query_heads", [8, 16, 40], ids=["gqa1", "gqa2", "gqa5"])
def test_prefill_gqa_ratios(query_heads):
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    pool, bits = make_pool(12, 2, 8, seed=query_heads)
    block_ids = np.arange(11, -1, -1, dtype=np.int32)
    q = torch.randn(query_heads, 45, 128, device="cuda").to(torch.bfloat16)
    print(f"prefill gqa heads={query_heads}", flush=True)
    out = paged_prefill_attention_hip(q, pool, 0, torch.from_numpy(block_ids).cuda(), 77, query_heads // 8)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, 0, block_ids, 77, query_heads // 8))


@pytest.mark.parametrize("path", ["staged", "direct"])
@pytest.mark.parametrize("start,tokens", [(0, 24), (300, 90)])
def test_prefill_reads_fp8_records(start, tokens, path, monkeypatch):
    """FP8-record pools: the history staged as BF16 in the workspace, or read directly by the
    FP8 form of the kernel (LAYOVER_PREFILL_FP8=direct)."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_FP8", path)

    end = start + tokens
    blocks = -(-end // 16)
    pool, state = make_pool(blocks, 2, 8, seed=7, fp8=True)
    block_ids = np.random.default_rng(8).permutation(blocks).astype(np.int32)
    q = torch.randn(32, tokens, 128, device="cuda").to(torch.bfloat16)
    print(f"prefill fp8 {path} start={start} tokens={tokens}", flush=True)
    out = paged_prefill_attention_hip(q, pool, 1, torch.from_numpy(block_ids).cuda(), start, 4)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), state, 1, block_ids, start, 4))


@pytest.mark.parametrize("form", ["bf16", "fp8_staged", "fp8_direct"])
def test_slots_past_the_chunk_end_never_reach_the_output(form, monkeypatch):
    """NaN in every slot past the chunk's end (FP8 records: NaN codes there) never reaches the
    output, on a BF16 pool and on FP8 records staged as BF16 or read directly."""
    from layover_amd.kernels.hip_decode import Fp8KVPool
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_FP8", "direct" if form == "fp8_direct" else "staged")
    pool, bits = make_pool(4, 1, 8, seed=11)
    poisoned = bits.copy()
    poisoned[3, :, 0, :, 9:] = 0x7FC0  # NaN in every slot of the last block past token 57
    if form == "bf16":
        pool.copy_(torch.from_numpy(poisoned.view(np.int16)).cuda().view(torch.bfloat16))
    else:
        records = oracle.quantize_records(poisoned, list(range(4)), 16 * 128, 16)
        bits = np.zeros_like(poisoned)
        oracle.dequantize_records(records, list(range(4)), bits, 16 * 128, 16)
        bits[3, :, 0, :, 9:] = 0  # the oracle reads only tokens before the end
        pool = Fp8KVPool(torch.from_numpy(records.reshape(4, -1)).cuda(), 1, 8, 16, 128)
    block_ids = np.array([2, 0, 1, 3], dtype=np.int32)
    q = torch.randn(32, 20, 128, device="cuda").to(torch.bfloat16)
    out = paged_prefill_attention_hip(q, pool, 0, torch.from_numpy(block_ids).cuda(), 37, 4)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, 0, block_ids, 37, 4))


def test_reference_signature_after_writing_the_chunk():
    """cache.chunk + write_at + prefill_attention, as the reference's forward_prefill runs
    them (model.py:131-135), for a first chunk and a later one."""
    from layover_amd.config import ModelConfig
    from layover_amd.kernels.hip_prefill import prefill_attention
    from layover_amd.kv.paged_cache import BlockTable, PagedKVCache

    cache = PagedKVCache(ModelConfig.qwen3_4b(), 20, device="cuda")
    table = BlockTable(cache.allocator.alloc(9), 0)
    for start, count in ((0, 70), (70, 61)):
        chunk = cache.chunk(table, start, count)
        k = torch.randn(8, count, 128, device="cuda").to(torch.bfloat16)
        v = torch.randn(8, count, 128, device="cuda").to(torch.bfloat16)
        q = torch.randn(32, count, 128, device="cuda").to(torch.bfloat16)
        for layer in (0, 35):
            cache.write_at(chunk.write_blocks, chunk.write_slots, layer, k, v)
        out = prefill_attention(q, k, v, cache, 35, chunk, 4)
        torch.cuda.synchronize()
        bits = cache.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, 35, chunk.block_ids.cpu().numpy(), start, 4))


def test_prefill_refuses_what_it_cannot_run():
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    pool, _ = make_pool(3, 1, 8, seed=1)
    q = torch.zeros(32, 10, 128, dtype=torch.bfloat16, device="cuda")
    ids = torch.arange(3, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="blocks cannot hold"):
        paged_prefill_attention_hip(q, pool, 0, ids[:1], 10, 4)
    with pytest.raises(ValueError, match="KV heads"):
        paged_prefill_attention_hip(q, pool, 0, ids, 0, 3)
    with pytest.raises(ValueError, match="int32"):
        paged_prefill_attention_hip(q, pool, 0, ids.long(), 0, 4)
    with pytest.raises(ValueError, match="BF16"):
        paged_prefill_attention_hip(q.float(), pool, 0, ids, 0, 4)


@pytest.mark.parametrize("kernel", ["staged", "lds", "register_only"])
def test_prefill_fp8_tiny_groups_take_the_exact_decode(kernel, monkeypatch):
    """Groups scaled by 2^-114 get shifts below -117, where the hardware convert times
    2^shift could leave BF16's normal range; those blocks are decoded with the reference's
    integer decode instead. Every V group and the K groups of half the blocks are scaled, and
    the output (about 2^-114 in size) is compared after scaling back by 2^114."""
    from layover_amd.kernels.hip_decode import Fp8KVPool
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_KERNEL", "1" if kernel == "register_only" else "0")
    monkeypatch.setenv("LAYOVER_PREFILL_FP8", "staged" if kernel == "staged" else "direct")
    blocks, layers = 8, 2
    rng = np.random.default_rng(21)
    values = rng.standard_normal((blocks, 2, layers, 8, 16, 128), dtype=np.float32)
    values[::2, 0] *= np.float32(2.0**-114)
    values[:, 1] *= np.float32(2.0**-114)
    bits = oracle.bf16_bits(values)
    group_elems, groups = 16 * 128, 2 * layers * 8
    records = oracle.quantize_records(bits, list(range(blocks)), group_elems, groups)
    shifts = records.reshape(blocks, -1)[:, group_elems * groups :].copy().view(np.int16)
    assert (shifts < -117).sum() >= blocks * layers * 8 * 3 // 2
    state = np.zeros_like(bits)
    oracle.dequantize_records(records, list(range(blocks)), state, group_elems, groups)
    pool = Fp8KVPool(torch.from_numpy(records.reshape(blocks, -1)).cuda(), layers, 8, 16, 128)
    block_ids = np.array([3, 0, 6, 1, 4, 7, 2, 5], dtype=np.int32)
    q = torch.randn(32, 60, 128, device="cuda").to(torch.bfloat16)
    print(f"prefill fp8 exact decode, {kernel}", flush=True)
    out = paged_prefill_attention_hip(q, pool, 1, torch.from_numpy(block_ids).cuda(), 50, 4)
    torch.cuda.synchronize()
    reference = oracle.prefill_attention(q.float().cpu().numpy(), state, 1, block_ids, 50, 4)
    assert_close(out.float() * 2.0**114, reference * 2.0**114)


@pytest.mark.parametrize("splits", ["1", "3", "7"])
@pytest.mark.parametrize("fp8", [False, True, "direct"], ids=["bf16_pool", "fp8_pool", "fp8_pool_direct"])
@pytest.mark.parametrize("start,tokens", [(0, 37), (1000, 130), (4090, 7), (300, 90)])
def test_split_keys_match_the_oracle(start, tokens, fp8, splits, monkeypatch):
    """Split-K: each tile's key steps spread over 1, 3 or 7 workgroups whose partials are
    merged. Splits that hold no visible key for some rows (or none at all) must contribute
    nothing, not NaN."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", splits)
    monkeypatch.setenv("LAYOVER_PREFILL_FP8", "direct" if fp8 == "direct" else "staged")
    end = start + tokens
    blocks = -(-end // 16)
    pool, state = make_pool(blocks, 2, 8, seed=tokens, fp8=fp8)
    block_ids = np.random.default_rng(start).permutation(blocks).astype(np.int32)
    q = torch.randn(32, tokens, 128, device="cuda").to(torch.bfloat16)
    print(f"prefill split={splits} fp8={fp8} start={start} tokens={tokens}", flush=True)
    out = paged_prefill_attention_hip(q, pool, 1, torch.from_numpy(block_ids).cuda(), start, 4)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), state, 1, block_ids, start, 4))


@settings(max_examples=25, deadline=None, derandomize=True)
@given(
    seed=st.integers(0, 2**16),
    start=st.integers(0, 1500),
    tokens=st.integers(1, 96),
    kv_heads=st.integers(1, 4),
    gqa=st.integers(1, 5),
    layers=st.integers(1, 3),
    fp8=st.booleans(),
    splits=st.sampled_from([None, "2", "5"]),
)
def test_prefill_over_drawn_chunks_matches_the_oracle(seed, start, tokens, kv_heads, gqa, layers, fp8, splits):
    """Drawn chunks (start 0-1,500, 1-96 tokens, so chunks begin and end anywhere in a block),
    1-4 KV heads at GQA 1-5, BF16 pools and FP8 records (not 16-byte aligned unless layers x
    KV heads is a multiple of 4: then always staged), the split count chosen by the
    library or forced to 2 or 5; shuffled block ids with spare blocks in the pool. The split
    count is set in the environment around each draw (hypothesis runs every draw inside one
    call of the test, so a fixture could not)."""
    saved = os.environ.pop("LAYOVER_PREFILL_SPLITS", None)
    if splits is not None:
        os.environ["LAYOVER_PREFILL_SPLITS"] = splits
    try:
        drawn_prefill_case(seed, start, tokens, kv_heads, gqa, layers, fp8, splits)
    finally:
        os.environ.pop("LAYOVER_PREFILL_SPLITS", None)
        if saved is not None:
            os.environ["LAYOVER_PREFILL_SPLITS"] = saved


def drawn_prefill_case(seed, start, tokens, kv_heads, gqa, layers, fp8, splits):
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    end = start + tokens
    used = -(-end // 16)
    blocks = used + 2
    layer = seed % layers
    pool, bits = make_pool(blocks, layers, kv_heads, seed=seed, fp8=fp8)
    rng = np.random.default_rng(seed)
    block_ids = rng.permutation(blocks)[:used].astype(np.int32)
    q = (torch.randn(kv_heads * gqa, tokens, 128, generator=torch.Generator().manual_seed(seed)) * 2).to(torch.bfloat16).cuda()
    print(f"prefill case start={start} tokens={tokens} kv={kv_heads} gqa={gqa} layers={layers} fp8={fp8} splits={splits}", flush=True)
    out = paged_prefill_attention_hip(q, pool, layer, torch.from_numpy(block_ids).cuda(), start, gqa)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, layer, block_ids, start, gqa))


@pytest.mark.parametrize("layers,kv_heads", [(1, 1), (3, 2), (5, 1)])
def test_unaligned_fp8_records_are_staged_and_match_the_oracle(layers, kv_heads):
    """Records of 2 x layers x kv_heads groups of 2,050 bytes that are not 16-byte aligned are
    read 2 bytes at a time into the BF16 stage, whatever LAYOVER_PREFILL_FP8 asks; the form
    without a workspace, which reads records in place, refuses them."""
    from layover_amd.kernels import _lib
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    assert (2 * layers * kv_heads * 2050) % 16
    start, tokens, gqa = 250, 40, 2
    used = -(-(start + tokens) // 16)
    pool, bits = make_pool(used + 1, layers, kv_heads, seed=layers * 10 + kv_heads, fp8=True)
    block_ids = np.random.default_rng(layers).permutation(used + 1)[:used].astype(np.int32)
    q = torch.randn(kv_heads * gqa, tokens, 128, device="cuda").to(torch.bfloat16)
    print(f"unaligned fp8 records layers={layers} kv={kv_heads}", flush=True)
    out = paged_prefill_attention_hip(q, pool, layers - 1, torch.from_numpy(block_ids).cuda(), start, gqa)
    torch.cuda.synchronize()
    assert_close(out, oracle.prefill_attention(q.float().cpu().numpy(), bits, layers - 1, block_ids, start, gqa))

    shape = _lib.PrefillShape(tokens, start, kv_heads * gqa, kv_heads, 128, layers, 16, layers - 1, _lib.LK_BF16, _lib.LK_FP8_RECORD,
                              1.0 / 128**0.5)
    lib = _lib.load()
    ids = torch.from_numpy(block_ids).cuda()
    status = lib.lk_paged_prefill(shape, q.data_ptr(), pool.records.data_ptr(), ids.data_ptr(), used, out.data_ptr(), None)
    assert status == _lib.LK_ERR_INVALID and b"16-byte aligned" in lib.lk_last_error()


@pytest.mark.parametrize("start,tokens,kv_heads,gqa", [(0, 64, 4, 4), (100, 64, 4, 4), (0, 64, 4, 3), (0, 64, 4, 5), (4, 57, 4, 4)])
@pytest.mark.parametrize("fp8", [False, True], ids=["bf16_pool", "fp8_pool"])
def test_prefill_gives_the_same_bits_on_every_launch(start, tokens, kv_heads, gqa, fp8):
    """Six launches of the same chunk give identical outputs bit for bit. A maximum written as
    inline assembly once read matrix-core results without the wait states the compiler
    inserts for its own instructions: the second 16 rows of a wave then varied from launch
    to launch (still within the north-star tolerance), at GQA 3-5 with two or more key steps."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    end = start + tokens
    used = -(-end // 16)
    pool, _ = make_pool(used + 2, 2, kv_heads, seed=tokens + gqa, fp8=fp8)
    block_ids = torch.from_numpy(np.random.default_rng(start).permutation(used + 2)[:used].astype(np.int32)).cuda()
    q = (torch.randn(kv_heads * gqa, tokens, 128, generator=torch.Generator().manual_seed(7)) * 2).to(torch.bfloat16).cuda()
    print(f"prefill repeat start={start} tokens={tokens} kv={kv_heads} gqa={gqa} fp8={fp8}", flush=True)
    first = paged_prefill_attention_hip(q, pool, 1, block_ids, start, gqa).clone()
    for _ in range(5):
        again = paged_prefill_attention_hip(q, pool, 1, block_ids, start, gqa)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))


@pytest.mark.parametrize("bias", [None, "-6", "-40", "30"], ids=["bias_default", "bias_-6", "bias_-40", "bias_30"])
@pytest.mark.parametrize("fp8", [False, True, "direct"], ids=["bf16_pool", "fp8_pool", "fp8_pool_direct"])
@pytest.mark.parametrize("start,tokens,kv_heads,gqa", [(0, 512, 4, 4), (300, 421, 2, 3), (0, 200, 8, 4)])
def test_paired_key_halves_match_the_oracle_and_repeat(start, tokens, kv_heads, gqa, fp8, bias, monkeypatch):
    """Unsplit chunks whose grid is resident at once divide each heavy tile's key steps between
    the two workgroups of a CU pair; the side that finishes second merges both states. The
    split point moves with LAYOVER_PREFILL_PAIR_BIAS (-40: the heavy side keeps one step;
    30: few or no tiles divide). Results match the oracle, and repeated launches give the same
    bits although which side merges can change from launch to launch."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", "1")
    monkeypatch.setenv("LAYOVER_PREFILL_FP8", "direct" if fp8 == "direct" else "staged")
    if bias is not None:
        monkeypatch.setenv("LAYOVER_PREFILL_PAIR_BIAS", bias)
    end = start + tokens
    used = -(-end // 16)
    pool, state = make_pool(used + 1, 2, kv_heads, seed=tokens + kv_heads, fp8=fp8)
    block_ids = np.random.default_rng(tokens).permutation(used + 1)[:used].astype(np.int32)
    ids = torch.from_numpy(block_ids).cuda()
    q = torch.randn(kv_heads * gqa, tokens, 128, generator=torch.Generator().manual_seed(tokens)).to(torch.bfloat16).cuda()
    print(f"prefill pair halves start={start} tokens={tokens} kv={kv_heads} gqa={gqa} fp8={fp8} bias={bias}", flush=True)
    first = paged_prefill_attention_hip(q, pool, 1, ids, start, gqa).clone()
    torch.cuda.synchronize()
    assert_close(first, oracle.prefill_attention(q.float().cpu().numpy(), state, 1, block_ids, start, gqa))
    for _ in range(3):
        again = paged_prefill_attention_hip(q, pool, 1, ids, start, gqa)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16_pool", "fp8_pool"])
def test_paired_key_halves_replay_in_a_graph(fp8, monkeypatch):
    """A chunk whose heavy tiles divide, captured in a HIP graph: every replay runs with the
    launch tag fixed at capture, so the pair words must be left clean by each launch's merges
    for the next replay to pair up afresh. Before each of four replays the queries change in
    place and an eager launch (its own workspace) gives the expected output; each replay must
    equal it bit for bit, which a merge with the previous replay's state would not."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", "1")
    monkeypatch.setenv("LAYOVER_PREFILL_PAIR_BIAS", "-6")
    start, tokens, kv_heads, gqa = 0, 512, 4, 4
    used = -(-(start + tokens) // 16)
    pool, state = make_pool(used + 1, 2, kv_heads, seed=77, fp8=fp8)
    block_ids = np.random.default_rng(77).permutation(used + 1)[:used].astype(np.int32)
    ids = torch.from_numpy(block_ids).cuda()
    q = torch.randn(kv_heads * gqa, tokens, 128, generator=torch.Generator().manual_seed(77)).to(torch.bfloat16).cuda()
    print(f"prefill pair halves in a graph fp8={fp8}", flush=True)
    eager = paged_prefill_attention_hip(q, pool, 1, ids, start, gqa).clone()
    torch.cuda.synchronize()
    assert_close(eager, oracle.prefill_attention(q.float().cpu().numpy(), state, 1, block_ids, start, gqa))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_prefill_attention_hip(q, pool, 1, ids, start, gqa)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = paged_prefill_attention_hip(q, pool, 1, ids, start, gqa)
    for replay in range(4):
        # New queries each time, so a merge with a state left by the previous replay would show.
        q.copy_(torch.randn(q.shape, generator=torch.Generator().manual_seed(100 + replay)).to(torch.bfloat16))
        expected = paged_prefill_attention_hip(q, pool, 1, ids, start, gqa).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), expected.view(torch.int16))
