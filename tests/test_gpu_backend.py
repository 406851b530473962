"""NativeBackend on the GPU: the orderings and edge cases the reference's own GPU transfer tests
cover (reference tests/test_transfer.py:529-644), with bytes checked exactly against the
oracle instead of CRCs and error bounds: payloads against oracle.gather / quantize_records of
what the pool holds, restores against oracle.scatter / dequantize_records."""

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import oracle

pytestmark = pytest.mark.gpu


def pool_bits(cache, ids=None):
    """The pool (or the listed blocks of it) as BF16 bit patterns on the host."""
    pool = cache.pool if ids is None else cache.pool[torch.tensor(ids, device=cache.pool.device)]
    return pool.view(torch.int16).cpu().numpy().view(np.uint16)


def qwen_cache(blocks, seed):
    from layover_amd.config import ModelConfig
    from layover_amd.kv.paged_cache import PagedKVCache

    cache = PagedKVCache(ModelConfig.qwen3_4b(), blocks, device="cuda", fill=False)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    cache.pool.copy_(torch.randn(cache.pool.shape, generator=gen, device="cuda").to(torch.bfloat16))
    return cache


def expected_payload(cache, ids, fp8):
    from layover_amd.kernels.fp8 import Fp8Layout

    bits = pool_bits(cache, ids)
    local = list(range(len(ids)))
    if fp8:
        layout = Fp8Layout.from_cache(cache)
        return oracle.quantize_records(bits, local, layout.group_elems, layout.groups_per_block)
    return oracle.gather(bits, cache.block_bytes, local)


def payload_bytes(ticket):
    payload = ticket.payload
    return payload.memory.numpy()[: payload.num_blocks * payload.record_bytes]


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_two_overlapping_offloads_through_small_staging_are_both_exact(fp8):
    """Two swap-outs started before either is waited for share the engine's two staging slots
    (3 blocks each); each payload holds exactly its own blocks."""
    from layover_amd.kv.transfer import NativeBackend

    print(f"two overlapping offloads fp8={fp8}", flush=True)
    cache = qwen_cache(40, seed=11)
    backend = NativeBackend("cuda", staging_bytes=3 * cache.block_bytes, ids_capacity=256)
    try:
        order = [int(i) for i in np.random.default_rng(3).permutation(40)]
        first_ids, second_ids = order[:17], order[17:30]
        first = backend.start_out(cache, first_ids, fp8)
        second = backend.start_out(cache, second_ids, fp8)
        second.wait()
        first.wait()
        assert np.array_equal(payload_bytes(first), expected_payload(cache, first_ids, fp8))
        assert np.array_equal(payload_bytes(second), expected_payload(cache, second_ids, fp8))
    finally:
        backend.close()


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_writes_queued_on_torchs_stream_reach_the_swap_out(fp8):
    """A block written by work still queued on torch's current stream when start_out is
    called must leave with the written values: the backend orders its first kernel after the
    caller's stream. The write is a chain of large matrix products, so it is still running
    when the swap starts."""
    from layover_amd.kv.transfer import NativeBackend

    print(f"queued writes reach the swap-out fp8={fp8}", flush=True)
    cache = qwen_cache(16, seed=12)
    backend = NativeBackend("cuda", staging_bytes=8 * cache.block_bytes, ids_capacity=64)
    try:
        for round_number in range(8):
            block = (5 * round_number) % 16
            noise = torch.randn(cache.pool[block].shape, device="cuda")
            cache.pool[block] = (noise @ noise.transpose(-1, -2) @ noise).to(torch.bfloat16)
            ticket = backend.start_out(cache, [block], fp8)
            ticket.wait()
            torch.cuda.synchronize()
            assert np.array_equal(payload_bytes(ticket), expected_payload(cache, [block], fp8)), f"round {round_number}"
            backend.free(ticket.payload)
    finally:
        backend.close()


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_close_while_a_multi_segment_offload_is_in_flight_waits_for_it(fp8):
    from layover_amd.kv.transfer import NativeBackend

    print(f"close mid-flight fp8={fp8}", flush=True)
    cache = qwen_cache(48, seed=13)
    backend = NativeBackend("cuda", staging_bytes=3 * cache.block_bytes, ids_capacity=128)
    ids = [int(i) for i in np.random.default_rng(4).permutation(48)[:40]]
    ticket = backend.start_out(cache, ids, fp8)
    backend.close()
    assert ticket.done()
    assert backend.engine.closed
    torch.cuda.synchronize()


def test_fp8_kernels_run_on_the_backends_stream_not_the_callers():
    """The FP8 kernels are ordered against the copies through the engine's slot events on a
    stream of the backend's own, so a caller's later work on its current stream does not queue
    behind them (reference transfer.py's per-block FP8 path runs off the calling stream too)."""
    from layover_amd.kv.transfer import NativeBackend

    cache = qwen_cache(8, seed=14)
    backend = NativeBackend("cuda", staging_bytes=4 * cache.block_bytes, ids_capacity=64)
    try:
        backend.prepare(cache, fp8=True)
        callers = torch.cuda.current_stream().cuda_stream
        ticket = backend.start_out(cache, [3, 1, 6], fp8=True)
        assert torch.cuda.current_stream().cuda_stream == callers  # the lane is left on return
        ticket.wait()
        stream = backend.kernel_stream
        assert stream is not None
        assert stream.cuda_stream != callers
        assert np.array_equal(payload_bytes(ticket), expected_payload(cache, [3, 1, 6], True))
        backend.start_in(cache, [2, 5, 7], ticket.payload).wait()
        assert torch.cuda.current_stream().cuda_stream == callers
    finally:
        backend.close()


def test_qwen3_4b_blocks_past_4_gib_round_trip_in_both_formats():
    """The real 2,359,296-byte block at ids whose byte offsets need more than 32 bits: BF16
    out and in byte-exact, FP8 out bit-exact against the oracle and in equal to the oracle's
    dequantization."""
    from layover_amd.config import ModelConfig
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.paged_cache import PagedKVCache
    from layover_amd.kv.transfer import NativeBackend

    print("blocks past 4 GiB: 2,048-block pool", flush=True)
    cache = PagedKVCache(ModelConfig.qwen3_4b(), 2048, device="cuda", fill=False)
    assert cache.block_bytes == 2_359_296
    ids, targets = [2047, 2000, 1900, 1], [1950, 1820, 2, 2040]
    assert ids[0] * cache.block_bytes > 1 << 32 and targets[-1] * cache.block_bytes > 1 << 32
    gen = torch.Generator(device="cuda").manual_seed(15)
    for block in ids:
        cache.pool[block] = torch.randn(cache.pool[block].shape, generator=gen, device="cuda").to(torch.bfloat16)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cuda", staging_bytes=3 * cache.block_bytes, ids_capacity=64)
    try:
        source = pool_bits(cache, ids)
        bf16 = backend.start_out(cache, ids, False)
        bf16.wait()
        assert np.array_equal(payload_bytes(bf16), oracle.gather(source, cache.block_bytes, [0, 1, 2, 3]))
        backend.start_in(cache, targets, bf16.payload).wait()
        assert np.array_equal(pool_bits(cache, targets), source)

        records = backend.start_out(cache, ids, True)
        records.wait()
        expected = oracle.quantize_records(source, [0, 1, 2, 3], layout.group_elems, layout.groups_per_block)
        assert np.array_equal(payload_bytes(records), expected)
        backend.start_in(cache, targets, records.payload).wait()
        restored = np.zeros_like(source)
        oracle.dequantize_records(expected, [0, 1, 2, 3], restored, layout.group_elems, layout.groups_per_block)
        assert np.array_equal(pool_bits(cache, targets), restored)
    finally:
        backend.close()
        del cache
        torch.cuda.empty_cache()


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_per_block_baseline_equals_the_oracle(fp8):
    """The per-block baseline (reference transfer.py:435-473) moves the same bytes as the
    staged swap: payload equal to the oracle's, restore equal to the oracle's round trip."""
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.transfer import NativeBackend

    print(f"per-block baseline fp8={fp8}", flush=True)
    cache = qwen_cache(20, seed=16)
    backend = NativeBackend("cuda", staging_bytes=3 * cache.block_bytes, ids_capacity=64)
    try:
        ids, targets = [17, 3, 11, 0, 8], [1, 2, 19, 5, 13]
        source = pool_bits(cache, ids)
        ticket = backend.start_out_per_block(cache, ids, fp8)
        ticket.wait()
        expected = expected_payload(cache, ids, fp8)
        assert np.array_equal(payload_bytes(ticket), expected)
        backend.start_in_per_block(cache, targets, ticket.payload).wait()
        if fp8:
            layout = Fp8Layout.from_cache(cache)
            restored = np.zeros_like(source)
            oracle.dequantize_records(expected, list(range(5)), restored, layout.group_elems, layout.groups_per_block)
        else:
            restored = source
        assert np.array_equal(pool_bits(cache, targets), restored)
        assert backend.engine.stats()["memcpys"] == 10
    finally:
        backend.close()


@settings(max_examples=30, deadline=None, derandomize=True)
@given(
    seed=st.integers(0, 2**16),
    fp8=st.booleans(),
    slot_blocks=st.integers(1, 5),
    slack=st.floats(0.0, 0.99),
    count=st.integers(1, 25),
    num_staging=st.integers(2, 3),
)
def test_staged_swaps_over_drawn_staging_and_counts_equal_the_oracle(seed, fp8, slot_blocks, slack, count, num_staging):
    """Drawn staging slots (1-5 records or blocks, plus a part of one more that no whole block
    fits in) and 1-25 blocks out of the reference's micro shape, so transfers take one segment
    or many with a ragged last one, through two or three slots; out ids may repeat. Payload
    bytes equal the oracle's gather or records, and the restore into distinct ids equals the
    oracle's scatter or dequantization."""
    from layover_amd.config import ModelConfig
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.paged_cache import PagedKVCache
    from layover_amd.kv.transfer import NativeBackend

    cache = PagedKVCache(ModelConfig.micro(), 32, device="cuda", fill=False)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    cache.pool.copy_((torch.randn(cache.pool.shape, generator=gen, device="cuda") * 4).to(torch.bfloat16))
    unit = Fp8Layout.from_cache(cache).record_bytes if fp8 else cache.block_bytes
    staging = slot_blocks * unit + int(slack * unit) // 8 * 8
    rng = np.random.default_rng(seed)
    out_ids = [int(i) for i in rng.integers(0, 32, count)]
    in_ids = [int(i) for i in rng.permutation(32)[:count]]
    print(f"staged swap case fp8={fp8} staging={staging} ({slot_blocks} per slot) x{num_staging} count={count}", flush=True)
    backend = NativeBackend("cuda", staging_bytes=staging, num_staging=num_staging, ids_capacity=64)
    try:
        source = pool_bits(cache, out_ids)
        ticket = backend.start_out(cache, out_ids, fp8)
        ticket.wait()
        expected = expected_payload(cache, out_ids, fp8)
        assert np.array_equal(payload_bytes(ticket), expected)
        before = pool_bits(cache)
        backend.start_in(cache, in_ids, ticket.payload).wait()
        reference = before.reshape(32, -1).copy()
        if fp8:
            layout = Fp8Layout.from_cache(cache)
            restored = np.zeros_like(source)
            oracle.dequantize_records(expected, list(range(count)), restored, layout.group_elems, layout.groups_per_block)
            reference[in_ids] = restored.reshape(count, -1)
        else:
            reference[in_ids] = source.reshape(count, -1)
        assert np.array_equal(pool_bits(cache).reshape(32, -1), reference)
        backend.free(ticket.payload)
    finally:
        backend.close()
