"""The HIP flavour of the transfer library and the FP8 swap pipeline on the GPU.

Bytes are checked exactly: BF16 blocks by CRC and comparison (reference test_native.py:
434-476), FP8 payloads against the oracle's records and restored pools against the oracle's
dequantization (reference test_transfer.py:546-569)."""

import ctypes
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

BLOCK = 8192


@pytest.fixture
def gpu_engine():
    from layover_amd.kv.native import Engine

    torch.cuda.synchronize()
    created = Engine("hip", staging_bytes=4 * BLOCK, ids_capacity=64)
    yield created
    created.destroy()


def filled_pool(blocks, block_bytes=BLOCK, seed=0):
    return torch.randint(0, 256, (blocks * block_bytes,), dtype=torch.uint8, generator=torch.Generator().manual_seed(seed))


def host_bytes(pointer, nbytes):
    return bytes((ctypes.c_uint8 * nbytes).from_address(pointer))


def blocks_of(pool, ids, block_bytes=BLOCK):
    return b"".join(pool[i * block_bytes : (i + 1) * block_bytes].numpy().tobytes() for i in ids)


def test_flavor_is_hip(gpu_engine):
    from layover_amd.kv.native import load_library

    assert load_library("hip").lt_flavor() == b"hip"


def test_gather_scatter_round_trip_is_byte_exact(gpu_engine):
    cpu = filled_pool(32)
    pool = cpu.cuda()
    ids = [int(i) for i in np.random.default_rng(0).permutation(32)[:24]]
    before = zlib.crc32(blocks_of(cpu, ids))
    host = gpu_engine.host_alloc(24 * BLOCK)
    transfer = gpu_engine.out_gather(pool.data_ptr(), BLOCK, ids, host)
    gpu_engine.wait(transfer)
    gpu_engine.release(transfer)
    assert zlib.crc32(host_bytes(host, 24 * BLOCK)) == before
    assert host_bytes(host, 24 * BLOCK) == oracle.gather(cpu.numpy(), BLOCK, ids).tobytes()
    pool.zero_()
    torch.cuda.current_stream().synchronize()
    transfer = gpu_engine.in_scatter(pool.data_ptr(), BLOCK, ids, host)
    gpu_engine.wait(transfer)
    gpu_engine.release(transfer)
    assert zlib.crc32(blocks_of(pool.cpu(), ids)) == before
    assert gpu_engine.stats()["kernels"] == 12


@pytest.mark.parametrize("block_bytes", [8, 64, 65536 + 8, 2_359_296], ids=lambda b: f"{b}B")
def test_odd_block_sizes_take_the_narrow_copy_and_stay_exact(block_bytes):
    from layover_amd.kv.native import Engine

    engine = Engine("hip", staging_bytes=3 * block_bytes, ids_capacity=16)
    try:
        cpu = filled_pool(7, block_bytes, seed=block_bytes)
        pool = cpu.cuda()
        ids = [6, 0, 3, 5, 1]
        host = engine.host_alloc(len(ids) * block_bytes)
        transfer = engine.out_gather(pool.data_ptr(), block_bytes, ids, host)
        engine.wait(transfer)
        engine.release(transfer)
        assert host_bytes(host, len(ids) * block_bytes) == blocks_of(cpu, ids, block_bytes)
        target = torch.zeros_like(pool)
        transfer = engine.in_scatter(target.data_ptr(), block_bytes, [2, 4, 6, 1, 0], host)
        engine.wait(transfer)
        engine.release(transfer)
        assert blocks_of(target.cpu(), [2, 4, 6, 1, 0], block_bytes) == blocks_of(cpu, ids, block_bytes)
        assert blocks_of(target.cpu(), [3, 5], block_bytes) == bytes(2 * block_bytes)
    finally:
        engine.destroy()


def test_a_host_pointer_passed_as_the_pool_is_refused(gpu_engine):
    from layover_amd.kv.native import NativeError

    pool = filled_pool(4)
    host = gpu_engine.host_alloc(BLOCK)
    with pytest.raises(NativeError, match="not memory of HIP device"):
        gpu_engine.out_gather(pool.data_ptr(), BLOCK, [1], host)
    gpu_engine.host_free(host)
    # Refusal is LT_ERR_INVALID: the engine still works.
    pool = filled_pool(4).cuda()
    host = gpu_engine.host_alloc(BLOCK)
    transfer = gpu_engine.out_gather(pool.data_ptr(), BLOCK, [2], host)
    gpu_engine.wait(transfer)
    gpu_engine.release(transfer)


def test_per_block_baseline_round_trip(gpu_engine):
    cpu = filled_pool(8)
    pool = cpu.cuda()
    ids = [5, 0, 3]
    host = gpu_engine.host_alloc(3 * BLOCK)
    transfer = gpu_engine.out_per_block(pool.data_ptr(), BLOCK, ids, host)
    gpu_engine.wait(transfer)
    gpu_engine.release(transfer)
    assert host_bytes(host, 3 * BLOCK) == blocks_of(cpu, ids)


def test_destroy_mid_flight_waits():
    from layover_amd.kv.native import Engine

    engine = Engine("hip", staging_bytes=1 << 22, ids_capacity=4096)
    block = 1 << 20
    pool = filled_pool(256, block).cuda()
    host = engine.host_alloc(256 * block)
    engine.out_gather(pool.data_ptr(), block, list(range(256)), host)
    engine.destroy()
    assert engine.closed
    torch.cuda.synchronize()


def qwen_cache(blocks, seed=0, config=None):
    from layover_amd.config import ModelConfig
    from layover_amd.kv.paged_cache import PagedKVCache

    config = config or ModelConfig.qwen3_4b()
    cache = PagedKVCache(config, blocks, device="cuda", fill=False)
    rng = np.random.default_rng(seed)
    bits = oracle.bf16_bits(rng.standard_normal(cache.pool.shape, dtype=np.float32))
    cache.pool.copy_(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16))
    return cache, bits


@pytest.mark.parametrize("staging_records", [3, 113], ids=["many_segments", "one_segment"])
def test_fp8_swap_round_trip_is_bit_exact_against_the_oracle(staging_records):
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.transfer import NativeBackend

    cache, bits = qwen_cache(24, seed=staging_records)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cuda", staging_bytes=staging_records * layout.record_bytes + 100, ids_capacity=256)
    try:
        out_ids = [int(i) for i in np.random.default_rng(1).permutation(24)[:10]]
        ticket = backend.start_out(cache, out_ids, fp8=True)
        ticket.wait()
        expected = oracle.quantize_records(bits, out_ids, layout.group_elems, layout.groups_per_block)
        assert np.array_equal(ticket.payload.memory.numpy()[: expected.size], expected)

        in_ids = [int(i) for i in np.random.default_rng(2).permutation(24)[:10]]
        before = cache.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        backend.start_in(cache, in_ids, ticket.payload).wait()
        after = cache.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        reference = before.copy()
        oracle.dequantize_records(expected, in_ids, reference, layout.group_elems, layout.groups_per_block)
        assert np.array_equal(after, reference)
        backend.free(ticket.payload)
    finally:
        backend.close()


def test_bf16_swap_round_trip_through_the_backend():
    from layover_amd.kv.transfer import NativeBackend

    cache, bits = qwen_cache(12, seed=3)
    backend = NativeBackend("cuda", staging_bytes=5 * cache.block_bytes, ids_capacity=64)
    try:
        out_ids = [7, 2, 9, 0, 11, 4, 5]
        ticket = backend.start_out(cache, out_ids, fp8=False)
        ticket.wait()
        expected = oracle.gather(bits, cache.block_bytes, out_ids)
        assert np.array_equal(ticket.payload.memory.numpy()[: expected.size], expected)
        in_ids = [1, 3, 6, 8, 10, 2, 0]
        backend.start_in(cache, in_ids, ticket.payload).wait()
        after = cache.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        reference = bits.copy()
        oracle.scatter(reference, cache.block_bytes, in_ids, expected)
        assert np.array_equal(after, reference)
    finally:
        backend.close()


@pytest.mark.parametrize("fp8", [True, False], ids=["fp8", "bf16"])
def test_cpu_tier_offload_and_prefix_restore_on_the_gpu(fp8):
    """CpuTier over the HIP backend (reference tier.py:41-186): the table's blocks stay held
    until the copy completes, and a restored prefix equals the oracle's round trip."""
    from layover_amd.kernels.fp8 import Fp8Layout
    from layover_amd.kv.paged_cache import BlockTable
    from layover_amd.kv.tier import CpuTier
    from layover_amd.kv.transfer import NativeBackend

    cache, bits = qwen_cache(16, seed=7 + fp8)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cuda", staging_bytes=3 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=12, backend=backend, fp8=fp8)
    try:
        tier.prepare(cache)
        table = BlockTable(cache.allocator.alloc(6), 6 * 16 - 5)
        ids = list(table.blocks)
        handle = tier.start_offload(cache, table)
        assert table.blocks == [] and tier.used_blocks == 6
        tier.wait_for(handle)
        assert cache.allocator.num_used == 0 and not handle.in_flight
        if fp8:
            expected = oracle.quantize_records(bits, ids, layout.group_elems, layout.groups_per_block)
        else:
            expected = oracle.gather(bits, cache.block_bytes, ids)
        assert np.array_equal(handle.payload.memory.numpy()[: expected.size], expected)

        cache.pool.zero_()
        prefix, ticket = tier.start_restore(cache, handle, blocks=4)
        ticket.wait()
        tier.poll()
        assert prefix.num_tokens == 64 and tier.used_blocks == 0
        after = cache.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        reference = np.zeros_like(bits)
        if fp8:
            oracle.dequantize_records(expected, prefix.blocks, reference, layout.group_elems, layout.groups_per_block)
        else:
            oracle.scatter(reference, cache.block_bytes, prefix.blocks, expected)
        assert np.array_equal(after, reference)
    finally:
        backend.close()


def test_staging_too_large_for_one_block_copy_launch_is_a_caller_error():
    """A staging buffer holding more 512-byte chunks of a block than one block-copy dispatch
    moves (2^32 work-items, 64 lanes per chunk) is refused with LT_ERR_INVALID, a caller error
    that leaves the engine usable, before any staging is allocated (64 GiB are asked for and
    never allocated): no transfer or kernel is counted."""
    from layover_amd.kv.native import LT_ERR_INVALID, Engine, NativeError

    torch.cuda.synchronize()
    engine = Engine("hip", staging_bytes=64 << 30, ids_capacity=64)
    try:
        block = 2_359_296
        pool = torch.zeros(2 * block, dtype=torch.uint8, device="cuda")
        host = engine.host_alloc(block)
        with pytest.raises(NativeError) as refused:
            engine.out_gather(pool.data_ptr(), block, [1], host)
        assert refused.value.status == LT_ERR_INVALID and "too many chunks" in str(refused.value)
        stats = engine.stats()
        assert stats["transfers"] == 0 and stats["kernels"] == 0, stats
        engine.host_free(host)
    finally:
        engine.destroy()
