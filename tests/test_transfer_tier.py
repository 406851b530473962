"""NativeBackend and CpuTier on the host flavour (reference tests/test_transfer.py and
tests/test_tier.py behaviour): tickets, segmenting, the FP8 ext_* orchestration under slow
and paused streams, blocks held until an offload completes, prefix restores, drops.

The FP8 orchestration runs here with a stand-in codec defined below (a byte copy of each
block's first record_bytes bytes), because this package has no CPU quantizer: what is under
test is the ordering of kernels and copies, not the arithmetic, which the GPU tests check
against the oracle."""

import numpy as np
import pytest
import torch

from layover_amd.config import ModelConfig
from layover_amd.kernels.fp8 import Fp8Layout
from layover_amd.kv.native import build_host
from layover_amd.kv.paged_cache import BlockTable, PagedKVCache
from layover_amd.kv.tier import CpuTier
from layover_amd.kv.transfer import NativeBackend, PlainCopyBackend, ReadyTicket
from oracle import oracle

CFG = ModelConfig.micro()


@pytest.fixture(scope="module", autouse=True)
def built():
    build_host()


def filled_cache(blocks=12, seed=0):
    cache = PagedKVCache(CFG, blocks)
    generator = torch.Generator().manual_seed(seed)
    cache.pool.copy_(torch.randn(cache.pool.shape, generator=generator).to(torch.bfloat16))
    return cache


def block_bytes(cache, ids):
    return b"".join(cache.pool[i].contiguous().view(torch.uint8).numpy().tobytes() for i in ids)


def stand_in_codec(layout):
    """Record = the block's first record_bytes bytes. Deterministic and order-revealing."""

    def quantize(pool, ids, stage, lay):
        flat = pool.view(torch.uint8).reshape(pool.shape[0], -1)
        for i, block in enumerate(ids.tolist()):
            stage[i * lay.record_bytes : (i + 1) * lay.record_bytes] = flat[block, : lay.record_bytes]

    def dequantize(stage, ids, pool, lay):
        flat = pool.view(torch.uint8).reshape(pool.shape[0], -1)
        for i, block in enumerate(ids.tolist()):
            flat[block, : lay.record_bytes] = stage[i * lay.record_bytes : (i + 1) * lay.record_bytes]

    return quantize, dequantize


def test_bf16_round_trip_through_segments_is_byte_exact():
    cache = filled_cache(12)
    backend = NativeBackend("cpu", staging_bytes=3 * cache.block_bytes, ids_capacity=64)
    try:
        out_ids, in_ids = [9, 2, 7, 0, 11, 4, 5], [1, 3, 6, 8, 10, 2, 0]
        before = block_bytes(cache, out_ids)
        ticket = backend.start_out(cache, out_ids)
        ticket.wait()
        assert ticket.payload.memory.numpy().tobytes()[: len(before)] == before
        assert ticket.payload.memory.numpy().tobytes()[: len(before)] == oracle.gather(cache.pool.view(torch.uint8).numpy(), cache.block_bytes, out_ids).tobytes()
        backend.start_in(cache, in_ids, ticket.payload).wait()
        assert block_bytes(cache, in_ids) == before
        assert backend.engine.stats()["kernels"] == 6  # 3 segments each way
        backend.free(ticket.payload)
    finally:
        backend.close()


def test_empty_transfers_are_ready_at_once():
    cache = filled_cache(4)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=8)
    try:
        ticket = backend.start_out(cache, [])
        assert isinstance(ticket, ReadyTicket) and ticket.payload.num_blocks == 0
        assert backend.start_in(cache, [], ticket.payload).done()
    finally:
        backend.close()


def test_out_of_range_blocks_are_refused_before_anything_moves():
    cache = filled_cache(4)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=8)
    try:
        with pytest.raises(ValueError, match="outside a pool"):
            backend.start_out(cache, [1, 4])
        assert backend.engine.stats()["transfers"] == 0
    finally:
        backend.close()


@pytest.mark.parametrize("delay_us", [0, 2000])
def test_fp8_orchestration_orders_kernels_against_copies(delay_us):
    cache = filled_cache(16)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cpu", staging_bytes=2 * layout.record_bytes + 7, ids_capacity=64, fp8_kernels=stand_in_codec(layout))
    try:
        backend.engine.set_copy_delay_us(delay_us)
        out_ids = [15, 3, 8, 0, 12, 1, 9]
        flat = cache.pool.view(torch.uint8).reshape(16, -1)
        expected = b"".join(flat[i, : layout.record_bytes].numpy().tobytes() for i in out_ids)
        ticket = backend.start_out(cache, out_ids, fp8=True)
        ticket.wait()
        assert ticket.payload.fp8 and ticket.payload.record_bytes == layout.record_bytes
        assert ticket.payload.memory.numpy().tobytes() == expected
        in_ids = [2, 4, 5, 6, 7, 10, 11]
        backend.start_in(cache, in_ids, ticket.payload).wait()
        got = b"".join(flat[i, : layout.record_bytes].numpy().tobytes() for i in in_ids)
        assert got == expected
        assert backend.engine.stats()["memcpys"] == 8  # 4 segments of at most 2 records, each way
    finally:
        backend.close()


@pytest.mark.parametrize("delay_us", [0, 1500])
def test_per_block_baseline_copies_once_per_block_or_record(delay_us):
    """start_out_per_block / start_in_per_block (reference transfer.py:435-473): no staging,
    one copy per block each way (BF16) or per record after the whole stand-in quantize (FP8),
    and the same bytes as the staged path."""
    cache = filled_cache(16, seed=4)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=64, fp8_kernels=stand_in_codec(layout))
    try:
        backend.engine.set_copy_delay_us(delay_us)
        out_ids, in_ids = [14, 2, 9, 0, 5], [1, 3, 4, 6, 7]
        bf16 = backend.start_out_per_block(cache, out_ids)
        bf16.wait()
        assert bf16.payload.memory.numpy().tobytes() == block_bytes(cache, out_ids)
        backend.start_in_per_block(cache, in_ids, bf16.payload).wait()
        assert block_bytes(cache, in_ids) == block_bytes(cache, out_ids)
        assert backend.engine.stats()["memcpys"] == 10 and backend.engine.stats()["kernels"] == 0

        flat = cache.pool.view(torch.uint8).reshape(16, -1)
        expected = b"".join(flat[i, : layout.record_bytes].numpy().tobytes() for i in out_ids)
        records = backend.start_out_per_block(cache, out_ids, fp8=True)
        records.wait()
        assert records.payload.fp8 and records.payload.memory.numpy().tobytes() == expected
        targets = [8, 10, 11, 12, 13]
        backend.start_in_per_block(cache, targets, records.payload).wait()
        assert b"".join(flat[i, : layout.record_bytes].numpy().tobytes() for i in targets) == expected
        assert backend.engine.stats()["memcpys"] == 20
        assert isinstance(backend.start_out_per_block(cache, []), ReadyTicket)
    finally:
        backend.close()


def test_fp8_offload_is_not_done_while_the_copy_stream_is_held():
    cache = filled_cache(8)
    layout = Fp8Layout.from_cache(cache)
    backend = NativeBackend("cpu", staging_bytes=layout.record_bytes, ids_capacity=64, fp8_kernels=stand_in_codec(layout))
    try:
        backend.engine.set_paused(True)
        ticket = backend.start_out(cache, [1, 2, 3], fp8=True)
        assert not ticket.done()
        backend.engine.set_paused(False)
        ticket.wait()
        assert ticket.done()
    finally:
        backend.close()


def test_plain_backend_round_trips_bf16():
    cache = filled_cache(6)
    backend = PlainCopyBackend()
    before = block_bytes(cache, [4, 1])
    ticket = backend.start_out(cache, [4, 1])
    assert ticket.done()
    backend.start_in(cache, [0, 5], ticket.payload)
    assert block_bytes(cache, [0, 5]) == before


# CpuTier


def allocated_table(cache, tokens):
    ids = cache.allocator.alloc(cache.blocks_for(tokens))
    return BlockTable(ids, tokens)


def test_tier_holds_blocks_until_the_offload_completes_then_frees_them():
    cache = filled_cache(10)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=8, backend=backend)
    try:
        table = allocated_table(cache, 5 * 16 - 3)
        ids = list(table.blocks)
        before = block_bytes(cache, ids)
        backend.engine.set_paused(True)
        handle = tier.start_offload(cache, table)
        assert table.blocks == [] and table.num_tokens == 0
        assert handle.in_flight and tier.in_flight == 1
        assert all(cache.allocator.refcount(b) == 1 for b in ids)  # held by the tier
        assert tier.blocks_freeing() == 5
        backend.engine.set_paused(False)
        tier.wait_for(handle)
        assert not handle.in_flight and tier.bytes_out == 5 * cache.block_bytes
        assert all(cache.allocator.refcount(b) == 0 for b in ids)
        assert tier.used_blocks == 5 and tier.peak_used_blocks == 5

        restored = tier.restore(cache, handle)
        assert restored.num_tokens == 5 * 16 - 3 and len(restored.blocks) == 5
        assert block_bytes(cache, restored.blocks) == before
        assert tier.used_blocks == 0 and tier.bytes_in == 5 * cache.block_bytes
    finally:
        backend.close()


def test_tier_restores_a_prefix_and_refuses_more_than_it_holds():
    cache = filled_cache(10)
    backend = NativeBackend("cpu", staging_bytes=4 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=8, backend=backend)
    try:
        table = allocated_table(cache, 4 * 16)
        before = block_bytes(cache, table.blocks[:2])
        handle = tier.offload(cache, table)
        with pytest.raises(ValueError):
            tier.start_restore(cache, handle, blocks=5)
        prefix, ticket = tier.start_restore(cache, handle, blocks=2)
        ticket.wait()
        tier.poll()
        assert prefix.num_tokens == 32 and block_bytes(cache, prefix.blocks) == before
        assert tier.used_blocks == 0
    finally:
        backend.close()


def test_tier_capacity_and_in_flight_restore_refusal():
    cache = filled_cache(10)
    backend = NativeBackend("cpu", staging_bytes=4 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=3, backend=backend)
    try:
        with pytest.raises(MemoryError):
            tier.start_offload(cache, allocated_table(cache, 4 * 16))
        backend.engine.set_paused(True)
        handle = tier.start_offload(cache, allocated_table(cache, 2 * 16))
        with pytest.raises(RuntimeError, match="in flight"):
            tier.start_restore(cache, handle)
        backend.engine.set_paused(False)
        tier.flush()
        assert tier.in_flight == 0
    finally:
        backend.close()


def test_dropping_an_offload_in_flight_frees_it_when_it_completes():
    cache = filled_cache(10)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=8, backend=backend)
    try:
        backend.engine.set_paused(True)
        handle = tier.start_offload(cache, allocated_table(cache, 3 * 16))
        tier.drop(handle)
        assert tier.used_blocks == 3
        backend.engine.set_paused(False)
        tier.flush()
        assert tier.used_blocks == 0 and cache.allocator.num_used == 0
    finally:
        backend.close()


def test_blocks_shared_with_a_live_owner_are_not_counted_as_freeing():
    cache = filled_cache(10)
    backend = NativeBackend("cpu", staging_bytes=2 * cache.block_bytes, ids_capacity=64)
    tier = CpuTier(capacity_blocks=8, backend=backend)
    try:
        table = allocated_table(cache, 3 * 16)
        shared = table.blocks[0]
        cache.allocator.incref(shared)  # a fork still uses the first block
        backend.engine.set_paused(True)
        tier.start_offload(cache, table)
        assert tier.blocks_freeing() == 2
        assert tier.blocks_freeing(also_evictable={shared}) == 3
        backend.engine.set_paused(False)
        tier.flush()
        assert cache.allocator.refcount(shared) == 1
    finally:
        backend.close()
