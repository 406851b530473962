"""lk_gather_blocks / lk_scatter_blocks (layover_amd.kernels.blocks) on the GPU: bytes equal
to the oracle's gather and scatter (oracle/kv_oracle.c, after pack.h:41-68) for the Qwen3-4B
block, for block sizes that take the 8-byte-word path, and at block offsets past 4 GiB; and
equal to what the transfer engine's own staged gather delivers."""

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import oracle

pytestmark = pytest.mark.gpu


def random_pool(blocks, block_bytes, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, 256, (blocks, block_bytes), dtype=torch.uint8, generator=gen, device="cuda")


@pytest.mark.parametrize("block_bytes", [2_359_296, 65_536 + 8, 24, 8], ids=["qwen3_4b", "chunk_plus_8", "24_bytes", "8_bytes"])
def test_gather_then_scatter_equal_the_oracle(block_bytes):
    from layover_amd.kernels.blocks import gather_blocks, scatter_blocks

    print(f"block copies: block_bytes {block_bytes}", flush=True)
    blocks = 40
    pool = random_pool(blocks, block_bytes, seed=block_bytes % 1000)
    before = pool.cpu().numpy()
    order = np.random.default_rng(block_bytes % 97).permutation(blocks)
    out_ids, in_ids = [int(i) for i in order[:13]], [int(i) for i in order[13:26]]
    staging = torch.empty(13 * block_bytes, dtype=torch.uint8, device="cuda")
    gather_blocks(pool, torch.tensor(out_ids, dtype=torch.int32, device="cuda"), staging)
    expected = oracle.gather(before.reshape(-1), block_bytes, out_ids)
    assert np.array_equal(staging.cpu().numpy(), expected)
    scatter_blocks(staging, torch.tensor(in_ids, dtype=torch.int32, device="cuda"), pool)
    reference = before.reshape(-1).copy()
    oracle.scatter(reference, block_bytes, in_ids, expected)
    assert np.array_equal(pool.cpu().numpy().reshape(-1), reference)


def test_block_copies_reach_past_4_gib_and_match_the_engine():
    from layover_amd.kernels.blocks import gather_blocks, scatter_blocks
    from layover_amd.kv.native import Engine

    block_bytes = 2_359_296
    print("block copies past 4 GiB: 2,048-block pool", flush=True)
    pool = torch.empty(2048, block_bytes, dtype=torch.uint8, device="cuda")
    ids = [2047, 1901, 3, 2002]
    assert ids[0] * block_bytes > 1 << 32
    gen = torch.Generator(device="cuda").manual_seed(5)
    for block in ids:
        pool[block] = torch.randint(0, 256, (block_bytes,), dtype=torch.uint8, generator=gen, device="cuda")
    source = torch.stack([pool[b] for b in ids]).cpu().numpy().reshape(-1)
    staging = torch.empty(len(ids) * block_bytes, dtype=torch.uint8, device="cuda")
    gather_blocks(pool, torch.tensor(ids, dtype=torch.int32, device="cuda"), staging)
    assert np.array_equal(staging.cpu().numpy(), source)

    torch.cuda.synchronize()
    engine = Engine("hip", staging_bytes=2 * block_bytes, ids_capacity=64)
    try:
        host = engine.host_alloc(len(ids) * block_bytes)
        engine.wait(handle := engine.out_gather(pool.data_ptr(), block_bytes, ids, host))
        engine.release(handle)
        import ctypes

        through_engine = np.frombuffer((ctypes.c_uint8 * (len(ids) * block_bytes)).from_address(host), dtype=np.uint8).copy()
        engine.host_free(host)
    finally:
        engine.destroy()
    assert np.array_equal(through_engine, source)

    targets = torch.tensor([2040, 7, 1999, 2046], dtype=torch.int32, device="cuda")
    scatter_blocks(staging, targets, pool)
    assert np.array_equal(torch.stack([pool[int(b)] for b in targets.tolist()]).cpu().numpy().reshape(-1), source)
    del pool
    torch.cuda.empty_cache()


def test_wrapper_refuses_what_the_kernels_cannot_take():
    from layover_amd.kernels.blocks import gather_blocks

    pool = torch.zeros(4, 64, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        gather_blocks(pool, torch.tensor([0, 1], dtype=torch.int64, device="cuda"), torch.empty(128, dtype=torch.uint8, device="cuda"))
    with pytest.raises(ValueError):
        gather_blocks(pool, torch.tensor([0, 1], dtype=torch.int32, device="cuda"), torch.empty(64, dtype=torch.uint8, device="cuda"))


@settings(max_examples=50, deadline=None, derandomize=True)
@given(
    words=st.integers(1, 9000),
    pool_blocks=st.integers(1, 24),
    picks=st.lists(st.integers(0, 10**6), min_size=0, max_size=24),
    pool_offset=st.sampled_from([0, 8]),
    staging_offset=st.sampled_from([0, 8]),
    seed=st.integers(0, 2**16),
)
def test_block_copies_over_drawn_sizes_counts_and_alignments(words, pool_blocks, picks, pool_offset, staging_offset, seed):
    """Drawn cases: block sizes of 8 to 72,000 bytes (whole 1 KiB chunks or a ragged last one,
    16- or only 8-byte aligned: both word widths), 0-24 blocks, gather ids that repeat, pool
    and staging placed 0 or 8 bytes into their allocations. Bytes equal the oracle's gather
    and scatter; the bytes before and after the copied ranges keep their sentinels."""
    from layover_amd.kernels.blocks import gather_blocks, scatter_blocks

    block_bytes = 8 * words
    print(f"block copy case: {block_bytes} B x {len(picks)} of {pool_blocks}, offsets {pool_offset}/{staging_offset}", flush=True)
    rng = np.random.default_rng(seed)
    pool_total = torch.from_numpy(rng.integers(0, 256, pool_offset + pool_blocks * block_bytes + 64, dtype=np.uint8)).cuda()
    pool = pool_total[pool_offset : pool_offset + pool_blocks * block_bytes].view(pool_blocks, block_bytes)
    before = pool_total.cpu().numpy()
    out_ids = [p % pool_blocks for p in picks]
    staging_total = torch.full((staging_offset + len(out_ids) * block_bytes + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    staging = staging_total[staging_offset : staging_offset + len(out_ids) * block_bytes]

    gather_blocks(pool, torch.tensor(out_ids, dtype=torch.int32, device="cuda"), staging)
    got = staging_total.cpu().numpy()
    expected = oracle.gather(before[pool_offset : pool_offset + pool_blocks * block_bytes], block_bytes, out_ids)
    assert np.array_equal(got[staging_offset : staging_offset + expected.size], expected)
    assert (got[:staging_offset] == 0xA5).all() and (got[staging_offset + expected.size :] == 0xA5).all()

    # Scatter into distinct ids (two writers of one block would race), from the gathered bytes.
    in_ids = [int(i) for i in rng.permutation(pool_blocks)[: min(len(out_ids), pool_blocks)]]
    scatter_blocks(staging[: len(in_ids) * block_bytes], torch.tensor(in_ids, dtype=torch.int32, device="cuda"), pool)
    reference = before.copy()
    oracle.scatter(reference[pool_offset : pool_offset + pool_blocks * block_bytes], block_bytes, in_ids, expected[: len(in_ids) * block_bytes])
    assert np.array_equal(pool_total.cpu().numpy(), reference)


def test_copies_and_record_kernels_of_nothing_accept_null_pointers():
    """count 0 is a no-op whatever the pointers (an empty torch tensor's data pointer is null);
    a bad block size is still refused."""
    from layover_amd.kernels import _lib

    kernels = _lib.load()
    assert kernels.lk_gather_blocks(None, None, 0, 64, None, None) == _lib.LK_OK
    assert kernels.lk_scatter_blocks(None, None, 0, 64, None, None) == _lib.LK_OK
    assert kernels.lk_gather_blocks(None, None, 0, 12, None, None) == _lib.LK_ERR_INVALID
    assert kernels.lk_fp8_quantize(None, None, 0, None, 2048, 576, None) == _lib.LK_OK
    assert kernels.lk_fp8_dequantize(None, None, 0, None, 2048, 576, None) == _lib.LK_OK
