"""lk_gather_blocks / lk_scatter_blocks (layover_amd.kernels.blocks) on the GPU: bytes equal
to the oracle's gather and scatter (oracle/kv_oracle.c, after pack.h:41-68) for the Qwen3-4B
block, for block sizes that take the 8-byte-word path, and at block offsets past 4 GiB; and
equal to what the transfer engine's own staged gather delivers."""

import numpy as np
import pytest
import torch

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
