"""PagedKVCache's host-side helpers on CPU tensors, against element-by-element loops over the
layout [block, kind, layer, kv_head, slot, dim] (paged_cache.py:40-49 of the reference)."""

import numpy as np
import pytest
import torch

from layover_amd.config import ModelConfig
from layover_amd.kv.paged_cache import KEY, VALUE, BlockTable, PagedKVCache


@pytest.fixture
def cache():
    made = PagedKVCache(ModelConfig.micro(), 10)
    made.pool.copy_(torch.randn(made.pool.shape, generator=torch.Generator().manual_seed(1)).to(made.pool.dtype))
    return made


def test_write_at_stores_each_token_at_its_block_and_slot(cache):
    _, _, layers, heads, slots, dim = cache.pool.shape
    blocks = torch.tensor([7, 2, 2, 9, 0])
    where = torch.tensor([3, 0, 5, slots - 1, 1])
    k = torch.randn(heads, 5, dim)
    v = torch.randn(heads, 5, dim)
    expected = cache.pool.clone()
    for t in range(5):
        for h in range(heads):
            expected[blocks[t], KEY, 1, h, where[t]] = k[h, t].to(expected.dtype)
            expected[blocks[t], VALUE, 1, h, where[t]] = v[h, t].to(expected.dtype)
    cache.write_at(blocks, where, 1, k, v)
    assert torch.equal(cache.pool, expected)


def test_read_blocks_concatenates_the_blocks_tokens_in_order(cache):
    ids = torch.tensor([4, 1, 8])
    slots = cache.pool.shape[4]
    end = 2 * slots + 3
    k, v = cache.read_blocks(ids, 1, end)
    heads = cache.pool.shape[3]
    for h in range(heads):
        for t in range(end):
            block, slot = int(ids[t // slots]), t % slots
            assert torch.equal(k[h, t], cache.pool[block, KEY, 1, h, slot])
            assert torch.equal(v[h, t], cache.pool[block, VALUE, 1, h, slot])
    assert k.shape == (heads, end, cache.pool.shape[5])


def test_chunk_locations_name_every_token(cache):
    slots = cache.block_tokens
    table = BlockTable([6, 3, 9, 1], 4 * slots)
    history, blocks, where = cache.chunk_locations(table, slots - 2, slots + 5)
    assert history.dtype == torch.int32 and history.tolist() == [6, 3, 9]
    positions = range(slots - 2, 2 * slots + 3)
    assert blocks.tolist() == [table.blocks[p // slots] for p in positions]
    assert where.tolist() == [p % slots for p in positions]
    with pytest.raises(ValueError):
        cache.chunk_locations(table, 3 * slots, 2 * slots)


def test_decode_rows_pack_write_position_length_and_padded_table(cache):
    slots = cache.block_tokens
    rows = cache.decode_rows([BlockTable([3, 7], slots + 4), BlockTable([5], 1), BlockTable([1, 2, 9], 3 * slots)], width=4).numpy()
    assert rows.dtype == np.int32
    assert rows.tolist() == [[7, 3, slots + 4, 3, 7, 0, 0], [5, 0, 1, 5, 0, 0, 0], [9, slots - 1, 3 * slots, 1, 2, 9, 0]]
    for bad in ([BlockTable([3], slots + 1)], [BlockTable([3], 0)], [BlockTable([10], 1)], [BlockTable([-1], 1)]):
        with pytest.raises(ValueError):
            cache.decode_rows(bad)
    with pytest.raises(ValueError):
        cache.decode_rows([BlockTable([1, 2, 3], 5)], width=2)
