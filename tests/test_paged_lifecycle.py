"""A sequence's blocks in PagedKVCache (reference paged_cache.py:58-101, :130-141, :171-175):
growth, copy-on-write, fork, truncate, release and range reads/writes, on CPU tensors.

The property test drives several tables through random operations beside a plain model: each
table's tokens as a list of values, and each block's owners. Every token written stores its
value in every element of that token's K and V (both layers, every head), (values BF16 holds
exactly), so a read of a table must return exactly the model's list, whatever sharing and copying happened between;
and the allocator's reference counts must equal the number of tables listing each block (the
reference's allocator state machine, tests/test_kv_properties.py:13-157, checks the same
counts)."""

import pytest
import torch
from hypothesis import settings
from hypothesis import strategies as st
from hypothesis.stateful import RuleBasedStateMachine, invariant, precondition, rule

from layover_amd.config import ModelConfig
from layover_amd.kv.allocator import OutOfBlocks
from layover_amd.kv.paged_cache import BlockTable, PagedKVCache

CFG = ModelConfig.micro()


def write_tokens(cache, table, start, values):
    """Store `values` (one per token) as tokens [start, start + len) of every layer."""
    heads, dim = CFG.num_key_value_heads, CFG.head_dim
    k = torch.tensor(values, dtype=torch.float32)[None, :, None].expand(heads, len(values), dim)
    for layer in range(CFG.num_hidden_layers):
        cache.write_range(table, layer, start, k, -k)


def read_tokens(cache, table):
    """The value of each of the table's tokens, after checking every element agrees."""
    if table.num_tokens == 0:
        return []
    values = None
    for layer in range(CFG.num_hidden_layers):
        k, v = cache.read_range(table, layer, table.num_tokens)
        assert k.shape == (CFG.num_key_value_heads, table.num_tokens, CFG.head_dim)
        assert torch.equal(v, -k)
        column = k[0, :, 0]
        assert torch.equal(k, column[None, :, None].expand_as(k))
        values = column if values is None else values
        assert torch.equal(column, values)
    return [float(x) for x in values]


def test_prepare_write_grows_then_copies_a_shared_partial_block_before_the_write():
    cache = PagedKVCache(CFG, 8)
    parent = BlockTable()
    cache.prepare_write(parent, 0, 20)
    write_tokens(cache, parent, 0, list(range(1, 21)))
    child = cache.fork(parent, 18)
    assert child.blocks == parent.blocks and child.num_tokens == 18
    assert [cache.allocator.refcount(b) for b in parent.blocks] == [2, 2]
    cache.prepare_write(child, 18, 19)
    write_tokens(cache, child, 18, [99])
    assert child.blocks[0] == parent.blocks[0] and child.blocks[1] != parent.blocks[1]
    assert read_tokens(cache, parent) == list(range(1, 21))
    assert read_tokens(cache, child) == list(range(1, 19)) + [99]
    cache.release(parent)
    assert parent.blocks == [] and parent.num_tokens == 0
    assert cache.allocator.num_used == 2
    cache.release(child)
    assert cache.allocator.num_used == 0


def test_fork_past_the_end_and_growth_past_the_pool_are_refused_without_side_effects():
    cache = PagedKVCache(CFG, 3)
    table = BlockTable()
    cache.prepare_write(table, 0, 17)
    with pytest.raises(ValueError):
        cache.fork(table, 18)
    with pytest.raises(OutOfBlocks):
        cache.prepare_write(table, 17, 64)
    assert len(table.blocks) == 2 and table.num_tokens == 17 and cache.allocator.num_used == 2


def test_truncate_keeps_a_partial_block_and_frees_the_rest():
    cache = PagedKVCache(CFG, 6)
    table = BlockTable()
    cache.prepare_write(table, 0, 50)
    write_tokens(cache, table, 0, list(range(50)))
    cache.truncate(table, 17)
    assert len(table.blocks) == 2 and table.num_tokens == 17 and cache.allocator.num_used == 2
    assert read_tokens(cache, table) == list(range(17))
    table_rows, lengths = cache.block_table_tensor([table])
    assert table_rows.tolist() == [table.blocks] and lengths.tolist() == [17]


class TablesMachine(RuleBasedStateMachine):
    BLOCKS = 24

    def __init__(self):
        super().__init__()
        self.cache = PagedKVCache(CFG, self.BLOCKS)
        self.tables: list[BlockTable] = []
        self.model: list[list[float]] = []
        self.next_value = 1.0

    def _values(self, count):
        """Distinct values that BF16 holds exactly: 8-bit significands 128..255 times powers of
        two."""
        first = int(self.next_value)
        self.next_value += count
        return [(128 + n % 128) * 2.0 ** (n // 128 - 20) for n in range(first, first + count)]

    @rule(count=st.integers(1, 40))
    def new_sequence(self, count):
        table = BlockTable()
        try:
            self.cache.prepare_write(table, 0, count)
        except OutOfBlocks:
            self.cache.release(table)
            return
        values = self._values(count)
        write_tokens(self.cache, table, 0, values)
        self.tables.append(table)
        self.model.append(values)

    @precondition(lambda self: self.tables)
    @rule(which=st.integers(0, 1000), count=st.integers(1, 20))
    def append(self, which, count):
        i = which % len(self.tables)
        table = self.tables[i]
        start = table.num_tokens
        before = (list(table.blocks), table.num_tokens, self.cache.allocator.num_used)
        try:
            self.cache.prepare_write(table, start, start + count)
        except OutOfBlocks:
            # Growth is all or nothing per allocation; a failed copy leaves the table usable.
            self.cache.truncate(table, before[1])
            return
        values = self._values(count)
        write_tokens(self.cache, table, start, values)
        self.model[i] = self.model[i] + values

    @precondition(lambda self: self.tables)
    @rule(which=st.integers(0, 1000), fraction=st.floats(0, 1))
    def fork(self, which, fraction):
        i = which % len(self.tables)
        tokens = int(self.tables[i].num_tokens * fraction)
        self.tables.append(self.cache.fork(self.tables[i], tokens))
        self.model.append(self.model[i][:tokens])

    @precondition(lambda self: self.tables)
    @rule(which=st.integers(0, 1000), fraction=st.floats(0, 1))
    def truncate(self, which, fraction):
        i = which % len(self.tables)
        tokens = int(self.tables[i].num_tokens * fraction)
        self.cache.truncate(self.tables[i], tokens)
        self.model[i] = self.model[i][:tokens]

    @precondition(lambda self: self.tables)
    @rule(which=st.integers(0, 1000))
    def release(self, which):
        i = which % len(self.tables)
        self.cache.release(self.tables.pop(i))
        self.model.pop(i)

    @invariant()
    def contents_match_the_model(self):
        for table, values in zip(self.tables, self.model):
            assert table.num_tokens == len(values)
            assert len(table.blocks) == self.cache.blocks_for(table.num_tokens)
            assert read_tokens(self.cache, table) == values

    @invariant()
    def reference_counts_are_the_number_of_holders(self):
        holders = {}
        for table in self.tables:
            for block in table.blocks:
                holders[block] = holders.get(block, 0) + 1
        for block in range(self.BLOCKS):
            assert self.cache.allocator.refcount(block) == holders.get(block, 0)
        assert self.cache.allocator.num_used == len(holders)


TablesMachine.TestCase.settings = settings(max_examples=30, stateful_step_count=25, deadline=None, derandomize=True)
test_tables_behave_like_lists_of_tokens = TablesMachine.TestCase
