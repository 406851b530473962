"""HIP graphs for the decode data path at small batch sizes.

Mirrors the reference's layover/decode_graphs.py:1-100 on this path. At batch 1 the GPU's
attention work per layer is tens of microseconds, so issuing each layer's launches from
Python sets the pace; a graph records a step's launches once and replays them as one. The
reference captures its whole model step; the model is outside this package, so the unit
captured here is the data path's share of a step: for every layer, the new token's K/V write
into the pool (model.py:139-140: what hip_decode.write_tokens, or Fp8KVPool.write for an
FP8-resident pool, does) and paged decode attention over the block table, as one launch
(hip_decode.run_kernel_append: the workgroups that read a row's last block write its token
first).

As in the reference, each captured batch size gets fixed input tensors: one packed int32
block of rows (write block, write slot, length, block table of fixed width, as
PagedKVCache.decode_rows builds them), q for every layer, and the new tokens' K and V. A
batch smaller than a captured size is padded with rows of length 1 that write and read slot 0
of scratch blocks reserved here and never handed out, one block per padding row (rows of a
fused write name distinct blocks), so a padded row cannot touch a real sequence's KV. Larger
batches, or tables wider than the captured width, get None and run eagerly. The decode
workspace of each size is allocated once, before capture.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from layover_amd.kernels import hip_decode
from layover_amd.kernels.hip_decode import Fp8KVPool
from layover_amd.kv.paged_cache import BlockTable, PagedKVCache

DEFAULT_SIZES = (1, 2, 4, 8)


class Replay:
    """One captured (or eager) step: call it to run the step again; `out` is the tensor every
    run refreshes; `memory_pool` is the graph memory pool for the next capture to share."""

    def __init__(self, run: Callable[[], None], out: torch.Tensor, memory_pool):
        self.run, self.out, self.memory_pool = run, out, memory_pool

    def __call__(self) -> None:
        self.run()


def hip_graph(step: Callable[[], torch.Tensor], memory_pool=None) -> Replay:
    """Records `step` as a HIP graph. torch's capture rules come first: the step runs twice on
    a side stream that waited for the current one (so lazy allocations and library set-up
    happen outside the capture), then the current stream waits for that warm-up."""
    warm = torch.cuda.Stream()
    current = torch.cuda.current_stream()
    warm.wait_stream(current)
    with torch.cuda.stream(warm):
        step()
        step()
    current.wait_stream(warm)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=memory_pool):
        out = step()
    return Replay(graph.replay, out, graph.pool())


def eager_graph(step: Callable[[], torch.Tensor], memory_pool=None) -> Replay:
    """No capture: every run launches `step` again and copies its result into the same output
    tensor, so callers see the buffers a graph would give them."""
    out = step()
    return Replay(lambda: out.copy_(step()), out, memory_pool)


class DecodeAttentionGraphs:
    def __init__(self, cache: PagedKVCache, query_heads: int, pool: torch.Tensor | Fp8KVPool | None = None,
                 sizes: tuple[int, ...] = DEFAULT_SIZES, max_tokens: int | None = None, capture: Callable = hip_graph,
                 q_dtype: torch.dtype = torch.bfloat16):
        """cache supplies the block allocator (for the scratch block) and the shape; `pool`
        is what the steps write and read: the cache's BF16 pool by default, or an Fp8KVPool
        of the same number of blocks."""
        self.cache = cache
        self.pool = cache.pool if pool is None else pool
        cfg = cache.cfg
        self.layers, self.kv_heads, self.head_dim = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
        if query_heads % self.kv_heads:
            raise ValueError(f"{query_heads} query heads do not divide into {self.kv_heads} KV heads")
        self.query_heads = query_heads
        self.groups = query_heads // self.kv_heads
        self.sizes = tuple(sorted(sizes))
        max_tokens = max_tokens or cache.allocator.num_blocks * cache.block_tokens
        self.width = min(cache.blocks_for(max_tokens), cache.allocator.num_blocks)
        # One scratch block per row of the largest size (the packed rows start as all padding):
        # rows of a fused write must name distinct blocks, or two rows re-encoding one FP8
        # group would race.
        self.scratch_blocks = cache.allocator.alloc(max(self.sizes))
        self.scratch = self.scratch_blocks[0]
        device = cache.device
        largest = self.sizes[-1]
        self.packed = torch.zeros(largest, 3 + self.width, dtype=torch.int32, device=device)
        self.packed.copy_(self._padding(largest))
        self.q = torch.zeros(self.layers, largest, query_heads, self.head_dim, dtype=q_dtype, device=device)
        kv_dtype = torch.bfloat16 if isinstance(self.pool, Fp8KVPool) else self.pool.dtype
        self.k_new = torch.zeros(self.layers, largest, self.kv_heads, self.head_dim, dtype=kv_dtype, device=device)
        self.v_new = torch.zeros_like(self.k_new)
        # Table widths captured for every size: the full width and its halvings down to 64
        # blocks. The kernel's split geometry follows the table's width (the lengths are only
        # on the device), so a short batch in a wide table would pay for splits that hold
        # nothing: batch 8 at 4,096 tokens in a 2,048-block table measured 38.6 us per layer
        # against 30.3 in a 256-block one. A step replays the narrowest width its rows fit,
        # as a view of the same packed rows (the table's row stride stays 3 + width).
        self.widths = [self.width]
        while self.widths[-1] // 2 >= 64:
            self.widths.append(self.widths[-1] // 2)
        self._workspaces = {}
        for size in self.sizes:
            for width in self.widths:
                shape = hip_decode.decode_shape(self.q[0, :size], self.pool, 0, self.packed[:size, 3 : 3 + width], self.groups)
                self._workspaces[size, width] = torch.empty(max(hip_decode.workspace_bytes(shape), 4), dtype=torch.uint8, device=device)
        self._replays: dict[tuple[int, int], Replay] = {}
        memory_pool = None
        for size in reversed(self.sizes):  # largest first, so the smaller ones fit in its pool
            for width in self.widths:
                self._replays[size, width] = capture(lambda size=size, width=width: self._step(size, width), memory_pool)
                memory_pool = self._replays[size, width].memory_pool

    def _padding(self, rows: int, first: int = 0) -> torch.Tensor:
        """`rows` rows of length 1, each writing and reading slot 0 of a scratch block of its
        own; `first` is the index of the first padding row among a step's padding rows."""
        padding = torch.zeros(rows, 3 + self.width, dtype=torch.int32)
        for i in range(rows):
            block = self.scratch_blocks[first + i]
            padding[i, 0], padding[i, 2], padding[i, 3] = block, 1, block
        return padding

    def _step(self, size: int, width: int) -> torch.Tensor:
        packed = self.packed[:size]
        table, lengths = packed[:, 3 : 3 + width], packed[:, 2]
        blocks, slots = packed[:, 0], packed[:, 1]
        out = torch.empty(self.layers, size, self.query_heads, self.head_dim, dtype=self.q.dtype, device=self.q.device)
        workspace = self._workspaces[size, width]
        for layer in range(self.layers):
            # The token write and attention as one launch (the write position is the row's last
            # token, as decode_rows packs it): lk_paged_decode_append.
            hip_decode.run_kernel_append(self.q[layer, :size], self.pool, layer, table, lengths, self.groups, blocks, slots,
                                         self.k_new[layer, :size], self.v_new[layer, :size], out[layer], workspace)
        return out

    def release(self) -> None:
        """Gives the scratch blocks back to the cache's allocator; the graphs are unusable after."""
        for block in self.scratch_blocks:
            self.cache.allocator.decref(block)
        self.scratch_blocks = []

    def replay(self, size: int, width: int | None = None) -> torch.Tensor:
        """Replay the captured step of `size` rows and `width` table columns (the full width by
        default) on the buffers as they stand; returns the output tensor that every replay of
        this size and width refreshes."""
        replay = self._replays[size, width or self.width]
        replay()
        return replay.out

    def step_eager(self, size: int, width: int | None = None) -> torch.Tensor:
        """The same step launched eagerly on the same buffers, for comparison."""
        return self._step(size, width or self.width)

    def size_for(self, batch: int) -> int | None:
        return next((size for size in self.sizes if size >= batch), None)

    def width_for(self, tables: list[BlockTable]) -> int | None:
        """The narrowest captured table width the tables fit, or None."""
        needed = max(len(t.blocks) for t in tables)
        return min((w for w in self.widths if w >= needed), default=None)

    def run(self, tables: list[BlockTable], q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor) -> torch.Tensor | None:
        """Attention outputs [layers, batch, query_heads, head_dim] for one decode step of
        tables already prepared for writing (each num_tokens counts the new token), or None
        when no graph fits. q is [layers, batch, query_heads, head_dim]; k_new and v_new are
        [layers, batch, kv_heads, head_dim]. Rows are checked on the host by decode_rows, as
        an eager step's are (reference decode_graphs.py:88-100)."""
        size, width = self.size_for(len(tables)), self.width_for(tables)
        if size is None or width is None:
            return None
        batch = len(tables)
        rows = torch.cat([self.cache.decode_rows(tables, self.width), self._padding(size - batch)])
        self.packed[:size].copy_(rows.to(self.packed.device), non_blocking=True)
        self.q[:, :batch].copy_(q)
        self.q[:, batch:size].zero_()
        self.k_new[:, :batch].copy_(k_new)
        self.v_new[:, :batch].copy_(v_new)
        self.k_new[:, batch:size].zero_()
        self.v_new[:, batch:size].zero_()
        out = self.replay(size, width)
        # The graph refreshes the same tensor on its next replay.
        return out[:, :batch].clone()
