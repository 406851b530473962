"""The paged KV pool the data path moves and reads (mirrors layover/kv/paged_cache.py).

Pool layout [block, kind, layer, kv_head, slot, dim], kind 0 = K and 1 = V
(paged_cache.py:40-49): all layers of a block are contiguous, so a block moves as one range
and its FP8 record's groups are (kind, layer, kv_head) in pool order. decode_rows builds the
reference's decode table rows (paged_cache.py:154-169).

A sequence's BlockTable lists its blocks in token order. Growing, sharing and releasing
tables (the reference's paged_cache.py:58-101) belong to the engine's scheduler, outside this
data path; callers build tables from the allocator's ids.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from layover_amd.config import ModelConfig
from layover_amd.kv.allocator import BlockAllocator

KEY, VALUE = 0, 1


@dataclass
class BlockTable:
    blocks: list[int] = field(default_factory=list)
    num_tokens: int = 0


@dataclass
class PrefillChunk:
    """Tokens [start, end) of one sequence as every layer of a prefill chunk sees them
    (model.py:40-50): the ids of every block those tokens and the ones before them occupy,
    and each chunk token's block and slot."""

    start: int
    end: int
    block_ids: torch.Tensor
    write_blocks: torch.Tensor
    write_slots: torch.Tensor

    @property
    def tokens(self) -> int:
        return self.end - self.start


@dataclass(frozen=True)
class DecodeBatch:
    write_blocks: torch.Tensor
    write_slots: torch.Tensor
    table: torch.Tensor
    lengths: torch.Tensor


class PagedKVCache:
    def __init__(self, cfg: ModelConfig, num_blocks: int, device="cpu", dtype=torch.bfloat16, block_tokens: int = 16,
                 fill: bool = True):
        self.cfg = cfg
        self.block_tokens = block_tokens
        self.device = torch.device(device)
        self.dtype = dtype
        self.allocator = BlockAllocator(num_blocks)
        shape = (num_blocks, 2, cfg.num_hidden_layers, cfg.num_key_value_heads, block_tokens, cfg.head_dim)
        self.pool = torch.zeros(shape, dtype=dtype, device=self.device) if fill else torch.empty(shape, dtype=dtype, device=self.device)

    @property
    def block_bytes(self) -> int:
        return self.pool[0].numel() * self.pool.element_size()

    def blocks_for(self, tokens: int) -> int:
        return -(-tokens // self.block_tokens)

    def _upload(self, values) -> torch.Tensor:
        """Host values to the pool's device as one copy. On a GPU it goes through pinned memory
        so that it is queued behind work already launched instead of waiting for it
        (paged_cache.py:103-108)."""
        host = torch.as_tensor(values)
        if self.device.type == "cuda":
            host = host.pin_memory()
        return host.to(self.device, non_blocking=True)

    def chunk_locations(self, table: BlockTable, start: int, count: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Where tokens [start, start + count) of a table live (paged_cache.py:110-116): the
        int32 ids of every block holding them or an earlier token (what a prefill chunk's
        attention reads), then each of the tokens' block id and slot (where its K/V go)."""
        end = start + count
        if start < 0 or count < 1 or end > len(table.blocks) * self.block_tokens:
            raise ValueError(f"tokens [{start}, {end}) do not fit a table of {len(table.blocks)} blocks")
        history = self._upload(np.asarray(table.blocks[: self.blocks_for(end)], dtype=np.int32))
        positions = torch.arange(start, end, device=self.device)
        block_index = torch.div(positions, self.block_tokens, rounding_mode="floor")
        return history, history.index_select(0, block_index).long(), positions - block_index * self.block_tokens

    def chunk(self, table: BlockTable, start: int, count: int) -> PrefillChunk:
        return PrefillChunk(start, start + count, *self.chunk_locations(table, start, count))

    def write_at(self, blocks: torch.Tensor, slots: torch.Tensor, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """k and v, [kv_heads, count, head_dim], stored token by token at (blocks[t], slots[t])
        of `layer` (paged_cache.py:118-122). The pool is addressed as rows of head_dim values:
        row ((block * 2 + kind) * layers + layer) * kv_heads * slots + head * slots + slot."""
        _, _, layers, kv_heads, slots_per_block, head_dim = self.pool.shape
        rows = self.pool.view(-1, head_dim)
        heads = torch.arange(kv_heads, device=self.device) * slots_per_block
        for kind, values in ((KEY, k), (VALUE, v)):
            first = ((blocks.long() * 2 + kind) * layers + layer) * kv_heads * slots_per_block + slots.long()
            index = (first[:, None] + heads[None, :]).reshape(-1)  # [count * kv_heads], token-major
            rows.index_copy_(0, index, values.to(self.dtype).transpose(0, 1).reshape(-1, head_dim))

    def read_blocks(self, ids: torch.Tensor, layer: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
        """K and V of the first `end` tokens held in blocks `ids`, each [kv_heads, end,
        head_dim] (paged_cache.py:124-128): the gather that the paged prefill kernel avoids."""
        picked = self.pool[:, :, layer].index_select(0, ids.long())  # [n, 2, kv_heads, slots, head_dim]
        kv_heads, head_dim = picked.shape[2], picked.shape[4]
        flat = picked.permute(1, 2, 0, 3, 4).reshape(2, kv_heads, -1, head_dim)[:, :, :end]
        return flat[KEY], flat[VALUE]

    def write_range(self, table: BlockTable, layer: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """k and v, [kv_heads, count, head_dim], stored at tokens [start, start + count) of the
        table (paged_cache.py:130-136); the table must already list those tokens' blocks."""
        _, blocks, slots = self.chunk_locations(table, start, k.shape[1])
        self.write_at(blocks, slots, layer, k, v)

    def read_range(self, table: BlockTable, layer: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
        """K and V of the table's first `end` tokens, each [kv_heads, end, head_dim]
        (paged_cache.py:138-141)."""
        ids = self._upload(np.asarray(table.blocks[: self.blocks_for(end)], dtype=np.int64))
        return self.read_blocks(ids, layer, end)

    def decode_rows(self, tables: list[BlockTable], width: int | None = None) -> torch.Tensor:
        """One packed int32 row per table (paged_cache.py:154-169): the block and slot of its
        last token (where this step writes), its length, then its blocks, padded to `width`
        with block 0 (a real block; nothing reads past a length). Checked here on the host,
        so the decode kernel can run trusted."""
        width = max(len(t.blocks) for t in tables) if width is None else width
        rows = np.zeros((len(tables), 3 + width), dtype=np.int32)
        for row, t in zip(rows, tables):
            ids = np.asarray(t.blocks, dtype=np.int64)
            if not 1 <= t.num_tokens <= ids.size * self.block_tokens:
                raise ValueError(f"a table of {ids.size} blocks cannot hold {t.num_tokens} tokens")
            if ids.size and (ids.min() < 0 or ids.max() >= self.allocator.num_blocks):
                raise ValueError(f"block ids {t.blocks} are outside a pool of {self.allocator.num_blocks} blocks")
            if ids.size > width:
                raise ValueError(f"a table of {ids.size} blocks does not fit a width of {width}")
            where, slot = divmod(t.num_tokens - 1, self.block_tokens)
            row[:3] = (ids[where], slot, t.num_tokens)
            row[3 : 3 + ids.size] = ids
        return torch.from_numpy(rows)

    def decode_batch(self, tables: list[BlockTable]) -> DecodeBatch:
        """decode_rows on the device, as the views one decode step's layers take."""
        packed = self._upload(self.decode_rows(tables))
        return DecodeBatch(packed[:, 0].long(), packed[:, 1].long(), packed[:, 3:], packed[:, 2])

    def block_table_tensor(self, tables: list[BlockTable]) -> tuple[torch.Tensor, torch.Tensor]:
        """The decode batch's padded block table [batch, width] and lengths [batch]
        (paged_cache.py:171-175)."""
        batch = self.decode_batch(tables)
        return batch.table, batch.lengths
