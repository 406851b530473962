"""The paged KV pool the data path moves and reads (mirrors layover/kv/paged_cache.py).

Pool layout [block, kind, layer, kv_head, slot, dim], kind 0 = K and 1 = V
(paged_cache.py:40-49): all layers of a block are contiguous, so a block moves as one range
and its FP8 record's groups are (kind, layer, kv_head) in pool order. decode_rows builds the
reference's decode table rows (paged_cache.py:154-169).
"""

from __future__ import annotations

from dataclasses import dataclass, field

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

    def _to_device(self, host: torch.Tensor) -> torch.Tensor:
        """One copy to the device, from pinned memory so it queues behind launched work
        (paged_cache.py:103-108)."""
        if self.device.type != "cuda":
            return host.to(self.device)
        return host.pin_memory().to(self.device, non_blocking=True)

    def chunk_locations(self, table: BlockTable, start: int, count: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """For tokens [start, start + count): the ids of every block they and the tokens before
        them occupy (int32), then each token's block and slot (paged_cache.py:110-116)."""
        if start < 0 or count < 1 or start + count > len(table.blocks) * self.block_tokens:
            raise ValueError(f"tokens [{start}, {start + count}) do not fit a table of {len(table.blocks)} blocks")
        ids = self._to_device(torch.tensor(table.blocks[: self.blocks_for(start + count)], dtype=torch.int32))
        positions = torch.arange(start, start + count, device=self.device)
        return ids, ids[positions // self.block_tokens].long(), positions % self.block_tokens

    def chunk(self, table: BlockTable, start: int, count: int) -> PrefillChunk:
        return PrefillChunk(start, start + count, *self.chunk_locations(table, start, count))

    def write_at(self, blocks: torch.Tensor, slots: torch.Tensor, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Store k and v of shape [kv_heads, count, head_dim] at the given blocks and slots
        (paged_cache.py:118-122)."""
        self.pool[blocks, KEY, layer, :, slots] = k.transpose(0, 1).to(self.dtype)
        self.pool[blocks, VALUE, layer, :, slots] = v.transpose(0, 1).to(self.dtype)

    def read_blocks(self, ids: torch.Tensor, layer: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
        """K and V of the first `end` tokens held in blocks `ids`, as [kv_heads, end, head_dim]
        (paged_cache.py:124-128): the gather the paged prefill kernel avoids."""
        ids = ids.long()
        k = self.pool[ids, KEY, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :end]
        v = self.pool[ids, VALUE, layer].permute(1, 0, 2, 3).flatten(1, 2)[:, :end]
        return k, v

    def decode_rows(self, tables: list[BlockTable], width: int | None = None) -> torch.Tensor:
        """int32 [batch, 3 + width]: write block, write slot, length, then the block table padded
        with block 0 (paged_cache.py:154-169). Checked on the host, so the decode kernel can
        run trusted."""
        width = max(len(t.blocks) for t in tables) if width is None else width
        rows = []
        for t in tables:
            if not 1 <= t.num_tokens <= len(t.blocks) * self.block_tokens:
                raise ValueError(f"a table of {len(t.blocks)} blocks cannot hold {t.num_tokens} tokens")
            if t.blocks and not 0 <= min(t.blocks) <= max(t.blocks) < self.allocator.num_blocks:
                raise ValueError(f"block ids {t.blocks} are outside a pool of {self.allocator.num_blocks} blocks")
            if len(t.blocks) > width:
                raise ValueError(f"a table of {len(t.blocks)} blocks does not fit a width of {width}")
            last = t.num_tokens - 1
            rows.append([t.blocks[last // self.block_tokens], last % self.block_tokens, t.num_tokens, *t.blocks,
                         *[0] * (width - len(t.blocks))])
        return torch.tensor(rows, dtype=torch.int32)

    def decode_batch(self, tables: list[BlockTable]) -> DecodeBatch:
        rows = self.decode_rows(tables)
        packed = rows.pin_memory().to(self.device, non_blocking=True) if self.device.type == "cuda" else rows
        return DecodeBatch(packed[:, 0].long(), packed[:, 1].long(), packed[:, 3:], packed[:, 2])
