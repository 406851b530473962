"""Block ids of a paged KV pool, handed out and reference counted.

Serves the role of the reference's layover/kv/allocator.py (:15-60) with the same interface
(alloc / incref / decref / refcount / num_free / num_used, OutOfBlocks leaving no trace), on
a different policy: every allocation takes the lowest free ids, from a heap. The live part of
the pool then stays packed at its low end whatever order blocks come back in, which keeps the
decode kernel's block reads within the fewest pages of the pool.
"""

from __future__ import annotations

import heapq
from array import array


class OutOfBlocks(RuntimeError):
    """Fewer free blocks than asked for. Nothing was allocated."""


class BlockAllocator:
    def __init__(self, num_blocks: int):
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self.num_blocks = num_blocks
        self._counts = array("I", bytes(4 * num_blocks))  # references per block, 0 = free
        self._free = list(range(num_blocks))  # a valid heap as it stands

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._free)

    def alloc(self, count: int = 1) -> list[int]:
        """`count` blocks, each with one reference, lowest ids first; all or nothing."""
        if count < 0:
            raise ValueError("count must not be negative")
        if count > len(self._free):
            raise OutOfBlocks(f"{count} blocks wanted, {len(self._free)} free")
        taken = [heapq.heappop(self._free) for _ in range(count)]
        for block in taken:
            self._counts[block] = 1
        return taken

    def refcount(self, block: int) -> int:
        return self._counts[block]

    def incref(self, block: int) -> None:
        self._require_live(block)
        self._counts[block] += 1

    def decref(self, block: int) -> bool:
        """Drops one reference; True when that was the last and the block is free again."""
        self._require_live(block)
        self._counts[block] -= 1
        if self._counts[block]:
            return False
        heapq.heappush(self._free, block)
        return True

    def _require_live(self, block: int) -> None:
        if self._counts[block] == 0:
            raise ValueError(f"block {block} is not allocated")
