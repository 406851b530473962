"""CPU memory tier for the KV blocks of paused sessions, asynchronous over a TransferBackend.

Mirrors the reference's layover/kv/tier.py:41-186 (same class, methods and semantics):
  - start_offload moves a table's blocks out and empties the table at once; the pool blocks
    stay referenced by the tier until the copy completes, and only then go back to the
    allocator (a block still being read must not be handed to another session);
  - start_restore allocates fresh blocks for a prefix of a handle and copies into them; the
    caller owns them immediately but must not touch them until the ticket is done, and the
    handle's host memory is released when the restore completes;
  - poll() settles whatever finished, never blocking; flush()/wait_for() block;
  - drop() forgets a handle (one still offloading frees itself when the copy completes);
  - blocks_freeing() counts pool blocks that completing offloads will give back.
Whether a tier stores BF16 or FP8 records is fixed when it is built.
"""

from __future__ import annotations

from collections.abc import Collection
from dataclasses import dataclass, field

from layover_amd.kv.paged_cache import BlockTable, PagedKVCache
from layover_amd.kv.transfer import Payload, PlainCopyBackend, ReadyTicket, Ticket, TransferBackend


@dataclass(eq=False)
class CpuHandle:
    num_tokens: int
    num_blocks: int
    payload: Payload
    ticket: Ticket | None = None
    held: list[int] = field(default_factory=list)  # pool blocks referenced until the offload completes
    cache: PagedKVCache | None = None
    dropped: bool = False

    @property
    def in_flight(self) -> bool:
        return self.ticket is not None


@dataclass(eq=False)
class _Restore:
    ticket: Ticket
    handle: CpuHandle
    bytes_moved: int


class CpuTier:
    def __init__(self, capacity_blocks: int, backend: TransferBackend | None = None, fp8: bool = False):
        self.capacity_blocks = capacity_blocks
        self.backend = backend or PlainCopyBackend()
        self.fp8 = fp8
        self.used_blocks = 0
        self.peak_used_blocks = 0
        self.bytes_out = 0
        self.bytes_in = 0
        self._offloading: list[CpuHandle] = []
        self._restoring: list[_Restore] = []

    @property
    def bytes_moved(self) -> int:
        return self.bytes_out + self.bytes_in

    @property
    def in_flight(self) -> int:
        return len(self._offloading) + len(self._restoring)

    def has_room(self, blocks: int) -> bool:
        return self.used_blocks + blocks <= self.capacity_blocks

    def prepare(self, cache: PagedKVCache) -> None:
        self.backend.prepare(cache, self.fp8)

    def start_offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        """Begin copying a table's blocks out; the table is empty afterwards."""
        blocks = list(table.blocks)
        if not self.has_room(len(blocks)):
            raise MemoryError("CPU tier is full")
        ticket = self.backend.start_out(cache, blocks, self.fp8)
        handle = CpuHandle(table.num_tokens, len(blocks), ticket.payload, ticket, blocks, cache)
        self.used_blocks += len(blocks)
        self.peak_used_blocks = max(self.peak_used_blocks, self.used_blocks)
        table.blocks = []
        table.num_tokens = 0
        self._offloading.append(handle)
        self.poll()
        return handle

    def start_restore(self, cache: PagedKVCache, handle: CpuHandle, blocks: int | None = None) -> tuple[BlockTable, Ticket]:
        """Begin copying a handle's first `blocks` blocks (all by default) into new blocks."""
        if handle.in_flight:
            raise RuntimeError("the handle's offload is still in flight")
        count = handle.num_blocks if blocks is None else blocks
        if count > handle.num_blocks:
            raise ValueError(f"handle holds {handle.num_blocks} blocks, asked for {count}")
        ids = cache.allocator.alloc(count)
        ticket = self.backend.start_in(cache, ids, handle.payload) if count else ReadyTicket()
        table = BlockTable(ids, min(handle.num_tokens, count * cache.block_tokens))
        self._restoring.append(_Restore(ticket, handle, count * handle.payload.record_bytes))
        self.poll()
        return table, ticket

    def poll(self) -> bool:
        """Settle completed copies without blocking; returns whether any completed."""
        settled = False
        still = []
        for handle in self._offloading:
            if handle.ticket.done():
                self._offload_done(handle)
                settled = True
            else:
                still.append(handle)
        self._offloading = still
        pending = []
        for restore in self._restoring:
            if restore.ticket.done():
                self.bytes_in += restore.bytes_moved
                self._free(restore.handle)
                settled = True
            else:
                pending.append(restore)
        self._restoring = pending
        return settled

    def _offload_done(self, handle: CpuHandle) -> None:
        for block in handle.held:
            handle.cache.allocator.decref(block)
        handle.held = []
        handle.ticket = None
        self.bytes_out += handle.payload.nbytes
        if handle.dropped:
            self._free(handle)

    def _free(self, handle: CpuHandle) -> None:
        self.backend.free(handle.payload)
        self.used_blocks -= handle.num_blocks

    def blocks_freeing(self, also_evictable: Collection[int] = ()) -> int:
        """Pool blocks that return to the free list once offloads in flight complete: every
        reference is held by offloads, apart from at most one owner named in also_evictable."""
        counts: dict[tuple[int, int], int] = {}
        allocators = {}
        for handle in self._offloading:
            allocators[id(handle.cache)] = handle.cache.allocator
            for block in handle.held:
                key = (id(handle.cache), block)
                counts[key] = counts.get(key, 0) + 1
        freeing = 0
        for (cache_id, block), held in counts.items():
            others = allocators[cache_id].refcount(block) - held
            if others == 0 or (others == 1 and block in also_evictable):
                freeing += 1
        return freeing

    def next_ready_at(self) -> float | None:
        times = [t.ready_at for t in [h.ticket for h in self._offloading] + [r.ticket for r in self._restoring] if t.ready_at is not None]
        return min(times) if times else None

    def flush(self) -> None:
        for handle in self._offloading:
            handle.ticket.wait()
        for restore in self._restoring:
            restore.ticket.wait()
        self.poll()

    def wait_for(self, handle: CpuHandle) -> None:
        if handle.in_flight:
            handle.ticket.wait()
            self.poll()

    def offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        handle = self.start_offload(cache, table)
        self.wait_for(handle)
        return handle

    def restore(self, cache: PagedKVCache, handle: CpuHandle) -> BlockTable:
        self.wait_for(handle)
        table, ticket = self.start_restore(cache, handle)
        ticket.wait()
        self.poll()
        return table

    def drop(self, handle: CpuHandle) -> None:
        if handle.in_flight:
            handle.dropped = True
        else:
            self._free(handle)
