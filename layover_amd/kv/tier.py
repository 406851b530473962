"""A CPU memory tier for the KV blocks of paused sessions, over a TransferBackend.

Plays the part of the reference's layover/kv/tier.py (:41-186) with its interface and rules:

- An offload empties the caller's table at once, but the pool blocks it reads stay
  referenced by the tier until its copy has finished; only then are they given back, so no
  block is handed to another session while it is still being read.
- A restore allocates fresh blocks for a prefix of a handle (all of it by default). They are
  the caller's at once and must not be read before the restore's ticket is done; the
  handle's CPU memory is returned when the restore finishes.
- poll() settles finished copies without blocking; wait_for() and flush() block.
- drop() forgets a handle; one still being offloaded is released when its copy finishes.
- Whether a tier keeps BF16 blocks or FP8 records is fixed when it is built.

Copies under way are kept as jobs, each knowing what to do when its ticket completes.
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Collection
from dataclasses import dataclass, field

from layover_amd.kv.paged_cache import BlockTable, PagedKVCache
from layover_amd.kv.transfer import Payload, PlainCopyBackend, ReadyTicket, Ticket, TransferBackend


@dataclass(eq=False)
class CpuHandle:
    """One offloaded table: its token count, its blocks' records in `payload`, and, while the
    offload is under way, its ticket and the pool blocks it still holds."""

    num_tokens: int
    num_blocks: int
    payload: Payload
    ticket: Ticket | None = None
    held: list[int] = field(default_factory=list)
    cache: PagedKVCache | None = None
    dropped: bool = False

    @property
    def in_flight(self) -> bool:
        return self.ticket is not None


@dataclass(eq=False)
class _Job:
    ticket: Ticket
    handle: CpuHandle
    restore_bytes: int = 0  # 0 for an offload
    is_offload: bool = True


class CpuTier:
    def __init__(self, capacity_blocks: int, backend: TransferBackend | None = None, fp8: bool = False):
        self.capacity_blocks = capacity_blocks
        self.backend = backend if backend is not None else PlainCopyBackend()
        self.fp8 = fp8
        self.used_blocks = 0
        self.peak_used_blocks = 0
        self.bytes_out = 0
        self.bytes_in = 0
        self._jobs: list[_Job] = []

    @property
    def bytes_moved(self) -> int:
        return self.bytes_out + self.bytes_in

    @property
    def in_flight(self) -> int:
        return len(self._jobs)

    def has_room(self, blocks: int) -> bool:
        return self.used_blocks + blocks <= self.capacity_blocks

    def prepare(self, cache: PagedKVCache) -> None:
        self.backend.prepare(cache, self.fp8)

    def start_offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        """Starts copying the table's blocks out and empties the table."""
        blocks = list(table.blocks)
        if not self.has_room(len(blocks)):
            raise MemoryError("CPU tier is full")
        ticket = self.backend.start_out(cache, blocks, self.fp8)
        handle = CpuHandle(table.num_tokens, len(blocks), ticket.payload, ticket, blocks, cache)
        self._charge(len(blocks))
        table.blocks, table.num_tokens = [], 0
        self._jobs.append(_Job(ticket, handle))
        self.poll()
        return handle

    def start_restore(self, cache: PagedKVCache, handle: CpuHandle, blocks: int | None = None) -> tuple[BlockTable, Ticket]:
        """Starts copying the handle's first `blocks` blocks into newly allocated ones. Restoring
        only a prefix leaves the rest unallocated, rather than copying blocks nobody reads."""
        if handle.in_flight:
            raise RuntimeError("the handle's offload is still in flight")
        count = handle.num_blocks if blocks is None else blocks
        if not 0 <= count <= handle.num_blocks:
            raise ValueError(f"the handle holds {handle.num_blocks} blocks; {count} asked for")
        ids = cache.allocator.alloc(count)
        ticket = self.backend.start_in(cache, ids, handle.payload) if count else ReadyTicket()
        table = BlockTable(ids, min(handle.num_tokens, count * cache.block_tokens))
        self._jobs.append(_Job(ticket, handle, count * handle.payload.record_bytes, is_offload=False))
        self.poll()
        return table, ticket

    def poll(self) -> bool:
        """Settles every finished copy; returns whether there was one."""
        finished = [job for job in self._jobs if job.ticket.done()]
        self._jobs = [job for job in self._jobs if job not in finished]
        for job in finished:
            self._settle(job)
        return bool(finished)

    def _settle(self, job: _Job) -> None:
        handle = job.handle
        if job.is_offload:
            for block in handle.held:
                handle.cache.allocator.decref(block)
            handle.held, handle.ticket = [], None
            self.bytes_out += handle.payload.nbytes
            if handle.dropped:
                self._release(handle)
        else:
            self.bytes_in += job.restore_bytes
            self._release(handle)

    def _charge(self, blocks: int) -> None:
        self.used_blocks += blocks
        self.peak_used_blocks = max(self.peak_used_blocks, self.used_blocks)

    def _release(self, handle: CpuHandle) -> None:
        self.backend.free(handle.payload)
        self.used_blocks -= handle.num_blocks

    def blocks_freeing(self, also_evictable: Collection[int] = ()) -> int:
        """Pool blocks that finishing offloads will return to the free list: those whose every
        reference is held by offloads, or all but one held by an owner that `also_evictable`
        says gives the block up under pressure. Offloads may share a block (a fork's table
        starts with its parent's), so references are counted per (pool, block)."""
        holds: Counter = Counter()
        pools = {}
        for job in self._jobs:
            if job.is_offload:
                pools[id(job.handle.cache)] = job.handle.cache.allocator
                holds.update((id(job.handle.cache), block) for block in job.handle.held)
        freeing = 0
        for (pool, block), held in holds.items():
            rest = pools[pool].refcount(block) - held
            freeing += rest == 0 or (rest == 1 and block in also_evictable)
        return freeing

    def next_ready_at(self) -> float | None:
        """The earliest finish among copies timed on a virtual clock, if any."""
        times = [job.ticket.ready_at for job in self._jobs if job.ticket.ready_at is not None]
        return min(times, default=None)

    def flush(self) -> None:
        for job in self._jobs:
            job.ticket.wait()
        self.poll()

    def wait_for(self, handle: CpuHandle) -> None:
        if handle.in_flight:
            handle.ticket.wait()
            self.poll()

    def offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        """start_offload, then wait for it: the blocks are free again on return."""
        handle = self.start_offload(cache, table)
        self.wait_for(handle)
        return handle

    def restore(self, cache: PagedKVCache, handle: CpuHandle) -> BlockTable:
        """The whole handle back into new blocks, finished on return."""
        self.wait_for(handle)
        table, ticket = self.start_restore(cache, handle)
        ticket.wait()
        self.poll()
        return table

    def drop(self, handle: CpuHandle) -> None:
        if handle.in_flight:
            handle.dropped = True
        else:
            self._release(handle)
