"""A CPU memory tier for the KV blocks of paused sessions, over a TransferBackend.

Plays the part of the reference's layover/kv/tier.py (:41-186), with its public names
(CpuTier, CpuHandle and the attributes its callers read) and its rules:

- An offload empties the caller's table at once, but the pool blocks it reads stay
  referenced by the tier until its copy has finished; only then are they given back, so no
  block is handed to another session while it is still being read.
- A restore allocates fresh blocks for a prefix of a handle (all of it by default). They are
  the caller's at once and must not be read before the restore's ticket is done; the
  handle's CPU memory is returned when the restore finishes.
- poll() settles finished copies without blocking; wait_for() and flush() block.
- drop() forgets a handle; one still being offloaded is released when its copy finishes.
- Whether a tier keeps BF16 blocks or FP8 records is fixed when it is built.

Organisation: every copy under way is an object (_Offload or _Restore) that knows what
finishing it means for the tier; the tier keeps them in start order and settles the ones
whose tickets are done.
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Collection

from layover_amd.kv.paged_cache import BlockTable, PagedKVCache
from layover_amd.kv.transfer import Payload, PlainCopyBackend, ReadyTicket, Ticket, TransferBackend


class CpuHandle:
    """One offloaded table. `payload` holds its blocks' records in CPU memory; `held` lists
    the pool blocks its offload still references (empty once the copy has finished)."""

    def __init__(self, num_tokens: int, num_blocks: int, payload: Payload):
        self.num_tokens = num_tokens
        self.num_blocks = num_blocks
        self.payload = payload
        self.held: list[int] = []
        self._copying: _Offload | None = None  # the offload, until it has finished
        self._forgotten = False  # drop() came while the offload was still copying

    @property
    def in_flight(self) -> bool:
        return self._copying is not None


class _Copy:
    """A copy under way and its ticket."""

    def __init__(self, ticket: Ticket, handle: CpuHandle):
        self.ticket = ticket
        self.handle = handle

    def finish(self, tier: CpuTier) -> None:
        raise NotImplementedError


class _Offload(_Copy):
    def __init__(self, ticket: Ticket, handle: CpuHandle, cache: PagedKVCache):
        super().__init__(ticket, handle)
        self.cache = cache

    def finish(self, tier: CpuTier) -> None:
        handle = self.handle
        for block in handle.held:
            self.cache.allocator.decref(block)
        handle.held = []
        handle._copying = None
        tier.bytes_out += handle.payload.nbytes
        if handle._forgotten:
            tier._give_back(handle)


class _Restore(_Copy):
    def __init__(self, ticket: Ticket, handle: CpuHandle, nbytes: int):
        super().__init__(ticket, handle)
        self.nbytes = nbytes

    def finish(self, tier: CpuTier) -> None:
        tier.bytes_in += self.nbytes
        tier._give_back(self.handle)


class CpuTier:
    def __init__(self, capacity_blocks: int, backend: TransferBackend | None = None, fp8: bool = False):
        self.capacity_blocks = capacity_blocks
        self.backend = backend if backend is not None else PlainCopyBackend()
        self.fp8 = fp8
        self.used_blocks = 0
        self.peak_used_blocks = 0
        self.bytes_out = 0
        self.bytes_in = 0
        self._copies: list[_Copy] = []

    # -- state ---------------------------------------------------------------------------

    @property
    def bytes_moved(self) -> int:
        return self.bytes_in + self.bytes_out

    @property
    def in_flight(self) -> int:
        return len(self._copies)

    def has_room(self, blocks: int) -> bool:
        return blocks <= self.capacity_blocks - self.used_blocks

    def prepare(self, cache: PagedKVCache) -> None:
        """Lets the backend set up what a first transfer would otherwise pay for."""
        self.backend.prepare(cache, self.fp8)

    # -- starting copies -----------------------------------------------------------------

    def start_offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        """Starts copying the table's blocks out and empties the table."""
        blocks = list(table.blocks)
        if not self.has_room(len(blocks)):
            raise MemoryError("CPU tier is full")
        ticket = self.backend.start_out(cache, blocks, self.fp8)
        handle = CpuHandle(table.num_tokens, len(blocks), ticket.payload)
        handle.held = blocks  # the table's references pass to the offload
        handle._copying = _Offload(ticket, handle, cache)
        self.used_blocks += len(blocks)
        self.peak_used_blocks = max(self.peak_used_blocks, self.used_blocks)
        table.blocks, table.num_tokens = [], 0
        self._begin(handle._copying)
        return handle

    def start_restore(self, cache: PagedKVCache, handle: CpuHandle, blocks: int | None = None) -> tuple[BlockTable, Ticket]:
        """Starts copying the handle's first `blocks` blocks (all by default) into newly
        allocated ones. Restoring only a prefix leaves the rest unallocated, rather than
        copying blocks nobody reads."""
        if handle.in_flight:
            raise RuntimeError("the handle's offload is still in flight")
        wanted = handle.num_blocks if blocks is None else blocks
        if wanted < 0 or wanted > handle.num_blocks:
            raise ValueError(f"the handle holds {handle.num_blocks} blocks; {wanted} asked for")
        fresh = cache.allocator.alloc(wanted)
        ticket = ReadyTicket() if wanted == 0 else self.backend.start_in(cache, fresh, handle.payload)
        tokens = min(handle.num_tokens, wanted * cache.block_tokens)
        self._begin(_Restore(ticket, handle, wanted * handle.payload.record_bytes))
        return BlockTable(fresh, tokens), ticket

    def _begin(self, copy: _Copy) -> None:
        self._copies.append(copy)
        self.poll()

    # -- finishing copies ----------------------------------------------------------------

    def poll(self) -> bool:
        """Settles every finished copy, in start order; returns whether there was one."""
        running, done = [], []
        for copy in self._copies:
            (done if copy.ticket.done() else running).append(copy)
        self._copies = running
        for copy in done:
            copy.finish(self)
        return len(done) > 0

    def flush(self) -> None:
        """Waits for every copy under way and settles them."""
        for copy in list(self._copies):
            copy.ticket.wait()
        self.poll()

    def wait_for(self, handle: CpuHandle) -> None:
        """Waits for the handle's offload, if it is still copying, and settles it."""
        if handle._copying is not None:
            handle._copying.ticket.wait()
            self.poll()

    def _give_back(self, handle: CpuHandle) -> None:
        self.backend.free(handle.payload)
        self.used_blocks -= handle.num_blocks

    # -- blocking forms ------------------------------------------------------------------

    def offload(self, cache: PagedKVCache, table: BlockTable) -> CpuHandle:
        """start_offload, finished on return: the pool blocks are free again."""
        handle = self.start_offload(cache, table)
        self.wait_for(handle)
        return handle

    def restore(self, cache: PagedKVCache, handle: CpuHandle) -> BlockTable:
        """The whole handle back into new blocks, finished on return."""
        self.wait_for(handle)
        restored, ticket = self.start_restore(cache, handle)
        ticket.wait()
        self.poll()
        return restored

    def drop(self, handle: CpuHandle) -> None:
        """Forgets a handle; its CPU memory goes back now, or when its offload finishes."""
        if handle.in_flight:
            handle._forgotten = True
            return
        self._give_back(handle)

    # -- scheduling hints ----------------------------------------------------------------

    def blocks_freeing(self, also_evictable: Collection[int] = ()) -> int:
        """Pool blocks that finishing offloads will return to the free list: those whose every
        reference is held by offloads, or all but one held by an owner that `also_evictable`
        says gives the block up under pressure. Offloads may share a block (a fork's table
        starts with its parent's), so references are counted per (pool, block)."""
        held_by_offloads: Counter = Counter()
        allocators = {}
        for copy in self._copies:
            if isinstance(copy, _Offload):
                allocators[id(copy.cache)] = copy.cache.allocator
                held_by_offloads.update((id(copy.cache), block) for block in copy.handle.held)
        total = 0
        for (pool, block), held in held_by_offloads.items():
            others = allocators[pool].refcount(block) - held
            if others == 0 or (others == 1 and block in also_evictable):
                total += 1
        return total

    def next_ready_at(self) -> float | None:
        """The earliest finish among copies timed on a virtual clock, if any."""
        clocks = [copy.ticket.ready_at for copy in self._copies if copy.ticket.ready_at is not None]
        return min(clocks) if clocks else None
