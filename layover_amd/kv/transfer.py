"""KV blocks between the pool and pinned CPU memory, behind tickets.

The interface is the reference's layover/kv/transfer.py one, so CpuTier and a scheduler
drive it unchanged: a backend's start_out / start_in return a Ticket (done() never blocks,
wait() does) whose payload is an array of equal records in CPU memory, any prefix of which
can be restored; free / prepare / pin_stats / close as there (transfer.py:45-117).

PlainCopyBackend (transfer.py:120-144) copies through torch and is finished on return.

NativeBackend (transfer.py:289-565) drives the swap library (include/layover_transfer.h):
  BF16   lt_out_gather / lt_in_scatter: the library's gather or scatter kernel and one DMA
         per staging segment, overlapped over two slots.
  FP8    this package's fused kernels (lk_fp8_quantize / lk_fp8_dequantize) write or read
         record segments in staging tensors owned here, on a stream of this backend; the
         library's per-slot events (lt_ext_*) order each segment's kernel against its DMA on
         the library's copy stream. All of a transfer's block ids go to the device once, from
         pinned memory, ahead of its first kernel.
On the host flavour the same orchestration runs on host threads; the FP8 kernels must then
be given (`fp8_kernels`), because this package has no CPU codec.
"""

from __future__ import annotations

import contextlib

import ctypes
from abc import ABC, abstractmethod
from collections.abc import Callable
from dataclasses import dataclass

import torch

from layover_amd.kernels.fp8 import Fp8Layout, dequantize_blocks, quantize_blocks
from layover_amd.kv.native import SLOT_FILLED, SLOT_RELEASED, Engine, HostMemoryError, NativeError, NativeUnavailable, build_host
from layover_amd.kv.paged_cache import PagedKVCache

__all__ = [
    "HostMemoryError",
    "NativeBackend",
    "NativeError",
    "NativeUnavailable",
    "Payload",
    "PlainCopyBackend",
    "ReadyTicket",
    "Ticket",
    "TransferBackend",
    "make_backend",
]

# The engine counters that describe pinning stalls, as the reference reports them.
PIN_STATS = ("host_pins", "host_pin_bytes", "host_pin_ns", "host_pin_max_ns", "host_pin_failures")


class Payload:
    """Offloaded blocks in CPU memory: num_blocks records of record_bytes (FP8 records or raw
    BF16 blocks) in `memory`, a flat uint8 tensor. Valid once the offload's ticket is done."""

    def __init__(self, memory: torch.Tensor | None, num_blocks: int, record_bytes: int, fp8: bool, pointer: int | None = None):
        self.memory = memory
        self.num_blocks = num_blocks
        self.record_bytes = record_bytes
        self.fp8 = fp8
        self.pointer = pointer  # the engine's pinned buffer, when the engine owns the memory

    @property
    def nbytes(self) -> int:
        return self.num_blocks * self.record_bytes


class Ticket(ABC):
    """A copy under way."""

    payload: Payload | None = None
    ready_at: float | None = None  # for copies timed on a virtual clock; real ones leave it None

    @abstractmethod
    def done(self) -> bool:
        """Whether the copy has finished; never blocks."""

    @abstractmethod
    def wait(self) -> None:
        """Blocks until the copy has finished."""


class ReadyTicket(Ticket):
    def __init__(self, payload: Payload | None = None):
        self.payload = payload

    def done(self) -> bool:
        return True

    def wait(self) -> None:
        return None


class TransferBackend(ABC):
    name = ""

    @abstractmethod
    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        """Copy `blocks` out, in order, into ticket.payload. The caller keeps them allocated and
        unwritten until the ticket is done."""

    @abstractmethod
    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        """Copy the payload's first len(blocks) records into `blocks`. The caller keeps the
        payload alive and the blocks unread until the ticket is done."""

    def free(self, payload: Payload) -> None:
        """Return a payload's memory; its offload and restores must have finished."""

    def prepare(self, cache: PagedKVCache, fp8: bool = False) -> None:
        """Do first-use work (staging) now rather than inside the first transfer."""

    def pin_stats(self) -> dict[str, int]:
        return {}

    def close(self) -> None:
        return None


def record_bytes(cache: PagedKVCache, fp8: bool) -> int:
    return Fp8Layout.from_cache(cache).record_bytes if fp8 else cache.block_bytes


class PlainCopyBackend(TransferBackend):
    """Copies through torch, finished when they return. BF16 blocks are gathered and scattered
    at most `piece` blocks per torch call: one index kernel over thousands of 2.36 MB blocks
    is more than it should be asked for (such a gather faulted on a 12 GiB pool)."""

    name = "plain"
    piece = 256

    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        index = torch.tensor(blocks, dtype=torch.long, device=cache.device)
        if fp8:
            layout = Fp8Layout.from_cache(cache)
            stage = torch.empty(len(blocks) * layout.record_bytes, dtype=torch.uint8, device=cache.device)
            quantize_blocks(cache.pool, index.to(torch.int32), stage, layout)
            host = stage.cpu()
        else:
            host = torch.empty(len(blocks) * cache.block_bytes, dtype=torch.uint8)
            for first in range(0, len(blocks), self.piece):
                part = cache.pool.index_select(0, index[first : first + self.piece]).cpu().view(torch.uint8).reshape(-1)
                host[first * cache.block_bytes : first * cache.block_bytes + part.numel()] = part
        return ReadyTicket(Payload(host, len(blocks), record_bytes(cache, fp8), fp8))

    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        index = torch.tensor(blocks, dtype=torch.long, device=cache.device)
        records = payload.memory[: len(blocks) * payload.record_bytes].to(cache.device)
        if payload.fp8:
            dequantize_blocks(records, index.to(torch.int32), cache.pool, Fp8Layout.from_cache(cache))
        else:
            rows = records.view(cache.pool.dtype).view(len(blocks), *cache.pool.shape[1:])
            for first in range(0, len(blocks), self.piece):
                cache.pool.index_copy_(0, index[first : first + self.piece], rows[first : first + self.piece])
        return ReadyTicket()


class _EngineTicket(Ticket):
    """An lt_transfer of the backend's engine, released as soon as it is seen finished; it
    keeps the tensors its kernels use alive until then."""

    def __init__(self, engine: Engine, handle: int, payload: Payload | None, holds: list):
        self.payload = payload
        self._engine = engine
        self._handle: int | None = handle
        self._holds: list | None = holds

    def _finished(self) -> None:
        self._engine.release(self._handle)
        self._handle, self._holds = None, None

    def done(self) -> bool:
        if self._handle is None or self._engine.closed:  # closing the engine waited for it
            return True
        if self._engine.poll(self._handle):
            self._finished()
            return True
        return False

    def wait(self) -> None:
        if self._handle is None or self._engine.closed:
            return
        self._engine.wait(self._handle)
        self._finished()


Fp8Kernel = Callable[[torch.Tensor, torch.Tensor, torch.Tensor, Fp8Layout], None]


@dataclass
class _Segment:
    slot: int
    first: int  # index of its first block within the transfer
    count: int


class _KernelLane:
    """Where this backend's FP8 kernels run: a torch stream of its own on a GPU, the engine's
    caller stream (a host thread) on the host flavour."""

    def __init__(self, engine: Engine, device: torch.device):
        self._engine = engine
        self._device = device
        self._stream = torch.cuda.Stream(device=device) if engine.flavor == "hip" else None
        self._entered = False

    @property
    def handle(self) -> int:
        return self._stream.cuda_stream if self._stream is not None else self._engine.host_stream()

    @property
    def stream(self):
        return self._stream

    @contextlib.contextmanager
    def active(self):
        """Makes the lane torch's current stream for a whole transfer, so its uploads and
        kernels are queued without switching streams once per launch (about 7 us each)."""
        if self._stream is None or self._entered:
            yield
            return
        with torch.cuda.stream(self._stream):
            self._entered = True
            try:
                yield
            finally:
                self._entered = False

    def run(self, work: Callable[[], None], holds: list) -> None:
        if self._stream is None:
            holds.append(self._engine.host_call(self.handle, work))
            return
        with self.active():
            work()

    def upload(self, blocks: list[int], holds: list) -> torch.Tensor:
        """The block ids as int32 on the device, copied from pinned memory in this lane's
        order (from pageable memory the copy would block the host until the stream drains)."""
        if self._stream is None:
            return torch.tensor(blocks, dtype=torch.int32)
        pinned = torch.tensor(blocks, dtype=torch.int32, pin_memory=True)
        with self.active():
            on_device = pinned.to(self._device, non_blocking=True)
        holds += [pinned, on_device]
        return on_device


class NativeBackend(TransferBackend):
    """Staged swaps through the native library; see the module docstring."""

    name = "native"

    def __init__(self, device: torch.device | str = "cpu", staging_bytes: int = 128 << 20, num_staging: int = 2,
                 ids_capacity: int = 1 << 20, host_cache_bytes: int = 8 << 30, fp8_impl: str | None = None,
                 fp8_kernels: tuple[Fp8Kernel, Fp8Kernel] | None = None):
        self.device = torch.device(device)
        if self.device.type == "cuda":
            self.flavor = "hip"  # torch-ROCm's name for the GPU; the library's flavour is hip
        elif self.device.type == "cpu":
            self.flavor = "host"
            build_host()
        else:
            raise ValueError(f"no native transfer path for device {device}")
        if fp8_impl not in (None, "hip"):
            raise ValueError(f"the FP8 kernels here are the 'hip' ones, not {fp8_impl!r}")
        ordinal = (self.device.index or 0) if self.flavor == "hip" else 0
        self.engine = Engine(self.flavor, ordinal, staging_bytes, num_staging, ids_capacity, host_cache_bytes)
        self._quantize, self._dequantize = fp8_kernels or (quantize_blocks, dequantize_blocks)
        self._lane: _KernelLane | None = None
        self._stages: list[torch.Tensor] = []
        self._turn = 0
        self._payloads: dict[int, Payload] = {}  # pinned payloads by id(), freed on close

    @property
    def kernel_stream(self):
        """The torch stream the FP8 kernels run on (None before the first FP8 use, and on the
        host flavour)."""
        return self._lane.stream if self._lane is not None else None

    @property
    def stages(self) -> list[torch.Tensor]:
        """The FP8 staging tensors, one per slot."""
        return self._stages

    # -- lifetime and memory --

    def close(self) -> None:
        self.engine.destroy()
        for payload in self._payloads.values():
            payload.memory = None
        self._payloads.clear()
        self._stages = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def pin_stats(self) -> dict[str, int]:
        if self.engine.closed:
            return {}
        counters = self.engine.stats()
        return {name: counters[name] for name in PIN_STATS}

    def _pinned_payload(self, count: int, record: int, fp8: bool) -> Payload:
        size = count * record
        pointer = self.engine.host_alloc(size)
        view = torch.frombuffer((ctypes.c_uint8 * size).from_address(pointer), dtype=torch.uint8)
        payload = Payload(view, count, record, fp8, pointer)
        self._payloads[id(payload)] = payload
        return payload

    def free(self, payload: Payload) -> None:
        if payload.pointer is None or self.engine.closed:
            return
        self._payloads.pop(id(payload), None)
        self.engine.host_free(payload.pointer)
        payload.memory, payload.pointer = None, None

    def _check(self, cache: PagedKVCache, blocks: list[int] = ()) -> None:
        if cache.device.type != self.device.type:
            raise ValueError(f"the pool is on {cache.device}; this backend moves {self.device} memory")
        # The kernels index the pool with these ids as given; a wild one would fault the GPU.
        if blocks and (min(blocks) < 0 or max(blocks) >= cache.allocator.num_blocks):
            raise ValueError(f"block ids {min(blocks)}..{max(blocks)} are outside a pool of {cache.allocator.num_blocks}")

    def prepare(self, cache: PagedKVCache, fp8: bool = False) -> None:
        self._check(cache)
        if fp8:
            self._fp8_ready(Fp8Layout.from_cache(cache))
        else:
            self.engine.prepare_staging()

    # -- transfers --

    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        self._check(cache, blocks)
        # The gather runs on streams of its own: waiting here for torch's current stream is
        # what makes it see KV writes still queued there (transfer.py:388-401). Only that
        # stream: a device-wide wait would also wait for copies in flight.
        if self.flavor == "hip":
            torch.cuda.current_stream(self.device).synchronize()
        if not blocks:
            return ReadyTicket(Payload(torch.empty(0, dtype=torch.uint8), 0, record_bytes(cache, fp8), fp8))
        if fp8:
            return self._fp8(cache, blocks, None)
        payload = self._pinned_payload(len(blocks), cache.block_bytes, False)
        handle = self.engine.out_gather(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
        return _EngineTicket(self.engine, handle, payload, [])

    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        self._check(cache, blocks)
        if not blocks:
            return ReadyTicket()
        if payload.fp8:
            return self._fp8(cache, blocks, payload)
        handle = self.engine.in_scatter(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
        return _EngineTicket(self.engine, handle, None, [])

    # -- the per-block baseline (transfer.py:435-473) --

    def start_out_per_block(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        """start_out without staging: one copy per block (or, for FP8, one per record after
        the whole quantize has run), the measured baseline of bench/transfer_gather.py."""
        self._check(cache, blocks)
        if self.flavor == "hip":
            torch.cuda.current_stream(self.device).synchronize()
        if not blocks:
            return ReadyTicket(Payload(torch.empty(0, dtype=torch.uint8), 0, record_bytes(cache, fp8), fp8))
        if not fp8:
            payload = self._pinned_payload(len(blocks), cache.block_bytes, False)
            handle = self.engine.out_per_block(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
            return _EngineTicket(self.engine, handle, payload, [])
        layout, stage, holds = self._whole_stage(cache, len(blocks))
        ids = self._lane.upload(blocks, holds)
        self._lane.run(lambda: self._quantize(cache.pool, ids, stage, layout), holds)
        self._settle_lane()
        payload = self._pinned_payload(len(blocks), layout.record_bytes, True)
        handle = self.engine.out_per_block(stage.data_ptr(), layout.record_bytes, list(range(len(blocks))), payload.pointer)
        return _EngineTicket(self.engine, handle, payload, holds)

    def start_in_per_block(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        """start_in without staging: one copy per block, or for FP8 one per record into a
        stage the size of the payload, then the whole dequantize."""
        self._check(cache, blocks)
        if not blocks:
            return ReadyTicket()
        if not payload.fp8:
            handle = self.engine.in_per_block(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
            return _EngineTicket(self.engine, handle, None, [])
        layout, stage, holds = self._whole_stage(cache, len(blocks))
        copies = self.engine.in_per_block(stage.data_ptr(), layout.record_bytes, list(range(len(blocks))), payload.pointer)
        self.engine.wait(copies)
        self.engine.release(copies)
        ids = self._lane.upload(blocks, holds)
        self._lane.run(lambda: self._dequantize(stage, ids, cache.pool, layout), holds)
        return _EngineTicket(self.engine, self.engine.ext_finish(self._lane.handle), None, holds)

    def _whole_stage(self, cache: PagedKVCache, count: int) -> tuple[Fp8Layout, torch.Tensor, list]:
        layout = Fp8Layout.from_cache(cache)
        self._fp8_ready(layout)
        stage = torch.empty(count * layout.record_bytes, dtype=torch.uint8, device=self.device)
        return layout, stage, [cache.pool, stage]

    def _settle_lane(self) -> None:
        """Wait on the host until the work queued on the kernel lane has run."""
        handle = self.engine.ext_finish(self._lane.handle)
        self.engine.wait(handle)
        self.engine.release(handle)

    # -- FP8 --

    def _fp8_ready(self, layout: Fp8Layout) -> None:
        if self.engine.staging_bytes < layout.record_bytes:
            raise ValueError(f"a {self.engine.staging_bytes}-byte staging slot cannot hold one {layout.record_bytes}-byte record")
        if not self._stages:
            self._stages = [torch.empty(self.engine.staging_bytes, dtype=torch.uint8, device=self.device)
                            for _ in range(self.engine.num_staging)]
        if self._lane is None:
            self._lane = _KernelLane(self.engine, self.device)

    def _segments(self, blocks: int, per_segment: int):
        for first in range(0, blocks, per_segment):
            slot, self._turn = self._turn, (self._turn + 1) % len(self._stages)
            yield _Segment(slot, first, min(per_segment, blocks - first))

    def _fp8(self, cache: PagedKVCache, blocks: list[int], restore_from: Payload | None) -> Ticket:
        """One FP8 transfer: out (restore_from None) quantizes segments into staging and copies
        them to a new payload; in copies segments of restore_from to staging and dequantizes
        them into `blocks`."""
        layout = Fp8Layout.from_cache(cache)
        self._fp8_ready(layout)
        record = layout.record_bytes
        out = restore_from is None
        payload = self._pinned_payload(len(blocks), record, True) if out else restore_from
        lane, engine = self._lane, self.engine
        holds: list = [cache.pool]
        with lane.active():
            self._fp8_segments(cache, blocks, layout, payload, out, holds)
        # Out ends with the last copy (copy stream); in ends with the last kernel (our lane).
        handle = engine.ext_finish(None if out else lane.handle)
        return _EngineTicket(engine, handle, payload if out else None, holds)

    def _fp8_segments(self, cache: PagedKVCache, blocks: list[int], layout: Fp8Layout, payload: Payload, out: bool,
                      holds: list) -> None:
        lane, engine, record = self._lane, self.engine, layout.record_bytes
        ids = lane.upload(blocks, holds)
        for seg in self._segments(len(blocks), engine.staging_bytes // record):
            stage = self._stages[seg.slot]
            seg_ids = ids[seg.first : seg.first + seg.count]
            host = payload.pointer + seg.first * record
            nbytes = seg.count * record
            if out:
                engine.ext_wait(lane.handle, seg.slot, SLOT_RELEASED)
                lane.run(lambda stage=stage, seg_ids=seg_ids: self._quantize(cache.pool, seg_ids, stage, layout), holds)
                engine.ext_record(lane.handle, seg.slot, SLOT_FILLED)
                engine.ext_copy_out(stage.data_ptr(), host, nbytes, seg.slot)
            else:
                engine.ext_copy_in(stage.data_ptr(), host, nbytes, seg.slot)
                engine.ext_wait(lane.handle, seg.slot, SLOT_FILLED)
                lane.run(lambda stage=stage, seg_ids=seg_ids: self._dequantize(stage, seg_ids, cache.pool, layout), holds)
                engine.ext_record(lane.handle, seg.slot, SLOT_RELEASED)


def make_backend(name: str, device: torch.device | str = "cpu", **options) -> TransferBackend:
    backends = {"plain": lambda: PlainCopyBackend(), "native": lambda: NativeBackend(device, **options)}
    if name not in backends:
        raise ValueError(f"unknown transfer backend {name!r}")
    return backends[name]()
