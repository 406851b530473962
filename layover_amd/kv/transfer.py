"""Moving KV blocks between the pool and pinned CPU memory, behind tickets.

Mirrors the reference's layover/kv/transfer.py: Payload / Ticket (:45-82), PlainCopyBackend
(:120-144) and NativeBackend (:289-565) with the same start_out / start_in / free / prepare /
pin_stats / close interface, so CpuTier and the scheduler drive it unchanged.

NativeBackend on MI355X:
  - BF16 blocks: lt_out_gather / lt_in_scatter of the HIP flavour (gather kernel into a
    staging slot, SDMA copy to pinned memory on the engine's copy stream, two slots so the
    next gather overlaps the previous copy).
  - FP8 records: the fused gather+quantize kernel (lk_fp8_quantize) writes a record segment
    into a staging tensor on this backend's own stream, and the engine's lt_ext_* events
    order it against the copy stream's DMA of that segment (layover_transfer.h:84-96). Swap-in
    mirrors it with lk_fp8_dequantize into freshly assigned block ids. The block ids of a
    transfer are uploaded once, from pinned memory, on the same stream as the kernels.
The host flavour runs the same orchestration on host threads for tests; its FP8 kernels
must be supplied by the caller (`fp8_kernels`), since this package has no CPU quantizer.
"""

from __future__ import annotations

import ctypes
from abc import ABC, abstractmethod
from collections.abc import Callable

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

PIN_STATS = ("host_pins", "host_pin_bytes", "host_pin_ns", "host_pin_max_ns", "host_pin_failures")


class Payload:
    """Offloaded blocks in CPU memory, an array of equal records; valid once its ticket is done."""

    def __init__(self, memory: torch.Tensor, num_blocks: int, record_bytes: int, fp8: bool, pointer: int | None = None):
        self.memory: torch.Tensor | None = memory
        self.num_blocks = num_blocks
        self.record_bytes = record_bytes
        self.fp8 = fp8
        self.pointer = pointer

    @property
    def nbytes(self) -> int:
        return self.num_blocks * self.record_bytes


class Ticket(ABC):
    """A copy in progress. done() never blocks; wait() does."""

    payload: Payload | None = None
    ready_at: float | None = None

    @abstractmethod
    def done(self) -> bool: ...

    @abstractmethod
    def wait(self) -> None: ...


class ReadyTicket(Ticket):
    def __init__(self, payload: Payload | None = None):
        self.payload = payload

    def done(self) -> bool:
        return True

    def wait(self) -> None:
        pass


class TransferBackend(ABC):
    name = ""

    @abstractmethod
    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        """Begin copying blocks to CPU memory; the caller keeps them unwritten until done."""

    @abstractmethod
    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        """Begin copying the first len(blocks) records into `blocks`."""

    def free(self, payload: Payload) -> None:
        """Give back a payload's memory. Its offload and restores must be done."""

    def prepare(self, cache: PagedKVCache, fp8: bool = False) -> None:
        """Do first-use work now (staging allocation)."""

    def pin_stats(self) -> dict[str, int]:
        return {}

    def close(self) -> None:
        pass


def record_bytes(cache: PagedKVCache, fp8: bool) -> int:
    return Fp8Layout.from_cache(cache).record_bytes if fp8 else cache.block_bytes


class PlainCopyBackend(TransferBackend):
    """One tensor per offload through torch, finished before it returns (transfer.py:120-144)."""

    name = "plain"

    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        ids = torch.tensor(blocks, device=cache.device, dtype=torch.long)
        if fp8:
            layout = Fp8Layout.from_cache(cache)
            stage = torch.empty(len(blocks) * layout.record_bytes, dtype=torch.uint8, device=cache.device)
            quantize_blocks(cache.pool, ids.int(), stage, layout)
            memory = stage.to("cpu")
        else:
            memory = cache.pool[ids].to("cpu", copy=True).reshape(-1).view(torch.uint8)
        return ReadyTicket(Payload(memory, len(blocks), record_bytes(cache, fp8), fp8))

    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        ids = torch.tensor(blocks, device=cache.device, dtype=torch.long)
        used = payload.memory[: len(blocks) * payload.record_bytes]
        if payload.fp8:
            dequantize_blocks(used.to(cache.device), ids.int(), cache.pool, Fp8Layout.from_cache(cache))
        else:
            shape = (len(blocks), *cache.pool.shape[1:])
            cache.pool[ids] = used.view(cache.pool.dtype).reshape(shape).to(cache.device)
        return ReadyTicket()


class _NativeTicket(Ticket):
    def __init__(self, backend: "NativeBackend", transfer: int, payload: Payload | None, keepalive: list):
        self.payload = payload
        self._backend = backend
        self._transfer = transfer
        self._keepalive = keepalive

    def _settle(self) -> None:
        self._backend.engine.release(self._transfer)
        self._transfer = None
        self._keepalive = None

    def done(self) -> bool:
        if self._transfer is None or self._backend.engine.closed:
            return True
        if not self._backend.engine.poll(self._transfer):
            return False
        self._settle()
        return True

    def wait(self) -> None:
        if self._transfer is None or self._backend.engine.closed:
            return
        self._backend.engine.wait(self._transfer)
        self._settle()


Fp8Kernel = Callable[[torch.Tensor, torch.Tensor, torch.Tensor, Fp8Layout], None]


class NativeBackend(TransferBackend):
    """Gather into staging, one DMA per segment on a dedicated copy stream, events in between."""

    name = "native"

    def __init__(
        self,
        device: torch.device | str = "cpu",
        staging_bytes: int = 128 << 20,
        num_staging: int = 2,
        ids_capacity: int = 1 << 20,
        host_cache_bytes: int = 8 << 30,
        fp8_impl: str | None = None,
        fp8_kernels: tuple[Fp8Kernel, Fp8Kernel] | None = None,
    ):
        self.device = torch.device(device)
        if self.device.type not in ("cpu", "cuda"):
            raise ValueError(f"no native transfer path for device {device}")
        # torch-ROCm names its GPUs "cuda"; this library's flavour for them is "hip".
        self.flavor = "hip" if self.device.type == "cuda" else "host"
        if self.flavor == "host":
            build_host()
        index = (self.device.index or 0) if self.flavor == "hip" else 0
        self.engine = Engine(self.flavor, index, staging_bytes, num_staging, ids_capacity, host_cache_bytes)
        if fp8_impl not in (None, "hip"):
            raise ValueError(f"this build has only the 'hip' FP8 implementation, not {fp8_impl!r}")
        if fp8_kernels is None:
            fp8_kernels = (quantize_blocks, lambda stage, ids, pool, layout: dequantize_blocks(stage, ids, pool, layout))
        self._quantize, self._dequantize = fp8_kernels
        self._next_stage = 0
        self._stages: list[torch.Tensor] = []
        self._stream = None
        self._live: list[Payload] = []

    def close(self) -> None:
        self.engine.destroy()
        for payload in self._live:
            payload.memory = None
        self._live = []
        self._stages = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def pin_stats(self) -> dict[str, int]:
        if self.engine.closed:
            return {}
        stats = self.engine.stats()
        return {name: stats[name] for name in PIN_STATS}

    # Memory

    def _host_payload(self, count: int, record: int, fp8: bool) -> Payload:
        nbytes = count * record
        pointer = self.engine.host_alloc(nbytes)
        buffer = (ctypes.c_uint8 * nbytes).from_address(pointer)
        payload = Payload(torch.frombuffer(buffer, dtype=torch.uint8), count, record, fp8, pointer)
        self._live.append(payload)
        return payload

    def free(self, payload: Payload) -> None:
        if payload.pointer is None or self.engine.closed:
            return
        self._live.remove(payload)
        self.engine.host_free(payload.pointer)
        payload.memory = None
        payload.pointer = None

    def _check_cache(self, cache: PagedKVCache, blocks: list[int] | None = None) -> None:
        if cache.device.type != self.device.type:
            raise ValueError(f"pool is on {cache.device}, this backend drives {self.device}")
        # Kernels index the pool with these unchecked; a wild id would fault the GPU.
        if blocks and not (0 <= min(blocks) and max(blocks) < cache.allocator.num_blocks):
            raise ValueError(f"block ids {min(blocks)}..{max(blocks)} are outside a pool of {cache.allocator.num_blocks}")

    def prepare(self, cache: PagedKVCache, fp8: bool = False) -> None:
        self._check_cache(cache)
        if fp8:
            self._ensure_stages(Fp8Layout.from_cache(cache))
        else:
            self.engine.prepare_staging()

    def _sync_torch(self) -> None:
        # Offload kernels run on other streams; this makes them see KV writes queued on torch's
        # current stream (transfer.py:388-401). Only the current stream: a device-wide sync
        # would also wait for copies in flight and destroy the overlap.
        if self.flavor == "hip":
            torch.cuda.current_stream(self.device).synchronize()

    # BF16

    def start_out(self, cache: PagedKVCache, blocks: list[int], fp8: bool = False) -> Ticket:
        self._check_cache(cache, blocks)
        self._sync_torch()
        if not blocks:
            return ReadyTicket(Payload(torch.empty(0, dtype=torch.uint8), 0, record_bytes(cache, fp8), fp8))
        if fp8:
            return self._fp8_out(cache, blocks)
        payload = self._host_payload(len(blocks), cache.block_bytes, False)
        transfer = self.engine.out_gather(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
        return _NativeTicket(self, transfer, payload, [])

    def start_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        self._check_cache(cache, blocks)
        if not blocks:
            return ReadyTicket()
        if payload.fp8:
            return self._fp8_in(cache, blocks, payload)
        transfer = self.engine.in_scatter(cache.pool.data_ptr(), cache.block_bytes, blocks, payload.pointer)
        return _NativeTicket(self, transfer, None, [])

    # FP8

    def _ensure_stages(self, layout: Fp8Layout) -> None:
        if self.engine.staging_bytes < layout.record_bytes:
            raise ValueError(f"staging of {self.engine.staging_bytes} bytes cannot hold one {layout.record_bytes} byte record")
        if not self._stages:
            self._stages = [torch.empty(self.engine.staging_bytes, dtype=torch.uint8, device=self.device) for _ in range(self.engine.num_staging)]
        if self.flavor == "hip" and self._stream is None:
            self._stream = torch.cuda.Stream(device=self.device)

    def _stream_handle(self) -> int:
        return self._stream.cuda_stream if self.flavor == "hip" else self.engine.host_stream()

    def _launch(self, fn: Callable[[], None], keepalive: list) -> None:
        if self.flavor == "hip":
            with torch.cuda.stream(self._stream):
                fn()
        else:
            keepalive.append(self.engine.host_call(self.engine.host_stream(), fn))

    def _device_ids(self, blocks: list[int], keepalive: list) -> torch.Tensor:
        """All of a transfer's block ids on the device, uploaded once from pinned memory in
        stream order (an upload from pageable memory would synchronize)."""
        ids = torch.tensor(blocks, dtype=torch.int32)
        if self.flavor != "hip":
            return ids
        pinned = ids.pin_memory()
        uploaded = torch.empty_like(ids, device=self.device)
        with torch.cuda.stream(self._stream):
            uploaded.copy_(pinned, non_blocking=True)
        keepalive.extend((pinned, uploaded))
        return uploaded

    def _take_stage(self) -> int:
        stage = self._next_stage
        self._next_stage = (stage + 1) % len(self._stages)
        return stage

    def _fp8_out(self, cache: PagedKVCache, blocks: list[int]) -> Ticket:
        layout = Fp8Layout.from_cache(cache)
        self._ensure_stages(layout)
        payload = self._host_payload(len(blocks), layout.record_bytes, True)
        per_segment = self.engine.staging_bytes // layout.record_bytes
        stream = self._stream_handle()
        keepalive: list = [cache.pool]
        ids = self._device_ids(blocks, keepalive)
        for start in range(0, len(blocks), per_segment):
            count = min(per_segment, len(blocks) - start)
            slot = self._take_stage()
            stage = self._stages[slot]
            self.engine.ext_wait(stream, slot, SLOT_RELEASED)
            self._launch(lambda stage=stage, start=start, count=count: self._quantize(cache.pool, ids[start : start + count], stage, layout), keepalive)
            self.engine.ext_record(stream, slot, SLOT_FILLED)
            self.engine.ext_copy_out(stage.data_ptr(), payload.pointer + start * layout.record_bytes, count * layout.record_bytes, slot)
        return _NativeTicket(self, self.engine.ext_finish(None), payload, keepalive)

    def _fp8_in(self, cache: PagedKVCache, blocks: list[int], payload: Payload) -> Ticket:
        layout = Fp8Layout.from_cache(cache)
        self._ensure_stages(layout)
        per_segment = self.engine.staging_bytes // layout.record_bytes
        stream = self._stream_handle()
        keepalive: list = [cache.pool]
        ids = self._device_ids(blocks, keepalive)
        for start in range(0, len(blocks), per_segment):
            count = min(per_segment, len(blocks) - start)
            slot = self._take_stage()
            stage = self._stages[slot]
            self.engine.ext_copy_in(stage.data_ptr(), payload.pointer + start * layout.record_bytes, count * layout.record_bytes, slot)
            self.engine.ext_wait(stream, slot, SLOT_FILLED)
            self._launch(lambda stage=stage, start=start, count=count: self._dequantize(stage, ids[start : start + count], cache.pool, layout), keepalive)
            self.engine.ext_record(stream, slot, SLOT_RELEASED)
        return _NativeTicket(self, self.engine.ext_finish(stream), None, keepalive)


def make_backend(name: str, device: torch.device | str = "cpu", **options) -> TransferBackend:
    if name == "plain":
        return PlainCopyBackend()
    if name == "native":
        return NativeBackend(device, **options)
    raise ValueError(f"unknown transfer backend {name!r}")
