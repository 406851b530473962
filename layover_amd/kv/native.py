"""ctypes binding of the transfer library (include/layover_transfer.h).

Mirrors the reference's layover/kv/native.py:1-265: the same signatures, the same library
path scheme (csrc/build/<flavor>-<OS>-<arch>/liblayover_transfer.so, or LAYOVER_NATIVE_LIB),
the same ABI and flavour checks, and the same error mapping (NOMEM -> HostMemoryError,
anything else -> NativeError). Flavours are "host" and "hip"; torch-ROCm reports its GPUs as
device type "cuda", and the flavour for those is "hip".
"""

from __future__ import annotations

import ctypes
import os
import platform
import subprocess
from ctypes import POINTER, byref, c_char_p, c_int, c_uint32, c_uint64, c_void_p
from pathlib import Path

from layover_amd import CSRC_DIR

ABI_VERSION = 2
LIBRARY_NAME = "liblayover_transfer.so"
SLOT_FILLED, SLOT_RELEASED = 0, 1
_ERR_NOMEM = 4


class NativeError(RuntimeError):
    """The transfer library reported a failure, with its message."""


class HostMemoryError(NativeError):
    """Host memory could not be pinned. Nothing was enqueued and the engine stays usable."""


class NativeUnavailable(RuntimeError):
    """The transfer library has not been built for this machine."""


class Stats(ctypes.Structure):
    _fields_ = [
        (name, c_uint64)
        for name in (
            "kernels", "memcpys", "ids_uploads", "stream_waits", "bytes_to_host", "bytes_to_device", "transfers",
            "host_bytes_live", "host_bytes_held", "host_pins", "host_pin_bytes", "host_pin_ns", "host_pin_max_ns",
            "host_pin_failures",
        )
    ]

    def as_dict(self) -> dict[str, int]:
        return {name: getattr(self, name) for name, _ in self._fields_}


HOST_KERNEL = ctypes.CFUNCTYPE(c_int, c_void_p)
_BLOCKS = (c_void_p, c_void_p, c_uint64, POINTER(c_uint32), c_uint32, c_void_p, POINTER(c_void_p))
SIGNATURES = {
    "lt_create": (c_int, c_uint64, c_uint32, c_uint32, c_uint64, POINTER(c_void_p)),
    "lt_destroy": (c_void_p,),
    "lt_prepare_staging": (c_void_p,),
    "lt_get_stats": (c_void_p, POINTER(Stats)),
    "lt_host_alloc": (c_void_p, c_uint64, POINTER(c_void_p)),
    "lt_host_free": (c_void_p, c_void_p),
    "lt_out_gather": _BLOCKS,
    "lt_in_scatter": _BLOCKS,
    "lt_out_per_block": _BLOCKS,
    "lt_in_per_block": _BLOCKS,
    "lt_ext_wait": (c_void_p, c_void_p, c_uint32, c_int),
    "lt_ext_record": (c_void_p, c_void_p, c_uint32, c_int),
    "lt_ext_copy_out": (c_void_p, c_void_p, c_void_p, c_uint64, c_uint32),
    "lt_ext_copy_in": (c_void_p, c_void_p, c_void_p, c_uint64, c_uint32),
    "lt_ext_finish": (c_void_p, c_void_p, POINTER(c_void_p)),
    "lt_poll": (c_void_p, c_void_p, POINTER(c_int)),
    "lt_wait": (c_void_p, c_void_p),
    "lt_release": (c_void_p, c_void_p),
    "lt_host_stream": (c_void_p, POINTER(c_void_p)),
    "lt_host_call": (c_void_p, c_void_p, HOST_KERNEL, c_void_p),
    "lt_host_set_paused": (c_void_p, c_int),
    "lt_host_set_copy_delay_us": (c_void_p, c_uint32),
    "lt_host_set_pin_limit": (c_void_p, c_uint64),
}

_loaded: dict[str, ctypes.CDLL] = {}


def build_dir(flavor: str) -> Path:
    return CSRC_DIR / "build" / f"{flavor}-{platform.system()}-{platform.machine()}"


def library_path(flavor: str) -> Path:
    override = os.environ.get("LAYOVER_NATIVE_LIB")
    if override:
        return Path(override)
    return build_dir(flavor) / LIBRARY_NAME


def build_host() -> Path:
    """Build the host flavour if needed, for tests; make decides whether anything changed."""
    subprocess.run(["make", "-s", "-C", str(CSRC_DIR), "host"], check=True, capture_output=True, text=True)
    return library_path("host")


def hip_runtimes_loaded(name: str = "libamdhip64") -> list[str]:
    """Paths of every libamdhip64 (or other runtime `name`) mapped into this process; exactly
    one is safe."""
    seen = []
    with open("/proc/self/maps") as maps:
        for line in maps:
            path = line.split()[-1] if "/" in line else ""
            if name in path and path not in seen:
                seen.append(path)
    return seen


def load_library(flavor: str, path: Path | str | None = None) -> ctypes.CDLL:
    """Load a flavour, refusing a stale or mismatched build instead of misreading its ABI.

    `path` overrides where the library is read from (tests load the reference's own host
    build through it to compare behaviour)."""
    path = Path(path) if path is not None else library_path(flavor)
    key = f"{flavor}:{path}"
    if key in _loaded:
        return _loaded[key]
    if not path.exists():
        raise NativeUnavailable(f"{path} does not exist: run 'make -C {CSRC_DIR} {flavor}'")
    if flavor == "hip":
        # torch's HIP runtime must be the one in the process before this library binds to
        # libamdhip64.so.7, or pool pointers and streams would belong to another runtime.
        import torch  # noqa: F401
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as error:
        raise NativeUnavailable(f"{path} cannot be loaded: {error}") from error
    if flavor == "hip" and len(hip_runtimes_loaded()) > 1:
        raise NativeUnavailable(f"two HIP runtimes are loaded: {hip_runtimes_loaded()}")
    if flavor == "hip" and len(hip_runtimes_loaded("libhsa-runtime64")) > 1:
        # A profiler maps a second HSA runtime beside the one HIP runs on; SDMA copies issued
        # through it would not know HIP's allocations, so copies to the host stay with HIP.
        os.environ.pop("LAYOVER_D2H", None)
    lib.lt_abi_version.restype = c_int
    lib.lt_flavor.restype = c_char_p
    lib.lt_last_error.restype = c_char_p
    if hasattr(lib, "lt_sdma_copies"):  # this build's extension; the reference's library lacks it
        lib.lt_sdma_copies.restype = ctypes.c_uint64
        lib.lt_sdma_copies.argtypes = []
    if lib.lt_abi_version() != ABI_VERSION:
        raise NativeUnavailable(f"{path} has ABI {lib.lt_abi_version()}, expected {ABI_VERSION}: rebuild it")
    built = lib.lt_flavor().decode()
    if built != flavor:
        raise NativeUnavailable(f"{path} is the {built} flavor, expected {flavor}")
    for name, argtypes in SIGNATURES.items():
        function = getattr(lib, name)
        function.argtypes = list(argtypes)
        function.restype = c_int
    _loaded[key] = lib
    return lib


class Engine:
    """One lt_engine. Only the thread driving transfers may call it (native.py:129-265)."""

    def __init__(
        self,
        flavor: str = "host",
        device: int = 0,
        staging_bytes: int = 128 << 20,
        num_staging: int = 2,
        ids_capacity: int = 1 << 20,
        host_cache_bytes: int = 8 << 30,
        library: Path | str | None = None,
    ):
        self.flavor = flavor
        self.staging_bytes = staging_bytes
        self.num_staging = num_staging
        self._handle = None
        self._kernel_failure: BaseException | None = None
        self._lib = load_library(flavor, library)
        handle = c_void_p()
        self._check(self._lib.lt_create(device, staging_bytes, num_staging, ids_capacity, host_cache_bytes, byref(handle)))
        self._handle = handle

    def _check(self, status: int) -> None:
        if status != 0:
            message = self._lib.lt_last_error().decode()
            if status == _ERR_NOMEM:
                raise HostMemoryError(message)
            if self._kernel_failure is not None:
                raise NativeError(f"{message}: {self._kernel_failure!r}") from self._kernel_failure
            raise NativeError(message)

    def _open(self) -> c_void_p:
        if self._handle is None:
            raise NativeError("the transfer engine is closed")
        return self._handle

    @property
    def closed(self) -> bool:
        return self._handle is None

    def destroy(self) -> None:
        """Waits for transfers in flight and frees everything. Safe to repeat."""
        if self._handle is None:
            return
        handle, self._handle = self._handle, None
        self._check(self._lib.lt_destroy(handle))

    def prepare_staging(self) -> None:
        self._check(self._lib.lt_prepare_staging(self._open()))

    def stats(self) -> dict[str, int]:
        out = Stats()
        self._check(self._lib.lt_get_stats(self._open(), byref(out)))
        return out.as_dict()

    def host_alloc(self, nbytes: int) -> int:
        pointer = c_void_p()
        self._check(self._lib.lt_host_alloc(self._open(), nbytes, byref(pointer)))
        return pointer.value

    def host_free(self, pointer: int) -> None:
        self._check(self._lib.lt_host_free(self._open(), c_void_p(pointer)))

    def _blocks(self, function, pool: int | None, block_bytes: int, ids: list[int], host: int | None) -> int:
        array = (c_uint32 * len(ids))(*ids)
        transfer = c_void_p()
        self._check(function(self._open(), c_void_p(pool), block_bytes, array, len(ids), c_void_p(host), byref(transfer)))
        return transfer.value

    def out_gather(self, pool: int, block_bytes: int, ids: list[int], host: int) -> int:
        return self._blocks(self._lib.lt_out_gather, pool, block_bytes, ids, host)

    def in_scatter(self, pool: int, block_bytes: int, ids: list[int], host: int) -> int:
        return self._blocks(self._lib.lt_in_scatter, pool, block_bytes, ids, host)

    def out_per_block(self, pool: int, block_bytes: int, ids: list[int], host: int) -> int:
        return self._blocks(self._lib.lt_out_per_block, pool, block_bytes, ids, host)

    def in_per_block(self, pool: int, block_bytes: int, ids: list[int], host: int) -> int:
        return self._blocks(self._lib.lt_in_per_block, pool, block_bytes, ids, host)

    def ext_wait(self, stream: int | None, slot: int, which: int) -> None:
        self._check(self._lib.lt_ext_wait(self._open(), c_void_p(stream), slot, which))

    def ext_record(self, stream: int | None, slot: int, which: int) -> None:
        self._check(self._lib.lt_ext_record(self._open(), c_void_p(stream), slot, which))

    def ext_copy_out(self, staging: int, host: int, nbytes: int, slot: int) -> None:
        self._check(self._lib.lt_ext_copy_out(self._open(), c_void_p(staging), c_void_p(host), nbytes, slot))

    def ext_copy_in(self, staging: int, host: int, nbytes: int, slot: int) -> None:
        self._check(self._lib.lt_ext_copy_in(self._open(), c_void_p(staging), c_void_p(host), nbytes, slot))

    def ext_finish(self, stream: int | None) -> int:
        transfer = c_void_p()
        self._check(self._lib.lt_ext_finish(self._open(), c_void_p(stream), byref(transfer)))
        return transfer.value

    def poll(self, transfer: int) -> bool:
        done = c_int()
        self._check(self._lib.lt_poll(self._open(), c_void_p(transfer), byref(done)))
        return bool(done.value)

    def wait(self, transfer: int) -> None:
        self._check(self._lib.lt_wait(self._open(), c_void_p(transfer)))

    def release(self, transfer: int) -> None:
        self._check(self._lib.lt_release(self._open(), c_void_p(transfer)))

    def host_stream(self) -> int:
        stream = c_void_p()
        self._check(self._lib.lt_host_stream(self._open(), byref(stream)))
        return stream.value

    def host_call(self, stream: int, fn) -> HOST_KERNEL:
        """Run fn on a host stream. Keep the returned callback alive until it has run."""

        def trampoline(_context):
            try:
                fn()
                return 0
            except BaseException as failure:  # an exception must not cross into C++
                self._kernel_failure = failure
                return 1

        callback = HOST_KERNEL(trampoline)
        self._check(self._lib.lt_host_call(self._open(), c_void_p(stream), callback, None))
        return callback

    def set_paused(self, paused: bool) -> None:
        self._check(self._lib.lt_host_set_paused(self._open(), int(paused)))

    def set_copy_delay_us(self, delay_us: int) -> None:
        self._check(self._lib.lt_host_set_copy_delay_us(self._open(), delay_us))

    def set_pin_limit(self, nbytes: int) -> None:
        self._check(self._lib.lt_host_set_pin_limit(self._open(), nbytes))
