"""ctypes front end of the swap library, include/layover_transfer.h.

Plays the part of the reference's layover/kv/native.py for this package: it finds the built
library of a flavour, refuses one whose ABI version or flavour is not what was asked for,
declares every entry point's argument types, and turns a non-zero status into an exception
carrying lt_last_error(): LT_ERR_NOMEM becomes HostMemoryError (survivable), anything else
NativeError. Flavours: "host" (host threads) and "hip" (MI355X); torch-ROCm calls its GPUs
"cuda", and the flavour for them is "hip".

Where a library is looked for: LAYOVER_NATIVE_LIB if set, else
layover_amd/csrc/build/<flavour>-<OS>-<arch>/liblayover_transfer.so, the layout the
reference's native/Makefile uses. `path=` points a load at another build (the tests load
the reference's own host library that way to compare behaviour).
"""

from __future__ import annotations

import ctypes
import os
import platform
import subprocess
from pathlib import Path

from layover_amd import CSRC_DIR

ABI_VERSION = 2
LIBRARY_NAME = "liblayover_transfer.so"
SLOT_FILLED, SLOT_RELEASED = 0, 1
LT_OK, LT_ERR_INVALID, LT_ERR_DEVICE, LT_ERR_UNSUPPORTED, LT_ERR_NOMEM = range(5)


class NativeError(RuntimeError):
    """The swap library refused a call or failed; the message is the library's own."""

    def __init__(self, message: str, status: int = LT_ERR_DEVICE):
        super().__init__(message)
        self.status = status


class HostMemoryError(NativeError):
    """Pinned host memory ran out. Nothing was enqueued and the engine stays usable."""


class NativeUnavailable(RuntimeError):
    """No usable build of the swap library for this machine and flavour."""


# lt_stats, in the header's field order.
STAT_FIELDS = (
    "kernels", "memcpys", "ids_uploads", "stream_waits", "bytes_to_host", "bytes_to_device", "transfers",
    "host_bytes_live", "host_bytes_held", "host_pins", "host_pin_bytes", "host_pin_ns", "host_pin_max_ns", "host_pin_failures",
)


class Stats(ctypes.Structure):
    _fields_ = [(field, ctypes.c_uint64) for field in STAT_FIELDS]

    def as_dict(self) -> dict[str, int]:
        return {field: int(getattr(self, field)) for field in STAT_FIELDS}


HOST_KERNEL = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)

# Every status-returning entry point, one line each: name, then its parameters in the
# header's order. p = pointer, i = int, u32 / u64 = unsigned, ids = const uint32_t*,
# out = pointer to a pointer, stats = lt_stats*, done = int*, kernel = lt_host_kernel.
_PROTOTYPES = """
lt_create                 i u64 u32 u32 u64 out
lt_destroy                p
lt_prepare_staging        p
lt_get_stats              p stats
lt_host_alloc             p u64 out
lt_host_free              p p
lt_out_gather             p p u64 ids u32 p out
lt_in_scatter             p p u64 ids u32 p out
lt_out_per_block          p p u64 ids u32 p out
lt_in_per_block           p p u64 ids u32 p out
lt_ext_wait               p p u32 i
lt_ext_record             p p u32 i
lt_ext_copy_out           p p p u64 u32
lt_ext_copy_in            p p p u64 u32
lt_ext_finish             p p out
lt_poll                   p p done
lt_wait                   p p
lt_release                p p
lt_host_stream            p out
lt_host_call              p p kernel p
lt_host_set_paused        p i
lt_host_set_copy_delay_us p u32
lt_host_set_pin_limit     p u64
"""

_CTYPE = {
    "p": ctypes.c_void_p,
    "i": ctypes.c_int,
    "u32": ctypes.c_uint32,
    "u64": ctypes.c_uint64,
    "ids": ctypes.POINTER(ctypes.c_uint32),
    "out": ctypes.POINTER(ctypes.c_void_p),
    "stats": ctypes.POINTER(Stats),
    "done": ctypes.POINTER(ctypes.c_int),
    "kernel": HOST_KERNEL,
}

SIGNATURES: dict[str, tuple] = {
    fields[0]: tuple(_CTYPE[code] for code in fields[1:]) for fields in (line.split() for line in _PROTOTYPES.strip().splitlines())
}

_libraries: dict[tuple[str, str], ctypes.CDLL] = {}


def build_dir(flavor: str) -> Path:
    return CSRC_DIR / "build" / f"{flavor}-{platform.system()}-{platform.machine()}"


def library_path(flavor: str) -> Path:
    chosen = os.environ.get("LAYOVER_NATIVE_LIB")
    return Path(chosen) if chosen else build_dir(flavor) / LIBRARY_NAME


def build_host() -> Path:
    """Make the host flavour if its sources changed (tests call this; it needs only g++)."""
    subprocess.run(["make", "-s", "-C", str(CSRC_DIR), "host"], check=True, capture_output=True, text=True)
    return library_path("host")


def hip_runtimes_loaded(name: str = "libamdhip64") -> list[str]:
    """Distinct mapped files whose path contains `name`. One HIP runtime per process is the
    only safe number: pointers, streams and events of one are meaningless to another."""
    found: list[str] = []
    with open("/proc/self/maps") as maps:
        for line in maps:
            fields = line.split()
            if len(fields) >= 6 and name in fields[-1] and fields[-1] not in found:
                found.append(fields[-1])
    return found


def load_library(flavor: str, path: Path | str | None = None) -> ctypes.CDLL:
    """The library of `flavour`, loaded once per path, with every entry point declared."""
    where = Path(path) if path is not None else library_path(flavor)
    key = (flavor, str(where))
    if key in _libraries:
        return _libraries[key]
    if not where.exists():
        raise NativeUnavailable(f"{where} does not exist: build it with 'make -C {CSRC_DIR} {flavor}'")
    if flavor == "hip":
        # torch brings its own libamdhip64.so.7; it must be mapped before this library binds
        # that soname, so both share one runtime.
        import torch  # noqa: F401
    try:
        library = ctypes.CDLL(str(where))
    except OSError as error:
        raise NativeUnavailable(f"{where} cannot be loaded: {error}") from error
    if flavor == "hip" and len(hip_runtimes_loaded()) != 1:
        raise NativeUnavailable(f"expected one HIP runtime in the process, found {hip_runtimes_loaded()}")
    library.lt_abi_version.restype = ctypes.c_int
    library.lt_flavor.restype = ctypes.c_char_p
    library.lt_last_error.restype = ctypes.c_char_p
    version, built = library.lt_abi_version(), library.lt_flavor().decode()
    if version != ABI_VERSION:
        raise NativeUnavailable(f"{where} speaks ABI {version}, this binding ABI {ABI_VERSION}: rebuild it")
    if built != flavor:
        raise NativeUnavailable(f"{where} is a {built} build, not {flavor}")
    for name, params in SIGNATURES.items():
        entry = getattr(library, name)
        entry.argtypes = list(params)
        entry.restype = ctypes.c_int
    _libraries[key] = library
    return library


def _id_array(ids) -> ctypes.Array:
    return (ctypes.c_uint32 * len(ids))(*ids)


class Engine:
    """One lt_engine. Driven by one thread only, like the library itself."""

    def __init__(self, flavor: str = "host", device: int = 0, staging_bytes: int = 128 << 20, num_staging: int = 2,
                 ids_capacity: int = 1 << 20, host_cache_bytes: int = 8 << 30, library: Path | str | None = None):
        self.flavor = flavor
        self.staging_bytes = staging_bytes
        self.num_staging = num_staging
        self.ids_capacity = ids_capacity
        self._lib = load_library(flavor, library)
        self._handle: ctypes.c_void_p | None = None
        # The exception a host kernel raised, kept to explain the device error it causes.
        self._kernel_error: BaseException | None = None
        created = ctypes.c_void_p()
        self._call("lt_create", device, staging_bytes, num_staging, ids_capacity, host_cache_bytes, ctypes.byref(created), engine=False)
        self._handle = created

    # -- plumbing --

    def _call(self, name: str, *args, engine: bool = True) -> None:
        if engine:
            if self._handle is None:
                raise NativeError("the swap engine is closed", LT_ERR_INVALID)
            args = (self._handle, *args)
        status = getattr(self._lib, name)(*args)
        if status == LT_OK:
            return
        message = self._lib.lt_last_error().decode()
        if status == LT_ERR_NOMEM:
            raise HostMemoryError(message, status)
        if self._kernel_error is not None:
            raise NativeError(f"{message}: {self._kernel_error!r}", status) from self._kernel_error
        raise NativeError(message, status)

    def _returning_pointer(self, name: str, *args) -> int | None:
        result = ctypes.c_void_p()
        self._call(name, *args, ctypes.byref(result))
        return result.value

    @property
    def closed(self) -> bool:
        return self._handle is None

    def destroy(self) -> None:
        """Waits for everything in flight, then frees it all. A second call does nothing."""
        if self._handle is None:
            return
        handle, self._handle = self._handle, None
        self._call("lt_destroy", handle, engine=False)

    # -- memory and counters --

    def prepare_staging(self) -> None:
        self._call("lt_prepare_staging")

    def stats(self) -> dict[str, int]:
        snapshot = Stats()
        self._call("lt_get_stats", ctypes.byref(snapshot))
        return snapshot.as_dict()

    def host_alloc(self, nbytes: int) -> int:
        return self._returning_pointer("lt_host_alloc", nbytes)

    def host_free(self, pointer: int) -> None:
        self._call("lt_host_free", pointer)

    # -- transfers; each returns the lt_transfer handle as an int --

    def out_gather(self, pool: int, block_bytes: int, ids, host: int) -> int:
        return self._returning_pointer("lt_out_gather", pool, block_bytes, _id_array(ids), len(ids), host)

    def in_scatter(self, pool: int, block_bytes: int, ids, host: int) -> int:
        return self._returning_pointer("lt_in_scatter", pool, block_bytes, _id_array(ids), len(ids), host)

    def out_per_block(self, pool: int, block_bytes: int, ids, host: int) -> int:
        return self._returning_pointer("lt_out_per_block", pool, block_bytes, _id_array(ids), len(ids), host)

    def in_per_block(self, pool: int, block_bytes: int, ids, host: int) -> int:
        return self._returning_pointer("lt_in_per_block", pool, block_bytes, _id_array(ids), len(ids), host)

    def ext_wait(self, stream: int | None, slot: int, which: int) -> None:
        self._call("lt_ext_wait", stream, slot, which)

    def ext_record(self, stream: int | None, slot: int, which: int) -> None:
        self._call("lt_ext_record", stream, slot, which)

    def ext_copy_out(self, staging: int, host: int, nbytes: int, slot: int) -> None:
        self._call("lt_ext_copy_out", staging, host, nbytes, slot)

    def ext_copy_in(self, staging: int, host: int, nbytes: int, slot: int) -> None:
        self._call("lt_ext_copy_in", staging, host, nbytes, slot)

    def ext_finish(self, stream: int | None) -> int:
        return self._returning_pointer("lt_ext_finish", stream)

    def poll(self, transfer: int) -> bool:
        done = ctypes.c_int()
        self._call("lt_poll", transfer, ctypes.byref(done))
        return done.value != 0

    def wait(self, transfer: int) -> None:
        self._call("lt_wait", transfer)

    def release(self, transfer: int) -> None:
        self._call("lt_release", transfer)

    # -- host flavour only --

    def host_stream(self) -> int:
        return self._returning_pointer("lt_host_stream")

    def host_call(self, stream: int, fn) -> HOST_KERNEL:
        """Queue fn() on a host stream. The returned callback must stay referenced until it
        has run; an exception in fn becomes a device failure of the engine."""

        def kernel(_context) -> int:
            try:
                fn()
            except BaseException as error:  # nothing may unwind into the C++ worker thread
                self._kernel_error = error
                return 1
            return 0

        callback = HOST_KERNEL(kernel)
        self._call("lt_host_call", stream, callback, None)
        return callback

    def set_paused(self, paused: bool) -> None:
        self._call("lt_host_set_paused", 1 if paused else 0)

    def set_copy_delay_us(self, delay_us: int) -> None:
        self._call("lt_host_set_copy_delay_us", delay_us)

    def set_pin_limit(self, nbytes: int) -> None:
        self._call("lt_host_set_pin_limit", nbytes)
