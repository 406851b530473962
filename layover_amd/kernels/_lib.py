"""Loader of liblayover_kernels.so (include/layover_kernels.h) through ctypes.

The library is built in-tree (layover_amd/csrc, `make hip`) and loaded after torch, so it
binds to torch's HIP runtime. There is no fallback: without the library every kernel call
raises KernelsUnavailable.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_uint32, c_uint64, c_void_p

from layover_amd.kv.native import NativeUnavailable, build_dir, hip_runtimes_loaded

ABI_VERSION = 3
LK_BF16, LK_F32, LK_FP8_RECORD = 0, 1, 2
LK_OK, LK_ERR_INVALID, LK_ERR_DEVICE = 0, 1, 2
LK_DECODE_SHARED_BLOCKS = 1
LIBRARY_NAME = "liblayover_kernels.so"


class KernelsUnavailable(NativeUnavailable):
    """The HIP kernel library is not built or cannot be loaded."""


class KernelError(RuntimeError):
    """A kernel entry point refused its arguments or its launch failed."""


class DecodeShape(ctypes.Structure):
    _fields_ = [
        ("batch", c_uint32),
        ("query_heads", c_uint32),
        ("kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("layers", c_uint32),
        ("slots", c_uint32),
        ("layer", c_uint32),
        ("table_width", c_uint32),
        ("q_format", c_int32),
        ("kv_format", c_int32),
        ("scale", c_float),
        ("table_stride", c_uint32),
        ("lengths_stride", c_uint32),
        ("flags", c_uint32),
    ]


class PrefillShape(ctypes.Structure):
    _fields_ = [
        ("tokens", c_uint32),
        ("start", c_uint32),
        ("query_heads", c_uint32),
        ("kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("layers", c_uint32),
        ("slots", c_uint32),
        ("layer", c_uint32),
        ("q_format", c_int32),
        ("kv_format", c_int32),
        ("scale", c_float),
    ]


_RECORDS = [c_void_p, c_void_p, c_uint32, c_void_p, c_uint64, c_uint32, c_void_p]
SIGNATURES = {
    "lk_fp8_quantize": (c_int, _RECORDS),
    "lk_fp8_dequantize": (c_int, _RECORDS),
    "lk_fp8_encode": (c_int, [c_void_p, c_void_p, c_uint64, c_int32, c_void_p]),
    "lk_fp8_decode": (c_int, [c_void_p, c_void_p, c_uint64, c_int32, c_void_p]),
    "lk_paged_decode_workspace": (c_uint64, [POINTER(DecodeShape)]),
    "lk_paged_decode": (c_int, [POINTER(DecodeShape), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p]),
    "lk_paged_decode_append": (c_int, [POINTER(DecodeShape), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_uint64, c_void_p]),
    "lk_paged_decode_static": (c_int, [POINTER(DecodeShape), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "lk_gather_blocks": (c_int, [c_void_p, c_void_p, c_uint32, c_uint64, c_void_p, c_void_p]),
    "lk_scatter_blocks": (c_int, [c_void_p, c_void_p, c_uint32, c_uint64, c_void_p, c_void_p]),
    "lk_stream_probe": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p]),
    "lk_stream_probe_mix": (c_int, [c_void_p, c_uint64, c_void_p, c_uint64, c_void_p]),
    "lk_tile_probe": (c_int, [POINTER(DecodeShape), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "lk_paged_prefill": (c_int, [POINTER(PrefillShape), c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p]),
    "lk_paged_prefill_workspace": (c_uint64, [POINTER(PrefillShape)]),
    "lk_paged_prefill_split": (c_int, [POINTER(PrefillShape), c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_uint64, c_void_p]),
    "lk_kv_write": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                            c_uint32, c_uint32, c_void_p]),
    "lk_fp8_append": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                              c_uint32, c_uint32, c_void_p]),
}

_lib: ctypes.CDLL | None = None


def library_path():
    return build_dir("hip") / LIBRARY_NAME


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (torch's HIP runtime first, see above)

    path = library_path()
    if not path.exists():
        raise KernelsUnavailable(f"{path} does not exist: build it with __graft_entry__.build() or 'make -C layover_amd/csrc hip'")
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as error:
        raise KernelsUnavailable(f"{path} cannot be loaded: {error}") from error
    if len(hip_runtimes_loaded()) > 1:
        raise KernelsUnavailable(f"two HIP runtimes are loaded: {hip_runtimes_loaded()}")
    lib.lk_abi_version.restype = c_int
    lib.lk_last_error.restype = c_char_p
    if lib.lk_abi_version() != ABI_VERSION:
        raise KernelsUnavailable(f"{path} has ABI {lib.lk_abi_version()}, expected {ABI_VERSION}")
    for name, (restype, argtypes) in SIGNATURES.items():
        function = getattr(lib, name)
        function.restype = restype
        function.argtypes = argtypes
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        raise KernelError(load().lk_last_error().decode())


def current_stream(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
