"""The C-ABI libraries load without a GPU and export exactly what include/*.h declares.
No compute calls: on a machine without a GPU only loading and symbol lookup are checked."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from layover_amd.kernels import _lib
from layover_amd.kv import native

ROOT = Path(__file__).resolve().parents[1]


def declared(header: str) -> set[str]:
    text = (ROOT / "include" / header).read_text()
    return set(re.findall(r"^\s*(?:int|uint64_t|const char\*)\s+(l[tk]_\w+)\(", text, flags=re.M))


def exported(path: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_transfer_header_declares_the_reference_abi():
    names = declared("layover_transfer.h")
    assert len(names) == 26
    assert {"lt_out_gather", "lt_in_scatter", "lt_ext_copy_out", "lt_ext_finish", "lt_host_set_pin_limit"} <= names
    assert set(native.SIGNATURES) | {"lt_abi_version", "lt_flavor", "lt_last_error"} == names


@pytest.mark.parametrize("flavor", ["host", "hip"])
def test_transfer_library_exports_every_declared_symbol(flavor):
    path = native.library_path(flavor)
    assert path.exists(), f"{path} is not built"
    symbols = exported(path)
    assert declared("layover_transfer.h") <= symbols
    assert not {s for s in symbols if s.startswith(("hip", "__hip", "hsa_"))}, "the library must not re-export the HIP or HSA runtime"


def test_kernel_library_exports_every_declared_symbol():
    path = _lib.library_path()
    assert path.exists(), f"{path} is not built"
    names = declared("layover_kernels.h")
    assert names == {"lk_abi_version", "lk_last_error", "lk_fp8_quantize", "lk_fp8_dequantize", "lk_fp8_encode",
                     "lk_fp8_decode", "lk_paged_decode_workspace", "lk_paged_decode", "lk_stream_probe", "lk_fp8_append", "lk_kv_write",
                     "lk_paged_prefill", "lk_paged_prefill_workspace", "lk_paged_prefill_split", "lk_stream_probe_mix", "lk_paged_decode_append",
                     "lk_paged_decode_static", "lk_tile_probe", "lk_gather_blocks", "lk_scatter_blocks"}
    assert names <= exported(path)
    assert set(_lib.SIGNATURES) | {"lk_abi_version", "lk_last_error"} == names


def test_hip_libraries_load_into_one_hip_runtime_without_a_gpu():
    lib = native.load_library("hip")
    assert lib.lt_abi_version() == 2 and lib.lt_flavor() == b"hip"
    kernels = _lib.load()
    assert kernels.lk_abi_version() == 3
    assert len(native.hip_runtimes_loaded()) == 1


def test_decode_workspace_depends_on_shape_only_and_refuses_nonsense():
    kernels = _lib.load()
    shape = _lib.DecodeShape(32, 32, 8, 128, 36, 16, 0, 2048, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    size = kernels.lk_paged_decode_workspace(shape)
    # 256 (sequence, KV head) units x 2,048 blocks / 4,096 -> 128-block splits, 16 per row:
    # FP32 partials [32, 32, 16, 128 + 2].
    assert size == 32 * 32 * 16 * (128 + 2) * 4
    bad = _lib.DecodeShape(32, 30, 8, 128, 36, 16, 0, 2048, _lib.LK_BF16, _lib.LK_BF16, 1.0)
    assert kernels.lk_paged_decode_workspace(bad) == 0


def test_fp8_append_refuses_bad_arguments_without_launching():
    kernels = _lib.load()
    one = ctypes.c_int32(0)
    ptr = ctypes.addressof(one)
    assert kernels.lk_fp8_append(None, ptr, ptr, 1, 1, ptr, ptr, 0, 36, 8, 16, 128, None) == _lib.LK_ERR_INVALID
    assert b"null" in kernels.lk_last_error()
    assert kernels.lk_fp8_append(ptr, ptr, ptr, 1, 1, ptr, ptr, 36, 36, 8, 16, 128, None) == _lib.LK_ERR_INVALID
    assert b"layer" in kernels.lk_last_error()
    assert kernels.lk_fp8_append(ptr, ptr, ptr, 0, 1, ptr, ptr, 0, 36, 8, 16, 128, None) == _lib.LK_ERR_INVALID
    assert kernels.lk_fp8_append(ptr, ptr, ptr, 1, 1, ptr, ptr, 0, 36, 0, 16, 128, None) == _lib.LK_ERR_INVALID


def test_block_copies_refuse_bad_arguments_without_launching():
    kernels = _lib.load()
    word = ctypes.c_uint64(0)
    ptr = ctypes.addressof(word)
    assert kernels.lk_gather_blocks(None, ptr, 1, 64, ptr, None) == _lib.LK_ERR_INVALID
    assert b"null" in kernels.lk_last_error()
    assert kernels.lk_scatter_blocks(ptr, None, 1, 64, ptr, None) == _lib.LK_ERR_INVALID
    assert kernels.lk_gather_blocks(ptr, ptr, 1, 12, ptr, None) == _lib.LK_ERR_INVALID
    assert b"8-byte" in kernels.lk_last_error()
    assert kernels.lk_scatter_blocks(ptr + 4, ptr, 1, 64, ptr, None) == _lib.LK_ERR_INVALID


def test_headers_are_plain_c(tmp_path):
    """Both headers compile as C99 with warnings as errors (the reference's bindings and any C
    host include them), and every declared entry point is a function of that name."""
    names = sorted(declared("layover_transfer.h") | declared("layover_kernels.h"))
    source = tmp_path / "abi.c"
    source.write_text(
        "#include \"layover_transfer.h\"\n#include \"layover_kernels.h\"\n"
        "typedef void (*entry)(void);\n"
        "const entry entries[] = {\n" + "".join(f"    (entry){name},\n" for name in names) + "};\n"
        "int main(void) { return entries[0] == 0; }\n")
    result = subprocess.run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-Wno-cast-function-type", "-fsyntax-only",
                             f"-I{ROOT / 'include'}", str(source)], capture_output=True, text=True)
    assert result.returncode == 0, result.stderr



def test_block_copies_beyond_one_dispatch_are_refused_without_launching():
    """A gather or scatter of more 512-byte chunks than one dispatch's 2^32 work-items hold
    (64 lanes per chunk) is refused with LK_ERR_INVALID before anything touches memory."""
    kernels = _lib.load()
    word = ctypes.c_uint64(0)
    ptr = ctypes.addressof(word)
    block_bytes = 1 << 20  # 2,048 chunks of 512 bytes
    limit = (2**32 - 1) // 64 // 2048  # blocks per launch
    for function in (kernels.lk_gather_blocks, kernels.lk_scatter_blocks):
        assert function(ptr, ptr, limit + 1, block_bytes, ptr, None) == _lib.LK_ERR_INVALID
        assert b"too many chunks" in kernels.lk_last_error()
    assert kernels.lk_gather_blocks(ptr, ptr, 1, 2**40, ptr, None) == _lib.LK_ERR_INVALID

