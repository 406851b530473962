"""MI355X-native KV-cache data path for Layover: swap (gather + FP8 quantize to pinned host
memory and back) and paged GQA decode attention, as hand-written gfx950 HIP kernels behind
the reference's C ABI (include/layover_transfer.h) and Python call sites."""

from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
