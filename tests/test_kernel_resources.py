"""Every gfx950 kernel keeps its working set in registers: no scratch memory, no spills and no
calls. A kernel that loses this silently slows down by 2x or more (an FP8 staging struct once
ended up in scratch behind a non-inlined lambda: its loads were waited for on the spot), so the
compiler's own resource report is checked here, on the CPU, by compiling to assembly with
each file's options from the Makefile."""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "layover_amd" / "csrc"
INCLUDE = Path(__file__).resolve().parents[1] / "include"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc is not installed")


def assembly(source: str, tmp_path: Path, *extra: str) -> str:
    out = tmp_path / (source + ".s")
    subprocess.run([HIPCC, "-std=c++17", "-O3", "--offload-arch=gfx950", f"-I{INCLUDE}", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", "-Wno-unused-command-line-argument", *extra, "--cuda-device-only", "-S", str(CSRC / source), "-o",
                    str(out)], check=True, capture_output=True, text=True)
    return out.read_text()


@pytest.mark.parametrize(
    "source,extra",
    [("kernels.hip", ()), ("prefill.hip", ("-mllvm", "--amdgpu-sched-strategy=max-ilp")), ("fp8_records.hip", ("-fgpu-flush-denormals-to-zero",))],
)
def test_kernels_use_no_scratch_spills_or_calls(source, extra, tmp_path):
    text = assembly(source, tmp_path, *extra)
    kernels = re.findall(r"\.name:\s+(\S+)\n\s+\.private_segment_fixed_size:\s+(\d+)", text)
    assert kernels, "no kernel metadata found"
    assert not [name for name, size in kernels if int(size)], f"kernels using scratch: {[k for k in kernels if int(k[1])]}"
    assert not re.findall(r"\.vgpr_spill_count:\s+[1-9]", text)
    assert not re.findall(r"\.sgpr_spill_count:\s+[1-9]", text)
    assert "s_swappc" not in text
