"""bench.py's command-line contract, checked without a GPU: it measures one GPU and refuses
--gpus above 1 with a message, before touching the GPU; its separate modes are offered."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = run_bench("--gpus", "2")
    assert result.returncode == 2
    assert "one GPU" in result.stderr and result.stdout == ""


def test_the_separate_modes_are_offered():
    text = run_bench("--help").stdout
    for flag in ("--steps", "--warmup", "--decode-scan", "--duplex", "--overlap-only", "--skip-cpu"):
        assert flag in text
