"""CPU check that the persistent GEMM schedule only ever addresses real tiles.

Compiles tests/sched_check.hip (host code only, against the kernel's own
lockstep_amd/csrc/lsmx_sched.h) and runs it: every tile is covered exactly
once and every prefetch stage -- including the refills past a workgroup's
last tile -- resolves to in-bounds rows and K offsets.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_gemm_schedule_stays_in_bounds(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "sched_check"
    subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950", "-o", str(exe),
                    str(ROOT / "tests" / "sched_check.hip")], check=True, capture_output=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 failures" in res.stdout
