"""Build liblsmx.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m lockstep_amd.build          # or lockstep_amd.build.build()

hipcc cross-compiles for gfx950 without a GPU present, so this runs on any
host with ROCm.  Every call compiles (no staleness check): callers that only
want to load the library use lockstep_amd._capi, which never compiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "liblsmx.so"
SOURCES = ["capi.hip", "quantize.hip", "gemm_f4f4.hip", "gemm_bf16f4.hip", "gemm_dense.hip", "gemm_dense_ring.hip", "gemm_f8f8.hip", "gemm_promote.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in the device code.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: ROCm is required to build liblsmx.so")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source to an object in parallel (each kernel is launched
    from its own translation unit, so no relocatable device code is needed),
    then link liblsmx.so."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [objdir / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[cc, *compile_flags, "-c", "-o", str(o), str(CSRC / s)] for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    print(f"built {LIB}", file=sys.stderr)
