"""lockstep_amd -- MI355X (gfx950) MXFP4 hot path of lockstep.

Modules mirror the reference's Python API:
    lockstep_amd.fp4          <- fp4.py
    lockstep_amd.mxfp4_gemm   <- mxfp4_gemm.py
    lockstep_amd.dual_gemm    <- dual_gemm.py
    lockstep_amd.fp4_linear   <- fp4_linear.py
    lockstep_amd.device       <- h100.py (device guard)
The kernels live in liblsmx.so (C ABI: include/lsmx.h), built by
lockstep_amd.build.
"""

__version__ = "0.1.0"
