"""ctypes binding of liblsmx.so (declared in include/lsmx.h).

Loading never compiles: build with `python -m lockstep_amd.build` (or
__graft_entry__.build()).  A missing library raises at import of the first
op that needs it -- there is no CPU or torch fallback for the kernels.
"""

from __future__ import annotations

import ctypes
import itertools
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblsmx.so"

OK = 0
ERR_SHAPE, ERR_ALIGN, ERR_DTYPE, ERR_DEVICE, ERR_LAUNCH, ERR_ARG = -1, -2, -3, -4, -5, -6
F32, BF16, F16, E4M3 = 0, 1, 2, 3
E8M0_IN_T, E8M0_OUT_KMAJOR = 1, 2
CODES_PACKED, CODES_UNPACKED = 0, 1
B_NCONTIG = 0x10  # lsmx_gemm_mx_promote op_fmt bit: B [K, ldb] N-contiguous E4M3
SCALE_E8M0, SCALE_F32, SCALE_E8M0_KMAJOR = 0, 1, 2

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> argtypes, in the order of include/lsmx.h
SIGNATURES = {
    "lsmx_version": [],
    "lsmx_last_error": [],
    "lsmx_device_check": [],
    "lsmx_quantize_mxfp4": [_vp, _int, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _int, _i64, _vp],
    "lsmx_quantize_mxfp4_batch": [_vp, _int, _int, _int, _vp],
    "lsmx_quantize_mxfp4_t": [_vp, _int, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _int, _i64, _vp],
    "lsmx_quantize_mxfp4_2d": [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp],
    "lsmx_quantize_mxfp4_2d_batch": [_vp, _int, _int, _int, _vp],
    "lsmx_round_e2m1": [_vp, _int, _i64, _vp, _vp],
    "lsmx_pack_fp4": [_vp, _vp, _i64, _vp],
    "lsmx_unpack_fp4": [_vp, _vp, _i64, _vp],
    "lsmx_dequantize_mxfp4": [_vp, _int, _i64, _vp, _int, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp],
    "lsmx_fp4_to_e4m3": [_vp, _vp, _i64, _vp],
    "lsmx_gemm_f4f4": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_f4f4_quant": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                             _vp, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_bf16f4": [_vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_bf16f4_workspace": [_i64, _i64, _i64, _int],
    "lsmx_gemm_bf16f4_ws": [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp,
                            _i64, _vp],
    "lsmx_gemm_bf16f4_noalloc": [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _int, _i64, _i64, _i64, _i64,
                                 _vp],
    "lsmx_gemm_wonly_f4": [_vp, _int, _i64, _vp, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_dual_bf16f4": [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _int, _i64, _i64, _i64,
                              _i64, _vp],
    "lsmx_gemm_dense": [_vp, _vp, _i64, _vp, _vp, _i64, _int, _int, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp],
    "lsmx_gemm_dense_nb": [_vp, _vp, _i64, _vp, _vp, _i64, _int, _int, _vp, _vp, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_f8f8": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp],
    "lsmx_gemm_f8f8_nb": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _vp],
    "lsmx_transpose": [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp],
    "lsmx_scale_to_e8m0": [_vp, _i64, _i64, _i64, _int, _vp, _i64, _vp],
    "lsmx_scale_to_e8m0_batch": [_vp, _int, _vp, _u64, _vp],
    "lsmx_gemm_mx_promote": [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _int, _vp, _int, _i64, _i64,
                             _i64, _i64, _vp, _u64, _vp],
}

RET_I64 = ("lsmx_gemm_bf16f4_workspace",)


class QItem(ctypes.Structure):
    """lsmx_q_item of include/lsmx.h."""
    _fields_ = [("x", _vp), ("rows", _i64), ("K", _i64), ("ldx", _i64), ("codes", _vp), ("ld_codes", _i64),
                ("scale", _vp), ("ld_scale", _i64)]


class Q2dItem(ctypes.Structure):
    """lsmx_q2d_item of include/lsmx.h."""
    _fields_ = [("x", _vp), ("rows", _i64), ("cols", _i64), ("ldx", _i64),
                ("codes_r", _vp), ("ld_codes_r", _i64), ("scale_r", _vp), ("ld_scale_r", _i64),
                ("codes_c", _vp), ("ld_codes_c", _i64), ("scale_c", _vp), ("ld_scale_c", _i64)]


class E8m0Item(ctypes.Structure):
    """lsmx_e8m0_item of include/lsmx.h."""
    _fields_ = [("s", _vp), ("rows", _i64), ("cols", _i64), ("lds", _i64), ("layout", _int), ("out", _vp),
                ("ldo", _i64)]


# Epochs for lsmx_scale_to_e8m0_batch's flag: unique within the process and
# starting at a random value, so no earlier content of a flag equals a new one.
_epochs = itertools.count((int.from_bytes(os.urandom(6), "little") << 16) | 1)


def next_epoch() -> int:
    return next(_epochs) & 0xFFFFFFFFFFFFFFFF


_lib = None
_lock = threading.Lock()


class LsmxError(RuntimeError):
    """A liblsmx call returned a non-zero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[lsmx {code}] {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load liblsmx.so once; raise loudly if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP kernels with "
                    "`python -m lockstep_amd.build` (no CPU fallback exists)")
            L = ctypes.CDLL(str(LIB_PATH))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = argtypes
                fn.restype = (ctypes.c_char_p if name in ("lsmx_version", "lsmx_last_error") else
                              ctypes.c_int64 if name in RET_I64 else ctypes.c_int)
            _lib = L
    return _lib


def version() -> str:
    return load().lsmx_version().decode()


def last_error() -> str:
    return load().lsmx_last_error().decode()


def call(name: str, *args) -> None:
    """Call an entry point and raise LsmxError on a non-zero status."""
    rc = getattr(load(), name)(*args)
    if rc != OK:
        raise LsmxError(rc, last_error())


def stream_of(t: torch.Tensor) -> int:
    """The raw hipStream_t of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {dt}: expected float32, bfloat16 or float16")


def require_device(*tensors: torch.Tensor) -> None:
    """The kernels take device memory only: refuse CPU tensors loudly."""
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "lockstep_amd runs its MXFP4 ops on a gfx950 GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")


_workspaces: dict = {}
_captured: list = []


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A device workspace of at least nbytes for the split-K GEMMs.

    Eager calls share one per (device, stream): calls on one stream are
    ordered, so they may share it.  It is kept for later calls and grown by
    replacing it with a larger one (the old one returns to torch's caching
    allocator, stream-ordered).

    A call made while the current stream is being captured into a graph gets
    a workspace of its own that is never freed: the graph's replays write to
    that address whenever they run, so it may neither be handed to another
    tensor (as a replaced cache entry would be) nor shared with other
    graphs, which can be replayed concurrently on other streams."""
    if torch.cuda.is_current_stream_capturing():
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _captured.append(ws)
        return ws
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws
