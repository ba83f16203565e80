"""MXFP4 linear layer on gfx950 -- drop-in for the reference's fp4_linear.py.

Forward (fp4_linear.py:34-40): quantize X and W along K to MXFP4 and run the
block-scaled FP4 x FP4 GEMM, output cast to x.dtype.  Here both quantizations
are the fused quantize+pack kernel (packed nibbles + E8M0 bytes, read straight
by the scaled MFMA GEMM).  Backward (fp4_linear.py:42-45): unquantized
straight-through, dX = gy @ w, dW = gy^T @ x at the input precision.

kernel() returns the gfx950 path, or None when no gfx950 GPU is present; the
reference's off-H100 fake-quant fallback does not exist here: without the
GPU path the layer raises.
"""

from __future__ import annotations

import functools

import torch
import torch.nn as nn

from . import _capi as C
from . import fp4
from .mxfp4_gemm import mxfp4_gemm_packed


@functools.cache
def kernel():
    """The gfx950 MXFP4 GEMM path (quantize + pack + scaled-MFMA GEMM), else None."""
    if not torch.cuda.is_available():
        return None
    try:
        C.load()
    except (OSError, RuntimeError):
        return None
    if C.load().lsmx_device_check() != C.OK:
        return None
    return _forward_hip


def path():
    return "hip-mxfp4" if kernel() else "unavailable"


def _forward_hip(x2: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    xp, xs = fp4.quantize_pack_mxfp4(x2)
    wp, ws = fp4.quantize_pack_mxfp4(w)
    return mxfp4_gemm_packed(xp, wp, xs, ws, out_dtype=x2.dtype)


class _MXFP4Matmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        k = kernel()
        if k is None:
            raise RuntimeError("MXFP4Linear needs a gfx950 GPU and liblsmx.so (path() == "
                               f"{path()!r}); there is no CPU fallback")
        return k(x, w)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        return (gy @ w.to(gy.dtype)).to(x.dtype), (gy.t() @ x.to(gy.dtype)).to(w.dtype)


class MXFP4Linear(nn.Linear):
    """nn.Linear whose forward GEMM runs in MXFP4 (bias unsupported)."""

    def __init__(self, fan_in, fan_out, bias=False):
        assert not bias, "MXFP4Linear has no bias"
        super().__init__(fan_in, fan_out, bias=False)

    def forward(self, x):
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
        with torch.autocast("cuda", enabled=False):
            y = _MXFP4Matmul.apply(x.reshape(-1, x.shape[-1]).to(dt), self.weight)
        return y.view(*x.shape[:-1], -1)
