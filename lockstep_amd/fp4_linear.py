"""MXFP4 linear layer on gfx950 -- drop-in for the reference's fp4_linear.py.

Forward (fp4_linear.py:34-40): quantize X and W along K to MXFP4 and run the
block-scaled FP4 x FP4 GEMM, output cast to x.dtype.  Here both quantizations
are the fused quantize+pack kernel (packed nibbles + E8M0 bytes, read straight
by the scaled MFMA GEMM).  Backward (fp4_linear.py:42-45): unquantized
straight-through, dX = gy @ w, dW = gy^T @ x at the input precision.

kernel() returns the gfx950 path, or None when no gfx950 GPU is present; the
reference's off-H100 fake-quant fallback does not exist here: without the
GPU path the layer raises.

MXFP4Linear(..., quantized_backward=True) (and mxfp4_matmul_q) also runs the
backward in MXFP4, which the reference does not: for Y = X W^T with X [T, K]
and W [N, K],
    dgrad  dX = dY W       contracts over N: dY quantized along its rows,
                           W along its columns (quantize_mxfp4_t),
    wgrad  dW = dY^T X     contracts over T: dY and X quantized along their
                           columns,
each followed by the block-scaled f4 x f4 GEMM with fp32 accumulation: six
quantizations and three GEMMs per linear, the scheme of train_step.py:3-6
with every GEMM in MXFP4.  T, N and K must be multiples of 128.
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
    # K-major E8M0 scales: the layout the GEMM streams fastest (same bits out)
    lay = "kmajor" if x2.shape[-1] % 128 == 0 else "rows"
    xp, xs = fp4.quantize_pack_mxfp4(x2, scale_layout=lay)
    wp, ws = fp4.quantize_pack_mxfp4(w, scale_layout=lay)
    return mxfp4_gemm_packed(xp, wp, xs, ws, out_dtype=x2.dtype)


def _mm_rows_cols(a: torch.Tensor, b: torch.Tensor, out_dtype) -> torch.Tensor:
    """a [M, R] @ b [R, N] in MXFP4: a quantized along its rows, b along its columns."""
    ap, as_ = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    bp, bs = fp4.quantize_mxfp4_t(b, scale_layout="kmajor")
    return mxfp4_gemm_packed(ap, bp, as_, bs, out_dtype=out_dtype)


def _mm_cols_cols(a: torch.Tensor, b: torch.Tensor, out_dtype) -> torch.Tensor:
    """a[R, M]^T @ b [R, N] in MXFP4: both quantized along their columns (axis R)."""
    ap, as_ = fp4.quantize_mxfp4_t(a, scale_layout="kmajor")
    bp, bs = fp4.quantize_mxfp4_t(b, scale_layout="kmajor")
    return mxfp4_gemm_packed(ap, bp, as_, bs, out_dtype=out_dtype)


def mxfp4_backward(gy: torch.Tensor, x: torch.Tensor, w: torch.Tensor):
    """(dX, dW) of Y = X W^T with both backward GEMMs in MXFP4.

    gy [T, N], x [T, K], w [N, K]; dX in x.dtype, dW in w.dtype."""
    T, K = x.shape
    N = w.shape[0]
    assert gy.shape == (T, N) and w.shape == (N, K), "shapes must be gy [T,N], x [T,K], w [N,K]"
    assert T % 128 == 0 and N % 128 == 0 and K % 128 == 0, \
        "the MXFP4 backward needs T, N and K to be multiples of 128"
    gy = gy.contiguous()
    dx = _mm_rows_cols(gy, w, x.dtype)          # dY [T,N] @ W [N,K]
    dw = _mm_cols_cols(gy, x, w.dtype)          # dY^T [N,T] @ X [T,K]
    return dx, dw


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


class _MXFP4MatmulQ(torch.autograd.Function):
    """_MXFP4Matmul with the backward GEMMs in MXFP4 too (see mxfp4_backward)."""

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
        return mxfp4_backward(gy, x, w)


def mxfp4_matmul(x2: torch.Tensor, w: torch.Tensor, quantized_backward: bool = False):
    """Y = X W^T with the forward in MXFP4; the backward in MXFP4 as well when
    quantized_backward, else unquantized straight-through (fp4_linear.py:42-45)."""
    fn = _MXFP4MatmulQ if quantized_backward else _MXFP4Matmul
    return fn.apply(x2, w)


class MXFP4Linear(nn.Linear):
    """nn.Linear whose forward GEMM runs in MXFP4 (bias unsupported).

    quantized_backward=False (the reference's behaviour) keeps the straight-
    through backward; True runs dgrad and wgrad as MXFP4 GEMMs."""

    def __init__(self, fan_in, fan_out, bias=False, quantized_backward=False):
        assert not bias, "MXFP4Linear has no bias"
        super().__init__(fan_in, fan_out, bias=False)
        self.quantized_backward = quantized_backward

    def forward(self, x):
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
        with torch.autocast("cuda", enabled=False):
            y = mxfp4_matmul(x.reshape(-1, x.shape[-1]).to(dt), self.weight, self.quantized_backward)
        return y.view(*x.shape[:-1], -1)
