"""MXFP4 linear layer on gfx950 -- drop-in for the reference's fp4_linear.py.

Forward (fp4_linear.py:34-40): quantize X and W along K to MXFP4 and run the
block-scaled FP4 x FP4 GEMM, output cast to x.dtype.  Here both quantizations
are the fused quantize+pack kernel (packed nibbles + E8M0 bytes, read straight
by the scaled MFMA GEMM).  Backward (fp4_linear.py:42-45): unquantized
straight-through, dX = gy @ w, dW = gy^T @ x at the input precision.

kernel() returns the packed-operand GEMM (mxfp4_gemm_packed, the callable the
reference's kernel() returns: fp4_linear.py:16-25) on a gfx950, or None when
no gfx950 GPU is present.  The reference's off-H100 fake-quant fallback does
not exist here: without the GPU path the layer raises, and path() says
"unavailable" where the reference would say "fake-quant".

MXFP4Linear(..., quantized_backward=True) (and mxfp4_matmul_q) also runs the
backward in MXFP4, which the reference does not: for Y = X W^T with X [T, K]
and W [N, K],
    dgrad  dX = dY W       contracts over N: dY quantized along its rows,
                           W along its columns (quantize_mxfp4_t),
    wgrad  dW = dY^T X     contracts over T: dY and X quantized along their
                           columns,
each followed by the block-scaled f4 x f4 GEMM with fp32 accumulation: the
scheme of train_step.py:3-6 with every GEMM in MXFP4.  Each of X, W and dY is
needed along two axes; fp4.quantize_pack_mxfp4_2d produces both forms from
one read, so a linear costs three quantization passes and three GEMMs.
T, N and K must be multiples of 128.
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
    """The gfx950 MXFP4 GEMM (mxfp4_gemm_packed: packed codes, scales, out_dtype),
    else None."""
    if not torch.cuda.is_available():
        return None
    try:
        C.load()
    except (OSError, RuntimeError):
        return None
    if C.load().lsmx_device_check() != C.OK:
        return None
    return mxfp4_gemm_packed


def path():
    return "hip-mxfp4" if kernel() else "unavailable"


def _forward_hip(x2: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The forward of fp4_linear.py:34-40 on the GPU: quantize X and W along K
    (fused quantize + pack kernels, E8M0 scales) and call kernel()."""
    # K-major E8M0 scales: the layout the GEMM streams fastest (same bits out)
    lay = "kmajor" if x2.shape[-1] % 128 == 0 else "rows"
    xp, xs = fp4.quantize_pack_mxfp4(x2, scale_layout=lay)
    wp, ws = fp4.quantize_pack_mxfp4(w, scale_layout=lay)
    return kernel()(xp, wp, xs, ws, out_dtype=x2.dtype)


def mxfp4_backward(gy: torch.Tensor, x: torch.Tensor, w: torch.Tensor):
    """(dX, dW) of Y = X W^T with both backward GEMMs in MXFP4.

    gy [T, N], x [T, K], w [N, K]; dX in x.dtype, dW in w.dtype."""
    T, K = x.shape
    N = w.shape[0]
    assert gy.shape == (T, N) and w.shape == (N, K), "shapes must be gy [T,N], x [T,K], w [N,K]"
    assert T % 128 == 0 and N % 128 == 0 and K % 128 == 0, \
        "the MXFP4 backward needs T, N and K to be multiples of 128"
    gy = gy.contiguous()
    # dY along N (dgrad) and along T (wgrad) from one read of dY
    gr, grs, gc, gcs = fp4.quantize_pack_mxfp4_2d(gy, scale_layout="kmajor")
    wc, wcs = fp4.quantize_mxfp4_t(w, scale_layout="kmajor")
    xc, xcs = fp4.quantize_mxfp4_t(x, scale_layout="kmajor")
    dx = mxfp4_gemm_packed(gr, wc, grs, wcs, out_dtype=x.dtype)     # dY [T,N] @ W [N,K]
    dw = mxfp4_gemm_packed(gc, xc, gcs, xcs, out_dtype=w.dtype)     # dY^T [N,T] @ X [T,K]
    return dx, dw


class _MXFP4Matmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        if kernel() is None:
            raise RuntimeError("MXFP4Linear needs a gfx950 GPU and liblsmx.so (path() == "
                               f"{path()!r}); there is no CPU fallback")
        return _forward_hip(x, w)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        return (gy @ w.to(gy.dtype)).to(x.dtype), (gy.t() @ x.to(gy.dtype)).to(w.dtype)


class _MXFP4MatmulQ(torch.autograd.Function):
    """_MXFP4Matmul with the backward GEMMs in MXFP4 too (see mxfp4_backward).

    When T, N and K are multiples of 128 the forward quantizes X and W along
    both axes in one pass each (fp4.quantize_pack_mxfp4_2d): the row forms
    feed the forward GEMM and the column forms -- exactly what the backward
    GEMMs need of X and W -- are saved instead of X and W, so the backward
    only quantizes dY (again both axes in one pass).  The gradients are bit
    for bit those of mxfp4_backward."""

    @staticmethod
    def forward(ctx, x, w):
        if kernel() is None:
            raise RuntimeError("MXFP4Linear needs a gfx950 GPU and liblsmx.so (path() == "
                               f"{path()!r}); there is no CPU fallback")
        T, K = x.shape
        N = w.shape[0]
        ctx.dtypes = (x.dtype, w.dtype)
        if T % 128 or N % 128 or K % 128:
            ctx.fused = False
            ctx.save_for_backward(x, w)
            return _forward_hip(x, w)
        ctx.fused = True
        xr, xrs, xc, xcs = fp4.quantize_pack_mxfp4_2d(x, scale_layout="kmajor")
        wr, wrs, wc, wcs = fp4.quantize_pack_mxfp4_2d(w, scale_layout="kmajor")
        ctx.save_for_backward(xc, xcs, wc, wcs)
        return mxfp4_gemm_packed(xr, wr, xrs, wrs, out_dtype=x.dtype)

    @staticmethod
    def backward(ctx, gy):
        if not ctx.fused:
            x, w = ctx.saved_tensors
            return mxfp4_backward(gy, x, w)
        xc, xcs, wc, wcs = ctx.saved_tensors
        gr, grs, gc, gcs = fp4.quantize_pack_mxfp4_2d(gy.contiguous(), scale_layout="kmajor")
        dx = mxfp4_gemm_packed(gr, wc, grs, wcs, out_dtype=ctx.dtypes[0])
        dw = mxfp4_gemm_packed(gc, xc, gcs, xcs, out_dtype=ctx.dtypes[1])
        return dx, dw


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
