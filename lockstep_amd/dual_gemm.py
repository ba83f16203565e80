"""Dual-batch GEMMs on gfx950 -- drop-in for the reference's dual_gemm.py.

The reference asks whether two FP4 GEMMs can share one fp32 accumulator
(dual_gemm.py:1-15) and times a fused two-accumulator kernel as the fair
baseline.  With a shared weight (train_step.py:52-53, `dual_separate(a1, a2,
b, b)`) the two-accumulator form is the useful one: here it runs with the
weight in MXFP4, one launch, each weight tile loaded and dequantized once
for both batches (lockstep_amd/csrc/gemm_bf16f4.hip, `dual_mxfp4`).

slot_offset and unpack_dual are the reference's host-side slot arithmetic
(dual_gemm.py:23-32).
"""

from __future__ import annotations

import math

import torch

from . import _capi as C
from . import fp4 as _fp4
from .mxfp4_gemm import _rows16, _scales


def slot_offset(K: int) -> int:
    """Minimum 2^s separation for a K-deep FP4 dot product (+1 guard for sign)."""
    return int(math.floor(math.log2(144 * K))) + 2


def unpack_dual(acc: torch.Tensor, s: int):
    """Split acc = C1 + 2^s * C2 back into the two results (host side)."""
    w = float(2 ** s)
    c2 = torch.round(acc / w)
    return acc - c2 * w, c2


# Tile configuration of the gfx950 dual kernel (the reference's CFG keys).
CFG = dict(BLOCK_M=128, BLOCK_N=256, BLOCK_K=64, num_warps=4, num_stages=2)
_SK = dict(BM=128, BN=128, BK=64, warps=8, stages=3)


def dual_mxfp4(a0, a1, w_pk, w_scale, out_dtype=torch.bfloat16):
    """C0 = a0 @ deq(W).T and C1 = a1 @ deq(W).T in one launch.

    a0, a1 [M, K] bf16; w_pk [N, K//2] packed MXFP4; w_scale [N, K//32]
    (fp32 powers of two or E8M0 bytes).  Returns (C0, C1), [M, N] each."""
    M, K = a0.shape
    N, Kh = w_pk.shape
    assert a1.shape == a0.shape, "a0 and a1 must have the same shape"
    assert K == 2 * Kh and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    C.require_device(a0, a1, w_pk, w_scale)
    a0 = _rows16(a0.to(torch.bfloat16))
    a1 = _rows16(a1.to(torch.bfloat16))
    if a0.stride(0) != a1.stride(0):
        a0, a1 = a0.contiguous(), a1.contiguous()
    w_pk = _rows16(w_pk)
    w_scale = _scales(w_scale, N, K // 32)
    c0 = torch.empty((M, N), device=a0.device, dtype=out_dtype)
    c1 = torch.empty_like(c0)
    if M == 0 or N == 0:
        return c0, c1
    C.call("lsmx_gemm_dual_bf16f4", a0.data_ptr(), a1.data_ptr(), a0.stride(0) if M > 1 else K,
           w_pk.data_ptr(), w_pk.stride(0) if N > 1 else Kh, w_scale.data_ptr(),
           w_scale.stride(0) if N > 1 else K // 32, _fp4._scale_fmt(w_scale), c0.data_ptr(),
           c1.data_ptr(), C.dtype_code(out_dtype), N, M, N, K, C.stream_of(c0))
    return c0, c1


def _dense_not_built(name):
    raise NotImplementedError(
        f"dual_gemm.{name} on dense (non-MXFP4) operands is not built yet on gfx950; "
        "use dual_mxfp4 for the shared-weight MXFP4 form")


def gemm(a, b):
    """Single GEMM, one fp32 accumulator, fp32 out. a [M,K], b [K,N]."""
    _dense_not_built("gemm")


def dual_packed(a1, a2s, b1, b2):
    """Returns the PACKED fp32 tile. Call unpack_dual(acc, s) to split it."""
    _dense_not_built("dual_packed")


def dual_separate(a1, a2, b1, b2):
    """Two GEMMs, two fp32 accumulators, one launch."""
    _dense_not_built("dual_separate")


def splitk_packed(a1, a2s, b1, b2, splits=8, **kw):
    _dense_not_built("splitk_packed")


def splitk_separate(a1, a2, b1, b2, splits=8, **kw):
    _dense_not_built("splitk_separate")
