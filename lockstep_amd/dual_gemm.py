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
from .mxfp4_gemm import _rows16, _wscales, kmajor_operand, mxfp4_gemm_bf16


def slot_offset(K: int) -> int:
    """Minimum 2^s separation for a K-deep FP4 dot product (+1 guard for sign)."""
    return int(math.floor(math.log2(144 * K))) + 2


def unpack_dual(acc: torch.Tensor, s: int):
    """Split acc = C1 + 2^s * C2 back into the two results (host side)."""
    w = float(2 ** s)
    c2 = torch.round(acc / w)
    return acc - c2 * w, c2


# Tile configuration of the gfx950 dense kernels under the reference's CFG
# keys: the persistent ring kernel that gemm / dual_packed / dual_separate
# run on (csrc/gemm_dense_ring.hip: 256 x 256 tiles, 64-deep K stages,
# 8 waves, a 2-slot LDS ring) ...
CFG = dict(BLOCK_M=256, BLOCK_N=256, BLOCK_K=64, num_warps=8, num_stages=2)
# ... and the 128 x 128 kernel that runs K slices with fp32 atomics when the
# output has fewer 256 x 256 tiles than the GPU has CUs (csrc/gemm_dense.hip:
# 4 waves, double-buffered LDS).
_SK = dict(BM=128, BN=128, BK=64, warps=4, stages=2)


def dual_mxfp4(a0, a1, w_pk, w_scale, out_dtype=torch.bfloat16):
    """C0 = a0 @ deq(W).T and C1 = a1 @ deq(W).T in one launch.

    a0, a1 [M, K] bf16; w_pk [N, K//2] packed MXFP4; w_scale [N, K//32]
    (fp32 powers of two or E8M0 bytes).  Returns (C0, C1), [M, N] each.
    fp32 / fp16 batches are not narrowed to bf16: they run as two launches
    of the exact-split weight-only kernel (mxfp4_gemm_bf16), which reads W
    once per batch."""
    M, K = a0.shape
    N, Kh = w_pk.shape
    assert a1.shape == a0.shape, "a0 and a1 must have the same shape"
    assert K == 2 * Kh and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    if w_scale.dim() != 2 or tuple(w_scale.shape) != (N, K // 32):
        raise AssertionError(f"scale must be [{N}, {K // 32}] (rows, K//32), got {list(w_scale.shape)}")
    if a0.dtype != a1.dtype:
        raise TypeError(f"a0 and a1 dtypes differ: {a0.dtype} and {a1.dtype}")
    C.require_device(a0, a1, w_pk, w_scale)
    if a0.dtype != torch.bfloat16:
        return (mxfp4_gemm_bf16(a0, w_pk, w_scale, out_dtype=out_dtype),
                mxfp4_gemm_bf16(a1, w_pk, w_scale, out_dtype=out_dtype))
    a0 = _rows16(a0)
    a1 = _rows16(a1)
    if a0.stride(0) != a1.stride(0):
        a0, a1 = a0.contiguous(), a1.contiguous()
    w_pk = _rows16(w_pk)
    w_scale = _wscales(w_scale, N, K // 32)
    c0 = torch.empty((M, N), device=a0.device, dtype=out_dtype)
    c1 = torch.empty_like(c0)
    if M == 0 or N == 0:
        return c0, c1
    if K == 0:   # no K iteration: zeros
        return c0.zero_(), c1.zero_()
    nws = C.load().lsmx_gemm_bf16f4_workspace(M, N, K, 1)
    ws = C.workspace(a0.device, nws) if nws > 0 else None
    C.call("lsmx_gemm_bf16f4_ws", a0.data_ptr(), a1.data_ptr(), a0.stride(0) if M > 1 else K,
           w_pk.data_ptr(), w_pk.stride(0) if N > 1 else Kh, w_scale.data_ptr(),
           w_scale.stride(0) if N > 1 else K // 32, _fp4._scale_fmt(w_scale), c0.data_ptr(),
           c1.data_ptr(), C.dtype_code(out_dtype), N, M, N, K, ws.data_ptr() if ws is not None else None, nws,
           C.stream_of(c0))
    return c0, c1


# Dense operands (the reference's dual_gemm.py takes bf16 / fp16 / e4m3 tensors
# holding integer q-grid values, dual_gemm.py:1-15, train_step.py:90-105) run
# on lockstep_amd/csrc/gemm_dense.hip: 128 x 128 tiles, 64-deep K stages,
# fp32 accumulation on MFMA, fp32 outputs.
_DENSE = {torch.bfloat16: C.BF16, torch.float16: C.F16, torch.float8_e4m3fn: C.E4M3}
_BK = 64


def _ncontig(b: torch.Tensor, N: int) -> bool:
    """B [K, N] with unit stride along N, N % 8 == 0, 16-byte aligned rows and
    a row stride the N-contiguous kernel takes (at most 2^22 elements)."""
    ld = b.stride(0) if b.shape[0] > 1 else N
    return N % 8 == 0 and (b.stride(1) == 1 or N <= 1) and ld >= N and ld <= (1 << 22) and b.data_ptr() % 16 == 0 and \
        (ld * b.element_size()) % 16 == 0


def _dense(mode, a1, a2, b1, b2, out, splits=1):
    """Launch one dense kernel.  mode 0: out[0] = a1 b1; 1: out[0] = a1 b1 + a2 b2;
    2: out[0] = a1 b1, out[1] = a2 b2.  b* are [K, N]; a2 and b2 share a1's and
    b1's layouts (as the reference's kernels assume)."""
    M, K = a1.shape
    N = b1.shape[1]
    C.require_device(a1, b1, *([a2, b2] if mode else []))
    dt = a1.dtype
    if dt not in _DENSE:
        raise TypeError(f"dense GEMMs take bfloat16, float16 or float8_e4m3fn operands, got {dt}")
    for t in ([b1] + ([a2, b2] if mode else [])):
        if t.dtype != dt:
            raise TypeError(f"operand dtypes differ: {dt} and {t.dtype}")
    if mode:
        if a2.shape != a1.shape or b2.shape != b1.shape:
            raise ValueError("a1/a2 and b1/b2 must have the same shapes")
    if b1.shape[0] != K:
        raise ValueError(f"inner dimensions differ: a is [{M}, {K}], b is {list(b1.shape)}")
    if M == 0 or N == 0:
        return
    if K == 0:
        for o in out:
            o.zero_()
        return
    code = _DENSE[dt]
    if splits == 1 and dt != torch.float8_e4m3fn and _ncontig(b1, N) and (not mode or (
            _ncontig(b2, N) and b2.stride(0) == b1.stride(0))):
        # B as the reference passes it, [K, N] N-contiguous: the kernel reads
        # it directly (no transpose)
        a1 = _rows16(a1)
        a2p = 0
        if mode:
            a2 = _rows16(a2)
            if a2.stride(0) != a1.stride(0) and M > 1:
                a1, a2 = a1.contiguous(), a2.contiguous()
            a2p = a2.data_ptr()
        c1 = out[1].data_ptr() if mode == 2 else 0
        C.call("lsmx_gemm_dense_nb", a1.data_ptr(), a2p, a1.stride(0) if M > 1 else K, b1.data_ptr(),
               b2.data_ptr() if mode else 0, b1.stride(0) if K > 1 else N, code, mode, out[0].data_ptr(), c1, N, M,
               N, K, C.stream_of(out[0]))
        return
    raw = (lambda t: t.view(torch.uint8)) if dt == torch.float8_e4m3fn else (lambda t: t)
    a1 = _rows16(raw(a1))
    bt1 = kmajor_operand(raw(b1))
    a2p = bt2p = 0
    if mode:
        a2 = _rows16(raw(a2))
        if a2.stride(0) != a1.stride(0) and M > 1:
            a1, a2 = a1.contiguous(), a2.contiguous()
        bt2 = bt1 if b2 is b1 else kmajor_operand(raw(b2))
        if bt2.stride(0) != bt1.stride(0) and N > 1:
            bt1, bt2 = bt1.contiguous(), bt2.contiguous()
        a2p, bt2p = a2.data_ptr(), bt2.data_ptr()
    c1 = out[1].data_ptr() if mode == 2 else 0
    C.call("lsmx_gemm_dense", a1.data_ptr(), a2p, a1.stride(0) if M > 1 else K, bt1.data_ptr(), bt2p,
           bt1.stride(0) if N > 1 else K, code, mode, out[0].data_ptr(), c1, N, M, N, K, splits,
           C.stream_of(out[0]))


def gemm(a, b):
    """Single GEMM, one fp32 accumulator, fp32 out. a [M,K], b [K,N]."""
    M, K = a.shape
    N = b.shape[1]
    assert K % 64 == 0, "K must be a multiple of 64 (max BLOCK_K); zero-pad if shorter"
    out = torch.empty((M, N), device=a.device, dtype=torch.float32)
    _dense(0, a, None, b, None, (out,))
    return out


def dual_packed(a1, a2s, b1, b2):
    """Returns the PACKED fp32 tile. Call unpack_dual(acc, s) to split it."""
    M, K = a1.shape
    N = b1.shape[1]
    assert K % 64 == 0, "K must be a multiple of 64 (max BLOCK_K); zero-pad if shorter"
    out = torch.empty((M, N), device=a1.device, dtype=torch.float32)
    _dense(1, a1, a2s, b1, b2, (out,))
    return out


def dual_separate(a1, a2, b1, b2):
    """Two GEMMs, two fp32 accumulators, one launch.  With b1 is b2 (the
    shared-weight form) B is transposed once and each B tile feeds both."""
    M, K = a1.shape
    N = b1.shape[1]
    assert K % 64 == 0, "K must be a multiple of 64 (max BLOCK_K); zero-pad if shorter"
    c1 = torch.empty((M, N), device=a1.device, dtype=torch.float32)
    c2 = torch.empty_like(c1)
    _dense(2, a1, a2, b1, b2, (c1, c2))
    return c1, c2


def _splitk_check(K, splits, p):
    assert K % (splits * p["BK"]) == 0, "K must divide splits*BK"
    if (K // splits) % _BK:
        raise ValueError(f"each split's K ({K // splits}) must be a multiple of {_BK} on gfx950")


_RING_TILE = 256


def _launch_splits(a1, N, mode, splits):
    """K slices to launch.  The reference splits K to give a small output
    enough workgroups (dual_gemm.py:258-289); the sum is the same either way.
    When the 256 x 256 output tiles of the persistent bf16/fp16 kernel already
    number at least one per CU, the slices would only add atomic traffic, so
    each tile takes the whole K (one summation order, no atomics)."""
    M = a1.shape[0]
    if a1.dtype not in (torch.bfloat16, torch.float16):
        return splits
    C.require_device(a1)
    tiles = -(-M // _RING_TILE) * -(-N // _RING_TILE) * (2 if mode == 2 else 1)
    cus = torch.cuda.get_device_properties(a1.device).multi_processor_count
    return 1 if tiles >= cus else splits


def splitk_packed(a1, a2s, b1, b2, splits=8, **kw):
    """Packed accumulator over `splits` K slices, fp32 atomic adds into a zeroed
    output (or the whole K per tile when the output tiles fill the GPU)."""
    p = {**_SK, **kw}
    M, K = a1.shape
    N = b1.shape[1]
    _splitk_check(K, splits, p)
    ls = _launch_splits(a1, N, 1, splits)
    # slices add into zeros; a whole-K launch writes every element
    out = (torch.zeros if ls > 1 else torch.empty)((M, N), device=a1.device, dtype=torch.float32)
    _dense(1, a1, a2s, b1, b2, (out,), ls)
    return out


def splitk_separate(a1, a2, b1, b2, splits=8, **kw):
    """Two accumulators over `splits` K slices, fp32 atomic adds into zeroed
    outputs (or the whole K per tile when the output tiles fill the GPU)."""
    p = {**_SK, **kw}
    M, K = a1.shape
    N = b1.shape[1]
    _splitk_check(K, splits, p)
    ls = _launch_splits(a1, N, 2, splits)
    alloc = torch.zeros if ls > 1 else torch.empty
    o1 = alloc((M, N), device=a1.device, dtype=torch.float32)
    o2 = alloc((M, N), device=a1.device, dtype=torch.float32)
    _dense(2, a1, a2, b1, b2, (o1, o2), ls)
    return o1, o2
