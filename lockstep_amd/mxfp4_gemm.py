"""MXFP4 GEMMs on gfx950's scaled MFMA -- drop-in for the reference's mxfp4_gemm.py.

The reference emulates MXFP4 on Hopper FP8 tensor cores and promotes to an
fp32 accumulator at every 32-block to apply the scales (mxfp4_gemm.py:1-14).
gfx950 has block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4 and its
32 x 32 x 64 form): each lane hands the instruction 32 FP4 codes of one row
plus that block's E8M0 scale, so no promotion step exists and the packed
nibbles go straight from HBM to the matrix cores.  Kernels:
lockstep_amd/csrc/gemm_f4f4.hip.

Same names and signatures as mxfp4_gemm.py:23-174; the `CFG` dict keeps the
reference's keys for callers that read it, with this build's tile sizes.
"""

from __future__ import annotations

import torch

from . import _capi as C
from . import fp4 as _fp4

# Tile configuration of the f4 x f4 kernel that runs at K % 256 == 0
# (csrc/gemm_f4f4.hip, gemm_f4f4_mx16_kernel), under the reference's CFG
# keys: 256 x 256 tiles, SUB*32 = 256 K codes (two 128-code MFMA K-steps)
# per stage, 4-row tile groups, 8 waves of 64 lanes, a 2-slot LDS ring.
CFG = dict(BLOCK_M=256, BLOCK_N=256, SUB=8, GROUP_M=4, num_warps=8, num_stages=2)


def _out_code(dt: torch.dtype) -> int:
    return C.dtype_code(dt)


def _rows16(t: torch.Tensor) -> torch.Tensor:
    """Unit stride along K and 16-byte aligned rows, else a contiguous copy."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 or (t.shape[0] > 1 and t.stride(0) % 16):
        t = t.contiguous()
    return t


def _scales(s: torch.Tensor, rows: int, nkb: int) -> torch.Tensor:
    """Row-major block scales [rows, nkb] with unit stride along the blocks
    and 4-byte aligned rows.  The kernels size their scale reads from the GEMM
    shape, so a tensor of any other shape is refused before any launch."""
    assert s.dim() == 2 and tuple(s.shape) == (rows, nkb), \
        f"scale must be [{rows}, {nkb}] (rows, K//32), got {list(s.shape)}"
    fmt_bytes = 4 if s.dtype == torch.float32 else 1
    if s.stride(-1) != 1 or (rows > 1 and (s.stride(0) * fmt_bytes) % (4 * fmt_bytes)) \
            or s.data_ptr() % (4 * fmt_bytes):
        s = s.contiguous()
    return s


def mxfp4_gemm_packed(a_pk, bt_pk, a_scale, b_scale, out_dtype=torch.bfloat16):
    """a_pk [M,K//2] uint8, bt_pk [N,K//2] uint8, a_scale [M,K//32], b_scale [N,K//32].

    Scales are fp32 (as fp4.quantize_mxfp4 returns) or E8M0 bytes (as
    fp4.quantize_pack_mxfp4 returns), row-major [rows, K//32] or K-major
    [K//128, rows, 4] (quantize_pack_mxfp4(..., scale_layout="kmajor")); both
    operands must use the same format.  Row-major scales are regrouped to
    K-major E8M0 on the device first (fp32 through lsmx_scale_to_e8m0_batch,
    E8M0 bytes through a dword transpose), so every format runs the same
    kernel and gives the same bits.  fp32 scales that are not all powers of
    two or NaN (1.5, 0, -2, inf ...; the quantizer never makes them) have no
    E8M0 form: the conversion flags them and lsmx_gemm_mx_promote then
    recomputes C with the reference's own promotion arithmetic
    (mxfp4_gemm.py:141-150), a vector-ALU-bound fallback; with powers of two
    that launch exits at once, and for scales fp4.quantize_mxfp4 returned
    (and nobody wrote since) it is not made.  Returns C = A @ B_T.T [M, N]
    in out_dtype, fp32 accumulate."""
    M, Kh = a_pk.shape
    N, Kh2 = bt_pk.shape
    K = Kh * 2
    assert Kh == Kh2 and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    assert a_scale.dtype == b_scale.dtype and a_scale.dim() == b_scale.dim(), \
        "a_scale and b_scale must share a format"
    if a_scale.dim() == 2:
        for s, rows in ((a_scale, M), (b_scale, N)):
            if tuple(s.shape) != (rows, K // 32):
                raise AssertionError(f"scale must be [{rows}, {K // 32}] (rows, K//32), got {list(s.shape)}")
    C.require_device(a_pk, bt_pk, a_scale, b_scale)
    a_pk, bt_pk = _rows16(a_pk), _rows16(bt_pk)
    c = torch.empty((M, N), device=a_pk.device, dtype=out_dtype)
    if M == 0 or N == 0:
        return c
    if K == 0:   # the reference's K loop runs no iteration: C = 0
        return c.zero_()
    if a_scale.dim() == 3:
        assert a_scale.dtype == torch.uint8, "K-major scales are E8M0 bytes"
        assert a_scale.shape == (K // 128, M, 4) and b_scale.shape == (K // 128, N, 4), \
            "K-major scales must be [K//128, rows, 4]"
        a_scale, b_scale = a_scale.contiguous(), b_scale.contiguous()
        fmt, lsa, lsb = C.SCALE_E8M0_KMAJOR, M, N
        promote = None
    elif a_scale.dtype == torch.uint8:
        # row-major E8M0 bytes: regroup to the K-major layout the GEMM
        # streams fastest (one dword per row per 128 codes, rows contiguous)
        a_scale = _e8m0_kmajor(a_scale, M, K // 32, transposed=False)
        b_scale = _e8m0_kmajor(b_scale, N, K // 32, transposed=False)
        fmt, lsa, lsb = C.SCALE_E8M0_KMAJOR, M, N
        promote = None
    else:
        # the reference's spelling (fp32 scales from quantize_mxfp4)
        exact = _fp4.e8m0_exact(a_scale, b_scale)
        sa32, sb32 = _f32_rows(a_scale), _f32_rows(b_scale)
        (a_scale, b_scale), flag, epoch = _e8m0_kmajor_flagged([(sa32, M, False), (sb32, N, False)], K // 32,
                                                               flagged=not exact)
        fmt, lsa, lsb = C.SCALE_E8M0_KMAJOR, M, N
        promote = None if exact else (sa32, False, sb32, False, flag, epoch)
    lda, ldb = a_pk.stride(0) if M > 1 else Kh, bt_pk.stride(0) if N > 1 else Kh
    C.call("lsmx_gemm_f4f4", a_pk.data_ptr(), lda, a_scale.data_ptr(), lsa, bt_pk.data_ptr(), ldb,
           b_scale.data_ptr(), lsb, fmt, c.data_ptr(), _out_code(out_dtype), N, M, N, K, C.stream_of(c))
    if promote is not None:
        _promote(a_pk, lda, bt_pk, ldb, C.CODES_PACKED, c, K, *promote)
    return c


def mxfp4_gemm_packed_q2d(a_pk, bt_pk, a_scale, b_scale, keep_output: bool = False):
    """C = mxfp4_gemm_packed(a_pk, bt_pk, a_scale, b_scale) in bf16, returned
    quantized along both axes:

        (row_packed, row_scale, col_packed, col_scale) ==
            fp4.quantize_pack_mxfp4_2d(C, scale_layout="kmajor")

    bit for bit, with C itself appended when keep_output.  Scales in and out
    are K-major E8M0 [K//128, rows, 4] (quantize_pack_mxfp4(...,
    scale_layout="kmajor")).  With M, N and K multiples of 256 the GEMM's
    epilogue quantizes its tile in registers (lsmx_gemm_f4f4_quant), so the
    bf16 C is written only when asked for and never read back; other shapes
    run the GEMM and then the two-axis quantizer."""
    M, Kh = a_pk.shape
    N, Kh2 = bt_pk.shape
    K = Kh * 2
    assert Kh == Kh2 and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    assert a_scale.dtype == torch.uint8 and a_scale.shape == (K // 128, M, 4) and b_scale.shape == (K // 128, N, 4), \
        "mxfp4_gemm_packed_q2d takes K-major E8M0 scales [K//128, rows, 4]"
    if M % 256 or N % 256 or K % 256:
        c = mxfp4_gemm_packed(a_pk, bt_pk, a_scale, b_scale, out_dtype=torch.bfloat16)
        from .fp4 import quantize_pack_mxfp4_2d
        r = quantize_pack_mxfp4_2d(c, scale_layout="kmajor")
        return (*r, c) if keep_output else r
    C.require_device(a_pk, bt_pk, a_scale, b_scale)
    a_pk, bt_pk = _rows16(a_pk), _rows16(bt_pk)
    a_scale, b_scale = a_scale.contiguous(), b_scale.contiguous()
    dev = a_pk.device
    rp = torch.empty((M, N // 2), dtype=torch.uint8, device=dev)
    rs = torch.empty((N // 128, M, 4), dtype=torch.uint8, device=dev)
    cp = torch.empty((N, M // 2), dtype=torch.uint8, device=dev)
    cs = torch.empty((M // 128, N, 4), dtype=torch.uint8, device=dev)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev) if keep_output else None
    if M and N:
        C.call("lsmx_gemm_f4f4_quant", a_pk.data_ptr(), a_pk.stride(0) if M > 1 else Kh, a_scale.data_ptr(), M,
               bt_pk.data_ptr(), bt_pk.stride(0) if N > 1 else Kh, b_scale.data_ptr(), N,
               c.data_ptr() if c is not None else None, N, rp.data_ptr(), N // 2, rs.data_ptr(), M,
               cp.data_ptr(), M // 2, cs.data_ptr(), N, M, N, K, C.stream_of(rp))
    return (rp, rs, cp, cs, c) if keep_output else (rp, rs, cp, cs)


_ACT = {torch.bfloat16: C.BF16, torch.float32: C.F32, torch.float16: C.F16}


def mxfp4_gemm_bf16(a, w_pk, w_scale, out_dtype=torch.bfloat16):
    """Weight-only GEMM: activations a [M,K] x MXFP4 weight w_pk [N,K//2] with
    w_scale [N,K//32] (fp32 powers of two or E8M0).  Returns a @ deq(W).T
    [M, N] in out_dtype, fp32 accumulate.

    bf16 activations run the bf16 MFMA kernels directly.  fp32 and fp16
    activations are not narrowed: each is split exactly into bf16 terms
    (lsmx_gemm_wonly_f4), so an fp32 X gives the arithmetic of an fp32
    matmul (the reference's fake-quant Y = X @ dequantize_mxfp4(W)^T)."""
    M, K = a.shape
    N, Kh = w_pk.shape
    assert K == 2 * Kh and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    if w_scale.dim() != 2 or tuple(w_scale.shape) != (N, K // 32):
        raise AssertionError(f"scale must be [{N}, {K // 32}] (rows, K//32), got {list(w_scale.shape)}")
    if a.dtype not in _ACT:
        raise TypeError(f"activations must be bfloat16, float32 or float16, got {a.dtype}")
    C.require_device(a, w_pk, w_scale)
    if M == 0 or N == 0 or K == 0:   # K == 0: no K iteration, zeros
        return torch.zeros((M, N), device=a.device, dtype=out_dtype)
    a = _rows16(a)
    w_pk = _rows16(w_pk)
    w_scale = _wscales(w_scale, N, K // 32)
    c = torch.empty((M, N), device=a.device, dtype=out_dtype)
    if a.dtype == torch.bfloat16:
        # with a workspace the library may split K (mid-size M against a wide W)
        nws = C.load().lsmx_gemm_bf16f4_workspace(M, N, K, 0)
        ws = C.workspace(a.device, nws) if nws > 0 else None
        C.call("lsmx_gemm_bf16f4_ws", a.data_ptr(), None, a.stride(0) if M > 1 else K, w_pk.data_ptr(),
               w_pk.stride(0) if N > 1 else Kh, w_scale.data_ptr(), w_scale.stride(0) if N > 1 else K // 32,
               _fp4._scale_fmt(w_scale), c.data_ptr(), None, _out_code(out_dtype), N, M, N, K,
               ws.data_ptr() if ws is not None else None, nws, C.stream_of(c))
        return c
    C.call("lsmx_gemm_wonly_f4", a.data_ptr(), _ACT[a.dtype], a.stride(0) if M > 1 else K, w_pk.data_ptr(),
           w_pk.stride(0) if N > 1 else Kh, w_scale.data_ptr(), w_scale.stride(0) if N > 1 else K // 32,
           _fp4._scale_fmt(w_scale), c.data_ptr(), _out_code(out_dtype), N, M, N, K, C.stream_of(c))
    return c


def _wscales(s: torch.Tensor, rows: int, nkb: int) -> torch.Tensor:
    """Weight scales for the weight-only kernels as E8M0 bytes [rows, nkb]
    with 16-byte aligned rows: fp32 powers of two are converted on the device
    (a non-power of two becomes E8M0 NaN, as the kernels' own fp32 path
    treats it), so that fp32 and E8M0 forms of one weight run the same
    kernels -- the ring and split-K kernels read E8M0 rows -- and give the
    same bits."""
    s = _scales(s, rows, nkb)
    if s.dtype == torch.float32:
        s = _e8m0_rows(s, rows, nkb, transposed=False)
    return s


def mxfp4_linear_w(a, w_pk, w_scale, out_dtype=None):
    """Y = a @ deq(W)^T for an unquantized activation a [..., K] (any of
    bf16 / fp32 / fp16) and a packed MXFP4 weight: the weight-only linear
    forward, output in a's dtype unless out_dtype is given."""
    K = a.shape[-1]
    y = mxfp4_gemm_bf16(a.reshape(-1, K), w_pk, w_scale, out_dtype=out_dtype or a.dtype)
    return y.reshape(*a.shape[:-1], w_pk.shape[0])


def _e8m0_rows(s: torch.Tensor, rows: int, nkb: int, transposed: bool) -> torch.Tensor:
    """Block scales as E8M0 bytes [rows, nkb]: from fp32 [rows, nkb] (or
    [nkb, rows] when transposed) through lsmx_scale_to_e8m0, or from E8M0
    bytes of the same shapes.  An fp32 scale that is not a power of two in
    [2^-127, 2^127] becomes E8M0 NaN, so the outputs that use it are NaN."""
    shape = (nkb, rows) if transposed else (rows, nkb)
    assert tuple(s.shape) == shape
    out = torch.empty((rows, nkb), device=s.device, dtype=torch.uint8)
    if rows == 0 or nkb == 0:
        return out
    if s.dtype == torch.uint8:
        if not transposed:
            return s.contiguous()
        if s.t().is_contiguous():
            return s.t()  # a transposed view of row-major bytes
        s = s.contiguous()
        C.call("lsmx_transpose", s.data_ptr(), 1, nkb, rows, rows, out.data_ptr(), nkb, C.stream_of(out))
        return out
    if s.dtype != torch.float32:
        s = s.float()
    if s.stride(-1) != 1:
        s = s.contiguous()
    C.call("lsmx_scale_to_e8m0", s.data_ptr(), shape[0], shape[1], s.stride(0) if shape[0] > 1 else shape[1],
           int(transposed), out.data_ptr(), nkb, C.stream_of(out))
    return out


def _e8m0_kmajor(s: torch.Tensor, rows: int, nkb: int, transposed: bool) -> torch.Tensor:
    """Block scales [rows, nkb] (or [nkb, rows] when transposed) as K-major
    E8M0 bytes [nkb//4, rows, 4], the layout the E4M3 GEMM streams fastest.
    fp32 scales go through lsmx_scale_to_e8m0 (non-powers of two become E8M0
    NaN as above); E8M0 bytes are regrouped with lsmx_transpose: row-major
    bytes [rows, nkb] are [rows, nkb/4] dwords, and their transpose
    [nkb/4, rows] is the K-major layout."""
    shape = (nkb, rows) if transposed else (rows, nkb)
    assert tuple(s.shape) == shape
    out = torch.empty((nkb // 4, rows, 4), device=s.device, dtype=torch.uint8)
    if rows == 0 or nkb == 0:
        return out
    if s.dtype == torch.uint8:
        rm = _e8m0_rows(s, rows, nkb, transposed).contiguous()
        if rm.data_ptr() % 4:
            rm = rm.clone()  # dword view: 4-byte aligned storage
        C.call("lsmx_transpose", rm.data_ptr(), 4, rows, nkb // 4, nkb // 4, out.data_ptr(), rows, C.stream_of(out))
        return out
    if s.dtype != torch.float32:
        s = s.float()
    if s.stride(-1) != 1:
        s = s.contiguous()
    layout = C.E8M0_OUT_KMAJOR | (C.E8M0_IN_T if transposed else 0)
    C.call("lsmx_scale_to_e8m0", s.data_ptr(), shape[0], shape[1], s.stride(0) if shape[0] > 1 else shape[1],
           layout, out.data_ptr(), rows, C.stream_of(out))
    return out


def _f32_rows(s: torch.Tensor) -> torch.Tensor:
    """fp32 scales with unit stride along the last axis."""
    if s.dtype != torch.float32:
        s = s.float()
    return s if s.stride(-1) == 1 or s.shape[-1] <= 1 else s.contiguous()


def _ld(s: torch.Tensor) -> int:
    return s.stride(0) if s.shape[0] > 1 else s.shape[1]


def _e8m0_kmajor_flagged(scales, nkb: int, flagged: bool = True):
    """fp32 block scales -> K-major E8M0 bytes [nkb//4, rows, 4] for the fast
    kernels, all tensors in one launch (lsmx_scale_to_e8m0_batch).  scales:
    (s, rows, transposed) with s [rows, nkb], or [nkb, rows] when transposed.
    Returns (outputs, flag, epoch): when flagged, the launch writes epoch to
    the device word flag if some scale is neither a power of two nor a NaN,
    which lsmx_gemm_mx_promote checks (flag None otherwise)."""
    dev = scales[0][0].device
    flag = torch.empty(1, dtype=torch.int64, device=dev) if flagged else None
    epoch = C.next_epoch() if flagged else 0
    items = (C.E8m0Item * len(scales))()
    outs = []
    for k, (s, rows, tr) in enumerate(scales):
        out = torch.empty((nkb // 4, rows, 4), device=dev, dtype=torch.uint8)
        items[k] = C.E8m0Item(s.data_ptr(), s.shape[0], s.shape[1], _ld(s), C.E8M0_IN_T if tr else 0,
                              out.data_ptr(), rows)
        outs.append(out)
    C.call("lsmx_scale_to_e8m0_batch", items, len(scales), flag.data_ptr() if flagged else None, epoch,
           C.stream_of(outs[0]))
    return outs, flag, epoch


def _promote(a, lda, bt, ldb, op_fmt, c, K, sa, sa_tr, sb, sb_tr, flag, epoch):
    """lsmx_gemm_mx_promote over c when flag == epoch: the reference's fp32
    promotion for scales the fast kernels cannot apply.  sa [M, K//32] (or
    [K//32, M] when sa_tr), likewise sb."""
    M, N = c.shape

    def strides(s, tr):  # (row stride, block stride); a size-1 axis gets its dense stride
        rows, nkb = (s.shape[1], s.shape[0]) if tr else s.shape
        r, k = (s.stride(1), s.stride(0)) if tr else (s.stride(0), s.stride(1))
        return (r if rows > 1 else (1 if tr else nkb)), (k if nkb > 1 else (rows if tr else 1))

    (sa_r, sa_k), (sb_r, sb_k) = strides(sa, sa_tr), strides(sb, sb_tr)
    C.call("lsmx_gemm_mx_promote", a.data_ptr(), lda, sa.data_ptr(), sa_r, sa_k, bt.data_ptr(), ldb,
           sb.data_ptr(), sb_r, sb_k, op_fmt, c.data_ptr(), _out_code(c.dtype), N, M, N, K, flag.data_ptr(),
           epoch, C.stream_of(c))


def kmajor_operand(b: torch.Tensor) -> torch.Tensor:
    """B [K, N] -> the K-contiguous [N, K] operand the kernels read: B.T itself
    when it already is K-contiguous with 16-byte aligned rows, else a
    transposed copy made on the device (lsmx_transpose)."""
    K, N = b.shape
    bt = b.t()
    if bt.stride(-1) == 1 and bt.data_ptr() % 16 == 0 and (N <= 1 or (bt.stride(0) * bt.element_size()) % 16 == 0):
        return bt
    out = torch.empty((N, K), device=b.device, dtype=b.dtype)
    if K == 0 or N == 0:
        return out
    if b.stride(-1) != 1:
        b = b.contiguous()
    C.call("lsmx_transpose", b.data_ptr(), b.element_size(), K, N, b.stride(0) if K > 1 else N, out.data_ptr(), K,
           C.stream_of(out))
    return out


def mxfp4_gemm_fp8(a_fp8, b_fp8, a_scale, b_scale, out_dtype=torch.bfloat16):
    """a_fp8 [M,K] K-contig, b_fp8 [K,N] N-contig, a_scale [M,K//32], b_scale [K//32,N].

    Operands are E4M3 bytes (float8_e4m3fn or uint8 views of them), normally
    holding E2M1 values (fp4.codes_to_e4m3).  Scales are fp32 as
    fp4.quantize_mxfp4 returns, or E8M0 bytes of the same shapes.  Returns
    C[m, n] = sum_kb a_scale[m, kb] b_scale[kb, n] (A_kb . B_kb) in out_dtype:
    the E4M3 products run on the scaled MFMA (v_mfma_scale_f32_32x32x64_
    f8f6f4, E4M3 mode) with the block scales applied by the instruction and
    fp32 accumulation (reference: mxfp4_gemm.py:29-87).  fp32 scales that are
    not all powers of two are flagged by their conversion and C is then
    recomputed with the reference's promotion (lsmx_gemm_mx_promote,
    mxfp4_gemm.py:52-63).  An N-contiguous B (N % 16 == 0) is read in place
    by both kernels (lsmx_gemm_f8f8_nb, LSMX_B_NCONTIG); otherwise B is
    transposed to K-contiguous rows on the device first unless b_fp8 is a
    transposed view of such rows."""
    M, K = a_fp8.shape
    K2, N = b_fp8.shape
    assert K == K2 and K % 128 == 0, "K must be a multiple of 128 (max BLOCK_K)"
    assert a_scale.shape == (M, K // 32) and b_scale.shape == (K // 32, N)
    C.require_device(a_fp8, b_fp8, a_scale, b_scale)
    for t in (a_fp8, b_fp8):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8):
            raise TypeError(f"mxfp4_gemm_fp8 takes float8_e4m3fn operands, got {t.dtype}")
    c = torch.empty((M, N), device=a_fp8.device, dtype=out_dtype)
    if M == 0 or N == 0:
        return c
    if K == 0:
        return c.zero_()
    a = _rows16(a_fp8.view(torch.uint8))
    b8 = b_fp8.view(torch.uint8)
    # fp32 scales (the reference's form) or E8M0 bytes, either way as K-major
    # E8M0 for the persistent 256 x 256-tile kernel (csrc/gemm_f8f8.hip)
    promote = None
    if a_scale.dtype == torch.uint8 or b_scale.dtype == torch.uint8:
        sa = _e8m0_kmajor(a_scale, M, K // 32, transposed=False)
        sb = _e8m0_kmajor(b_scale, N, K // 32, transposed=True)
    else:
        exact = _fp4.e8m0_exact(a_scale, b_scale)
        sa32, sb32 = _f32_rows(a_scale), _f32_rows(b_scale)
        (sa, sb), flag, epoch = _e8m0_kmajor_flagged([(sa32, M, False), (sb32, N, True)], K // 32,
                                                     flagged=not exact)
        promote = None if exact else (sa32, False, sb32, True, flag, epoch)
    fmt, lsa, lsb = C.SCALE_E8M0_KMAJOR, M, N
    lda = a.stride(0) if M > 1 else K
    ldn = b8.stride(0) if K > 1 else N
    if N % 16 == 0 and b8.stride(1) == 1 and N <= ldn < 0x7FFFFFFF // 256 and ldn % 16 == 0 and \
            b8.data_ptr() % 16 == 0:
        # B as the reference passes it, [K, N] N-contiguous: both kernels
        # read it in place with transposing LDS loads (no transpose)
        C.call("lsmx_gemm_f8f8_nb", a.data_ptr(), lda, sa.data_ptr(), lsa, b8.data_ptr(), ldn, sb.data_ptr(), lsb,
               c.data_ptr(), _out_code(out_dtype), N, M, N, K, C.stream_of(c))
        if promote is not None:
            _promote(a, lda, b8, ldn, C.E4M3 | C.B_NCONTIG, c, K, *promote)
        return c
    bt = kmajor_operand(b8)
    ldb = bt.stride(0) if N > 1 else K
    C.call("lsmx_gemm_f8f8", a.data_ptr(), lda, sa.data_ptr(), lsa, bt.data_ptr(), ldb, sb.data_ptr(), lsb, fmt,
           c.data_ptr(), _out_code(out_dtype), N, M, N, K, C.stream_of(c))
    if promote is not None:
        _promote(a, lda, bt, ldb, C.E4M3, c, K, *promote)
    return c
