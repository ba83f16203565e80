"""FP4 (E2M1) / MXFP4 primitives on gfx950 -- drop-in for the reference's fp4.py.

Same names, signatures, return dtypes and shapes as fp4.py:20-125.  The
quantizer, packing, unpacking, dequantization and E4M3 expansion run as HIP
kernels in liblsmx.so on the tensor's GPU and on torch's current stream;
they refuse CPU tensors (there is no CPU fallback).  The test-data helpers
(random_codes, codes_to_q, blockwise_exact_dot) and the fp64 reference GEMM
are plain torch, like the reference's, and run wherever their inputs live.

Layout conventions (fp4.py:3-8):
    A      : [M, K]      K-contiguous
    B      : [K, N]      N-contiguous   (for the fp8 path,  C = A @ B)
    B_T    : [N, K]      K-contiguous   (for the packed path, C = A @ B_T.T)
    A scale: [M, K//32]
    B scale: [K//32, N]  (fp8 path)  or  [N, K//32]  (packed path)

Additions beyond fp4.py: quantize_pack_mxfp4 (fused quantize + pack with
E8M0 byte scales, the form the GEMMs consume), quantize_mxfp4_t (quantize
along the other axis), and the E8M0 <-> fp32 scale conversions.
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from . import _capi as C

# fp32 scale tensors this module returned -- powers of two in [2^-127, 2^127]
# or NaN by construction -- by id, with the version counter and address they
# had then.  mxfp4_gemm_packed and mxfp4_gemm_fp8 skip the promotion launch
# for scales still in that state (an in-place write to the tensor or to any
# view of it bumps the shared version counter); any other fp32 scales are
# checked on the device.  Writes that bypass the version counter -- through
# `tensor.data`, or from outside torch (DLPack, raw pointers) -- are not seen:
# after such a write, pass a copy (`s.clone()`), which takes the checked path.
_E8M0_EXACT: dict = {}


def _mark_e8m0_exact(s: torch.Tensor) -> torch.Tensor:
    # Views (reshape of a fresh tensor returns one) are tracked through the
    # tensor that owns the storage: every view of it points to that one.
    b = s._base if s._base is not None else s
    key = id(b)
    _E8M0_EXACT[key] = (b._version, b.data_ptr())
    weakref.finalize(b, _E8M0_EXACT.pop, key, None)
    return s


def e8m0_exact(*scales: torch.Tensor) -> bool:
    """True when every tensor is an fp32 scale tensor returned by
    quantize_mxfp4 or e8m0_to_scale, or a view of one, and neither has been
    written since (views share the version counter of their base)."""
    def known(s):
        b = s._base if s._base is not None else s
        return _E8M0_EXACT.get(id(b)) == (b._version, b.data_ptr())
    return all(known(s) for s in scales)

# ---------------------------------------------------------------- E2M1 tables
# fp4.py:20-34
_E2M1_MAG = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]          # code & 7 -> magnitude
FP4_MAX = 6.0
FP4_EMAX = 2                                                   # max exponent of E2M1

E2M1_VALUES = torch.tensor(_E2M1_MAG + [-v for v in _E2M1_MAG], dtype=torch.float32)

# code -> E4M3 byte: sign<<7 | (exp+6)<<3 | mant<<2, with 0 and 0.5 special.
E2M1_TO_E4M3 = torch.tensor(
    [0x00, 0x30, 0x38, 0x3C, 0x40, 0x44, 0x48, 0x4C,
     0x80, 0xB0, 0xB8, 0xBC, 0xC0, 0xC4, 0xC8, 0xCC], dtype=torch.uint8)

# code -> 2*value as a signed integer (the exact integer grid).
E2M1_Q = torch.tensor([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12],
                      dtype=torch.int32)


def random_codes(shape, device="cpu") -> torch.Tensor:
    """Uniform over the 15 distinct E2M1 codes (negative zero excluded). fp4.py:37-40"""
    pick = torch.tensor([c for c in range(16) if c != 8], device=device, dtype=torch.uint8)
    return pick[torch.randint(0, 15, shape, device=device)]


def _round_to_e2m1(q: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest onto the E2M1 grid; 4-bit codes as uint8 (fp4.py:43-54).

    Ties go to the smaller magnitude, |q| clips at 6, the sign bit is copied
    (so -0.0 gives code 8) and NaN gives magnitude 7."""
    C.require_device(q)
    if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        q = q.float()
    qc = q.contiguous()
    out = torch.empty(qc.shape, dtype=torch.uint8, device=q.device)
    C.call("lsmx_round_e2m1", qc.data_ptr(), C.dtype_code(qc.dtype), qc.numel(), out.data_ptr(),
           C.stream_of(qc))
    return out


def _as_rows(x: torch.Tensor):
    """x [..., K] -> (2-D row view with unit stride along K, leading shape)."""
    *lead, K = x.shape
    x2 = x.reshape(-1, K) if x.dim() != 2 else x
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < K) \
            or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2, lead


def _src(x: torch.Tensor) -> torch.Tensor:
    # fp4.py:63 converts to fp32 first; fp32, bf16 and fp16 widen exactly in
    # the kernel, anything else is widened here.
    return x if x.dtype in (torch.float32, torch.bfloat16, torch.float16) else x.float()


def quantize_mxfp4(x: torch.Tensor, block: int = 32):
    """MXFP4 quantize along the last dim (fp4.py:57-72).

    Returns (codes uint8 [..., K], scale fp32 [..., K//block]).
    Shared scale follows OCP MX: 2^(floor(log2(amax)) - emax_elem), emax_elem = 2,
    with log2 rounded to float32 as torch computes it."""
    *lead, K = x.shape
    assert K % block == 0, f"K={K} must be a multiple of block={block}"
    C.require_device(x)
    x = _src(x)
    x2, lead = _as_rows(x)
    rows = x2.shape[0]
    codes = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    scale = torch.empty((rows, K // block), dtype=torch.float32, device=x.device)
    if x2.numel():   # an empty tensor has no storage to pass (fp4.py returns empty outputs)
        C.call("lsmx_quantize_mxfp4", x2.data_ptr(), C.dtype_code(x2.dtype), rows, K,
               x2.stride(0) if rows > 1 else K, block, codes.data_ptr(), C.CODES_UNPACKED, K,
               scale.data_ptr(), C.SCALE_F32, K // block, C.stream_of(x2))
    return codes.reshape(*lead, K), _mark_e8m0_exact(scale.reshape(*lead, K // block))


def quantize_pack_mxfp4(x: torch.Tensor, block: int = 32, scale_layout: str = "rows"):
    """Fused quantize_mxfp4 + pack_fp4 with E8M0 byte scales.

    Returns (packed uint8 [..., K//2], e8m0 uint8); the bytes equal
    pack_fp4(codes) and the exponent fields of quantize_mxfp4's scales.
    scale_layout "rows": e8m0 is [..., K//block] (row-major, like fp4.py's
    scales).  "kmajor" (2-D x, block 32, K % 128 == 0): e8m0 is
    [K//128, rows, 4], the layout the f4 x f4 GEMM streams fastest."""
    *lead, K = x.shape
    assert K % block == 0, f"K={K} must be a multiple of block={block}"
    C.require_device(x)
    x = _src(x)
    x2, lead = _as_rows(x)
    rows = x2.shape[0]
    packed = torch.empty((rows, K // 2), dtype=torch.uint8, device=x.device)
    if scale_layout == "kmajor":
        assert block == 32 and K % 128 == 0, "K-major scales need block 32 and K % 128 == 0"
        e8m0 = torch.empty((K // 128, rows, 4), dtype=torch.uint8, device=x.device)
        fmt, ld = C.SCALE_E8M0_KMAJOR, rows
    elif scale_layout == "rows":
        e8m0 = torch.empty((rows, K // block), dtype=torch.uint8, device=x.device)
        fmt, ld = C.SCALE_E8M0, K // block
    else:
        raise ValueError(f"scale_layout must be 'rows' or 'kmajor', got {scale_layout!r}")
    if x2.numel():
        C.call("lsmx_quantize_mxfp4", x2.data_ptr(), C.dtype_code(x2.dtype), rows, K,
               x2.stride(0) if rows > 1 else K, block, packed.data_ptr(), C.CODES_PACKED, K // 2,
               e8m0.data_ptr(), fmt, ld, C.stream_of(x2))
    if scale_layout == "kmajor":
        return packed.reshape(*lead, K // 2), e8m0
    return packed.reshape(*lead, K // 2), e8m0.reshape(*lead, K // block)


def quantize_pack_mxfp4_many(xs, scale_layout: str = "rows"):
    """[quantize_pack_mxfp4(x, 32, scale_layout) for x in xs], bit for bit.
    fp32 / bf16 / fp16 tensors of one dtype go to the device in one launch per
    group of up to 8 (lsmx_quantize_mxfp4_batch): the two operands of a GEMM
    stream through one launch instead of two."""
    if scale_layout not in ("rows", "kmajor"):
        raise ValueError(f"scale_layout must be 'rows' or 'kmajor', got {scale_layout!r}")
    km = scale_layout == "kmajor"
    out = [None] * len(xs)
    groups = {}
    for i, x in enumerate(xs):
        C.require_device(x)
        K = x.shape[-1]
        assert K % 32 == 0, f"K={K} must be a multiple of block=32"
        if km:
            assert x.dim() == 2 and K % 128 == 0, "K-major scales need a 2-D x with K % 128 == 0"
        x2, lead = _as_rows(_src(x))
        rows = x2.shape[0]
        packed = torch.empty((rows, K // 2), dtype=torch.uint8, device=x.device)
        if km:
            e8m0 = torch.empty((K // 128, rows, 4), dtype=torch.uint8, device=x.device)
            ld = rows
            out[i] = (packed.reshape(*lead, K // 2), e8m0)
        else:
            e8m0 = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
            ld = K // 32
            out[i] = (packed.reshape(*lead, K // 2), e8m0.reshape(*lead, K // 32))
        if x2.numel():
            item = C.QItem(x2.data_ptr(), rows, K, x2.stride(0) if rows > 1 else K, packed.data_ptr(), K // 2,
                           e8m0.data_ptr(), ld)
            groups.setdefault((x2.dtype, x.device), []).append((item, x2))
    for (dt, _), its in groups.items():
        for g0 in range(0, len(its), 8):
            part = its[g0:g0 + 8]
            items = (C.QItem * len(part))(*[it for it, _ in part])
            C.call("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), len(part), C.dtype_code(dt),
                   C.SCALE_E8M0_KMAJOR if km else C.SCALE_E8M0, C.stream_of(part[0][1]))
    return out


def kmajor_scales(e8m0: torch.Tensor) -> torch.Tensor:
    """Row-major E8M0 scales [rows, K//32] -> K-major [K//128, rows, 4] (a copy)."""
    rows, nb = e8m0.shape
    assert nb % 4 == 0, "K must be a multiple of 128"
    return e8m0.reshape(rows, nb // 4, 4).transpose(0, 1).contiguous()


def quantize_mxfp4_t(x: torch.Tensor, block: int = 32, packed: bool = True, e8m0: bool = True,
                     scale_layout: str = "rows"):
    """Quantize a 2-D x [K, N] along its FIRST axis, without a transpose copy.

    Equals quantize_pack_mxfp4(x.t().contiguous(), scale_layout=...) (packed,
    e8m0) or quantize_mxfp4(x.t().contiguous()) (packed=False, e8m0=False):
    outputs are laid out for x^T, codes [N, K//2 or K] and scales
    [N, K//block] ("rows") or [K//128, N, 4] ("kmajor", E8M0 and block 32)."""
    C.require_device(x)
    x = _src(x)
    assert x.dim() == 2, "quantize_mxfp4_t takes a 2-D tensor"
    K, N = x.shape
    assert K % block == 0, f"K={K} must be a multiple of block={block}"
    if x.stride(1) != 1 or (K > 1 and x.stride(0) < N):
        x = x.contiguous()
    codes = torch.empty((N, K // 2 if packed else K), dtype=torch.uint8, device=x.device)
    if scale_layout == "kmajor":
        assert e8m0 and block == 32 and K % 128 == 0, \
            "K-major scales need E8M0, block 32 and K % 128 == 0"
        scale = torch.empty((K // 128, N, 4), dtype=torch.uint8, device=x.device)
        fmt, ld = C.SCALE_E8M0_KMAJOR, N
    elif scale_layout == "rows":
        scale = torch.empty((N, K // block), dtype=torch.uint8 if e8m0 else torch.float32,
                            device=x.device)
        fmt, ld = (C.SCALE_E8M0 if e8m0 else C.SCALE_F32), K // block
    else:
        raise ValueError(f"scale_layout must be 'rows' or 'kmajor', got {scale_layout!r}")
    C.call("lsmx_quantize_mxfp4_t", x.data_ptr(), C.dtype_code(x.dtype), K, N,
           x.stride(0) if K > 1 else N, block, codes.data_ptr(),
           C.CODES_PACKED if packed else C.CODES_UNPACKED, codes.shape[1], scale.data_ptr(),
           fmt, ld, C.stream_of(x))
    return codes, scale


def quantize_pack_mxfp4_2d(x: torch.Tensor, scale_layout: str = "kmajor"):
    """Both MXFP4 forms of a 2-D x [R, C] from one read of x:

        (row_packed, row_scale) == quantize_pack_mxfp4(x, scale_layout=...)
        (col_packed, col_scale) == quantize_mxfp4_t(x, scale_layout=...)

    i.e. x quantized along its rows (blocks of 32 columns) and along its
    columns (blocks of 32 rows, laid out for x^T), E8M0 scales.  bf16 / fp16
    x with R and C multiples of 128 run the fused one-pass kernel
    (lsmx_quantize_mxfp4_2d); other inputs run the two quantizers."""
    C.require_device(x)
    assert x.dim() == 2, "quantize_pack_mxfp4_2d takes a 2-D tensor"
    R, Cn = x.shape
    if scale_layout not in ("rows", "kmajor"):
        raise ValueError(f"scale_layout must be 'rows' or 'kmajor', got {scale_layout!r}")
    if x.dtype not in (torch.bfloat16, torch.float16) or R % 128 or Cn % 128:
        rp, rs = quantize_pack_mxfp4(x, scale_layout=scale_layout)
        cp, cs = quantize_mxfp4_t(x, scale_layout=scale_layout)
        return rp, rs, cp, cs
    if x.stride(1) != 1 or (R > 1 and x.stride(0) < Cn) or x.data_ptr() % 16 or (x.stride(0) * 2) % 16:
        x = x.contiguous()
    rp = torch.empty((R, Cn // 2), dtype=torch.uint8, device=x.device)
    cp = torch.empty((Cn, R // 2), dtype=torch.uint8, device=x.device)
    if scale_layout == "kmajor":
        rs = torch.empty((Cn // 128, R, 4), dtype=torch.uint8, device=x.device)
        cs = torch.empty((R // 128, Cn, 4), dtype=torch.uint8, device=x.device)
        fmt, lsr, lsc = C.SCALE_E8M0_KMAJOR, R, Cn
    else:
        rs = torch.empty((R, Cn // 32), dtype=torch.uint8, device=x.device)
        cs = torch.empty((Cn, R // 32), dtype=torch.uint8, device=x.device)
        fmt, lsr, lsc = C.SCALE_E8M0, Cn // 32, R // 32
    if R and Cn:
        C.call("lsmx_quantize_mxfp4_2d", x.data_ptr(), C.dtype_code(x.dtype), R, Cn, x.stride(0) if R > 1 else Cn,
               rp.data_ptr(), Cn // 2, rs.data_ptr(), lsr, cp.data_ptr(), R // 2, cs.data_ptr(), lsc, fmt,
               C.stream_of(x))
    return rp, rs, cp, cs


def quantize_pack_mxfp4_2d_many(xs, scale_layout: str = "kmajor"):
    """[quantize_pack_mxfp4_2d(x, scale_layout) for x in xs], bit for bit.
    bf16 / fp16 tensors of one dtype with both sizes multiples of 128 go to
    the device in one launch per group of up to 8 (lsmx_quantize_mxfp4_2d_batch);
    any other tensor takes quantize_pack_mxfp4_2d on its own."""
    if scale_layout not in ("rows", "kmajor"):
        raise ValueError(f"scale_layout must be 'rows' or 'kmajor', got {scale_layout!r}")
    out = [None] * len(xs)
    groups = {}
    for i, x in enumerate(xs):
        C.require_device(x)
        assert x.dim() == 2, "quantize_pack_mxfp4_2d takes 2-D tensors"
        R, Cn = x.shape
        if x.dtype in (torch.bfloat16, torch.float16) and R % 128 == 0 and Cn % 128 == 0:
            groups.setdefault((x.dtype, x.device), []).append(i)
        else:
            out[i] = quantize_pack_mxfp4_2d(x, scale_layout=scale_layout)
    km = scale_layout == "kmajor"
    for (dt, dev), idx in groups.items():
        for g0 in range(0, len(idx), 8):
            part = idx[g0:g0 + 8]
            items = (C.Q2dItem * len(part))()
            keep = []
            for slot, i in enumerate(part):
                x = xs[i]
                R, Cn = x.shape
                if x.stride(1) != 1 or (R > 1 and x.stride(0) < Cn) or x.data_ptr() % 16 or (x.stride(0) * 2) % 16:
                    x = x.contiguous()
                rp = torch.empty((R, Cn // 2), dtype=torch.uint8, device=dev)
                cp = torch.empty((Cn, R // 2), dtype=torch.uint8, device=dev)
                if km:
                    rs = torch.empty((Cn // 128, R, 4), dtype=torch.uint8, device=dev)
                    cs = torch.empty((R // 128, Cn, 4), dtype=torch.uint8, device=dev)
                    lsr, lsc = R, Cn
                else:
                    rs = torch.empty((R, Cn // 32), dtype=torch.uint8, device=dev)
                    cs = torch.empty((Cn, R // 32), dtype=torch.uint8, device=dev)
                    lsr, lsc = Cn // 32, R // 32
                items[slot] = C.Q2dItem(x.data_ptr(), R, Cn, x.stride(0) if R > 1 else Cn, rp.data_ptr(), Cn // 2,
                                        rs.data_ptr(), lsr, cp.data_ptr(), R // 2, cs.data_ptr(), lsc)
                keep.append(x)
                out[i] = (rp, rs, cp, cs)
            C.call("lsmx_quantize_mxfp4_2d_batch", ctypes.addressof(items), len(part), C.dtype_code(dt),
                   C.SCALE_E8M0_KMAJOR if km else C.SCALE_E8M0, C.stream_of(keep[0]))
    return out


def e8m0_to_scale(e8m0: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes -> fp32 powers of two 2^(e - 127) (0xFF -> NaN; byte 0 ->
    2^-127, the fp32 subnormal 0x00400000).  Exact."""
    e = e8m0.to(torch.int32)
    s = torch.where(e == 0, torch.full_like(e, 0x00400000), e << 23).view(torch.float32)
    return _mark_e8m0_exact(torch.where(e8m0 == 255, torch.full_like(s, float("nan")), s))


def scale_to_e8m0(scale: torch.Tensor) -> torch.Tensor:
    """fp32 powers of two in [2^-127, 2^127] -> E8M0 bytes (the biased
    exponent; 2^-127 -> 0).  Exact inverse of e8m0_to_scale.  A scale with no
    E8M0 form (NaN, not a positive power of two) -> 0xFF (NaN), as the GEMMs
    treat it."""
    b = scale.contiguous().view(torch.int32)
    ex = (b >> 23) & 0x1FF                          # sign in bit 8: negatives fail
    pow2 = ((b & 0x7FFFFF) == 0) & (ex >= 1) & (ex <= 254)
    sub = b == 0x00400000
    e = torch.where(pow2, ex, torch.where(sub, torch.zeros_like(ex), torch.full_like(ex, 255)))
    return e.to(torch.uint8)


def _scale_fmt(scale: torch.Tensor) -> int:
    if scale.dtype == torch.float32:
        return C.SCALE_F32
    if scale.dtype == torch.uint8:
        return C.SCALE_E8M0
    raise TypeError(f"scale must be float32 (powers of two) or uint8 (E8M0), got {scale.dtype}")


def dequantize_mxfp4(codes: torch.Tensor, scale: torch.Tensor, block: int = 32):
    """fp32 values = E2M1_VALUES[codes] * scale, per block (fp4.py:75-78).

    `scale` may be fp32 (as quantize_mxfp4 returns) or E8M0 bytes."""
    C.require_device(codes, scale)
    *lead, K = codes.shape
    c2 = codes.reshape(-1, K).contiguous()
    s2 = scale.reshape(-1, K // block).contiguous()
    out = torch.empty(c2.shape, dtype=torch.float32, device=codes.device)
    C.call("lsmx_dequantize_mxfp4", c2.data_ptr(), C.CODES_UNPACKED, K, s2.data_ptr(),
           _scale_fmt(s2), K // block, c2.shape[0], K, block, out.data_ptr(), C.F32, K,
           C.stream_of(c2))
    return out.reshape(*lead, K)


def dequantize_packed(packed: torch.Tensor, scale: torch.Tensor, block: int = 32,
                      out_dtype: torch.dtype = torch.float32):
    """Packed nibbles [..., K//2] + scales -> values [..., K] in fp32 or bf16 (exact)."""
    C.require_device(packed, scale)
    *lead, Kh = packed.shape
    K = 2 * Kh
    p2 = packed.reshape(-1, Kh).contiguous()
    s2 = scale.reshape(-1, K // block).contiguous()
    out = torch.empty((p2.shape[0], K), dtype=out_dtype, device=packed.device)
    C.call("lsmx_dequantize_mxfp4", p2.data_ptr(), C.CODES_PACKED, Kh, s2.data_ptr(),
           _scale_fmt(s2), K // block, p2.shape[0], K, block, out.data_ptr(), C.dtype_code(out_dtype),
           K, C.stream_of(p2))
    return out.reshape(*lead, K)


def codes_to_e4m3(codes: torch.Tensor) -> torch.Tensor:
    """Lossless FP4 -> FP8(E4M3) cast via table lookup (fp4.py:81-83)."""
    C.require_device(codes)
    shape = codes.shape
    flat = codes.reshape(-1)
    n = flat.numel()
    pad = (-n) % 16
    if pad:
        flat = torch.cat([flat, torch.zeros(pad, dtype=torch.uint8, device=codes.device)])
    words = pack_fp4(flat.contiguous()).view(torch.int32)          # 8 codes per word
    out = torch.empty(words.numel() * 2, dtype=torch.int32, device=codes.device)
    C.call("lsmx_fp4_to_e4m3", words.data_ptr(), out.data_ptr(), words.numel(), C.stream_of(words))
    return out.view(torch.uint8)[:n].reshape(shape).view(torch.float8_e4m3fn)


def fp4_to_e4m3_words(words: torch.Tensor) -> torch.Tensor:
    """cuda/fp4_unpack.cuh:52-55 on a tensor of uint32 words (int32 storage):
    each word of 8 packed codes -> 2 words of E4M3 bytes."""
    C.require_device(words)
    w = words.contiguous()
    out = torch.empty(w.numel() * 2, dtype=torch.int32, device=w.device)
    C.call("lsmx_fp4_to_e4m3", w.data_ptr(), out.data_ptr(), w.numel(), C.stream_of(w))
    return out


def codes_to_q(codes: torch.Tensor) -> torch.Tensor:
    """FP4 code -> 2*value as int32 (the exact integer grid). fp4.py:86-88"""
    return E2M1_Q.to(codes.device)[codes.long()]


def pack_fp4(codes: torch.Tensor) -> torch.Tensor:
    """[..., K] uint8 codes -> [..., K//2] bytes; even index in the low nibble (fp4.py:91-94)."""
    assert codes.shape[-1] % 2 == 0
    C.require_device(codes)
    c = codes.contiguous()
    if c.data_ptr() % 16:
        c = c.clone()
    out = torch.empty((*c.shape[:-1], c.shape[-1] // 2), dtype=torch.uint8, device=c.device)
    C.call("lsmx_pack_fp4", c.data_ptr(), out.data_ptr(), out.numel(), C.stream_of(c))
    return out


def unpack_fp4(packed: torch.Tensor) -> torch.Tensor:
    """[..., K//2] bytes -> [..., K] codes (fp4.py:97-99)."""
    C.require_device(packed)
    p = packed.contiguous()
    if p.data_ptr() % 8:
        p = p.clone()
    out = torch.empty((*p.shape[:-1], p.shape[-1] * 2), dtype=torch.uint8, device=p.device)
    C.call("lsmx_unpack_fp4", p.data_ptr(), out.data_ptr(), p.numel(), C.stream_of(p))
    return out


# ------------------------------------------------------------------ references
def reference_mxfp4_gemm(a_codes, a_scale, b_codes, b_scale, block=32):
    """float64 reference for C = A @ B with A [M,K], B [K,N] (fp4.py:103-112).

    b_codes is [K, N] and b_scale is [K//block, N], so B is quantized along K.
    A test helper: plain torch in float64, on whatever device its inputs
    live (CPU included), independent of the HIP kernels it checks."""
    M, Ka = a_codes.shape
    Av = E2M1_VALUES.to(a_codes.device)[a_codes.long()].double()            # [M,K]
    A = (Av.reshape(M, Ka // block, block) * a_scale.double().unsqueeze(-1)).reshape(M, Ka)
    Bv = E2M1_VALUES.to(b_codes.device)[b_codes.long()].double()            # [K,N]
    K, N = Bv.shape
    B = (Bv.reshape(K // block, block, N) * b_scale.double().unsqueeze(1)).reshape(K, N)
    return (A @ B).float()


def blockwise_exact_dot(qa: torch.Tensor, qb: torch.Tensor, block: int = 32):
    """Exact integer dot products per block from the int grid (fp4.py:115-125).

    Returns int64 [.., K//block] of sum(qa*qb) per block; |sum| <= 144*block."""
    p = (qa.long() * qb.long())
    *lead, K = p.shape
    return p.reshape(*lead, K // block, block).sum(-1)
