"""CPU oracle for lockstep's MXFP4 path -- TEST INFRASTRUCTURE ONLY.

Python face of oracle/mxfp4_oracle.c (a C restatement of the reference's
fp4.py) plus the fp64 reference GEMMs of fp4.py:103-112.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker: the product package (lockstep_amd) never
imports it and has no CPU fallback.

Parity pins, per function (all in tests/test_oracle.py unless noted):
  round_e2m1      closed form (midpoint count), the reference's tie test
                  (tests/test_fp4.py:48-51), brute force over all 65536 bf16
                  bit patterns against torch.bucketize/abs/clamp/signbit
                  (library routines), golden fixtures from fp4.py
  e8m0 exponent   libm rule vs integer rule for every binade +-64 ulps and
                  random draws; libm rule vs torch.log2 (float32, the library
                  routine fp4.py:68 calls) on the same candidates; golden
                  fixtures from fp4.py
  quantize        the reference's property tests (tests/test_fp4.py:54-74),
                  golden fixtures (SHA-256 of codes and scales) from fp4.py
  pack/unpack     tests/test_fp4.py:34-39 and the closed form
  dequantize      closed form (exact power-of-two multiply), test_fp4.py:85-92
  e4m3 expansion  the reference's own C (oracle/_ref, built from
                  cuda/fp4_unpack.cuh) exhaustively over 16^4 nibble quads,
                  plus the 0xFEDCBA98 known answer of cuda/test_unpack.c:94
  reference_gemm  integer-grid exact products (bench.py:44-57) and brute
                  force over K on tiny shapes
  gemm_promote    power-of-two scales on the integer grid against the exact
                  fp64 product; one and two blocks with any scales against
                  numpy's float32 products and a single rounding of the exact
                  fp64 sum (which pins the fma of the update: the unfused
                  form is shown to differ); IEEE special scales (0, -2, inf,
                  NaN) on one block; random scales against fp64 within the
                  summation bound
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"

E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
E2M1_VALUES = np.concatenate([E2M1_MAG, -E2M1_MAG]).astype(np.float32)
E2M1_TO_E4M3 = np.array([0x00, 0x30, 0x38, 0x3C, 0x40, 0x44, 0x48, 0x4C,
                         0x80, 0xB0, 0xB8, 0xBC, 0xC0, 0xC4, 0xC8, 0xCC], dtype=np.uint8)
E2M1_Q = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], dtype=np.int32)

DTYPES = {"f32": 0, "bf16": 1, "f16": 2}

_lib = None


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    if Path("/root/reference/cuda/fp4_unpack.cuh").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        c_u8p = ctypes.POINTER(ctypes.c_uint8)
        L.orc_round_e2m1.restype = ctypes.c_uint8
        L.orc_round_e2m1.argtypes = [ctypes.c_float]
        L.orc_e8m0_exp_log2.restype = ctypes.c_int
        L.orc_e8m0_exp_log2.argtypes = [ctypes.c_float]
        L.orc_e8m0_exp_int.restype = ctypes.c_int
        L.orc_e8m0_exp_int.argtypes = [ctypes.c_float]
        L.orc_e8m0_window.restype = ctypes.c_int
        L.orc_e8m0_window.argtypes = [ctypes.c_int]
        L.orc_quantize.restype = ctypes.c_int
        L.orc_quantize.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_int64, ctypes.c_int, c_u8p,
                                   ctypes.POINTER(ctypes.c_float), ctypes.c_int]
        L.orc_pack_fp4.argtypes = [c_u8p, ctypes.c_int64, c_u8p]
        L.orc_unpack_fp4.argtypes = [c_u8p, ctypes.c_int64, c_u8p]
        L.orc_dequantize.argtypes = [c_u8p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
        L.orc_dequantize_packed_e8m0_f64.argtypes = [c_u8p, c_u8p, ctypes.c_int64, ctypes.c_int64,
                                                     ctypes.POINTER(ctypes.c_double)]
        L.orc_fp4x8_to_e4m3x8.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int64,
                                          ctypes.POINTER(ctypes.c_uint32),
                                          ctypes.POINTER(ctypes.c_uint32)]
        c_fp = ctypes.POINTER(ctypes.c_float)
        L.orc_gemm_promote.argtypes = [c_fp, c_fp, c_fp, ctypes.c_int64, ctypes.c_int64, c_fp, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_fp]
        L.orc_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def num_threads() -> int:
    return lib().orc_num_threads()


# ------------------------------------------------------------- scalar rules
def round_e2m1(q: float) -> int:
    """fp4.py:43-54 on one fp32 value."""
    return int(lib().orc_round_e2m1(float(np.float32(q))))


def e8m0_exp_log2(amax: float) -> int:
    """fp4.py:68 exponent via float32-rounded log2."""
    return int(lib().orc_e8m0_exp_log2(float(np.float32(amax))))


def e8m0_exp_int(amax: float) -> int:
    """fp4.py:68 exponent via the integer threshold rule (the GPU's rule)."""
    return int(lib().orc_e8m0_exp_int(float(np.float32(amax))))


def e8m0_window(k: int) -> int:
    return int(lib().orc_e8m0_window(int(k)))


# ----------------------------------------------------------------- quantize
def quantize_mxfp4(x: np.ndarray, block: int = 32, dtype: str | None = None, rule: str = "int"):
    """fp4.py:57-72 along the last axis.

    x: float32 array, or uint16 bit patterns with dtype "bf16"/"f16".
    Returns (codes uint8 [..., K], scale float32 [..., K/block])."""
    if dtype is None:
        dtype = "f32"
        x = np.ascontiguousarray(x, dtype=np.float32)
    else:
        x = np.ascontiguousarray(x, dtype=np.uint16)
    *lead, K = x.shape
    assert K % block == 0, f"K={K} must be a multiple of block={block}"
    rows = int(np.prod(lead)) if lead else 1
    codes = np.empty((rows, K), dtype=np.uint8)
    scale = np.empty((rows, K // block), dtype=np.float32)
    rc = lib().orc_quantize(x.ctypes.data, DTYPES[dtype], rows, K, K, block,
                            _p(codes, ctypes.c_uint8), _p(scale, ctypes.c_float),
                            1 if rule == "int" else 0)
    assert rc == 0
    return codes.reshape(*lead, K), scale.reshape(*lead, K // block)


def scale_to_e8m0(scale: np.ndarray) -> np.ndarray:
    """fp32 power-of-two scales -> E8M0 bytes (the fp32 exponent field;
    NaN -> 0xFF)."""
    s = np.ascontiguousarray(scale, dtype=np.float32)
    out = ((s.view(np.uint32) >> 23) & 0xFF).astype(np.uint8)
    out[np.isnan(s)] = 0xFF
    return out


def e8m0_to_scale(e: np.ndarray) -> np.ndarray:
    """E8M0 bytes -> fp32 2^(e-127): byte 0 is 2^-127 (a subnormal), 0xFF NaN."""
    e = np.asarray(e, dtype=np.uint8)
    out = (e.astype(np.uint32) << 23).view(np.float32).copy()
    out[e == 0] = np.float32(2.0 ** -127)
    out[e == 0xFF] = np.nan
    return out


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    """fp4.py:91-94."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    assert c.shape[-1] % 2 == 0
    out = np.empty((*c.shape[:-1], c.shape[-1] // 2), dtype=np.uint8)
    lib().orc_pack_fp4(_p(c, ctypes.c_uint8), out.size, _p(out, ctypes.c_uint8))
    return out


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    """fp4.py:97-99."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty((*p.shape[:-1], p.shape[-1] * 2), dtype=np.uint8)
    lib().orc_unpack_fp4(_p(p, ctypes.c_uint8), p.size, _p(out, ctypes.c_uint8))
    return out


def quantize_pack(x: np.ndarray, dtype: str | None = None):
    """Fused form the GPU quantizer produces: (packed [...,K/2], e8m0 [...,K/32])."""
    codes, scale = quantize_mxfp4(x, 32, dtype)
    return pack_fp4(codes), scale_to_e8m0(scale)


def dequantize_mxfp4(codes: np.ndarray, scale: np.ndarray, block: int = 32) -> np.ndarray:
    """fp4.py:75-78 (fp32, exact)."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(scale, dtype=np.float32)
    *lead, K = c.shape
    rows = c.size // K
    out = np.empty(c.shape, dtype=np.float32)
    lib().orc_dequantize(_p(c, ctypes.c_uint8), _p(s, ctypes.c_float), rows, K, block,
                         _p(out, ctypes.c_float))
    return out


def dequantize_packed(packed: np.ndarray, e8m0: np.ndarray) -> np.ndarray:
    """Packed nibbles + E8M0 bytes -> fp64 values [rows, K]."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    e = np.ascontiguousarray(e8m0, dtype=np.uint8)
    rows, kh = p.shape
    out = np.empty((rows, 2 * kh), dtype=np.float64)
    lib().orc_dequantize_packed_e8m0_f64(_p(p, ctypes.c_uint8), _p(e, ctypes.c_uint8), rows,
                                         2 * kh, _p(out, ctypes.c_double))
    return out


def fp4x8_to_e4m3x8(words: np.ndarray):
    """cuda/fp4_unpack.cuh:52-55 semantics: uint32 of 8 codes -> (lo, hi) uint32."""
    w = np.ascontiguousarray(words, dtype=np.uint32)
    lo = np.empty_like(w)
    hi = np.empty_like(w)
    lib().orc_fp4x8_to_e4m3x8(_p(w, ctypes.c_uint32), w.size, _p(lo, ctypes.c_uint32),
                              _p(hi, ctypes.c_uint32))
    return lo, hi


# ------------------------------------------------------------ reference GEMMs
def reference_gemm_packed(a_pk, a_e8m0, bt_pk, bt_e8m0, rows=None, cols=None) -> np.ndarray:
    """fp4.py:103-112 in the packed "TN" layout of mxfp4_gemm.py:161-174:
    C[m, n] = sum_k deq(A)[m, k] * deq(Bt)[n, k] in fp64.  Optional row and
    column index subsets give a sampled check at full size."""
    if rows is not None:
        a_pk, a_e8m0 = a_pk[rows], a_e8m0[rows]
    if cols is not None:
        bt_pk, bt_e8m0 = bt_pk[cols], bt_e8m0[cols]
    A = dequantize_packed(a_pk, a_e8m0)
    B = dequantize_packed(bt_pk, bt_e8m0)
    return A @ B.T


def reference_gemm_wonly(a: np.ndarray, w_pk, w_e8m0, rows=None, cols=None) -> np.ndarray:
    """Weight-only form (fp4_linear.py:40 with an unquantized activation):
    C = A . deq(W)^T in fp64; `a` is a float array (bf16 values widened)."""
    if rows is not None:
        a = a[rows]
    if cols is not None:
        w_pk, w_e8m0 = w_pk[cols], w_e8m0[cols]
    W = dequantize_packed(w_pk, w_e8m0)
    return np.asarray(a, dtype=np.float64) @ W.T


def gemm_promote(a_vals: np.ndarray, bt_vals: np.ndarray, sa: np.ndarray, sb: np.ndarray,
                 sb_transposed: bool = False) -> np.ndarray:
    """mxfp4_gemm.py:52-63 / 141-150 for fp32 scales of any value:
    acc = fma(p_kb, sa[m,kb] * sb[n,kb], acc) over the 32-blocks in order
    (orc_gemm_promote).  a_vals [M, K] and bt_vals [N, K] are operand values
    (E2M1 or E4M3, as float); sa [M, K/32]; sb [N, K/32], or [K/32, N] when
    sb_transposed (mxfp4_gemm_fp8's b_scale).  Returns fp32 [M, N]."""
    A = np.ascontiguousarray(a_vals, dtype=np.float32)
    B = np.ascontiguousarray(bt_vals, dtype=np.float32)
    sa = np.ascontiguousarray(sa, dtype=np.float32)
    sb = np.ascontiguousarray(sb, dtype=np.float32)
    M, K = A.shape
    N = B.shape[0]
    assert B.shape[1] == K and K % 32 == 0 and sa.shape == (M, K // 32)
    assert sb.shape == ((K // 32, N) if sb_transposed else (N, K // 32))
    sb_r, sb_k = (1, N) if sb_transposed else (K // 32, 1)
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_promote(_p(A, ctypes.c_float), _p(B, ctypes.c_float), _p(sa, ctypes.c_float), K // 32, 1,
                           _p(sb, ctypes.c_float), sb_r, sb_k, M, N, K, _p(out, ctypes.c_float))
    return out


def fp4_values(packed: np.ndarray) -> np.ndarray:
    """Packed E2M1 bytes [rows, K/2] -> float values [rows, K] (fp4.py:20-24)."""
    return E2M1_VALUES[unpack_fp4(packed)]


def max_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """bench.py:71 metric: max|got - ref| / max|ref|."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (den if den > 0 else 1.0))


# ------------------------------------------------- the reference's own C code
def ref_unpack_lib():
    """oracle/_ref/libref_unpack.so (cuda/fp4_unpack.cuh built from the
    reference sources), or None where the reference is not mounted and the
    library was not built."""
    path = REF_DIR / "libref_unpack.so"
    if not path.exists():
        return None
    L = ctypes.CDLL(str(path))
    L.ref_fp4x4_to_e4m3x4.restype = ctypes.c_uint32
    L.ref_fp4x4_to_e4m3x4.argtypes = [ctypes.c_uint32]
    L.ref_fp4_code_to_e4m3.restype = ctypes.c_uint8
    L.ref_fp4_code_to_e4m3.argtypes = [ctypes.c_uint8]
    return L


if os.environ.get("LSMX_ORACLE_BUILD") == "1":      # pragma: no cover
    build()
