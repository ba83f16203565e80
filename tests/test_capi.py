"""CPU tests of the C ABI: the library loads, exports every entry point the
header declares, and rejects bad arguments before touching a device.  No
compute call runs here (no GPU in this process)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from lockstep_amd import _capi as C

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lsmx.h"


def declared_symbols():
    src = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(lsmx_\w+)\s*\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    lib = C.load()
    names = declared_symbols()
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(C.SIGNATURES), "ctypes table and header disagree"


def test_header_constants_match_binding():
    src = HEADER.read_text()
    consts = dict((k, int(v)) for k, v in re.findall(r"#define (LSMX_\w+) (-?\d+)", src))
    assert consts["LSMX_OK"] == C.OK
    assert consts["LSMX_ERR_SHAPE"] == C.ERR_SHAPE and consts["LSMX_ERR_ALIGN"] == C.ERR_ALIGN
    assert consts["LSMX_ERR_DTYPE"] == C.ERR_DTYPE and consts["LSMX_ERR_DEVICE"] == C.ERR_DEVICE
    assert consts["LSMX_F32"] == C.F32 and consts["LSMX_BF16"] == C.BF16 and consts["LSMX_F16"] == C.F16
    assert consts["LSMX_CODES_PACKED"] == C.CODES_PACKED and consts["LSMX_SCALE_F32"] == C.SCALE_F32
    assert int(re.search(r"#define LSMX_B_NCONTIG (0x[0-9a-fA-F]+)", src).group(1), 16) == C.B_NCONTIG


def test_version_string():
    assert C.version().startswith("lsmx ") and "gfx950" in C.version()


def _rc(name, *args):
    return getattr(C.load(), name)(*args)


FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first


def test_null_pointer_is_rejected():
    assert _rc("lsmx_quantize_mxfp4", None, 0, 4, 64, 64, 32, FAKE, 0, 32, FAKE, 0, 2, None) == C.ERR_ARG
    assert "null" in C.last_error()


def test_block_multiple_is_rejected_with_reference_message():
    rc = _rc("lsmx_quantize_mxfp4", FAKE, 0, 4, 48, 48, 32, FAKE, 0, 24, FAKE, 0, 2, None)
    assert rc == C.ERR_SHAPE
    assert "K=48 must be a multiple of block=32" in C.last_error()   # fp4.py:65


def test_gemm_k_multiple_is_rejected_with_reference_message():
    rc = _rc("lsmx_gemm_f4f4", FAKE, 48, FAKE, 3, FAKE, 48, FAKE, 3, 0, FAKE, 1, 8, 8, 8, 96, None)
    assert rc == C.ERR_SHAPE
    assert "K must be a multiple of 128" in C.last_error()          # mxfp4_gemm.py:166


def test_bad_dtype_and_alignment_are_rejected():
    assert _rc("lsmx_quantize_mxfp4", FAKE, 7, 4, 64, 64, 32, FAKE, 0, 32, FAKE, 0, 2, None) == C.ERR_DTYPE
    misaligned = ctypes.c_void_p(0x1004)
    rc = _rc("lsmx_quantize_mxfp4", misaligned, 0, 4, 64, 64, 32, FAKE, 0, 32, FAKE, 0, 2, None)
    assert rc == C.ERR_ALIGN
    rc = _rc("lsmx_gemm_f4f4", FAKE, 64, FAKE, 4, FAKE, 64, FAKE, 4, 0, FAKE, 9, 8, 8, 8, 128, None)
    assert rc == C.ERR_DTYPE


def test_batched_quantizer_and_quantizing_gemm_validate_before_launch():
    """lsmx_quantize_mxfp4_2d_batch checks every item as lsmx_quantize_mxfp4_2d
    does, and at most 8 items; lsmx_gemm_f4f4_quant takes whole 256 x 256
    tiles and 256-deep K only."""
    assert _rc("lsmx_quantize_mxfp4_2d_batch", None, 1, C.BF16, C.SCALE_E8M0_KMAJOR, None) == C.ERR_ARG
    items = (C.Q2dItem * 9)()
    assert _rc("lsmx_quantize_mxfp4_2d_batch", ctypes.addressof(items), 9, C.BF16, C.SCALE_E8M0_KMAJOR,
               None) == C.ERR_SHAPE
    f = 0x1000
    items[0] = C.Q2dItem(f, 100, 128, 128, f, 64, f, 100, f, 64, f, 128)
    assert _rc("lsmx_quantize_mxfp4_2d_batch", ctypes.addressof(items), 1, C.BF16, C.SCALE_E8M0_KMAJOR,
               None) == C.ERR_SHAPE
    assert "multiples of 128" in C.last_error()
    items[0] = C.Q2dItem(f, 128, 128, 128, f, 64, f, 128, f, 64, f, 128)
    assert _rc("lsmx_quantize_mxfp4_2d_batch", ctypes.addressof(items), 1, C.F32, C.SCALE_E8M0_KMAJOR,
               None) == C.ERR_DTYPE
    q = lambda M, N, K: _rc("lsmx_gemm_f4f4_quant", FAKE, K // 2, FAKE, M, FAKE, K // 2, FAKE, N, None, N,  # noqa: E731
                            FAKE, N // 2, FAKE, M, FAKE, M // 2, FAKE, N, M, N, K, None)
    assert q(384, 256, 256) == C.ERR_SHAPE and "multiples of 256" in C.last_error()
    assert q(256, 256, 128) == C.ERR_SHAPE
    assert _rc("lsmx_gemm_f4f4_quant", None, 128, FAKE, 256, FAKE, 128, FAKE, 256, None, 256, FAKE, 128, FAKE,
               256, FAKE, 128, FAKE, 256, 256, 256, 256, None) == C.ERR_ARG


def test_row_quantizer_batch_validates_before_launch():
    """lsmx_quantize_mxfp4_batch takes 0 .. 8 items, E8M0 scales only, and
    checks each item as lsmx_quantize_mxfp4 does (block 32, packed codes)."""
    f = 0x1000
    items = (C.QItem * 9)()
    assert _rc("lsmx_quantize_mxfp4_batch", None, 1, C.F32, C.SCALE_E8M0, None) == C.ERR_ARG
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 9, C.F32, C.SCALE_E8M0, None) == C.ERR_SHAPE
    items[0] = C.QItem(f, 4, 64, 64, f, 32, f, 2)
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 1, C.F32, C.SCALE_F32, None) == C.ERR_DTYPE
    items[1] = C.QItem(f, 4, 48, 48, f, 24, f, 2)                 # K % 32 != 0
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 2, C.F32, C.SCALE_E8M0, None) == C.ERR_SHAPE
    items[1] = C.QItem(f + 4, 4, 64, 64, f, 32, f, 2)             # x rows not 16-byte aligned
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 2, C.F32, C.SCALE_E8M0, None) == C.ERR_ALIGN
    items[1] = C.QItem(f, 4, 64, 64, f, 32, f, 2)                 # K-major needs K % 128 == 0
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 2, C.F32, C.SCALE_E8M0_KMAJOR,
               None) == C.ERR_SHAPE
    items[1] = C.QItem(None, 4, 64, 64, f, 32, f, 2)
    assert _rc("lsmx_quantize_mxfp4_batch", ctypes.addressof(items), 2, C.F32, C.SCALE_E8M0, None) == C.ERR_ARG


def test_promotion_entry_points_validate_before_launch():
    """lsmx_scale_to_e8m0_batch takes 0 .. 4 items with K-major output and an
    8-byte aligned flag; lsmx_gemm_mx_promote takes packed FP4 or E4M3
    operands with 16-byte aligned rows and keeps every load offset in 32
    bits."""
    items = (C.E8m0Item * 5)()
    assert _rc("lsmx_scale_to_e8m0_batch", ctypes.addressof(items), 5, None, 0, None) == C.ERR_SHAPE
    assert _rc("lsmx_scale_to_e8m0_batch", None, 1, None, 0, None) == C.ERR_ARG
    f = 0x1000
    items[0] = C.E8m0Item(f, 64, 8, 8, C.E8M0_OUT_KMAJOR, f, 64)
    assert _rc("lsmx_scale_to_e8m0_batch", ctypes.addressof(items), 1, None, 0, None) == C.ERR_ARG
    items[0] = C.E8m0Item(f, 64, 6, 6, 0, f, 64)
    assert _rc("lsmx_scale_to_e8m0_batch", ctypes.addressof(items), 1, None, 0, None) == C.ERR_SHAPE
    items[0] = C.E8m0Item(f, 64, 8, 8, 0, f + 2, 64)
    assert _rc("lsmx_scale_to_e8m0_batch", ctypes.addressof(items), 1, None, 0, None) == C.ERR_ALIGN
    items[0] = C.E8m0Item(f, 64, 8, 8, 0, f, 64)
    assert _rc("lsmx_scale_to_e8m0_batch", ctypes.addressof(items), 1, f + 4, 0, None) == C.ERR_ALIGN

    def pm(op=C.CODES_PACKED, a=FAKE, lda=128, M=64, N=64, K=256, sa_r=8, c_dtype=C.F32):
        return _rc("lsmx_gemm_mx_promote", a, lda, FAKE, sa_r, 1, FAKE, 128, FAKE, 8, 1, op, FAKE, c_dtype, N, M, N,
                   K, None, 0, None)
    assert pm(op=C.BF16) == C.ERR_DTYPE
    assert pm(c_dtype=C.E4M3) == C.ERR_DTYPE
    assert pm(K=192) == C.ERR_SHAPE and "multiple of 128" in C.last_error()
    assert pm(lda=64) == C.ERR_SHAPE
    assert pm(op=C.E4M3) == C.ERR_SHAPE       # E4M3 rows are K bytes long
    assert pm(a=ctypes.c_void_p(0x1008)) == C.ERR_ALIGN
    assert pm(lda=1 << 24, K=256) == C.ERR_SHAPE and "too long" in C.last_error()
    assert pm(sa_r=1 << 24) == C.ERR_SHAPE and "2^31" in C.last_error()
    assert _rc("lsmx_gemm_mx_promote", None, 128, FAKE, 8, 1, FAKE, 128, FAKE, 8, 1, C.CODES_PACKED, FAKE, C.F32,
               64, 64, 64, 256, None, 0, None) == C.ERR_ARG
    # N-contiguous B (LSMX_B_NCONTIG): E4M3 only, N % 16 == 0, ldb >= N, 256 rows of ldb within 2^31

    def pmn(op=C.E4M3 | C.B_NCONTIG, N=64, ldb=64, K=256):
        return _rc("lsmx_gemm_mx_promote", FAKE, K, FAKE, 8, 1, FAKE, ldb, FAKE, 1, N, op, FAKE, C.F32, N, 64, N, K,
                   None, 0, None)
    assert pmn(op=C.CODES_PACKED | C.B_NCONTIG) == C.ERR_DTYPE and "LSMX_E4M3" in C.last_error()
    assert pmn(N=40, ldb=48) == C.ERR_SHAPE and "multiple of 16" in C.last_error()
    assert pmn(ldb=48) == C.ERR_SHAPE and "too small" in C.last_error()
    assert pmn(ldb=1 << 23) == C.ERR_SHAPE and "too long" in C.last_error()


def test_n_contiguous_e4m3_gemm_validates_before_launch():
    """lsmx_gemm_f8f8_nb: K % 128, N % 16, ldb >= N, K-major scale strides
    >= rows, 16-byte rows and leading dimensions below 2^31 / 256."""
    def nb(K=128, N=64, ldb=64, lda=128, ld_sa=8, ld_sb=64, c_dtype=C.BF16, b=FAKE):
        return _rc("lsmx_gemm_f8f8_nb", FAKE, lda, FAKE, ld_sa, b, ldb, FAKE, ld_sb, FAKE, c_dtype, N, 8, N, K, None)
    assert nb(K=192) == C.ERR_SHAPE and "multiple of 128" in C.last_error()
    assert nb(N=40, ldb=48, ld_sb=40) == C.ERR_SHAPE and "multiple of 16" in C.last_error()
    assert nb(ldb=48) == C.ERR_SHAPE and "too small" in C.last_error()
    assert nb(ld_sa=4) == C.ERR_SHAPE and nb(ld_sb=32) == C.ERR_SHAPE
    assert nb(c_dtype=C.E4M3) == C.ERR_DTYPE
    assert nb(b=ctypes.c_void_p(0x1008)) == C.ERR_ALIGN
    assert nb(ldb=1 << 23) == C.ERR_SHAPE and "too large" in C.last_error()
    assert _rc("lsmx_gemm_f8f8_nb", None, 128, FAKE, 8, FAKE, 64, FAKE, 64, FAKE, C.BF16, 64, 8, 64, 128,
               None) == C.ERR_ARG


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is present")
def test_device_guard_without_gpu():
    assert _rc("lsmx_device_check") == C.ERR_DEVICE


def test_python_api_refuses_cpu_tensors():
    from lockstep_amd import fp4
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fp4.quantize_mxfp4(torch.zeros(2, 32))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fp4.pack_fp4(torch.zeros(2, 32, dtype=torch.uint8))


def test_python_api_keeps_reference_asserts():
    from lockstep_amd import fp4, mxfp4_gemm
    with pytest.raises(AssertionError, match="K=48 must be a multiple of block=32"):
        fp4.quantize_mxfp4(torch.zeros(2, 48))
    with pytest.raises(AssertionError, match="K must be a multiple of 128"):
        mxfp4_gemm.mxfp4_gemm_packed(torch.zeros(4, 48, dtype=torch.uint8),
                                     torch.zeros(4, 48, dtype=torch.uint8),
                                     torch.ones(4, 3), torch.ones(4, 3))


def test_device_guard_module_exits_without_gfx950():
    from lockstep_amd import device
    if torch.cuda.is_available() and "gfx950" in torch.cuda.get_device_properties(0).gcnArchName:
        pytest.skip("running on a gfx950")
    with pytest.raises(SystemExit, match="needs an MI355X"):
        device.require_gfx950()


def test_fp4_linear_reports_path_without_gpu():
    from lockstep_amd import fp4_linear
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    assert fp4_linear.kernel() is None and fp4_linear.path() == "unavailable"


def test_slot_arithmetic():
    # tests/test_fp4.py:95-102 (dual slot split round trip)
    from lockstep_amd import dual_gemm as dg
    for k in (8, 32, 128):
        s = dg.slot_offset(k)
        c1 = torch.tensor([144.0 * k, -144.0 * k, 3.0], dtype=torch.float64)
        c2 = torch.tensor([-144.0 * k, 144.0 * k, -7.0], dtype=torch.float64)
        g1, g2 = dg.unpack_dual(c1 + c2 * 2.0 ** s, s)
        assert torch.equal(g1, c1) and torch.equal(g2, c2)


def test_quantized_backward_checks_shapes_before_any_kernel():
    from lockstep_amd import fp4_linear
    x = torch.zeros(100, 128)
    w = torch.zeros(128, 128)
    with pytest.raises(AssertionError, match="multiples of 128"):
        fp4_linear.mxfp4_backward(torch.zeros(100, 128), x, w)
    with pytest.raises(AssertionError, match="shapes must be"):
        fp4_linear.mxfp4_backward(torch.zeros(128, 64), torch.zeros(128, 128), w)
    layer = fp4_linear.MXFP4Linear(128, 128)
    assert layer.quantized_backward is False      # the reference's STE backward by default
    assert fp4_linear.MXFP4Linear(128, 128, quantized_backward=True).quantized_backward


def test_dense_entry_points_validate_before_launch():
    bf = C.BF16
    # fp32 operands are not a dense GEMM type
    assert _rc("lsmx_gemm_dense", FAKE, None, 64, FAKE, None, 64, C.F32, 0, FAKE, None, 8, 8, 8, 64, 1,
               None) == C.ERR_DTYPE
    rc = _rc("lsmx_gemm_dense", FAKE, None, 96, FAKE, None, 96, bf, 0, FAKE, None, 8, 8, 8, 96, 1, None)
    assert rc == C.ERR_SHAPE and "K must be a multiple of 64" in C.last_error()      # dual_gemm.py:219
    rc = _rc("lsmx_gemm_dense", FAKE, FAKE, 192, FAKE, FAKE, 192, bf, 2, FAKE, FAKE, 8, 8, 8, 192, 2, None)
    assert rc == C.ERR_SHAPE and "K must divide splits*BK" in C.last_error()         # dual_gemm.py:265
    # dual separate needs both outputs, dual modes both operand pairs
    assert _rc("lsmx_gemm_dense", FAKE, FAKE, 64, FAKE, FAKE, 64, bf, 2, FAKE, None, 8, 8, 8, 64, 1,
               None) == C.ERR_ARG
    assert _rc("lsmx_gemm_dense", FAKE, None, 64, FAKE, FAKE, 64, bf, 1, FAKE, None, 8, 8, 8, 64, 1,
               None) == C.ERR_ARG
    assert _rc("lsmx_gemm_dense", FAKE, None, 64, FAKE, None, 64, bf, 3, FAKE, None, 8, 8, 8, 64, 1,
               None) == C.ERR_ARG
    rc = _rc("lsmx_gemm_dense", ctypes.c_void_p(0x1008), None, 64, FAKE, None, 64, bf, 0, FAKE, None, 8, 8, 8,
             64, 1, None)
    assert rc == C.ERR_ALIGN
    rc = _rc("lsmx_gemm_f8f8", FAKE, 64, FAKE, 2, FAKE, 64, FAKE, 2, C.SCALE_E8M0, FAKE, C.BF16, 8, 8, 8, 64, None)
    assert rc == C.ERR_SHAPE and "K must be a multiple of 128" in C.last_error()     # mxfp4_gemm.py:78
    assert _rc("lsmx_gemm_f8f8", FAKE, 128, FAKE, 4, FAKE, 128, FAKE, 4, C.SCALE_E8M0, FAKE, 7, 8, 8, 8, 128,
               None) == C.ERR_DTYPE
    assert _rc("lsmx_gemm_f8f8", FAKE, 128, FAKE, 4, FAKE, 128, FAKE, 4, C.SCALE_F32, FAKE, C.BF16, 8, 8, 8, 128,
               None) == C.ERR_DTYPE
    # K-major scales need ld >= rows
    assert _rc("lsmx_gemm_f8f8", FAKE, 128, FAKE, 4, FAKE, 128, FAKE, 8, C.SCALE_E8M0_KMAJOR, FAKE, C.BF16, 8, 8,
               8, 128, None) == C.ERR_SHAPE
    assert _rc("lsmx_transpose", FAKE, 3, 4, 4, 4, FAKE, 4, None) == C.ERR_DTYPE
    assert _rc("lsmx_transpose", FAKE, 2, 4, 8, 4, FAKE, 4, None) == C.ERR_SHAPE
    assert _rc("lsmx_scale_to_e8m0", None, 4, 4, 4, 0, FAKE, 4, None) == C.ERR_ARG
    assert _rc("lsmx_scale_to_e8m0", FAKE, 4, 6, 6, C.E8M0_OUT_KMAJOR, FAKE, 4, None) == C.ERR_SHAPE   # 6 blocks
    assert _rc("lsmx_scale_to_e8m0", FAKE, 4, 8, 8, 4, FAKE, 8, None) == C.ERR_ARG


def test_dense_python_api_asserts_then_refuses_cpu():
    from lockstep_amd import dual_gemm as dg
    from lockstep_amd import mxfp4_gemm
    a = torch.zeros(4, 96, dtype=torch.bfloat16)
    b = torch.zeros(96, 4, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="K must be a multiple of 64"):
        dg.gemm(a, b)
    with pytest.raises(AssertionError, match="K must divide splits\\*BK"):
        dg.splitk_packed(a[:, :64], a[:, :64], b[:64], b[:64], splits=2)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        dg.dual_separate(a[:, :64], a[:, :64], b[:64], b[:64])
    f8 = torch.zeros(4, 64, dtype=torch.uint8).view(torch.float8_e4m3fn)
    with pytest.raises(AssertionError, match="K must be a multiple of 128"):
        mxfp4_gemm.mxfp4_gemm_fp8(f8, f8.t(), torch.ones(4, 2), torch.ones(2, 4))


def test_gemm_leading_dimensions_bounded_for_32bit_offsets():
    # 256 rows of codes or scales past a descriptor base must fit 32-bit offsets
    big = 1 << 24
    rc = _rc("lsmx_gemm_f4f4", FAKE, big, FAKE, 4, FAKE, 64, FAKE, 4, C.SCALE_E8M0, FAKE, C.BF16, 8, 8, 8, 128, None)
    assert rc == C.ERR_SHAPE and "32-bit" in C.last_error()
    rc = _rc("lsmx_gemm_f4f4", FAKE, 64, FAKE, 1 << 22, FAKE, 64, FAKE, 4, C.SCALE_F32, FAKE, C.BF16, 8, 8, 8, 128,
             None)
    assert rc == C.ERR_SHAPE and "32-bit" in C.last_error()
    rc = _rc("lsmx_gemm_bf16f4", FAKE, 1 << 27, FAKE, 64, FAKE, 4, C.SCALE_E8M0, FAKE, C.BF16, 8, 8, 8, 128, None)
    assert rc == C.ERR_SHAPE and "32-bit" in C.last_error()


def test_weight_only_entry_point_validates_activation_type():
    assert _rc("lsmx_gemm_wonly_f4", FAKE, 7, 128, FAKE, 64, FAKE, 4, C.SCALE_E8M0, FAKE, C.F32, 8, 8, 8, 128,
               None) == C.ERR_DTYPE
    # fp32 rows of 100 elements are not 16-byte multiples
    assert _rc("lsmx_gemm_wonly_f4", FAKE, C.F32, 130, FAKE, 64, FAKE, 4, C.SCALE_E8M0, FAKE, C.F32, 8, 8, 8, 128,
               None) == C.ERR_ALIGN


def test_scale_shapes_are_checked_before_any_device_work():
    from lockstep_amd import dual_gemm, mxfp4_gemm
    pk = torch.zeros((64, 64), dtype=torch.uint8)
    good = torch.full((64, 4), 127, dtype=torch.uint8)
    with pytest.raises(AssertionError, match="scale must be"):
        mxfp4_gemm.mxfp4_gemm_packed(pk, pk, good[:32], good)
    with pytest.raises(AssertionError, match="scale must be"):
        mxfp4_gemm.mxfp4_gemm_bf16(torch.zeros((8, 128), dtype=torch.bfloat16), pk, good[:, :3])
    a = torch.zeros((8, 128), dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="scale must be"):
        dual_gemm.dual_mxfp4(a, a, pk, good.t())
    with pytest.raises(TypeError, match="activations must be"):
        mxfp4_gemm.mxfp4_gemm_bf16(torch.zeros((8, 128), dtype=torch.float64), pk, good)


def test_two_axis_quantizer_validates_before_launch():
    def args(dt, R, cols, fmt):
        return (FAKE, dt, R, cols, cols, FAKE, cols // 2, FAKE, R, FAKE, R // 2, FAKE, cols, fmt, None)
    assert _rc("lsmx_quantize_mxfp4_2d", *args(C.F32, 256, 256, C.SCALE_E8M0_KMAJOR)) == C.ERR_DTYPE
    assert _rc("lsmx_quantize_mxfp4_2d", *args(C.BF16, 256, 256, C.SCALE_F32)) == C.ERR_DTYPE
    rc = _rc("lsmx_quantize_mxfp4_2d", *args(C.BF16, 200, 256, C.SCALE_E8M0_KMAJOR))
    assert rc == C.ERR_SHAPE and "multiples of 128" in C.last_error()


def test_split_k_plan_through_workspace_size():
    """The split-K plan of the bf16 x MXFP4 GEMM, read through the workspace
    size it asks for (fp32 partials [splits][batches][Mp][Np]; 256 CUs when
    no device is present).  Of the plans that fit one wave of workgroups the
    widest wins, then the one with the fewest partial bytes: M = 128 against
    N = 14336 takes 128 x 128 tiles in 2 slices (224 workgroups) rather than
    128 x 256 in 4; M = 256 keeps 128 x 256 in 2; whole-K shapes and skinny
    M ask for nothing."""
    L = C.load()
    ws = lambda M, N, K, dual=0: L.lsmx_gemm_bf16f4_workspace(M, N, K, dual)   # noqa: E731
    assert ws(128, 14336, 4096) == 2 * 128 * 14336 * 4
    assert ws(128, 14336, 4096, 1) == 2 * 2 * 128 * 14336 * 4
    assert ws(256, 14336, 2048) == 2 * 256 * 14336 * 4
    assert ws(64, 2304, 4096) == 4 * 128 * 2304 * 4
    assert ws(200, 1000, 2048) == 4 * 256 * 1024 * 4
    assert ws(1024, 14336, 4096) == 0 and ws(16, 14336, 4096) == 0
