"""GPU checks of block-scale handling and of the accumulation order of the
packed dual GEMM.

  - In the weight-only GEMMs (an extension of the reference, whose weight is
    MXFP4 with E8M0 scales) an fp32 scale with no E8M0 form (not a positive
    power of two in [2^-127, 2^127]) makes exactly the outputs that use it
    NaN.  mxfp4_gemm_packed and mxfp4_gemm_fp8 instead apply any fp32 scale
    as the reference does (tests/test_gpu_promote.py).
  - E8M0 byte 0 is 2^-127 in the dequantizer and in the scaled MFMA alike.
  - dual_packed adds its two products in alternating 64-deep K blocks, the
    order of the reference's loop (dual_gemm.py:59-61).
"""

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import dual_gemm, fp4, mxfp4_gemm
    return fp4, mxfp4_gemm, dual_gemm


@pytest.mark.parametrize("M", [1, 16, 256])
@pytest.mark.parametrize("act", [torch.bfloat16, torch.float32])
def test_weight_only_non_power_of_two_scales_poison_their_columns(dev, mods, M, act):
    """M = 1 runs the GEMV, 16 the decode kernel, 256 the tiled kernel (bf16)
    or the exact-split kernel (fp32)."""
    fp4, mg, _ = mods
    N, K = 256, 512
    g = torch.Generator(device=dev).manual_seed(M)
    a = torch.randn((M, K), device=dev, generator=g).to(act)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    codes, s = fp4.quantize_mxfp4(w)
    wpk = fp4.pack_fp4(codes)
    clean = mg.mxfp4_gemm_bf16(a, wpk, s, out_dtype=torch.float32)
    s2 = s.clone()
    s2[5, 2] = 1.5
    s2[9, 0] = -s2[9, 0]
    bad = mg.mxfp4_gemm_bf16(a, wpk, s2, out_dtype=torch.float32)
    assert bad[:, 5].isnan().all() and bad[:, 9].isnan().all()
    keep = torch.ones(N, dtype=torch.bool, device=dev)
    keep[5] = keep[9] = False
    assert torch.equal(bad[:, keep], clean[:, keep])
    # E8M0 bytes of the same scales: the clean result, bit for bit
    assert torch.equal(mg.mxfp4_gemm_bf16(a, wpk, fp4.scale_to_e8m0(s), out_dtype=torch.float32), clean)


def test_e8m0_byte_zero_is_two_to_minus_127(dev, mods, oracle):
    """Caller-supplied E8M0 byte 0: the dequantizer and the f4 x f4 GEMM both
    read it as 2^-127 (the oracle's ldexp(1, -127)); B's scales are large so
    that the products stay normal fp32 numbers."""
    fp4, mg, _ = mods
    rng = np.random.default_rng(7)
    M, N, K = 64, 96, 256
    ca = rng.integers(0, 16, (M, K), dtype=np.uint8)
    cb = rng.integers(0, 16, (N, K), dtype=np.uint8)
    ea = np.where(rng.random((M, K // 32)) < 0.5, 0, 120).astype(np.uint8)
    eb = rng.integers(190, 200, (N, K // 32)).astype(np.uint8)
    apk, bpk = oracle.pack_fp4(ca), oracle.pack_fp4(cb)
    deq = fp4.dequantize_packed(torch.from_numpy(apk).to(dev), torch.from_numpy(ea).to(dev))
    want = oracle.dequantize_packed(apk, ea)
    assert np.array_equal(deq.cpu().numpy().astype(np.float64), want)
    assert fp4.e8m0_to_scale(torch.zeros(1, dtype=torch.uint8)).item() == 2.0 ** -127
    c = mg.mxfp4_gemm_packed(*(torch.from_numpy(t).to(dev) for t in (apk, bpk, ea, eb)), out_dtype=torch.float32)
    ref = oracle.reference_gemm_packed(apk, ea, bpk, eb)
    assert oracle.max_rel(c.cpu().numpy(), ref) <= 1e-6


def test_short_scale_tensors_raise_before_launch(dev, mods):
    fp4, mg, dg = mods
    pk = torch.zeros((64, 64), dtype=torch.uint8, device=dev)
    good = torch.full((64, 4), 127, dtype=torch.uint8, device=dev)
    short = good[:32]
    with pytest.raises(AssertionError, match="scale must be"):
        mg.mxfp4_gemm_packed(pk, pk, short, good)
    with pytest.raises(AssertionError, match="scale must be"):
        mg.mxfp4_gemm_bf16(torch.zeros((8, 128), dtype=torch.bfloat16, device=dev), pk, short)
    with pytest.raises(AssertionError, match="scale must be"):
        a = torch.zeros((8, 128), dtype=torch.bfloat16, device=dev)
        dg.dual_mxfp4(a, a, pk, good[:, :2])


@pytest.mark.parametrize("path", ["ring", "splitk"])
def test_dual_packed_alternates_products_per_64_block(dev, mods, path):
    """Order-sensitive data: with one nonzero product per K block,
    A1.B1 = 2^25 (block 0) and -2^25 (block 1), A2.B2 = 1 and 1.  The
    reference's order (block 0 of A1.B1, block 0 of A2.B2, block 1 of each)
    gives 2^25 + 1 -> 2^25 (fp32 rounds to even), then 0, then 1.  Summing
    all of A1.B1 first would give 2.  "ring" is the persistent 256 x 256
    kernel; "splitk" (2 slices of K, the second all zeros) the 128 x 128
    kernel with fp32 atomics."""
    _, _, dg = mods
    K = 128 if path == "ring" else 256
    M = N = 64
    a1 = torch.zeros((M, K), dtype=torch.float32)
    b1 = torch.zeros((K, N), dtype=torch.float32)
    a2 = torch.zeros((M, K), dtype=torch.float32)
    b2 = torch.zeros((K, N), dtype=torch.float32)
    a1[:, 0], b1[0, :] = 2.0 ** 13, 2.0 ** 12
    a1[:, 64], b1[64, :] = -(2.0 ** 13), 2.0 ** 12
    a2[:, 0], b2[0, :] = 1.0, 1.0
    a2[:, 64], b2[64, :] = 1.0, 1.0
    t = [x.to(torch.bfloat16).to(dev) for x in (a1, a2, b1, b2)]
    if path == "ring":
        acc = dg.dual_packed(*t)
    else:
        acc = dg.splitk_packed(*t, splits=2)
    assert torch.equal(acc, torch.ones((M, N), device=dev))
