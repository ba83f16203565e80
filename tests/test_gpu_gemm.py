"""GPU parity of the block-scaled GEMMs against the fp64 oracle (fp4.py:103-112).

Tolerances (stated by the build's target, bench.py:71 metric
max|c - ref| / max|ref|):  fp32 output <= 1e-5,  bf16 output <= 1e-2.
Integer-grid inputs with unit scales must be bit-exact (bench.py:44-57).
"""

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import dual_gemm, fp4, fp4_linear, mxfp4_gemm
    return fp4, mxfp4_gemm, dual_gemm, fp4_linear


def quantized_operand(oracle, x: np.ndarray):
    codes, scale = oracle.quantize_mxfp4(x)
    return oracle.pack_fp4(codes), oracle.scale_to_e8m0(scale), scale


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_integer_grid_is_bit_exact(dev, mods, oracle):
    """bench.py:44-57: random codes, unit scales, K=128 -> C == (qa @ qb) / 4."""
    fp4, mg, _, _ = mods
    rng = np.random.default_rng(0)
    pick = np.array([c for c in range(16) if c != 8], dtype=np.uint8)
    ca = pick[rng.integers(0, 15, (256, 128))]
    cb = pick[rng.integers(0, 15, (256, 128))]
    ones_a = torch.ones((256, 4), device=dev)
    got = mg.mxfp4_gemm_packed(_dev(oracle.pack_fp4(ca), dev), _dev(oracle.pack_fp4(cb), dev),
                               ones_a, ones_a.clone(), out_dtype=torch.float32).cpu().numpy()
    qa, qb = oracle.E2M1_Q[ca].astype(np.float64), oracle.E2M1_Q[cb].astype(np.float64)
    assert np.array_equal(got.astype(np.float64), (qa @ qb.T) / 4.0)


def test_random_codes_and_scales(dev, mods, oracle):
    """cuda/mxfp4_mma_gemm.cu:204-252: codes 0..15 (incl. -0), scales 2^[-3,3]."""
    fp4, mg, _, _ = mods
    rng = np.random.default_rng(1234)
    M = N = K = 256
    ca = rng.integers(0, 16, (M, K), dtype=np.uint8)
    cb = rng.integers(0, 16, (N, K), dtype=np.uint8)
    ea = (127 + rng.integers(-3, 4, (M, K // 32))).astype(np.uint8)
    eb = (127 + rng.integers(-3, 4, (N, K // 32))).astype(np.uint8)
    ref = oracle.reference_gemm_packed(oracle.pack_fp4(ca), ea, oracle.pack_fp4(cb), eb)
    got = mg.mxfp4_gemm_packed(_dev(oracle.pack_fp4(ca), dev), _dev(oracle.pack_fp4(cb), dev),
                               _dev(ea, dev), _dev(eb, dev), out_dtype=torch.float32).cpu().numpy()
    assert oracle.max_rel(got, ref) <= 1e-6
    # each 32-block partial is exact, so only fp32 accumulation rounds
    el = np.abs(got - ref) / (np.abs(ref) + 1e-9)
    assert np.median(el) < 1e-7


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (1, 1, 128), (37, 129, 384), (300, 513, 128),
                                   (512, 256, 1024)])
def test_quantized_randn_matches_fp64(dev, mods, oracle, out_dtype, M, N, K):
    """bench.py:60-81 at small shapes, ragged M and N included."""
    fp4, mg, _, _ = mods
    a = gen.normal(M * 7 + K, (M, K))
    bt = gen.student_t3(N * 13 + K, (N, K), scale=0.05)
    apk, ae8, as32 = quantized_operand(oracle, a)
    bpk, be8, bs32 = quantized_operand(oracle, bt)
    ref = oracle.reference_gemm_packed(apk, ae8, bpk, be8)
    for sa, sb in ((ae8, be8), (as32, bs32)):      # E8M0 bytes and fp32 scales
        got = mg.mxfp4_gemm_packed(_dev(apk, dev), _dev(bpk, dev), _dev(sa, dev), _dev(sb, dev),
                                   out_dtype=out_dtype)
        assert got.dtype == out_dtype and got.shape == (M, N)
        assert oracle.max_rel(got.float().cpu().numpy(), ref) <= TOL[out_dtype]


def test_gpu_quantized_operands_end_to_end(dev, mods, oracle):
    """Quantize on the GPU, multiply on the GPU, compare with the oracle chain."""
    fp4, mg, _, _ = mods
    a = torch.randn(512, 2048, device=dev)
    b = torch.randn(384, 2048, device=dev) * 0.02
    apk, ae8 = fp4.quantize_pack_mxfp4(a)
    bpk, be8 = fp4.quantize_pack_mxfp4(b)
    c = mg.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.float32)
    ref = oracle.reference_gemm_packed(*[t.cpu().numpy() for t in (apk, ae8, bpk, be8)])
    assert oracle.max_rel(c.cpu().numpy(), ref) <= 1e-5
    # the reference API spelling: fp32 scales from quantize_mxfp4 + pack_fp4
    ac, as_ = fp4.quantize_mxfp4(a)
    bc, bs_ = fp4.quantize_mxfp4(b)
    c2 = mg.mxfp4_gemm_packed(fp4.pack_fp4(ac), fp4.pack_fp4(bc), as_, bs_, out_dtype=torch.float32)
    assert torch.equal(c, c2)


def test_full_size_8192_cubed_sampled(dev, mods, oracle):
    """BASELINE cfg4 at full size: A, B = 0.05 * t3 [8192, 8192], quantized on
    the fly, f4 x f4, bf16 out; sampled rows/columns vs fp64 (the sampling of
    cuda/mxfp4_mma_gemm.cu:235-236)."""
    fp4, mg, _, _ = mods
    n = 8192
    g = torch.Generator(device=dev).manual_seed(4001)

    def t3():
        z = torch.randn((n, n), device=dev, generator=g)
        chi = torch.zeros_like(z)
        for _ in range(3):
            chi += torch.randn((n, n), device=dev, generator=g).square()
        return z / torch.sqrt(chi / 3.0) * 0.05

    a, b = t3(), t3()
    apk, ae8 = fp4.quantize_pack_mxfp4(a)
    bpk, be8 = fp4.quantize_pack_mxfp4(b)
    del a, b
    c = mg.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.bfloat16)
    rows = np.arange(0, n, 37)
    cols = np.arange(0, n, 41)
    ref = oracle.reference_gemm_packed(apk.cpu().numpy(), ae8.cpu().numpy(), bpk.cpu().numpy(),
                                       be8.cpu().numpy(), rows=rows, cols=cols)
    got = c.float().cpu().numpy()[np.ix_(rows, cols)]
    assert oracle.max_rel(got, ref) <= 1e-2
    c32 = mg.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.float32)
    assert oracle.max_rel(c32.cpu().numpy()[np.ix_(rows, cols)], ref) <= 1e-5
    # bf16 output is the RNE rounding of the fp32 result
    assert torch.equal(c, c32.to(torch.bfloat16))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(1, 256, 4096), (2, 300, 640), (1, 14336, 4096), (16, 300, 512), (100, 512, 128),
                                   (256, 256, 1024), (513, 1024, 256), (1, 300, 640), (1, 17, 8192), (1, 1, 128)])
def test_weight_only_bf16_x_fp4(dev, mods, oracle, out_dtype, M, N, K):
    fp4, mg, _, _ = mods
    a = gen.to_bf16_bits(gen.normal(M + 5 * K, (M, K)))
    w = gen.normal(N + 3 * K, (N, K), std=0.02)
    wpk, we8, ws32 = quantized_operand(oracle, w)
    ref = oracle.reference_gemm_wonly(gen.bf16_bits_to_f32(a), wpk, we8)
    at = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    for s in (we8, ws32):
        got = mg.mxfp4_gemm_bf16(at, _dev(wpk, dev), _dev(s, dev), out_dtype=out_dtype)
        assert oracle.max_rel(got.float().cpu().numpy(), ref) <= TOL[out_dtype]


@pytest.mark.parametrize("M,N,K", [(2, 700, 512), (3, 300, 1536), (8, 1000, 4096), (16, 520, 8192),
                                   (16, 260, 4608), (5, 14336, 4096)])
def test_weight_only_decode_shapes(dev, mods, oracle, M, N, K):
    """2 <= M <= 16 with K % 512 == 0 runs the decode kernel: 512-deep slices
    per wave, 4096-deep passes (K = 8192: two; 4608: a second pass with one
    live slice), ragged weight rows.  fp32 output vs the fp64 oracle; E8M0
    bytes and fp32 powers of two give the same bits; the dual form gives the
    single form's bits for both batches."""
    fp4, mg, dg, _ = mods
    g = torch.Generator(device=dev).manual_seed(M * 131 + N + K)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    codes, s32 = fp4.quantize_mxfp4(w)
    wpk = fp4.pack_fp4(codes)
    we8 = fp4.scale_to_e8m0(s32)
    c = mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32)
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy())
    assert oracle.max_rel(c.cpu().numpy(), ref) <= 1e-5
    assert torch.equal(mg.mxfp4_gemm_bf16(a, wpk, s32, out_dtype=torch.float32), c)
    c0, c1 = dg.dual_mxfp4(a, a1, wpk, we8, out_dtype=torch.float32)
    assert torch.equal(c0, c)
    assert torch.equal(c1, mg.mxfp4_gemm_bf16(a1, wpk, we8, out_dtype=torch.float32))


@pytest.mark.parametrize("M,N,K", [(17, 4096, 512), (32, 5000, 4608), (48, 14336, 8192), (64, 14336, 4096),
                                   (40, 16384, 1024)])
def test_weight_only_mid_m_shapes(dev, mods, oracle, M, N, K):
    """17 <= M <= 64 against 16 .. 64 weight rows per CU with K % 512 == 0
    runs the mid-M kernel (no split-K workspace is asked for): activation
    groups of 64 rows (the dual forms of M = 48 and 64 have two; with
    K = 8192 each group reloads its weight slices), a second pass with one
    live slice (K = 4608), two live waves (K = 1024), ragged weight rows.
    fp32 output vs the fp64 oracle; E8M0 bytes and fp32 powers of two give
    the same bits; the dual form gives the single form's bits for both
    batches; bf16 and fp16 outputs are the fp32 result rounded."""
    from lockstep_amd import _capi as C
    fp4, mg, dg, _ = mods
    assert C.load().lsmx_gemm_bf16f4_workspace(M, N, K, 0) == 0
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    codes, s32 = fp4.quantize_mxfp4(w)
    wpk = fp4.pack_fp4(codes)
    we8 = fp4.scale_to_e8m0(s32)
    c = mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32)
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy())
    assert oracle.max_rel(c.cpu().numpy(), ref) <= 1e-5
    assert torch.equal(mg.mxfp4_gemm_bf16(a, wpk, s32, out_dtype=torch.float32), c)
    c0, c1 = dg.dual_mxfp4(a, a1, wpk, we8, out_dtype=torch.float32)
    assert torch.equal(c0, c)
    assert torch.equal(c1, mg.mxfp4_gemm_bf16(a1, wpk, we8, out_dtype=torch.float32))
    for dt in (torch.bfloat16, torch.float16):
        assert torch.equal(mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=dt), c.to(dt))


def test_weight_only_mid_m_special_scale_bytes(dev, mods, oracle):
    """E8M0 bytes 0 (2^-127) and 255 (NaN) in the mid-M kernel: the NaN
    byte's column is NaN, the others match the oracle."""
    fp4, mg, _, _ = mods
    M, N, K = 40, 14336, 4096
    g = torch.Generator(device=dev).manual_seed(78)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    bad = we8.clone()
    bad[7, 5] = 255
    bad[9000, 31] = 0
    c = mg.mxfp4_gemm_bf16(a, wpk, bad, out_dtype=torch.float32).cpu().numpy()
    assert np.isnan(c[:, 7]).all()
    keep = np.ones(N, dtype=bool)
    keep[7] = False
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), bad.cpu().numpy())
    assert not np.isnan(c[:, keep]).any()
    assert oracle.max_rel(c[:, keep], ref[:, keep]) <= 1e-5


def test_weight_only_decode_nan_scale_byte(dev, mods, oracle):
    """An E8M0 byte 255 (NaN) in one block of a weight row makes that output
    column NaN and leaves the others as the oracle computes them (the decode
    kernel then takes its exact scale conversion for the whole wave)."""
    fp4, mg, _, _ = mods
    M, N, K = 4, 300, 1024
    g = torch.Generator(device=dev).manual_seed(77)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    bad = we8.clone()
    bad[7, 5] = 255
    bad[123, 31] = 255
    c = mg.mxfp4_gemm_bf16(a, wpk, bad, out_dtype=torch.float32).cpu().numpy()
    assert np.isnan(c[:, 7]).all() and np.isnan(c[:, 123]).all()
    keep = np.ones(N, dtype=bool)
    keep[[7, 123]] = False
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy())
    assert not np.isnan(c[:, keep]).any()
    assert oracle.max_rel(c[:, keep], ref[:, keep]) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 512), (128, 14336, 512), (1000, 1000, 256), (1500, 4000, 512)])
def test_weight_only_tile_paths(dev, mods, oracle, M, N, K):
    """Large M runs 256 x 256 tiles, mid M (cfg3's M = 128) 128 x 128 tiles, and a single launch whose
    256 x 256 tiles would leave CUs idle 128 x 256 tiles (1500 x 4000, ragged in both): all match the fp64
    oracle on sampled rows, and give the same bits."""
    fp4, mg, _, _ = mods
    g = torch.Generator(device=dev).manual_seed(M + N)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    c = mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32)
    rows = np.arange(0, M, max(1, M // 48))
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy(), rows=rows)
    assert oracle.max_rel(c.cpu().numpy()[rows], ref) <= 1e-5
    # a row slice runs a different tile size (or grid) and must give the same bits
    part = mg.mxfp4_gemm_bf16(a[:64 + M // 4], wpk, we8, out_dtype=torch.float32)
    assert torch.equal(part, c[:64 + M // 4])


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (100, 300, 256), (1, 256, 128), (2, 520, 384), (1, 4096, 4096),
                                   (1500, 4000, 512)])
def test_dual_batch_matches_single_and_oracle(dev, mods, oracle, M, N, K):
    """cfg2 (and ragged shapes): two bf16 batches share one MXFP4 weight."""
    fp4, mg, dg, _ = mods
    g = torch.Generator(device=dev).manual_seed(2001)
    a0 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    c0, c1 = dg.dual_mxfp4(a0, a1, wpk, we8, out_dtype=torch.float32)
    s0 = mg.mxfp4_gemm_bf16(a0, wpk, we8, out_dtype=torch.float32)
    s1 = mg.mxfp4_gemm_bf16(a1, wpk, we8, out_dtype=torch.float32)
    assert torch.equal(c0, s0) and torch.equal(c1, s1)      # same order of summation
    rows = np.arange(0, M, max(1, M // 64))
    for a, c in ((a0, c0), (a1, c1)):
        ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy(),
                                          rows=rows)
        assert oracle.max_rel(c.cpu().numpy()[rows], ref) <= 1e-5
    b0, b1 = dg.dual_mxfp4(a0, a1, wpk, we8)
    assert torch.equal(b0, c0.to(torch.bfloat16)) and torch.equal(b1, c1.to(torch.bfloat16))


def test_fp4_linear_forward_backward(dev, mods, oracle):
    """fp4_linear.py:34-45: MXFP4 forward (X and W quantized), STE backward."""
    fp4, mg, _, fl = mods
    assert fl.path() == "hip-mxfp4"
    # kernel() returns the packed-operand GEMM, as fp4_linear.py:16-25 does
    assert fl.kernel() is mg.mxfp4_gemm_packed
    torch.manual_seed(0)
    layer = fl.MXFP4Linear(1024, 512).to(dev)
    x = torch.randn(4, 64, 1024, device=dev, requires_grad=True)
    y = layer(x)
    assert y.shape == (4, 64, 512) and y.dtype == torch.float32
    xq = oracle.quantize_pack(x.detach().reshape(-1, 1024).cpu().numpy())
    wq = oracle.quantize_pack(layer.weight.detach().cpu().numpy())
    ref = oracle.reference_gemm_packed(xq[0], xq[1], wq[0], wq[1])
    assert oracle.max_rel(y.detach().reshape(-1, 512).cpu().numpy(), ref) <= 1e-5
    gy = torch.randn_like(y)
    y.backward(gy)
    gx = gy.reshape(-1, 512) @ layer.weight
    gw = gy.reshape(-1, 512).t() @ x.detach().reshape(-1, 1024)
    assert torch.allclose(x.grad.reshape(-1, 1024), gx) and torch.allclose(layer.weight.grad, gw)
    with torch.no_grad():
        yb = layer(x.detach().to(torch.bfloat16))
    assert yb.dtype == torch.bfloat16
    assert oracle.max_rel(yb.float().reshape(-1, 512).cpu().numpy(),
                          oracle.reference_gemm_packed(*oracle.quantize_pack(
                              gen.to_bf16_bits(x.detach().reshape(-1, 1024).cpu().numpy()), "bf16"),
                              wq[0], wq[1])) <= 1e-2


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (37, 129, 384), (300, 513, 128), (1024, 768, 2048)])
def test_kmajor_scales_give_identical_gemm(dev, mods, oracle, M, N, K):
    """The K-major scale layout is a relayout only: same bits out."""
    fp4, mg, _, _ = mods
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    a = torch.randn((M, K), device=dev, generator=g)
    b = torch.randn((N, K), device=dev, generator=g) * 0.02
    apk, ae8 = fp4.quantize_pack_mxfp4(a)
    bpk, be8 = fp4.quantize_pack_mxfp4(b)
    _, ak = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    _, bk = fp4.quantize_pack_mxfp4(b, scale_layout="kmajor")
    c_rows = mg.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.float32)
    c_km = mg.mxfp4_gemm_packed(apk, bpk, ak, bk, out_dtype=torch.float32)
    assert torch.equal(c_rows, c_km)
    ref = oracle.reference_gemm_packed(*[t.cpu().numpy() for t in (apk, ae8, bpk, be8)])
    assert oracle.max_rel(c_km.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(128, 14336, 4096), (200, 1000, 2048), (256, 4096, 1024), (64, 2304, 4096),
                                   (256, 14336, 2048)])
def test_weight_only_split_k(dev, mods, oracle, M, N, K):
    """Mid-size M against a wide weight splits K (lsmx_gemm_bf16f4_ws): each
    slice's fp32 partial tile goes to a workspace and a second kernel adds
    the slices in slice order.  128 x 128 tiles in 2 or 4 slices at the
    first four shapes, 128 x 256 tiles in 2 at the last.  vs fp64; repeated calls and the dual form
    give the same bits; a call at another shape in between (sharing the
    cached workspace) does not disturb them."""
    fp4, mg, dg, _ = mods
    from lockstep_amd import _capi
    assert _capi.load().lsmx_gemm_bf16f4_workspace(M, N, K, 0) > 0, "this shape must take the split-K path"
    g = torch.Generator(device=dev).manual_seed(M * 7 + K)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    c = mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32)
    rows = np.unique(np.linspace(0, M - 1, 40).astype(np.int64))
    cols = np.arange(0, N, 3)
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy(),
                                      rows=rows, cols=cols)
    assert oracle.max_rel(c.cpu().numpy()[np.ix_(rows, cols)], ref) <= 1e-5
    other = mg.mxfp4_gemm_bf16(a[:, :K // 2].contiguous(), wpk[:N // 2, :K // 4].contiguous(),
                               we8[:N // 2, :K // 64].contiguous(), out_dtype=torch.float32)
    assert other.shape == (M, N // 2)
    assert torch.equal(mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32), c)
    c0, c1 = dg.dual_mxfp4(a, a1, wpk, we8, out_dtype=torch.float32)
    assert torch.equal(c0, c)
    assert torch.equal(c1, mg.mxfp4_gemm_bf16(a1, wpk, we8, out_dtype=torch.float32))
    b16 = mg.mxfp4_gemm_bf16(a, wpk, we8)
    assert torch.equal(b16, c.to(torch.bfloat16))


def test_weight_only_split_k_on_two_streams(dev, mods):
    """Split-K calls running at once on two streams use one workspace per stream: the concurrent
    results equal the sequential ones bit for bit, three rounds in a row."""
    fp4, mg, _, _ = mods
    g = torch.Generator(device=dev).manual_seed(99)
    M, N, K = 128, 14336, 4096
    a = [torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16) for _ in range(2)]
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    want = [mg.mxfp4_gemm_bf16(x, wpk, we8, out_dtype=torch.float32) for x in a]
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    for _ in range(3):
        got = []
        for x, s in zip(a, streams):
            s.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(s):
                got.append(mg.mxfp4_gemm_bf16(x, wpk, we8, out_dtype=torch.float32))
        torch.cuda.synchronize(dev)
        for y, ref in zip(got, want):
            assert torch.equal(y, ref)


@pytest.mark.parametrize("adt", [torch.float32, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 1024, 1024), (1000, 2100, 512), (4096, 4096, 256), (512, 2048, 256),
                                   (1, 300, 128), (70, 130, 384), (70, 130, 2048), (33, 40, 256)])
def test_weight_only_wide_activations(dev, mods, oracle, adt, M, N, K):
    """fp32 and fp16 activations (lsmx_gemm_wonly_f4): each activation is
    split exactly into bf16 terms, so Y = X . deq(W)^T has the arithmetic of
    an fp32 matmul (fp4.py:75-78 dequantization, fp4_linear.py:40's
    fake-quant forward with an unquantized X).  All tile shapes on 256 CUs
    (64 x 128; 64 x 64 at 512 x 2048; 32 x 32 split four ways along K for
    the smaller outputs, with four K groups of 4 waves when K / 64 % 4 == 0:
    cfg1's 256 x 1024 x 1024, 70 x 130 x 2048 and 33 x 40 x 256 with one
    stage per group), ragged edges; fp32 output <=
    1e-5 vs fp64; bf16 output is the RNE of the fp32 one; fp32 scales give
    the same bits as E8M0 bytes; a row holding +-Inf gives the oracle's
    non-finite pattern."""
    fp4, mg, _, _ = mods
    g = torch.Generator(device=dev).manual_seed(M + 3 * N + K)
    x = torch.randn((M, K), device=dev, generator=g)
    x[:, ::7] *= 1e-3                                            # terms mid and lo carry real bits
    x = x.to(adt)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    _, ws32 = fp4.quantize_mxfp4(w)
    c = mg.mxfp4_gemm_bf16(x, wpk, we8, out_dtype=torch.float32)
    ref = oracle.reference_gemm_wonly(x.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy())
    assert oracle.max_rel(c.cpu().numpy(), ref) <= 1e-5
    assert torch.equal(mg.mxfp4_gemm_bf16(x, wpk, ws32, out_dtype=torch.float32), c)
    assert torch.equal(mg.mxfp4_gemm_bf16(x, wpk, we8), c.to(torch.bfloat16))
    if M > 1:
        xs = x.clone()
        xs[M // 2, K // 3] = float("inf")
        xs[M - 1, 5] = float("-inf")
        cs = mg.mxfp4_gemm_bf16(xs, wpk, we8, out_dtype=torch.float32).cpu().numpy()
        rs = oracle.reference_gemm_wonly(xs.float().cpu().numpy(), wpk.cpu().numpy(), we8.cpu().numpy())
        assert np.array_equal(np.isnan(cs), np.isnan(rs)) and np.array_equal(np.isposinf(cs), np.isposinf(rs))
        assert np.array_equal(np.isneginf(cs), np.isneginf(rs))
        fin = np.isfinite(rs)
        assert oracle.max_rel(cs[fin], rs[fin]) <= 1e-5
