"""GPU checks of fp32 block scales of any value (lsmx_scale_to_e8m0_batch +
lsmx_gemm_mx_promote), through the reference's spelling of mxfp4_gemm_packed
and mxfp4_gemm_fp8.

The reference promotes every 32-block product to fp32 and multiplies the two
fp32 scales there (mxfp4_gemm.py:52-63, 141-150).  The fast kernels apply
E8M0 exponents inside the scaled MFMA, which is the same only for powers of
two; any other scale is flagged by the scale conversion and the output is
recomputed by the promotion kernel.  The oracle's gemm_promote restates the
reference's loop (with the fma Triton contracts `acc += p * s` to); on the
E2M1 grid every block product is exact, so the GPU must match it bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import _capi as C
    from lockstep_amd import fp4, mxfp4_gemm
    return C, fp4, mxfp4_gemm


def _codes(rng, rows, K):
    return rng.integers(0, 16, (rows, K), dtype=np.uint8)


def _same(got: torch.Tensor, want32: np.ndarray):
    """got (fp32 or bf16) equals the oracle's fp32 result rounded to got's
    dtype, NaN positions included."""
    w = torch.from_numpy(want32)
    if got.dtype != torch.float32:
        w = w.to(got.dtype)
    g = got.cpu()
    np.testing.assert_array_equal(g.float().numpy(), w.float().numpy())


SHAPES = [(256, 256, 256), (300, 200, 384), (1, 130, 128), (129, 1, 1152), (520, 384, 4096)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_packed_any_scales_match_the_promotion_oracle(dev, mods, oracle, M, N, K, out):
    """Random fp32 scales in (-2, 2): ragged tiles, K % 256 == 128 (a half
    chunk), single rows and columns."""
    C, fp4, mg = mods
    rng = np.random.default_rng(M * 7 + N + K)
    ca, cb = _codes(rng, M, K), _codes(rng, N, K)
    sa = rng.uniform(-2, 2, (M, K // 32)).astype(np.float32)
    sb = rng.uniform(-2, 2, (N, K // 32)).astype(np.float32)
    got = mg.mxfp4_gemm_packed(torch.from_numpy(oracle.pack_fp4(ca)).to(dev),
                               torch.from_numpy(oracle.pack_fp4(cb)).to(dev),
                               torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev), out_dtype=out)
    _same(got, oracle.gemm_promote(oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb], sa, sb))


def test_one_odd_scale_recomputes_the_whole_output(dev, mods, oracle):
    """Quantizer scales (powers of two) with one 1.5 and one -2: every output
    equals the promotion oracle's (not only the row and column that use the
    odd scales), where the fast kernel alone would have made them NaN."""
    C, fp4, mg = mods
    M, N, K = 256, 320, 512
    a = gen.normal(41, (M, K))
    b = gen.normal(42, (N, K), std=0.02)
    ac, as_ = oracle.quantize_mxfp4(a)
    bc, bs_ = oracle.quantize_mxfp4(b)
    as_[5, 2] = 1.5
    bs_[7, 1] = -2.0
    got = mg.mxfp4_gemm_packed(torch.from_numpy(oracle.pack_fp4(ac)).to(dev),
                               torch.from_numpy(oracle.pack_fp4(bc)).to(dev),
                               torch.from_numpy(as_).to(dev), torch.from_numpy(bs_).to(dev),
                               out_dtype=torch.float32)
    assert not got.isnan().any()
    _same(got, oracle.gemm_promote(oracle.E2M1_VALUES[ac], oracle.E2M1_VALUES[bc], as_, bs_))


def test_power_of_two_scales_keep_the_fast_kernel_bits(dev, mods, oracle):
    """With the quantizer's scales the promotion launch exits at once: the
    reference's spelling gives the K-major E8M0 call's bits."""
    C, fp4, mg = mods
    M, N, K = 512, 384, 1024
    x = torch.from_numpy(gen.normal(43, (M, K))).to(dev)
    w = torch.from_numpy(gen.normal(44, (N, K), std=0.02)).to(dev)
    xc, xs = fp4.quantize_mxfp4(x)
    wc, ws = fp4.quantize_mxfp4(w)
    assert fp4.e8m0_exact(xs, ws)   # the quantizer's own scales: no promotion launch at all
    ref_spelling = mg.mxfp4_gemm_packed(fp4.pack_fp4(xc), fp4.pack_fp4(wc), xs, ws)
    xk = fp4.quantize_pack_mxfp4(x, scale_layout="kmajor")
    wk = fp4.quantize_pack_mxfp4(w, scale_layout="kmajor")
    fast = mg.mxfp4_gemm_packed(xk[0], wk[0], xk[1], wk[1])
    assert torch.equal(ref_spelling, fast)
    # copies of them are checked on the device: the flag stays clear and the
    # promotion launch exits
    xs2, ws2 = xs.clone(), ws.clone()
    assert not fp4.e8m0_exact(xs2, ws2)
    assert torch.equal(mg.mxfp4_gemm_packed(fp4.pack_fp4(xc), fp4.pack_fp4(wc), xs2, ws2), fast)
    # an in-place write to the quantizer's tensor takes it off the fast list
    xs[5, 2] = 1.5
    assert not fp4.e8m0_exact(xs)
    got = mg.mxfp4_gemm_packed(fp4.pack_fp4(xc), fp4.pack_fp4(wc), xs, ws, out_dtype=torch.float32)
    _same(got, oracle.gemm_promote(oracle.E2M1_VALUES[xc.cpu().numpy()], oracle.E2M1_VALUES[wc.cpu().numpy()],
                                   xs.cpu().numpy(), ws.cpu().numpy()))


def test_nan_scales_stay_on_the_fast_kernel(dev, mods, oracle):
    """A NaN fp32 scale is E8M0 NaN: it does not set the flag, and the output
    is the E8M0 call's (NaN in every output that uses the scale, as the
    reference's multiply makes it; the others unchanged)."""
    C, fp4, mg = mods
    M, N, K = 256, 256, 512
    x = torch.from_numpy(gen.normal(45, (M, K))).to(dev)
    w = torch.from_numpy(gen.normal(46, (N, K), std=0.02)).to(dev)
    xk = fp4.quantize_pack_mxfp4(x)
    wk = fp4.quantize_pack_mxfp4(w)
    ea, eb = xk[1].clone(), wk[1].clone()
    ea[3, 1] = 255
    eb[9, 4] = 255
    want = mg.mxfp4_gemm_packed(xk[0], wk[0], ea, eb, out_dtype=torch.float32)
    sa, sb = fp4.e8m0_to_scale(ea).clone(), fp4.e8m0_to_scale(eb).clone()   # untagged copies
    got = mg.mxfp4_gemm_packed(xk[0], wk[0], sa, sb, out_dtype=torch.float32)
    assert bool(got[3].isnan().all()) and bool(got[:, 9].isnan().all())
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())


def test_special_scales_follow_ieee(dev, mods, oracle):
    """0, negative, +-inf, NaN, subnormal and huge scales: the reference's
    fp32 products, NaN and inf positions included."""
    C, fp4, mg = mods
    rng = np.random.default_rng(3)
    M, N, K = 64, 48, 256
    specials = np.float32([0.0, -2.0, np.inf, -np.inf, np.nan, 1e-40, 1.5, 3.0e38, 2.0 ** -127, 0.75])
    ca, cb = _codes(rng, M, K), _codes(rng, N, K)
    ca[0] = 0
    sa = rng.uniform(0.5, 2, (M, K // 32)).astype(np.float32)
    sb = rng.uniform(0.5, 2, (N, K // 32)).astype(np.float32)
    sa[:len(specials), 3] = specials
    sb[:len(specials), 5] = specials[::-1]
    got = mg.mxfp4_gemm_packed(torch.from_numpy(oracle.pack_fp4(ca)).to(dev),
                               torch.from_numpy(oracle.pack_fp4(cb)).to(dev),
                               torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev),
                               out_dtype=torch.float32)
    want = oracle.gemm_promote(oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb], sa, sb)
    assert np.isnan(want).any() and np.isinf(want).any()
    _same(got, want)


def _e4m3(fp4, dev, codes):
    return fp4.codes_to_e4m3(torch.from_numpy(codes).to(dev))


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (200, 300, 384), (1, 64, 128), (130, 528, 1152), (300, 48, 384)])
def test_fp8_any_scales_match_the_promotion_oracle(dev, mods, oracle, M, N, K):
    """mxfp4_gemm_fp8 with E4M3 operands holding E2M1 values and fp32 scales
    in (-2, 2); b_scale is the reference's [K/32, N].  N % 16 == 0 reads the
    N-contiguous B in place in both kernels; N = 300 transposes it first."""
    C, fp4, mg = mods
    rng = np.random.default_rng(M + 3 * N + K)
    ca, cb = _codes(rng, M, K), _codes(rng, K, N)
    sa = rng.uniform(-2, 2, (M, K // 32)).astype(np.float32)
    sb = rng.uniform(-2, 2, (K // 32, N)).astype(np.float32)
    got = mg.mxfp4_gemm_fp8(_e4m3(fp4, dev, ca), _e4m3(fp4, dev, cb), torch.from_numpy(sa).to(dev),
                            torch.from_numpy(sb).to(dev), out_dtype=torch.float32)
    want = oracle.gemm_promote(oracle.E2M1_VALUES[ca], np.ascontiguousarray(oracle.E2M1_VALUES[cb].T), sa, sb,
                               sb_transposed=True)
    _same(got, want)


def test_fp8_off_grid_operands_within_the_summation_bound(dev, mods, oracle):
    """Finite E4M3 bytes off the E2M1 grid: a 32-term block product then
    spans more bits than fp32 holds, and the matrix cores sum it with an
    internal precision of their own (the reference's docstring puts Hopper's
    FP8 MMA at ~14 bits, mxfp4_gemm.py:7-11), so the comparison with the
    oracle (exact products, one rounding per block) is within 2^-12 of the
    sum of absolute terms, not bit for bit."""
    C, fp4, mg = mods
    M, N, K = 128, 192, 512
    g = torch.Generator(device=dev).manual_seed(5)

    def e4m3(shape):
        x = torch.randint(0, 256, shape, dtype=torch.uint8, device=dev, generator=g)
        return torch.where((x & 0x7F) == 0x7F, x ^ 1, x).view(torch.float8_e4m3fn)
    a, b = e4m3((M, K)), e4m3((K, N))
    sa = (torch.rand((M, K // 32), device=dev, generator=g) * 3 - 1.5)
    sb = (torch.rand((K // 32, N), device=dev, generator=g) * 3 - 1.5)
    got = mg.mxfp4_gemm_fp8(a, b, sa, sb, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    A, B = a.float().cpu().numpy(), np.ascontiguousarray(b.float().cpu().numpy().T)
    san, sbn = sa.cpu().numpy(), sb.cpu().numpy()
    want = oracle.gemm_promote(A, B, san, sbn, sb_transposed=True).astype(np.float64)
    mag = oracle.gemm_promote(np.abs(A), np.abs(B), np.abs(san), np.abs(sbn), sb_transposed=True).astype(np.float64)
    err = float((np.abs(got - want) / mag).max())
    assert err <= 2.0 ** -12, err


@pytest.mark.parametrize("M,N,K,pad", [(256, 256, 256, 0), (130, 400, 1152, 16), (1, 16, 128, 48), (300, 144, 384, 0)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_capi_promotion_reads_n_contiguous_b(dev, mods, oracle, M, N, K, pad, out):
    """lsmx_gemm_mx_promote with op_fmt LSMX_E4M3 | LSMX_B_NCONTIG on B
    [K, N + pad] gives the bits of the same call on B's K-contiguous
    transpose, and the oracle's; N % 16 != 0 and packed operands with the
    bit are refused."""
    C, fp4, mg = mods
    rng = np.random.default_rng(M + N + K + pad)
    ca, cb = _codes(rng, M, K), _codes(rng, K, N + pad)
    sa = rng.uniform(-2, 2, (M, K // 32)).astype(np.float32)
    sb = rng.uniform(-2, 2, (K // 32, N)).astype(np.float32)
    a, b = _e4m3(fp4, dev, ca).view(torch.uint8), _e4m3(fp4, dev, cb).view(torch.uint8)
    bt = b[:, :N].t().contiguous()
    tsa, tsb = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
    code = C.F32 if out == torch.float32 else C.BF16
    c0, c1 = torch.empty((M, N), device=dev, dtype=out), torch.empty((M, N), device=dev, dtype=out)
    C.call("lsmx_gemm_mx_promote", a.data_ptr(), K, tsa.data_ptr(), K // 32, 1, bt.data_ptr(), K, tsb.data_ptr(), 1,
           N, C.E4M3, c0.data_ptr(), code, N, M, N, K, None, 0, C.stream_of(c0))
    C.call("lsmx_gemm_mx_promote", a.data_ptr(), K, tsa.data_ptr(), K // 32, 1, b.data_ptr(), N + pad,
           tsb.data_ptr(), 1, N, C.E4M3 | C.B_NCONTIG, c1.data_ptr(), code, N, M, N, K, None, 0, C.stream_of(c1))
    torch.cuda.synchronize(dev)
    assert torch.equal(c0, c1)
    _same(c1, oracle.gemm_promote(oracle.E2M1_VALUES[ca], np.ascontiguousarray(oracle.E2M1_VALUES[cb][:, :N].T),
                                  sa, sb, sb_transposed=True))
    if M == 1:
        lib = C.load()
        rc = lib.lsmx_gemm_mx_promote(a.data_ptr(), K, tsa.data_ptr(), K // 32, 1, b.data_ptr(), N + pad,
                                      tsb.data_ptr(), 1, N, C.E4M3 | C.B_NCONTIG, c1.data_ptr(), code, N, M, N - 8,
                                      K, None, 0, C.stream_of(c1))
        assert rc == C.ERR_SHAPE and "multiple of 16" in C.last_error()
        rc = lib.lsmx_gemm_mx_promote(a.data_ptr(), K, tsa.data_ptr(), K // 32, 1, b.data_ptr(), N + pad,
                                      tsb.data_ptr(), 1, N, C.CODES_PACKED | C.B_NCONTIG, c1.data_ptr(), code, N, M,
                                      N, K, None, 0, C.stream_of(c1))
        assert rc == C.ERR_DTYPE


def test_capi_flag_gates_the_promotion_launch(dev, mods, oracle):
    """lsmx_gemm_mx_promote: with a NULL flag it computes; with a flag that
    holds another epoch it writes nothing; with the matching epoch it
    computes."""
    C, fp4, mg = mods
    rng = np.random.default_rng(12)
    M, N, K = 130, 70, 256
    ca, cb = _codes(rng, M, K), _codes(rng, N, K)
    sa = rng.uniform(-2, 2, (M, K // 32)).astype(np.float32)
    sb = rng.uniform(-2, 2, (N, K // 32)).astype(np.float32)
    apk, bpk = (torch.from_numpy(oracle.pack_fp4(c)).to(dev) for c in (ca, cb))
    tsa, tsb = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
    want = oracle.gemm_promote(oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb], sa, sb)
    flag = torch.tensor([1234], dtype=torch.int64, device=dev)
    for fl, epoch, computes in ((None, 0, True), (flag, 999, False), (flag, 1234, True)):
        c = torch.full((M, N), -7.0, device=dev)
        C.call("lsmx_gemm_mx_promote", apk.data_ptr(), K // 2, tsa.data_ptr(), K // 32, 1, bpk.data_ptr(), K // 2,
               tsb.data_ptr(), K // 32, 1, C.CODES_PACKED, c.data_ptr(), C.F32, N, M, N, K,
               fl.data_ptr() if fl is not None else None, epoch, C.stream_of(c))
        if computes:
            _same(c, want)
        else:
            assert bool((c == -7.0).all())


@pytest.mark.parametrize("bad", [False, True])
def test_scale_batch_matches_single_conversions_and_flags(dev, mods, oracle, bad):
    """lsmx_scale_to_e8m0_batch over three tensors (row-major and [blocks,
    rows] inputs, partial 64 x 16 tiles, one empty) writes the bytes
    lsmx_scale_to_e8m0 writes, and writes its epoch to the flag exactly when
    a scale is neither a power of two nor a NaN."""
    C, fp4, mg = mods
    rng = np.random.default_rng(21 + bad)
    shapes = [(300, 40, False), (72, 300, True), (0, 8, False)]
    items = (C.E8m0Item * len(shapes))()
    keep, outs, refs = [], [], []
    for k, (r, cl, tin) in enumerate(shapes):
        s = np.ldexp(np.ones((r, cl)), rng.integers(-127, 128, size=(r, cl))).astype(np.float32)
        if r and cl:
            s[2, 3] = np.nan          # E8M0 has NaN: never flagged
        if bad and k == 1:
            s[17, 5] = 1.5
        x = torch.from_numpy(s).to(dev)
        orows, blocks = (cl, r) if tin else (r, cl)
        out = torch.full((max(blocks // 4, 1), orows, 4), 7, dtype=torch.uint8, device=dev)
        ref = out.clone()
        items[k] = C.E8m0Item(x.data_ptr(), r, cl, cl, C.E8M0_IN_T if tin else 0, out.data_ptr(), orows)
        if r and cl:
            C.call("lsmx_scale_to_e8m0", x.data_ptr(), r, cl, cl, C.E8M0_OUT_KMAJOR | (C.E8M0_IN_T if tin else 0),
                   ref.data_ptr(), orows, C.stream_of(ref))
        keep.append(x)
        outs.append(out)
        refs.append(ref)
    flag = torch.tensor([5], dtype=torch.int64, device=dev)
    C.call("lsmx_scale_to_e8m0_batch", items, len(shapes), flag.data_ptr(), 77, C.stream_of(flag))
    for out, ref in zip(outs, refs):
        assert torch.equal(out, ref)
    assert int(flag.item()) == (77 if bad else 5)


def test_promotion_at_4096_cubed_sampled(dev, mods, oracle):
    """The promotion kernel over a 4096^3 product with random scales, checked
    on sampled rows and columns (the oracle on the sampled operand rows)."""
    C, fp4, mg = mods
    M = N = K = 4096
    g = torch.Generator(device=dev).manual_seed(9)
    apk = torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, device=dev, generator=g)
    bpk = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=g)
    sa = torch.rand((M, K // 32), device=dev, generator=g) * 2 - 1
    sb = torch.rand((N, K // 32), device=dev, generator=g) * 2 - 1
    got = mg.mxfp4_gemm_packed(apk, bpk, sa, sb, out_dtype=torch.float32)
    rows = np.array([0, 1, 127, 128, 2049, 4095])
    cols = np.array([0, 5, 255, 256, 3000, 4095])
    A = oracle.fp4_values(apk[rows].cpu().numpy())
    B = oracle.fp4_values(bpk[cols].cpu().numpy())
    want = oracle.gemm_promote(A, B, sa[rows].cpu().numpy(), sb[cols].cpu().numpy())
    _same(got[rows][:, cols], want)
