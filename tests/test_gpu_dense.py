"""GPU parity of the dense GEMM family (dual_gemm.py) and of mxfp4_gemm_fp8.

Closed forms pin these: the reference's operands hold integer q-grid values
(fp4.codes_to_q, |q| <= 12), so every product and every partial sum up to
2^24 is exact in fp32 and the result must equal the fp64 integer product bit
for bit (train_step.py:118-137, bench.py:44-57).  Random-normal operands are
checked against fp64 with max|c - ref| / max|ref| <= 1e-5 (fp32 output) and
<= 1e-2 (bf16 output), the reference's own metric (bench.py:71).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float8_e4m3fn]


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import _capi, dual_gemm, fp4, mxfp4_gemm
    return dual_gemm, mxfp4_gemm, fp4, _capi


def q_grid(rng, shape):
    """Integer grid values of random E2M1 codes, negative zero excluded (fp4.py:37-41)."""
    pick = np.array([0, 1, 2, 3, 4, 6, 8, 12, -1, -2, -3, -4, -6, -8, -12], dtype=np.float64)
    return pick[rng.integers(0, 15, shape)]


def on(dev, x, dt):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dt).to(dev)


def f64(t):
    return t.float().cpu().numpy().astype(np.float64)


SHAPES = [(256, 256, 256), (200, 136, 192), (1, 1, 64), (130, 70, 128), (384, 512, 1024)]


@pytest.mark.parametrize("dt", DTYPES, ids=str)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_integer_grid_exact(dev, mods, dt, M, N, K):
    dg = mods[0]
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a, b = q_grid(rng, (M, K)), q_grid(rng, (K, N))
    got = dg.gemm(on(dev, a, dt), on(dev, b, dt))
    assert got.dtype == torch.float32 and got.shape == (M, N)
    assert np.array_equal(f64(got), a @ b)


@pytest.mark.parametrize("dt", DTYPES, ids=str)
@pytest.mark.parametrize("shared", [False, True], ids=["b1!=b2", "shared-W"])
@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (190, 300, 256), (64, 33, 64)])
def test_dual_separate_integer_grid_exact(dev, mods, dt, shared, M, N, K):
    """train_step.py:52-53 (`dual_separate(a1, a2, W, W)`) and dual_gemm.py:244-255."""
    dg = mods[0]
    rng = np.random.default_rng(K + M)
    a1, a2 = q_grid(rng, (M, K)), q_grid(rng, (M, K))
    b1 = q_grid(rng, (K, N))
    b2 = b1 if shared else q_grid(rng, (K, N))
    tb1 = on(dev, b1, dt)
    tb2 = tb1 if shared else on(dev, b2, dt)
    c1, c2 = dg.dual_separate(on(dev, a1, dt), on(dev, a2, dt), tb1, tb2)
    assert np.array_equal(f64(c1), a1 @ b1) and np.array_equal(f64(c2), a2 @ b2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
def test_ring_kernel_walks_several_tiles_per_workgroup(dev, mods, dt):
    """More 256 x 256 tiles than CUs: the persistent ring kernel's workgroups
    take several tiles each, across both problems of dual_separate and both K
    halves of dual_packed, with ragged edge tiles; exact on the integer grid."""
    dg = mods[0]
    rng = np.random.default_rng(77)
    M, N, K = 4352 + 40, 4352 + 24, 128   # 18 x 18 = 324 tiles
    a1, a2 = q_grid(rng, (M, K)), q_grid(rng, (M, K))
    b1, b2 = q_grid(rng, (K, N)), q_grid(rng, (K, N))
    ta1, ta2, tb1, tb2 = on(dev, a1, dt), on(dev, a2, dt), on(dev, b1, dt), on(dev, b2, dt)
    r1, r2 = a1 @ b1, a2 @ b2
    assert np.array_equal(f64(dg.gemm(ta1, tb1)), r1)
    c1, c2 = dg.dual_separate(ta1, ta2, tb1, tb2)
    assert np.array_equal(f64(c1), r1) and np.array_equal(f64(c2), r2)
    s1, s2 = dg.dual_separate(ta1, ta2, tb1, tb1)
    assert np.array_equal(f64(s1), r1) and np.array_equal(f64(s2), a2 @ b1)
    assert np.array_equal(f64(dg.dual_packed(ta1, ta2, tb1, tb2)), r1 + r2)


@pytest.mark.parametrize("dt", DTYPES, ids=str)
@pytest.mark.parametrize("shared", [False, True], ids=["b1!=b2", "shared-W"])
def test_dual_packed_is_concatenated_k_gemm(dev, mods, dt, shared):
    """One accumulator: acc = A1.B1 + A2.B2 (dual_gemm.py:42-72), equal to the
    GEMM over the K-concatenation [A1 | A2] . [B1; B2] on the integer grid,
    where every order of the additions is exact (the order itself is pinned
    by tests/test_gpu_scales.py)."""
    dg = mods[0]
    rng = np.random.default_rng(5)
    M, N, K = 160, 200, 320
    a1, a2 = q_grid(rng, (M, K)), q_grid(rng, (M, K))
    b1 = q_grid(rng, (K, N))
    b2 = b1 if shared else q_grid(rng, (K, N))
    tb1 = on(dev, b1, dt)
    tb2 = tb1 if shared else on(dev, b2, dt)
    acc = dg.dual_packed(on(dev, a1, dt), on(dev, a2, dt), tb1, tb2)
    assert np.array_equal(f64(acc), a1 @ b1 + a2 @ b2)
    cat = dg.gemm(on(dev, np.concatenate([a1, a2], 1), dt), on(dev, np.concatenate([b1, b2], 0), dt))
    assert torch.equal(acc, cat)


def test_packed_slots_round_trip_where_exact(dev, mods):
    """train_step.py:58-59 / bench.py:122-128: with 2*bits(144K)+1 <= 24 the
    packed accumulator splits back into both products exactly (K = 16, padded
    to 64 with zeros as bench.py:139-149 does)."""
    dg = mods[0]
    rng = np.random.default_rng(11)
    k, kp, M, N = 16, 64, 256, 256
    s = dg.slot_offset(k)
    q = [q_grid(rng, sh) for sh in ((M, k), (M, k), (k, N), (k, N))]
    # every partial sum, in any order, stays an integer below 2^24
    bound = np.abs(q[0]) @ np.abs(q[2]) + 2.0 ** s * (np.abs(q[1]) @ np.abs(q[3]))
    assert bound.max() < 2 ** 24
    pad = [np.pad(q[0], ((0, 0), (0, kp - k))), np.pad(q[1], ((0, 0), (0, kp - k))),
           np.pad(q[2], ((0, kp - k), (0, 0))), np.pad(q[3], ((0, kp - k), (0, 0)))]
    acc = dg.dual_packed(on(dev, pad[0], torch.bfloat16), on(dev, pad[1] * 2.0 ** s, torch.bfloat16),
                         on(dev, pad[2], torch.bfloat16), on(dev, pad[3], torch.bfloat16))
    ref = q[0] @ q[2] + (q[1] @ q[3]) * 2.0 ** s
    assert np.array_equal(f64(acc), ref)          # the accumulator itself is exact
    g1, g2 = dg.unpack_dual(acc.double(), s)
    assert np.array_equal(g1.cpu().numpy(), q[0] @ q[2]) and np.array_equal(g2.cpu().numpy(), q[1] @ q[3])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float8_e4m3fn], ids=str)
@pytest.mark.parametrize("splits", [2, 4, 8])
def test_splitk_integer_grid_exact(dev, mods, dt, splits):
    """dual_gemm.py:258-289: partials over K slices, atomic adds into zeros."""
    dg = mods[0]
    rng = np.random.default_rng(splits)
    M, N, K = 200, 260, 1024
    a1, a2 = q_grid(rng, (M, K)), q_grid(rng, (M, K))
    b1, b2 = q_grid(rng, (K, N)), q_grid(rng, (K, N))
    t = [on(dev, x, dt) for x in (a1, a2, b1, b2)]
    o1, o2 = dg.splitk_separate(*t, splits=splits)
    assert np.array_equal(f64(o1), a1 @ b1) and np.array_equal(f64(o2), a2 @ b2)
    acc = dg.splitk_packed(*t, splits)
    assert np.array_equal(f64(acc), a1 @ b1 + a2 @ b2)
    s1, s2 = dg.splitk_separate(t[0], t[1], t[2], t[2], splits=splits)   # shared weight
    assert np.array_equal(f64(s1), a1 @ b1) and np.array_equal(f64(s2), a2 @ b1)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
def test_splitk_with_tiles_for_every_cu(dev, mods, dt):
    """An output with at least one 256 x 256 tile per CU runs the whole K per
    tile (no slices, no atomics); the sums are those of the sliced form,
    exact on the integer grid."""
    dg = mods[0]
    assert dg._launch_splits(torch.empty((4096, 64), device=dev, dtype=dt), 4096, 2, 4) == 1
    assert dg._launch_splits(torch.empty((200, 64), device=dev, dtype=dt), 260, 2, 4) == 4
    rng = np.random.default_rng(79)
    M, N, K = 4096, 4352 + 24, 256
    a1, a2 = q_grid(rng, (M, K)), q_grid(rng, (M, K))
    b1, b2 = q_grid(rng, (K, N)), q_grid(rng, (K, N))
    t = [on(dev, x, dt) for x in (a1, a2, b1, b2)]
    r1, r2 = a1 @ b1, a2 @ b2
    o1, o2 = dg.splitk_separate(*t, splits=4)
    assert np.array_equal(f64(o1), r1) and np.array_equal(f64(o2), r2)
    assert np.array_equal(f64(dg.splitk_packed(*t, 2)), r1 + r2)


def test_splitk_keeps_reference_assert(dev, mods):
    dg = mods[0]
    a = torch.zeros((128, 192), device=dev, dtype=torch.bfloat16)
    b = torch.zeros((192, 128), device=dev, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="K must divide splits\\*BK"):
        dg.splitk_separate(a, a, b, b, splits=8)
    with pytest.raises(AssertionError, match="K must be a multiple of 64"):
        dg.gemm(a[:, :100], b[:100])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
def test_random_normal_against_fp64(dev, mods, dt):
    dg = mods[0]
    g = torch.Generator().manual_seed(3)
    M, N, K = 512, 384, 2048
    a, b = torch.randn((M, K), generator=g).to(dt), torch.randn((K, N), generator=g).to(dt)
    ref = a.double() @ b.double()
    c = dg.gemm(a.to(dev), b.to(dev)).double().cpu()
    assert ((c - ref).abs().max() / ref.abs().max()).item() <= 1e-5
    c1, c2 = dg.dual_separate(a.to(dev), a.to(dev), b.to(dev), b.to(dev))
    assert torch.equal(c1, c2) and torch.equal(c1.double().cpu(), c)


def test_transposed_view_operand_is_read_in_place(dev, mods):
    """b = W.t() of a K-contiguous W [N, K] needs no transposed copy; the
    result must equal the one through a copied N-contiguous b."""
    dg = mods[0]
    rng = np.random.default_rng(9)
    M, N, K = 96, 160, 256
    a, w = q_grid(rng, (M, K)), q_grid(rng, (N, K))
    ta, tw = on(dev, a, torch.bfloat16), on(dev, w, torch.bfloat16)
    c_view = dg.gemm(ta, tw.t())
    c_copy = dg.gemm(ta, tw.t().contiguous())
    assert torch.equal(c_view, c_copy) and np.array_equal(f64(c_view), a @ w.T)


def test_empty_and_zero_k(dev, mods):
    dg, mg = mods[0], mods[1]
    a = torch.zeros((0, 64), device=dev, dtype=torch.bfloat16)
    b = torch.zeros((64, 8), device=dev, dtype=torch.bfloat16)
    assert dg.gemm(a, b).shape == (0, 8)
    z = dg.gemm(torch.ones((4, 0), device=dev, dtype=torch.bfloat16), torch.ones((0, 8), device=dev,
                                                                                   dtype=torch.bfloat16))
    assert z.shape == (4, 8) and not z.any()
    f8 = torch.zeros((4, 0), device=dev, dtype=torch.uint8).view(torch.float8_e4m3fn)
    z = mg.mxfp4_gemm_fp8(f8, f8.t(), torch.ones((4, 0), device=dev), torch.ones((0, 4), device=dev),
                          out_dtype=torch.float32)
    assert z.shape == (4, 4) and not z.any()
    # the f4 x f4 and weight-only GEMMs: K = 0 gives zeros (no K iteration),
    # an empty side an empty output
    pk, e8 = torch.zeros((4, 0), device=dev, dtype=torch.uint8), torch.zeros((4, 0), device=dev, dtype=torch.uint8)
    z = mg.mxfp4_gemm_packed(pk, pk, e8, e8)
    assert z.shape == (4, 4) and not z.any()
    z = mg.mxfp4_gemm_packed(pk, pk, torch.ones((4, 0), device=dev), torch.ones((4, 0), device=dev))
    assert z.shape == (4, 4) and not z.any()
    z = mg.mxfp4_gemm_bf16(torch.ones((3, 0), device=dev, dtype=torch.bfloat16), pk, e8)
    assert z.shape == (3, 4) and not z.any()
    z = mg.mxfp4_gemm_bf16(torch.ones((3, 0), device=dev), pk, e8, out_dtype=torch.float32)
    assert z.shape == (3, 4) and not z.any()
    z0, z1 = dg.dual_mxfp4(torch.ones((3, 0), device=dev, dtype=torch.bfloat16),
                           torch.ones((3, 0), device=dev, dtype=torch.bfloat16), pk, e8)
    assert z0.shape == z1.shape == (3, 4) and not z0.any() and not z1.any()
    assert mg.mxfp4_gemm_packed(torch.zeros((0, 64), device=dev, dtype=torch.uint8),
                                torch.zeros((8, 64), device=dev, dtype=torch.uint8),
                                torch.zeros((0, 4), device=dev, dtype=torch.uint8),
                                torch.zeros((8, 4), device=dev, dtype=torch.uint8)).shape == (0, 8)


@pytest.mark.parametrize("elem", [1, 2, 4])
@pytest.mark.parametrize("rows,cols,pad", [(1, 1, 5), (33, 65, 5), (256, 96, 5), (1000, 3, 5), (128, 192, 0),
                                           (192, 320, 0), (100, 80, 0), (512, 640, 0), (200, 130, 0)])
def test_transpose_exact(dev, mods, elem, rows, cols, pad):
    """Element-by-element (pad 5: unaligned rows) and 16-byte (pad 0) paths, full and edge tiles; the full
    tiles transpose blocks of 4 bytes, 2 halves or 1 dword in registers."""
    C = mods[3]
    dt = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[elem]
    x = torch.randint(0, 100, (rows, cols + pad), dtype=torch.int32).to(dt).to(dev)[:, :cols]
    y = torch.full((cols, rows), -1, dtype=dt, device=dev)
    C.call("lsmx_transpose", x.data_ptr(), elem, rows, cols, x.stride(0), y.data_ptr(), rows, C.stream_of(y))
    assert torch.equal(y.cpu(), x.t().cpu())


@pytest.mark.parametrize("tin", [False, True])
@pytest.mark.parametrize("misalign", [0, 1])
@pytest.mark.parametrize("pad", [3, 4])
def test_scale_to_e8m0_layouts(dev, mods, oracle, tin, misalign, pad):
    """lsmx_scale_to_e8m0 in all four layouts: powers of two 2^-127 .. 2^127 give the oracle's exponent bytes,
    anything else 0xFF; the K-major output (four blocks per thread, whole-dword stores, byte stores at an odd
    address) holds the row-major output's bytes regrouped, and no byte outside it is written.  pad = 4 gives
    16-byte aligned fp32 rows, which the row-major-in, K-major-out form converts through an LDS tile (64 rows
    x 16 groups; 300 rows and 10 groups leave both edges partial)."""
    C = mods[3]
    rng = np.random.default_rng(11)
    orows, blocks = 300, 40
    s = np.ldexp(np.ones((orows, blocks)), rng.integers(-127, 128, size=(orows, blocks))).astype(np.float32)
    bad = rng.random((orows, blocks)) < 0.05
    s[bad] = rng.choice(np.float32([1.5, -2.0, 0.0, np.inf, 3.0]), size=int(bad.sum()))
    want = oracle.scale_to_e8m0(s)
    want[bad] = 0xFF
    src = np.ascontiguousarray(s.T) if tin else s      # IN_T: element (block, row)
    lds = src.shape[1] + pad
    x = torch.zeros((src.shape[0], lds), dtype=torch.float32)
    x[:, :src.shape[1]] = torch.from_numpy(src)
    x = x.to(dev)
    lay = C.E8M0_IN_T if tin else 0
    ldo = blocks + 5
    y = torch.full((orows * ldo,), 7, dtype=torch.uint8, device=dev)
    C.call("lsmx_scale_to_e8m0", x.data_ptr(), src.shape[0], src.shape[1], lds, lay, y.data_ptr(), ldo,
           C.stream_of(y))
    yr = y.cpu().numpy().reshape(orows, ldo)
    assert np.array_equal(yr[:, :blocks], want) and (yr[:, blocks:] == 7).all()
    ldk = orows + 2
    buf = torch.full((misalign + blocks // 4 * ldk * 4,), 7, dtype=torch.uint8, device=dev)
    C.call("lsmx_scale_to_e8m0", x.data_ptr(), src.shape[0], src.shape[1], lds, lay | C.E8M0_OUT_KMAJOR,
           buf.data_ptr() + misalign, ldk, C.stream_of(buf))
    raw = buf.cpu().numpy()
    yk = raw[misalign:].reshape(blocks // 4, ldk, 4)
    assert np.array_equal(yk[:, :orows, :], want.reshape(orows, blocks // 4, 4).transpose(1, 0, 2))
    assert (yk[:, orows:, :] == 7).all() and (raw[:misalign] == 7).all()


# ----------------------------------------------------------- mxfp4_gemm_fp8
def e4m3_of_codes(dev, fp4, codes):
    return fp4.codes_to_e4m3(torch.from_numpy(codes).to(dev))


def test_fp8_unit_scales_bit_exact(dev, mods, oracle):
    """bench.py:41-57: random codes, unit scales, K = 128 -> C == (qa @ qb) / 4."""
    _, mg, fp4, _ = mods
    rng = np.random.default_rng(0)
    pick = np.array([c for c in range(16) if c != 8], dtype=np.uint8)
    ca, cb = pick[rng.integers(0, 15, (256, 128))], pick[rng.integers(0, 15, (128, 256))]
    sa = torch.ones((256, 4), device=dev)
    sb = torch.ones((4, 256), device=dev)
    got = mg.mxfp4_gemm_fp8(e4m3_of_codes(dev, fp4, ca), e4m3_of_codes(dev, fp4, cb), sa, sb,
                            out_dtype=torch.float32)
    qa, qb = oracle.E2M1_Q[ca].astype(np.float64), oracle.E2M1_Q[cb].astype(np.float64)
    assert np.array_equal(f64(got), (qa @ qb) / 4.0)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (200, 136, 384), (1, 300, 128)])
def test_fp8_random_codes_and_scales(dev, mods, oracle, out_dtype, M, N, K):
    """cuda/mxfp4_mma_gemm.cu:204-252: codes 0..15 (incl. -0), scales 2^[-3,3]."""
    _, mg, fp4, _ = mods
    rng = np.random.default_rng(M + K)
    ca, cb = rng.integers(0, 16, (M, K), dtype=np.uint8), rng.integers(0, 16, (K, N), dtype=np.uint8)
    sa = np.exp2(rng.integers(-3, 4, (M, K // 32))).astype(np.float32)
    sb = np.exp2(rng.integers(-3, 4, (K // 32, N))).astype(np.float32)
    ref = oracle.dequantize_mxfp4(ca, sa).astype(np.float64) @ \
        oracle.dequantize_mxfp4(cb.T.copy(), sb.T.copy()).astype(np.float64).T
    got = mg.mxfp4_gemm_fp8(e4m3_of_codes(dev, fp4, ca), e4m3_of_codes(dev, fp4, cb),
                            torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev), out_dtype=out_dtype)
    assert got.dtype == out_dtype and got.shape == (M, N)
    tol = 1e-6 if out_dtype == torch.float32 else 1e-2
    assert oracle.max_rel(f64(got), ref) <= tol
    # E8M0 byte scales of the same shapes give the same result
    got8 = mg.mxfp4_gemm_fp8(e4m3_of_codes(dev, fp4, ca), e4m3_of_codes(dev, fp4, cb),
                             torch.from_numpy(oracle.scale_to_e8m0(sa)).to(dev),
                             torch.from_numpy(oracle.scale_to_e8m0(sb)).to(dev), out_dtype=out_dtype)
    assert torch.equal(got, got8)


def test_fp8_quantized_randn_matches_fp64(dev, mods, oracle):
    """bench.py:60-73: randn -> quantize (A along K, B transposed along K) ->
    codes_to_e4m3 -> mxfp4_gemm_fp8 vs the fp64 reference, rel < 1e-5; the
    packed kernel on the same operands agrees."""
    _, mg, fp4, _ = mods
    g = torch.Generator().manual_seed(7)
    M, N, K = 384, 256, 1024
    a, b = torch.randn((M, K), generator=g), torch.randn((K, N), generator=g)
    a_codes, a_scale = oracle.quantize_mxfp4(a.numpy())
    bt_codes, bt_scale = oracle.quantize_mxfp4(b.t().contiguous().numpy())
    ref = oracle.dequantize_mxfp4(a_codes, a_scale).astype(np.float64) @ \
        oracle.dequantize_mxfp4(bt_codes, bt_scale).astype(np.float64).T
    c = mg.mxfp4_gemm_fp8(e4m3_of_codes(dev, fp4, a_codes), e4m3_of_codes(dev, fp4, bt_codes.T.copy()),
                          torch.from_numpy(a_scale).to(dev), torch.from_numpy(bt_scale.T.copy()).to(dev),
                          out_dtype=torch.float32)
    assert oracle.max_rel(f64(c), ref) <= 1e-5
    cp = mg.mxfp4_gemm_packed(torch.from_numpy(oracle.pack_fp4(a_codes)).to(dev),
                              torch.from_numpy(oracle.pack_fp4(bt_codes)).to(dev),
                              torch.from_numpy(a_scale).to(dev), torch.from_numpy(bt_scale).to(dev),
                              out_dtype=torch.float32)
    assert oracle.max_rel(f64(cp), ref) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (300, 200, 384), (1, 256, 128), (2048, 2048, 2048)])
def test_fp8_kmajor_kernel_matches_rowmajor_kernel(dev, mods, M, N, K):
    """The persistent 256 x 256 E4M3 kernel (K-major scales) and the 128 x 128
    one (row-major scales) accumulate the same 64-deep K-steps in the same
    order: identical bits, on random E4M3 bytes (finite) and scales 2^[-4,4]."""
    C = mods[3]
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    def e4m3(rows):
        x = torch.randint(0, 256, (rows, K), dtype=torch.uint8, device=dev, generator=g)
        return torch.where((x & 0x7F) == 0x7F, x ^ 1, x)          # no NaN encodings
    a, bt = e4m3(M), e4m3(N)
    ea = torch.randint(123, 132, (M, K // 32), dtype=torch.uint8, device=dev, generator=g)
    eb = torch.randint(123, 132, (N, K // 32), dtype=torch.uint8, device=dev, generator=g)
    eak = ea.reshape(M, K // 128, 4).transpose(0, 1).contiguous()
    ebk = eb.reshape(N, K // 128, 4).transpose(0, 1).contiguous()
    out = []
    for fmt, sa, sb, la, lb in ((C.SCALE_E8M0, ea, eb, K // 32, K // 32), (C.SCALE_E8M0_KMAJOR, eak, ebk, M, N)):
        c = torch.full((M, N), float("nan"), device=dev)
        C.call("lsmx_gemm_f8f8", a.data_ptr(), K, sa.data_ptr(), la, bt.data_ptr(), K, sb.data_ptr(), lb, fmt,
               c.data_ptr(), C.F32, N, M, N, K, C.stream_of(c))
        out.append(c)
    assert not out[1].isnan().any()
    assert torch.equal(out[0], out[1])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("M,N,K,pad", [(256, 256, 64, 0), (300, 520, 192, 8), (37, 40, 128, 24), (1, 264, 64, 8),
                                       (512, 1024, 1024, 0)])
def test_n_contiguous_b_matches_transposed_b(dev, mods, dt, mode, M, N, K, pad):
    """lsmx_gemm_dense_nb (B [K, ldb] N-contiguous, transposing LDS reads)
    gives lsmx_gemm_dense's bits on B's transpose: the same sums in the same
    order, on random data where the order shows.  Ragged tiles (columns and
    rows past N and M), padded B rows (ldb > N), every mode; N % 8 != 0 is
    refused (dual_gemm then transposes B, as before)."""
    from lockstep_amd import _capi as C
    g = torch.Generator(device=dev).manual_seed(M + N + K + mode)
    a = [torch.randn((M, K), device=dev, generator=g).to(dt) for _ in range(2)]
    b = [torch.randn((K, N + pad), device=dev, generator=g).to(dt)[:, :N] for _ in range(2)]
    bt = [x.t().contiguous() for x in b]
    code = C.BF16 if dt == torch.bfloat16 else C.F16
    outs = []
    for nb in (False, True):
        c = [torch.zeros((M, N), device=dev) for _ in range(2)]
        if nb:
            args = (a[0].data_ptr(), a[1].data_ptr(), K, b[0].data_ptr(), b[1].data_ptr(), N + pad, code, mode,
                    c[0].data_ptr(), c[1].data_ptr(), N, M, N, K, C.stream_of(c[0]))
            C.call("lsmx_gemm_dense_nb", *args)
        else:
            C.call("lsmx_gemm_dense", a[0].data_ptr(), a[1].data_ptr(), K, bt[0].data_ptr(), bt[1].data_ptr(), K,
                   code, mode, c[0].data_ptr(), c[1].data_ptr(), N, M, N, K, 1, C.stream_of(c[0]))
        outs.append(c)
    torch.cuda.synchronize(dev)
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)
    if mode == 0 and M == 1:
        rc = C.load().lsmx_gemm_dense_nb(a[0].data_ptr(), None, K, b[0].data_ptr(), None, N + pad, code, 0,
                                         outs[1][0].data_ptr(), None, N, M, N - 1, K, C.stream_of(outs[1][0]))
        assert rc == C.ERR_SHAPE and "multiple of 8" in C.last_error()
    ref = a[0].double() @ b[0].double() + (a[1].double() @ b[1].double() if mode == 1 else 0)
    assert (outs[1][0].double() - ref).abs().max() <= 1e-5 * ref.abs().max()


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,pad", [(256, 256, 128, 0), (300, 528, 384, 16), (37, 48, 256, 32), (1, 272, 128, 0),
                                       (512, 1024, 2048, 0)])
def test_fp8_n_contiguous_b_matches_transposed_b(dev, mods, M, N, K, pad, out_dtype):
    """lsmx_gemm_f8f8_nb (E4M3 B [K, ldb] N-contiguous, transposing LDS reads)
    gives lsmx_gemm_f8f8's bits on B's transpose, with K-major E8M0 scales of
    random exponents; ragged tiles and padded rows; N % 16 != 0 is refused
    (mxfp4_gemm_fp8 then transposes B, as before)."""
    from lockstep_amd import _capi as C
    from lockstep_amd import fp4
    _, mg = mods[0], mods[1]
    g = torch.Generator(device=dev).manual_seed(M * 3 + N + K)
    a = fp4.codes_to_e4m3(torch.randint(0, 16, (M, K), device=dev, generator=g).to(torch.uint8)).view(torch.uint8)
    b = fp4.codes_to_e4m3(torch.randint(0, 16, (K, N + pad), device=dev, generator=g).to(torch.uint8)).view(
        torch.uint8)[:, :N]
    bt = b.t().contiguous()
    sa = torch.randint(120, 134, (K // 128, M, 4), device=dev, generator=g).to(torch.uint8)
    sb = torch.randint(120, 134, (K // 128, N, 4), device=dev, generator=g).to(torch.uint8)
    code = {torch.float32: C.F32, torch.bfloat16: C.BF16}[out_dtype]
    c0 = torch.empty((M, N), device=dev, dtype=out_dtype)
    c1 = torch.empty_like(c0)
    C.call("lsmx_gemm_f8f8", a.data_ptr(), K, sa.data_ptr(), M, bt.data_ptr(), K, sb.data_ptr(), N,
           C.SCALE_E8M0_KMAJOR, c0.data_ptr(), code, N, M, N, K, C.stream_of(c0))
    C.call("lsmx_gemm_f8f8_nb", a.data_ptr(), K, sa.data_ptr(), M, b.data_ptr(), N + pad, sb.data_ptr(), N,
           c1.data_ptr(), code, N, M, N, K, C.stream_of(c1))
    torch.cuda.synchronize(dev)
    assert torch.equal(c0, c1)
    # the Python wrapper takes the in-place path for E8M0 scales and gives the same bits
    b_s = sb.permute(0, 2, 1).reshape(K // 32, N)          # [K/32, N] row-major E8M0 of the same scales
    a_s = sa.permute(1, 0, 2).reshape(M, K // 32)
    got = mg.mxfp4_gemm_fp8(a.view(torch.float8_e4m3fn), b.view(torch.float8_e4m3fn), a_s, b_s, out_dtype=out_dtype)
    assert torch.equal(got, c1)
    if M == 1:
        rc = C.load().lsmx_gemm_f8f8_nb(a.data_ptr(), K, sa.data_ptr(), M, b.data_ptr(), N + pad, sb.data_ptr(), N,
                                        c1.data_ptr(), code, N, M, N - 8, K, C.stream_of(c1))
        assert rc == C.ERR_SHAPE and "multiple of 16" in C.last_error()
