"""GPU parity of the quantize / pack / unpack / dequantize / E4M3 kernels.

Bar: bit-exact.  Each kernel result is compared byte for byte with the CPU
oracle on the same input, and the quantizer also against the digests the
reference fp4.py produced (tests/golden/).
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def to_dev(x: np.ndarray, dtype: str, dev):
    if dtype == "bf16":
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    if dtype == "f16":
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.float16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


@pytest.fixture(scope="module")
def fp4mod(dev):
    from lockstep_amd import fp4
    return fp4


def test_quantize_matches_reference_golden(dev, fp4mod):
    """GPU codes/scales digest-equal to the reference fp4.py's on the golden inputs."""
    from .test_oracle import golden_inputs
    cases = json.loads((GOLD / "fp4_golden.json").read_text())["cases"]
    for name, x in golden_inputs().items():
        c = cases[name]
        xt = to_dev(x, c["dtype"], dev)
        codes, scale = fp4mod.quantize_mxfp4(xt, c["block"])
        codes, scale = codes.cpu().numpy(), scale.cpu().numpy()
        assert sha(codes) == c["codes_sha256"], name
        assert sha(scale.view(np.uint32)) == c["scale_sha256"], name


def test_round_all_bf16_patterns_matches_reference(dev, fp4mod):
    arrays = np.load(GOLD / "fp4_golden.npz")
    allbf = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    got = fp4mod._round_to_e2m1(torch.from_numpy(allbf.copy()).to(dev)).cpu().numpy()
    assert np.array_equal(got, arrays["round_all_bf16__codes"])
    # bf16 bit patterns built directly (a float32 -> bf16 cast would canonicalize NaNs)
    bits = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16).copy())
    got16 = fp4mod._round_to_e2m1(bits.view(torch.bfloat16).to(dev)).cpu().numpy()
    assert np.array_equal(got16, arrays["round_all_bf16__codes"])


SHAPES = [(1, 32), (3, 96), (7, 1056), (64, 4096), (257, 512), (1000, 64)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("block", [32, 16])
def test_quantize_packed_e8m0_matches_oracle(dev, fp4mod, oracle, dtype, block):
    for i, (rows, K) in enumerate(SHAPES):
        if K % block:
            continue
        x = gen.student_t3(100 + i, (rows, K), scale=0.05)
        if dtype == "bf16":
            xh = gen.to_bf16_bits(x)
            ref_codes, ref_scale = oracle.quantize_mxfp4(xh, block, "bf16")
        elif dtype == "f16":
            xh = x.astype(np.float16).view(np.uint16)
            ref_codes, ref_scale = oracle.quantize_mxfp4(xh, block, "f16")
        else:
            xh = x
            ref_codes, ref_scale = oracle.quantize_mxfp4(x, block)
        xt = to_dev(xh, dtype, dev)
        packed, e8 = fp4mod.quantize_pack_mxfp4(xt, block)
        assert np.array_equal(packed.cpu().numpy(), oracle.pack_fp4(ref_codes)), (rows, K)
        assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(ref_scale)), (rows, K)
        codes, scale = fp4mod.quantize_mxfp4(xt, block)
        assert np.array_equal(codes.cpu().numpy(), ref_codes), (rows, K)
        assert np.array_equal(scale.cpu().numpy().view(np.uint32), ref_scale.view(np.uint32))


def test_quantize_strided_rows_and_leading_dims(dev, fp4mod, oracle):
    x = gen.normal(31, (2, 5, 8, 256))
    codes, scale = fp4mod.quantize_mxfp4(to_dev(x, "f32", dev))
    rc, rs = oracle.quantize_mxfp4(x)
    assert codes.shape == (2, 5, 8, 256) and scale.shape == (2, 5, 8, 8)
    assert np.array_equal(codes.cpu().numpy(), rc)
    big = torch.from_numpy(gen.normal(32, (64, 1024))).to(dev)
    view = big[:, 256:768]                                   # row stride 1024, offset 1 KiB
    pk, e8 = fp4mod.quantize_pack_mxfp4(view)
    rc, rs = oracle.quantize_mxfp4(view.cpu().numpy())
    assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc))
    assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(rs))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("block", [32, 16])
def test_quantize_transposed_axis_matches_oracle(dev, fp4mod, oracle, dtype, block):
    for (K, N) in [(32, 1), (64, 300), (1024, 96), (4096, 257), (512, 384)]:   # the last on whole 128 x 128 tiles
        if K % block:
            continue
        x = gen.normal(41 + K, (K, N), std=0.02)
        if dtype == "bf16":
            xh = gen.to_bf16_bits(x)
            rc, rs = oracle.quantize_mxfp4(np.ascontiguousarray(xh.T), block, "bf16")
        else:
            xh = x
            rc, rs = oracle.quantize_mxfp4(np.ascontiguousarray(x.T), block)
        xt = to_dev(xh, dtype, dev)
        pk, e8 = fp4mod.quantize_mxfp4_t(xt, block)
        assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc)), (K, N)
        assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(rs)), (K, N)
        codes, scale = fp4mod.quantize_mxfp4_t(xt, block, packed=False, e8m0=False)
        assert np.array_equal(codes.cpu().numpy(), rc)
        assert np.array_equal(scale.cpu().numpy().view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_quantize_transposed_axis_column_pairs(dev, fp4mod, oracle, dtype):
    """16-bit inputs read in place along the column axis: odd and even
    leading dimensions, starts 2 bytes past a 4-byte boundary and odd and
    even column counts all match the oracle."""
    K, W = 256, 131
    x = gen.normal(97, (K, W), std=0.03)
    xh = gen.to_bf16_bits(x) if dtype == "bf16" else x.astype(np.float16).view(np.uint16)
    big = to_dev(xh, dtype, dev)                              # [256, 131]: ldx odd
    for lo, hi in [(0, 130), (1, 129), (2, 130), (0, 131)]:
        view = big[:, lo:hi] if (lo, hi) != (0, 131) else big
        if (lo, hi) == (2, 130):
            view = big[:, :130].contiguous()[:, lo:hi]       # ldx 130, start 4 bytes in
        rc, rs = oracle.quantize_mxfp4(np.ascontiguousarray(view.cpu().view(torch.int16).numpy().view(np.uint16).T),
                                       32, dtype)
        pk, e8 = fp4mod.quantize_mxfp4_t(view, 32)
        assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc)), (lo, hi)
        assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(rs)), (lo, hi)
    xc = big[:, :130].contiguous()
    rc, rs = oracle.quantize_mxfp4(np.ascontiguousarray(xc.cpu().view(torch.int16).numpy().view(np.uint16).T),
                                   32, dtype)
    pk, e8 = fp4mod.quantize_mxfp4_t(xc, 32)
    assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc))
    assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(rs))


def test_quantize_full_size_cfg4_operand(dev, fp4mod, oracle):
    """BASELINE cfg4 operand at full size: A [8192, 8192] = 0.05 * t3, fp32."""
    g = torch.Generator(device=dev).manual_seed(4001)
    z = torch.randn((8192, 8192), device=dev, generator=g)
    chi = torch.randn((3, 8192, 8192), device=dev, generator=g).square().sum(0)
    x = (z / torch.sqrt(chi / 3.0) * 0.05).contiguous()
    del chi
    pk, e8 = fp4mod.quantize_pack_mxfp4(x)
    xc = x.cpu().numpy()
    rc, rs = oracle.quantize_mxfp4(xc)
    assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc))
    assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(rs))
    # idempotence: quantizing the dequantized tensor reproduces the same bytes
    deq = fp4mod.dequantize_packed(pk, e8)
    pk2, e82 = fp4mod.quantize_pack_mxfp4(deq)
    nz = (e8 != 127)
    assert torch.equal(pk2, pk)
    assert torch.equal(e82[nz], e8[nz])


def test_specials_nan_inf_negzero(dev, fp4mod):
    from .test_oracle import golden_inputs
    arrays = np.load(GOLD / "fp4_golden.npz")
    x = golden_inputs()["special"]
    codes, scale = fp4mod.quantize_mxfp4(to_dev(x, "f32", dev))
    assert np.array_equal(codes.cpu().numpy(), arrays["special__codes"])
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), arrays["special__scale"].view(np.uint32))
    pk, e8 = fp4mod.quantize_pack_mxfp4(to_dev(x, "f32", dev))
    assert int(e8[0, 0]) == 255 and int(e8[2, 0]) == 254 and int(e8[5, 0]) == 127


def test_pack_unpack_match_oracle(dev, fp4mod, oracle):
    rng = np.random.default_rng(7)
    for n in [2, 14, 16, 18, 1000, 4096 * 33 + 6]:
        codes = rng.integers(0, 16, (n,), dtype=np.uint8)
        pk = fp4mod.pack_fp4(torch.from_numpy(codes).to(dev))
        assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(codes)), n
        back = fp4mod.unpack_fp4(pk)
        assert np.array_equal(back.cpu().numpy(), codes), n
    allb = torch.arange(256, dtype=torch.uint8, device=dev)
    assert np.array_equal(fp4mod.unpack_fp4(allb).cpu().numpy(), oracle.unpack_fp4(np.arange(256, dtype=np.uint8)))


@pytest.mark.parametrize("block", [32, 16])
def test_dequantize_matches_oracle(dev, fp4mod, oracle, block):
    x = gen.student_t3(77, (96, 512), scale=0.05)
    rc, rs = oracle.quantize_mxfp4(x, block)
    want = oracle.dequantize_mxfp4(rc, rs, block)
    got = fp4mod.dequantize_mxfp4(torch.from_numpy(rc).to(dev), torch.from_numpy(rs).to(dev), block)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    e8 = torch.from_numpy(oracle.scale_to_e8m0(rs)).to(dev)
    pk = torch.from_numpy(oracle.pack_fp4(rc)).to(dev)
    got_bf = fp4mod.dequantize_packed(pk, e8, block, out_dtype=torch.bfloat16)
    assert torch.equal(got_bf.float().cpu(), torch.from_numpy(want))   # exact in bf16


def test_e4m3_expansion_exhaustive(dev, fp4mod, oracle):
    words = np.arange(1 << 16, dtype=np.uint32) * np.uint32(0x10001) ^ np.uint32(0x9E3779B9)
    words = np.concatenate([words, np.arange(1 << 16, dtype=np.uint32)])
    got = fp4mod.fp4_to_e4m3_words(torch.from_numpy(words.view(np.int32)).to(dev)).cpu().numpy().view(np.uint32)
    lo, hi = oracle.fp4x8_to_e4m3x8(words)
    assert np.array_equal(got[0::2], lo) and np.array_equal(got[1::2], hi)
    codes = torch.arange(16, dtype=torch.uint8, device=dev)
    e4 = fp4mod.codes_to_e4m3(codes)
    assert e4.dtype == torch.float8_e4m3fn
    assert torch.equal(e4.float().cpu(), fp4mod.E2M1_VALUES)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 255, 1027, 4096 * 3 + 2])
@pytest.mark.parametrize("offset", [0, 1])
def test_e4m3_expansion_ragged_and_unaligned(dev, fp4mod, oracle, n, offset):
    """Word counts that leave 1-3 words after the last whole quad (the
    16-byte kernel's tail lane), and a source starting 4 bytes past a 16-byte
    boundary (the one-word-per-lane kernel)."""
    rng = np.random.default_rng(n * 7 + offset)
    words = rng.integers(0, 1 << 32, size=n + offset, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev)[offset:]
    assert (src.data_ptr() % 16 == 0) == (offset == 0)
    got = fp4mod.fp4_to_e4m3_words(src).cpu().numpy().view(np.uint32)
    lo, hi = oracle.fp4x8_to_e4m3x8(words[offset:])
    assert np.array_equal(got[0::2], lo) and np.array_equal(got[1::2], hi)


def test_repeat_runs_are_bitwise_identical(dev, fp4mod):
    x = torch.randn(512, 4096, device=dev)
    a = fp4mod.quantize_pack_mxfp4(x)
    b = fp4mod.quantize_pack_mxfp4(x)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_quantize_kmajor_scale_layout(dev, fp4mod, oracle):
    """K-major E8M0 scales hold the same bytes as the row-major ones,
    rearranged to [K/128, rows, 4]."""
    for rows, K in [(1, 128), (37, 384), (300, 4096)]:
        x = gen.student_t3(rows + K, (rows, K), scale=0.05)
        rc, rs = oracle.quantize_mxfp4(x)
        pk, e8 = fp4mod.quantize_pack_mxfp4(to_dev(x, "f32", dev), scale_layout="kmajor")
        want = oracle.scale_to_e8m0(rs).reshape(rows, K // 128, 4).transpose(1, 0, 2)
        assert e8.shape == (K // 128, rows, 4)
        assert np.array_equal(e8.cpu().numpy(), want), (rows, K)
        assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(rc)), (rows, K)
        assert torch.equal(fp4mod.kmajor_scales(fp4mod.quantize_pack_mxfp4(to_dev(x, "f32", dev))[1]), e8)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_exact_ties_round_toward_smaller_magnitude(dev, fp4mod, oracle, dtype):
    """Elements at exactly 0.75, 1.75 and 3.5 times their block scale (fp4.py
    rounds those ties down, fp4.py:50-53) spread thinly over random blocks, so
    most waves hold none and a few hold one or two.  Packed codes, E8M0 bytes
    and the K-major layout equal the oracle's."""
    rows, K = 96, 1024
    x = gen.normal(4242, (rows, K)).astype(np.float32)
    # round to the input dtype first, so the block scales below are the ones
    # the dtype's values give (tie values have 2 significant bits: exact in all three)
    if dtype == "bf16":
        x = (gen.to_bf16_bits(x).astype(np.uint32) << 16).view(np.float32)
    elif dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
    ref_codes, ref_scale = oracle.quantize_mxfp4(x)
    e = np.log2(ref_scale).astype(np.int32)                      # block exponents, [rows, K/32]
    rng = np.random.default_rng(7)
    n_ties = 60
    rr = rng.integers(0, rows, n_ties)
    kk = rng.integers(0, K, n_ties)
    # never overwrite a block's largest element: the tie values lie below
    # the block's amax (>= 4 * 2^e), so every block scale is unchanged
    amax = np.abs(x).reshape(rows, K // 32, 32).max(axis=2)
    keep = np.abs(x[rr, kk]) < amax[rr, kk // 32]
    rr, kk = rr[keep], kk[keep]
    mult = rng.choice([0.75, 1.75, 3.5], len(rr)) * rng.choice([-1.0, 1.0], len(rr))
    x[rr, kk] = (mult * np.exp2(e[rr, kk // 32].astype(np.float64))).astype(np.float32)
    if dtype == "bf16":
        xh = gen.to_bf16_bits(x)
    elif dtype == "f16":
        xh = x.astype(np.float16).view(np.uint16)
    else:
        xh = x
    ref_codes, ref_scale = oracle.quantize_mxfp4(xh, 32, None if dtype == "f32" else dtype)
    assert np.array_equal(np.log2(ref_scale).astype(np.int32), e), "block scales must not move"
    q = ref_codes[rr, kk] & 7
    assert len(rr) > 40 and np.all(np.isin(q, [1, 3, 5])), "planted values must be ties the reference rounds down"
    xt = to_dev(xh, dtype, dev)
    packed, e8 = fp4mod.quantize_pack_mxfp4(xt)
    assert np.array_equal(packed.cpu().numpy(), oracle.pack_fp4(ref_codes))
    assert np.array_equal(e8.cpu().numpy(), oracle.scale_to_e8m0(ref_scale))
    pk, e8k = fp4mod.quantize_pack_mxfp4(xt, scale_layout="kmajor")
    assert np.array_equal(pk.cpu().numpy(), oracle.pack_fp4(ref_codes))
    want = oracle.scale_to_e8m0(ref_scale).reshape(rows, K // 128, 4).transpose(1, 0, 2)
    assert np.array_equal(e8k.cpu().numpy(), want)


def _both_forms_ref(oracle, xh, dtype):
    """The oracle's row form of x and row form of x^T (the column form)."""
    rc, rs = oracle.quantize_mxfp4(xh, 32, dtype)
    cc, cs = oracle.quantize_mxfp4(np.ascontiguousarray(xh.T), 32, dtype)
    return oracle.pack_fp4(rc), oracle.scale_to_e8m0(rs), oracle.pack_fp4(cc), oracle.scale_to_e8m0(cs)


def _kmajor(e8):
    rows, nb = e8.shape
    return e8.reshape(rows, nb // 4, 4).transpose(1, 0, 2)


def _check_2d(fp4mod, oracle, xh, dtype, dev, layouts=("kmajor", "rows")):
    rp, rs, cp, cs = _both_forms_ref(oracle, xh, dtype)
    xt = to_dev(xh, dtype, dev)
    for lay in layouts:
        grp, grs, gcp, gcs = fp4mod.quantize_pack_mxfp4_2d(xt, scale_layout=lay)
        assert np.array_equal(grp.cpu().numpy(), rp) and np.array_equal(gcp.cpu().numpy(), cp), lay
        want_r, want_c = (_kmajor(rs), _kmajor(cs)) if lay == "kmajor" else (rs, cs)
        assert np.array_equal(grs.cpu().numpy(), want_r) and np.array_equal(gcs.cpu().numpy(), want_c), lay
        # the same bytes as the two one-axis quantizers
        a = fp4mod.quantize_pack_mxfp4(xt, scale_layout=lay)
        b = fp4mod.quantize_mxfp4_t(xt, scale_layout=lay)
        assert torch.equal(a[0], grp) and torch.equal(a[1], grs) and torch.equal(b[0], gcp) and torch.equal(b[1], gcs)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("R,C", [(128, 128), (256, 384), (384, 1024), (2048, 8192)])
def test_quantize_both_axes_in_one_pass(dev, fp4mod, oracle, dtype, R, C):
    """quantize_pack_mxfp4_2d: row form == fp4.py:57-72 on x, column form ==
    fp4.py:57-72 on x.t().contiguous(), both layouts of E8M0 scales."""
    x = gen.student_t3(R + 3 * C, (R, C), scale=0.05)
    xh = gen.to_bf16_bits(x) if dtype == "bf16" else x.astype(np.float16).view(np.uint16)
    _check_2d(fp4mod, oracle, xh, dtype, dev)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_quantize_both_axes_ties_and_specials(dev, fp4mod, oracle, dtype):
    """Values on the quarter grid of 2^-3 with most 32-blocks (along either
    axis) reaching 5 or 6 units: their scale is 2^-3, and the many elements at
    0.75, 1.75 and 3.5 units are ties that fp4.py rounds toward the smaller
    magnitude along both axes.  Plus NaN, +-Inf and -0 blocks."""
    R, C = 256, 256
    rng = np.random.default_rng(11)
    grid = np.array([0, 0.25, 0.5, 0.75, 1, 1.25, 1.5, 1.75, 2, 2.5, 3, 3.5, 4, 5, 6], dtype=np.float64)
    x = rng.choice(grid, (R, C)) * rng.choice([-1.0, 1.0], (R, C)) * 0.125
    x = x.astype(np.float32)
    x[5, 40] = np.nan
    x[130, 7] = np.inf
    x[131, 9] = -np.inf
    x[64:96, 160:192] = -0.0
    x[200, 200:232] = 0.0
    xh = gen.to_bf16_bits(x) if dtype == "bf16" else x.astype(np.float16).view(np.uint16)
    rc, _ = oracle.quantize_mxfp4(xh, 32, dtype)
    assert np.isin(rc & 7, [1, 3, 5]).mean() > 0.2       # plenty of rounded-down ties
    _check_2d(fp4mod, oracle, xh, dtype, dev)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_quantize_both_axes_scale_range(dev, fp4mod, oracle, dtype):
    """Block absmaxes over the dtype's whole exponent range: 8 x 8 patches
    of N(0,1) scaled by 2^k, so every 32-block along either axis mixes four
    exponents.  Includes subnormal inputs, for bf16 whole tiles below
    fp4.py's 1e-30 clamp (scale byte 25), amaxes one 16-bit ulp below a
    power of two, and tiles near the dtype's largest finite value."""
    R, C = 256, 512
    rng = np.random.default_rng(23 if dtype == "bf16" else 29)
    lo, hi = (-140, 124) if dtype == "bf16" else (-24, 13)
    k = rng.integers(lo, hi, (R // 8, C // 8))
    k[0:4, 0:4] = lo + 5                                   # one 32 x 32 tile entirely tiny
    k[4:8, 8:12] = hi                                      # one tile near the top of the range
    x = rng.standard_normal((R, C)) * np.exp2(np.repeat(np.repeat(k, 8, 0), 8, 1).astype(np.float64))
    # amaxes one ulp below a power of two: 0.99609375 (bf16) / 0.99951171875 (fp16) * 2^j
    below = 1.0 - (2.0 ** -8 if dtype == "bf16" else 2.0 ** -11)
    for j, (r, c) in enumerate([(40, 70), (100, 300), (200, 33), (77, 500)]):
        x[r, c] = below * 2.0 ** (k[r // 8, c // 8] + 3)
    x = x.astype(np.float32)
    xh = gen.to_bf16_bits(x) if dtype == "bf16" else x.astype(np.float16).view(np.uint16)
    rc, rs = oracle.quantize_mxfp4(xh, 32, dtype)
    e8 = oracle.scale_to_e8m0(rs)
    if dtype == "bf16":
        assert (e8 == 25).any() and e8.max() > 200
    else:
        assert e8.min() < 110 and e8.max() > 130
    assert (rc & 7).max() == 7
    _check_2d(fp4mod, oracle, xh, dtype, dev)


def test_quantize_both_axes_falls_back_for_other_inputs(dev, fp4mod, oracle):
    """fp32 input, or sizes that are not multiples of 128, run the two
    one-axis kernels and give the same bytes."""
    for (R, C, dtype) in [(256, 256, "f32"), (96, 128, "bf16")]:
        x = gen.normal(R * C, (R, C))
        xh = x if dtype == "f32" else gen.to_bf16_bits(x)
        _check_2d(fp4mod, oracle, xh, None if dtype == "f32" else dtype, dev, layouts=("rows",))


def test_quantize_both_axes_batch(dev, fp4mod):
    """quantize_pack_mxfp4_2d_many: tensors of one dtype with sizes multiples
    of 128 share one launch (lsmx_quantize_mxfp4_2d_batch, up to 8 per
    launch), the rest run alone; every output equals the one-tensor call's
    bytes.  Includes an fp16 group beside a bf16 one, a transposed view, a
    zero tensor, a shape off the 128 grid and two launches for 11 tensors."""
    g = torch.Generator(device=dev).manual_seed(21)
    rn = lambda *s: torch.randn(s, device=dev, generator=g)   # noqa: E731
    xs = [rn(256, 384).to(torch.bfloat16), rn(1024, 128).to(torch.float16), rn(384, 256).to(torch.bfloat16).t(),
          (rn(2048, 8192) * 0.05).to(torch.bfloat16), torch.zeros((128, 128), device=dev, dtype=torch.bfloat16),
          rn(128, 256).to(torch.float16)]
    many = [(rn(128, 256) * (k + 1)).to(torch.bfloat16) for k in range(11)]
    # off the 128 grid (row-major scales only): the one-tensor path
    mixed = [rn(96, 256).to(torch.bfloat16), rn(128, 128).to(torch.bfloat16)]
    for group, lays in ((xs, ("kmajor", "rows")), (many, ("kmajor", "rows")), (mixed, ("rows",))):
        for lay in lays:
            got = fp4mod.quantize_pack_mxfp4_2d_many(group, scale_layout=lay)
            assert len(got) == len(group)
            for x, gt in zip(group, got):
                want = fp4mod.quantize_pack_mxfp4_2d(x, scale_layout=lay)
                for a, b in zip(gt, want):
                    assert a.shape == b.shape and torch.equal(a, b), (tuple(x.shape), lay)


def test_quantize_rows_batch(dev, fp4mod, oracle):
    """quantize_pack_mxfp4_many (lsmx_quantize_mxfp4_batch, up to 8 tensors
    per launch) gives quantize_pack_mxfp4's bytes for every tensor: fp32,
    bf16 and fp16 groups, rows of different lengths in one launch (the grid
    covers the longest), a strided view, a 3-D tensor, an empty tensor, NaN
    and Inf blocks, and two launches for 10 tensors; the oracle pins one
    tensor of the batch."""
    g = torch.Generator(device=dev).manual_seed(23)
    rn = lambda *s: torch.randn(s, device=dev, generator=g)   # noqa: E731
    odd = rn(64, 384)
    odd[3, 40] = float("nan")
    odd[7, 100] = float("inf")
    odd[9, :32] = 0.0
    xs = [rn(256, 8192) * 0.05, rn(300, 256), odd, rn(96, 1024)[:, 128:640], torch.empty((0, 128), device=dev),
          rn(2, 5, 128), rn(128, 384).to(torch.bfloat16), rn(64, 640).to(torch.float16), rn(1, 4096)]
    many = [rn(32, 128) * (k + 1) for k in range(10)]
    for group, lays in ((xs, ("rows",)), ([x for x in xs if x.dim() == 2 and x.shape[1] % 128 == 0], ("kmajor",)),
                        (many, ("rows", "kmajor"))):
        for lay in lays:
            got = fp4mod.quantize_pack_mxfp4_many(group, scale_layout=lay)
            assert len(got) == len(group)
            for x, gt in zip(group, got):
                want = fp4mod.quantize_pack_mxfp4(x, scale_layout=lay)
                for a, b in zip(gt, want):
                    assert a.shape == b.shape and torch.equal(a, b), (tuple(x.shape), x.dtype, lay)
    # the batch against the oracle directly, for the tensor with specials
    got = fp4mod.quantize_pack_mxfp4_many([xs[0], odd], scale_layout="rows")[1]
    codes, scale = oracle.quantize_mxfp4(odd.cpu().numpy(), 32)
    assert np.array_equal(got[0].cpu().numpy(), oracle.pack_fp4(codes))
    assert np.array_equal(got[1].cpu().numpy(), oracle.scale_to_e8m0(scale))
