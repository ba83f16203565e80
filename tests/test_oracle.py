"""CPU tests that pin the oracle (oracle/mxfp4_oracle.c) before it is trusted.

Each check ties an oracle function to something outside it: the reference's
own tests (tests/test_fp4.py), its C code (cuda/fp4_unpack.cuh built into
oracle/_ref), golden vectors written by the reference's fp4.py
(tests/golden/), the torch library routines fp4.py calls, or brute force.
"""

import hashlib
import importlib.util
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gen

ROOT = Path(__file__).resolve().parents[1]
GOLD = ROOT / "tests" / "golden"
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _golden_module():
    spec = importlib.util.spec_from_file_location("make_golden", GOLD / "make_golden.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def golden_inputs():
    """The inputs tests/golden/make_golden.py fed to the reference fp4.py."""
    mg = _golden_module()
    mult = np.ldexp(1.0 + (np.arange(64) % 7) / 8.0, np.arange(64) // 3 - 10)
    return {
        "cfg1_W": gen.normal(1002, (1024, 1024), std=0.02),
        "cfg1_X": gen.normal(1001, (256, 1024)),
        "w_slice": gen.normal(2003, (64, 4096), std=0.02),
        "a_bf16": gen.to_bf16_bits(gen.normal(2001, (64, 4096))),
        "t3_slice": gen.student_t3(4001, (64, 8192), scale=0.05),
        "blk16": gen.normal(7, (32, 512)),
        "logspace": (gen.normal(0, (64, 256)).astype(np.float64) * mult[:, None]).astype(np.float32),
        "edges": mg.edge_blocks(),
        "special": mg.special_blocks(),
    }


@pytest.fixture(scope="module")
def golden():
    return json.loads((GOLD / "fp4_golden.json").read_text())["cases"], np.load(GOLD / "fp4_golden.npz")


# ---------------------------------------------------------------- tables (A1)
def test_e4m3_table_decodes_to_e2m1_values(oracle):
    # tests/test_fp4.py:15-19, decoded by torch's float8_e4m3fn
    got = torch.from_numpy(oracle.E2M1_TO_E4M3.copy()).view(torch.float8_e4m3fn).float()
    assert torch.equal(got, torch.tensor(E2M1 + [-v for v in E2M1]))


def test_integer_grid_is_twice_the_value(oracle):
    # tests/test_fp4.py:22-24
    assert np.array_equal(oracle.E2M1_Q.astype(np.float32), 2 * oracle.E2M1_VALUES)


def test_e4m3_expansion_matches_reference_c_exhaustively(oracle):
    """All 16^4 nibble quadruples against cuda/fp4_unpack.cuh compiled from the
    reference (oracle/_ref), as cuda/test_unpack.c:13-23 does."""
    ref = oracle.ref_unpack_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference not mounted here)")
    quads = np.arange(1 << 16, dtype=np.uint32)
    lo, _ = oracle.fp4x8_to_e4m3x8(quads)
    want = np.array([ref.ref_fp4x4_to_e4m3x4(int(p)) for p in quads], dtype=np.uint32)
    assert np.array_equal(lo, want)
    for c in range(16):
        assert ref.ref_fp4_code_to_e4m3(c) == oracle.E2M1_TO_E4M3[c]


def test_e4m3_known_answer(oracle):
    # cuda/test_unpack.c:94-95: fp4x8(0xFEDCBA98) -> bcb8b080 ccc8c4c0
    lo, hi = oracle.fp4x8_to_e4m3x8(np.array([0xFEDCBA98], dtype=np.uint32))
    assert (int(lo[0]), int(hi[0])) == (0xBCB8B080, 0xCCC8C4C0)


def test_reference_unpack_binary_passes():
    exe = ROOT / "oracle" / "_ref" / "test_unpack"
    if not exe.exists():
        pytest.skip("oracle/_ref not built (reference not mounted here)")
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    assert "0 mismatches" in out


# ---------------------------------------------------------------- rounding (A2)
def test_ties_go_to_smaller_magnitude(oracle):
    # tests/test_fp4.py:48-51
    mids = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    got = [oracle.E2M1_VALUES[oracle.round_e2m1(m)] for m in mids]
    assert got == E2M1[:7]


def test_round_matches_reference_on_every_bf16_pattern(oracle, golden):
    """fp4.py:43-54 run by the reference on all 65536 bf16 bit patterns."""
    _, arrays = golden
    allbf = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    mine = np.array([oracle.round_e2m1(v) for v in allbf], dtype=np.uint8)
    assert np.array_equal(mine, arrays["round_all_bf16__codes"])


def test_round_against_torch_bucketize_dense_sweep(oracle):
    """Brute force on a dense fp32 sweep of [0, 8) and its negatives against
    torch.bucketize/abs/clamp/signbit, the library routines fp4.py:50-54 uses."""
    pos = np.arange(0, 8.0, 1.0 / 4096, dtype=np.float32)
    ulp = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
    edge = np.concatenate([np.nextafter(ulp, 0), ulp, np.nextafter(ulp, 9)]).astype(np.float32)
    x = np.concatenate([pos, -pos, edge, -edge, np.float32([np.inf, -np.inf, -0.0])])
    t = torch.from_numpy(x)
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    want = (torch.bucketize(t.abs().clamp(max=6.0), mids).to(torch.uint8)
            | (torch.signbit(t).to(torch.uint8) << 3)).numpy()
    mine = np.array([oracle.round_e2m1(v) for v in x], dtype=np.uint8)
    assert np.array_equal(mine, want)


# ---------------------------------------------------------------- E8M0 (A3')
def _edge_candidates():
    c = []
    for be in range(1, 255):
        top = (be + 1) << 23
        c += [top - 1 - j for j in range(100)]
        c += [(be << 23) + j for j in range(64)]
    c = np.array(c, dtype=np.uint32).view(np.float32)
    return c[np.isfinite(c)]


def test_e8m0_int_rule_equals_log2_rule_at_every_binade_edge(oracle):
    for a in _edge_candidates():
        assert oracle.e8m0_exp_int(a) == oracle.e8m0_exp_log2(a), a


def test_e8m0_log2_rule_equals_torch_log2(oracle):
    """fp4.py:68 calls torch.log2 on float32; compare on every edge candidate
    plus random draws across the whole positive range."""
    rng = np.random.default_rng(0)
    rand = rng.integers(1, 0x7F7FFFFF, 200000, dtype=np.uint32).view(np.float32)
    x = np.concatenate([_edge_candidates(), rand, np.float32([1e-30, 1e-31, 3.4028235e38])])
    t = torch.from_numpy(x.copy())
    want = (torch.floor(torch.log2(t.clamp(min=1e-30))) - 2).clamp(-127, 127).numpy().astype(int)
    mine_log2 = np.array([oracle.e8m0_exp_log2(v) for v in x])
    mine_int = np.array([oracle.e8m0_exp_int(v) for v in x])
    assert np.array_equal(mine_log2, want)
    assert np.array_equal(mine_int, want)


def test_e8m0_window_table_by_brute_force(oracle):
    """The window width per binade equals the count of values below 2^k whose
    float32-rounded log2 is k (brute force with the libm rule)."""
    for k in range(-99, 129):
        top = (k + 127) << 23 if k + 127 < 255 else 0x7F800000
        n = 0
        while n < 200:
            a = np.array([top - 1 - n], dtype=np.uint32).view(np.float32)[0]
            if oracle.e8m0_exp_log2(a) != k - 2:
                break
            n += 1
        assert n == oracle.e8m0_window(k), (k, n)


# ---------------------------------------------------------------- quantize (A3)
@pytest.mark.parametrize("block", [16, 32])
def test_quantize_properties(oracle, block):
    # tests/test_fp4.py:54-68, on the oracle
    x = (gen.normal(5, (64, 256)).astype(np.float64) * np.logspace(-3, 3, 64)[:, None]).astype(np.float32)
    codes, scale = oracle.quantize_mxfp4(x, block)
    assert np.array_equal(np.exp2(np.round(np.log2(scale))), scale)
    xb = x.reshape(64, -1, block)
    amax = np.abs(xb).max(-1)
    r = amax / scale
    assert ((r >= 4 * (1 - 1e-6)) & (r < 8)).all()
    y = oracle.dequantize_mxfp4(codes, scale, block).reshape(64, -1, block)
    err = np.abs(y - xb) / scale[..., None]
    assert (err <= 2.0 + 1e-6).all()


def test_zero_block_is_exact(oracle):
    # tests/test_fp4.py:71-74
    codes, scale = oracle.quantize_mxfp4(np.zeros((2, 32), np.float32))
    assert np.array_equal(scale, np.ones((2, 1), np.float32))
    assert np.array_equal(oracle.dequantize_mxfp4(codes, scale), np.zeros((2, 32), np.float32))


@pytest.mark.parametrize("rule", ["int", "log2"])
def test_quantize_matches_reference_golden(oracle, golden, rule):
    """Codes and scales digest-equal to what the reference fp4.py produced on
    the same inputs (tests/golden/make_golden.py)."""
    cases, _ = golden
    for name, x in golden_inputs().items():
        c = cases[name]
        codes, scale = oracle.quantize_mxfp4(x, c["block"], "bf16" if c["dtype"] == "bf16" else None,
                                             rule=rule)
        assert sha(codes) == c["codes_sha256"], name
        assert sha(scale.view(np.uint32)) == c["scale_sha256"], name


def test_golden_edges_distinguish_exact_exponent_rule(oracle, golden):
    """Planted mistake (oracle side): taking amax's exponent field instead of
    the float32 log2 changes the edge-case scales, so the fixture pins the rule."""
    cases, arrays = golden
    x = golden_inputs()["edges"]
    amax = np.abs(x).max(1)
    wrong = np.array([(int(a.view(np.uint32)) >> 23) - 127 - 2 if a >= 1e-30 else -102 for a in amax])
    gold_e = (arrays["edges__scale"].view(np.uint32)[:, 0] >> 23).astype(int) - 127
    assert (wrong != gold_e).sum() > 100


def test_golden_specials_nan_inf_negzero(oracle, golden):
    _, arrays = golden
    x = golden_inputs()["special"]
    codes, scale = oracle.quantize_mxfp4(x)
    assert np.array_equal(codes, arrays["special__codes"])
    assert np.array_equal(scale.view(np.uint32), arrays["special__scale"].view(np.uint32))
    # spot facts: NaN block -> NaN scale; -0 block -> code 8; Inf -> scale 2^127
    assert np.isnan(scale[0, 0]) and np.isnan(scale[1, 0])
    assert (codes[6] == 8).all()
    assert scale[2, 0] == np.float32(2.0 ** 127)


# ---------------------------------------------------------------- pack / dequant
def test_pack_unpack_roundtrip(oracle):
    # tests/test_fp4.py:34-39
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, (7, 64), dtype=np.uint8)
    packed = oracle.pack_fp4(codes)
    assert packed.shape == (7, 32)
    assert np.array_equal(oracle.unpack_fp4(packed), codes)
    assert (packed[0, 0] & 0x0F) == codes[0, 0]
    assert np.array_equal(packed, codes[:, 0::2] | (codes[:, 1::2] << 4))


def test_dequantize_closed_form(oracle):
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (4, 64), dtype=np.uint8)
    scale = np.ldexp(1.0, rng.integers(-20, 20, (4, 2))).astype(np.float32)
    got = oracle.dequantize_mxfp4(codes, scale)
    want = oracle.E2M1_VALUES[codes] * np.repeat(scale, 32, axis=1)
    assert np.array_equal(got, want)
    packed_deq = oracle.dequantize_packed(oracle.pack_fp4(codes), oracle.scale_to_e8m0(scale))
    assert np.array_equal(packed_deq, want.astype(np.float64))


# ---------------------------------------------------------------- GEMM oracle
def test_reference_gemm_integer_grid_is_exact(oracle):
    """bench.py:44-57: random codes, unit scales -> C = (qa @ qb) / 4 exactly."""
    rng = np.random.default_rng(3)
    pick = np.array([c for c in range(16) if c != 8], dtype=np.uint8)
    ca = pick[rng.integers(0, 15, (64, 128))]
    cb = pick[rng.integers(0, 15, (48, 128))]
    ones = np.full((64, 4), 127, np.uint8), np.full((48, 4), 127, np.uint8)
    got = oracle.reference_gemm_packed(oracle.pack_fp4(ca), ones[0], oracle.pack_fp4(cb), ones[1])
    qa = oracle.E2M1_Q[ca].astype(np.float64)
    qb = oracle.E2M1_Q[cb].astype(np.float64)
    assert np.array_equal(got, (qa @ qb.T) / 4.0)


def test_reference_gemm_brute_force_tiny(oracle):
    rng = np.random.default_rng(4)
    ca = rng.integers(0, 16, (3, 64), dtype=np.uint8)
    cb = rng.integers(0, 16, (2, 64), dtype=np.uint8)
    ea = rng.integers(120, 134, (3, 2)).astype(np.uint8)
    eb = rng.integers(120, 134, (2, 2)).astype(np.uint8)
    got = oracle.reference_gemm_packed(oracle.pack_fp4(ca), ea, oracle.pack_fp4(cb), eb)
    for m in range(3):
        for n in range(2):
            s = 0.0
            for k in range(64):
                va = float(oracle.E2M1_VALUES[ca[m, k]]) * 2.0 ** (int(ea[m, k // 32]) - 127)
                vb = float(oracle.E2M1_VALUES[cb[n, k]]) * 2.0 ** (int(eb[n, k // 32]) - 127)
                s += va * vb
            assert got[m, n] == s


def test_reference_gemm_wonly_brute_force_tiny(oracle):
    """The weight-only oracle (fp4_linear.py:40 with X left unquantized) by a
    scalar triple loop: x * (E2M1 value * 2^(e - 127)) summed in fp64, with
    E8M0 byte 0 (2^-127: all of weight row 1) and exponents 2^-9 .. 2^8, and
    the rows/cols subset selection.  The activations are multiples of 1/2 in
    [-4, 4], so within a weight row every product is a multiple of 2^-11 below
    2^13 and every sum is exact in fp64: the comparison is equality."""
    rng = np.random.default_rng(5)
    M, N, K = 3, 4, 96
    x = rng.integers(-8, 9, (M, K)).astype(np.float64) / 2.0
    cw = rng.integers(0, 16, (N, K), dtype=np.uint8)
    ew = rng.integers(118, 136, (N, K // 32)).astype(np.uint8)
    ew[1, :] = 0
    got = oracle.reference_gemm_wonly(x, oracle.pack_fp4(cw), ew)
    want = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                e = int(ew[n, k // 32])
                s += x[m, k] * float(oracle.E2M1_VALUES[cw[n, k]]) * (2.0 ** -127 if e == 0 else 2.0 ** (e - 127))
            want[m, n] = s
    assert np.array_equal(got, want)
    rows, cols = np.array([2, 0]), np.array([3, 1])
    assert np.array_equal(oracle.reference_gemm_wonly(x, oracle.pack_fp4(cw), ew, rows=rows, cols=cols),
                          want[np.ix_(rows, cols)])
    # a plausible mistake, the scale applied per K element instead of per
    # 32-block, fails the comparison
    wrong = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            wrong[m, n] = sum(x[m, k] * float(oracle.E2M1_VALUES[cw[n, k]]) * 2.0 ** (int(ew[n, min(k, K // 32 - 1)]) - 127)
                              for k in range(K))
    assert not np.array_equal(got, wrong)


def test_reference_gemm_matches_dequantized_matmul(oracle):
    # tests/test_fp4.py:85-92 on the oracle
    a = gen.normal(11, (8, 64))
    bt = gen.normal(12, (16, 64))
    ac, as_ = oracle.quantize_mxfp4(a)
    bc, bs = oracle.quantize_mxfp4(bt)
    ref = oracle.reference_gemm_packed(oracle.pack_fp4(ac), oracle.scale_to_e8m0(as_),
                                       oracle.pack_fp4(bc), oracle.scale_to_e8m0(bs))
    A = oracle.dequantize_mxfp4(ac, as_).astype(np.float64)
    B = oracle.dequantize_mxfp4(bc, bs).astype(np.float64)
    np.testing.assert_allclose(ref, A @ B.T, rtol=1e-12, atol=0)


def test_generator_is_deterministic():
    a = gen.normal(1, (4, 8))
    b = gen.normal(1, (4, 8))
    assert np.array_equal(a, b)
    z = gen.normal(9, (100000,)).astype(np.float64)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    assert sha(gen.normal(1002, (2, 4), std=0.02)) == sha(gen.normal(1002, (2, 4), std=0.02))


# ----------------------------------------------------- fp32 promotion GEMM
def _codes(rng, shape):
    return rng.integers(0, 16, size=shape, dtype=np.uint8)


def test_promote_pow2_scales_integer_grid_is_exact(oracle):
    # power-of-two scales 2^-1 .. 2^1 on the E2M1 grid: every partial sum is
    # a multiple of 2^-4 below 2^16, exact in fp32, so the promotion loop
    # equals the exact fp64 product of the dequantized operands
    rng = np.random.default_rng(5)
    M, N, K = 12, 10, 256
    ca, cb = _codes(rng, (M, K)), _codes(rng, (N, K))
    ea = rng.integers(126, 129, size=(M, K // 32)).astype(np.uint8)
    eb = rng.integers(126, 129, size=(N, K // 32)).astype(np.uint8)
    got = oracle.gemm_promote(oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb], oracle.e8m0_to_scale(ea),
                              oracle.e8m0_to_scale(eb))
    want = oracle.reference_gemm_packed(oracle.pack_fp4(ca), ea, oracle.pack_fp4(cb), eb)
    assert np.array_equal(got.astype(np.float64), want)


def _one_block_expected(p, sa, sb):
    # fl(p * fl(sa * sb)) with numpy's float32 multiply for the scale product
    # and one rounding of the exact fp64 product (p has <= 13 bits, the scale
    # 24, so the fp64 product is exact)
    with np.errstate(invalid="ignore", over="ignore"):
        s = (sa.astype(np.float32)[:, None] * sb.astype(np.float32)[None, :]).astype(np.float32)
        return (p.astype(np.float64) * s.astype(np.float64)).astype(np.float32)


def test_promote_one_block_any_scale(oracle):
    rng = np.random.default_rng(6)
    M, N = 9, 7
    ca, cb = _codes(rng, (M, 32)), _codes(rng, (N, 32))
    A, B = oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb]
    sa = (rng.uniform(0.3, 3.0, size=(M, 1))).astype(np.float32)
    sb = (rng.uniform(0.3, 3.0, size=(N, 1))).astype(np.float32)
    got = oracle.gemm_promote(A, B, sa, sb)
    p = A.astype(np.float64) @ B.astype(np.float64).T
    assert np.array_equal(got, _one_block_expected(p, sa[:, 0], sb[:, 0]))


def test_promote_special_scales_follow_ieee(oracle):
    # scales the E8M0 kernels cannot represent: zero, negative, inf, NaN,
    # subnormal, non-powers of two
    rng = np.random.default_rng(7)
    specials = np.array([0.0, -2.0, np.inf, -np.inf, np.nan, 1e-40, 1.5, 3.0e38], dtype=np.float32)
    M = N = len(specials)
    ca, cb = _codes(rng, (M, 32)), _codes(rng, (N, 32))
    ca[0] = 0  # an all-zero row meets inf and NaN scales
    A, B = oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb]
    got = oracle.gemm_promote(A, B, specials[:, None], specials[::-1].copy()[:, None])
    p = A.astype(np.float64) @ B.astype(np.float64).T
    want = _one_block_expected(p, specials, specials[::-1].copy())
    np.testing.assert_array_equal(got, want)  # NaN positions included
    assert np.isnan(got).any() and np.isinf(got).any() and (got == 0).any()


def test_promote_two_blocks_pin_the_fused_update(oracle):
    # two blocks: acc = fma(p2, s2, fl(p1 * s1)).  With scales in [0.5, 2)
    # the fp64 sum p2 * s2 + acc1 is exact, so one rounding of it is the fma.
    # The unfused form fl(fl(p2 * s2) + acc1) differs on some outputs, which
    # shows the comparison can tell the two apart.
    rng = np.random.default_rng(8)
    M, N = 64, 64
    ca, cb = _codes(rng, (M, 64)), _codes(rng, (N, 64))
    A, B = oracle.E2M1_VALUES[ca], oracle.E2M1_VALUES[cb]
    sa = rng.uniform(0.5, 2.0, size=(M, 2)).astype(np.float32)
    sb = rng.uniform(0.5, 2.0, size=(N, 2)).astype(np.float32)
    got = oracle.gemm_promote(A, B, sa, sb)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    p1, p2 = A64[:, :32] @ B64[:, :32].T, A64[:, 32:] @ B64[:, 32:].T
    acc1 = _one_block_expected(p1, sa[:, 0], sb[:, 0])
    s2 = (sa[:, 1][:, None] * sb[:, 1][None, :]).astype(np.float32)
    fused = (p2 * s2.astype(np.float64) + acc1.astype(np.float64)).astype(np.float32)
    unfused = ((p2 * s2.astype(np.float64)).astype(np.float32) + acc1).astype(np.float32)
    assert np.array_equal(got, fused)
    assert not np.array_equal(fused, unfused)


def test_promote_random_scales_near_fp64(oracle):
    rng = np.random.default_rng(9)
    M, N, K = 16, 12, 512
    ca, cb = _codes(rng, (M, K)), _codes(rng, (N, K))
    A, B = oracle.E2M1_VALUES[ca].astype(np.float64), oracle.E2M1_VALUES[cb].astype(np.float64)
    sa = rng.uniform(-3.0, 3.0, size=(M, K // 32)).astype(np.float32)
    sb = rng.uniform(-3.0, 3.0, size=(N, K // 32)).astype(np.float32)
    got = oracle.gemm_promote(A, B, sa, sb)
    Ad = A * np.repeat(sa.astype(np.float64), 32, axis=1)
    Bd = B * np.repeat(sb.astype(np.float64), 32, axis=1)
    want = Ad @ Bd.T
    bound = (np.abs(Ad) @ np.abs(Bd).T) * (K // 32 + 2) * 2.0 ** -24
    assert np.all(np.abs(got - want) <= bound)
    # the transposed layout of mxfp4_gemm_fp8's b_scale gives the same values
    got_t = oracle.gemm_promote(A, B, sa, np.ascontiguousarray(sb.T), sb_transposed=True)
    assert np.array_equal(got, got_t)
