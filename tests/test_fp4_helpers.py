"""CPU tests of the drop-in's torch-only helpers (no GPU): random_codes,
codes_to_q, blockwise_exact_dot, reference_mxfp4_gemm, the E8M0 <-> fp32
scale conversions and dual_gemm's slot arithmetic.

They mirror the reference's own checks (tests/test_fp4.py:22-24, 42-45,
77-92, 95-102) against lockstep_amd's spelling of these helpers, with the
quantized operands coming from the CPU oracle (the drop-in's quantizer runs
on the GPU only).
"""

import numpy as np
import torch

from lockstep_amd import dual_gemm, fp4
from oracle import gen

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_random_codes_skip_negative_zero():
    """tests/test_fp4.py:42-45."""
    torch.manual_seed(0)
    codes = fp4.random_codes((20000,))
    assert codes.dtype == torch.uint8 and codes.shape == (20000,)
    assert not (codes == 8).any()
    assert set(codes.unique().tolist()) == {c for c in range(16) if c != 8}


def test_codes_to_q_is_twice_the_value():
    """tests/test_fp4.py:22-24: the integer grid is 2 * value, for every code."""
    codes = torch.arange(16, dtype=torch.uint8)
    q = fp4.codes_to_q(codes)
    assert q.dtype == torch.int32
    assert torch.equal(q.float(), 2 * fp4.E2M1_VALUES)
    assert torch.equal(fp4.E2M1_VALUES, torch.tensor(E2M1 + [-v for v in E2M1]))


def test_blockwise_exact_dot_bound_and_value():
    """tests/test_fp4.py:77-82, plus a brute-force per-block sum."""
    torch.manual_seed(3)
    qa = fp4.codes_to_q(fp4.random_codes((4, 128)))
    qb = fp4.codes_to_q(fp4.random_codes((4, 128)))
    blocks = fp4.blockwise_exact_dot(qa, qb, 32)
    assert blocks.dtype == torch.int64 and blocks.shape == (4, 4)
    assert blocks.abs().max() <= 144 * 32
    assert torch.equal(blocks.sum(-1), (qa.long() * qb.long()).sum(-1))
    for r in range(4):
        for b in range(4):
            want = sum(int(qa[r, 32 * b + i]) * int(qb[r, 32 * b + i]) for i in range(32))
            assert int(blocks[r, b]) == want
    # the extreme: every product is 12 * 12 = 144
    top = torch.full((1, 32), 12, dtype=torch.int32)
    assert int(fp4.blockwise_exact_dot(top, top)[0, 0]) == 144 * 32


def _oracle_operand(oracle, x):
    codes, scale = oracle.quantize_mxfp4(x)
    return torch.from_numpy(codes), torch.from_numpy(scale)


def test_reference_gemm_runs_on_cpu_and_matches_dequantized_matmul(oracle):
    """tests/test_fp4.py:85-92: reference_mxfp4_gemm (B given [K, N], scales
    [K//32, N]) equals the fp64 product of the dequantized operands; computed
    here on CPU tensors, checked against the oracle's fp64 GEMM."""
    a = gen.normal(81, (8, 64))
    bt = gen.student_t3(82, (16, 64), scale=0.05)
    ac, as_ = _oracle_operand(oracle, a)
    bc, bs_ = _oracle_operand(oracle, bt)
    ref = fp4.reference_mxfp4_gemm(ac, as_, bc.t(), bs_.t())
    assert ref.dtype == torch.float32 and ref.shape == (8, 16) and ref.device.type == "cpu"
    want = oracle.reference_gemm_packed(oracle.pack_fp4(ac.numpy()), oracle.scale_to_e8m0(as_.numpy()),
                                        oracle.pack_fp4(bc.numpy()), oracle.scale_to_e8m0(bs_.numpy()))
    assert np.array_equal(ref.numpy(), want.astype(np.float32))
    # brute force over K on one element
    deq = lambda c, s, r, k: E2M1[c[r, k] & 7] * (-1 if c[r, k] & 8 else 1) * float(s[r, k // 32])  # noqa: E731
    v = sum(deq(ac, as_, 3, k) * deq(bc, bs_, 5, k) for k in range(64))
    assert np.float32(v) == ref[3, 5].item()


def test_reference_gemm_block_16():
    """block=16: the B scales broadcast over 16-row groups of K."""
    torch.manual_seed(4)
    a = fp4.random_codes((4, 32))
    b = fp4.random_codes((32, 6))
    sa = torch.exp2(torch.randint(-3, 4, (4, 2)).float())
    sb = torch.exp2(torch.randint(-3, 4, (2, 6)).float())
    ref = fp4.reference_mxfp4_gemm(a, sa, b, sb, block=16)
    A = fp4.E2M1_VALUES[a.long()].double() * sa.double().repeat_interleave(16, dim=1)
    B = fp4.E2M1_VALUES[b.long()].double() * sb.double().repeat_interleave(16, dim=0)
    assert torch.equal(ref, (A @ B).float())


def test_scale_e8m0_round_trip_and_edges():
    """Every E8M0 byte maps to 2^(e-127) (byte 0 to 2^-127, 0xFF to NaN) and
    back; fp32 scales with no E8M0 form map to 0xFF, as the GEMMs treat them."""
    e = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    s = fp4.e8m0_to_scale(e)
    want = torch.tensor([np.ldexp(1.0, i - 127) for i in range(255)], dtype=torch.float64).float()
    assert torch.equal(s[:255], want)
    assert s[0].item() == 2.0 ** -127 and torch.isnan(s[255])
    assert torch.equal(fp4.scale_to_e8m0(s), e)
    bad = torch.tensor([1.5, -2.0, 0.0, float("inf"), float("nan"), 3.0 * 2 ** -130, -0.0])
    assert fp4.scale_to_e8m0(bad).tolist() == [255] * 7


def test_dual_slot_split():
    """tests/test_fp4.py:95-102."""
    for k in (8, 32, 128):
        s = dual_gemm.slot_offset(k)
        c1 = torch.tensor([144.0 * k, -144.0 * k, 3.0], dtype=torch.float64)
        c2 = torch.tensor([-144.0 * k, 144.0 * k, -7.0], dtype=torch.float64)
        g1, g2 = dual_gemm.unpack_dual(c1 + c2 * 2.0 ** s, s)
        assert torch.equal(g1, c1) and torch.equal(g2, c2)


def test_e8m0_exact_tracks_the_module_s_own_scales():
    """fp4.e8m0_exact: true for fp32 scales e8m0_to_scale returned and views
    of them, false for copies and after an in-place write through any view
    (which bumps the version counter views share), so mxfp4_gemm_packed skips
    its promotion launch only for scales that are powers of two or NaN by
    construction."""
    import torch
    from lockstep_amd import fp4
    s = fp4.e8m0_to_scale(torch.tensor([[127, 0, 255, 130], [1, 2, 3, 4]], dtype=torch.uint8))
    assert fp4.e8m0_exact(s) and fp4.e8m0_exact(s.t()) and fp4.e8m0_exact(s.view(8)[1:])
    assert not fp4.e8m0_exact(s.clone()) and not fp4.e8m0_exact(s.t().contiguous()) and not fp4.e8m0_exact(torch.ones(2, 4))
    v = s.view(8)
    v[1] = 1.5
    assert not fp4.e8m0_exact(s) and not fp4.e8m0_exact(v)
    # quantize_mxfp4 marks a reshape of its output, which is a view
    r = fp4._mark_e8m0_exact(torch.ones(2, 4).reshape(2, 4))
    assert r._base is not None and fp4.e8m0_exact(r) and fp4.e8m0_exact(r[1:])
    t = fp4.e8m0_to_scale(torch.tensor([[127]], dtype=torch.uint8))
    key = id(t)
    del t
    assert key not in fp4._E8M0_EXACT
