"""GPU parity at the BASELINE configs' own sizes, on the kernel instances the
benchmark runs.

Each GEMM is compared with the CPU oracle's fp64 product of its own
quantized inputs (fp4.py:103-112 restated), on sampled rows and columns
where the full product would take the oracle too long; the quantized
operands themselves are checked byte for byte against the oracle's
quantizer (fp4.py:57-72 restated) at full size.  Tolerances (bench.py:71
metric max|c - ref| / max|ref|): fp32 output <= 1e-5, bf16 output <= 1e-2.

  cfg1  X[256,1024] fp32, W[1024,1024] ~ N(0,0.02): quantize bytes, the
        fp32 weight-only Y = X @ deq(W)^T and the fake-quant Y of
        fp4_linear.py:40 (both operands quantized)
  cfg3  bf16 A[M,4096] x W[14336,4096], M in {1,16,128,1024,8192}
  cfg4  the bench's instance: K-major E8M0 scales, bf16 out, 8192^3
  cfg5  tokens=8192, hidden=2048, ffn=8192: both forwards and the MXFP4
        dgrad / wgrad of both linears (train_step.py:3-6, 48-75)
"""

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import fp4, fp4_linear, mxfp4_gemm
    return fp4, mxfp4_gemm, fp4_linear


def _np(t):
    return t.cpu().numpy()


def _bf16_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


# ------------------------------------------------------------------- cfg1
def test_cfg1_quantize_and_both_products(dev, mods, oracle):
    fp4, mg, fl = mods
    x = gen.normal(1001, (256, 1024))
    w = gen.normal(1002, (1024, 1024), std=0.02)
    xt, wt = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    # quantize: codes and fp32 scales (fp4.py's own outputs) and the packed form
    wc, ws = fp4.quantize_mxfp4(wt)
    rc, rs = oracle.quantize_mxfp4(w)
    assert np.array_equal(_np(wc), rc) and np.array_equal(_np(ws), rs)
    wpk, we8 = fp4.quantize_pack_mxfp4(wt)
    assert np.array_equal(_np(wpk), oracle.pack_fp4(rc)) and np.array_equal(_np(we8), oracle.scale_to_e8m0(rs))
    # weight-only Y = X @ deq(W)^T with X fp32, as the config states
    ref = oracle.reference_gemm_wonly(x, _np(wpk), _np(we8))
    for s in (we8, ws):
        y = mg.mxfp4_gemm_bf16(xt, wpk, s, out_dtype=torch.float32)
        assert y.dtype == torch.float32 and y.shape == (256, 1024)
        assert oracle.max_rel(_np(y), ref) <= 1e-5
    # the reference's own CPU fake-quant path: F.linear(deq(q(X)), deq(q(W)))
    xq = oracle.quantize_pack(x)
    ref_fq = oracle.reference_gemm_packed(xq[0], xq[1], _np(wpk), _np(we8))
    y_fq = fl.MXFP4Linear(1024, 1024).to(dev)
    with torch.no_grad():
        y_fq.weight.copy_(wt)
        got = y_fq(xt)
    assert got.dtype == torch.float32 and oracle.max_rel(_np(got), ref_fq) <= 1e-5


# ------------------------------------------------------------------- cfg3
@pytest.fixture(scope="module")
def cfg3_weight(dev, mods, oracle):
    fp4 = mods[0]
    g = torch.Generator(device=dev).manual_seed(3003)
    w = torch.randn((14336, 4096), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    rpk, re8 = oracle.quantize_pack(_np(w))
    assert np.array_equal(_np(wpk), rpk) and np.array_equal(_np(we8), re8)
    return wpk, we8, rpk, re8


@pytest.mark.parametrize("M", [1, 16, 128, 1024, 8192])
def test_cfg3_weight_only_sweep(dev, mods, oracle, cfg3_weight, M):
    """The bench's cfg3 rows: each M runs its own kernel (GEMV, decode,
    split-K 128 x 256 ring, 256 x 256 ring) on the full [14336, 4096] weight."""
    fp4, mg, _ = mods
    wpk, we8, rpk, re8 = cfg3_weight
    g = torch.Generator(device=dev).manual_seed(3000 + M)
    a = torch.randn((M, 4096), device=dev, generator=g).to(torch.bfloat16)
    c16 = mg.mxfp4_gemm_bf16(a, wpk, we8)
    c32 = mg.mxfp4_gemm_bf16(a, wpk, we8, out_dtype=torch.float32)
    assert torch.equal(c16, c32.to(torch.bfloat16))           # bf16 out is RNE of the fp32 result
    rows = np.unique(np.linspace(0, M - 1, min(M, 48)).astype(np.int64))
    cols = np.arange(0, 14336, 7)
    ref = oracle.reference_gemm_wonly(a.float().cpu().numpy(), rpk, re8, rows=rows, cols=cols)
    sub = np.ix_(rows, cols)
    assert oracle.max_rel(_np(c32)[sub], ref) <= 1e-5
    assert oracle.max_rel(c16.float().cpu().numpy()[sub], ref) <= 1e-2


# ------------------------------------------------------------------- cfg4
def test_cfg4_bench_instance_kmajor_bf16(dev, mods, oracle):
    """The exact kernel instance bench.py times: 8192^3, both operands
    quantized on the fly from 0.05 * t3 fp32 with K-major E8M0 scales, bf16
    out; vs fp64 on rows every 37 and columns every 41
    (cuda/mxfp4_mma_gemm.cu:235-236), and bit-identical to the row-major
    scale layout."""
    fp4, mg, _ = mods
    n = 8192
    g = torch.Generator(device=dev).manual_seed(4001)

    def t3():
        z = torch.randn((n, n), device=dev, generator=g)
        chi = torch.zeros_like(z)
        for _ in range(3):
            chi += torch.randn((n, n), device=dev, generator=g).square()
        return (z / torch.sqrt(chi / 3.0) * 0.05).contiguous()

    a, b = t3(), t3()
    apk, aek = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    bpk, bek = fp4.quantize_pack_mxfp4(b, scale_layout="kmajor")
    _, ae8 = fp4.quantize_pack_mxfp4(a)
    _, be8 = fp4.quantize_pack_mxfp4(b)
    del a, b
    c = mg.mxfp4_gemm_packed(apk, bpk, aek, bek, out_dtype=torch.bfloat16)
    assert torch.equal(c, mg.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.bfloat16))
    # the K-major bytes are the row-major bytes regrouped
    assert torch.equal(aek, fp4.kmajor_scales(ae8)) and torch.equal(bek, fp4.kmajor_scales(be8))
    rows, cols = np.arange(0, n, 37), np.arange(0, n, 41)
    ref = oracle.reference_gemm_packed(_np(apk), _np(ae8), _np(bpk), _np(be8), rows=rows, cols=cols)
    assert oracle.max_rel(c.float().cpu().numpy()[np.ix_(rows, cols)], ref) <= 1e-2


# ------------------------------------------------------------------- cfg5
T5, H5, F5 = 8192, 2048, 8192


@pytest.fixture(scope="module")
def cfg5_run(dev, mods):
    """One MLP block (fc H -> F, out F -> H) forward + MXFP4 backward on the
    GPU, bf16 throughout, as bench.py's cfg5 step runs it."""
    _, _, fl = mods
    g = torch.Generator(device=dev).manual_seed(5001)
    x = torch.randn((T5, H5), device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn((F5, H5), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((H5, F5), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn((T5, H5), device=dev, generator=g).to(torch.bfloat16)
    h = fl._forward_hip(x, w1)                  # [T, F]
    y = fl._forward_hip(h, w2)                  # [T, H]
    dh, dw2 = fl.mxfp4_backward(dy, h, w2)      # dgrad + wgrad of out
    dx, dw1 = fl.mxfp4_backward(dh, x, w1)      # dgrad + wgrad of fc
    torch.cuda.synchronize()
    for t, shape in ((h, (T5, F5)), (y, (T5, H5)), (dh, (T5, F5)), (dw2, (H5, F5)), (dx, (T5, H5)),
                     (dw1, (F5, H5))):
        assert t.dtype == torch.bfloat16 and t.shape == shape
    return dict(x=x, w1=w1, w2=w2, dy=dy, h=h, y=y, dh=dh, dw2=dw2, dx=dx, dw1=dw1)


def _q_rows(oracle, t):
    """fp4.py:57-72 along the last axis of a bf16 tensor: (packed, e8m0)."""
    return oracle.quantize_pack(_bf16_bits(t), "bf16")


def _q_cols(oracle, t):
    """The same along the first axis: the oracle quantizes an explicit
    transposed copy."""
    return oracle.quantize_pack(np.ascontiguousarray(_bf16_bits(t).T), "bf16")


def _check(oracle, got, aq, bq, rows, cols):
    ref = oracle.reference_gemm_packed(aq[0], aq[1], bq[0], bq[1], rows=rows, cols=cols)
    return oracle.max_rel(got.float().cpu().numpy()[np.ix_(rows, cols)], ref)


@pytest.mark.parametrize("which", ["fc_fwd", "out_fwd", "out_dgrad", "out_wgrad", "fc_dgrad", "fc_wgrad"])
def test_cfg5_mlp_block_gemms(dev, oracle, cfg5_run, which):
    """Each of the six GEMMs against the oracle, given the inputs the GPU
    actually fed it (so errors do not compound along the chain):
      fwd    Y = q_rows(X) . q_rows(W)^T
      dgrad  dX = q_rows(dY) . q_cols(W)       (contraction over N)
      wgrad  dW = q_cols(dY)^T . q_cols(X)     (contraction over T)"""
    r = cfg5_run
    rng = np.random.default_rng(len(which))
    spec = {
        "fc_fwd": (r["h"], lambda: _q_rows(oracle, r["x"]), lambda: _q_rows(oracle, r["w1"])),
        "out_fwd": (r["y"], lambda: _q_rows(oracle, r["h"]), lambda: _q_rows(oracle, r["w2"])),
        "out_dgrad": (r["dh"], lambda: _q_rows(oracle, r["dy"]), lambda: _q_cols(oracle, r["w2"])),
        "out_wgrad": (r["dw2"], lambda: _q_cols(oracle, r["dy"]), lambda: _q_cols(oracle, r["h"])),
        "fc_dgrad": (r["dx"], lambda: _q_rows(oracle, r["dh"]), lambda: _q_cols(oracle, r["w1"])),
        "fc_wgrad": (r["dw1"], lambda: _q_cols(oracle, r["dh"]), lambda: _q_cols(oracle, r["x"])),
    }
    got, aq, bq = spec[which]
    M, N = got.shape
    rows = np.sort(rng.choice(M, 64, replace=False))
    cols = np.sort(rng.choice(N, 96, replace=False))
    assert _check(oracle, got, aq(), bq(), rows, cols) <= 1e-2


def test_cfg5_fused_h_and_dh_quantization(dev, oracle, mods, cfg5_run):
    """h and dh are only ever quantized, so the fc forward and the out dgrad
    GEMMs quantize them in their epilogue (mxfp4_gemm_packed_q2d): the four
    MXFP4 arrays of each equal the two-axis quantizer applied to the bf16 h
    and dh this chain computed, and sampled rows and columns of them equal
    the oracle's quantizer (fp4.py:57-72) of those bf16 values."""
    from lockstep_amd import fp4, mxfp4_gemm as mg
    r = cfg5_run
    q = {k: fp4.quantize_pack_mxfp4_2d(r[k], scale_layout="kmajor") for k in ("x", "w1", "w2", "dy")}
    fused = {"h": mg.mxfp4_gemm_packed_q2d(q["x"][0], q["w1"][0], q["x"][1], q["w1"][1]),
             "dh": mg.mxfp4_gemm_packed_q2d(q["dy"][0], q["w2"][2], q["dy"][1], q["w2"][3])}
    rng = np.random.default_rng(55)
    for name, got in fused.items():
        want = fp4.quantize_pack_mxfp4_2d(r[name], scale_layout="kmajor")
        for g_, w_ in zip(got, want):
            assert torch.equal(g_, w_), name
        rows = np.sort(rng.choice(T5, 24, replace=False))
        cols = np.sort(rng.choice(F5, 24, replace=False))
        rq, rsc = _q_rows(oracle, r[name][torch.from_numpy(rows).to(dev)])
        assert np.array_equal(got[0].cpu().numpy()[rows], rq)
        assert np.array_equal(got[1].cpu().numpy()[:, rows, :].transpose(1, 0, 2).reshape(len(rows), -1), rsc)
        cq, csc = _q_cols(oracle, r[name][:, torch.from_numpy(cols).to(dev)])
        assert np.array_equal(got[2].cpu().numpy()[cols], cq)
        assert np.array_equal(got[3].cpu().numpy()[:, cols, :].transpose(1, 0, 2).reshape(len(cols), -1), csc)
