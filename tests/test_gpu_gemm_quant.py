"""GPU: the f4 x f4 GEMM with a quantizing epilogue (lsmx_gemm_f4f4_quant)
writes, bit for bit, what the GEMM's bf16 output gives through the two-axis
quantizer: quantize_pack_mxfp4_2d(mxfp4_gemm_packed(...), "kmajor"), i.e.
quantize_mxfp4 (fp4.py:57-72) of C along its rows and of C^T along its rows.
The two-axis quantizer itself is pinned to the CPU oracle elsewhere; here the
GEMM + quantizer pair is the reference, and a sample of the codes is checked
against the oracle's quantizer directly as well."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import fp4, mxfp4_gemm
    return fp4, mxfp4_gemm


def _operands(fp4, dev, M, N, K, seed, special=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn((M, K), device=dev, generator=g)
    b = torch.randn((N, K), device=dev, generator=g) * 0.05
    if M >= 64:
        a[5] = 0.0                               # a zero row of C: scale byte 127, codes 0
    apk, ak = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    bpk, bk = fp4.quantize_pack_mxfp4(b, scale_layout="kmajor")
    if special:
        ak[0, 7, 1] = 255                        # E8M0 NaN: row 7 of C is NaN
        ak[:, 9, :] = 254                        # 2^127: row 9 overflows bf16 to +-Inf
        bk[0, 3, 2] = 255                        # column 3 of C is NaN
    return apk, ak, bpk, bk


def _check(fp4, mg, apk, ak, bpk, bk, keep):
    c = mg.mxfp4_gemm_packed(apk, bpk, ak, bk, out_dtype=torch.bfloat16)
    want = fp4.quantize_pack_mxfp4_2d(c, scale_layout="kmajor")
    got = mg.mxfp4_gemm_packed_q2d(apk, bpk, ak, bk, keep_output=keep)
    names = ("row codes", "row scales", "column codes", "column scales")
    for n, x, y in zip(names, got, want):
        assert x.shape == y.shape and torch.equal(x, y), f"{n} differ"
    if keep:
        assert torch.equal(got[4].view(torch.int16), c.view(torch.int16)), "bf16 C differs"
    return c, got


@pytest.mark.parametrize("keep", [False, True])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (512, 768, 1024), (1024, 512, 2048), (768, 1280, 512)])
def test_quant_epilogue_matches_gemm_then_quantizer(dev, mods, M, N, K, keep):
    fp4, mg = mods
    _check(fp4, mg, *_operands(fp4, dev, M, N, K, seed=M + 3 * N + K), keep)


def test_quant_epilogue_inf_and_nan(dev, mods):
    """Rows and columns of C that hold NaN (E8M0 NaN scales) and +-Inf (bf16
    overflow): the rare-path rules (scale 254 for an Inf block, the E8M0 NaN
    and sign-carrying codes for a NaN block) agree too."""
    fp4, mg = mods
    c, got = _check(fp4, mg, *_operands(fp4, dev, 512, 512, 512, seed=77, special=True), keep=True)
    assert bool(torch.isnan(c[7]).all()) and bool(torch.isinf(c[9]).any()) and bool(torch.isnan(c[:, 3]).all())
    rs = got[1].cpu().numpy()                     # [N/128][M][4]
    assert (rs[:, 7, :] == 255).all()


def test_quant_epilogue_cfg5_shape_against_oracle(dev, mods, oracle):
    """cfg5's fc forward (T=8192, H=2048 -> F=8192): the whole output against
    GEMM + quantizer, and rows / columns of it against the oracle's quantizer
    of the bf16 C."""
    fp4, mg = mods
    apk, ak, bpk, bk = _operands(fp4, dev, 8192, 8192, 2048, seed=5005)
    c, got = _check(fp4, mg, apk, ak, bpk, bk, keep=False)
    cb = c.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    rows = np.arange(0, 8192, 911)
    rq, rsc = oracle.quantize_pack(cb[rows], dtype="bf16")
    assert np.array_equal(got[0].cpu().numpy()[rows], rq)
    assert np.array_equal(got[1].cpu().numpy()[:, rows, :].transpose(1, 0, 2).reshape(len(rows), -1), rsc)
    cols = np.arange(3, 8192, 1013)
    cq, csc = oracle.quantize_pack(np.ascontiguousarray(cb[:, cols].T), dtype="bf16")
    assert np.array_equal(got[2].cpu().numpy()[cols], cq)
    assert np.array_equal(got[3].cpu().numpy()[:, cols, :].transpose(1, 0, 2).reshape(len(cols), -1), csc)


def test_quant_epilogue_other_shapes_fall_back(dev, mods):
    """M = 384 is not a whole number of 256-row tiles: the wrapper runs the
    GEMM and then the quantizer, with the same results."""
    fp4, mg = mods
    _check(fp4, mg, *_operands(fp4, dev, 384, 256, 512, seed=8), keep=True)
