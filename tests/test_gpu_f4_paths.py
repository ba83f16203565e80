"""GPU: every scale format of the f4 x f4 GEMM gives the same bits, and the
reference's call spelling runs the fast kernels.

lsmx_gemm_f4f4 runs K-major E8M0 scales with K % 256 == 0 on the 16 x 16 x 128
kernel and every other case (row-major E8M0, fp32 powers of two, K % 256 !=
0) on the 32 x 32 x 64 kernel.  Both accumulate each output over the same
32-blocks in the same order, so the C ABI's three scale formats must agree bit
for bit; the Python layer regroups every format to K-major, so the
reference's spelling -- quantize_mxfp4 (fp32 scales) + pack_fp4 +
mxfp4_gemm_packed, fp4_linear.py:36-39 -- must give the bits of the K-major
call.  The weight-only GEMM converts fp32 weight scales to E8M0 bytes, so the
ring and split-K kernels run for both forms and the bits agree too.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(dev):
    from lockstep_amd import _capi, fp4, mxfp4_gemm
    return _capi, fp4, mxfp4_gemm


def _c_abi_gemm(C, apk, bpk, sa, sb, fmt, M, N, K, out_dtype):
    c = torch.empty((M, N), device=apk.device, dtype=out_dtype)
    lsa = M if fmt == C.SCALE_E8M0_KMAJOR else sa.stride(0)
    lsb = N if fmt == C.SCALE_E8M0_KMAJOR else sb.stride(0)
    C.call("lsmx_gemm_f4f4", apk.data_ptr(), K // 2, sa.data_ptr(), lsa, bpk.data_ptr(), K // 2, sb.data_ptr(), lsb,
           fmt, c.data_ptr(), C.dtype_code(out_dtype), N, M, N, K, C.stream_of(c))
    return c


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (37, 129, 384), (300, 513, 128), (1024, 768, 2048),
                                   (513, 260, 1280)])
def test_c_abi_scale_formats_give_identical_bits(dev, mods, oracle, out_dtype, M, N, K):
    C, fp4, _ = mods
    g = torch.Generator(device=dev).manual_seed(M * 3 + N + K)
    a = torch.randn((M, K), device=dev, generator=g)
    b = torch.randn((N, K), device=dev, generator=g) * 0.02
    apk, ae8 = fp4.quantize_pack_mxfp4(a)
    bpk, be8 = fp4.quantize_pack_mxfp4(b)
    _, ak = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    _, bk = fp4.quantize_pack_mxfp4(b, scale_layout="kmajor")
    _, af = fp4.quantize_mxfp4(a)
    _, bf = fp4.quantize_mxfp4(b)
    c_km = _c_abi_gemm(C, apk, bpk, ak, bk, C.SCALE_E8M0_KMAJOR, M, N, K, out_dtype)
    c_rows = _c_abi_gemm(C, apk, bpk, ae8, be8, C.SCALE_E8M0, M, N, K, out_dtype)
    c_f32 = _c_abi_gemm(C, apk, bpk, af.contiguous(), bf.contiguous(), C.SCALE_F32, M, N, K, out_dtype)
    assert torch.equal(c_km, c_rows) and torch.equal(c_km, c_f32)
    ref = oracle.reference_gemm_packed(*[t.cpu().numpy() for t in (apk, ae8, bpk, be8)])
    tol = 1e-5 if out_dtype == torch.float32 else 1e-2
    assert oracle.max_rel(c_km.float().cpu().numpy(), ref) <= tol


def test_reference_spelling_at_cfg4_runs_the_kmajor_kernel(dev, mods, oracle):
    """cfg4 (8192^3, A, B = 0.05 * t3) through fp4_linear.py:36-39's spelling:
    fp32 scales from quantize_mxfp4, codes through pack_fp4, then
    mxfp4_gemm_packed -- bit-equal to the K-major E8M0 call over the whole
    [8192, 8192] bf16 output."""
    _, fp4, mg = mods
    n = 8192
    g = torch.Generator(device=dev).manual_seed(4001)

    def t3():
        z = torch.randn((n, n), device=dev, generator=g)
        chi = torch.zeros_like(z)
        for _ in range(3):
            chi += torch.randn((n, n), device=dev, generator=g).square()
        return z / torch.sqrt(chi / 3.0) * 0.05

    a, b = t3(), t3()
    ac, as32 = fp4.quantize_mxfp4(a)
    bc, bs32 = fp4.quantize_mxfp4(b)
    c_ref_spelling = mg.mxfp4_gemm_packed(fp4.pack_fp4(ac), fp4.pack_fp4(bc), as32, bs32)
    del ac, bc
    apk, ak = fp4.quantize_pack_mxfp4(a, scale_layout="kmajor")
    bpk, bk = fp4.quantize_pack_mxfp4(b, scale_layout="kmajor")
    del a, b
    c_km = mg.mxfp4_gemm_packed(apk, bpk, ak, bk)
    assert c_ref_spelling.dtype == torch.bfloat16
    assert torch.equal(c_ref_spelling, c_km)
    rows, cols = np.arange(0, n, 97), np.arange(0, n, 89)
    ar = mg._e8m0_rows(as32, n, n // 32, transposed=False).cpu().numpy()
    br = mg._e8m0_rows(bs32, n, n // 32, transposed=False).cpu().numpy()
    ref = oracle.reference_gemm_packed(apk.cpu().numpy(), ar, bpk.cpu().numpy(), br, rows=rows, cols=cols)
    assert oracle.max_rel(c_km.float().cpu().numpy()[np.ix_(rows, cols)], ref) <= 1e-2


@pytest.mark.parametrize("M", [1024, 128, 1])
def test_weight_only_fp32_and_e8m0_scales_give_identical_bits(dev, mods, M):
    """cfg3's weight [14336, 4096]: the fp32 form of the weight scales runs the
    kernels of the E8M0 form (ring at M = 1024, split-K at M = 128, GEMV at
    M = 1) and gives the same bits."""
    _, fp4, mg = mods
    N, K = 14336, 4096
    g = torch.Generator(device=dev).manual_seed(M + 77)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    _, ws32 = fp4.quantize_mxfp4(w)
    c8 = mg.mxfp4_gemm_bf16(a, wpk, we8)
    c32 = mg.mxfp4_gemm_bf16(a, wpk, ws32)
    assert torch.equal(c8, c32)


def test_split_k_weight_only_under_graph_capture(dev, mods):
    """A split-K weight-only GEMM captured in a CUDA graph owns its workspace:
    replays, interleaved with eager calls at other split shapes (which use and
    grow the cached per-stream workspace), give the eager bits every time."""
    C, fp4, mg = mods
    M, N, K = 128, 14336, 4096
    assert C.load().lsmx_gemm_bf16f4_workspace(M, N, K, 0) > 0, "this shape must take the split-K path"
    g = torch.Generator(device=dev).manual_seed(9)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    eager = mg.mxfp4_gemm_bf16(a, wpk, we8)
    w2 = torch.randn((2 * N, K), device=dev, generator=g) * 0.02
    w2pk, w2e8 = fp4.quantize_pack_mxfp4(w2)
    a2 = torch.randn((256, K), device=dev, generator=g).to(torch.bfloat16)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mg.mxfp4_gemm_bf16(a, wpk, we8)       # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = mg.mxfp4_gemm_bf16(a, wpk, we8)
    for _ in range(3):
        other = mg.mxfp4_gemm_bf16(a2, w2pk, w2e8)   # eager, larger workspace
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert other.shape == (256, 2 * N)
