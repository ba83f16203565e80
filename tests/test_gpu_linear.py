"""GPU parity of fp4_linear's MXFP4 forward and quantized backward (cfg5).

For Y = X W^T (X [T, K], W [N, K]) the quantized backward runs
    dX = q_rows(dY) . q_cols(W)        (contraction over N)
    dW = q_cols(dY)^T . q_cols(X)      (contraction over T)
with q_rows / q_cols = fp4.py:57-72 applied along the contraction axis.
The oracle composes its own quantizer on explicitly transposed copies with
the fp64 reference GEMM (fp4.py:103-112), the reference's straight-through
backward (fp4_linear.py:42-45) being the same two products unquantized.
Tolerances (bench.py:71 metric): fp32 out <= 1e-5, bf16 out <= 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fl(dev):
    from lockstep_amd import fp4_linear
    return fp4_linear


def _oracle_backward(oracle, gy, x, w):
    gq = oracle.quantize_pack(gy)                       # dY along N
    wq = oracle.quantize_pack(np.ascontiguousarray(w.T))  # W along N -> [K, N/2]
    dx = oracle.reference_gemm_packed(gq[0], gq[1], wq[0], wq[1])
    gtq = oracle.quantize_pack(np.ascontiguousarray(gy.T))  # dY along T -> [N, T/2]
    xtq = oracle.quantize_pack(np.ascontiguousarray(x.T))   # X along T -> [K, T/2]
    dw = oracle.reference_gemm_packed(gtq[0], gtq[1], xtq[0], xtq[1])
    return dx, dw


@pytest.mark.parametrize("T,K,N", [(256, 384, 512), (128, 128, 128), (512, 256, 384)])
def test_quantized_backward_matches_oracle(dev, fl, oracle, T, K, N):
    x = gen.normal(T * 7 + K, (T, K))
    w = gen.normal(N * 5 + K, (N, K), std=0.02)
    gy = gen.normal(T + N * 3, (T, N))
    xt, wt, gt = (torch.from_numpy(a).to(dev) for a in (x, w, gy))
    dx, dw = fl.mxfp4_backward(gt, xt, wt)
    assert dx.dtype == torch.float32 and dw.dtype == torch.float32
    rdx, rdw = _oracle_backward(oracle, gy, x, w)
    assert oracle.max_rel(dx.cpu().numpy(), rdx) <= 1e-5
    assert oracle.max_rel(dw.cpu().numpy(), rdw) <= 1e-5


def test_quantized_backward_through_autograd(dev, fl, oracle):
    """MXFP4Linear(quantized_backward=True): forward = the MXFP4 forward,
    grads = mxfp4_backward, bit for bit; the default stays straight-through."""
    T, K, N = 256, 512, 384
    torch.manual_seed(5)
    layer = fl.MXFP4Linear(K, N, quantized_backward=True).to(dev)
    x = torch.randn(2, T // 2, K, device=dev, requires_grad=True)
    y = layer(x)
    xq = oracle.quantize_pack(x.detach().reshape(-1, K).cpu().numpy())
    wq = oracle.quantize_pack(layer.weight.detach().cpu().numpy())
    assert oracle.max_rel(y.detach().reshape(-1, N).cpu().numpy(),
                          oracle.reference_gemm_packed(xq[0], xq[1], wq[0], wq[1])) <= 1e-5
    gy = torch.randn_like(y)
    y.backward(gy)
    dx, dw = fl.mxfp4_backward(gy.reshape(-1, N), x.detach().reshape(-1, K), layer.weight.detach())
    assert torch.equal(x.grad.reshape(-1, K), dx) and torch.equal(layer.weight.grad, dw)
    rdx, rdw = _oracle_backward(oracle, gy.reshape(-1, N).cpu().numpy(),
                                x.detach().reshape(-1, K).cpu().numpy(), layer.weight.detach().cpu().numpy())
    assert oracle.max_rel(dx.cpu().numpy(), rdx) <= 1e-5
    assert oracle.max_rel(dw.cpu().numpy(), rdw) <= 1e-5
    # default: the reference's unquantized straight-through backward
    ste = fl.MXFP4Linear(K, N).to(dev)
    assert ste.quantized_backward is False


def test_quantized_backward_bf16(dev, fl, oracle):
    """bf16 master weights and activations (cfg5 dtypes): bf16 grads <= 1e-2."""
    T, K, N = 256, 256, 512
    x = gen.to_bf16_bits(gen.normal(11, (T, K)))
    w = gen.to_bf16_bits(gen.normal(12, (N, K), std=0.02))
    gy = gen.to_bf16_bits(gen.normal(13, (T, N)))
    tb = [torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev) for a in (x, w, gy)]
    dx, dw = fl.mxfp4_backward(tb[2], tb[0], tb[1])
    assert dx.dtype == torch.bfloat16 and dw.dtype == torch.bfloat16
    f = [gen.bf16_bits_to_f32(a) for a in (gy, x, w)]
    rdx, rdw = _oracle_backward(oracle, *f)
    assert oracle.max_rel(dx.float().cpu().numpy(), rdx) <= 1e-2
    assert oracle.max_rel(dw.float().cpu().numpy(), rdw) <= 1e-2
    # the bf16 result is the RNE rounding of the fp32-output GEMMs
    dx32, dw32 = fl.mxfp4_backward(tb[2], tb[0].float(), tb[1].float())
    assert torch.equal(dx, dx32.to(torch.bfloat16)) and torch.equal(dw, dw32.to(torch.bfloat16))


def test_quantized_backward_rejects_ragged(dev, fl):
    x = torch.zeros((100, 128), device=dev)
    w = torch.zeros((128, 128), device=dev)
    with pytest.raises(AssertionError, match="multiples of 128"):
        fl.mxfp4_backward(torch.zeros((100, 128), device=dev), x, w)
