"""lsmx_gemm_bf16f4_noalloc: the weight-only GEMM with the split-K partial
tiles in the library's fixed device scratch instead of a caller workspace.

Called through the C-ABI and checked bit for bit against lsmx_gemm_bf16f4_ws
with a caller workspace (the same kernels in the same order), single and dual
form, on two calls in a row, the second at a smaller shape (the scratch keeps
the first call's partials; nothing in it has to start at zero), then a shape
that takes the whole-K kernels (no scratch)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(dev, fp4, M, N, K, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    a0 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    return a0, a1, wpk, we8


def _run(C, entry, a0, a1, wpk, we8, M, N, K, ws=None):
    c0 = torch.full((M, N), float("nan"), device=a0.device, dtype=torch.float32)
    c1 = torch.full_like(c0, float("nan")) if a1 is not None else None
    args = [a0.data_ptr(), a1.data_ptr() if a1 is not None else None, K, wpk.data_ptr(), K // 2, we8.data_ptr(),
            K // 32, C.SCALE_E8M0, c0.data_ptr(), c1.data_ptr() if c1 is not None else None, C.F32, N, M, N, K]
    if entry == "lsmx_gemm_bf16f4_ws":
        args += [ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0]
    C.call(entry, *args, C.stream_of(c0))
    return c0, c1


@pytest.mark.parametrize("dual", [False, True])
def test_noalloc_matches_workspace_form(dual):
    from lockstep_amd import _capi as C
    from lockstep_amd import fp4
    dev = torch.device("cuda", 0)
    L = C.load()
    # 1: M = 128 against a 14336 x 4096 weight (4 K slices, the largest
    # scratch use of this weight); 2: a smaller split shape; 3: whole K
    for M, N, K, split in ((128, 14336, 4096, True), (64, 2304, 2048, True), (2048, 4096, 1024, False)):
        print(f"[noalloc] dual={dual} M={M} N={N} K={K}", flush=True)
        need = L.lsmx_gemm_bf16f4_workspace(M, N, K, int(dual))
        assert (need > 0) == split
        a0, a1, wpk, we8 = _operands(dev, fp4, M, N, K, seed=M + N + K)
        a1 = a1 if dual else None
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev) if split else None
        ref0, ref1 = _run(C, "lsmx_gemm_bf16f4_ws", a0, a1, wpk, we8, M, N, K, ws)
        got0, got1 = _run(C, "lsmx_gemm_bf16f4_noalloc", a0, a1, wpk, we8, M, N, K)
        torch.cuda.synchronize()
        assert not torch.isnan(ref0).any()
        assert torch.equal(got0, ref0)
        if dual:
            assert torch.equal(got1, ref1)
        # a second call on the same scratch gives the same bits
        again, _ = _run(C, "lsmx_gemm_bf16f4_noalloc", a0, a1, wpk, we8, M, N, K)
        assert torch.equal(again, ref0)


def test_noalloc_validates_like_the_workspace_form():
    from lockstep_amd import _capi as C
    L = C.load()
    # a1 without c1
    rc = L.lsmx_gemm_bf16f4_noalloc(16, 16, 4096, 16, 2048, 16, 128, C.SCALE_E8M0, 16, None, C.F32, 14336, 128,
                                    14336, 4096, None)
    assert rc == C.ERR_ARG
    assert "a1 and c1" in C.last_error()


def test_noalloc_allocates_nothing_and_replays_under_graph_capture():
    """After a first call on the device (which looks up the scratch address),
    a call changes neither torch's allocator nor the device's free memory; and
    the call captured in a CUDA graph replays to the eager bits (the stated
    use: callers that cannot allocate, such as code under graph capture)."""
    from lockstep_amd import _capi as C
    from lockstep_amd import fp4
    dev = torch.device("cuda", 0)
    M, N, K = 128, 14336, 4096
    print(f"[noalloc] capture M={M} N={N} K={K}", flush=True)
    assert C.load().lsmx_gemm_bf16f4_workspace(M, N, K, 0) > 0, "this shape must use the scratch"
    a0, _, wpk, we8 = _operands(dev, fp4, M, N, K, seed=5)
    c = torch.empty((M, N), device=dev, dtype=torch.float32)

    def call():
        C.call("lsmx_gemm_bf16f4_noalloc", a0.data_ptr(), None, K, wpk.data_ptr(), K // 2, we8.data_ptr(), K // 32,
               C.SCALE_E8M0, c.data_ptr(), None, C.F32, N, M, N, K, C.stream_of(c))

    call()
    torch.cuda.synchronize()
    ref = c.clone()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    alloc0, reserved0 = torch.cuda.memory_allocated(), torch.cuda.memory_reserved()
    call()
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert (torch.cuda.memory_allocated(), torch.cuda.memory_reserved()) == (alloc0, reserved0)
    assert free1 == free0
    assert torch.equal(c, ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        c.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, ref)
