"""Benchmark of the MI355X MXFP4 hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--suite PATH]

Workload (BASELINE cfg4, the config the headline metric is quoted on):
A, B fp32 [8192, 8192] = 0.05 * Student-t(3), resident in HBM.  One step =
quantize A along K (fused quantize+pack, E8M0 scales) + quantize B along K +
f4 x f4 block-scaled GEMM (v_mfma_scale_f32_32x32x64_f8f6f4), bf16 out.

`value` is the whole step's rate, 2*M*N*K / step time.  `gemm` and `quantize`
give per-kernel rates from HIP events recorded on the stream the kernels run
on, and `roofline` prices the dominant kernel (the GEMM) against MI355X's
dense FP4 MFMA peak; `roofline_quantize` prices the quantizer against HBM.
`cpu_baseline` times the CPU oracle (a restatement of the reference's CPU
path: fp4.py quantizer + dequantize-then-fp32-matmul, the fake-quant branch
of fp4_linear.py:40) on this host, on rank 0 only.

--suite PATH also measures the other BASELINE configs (dual-batch cfg2, the
weight-only cfg3 sweep) and writes one JSON line each to PATH.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP4_TFLOPS = 10100.0     # MI355X dense MXFP4 MFMA
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    # ~10 ms of untimed steps: the first few milliseconds of load after idle
    # run ~5% slower while the clocks settle
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--size", type=int, default=8192)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--suite", default=None, help="also bench cfg2/cfg3, one JSON line each to this file")
    p.add_argument("--calib", action="store_true",
                   help="also run a plain 256 MiB device copy (the reference kernel for HBM counters)")
    return p.parse_args()


def median(xs):
    s = sorted(xs)
    return s[len(s) // 2] if s else float("nan")


def t3(n, gen, dev, torch):
    z = torch.randn((n, n), device=dev, generator=gen)
    chi = torch.zeros_like(z)
    for _ in range(3):
        chi += torch.randn((n, n), device=dev, generator=gen).square()
    return (z / torch.sqrt(chi / 3.0) * 0.05).contiguous()


def traffic_from_profiles(kernel_prefix: str):
    """HBM bytes per launch from committed rocprofv3 --pmc summaries, if any."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        data = json.loads(f.read_text())
        return data.get(kernel_prefix, {}).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


def cpu_baseline(n: int):
    """Time the CPU oracle on the cfg4 workload: quantize A and B (C oracle,
    OpenMP), dequantize, fp32 A @ B^T (numpy/OpenBLAS) -- the fake-quant CPU
    path of fp4_linear.py:40 restated.  Rate = 2*R*n*n / time for R rows of C
    (R = n unless that would exceed ~30 s)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    cores = min(len(os.sched_getaffinity(0)), 16)
    O.lib()
    rng = np.random.default_rng(4001)
    R = n
    a = (rng.standard_t(3, (R, n)) * 0.05).astype(np.float32)
    b = (rng.standard_t(3, (n, n)) * 0.05).astype(np.float32)
    with threadpool_limits(limits=cores):
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            ac, as_ = O.quantize_mxfp4(a)
            bc, bs_ = O.quantize_mxfp4(b)
            A = O.dequantize_mxfp4(ac, as_)
            B = O.dequantize_mxfp4(bc, bs_)
            C = A @ B.T
            times.append(time.perf_counter() - t0)
            del C, A, B
    t = min(times)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(2.0 * R * n * n / t / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "cpu_model": model,
            "sample": f"full cfg4 ({R}x{n}x{n}): quantize A and B with the C oracle (OpenMP, "
                      f"{O.num_threads()} threads), dequantize, fp32 A@B^T (numpy/OpenBLAS, {cores} threads); "
                      f"{t:.2f} s per step, best of 2",
            "seconds": round(t, 3)}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch

    from lockstep_amd import fp4, mxfp4_gemm
    from lockstep_amd import _capi

    _capi.load()
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(0)
    n = args.size
    g = torch.Generator(device=dev).manual_seed(4001)
    A = t3(n, g, dev, torch)
    B = t3(n, g, dev, torch)
    torch.cuda.synchronize()

    def step(ev=None):
        if ev:
            ev[0].record()
        apk, ae8 = fp4.quantize_pack_mxfp4(A, scale_layout="kmajor")
        if ev:
            ev[1].record()
        bpk, be8 = fp4.quantize_pack_mxfp4(B, scale_layout="kmajor")
        if ev:
            ev[2].record()
        c = mxfp4_gemm.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.bfloat16)
        if ev:
            ev[3].record()
        return c

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: exactly `steps` steps, synchronized on both sides
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    # per-kernel durations from HIP events on the kernels' stream; a spin
    # kernel ahead of each step keeps the GPU busy while the host enqueues,
    # so no event interval includes host launch time
    qa, qb, gm = [], [], []
    for _ in range(max(args.steps, 5)):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        torch.cuda._sleep(2_000_000)
        step(ev)
        torch.cuda.synchronize()
        qa.append(ev[0].elapsed_time(ev[1]))
        qb.append(ev[1].elapsed_time(ev[2]))
        gm.append(ev[2].elapsed_time(ev[3]))
    gemm_ms = median(gm)
    quant_ms = median(qa + qb)

    flop = 2.0 * n * n * n
    gemm_tflops = flop / (gemm_ms * 1e-3) / 1e12
    q_bytes = n * n * (4 + 0.5 + 1.0 / 32)            # fp32 in, packed nibbles + E8M0 out
    quant_gbs = q_bytes / (quant_ms * 1e-3) / 1e9
    value = flop / (ms_per_step * 1e-3) / 1e12

    out = {
        "metric": f"MXFP4 GEMM TFLOPS at {n}^3 (cfg4: on-the-fly quantize of A and B + f4xf4 GEMM)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 (e2m1 x e2m1, e8m0 scales, fp32 accumulate, bf16 out)",
        "data": "synthetic: A, B = 0.05 * Student-t(df=3), torch.Generator(seed 4001) on device, fp32",
        "config": {"workload": "cfg4 fully-FP4 GEMM", "M": n, "N": n, "K": n, "input_dtype": "f32",
                   "out_dtype": "bf16", "block": 32, "parallelism": "single GPU"},
        "device": props.name,
        "gemm": {"ms": round(gemm_ms, 4), "tflops": round(gemm_tflops, 1),
                 "frac_fp4_peak": round(gemm_tflops / PEAK_FP4_TFLOPS, 4)},
        "quantize": {"ms_per_operand": round(quant_ms, 4), "gbs": round(quant_gbs, 1),
                     "frac_hbm": round(quant_gbs / PEAK_HBM_GBS, 4),
                     "bytes_per_launch": int(q_bytes)},
        "roofline": {"bound": "mfma", "kernel": "gemm_f4f4_kernel", "achieved": round(gemm_tflops, 1),
                     "peak": PEAK_FP4_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / PEAK_FP4_TFLOPS, 4),
                     "traffic": traffic_from_profiles("gemm_f4f4_kernel")},
        "roofline_quantize": {"bound": "hbm", "kernel": "quantize_rows_kernel", "achieved": round(quant_gbs, 1),
                              "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(quant_gbs / PEAK_HBM_GBS, 4),
                              "traffic": traffic_from_profiles("quantize_rows_kernel")},
    }
    if args.suite:
        run_suite(args.suite, torch, dev)
    if args.calib:
        # plain copy of known size: 256 MiB read + 256 MiB written per launch
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).uniform_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = src.numel() * 4
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(n)
    print(json.dumps(out), flush=True)


def _time_events(fn, reps=20, warm=3):
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)   # the host enqueues fn while the GPU spins
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return median(ts)


def run_suite(path, torch, dev):
    """cfg2 (dual-batch) and cfg3 (weight-only sweep), one JSON line each."""
    from lockstep_amd import dual_gemm, fp4, mxfp4_gemm
    lines = []
    g = torch.Generator(device=dev).manual_seed(2001)
    # cfg2: A0, A1 bf16 [2048, 4096], W [4096, 4096] MXFP4
    a0 = torch.randn((2048, 4096), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((2048, 4096), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn((4096, 4096), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w)
    ms = _time_events(lambda: dual_gemm.dual_mxfp4(a0, a1, wpk, we8))
    fl = 2.0 * 2 * 2048 * 4096 * 4096
    lines.append({"config": "cfg2 dual-batch bf16 x mxfp4, 2x[2048,4096] . [4096,4096]^T", "ms": ms,
                  "tflops": fl / ms / 1e9, "frac_bf16_peak": fl / ms / 1e9 / PEAK_BF16_TFLOPS})
    ms2 = _time_events(lambda: (mxfp4_gemm.mxfp4_gemm_bf16(a0, wpk, we8), mxfp4_gemm.mxfp4_gemm_bf16(a1, wpk, we8)))
    lines[-1]["two_launch_ms"] = ms2
    # cfg3: W [14336, 4096], M sweep
    w3 = torch.randn((14336, 4096), device=dev, generator=g) * 0.02
    w3pk, w3e8 = fp4.quantize_pack_mxfp4(w3)
    for M in (1, 16, 128, 1024, 8192):
        a = torch.randn((M, 4096), device=dev, generator=g).to(torch.bfloat16)
        ms = _time_events(lambda: mxfp4_gemm.mxfp4_gemm_bf16(a, w3pk, w3e8))
        fl = 2.0 * M * 14336 * 4096
        by = 14336 * 4096 * (0.5 + 1 / 32) + 2 * M * 4096 + 2 * M * 14336
        lines.append({"config": f"cfg3 weight-only bf16 x mxfp4, M={M}, N=14336, K=4096", "ms": ms,
                      "tflops": fl / ms / 1e9, "gbs": by / ms / 1e6,
                      "frac_bf16_peak": fl / ms / 1e9 / PEAK_BF16_TFLOPS, "frac_hbm": by / ms / 1e6 / PEAK_HBM_GBS})
    lines.append(bench_cfg5(torch, dev))
    lines += bench_reference_rows(torch, dev)
    with open(path, "w") as f:
        for ln in lines:
            f.write(json.dumps(ln) + "\n")
            print(json.dumps(ln), file=sys.stderr, flush=True)


def bench_reference_rows(torch, dev, n=4096):
    """The throughput rows of the reference's own bench.py at its default
    4096^3 (bench.py:98-107 mxfp4 rows, :163-176 dual rows): mxfp4_gemm_fp8
    and mxfp4_gemm_packed, then the dense dual GEMMs on bf16 operands."""
    from lockstep_amd import dual_gemm as dg
    from lockstep_amd import fp4, mxfp4_gemm as mg
    g = torch.Generator(device=dev).manual_seed(4001)
    fl1 = 2.0 * n ** 3
    rows = []

    def row(name, ms, flops, peak):
        rows.append({"config": f"ref-bench {name}, {n}^3", "ms": ms, "tflops": flops / ms / 1e9,
                     "frac_peak": flops / ms / 1e9 / peak})

    a = torch.randn((n, n), device=dev, generator=g)
    b = torch.randn((n, n), device=dev, generator=g)
    a_pk, a_e8 = fp4.quantize_pack_mxfp4(a)
    bt_pk, bt_e8 = fp4.quantize_pack_mxfp4(b.t().contiguous())
    a_f8 = fp4.codes_to_e4m3(fp4.unpack_fp4(a_pk))
    bt_f8 = fp4.codes_to_e4m3(fp4.unpack_fp4(bt_pk))
    b_f8 = bt_f8.t().contiguous()                      # [K, N] N-contiguous, as the reference passes it
    a_s, bt_s = fp4.e8m0_to_scale(a_e8), fp4.e8m0_to_scale(bt_e8)
    b_s = bt_s.t().contiguous()
    row("mxfp4_gemm_fp8 (N-contiguous B: transposed on the device each call)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, b_f8, a_s, b_s)), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_fp8 (B passed as a view of K-contiguous rows)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, bt_f8.t(), a_s, bt_s.t())), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_fp8 (E8M0 byte scales, regrouped to K-major on the device)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, bt_f8.t(), a_e8, bt_e8.t())), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_packed (f4 x f4)", _time_events(lambda: mg.mxfp4_gemm_packed(a_pk, bt_pk, a_e8, bt_e8)),
        fl1, PEAK_FP4_TFLOPS)
    a1 = torch.randn((n, n), device=dev, generator=g).to(torch.bfloat16)
    a2 = torch.randn((n, n), device=dev, generator=g).to(torch.bfloat16)
    b1 = torch.randn((n, n), device=dev, generator=g).to(torch.bfloat16)
    b2 = torch.randn((n, n), device=dev, generator=g).to(torch.bfloat16)
    fl2 = 2 * fl1
    row("dual: 2x torch.matmul (two launches)", _time_events(lambda: (a1 @ b1, a2 @ b2)), fl2, PEAK_BF16_TFLOPS)
    row("dual: fused, two accumulators (dual_separate)", _time_events(lambda: dg.dual_separate(a1, a2, b1, b2)),
        fl2, PEAK_BF16_TFLOPS)
    row("dual: fused, one packed accumulator (dual_packed)",
        _time_events(lambda: dg.dual_packed(a1, a2, b1, b2)), fl2, PEAK_BF16_TFLOPS)
    # splitk_*: at 4096^2 the 256 x 256 output tiles already fill every CU, so
    # the library runs the whole K per tile; the sliced, atomic form is the
    # one it takes for small outputs (timed below at M = N = 512)
    for splits in (4, 8):
        row(f"dual: split-K={splits}, two accumulators (whole K per tile: the tiles fill the GPU)",
            _time_events(lambda s=splits: dg.splitk_separate(a1, a2, b1, b2, s)), fl2, PEAK_BF16_TFLOPS)
        row(f"dual: split-K={splits}, one accumulator (whole K per tile: the tiles fill the GPU)",
            _time_events(lambda s=splits: dg.splitk_packed(a1, a2, b1, b2, s)), fl2, PEAK_BF16_TFLOPS)
    sm = 512
    fls = 4.0 * sm * sm * n
    for splits in (4, 8):
        rows.append({"config": f"ref-bench dual: split-K={splits}, two accumulators, {sm}x{sm}x{n} (K slices, atomics)",
                     "ms": (ms := _time_events(lambda s=splits: dg.splitk_separate(a1[:sm], a2[:sm], b1[:, :sm],
                                                                                   b2[:, :sm], s))),
                     "tflops": fls / ms / 1e9, "frac_peak": fls / ms / 1e9 / PEAK_BF16_TFLOPS})
    row("dual_separate, shared weight (b1 is b2)", _time_events(lambda: dg.dual_separate(a1, a2, b1, b1)),
        fl2, PEAK_BF16_TFLOPS)
    bt1 = b1.t().contiguous()
    row("gemm (bf16, B a view of K-contiguous rows)", _time_events(lambda: dg.gemm(a1, bt1.t())), fl1,
        PEAK_BF16_TFLOPS)
    # FP4 -> E4M3 expansion throughput (cuda/mxfp4_mma_gemm.cu:270-287): 64 Mi
    # words of 8 codes, 4 bytes read and 8 written per word, source bytes 0x5A
    n32 = 64 << 20
    up = torch.full((n32,), 0x5A5A5A5A, dtype=torch.int32, device=dev)
    ms = _time_events(lambda: fp4.fp4_to_e4m3_words(up))
    by = 12.0 * n32
    rows.append({"config": "ref-bench fp4 -> e4m3 expansion, 64 Mi words (512 Mi codes)", "ms": ms,
                 "gbs": by / ms / 1e6, "frac_hbm": by / ms / 1e6 / PEAK_HBM_GBS})
    return rows


def bench_cfg5(torch, dev, T=8192, H=2048, F=8192):
    """cfg5: one MLP block (fc H->F, out F->H) forward + MXFP4 backward.
    Per linear: quantize X and W along K + GEMM (fprop), dY along N and W
    along its columns + GEMM (dgrad), dY and X along T + GEMM (wgrad)."""
    from lockstep_amd import fp4_linear as fl
    g = torch.Generator(device=dev).manual_seed(5001)
    x = torch.randn((T, H), device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn((F, H), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((H, F), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn((T, H), device=dev, generator=g).to(torch.bfloat16)

    def step():
        h = fl._forward_hip(x, w1)                 # [T, F]
        fl._forward_hip(h, w2)                     # [T, H]
        dh, _ = fl.mxfp4_backward(dy, h, w2)       # dgrad + wgrad of out
        fl.mxfp4_backward(dh, x, w1)               # dgrad + wgrad of fc
    ms = _time_events(step, reps=10, warm=2)
    fl_ = 6 * 2.0 * T * F * H
    return {"config": f"cfg5 MLP block fwd + MXFP4 bwd, tokens={T} hidden={H} ffn={F}, bf16 in/out",
            "ms": ms, "tflops": fl_ / ms / 1e9, "frac_fp4_peak": fl_ / ms / 1e9 / PEAK_FP4_TFLOPS,
            "work": "12 quantizations + 6 f4xf4 GEMMs (1.649e12 FLOP)"}


if __name__ == "__main__":
    main()
