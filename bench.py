"""Benchmark of the MI355X MXFP4 hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-configs] [--suite PATH]

Headline workload (BASELINE cfg4, the config the metric is quoted on):
A, B fp32 [8192, 8192] = 0.05 * Student-t(3), resident in HBM.  One step =
quantize A and B along K (fused quantize+pack, K-major E8M0 scales, both
operands in one launch) + f4 x f4 block-scaled GEMM
(v_mfma_scale_f32_16x16x128_f8f6f4), bf16 out.  `value` is 2*M*N*K / step
time over the timed region.

Order: the configs' GPU measurements, the cfg4 per-kernel timings (the
GEMM's back-to-back loop last), the headline (W warm-up steps, K timed
steps), then every CPU baseline: the headline's warm-up starts on a GPU
that has been under load, not after an idle period.

Alongside it:
  gemm / quantize     per-kernel rates from HIP events recorded on the
                      stream the kernels run on (median of isolated launches)
  gemm_sustained      the GEMM back to back (events around a loop of
                      launches): the rate under sustained load, when the
                      clock has dropped
  roofline            the dominant kernel (the GEMM) against MI355X's dense
                      FP4 MFMA peak, plus the fraction at the clock rocprof
                      measured for this kernel (GRBM_GUI_ACTIVE / duration,
                      profiles/clock.json)
  roofline_quantize   the quantizer against HBM
  configs             every BASELINE config (cfg1 ... cfg5) with its rate,
                      the roofline of its dominant kernel and its own
                      cpu_baseline
  cpu_baseline        the CPU oracle (a restatement of the reference's CPU
                      path: fp4.py quantizer + dequantize-then-fp32-matmul,
                      the fake-quant branch of fp4_linear.py:40) on this
                      host's cores, median of 3 runs after a warm-up

--suite PATH also measures the reference bench's own 4096^3 rows (its
mxfp4 and dual GEMM throughput rows) and writes one JSON line each to PATH.
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

PEAK_FP4_TFLOPS = 10100.0     # MI355X dense MXFP4 MFMA (2.4 GHz)
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
# vector-ALU fp32 operations issued without packed math (this build disables
# it): 256 CUs x 4 SIMDs x 16 lanes per clock x 2.4 GHz
PEAK_VALU_GOPS = 39321.6
NOMINAL_GHZ = 2.4


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--size", type=int, default=8192)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--no-configs", action="store_true", help="headline (cfg4) only")
    p.add_argument("--suite", default=None, help="also bench the reference bench's rows, JSON lines to this file")
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


def _profile_json(name):
    f = ROOT / "profiles" / name
    if not f.exists():
        return {}
    try:
        return json.loads(f.read_text())
    except (ValueError, OSError):
        return {}


def traffic_from_profiles(kernel_prefix: str):
    """HBM bytes per launch from committed rocprofv3 --pmc summaries, if any."""
    return _profile_json("traffic.json").get(kernel_prefix, {}).get("bytes_per_launch")


def clock_from_profiles(kernel_prefix: str):
    """Average graphics clock (GHz) rocprofv3 measured over this kernel's
    launches (GRBM_GUI_ACTIVE cycles per XCD / duration), if committed."""
    return _profile_json("clock.json").get(kernel_prefix, {}).get("ghz")


def roofline(bound, kernel, achieved, peak, unit, traffic=None, clock_ghz=None):
    r = {"bound": bound, "kernel": kernel, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "traffic": traffic}
    if clock_ghz:
        r["measured_clock_ghz"] = clock_ghz
        r["frac_at_measured_clock"] = round(achieved / (peak * clock_ghz / NOMINAL_GHZ), 4)
    return r


# ----------------------------------------------------------------- CPU legs
def cpu_cores():
    """Threads for the CPU legs: this process's CPUs, capped at the CPU share
    the host gives one GPU's job when it says so (OMP_NUM_THREADS)."""
    avail = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    return (min(avail, int(share)) if share and share.isdigit() and int(share) > 0 else avail), avail


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        return ""


def time_cpu(fn, runs=3):
    """Median wall time of `runs` calls after one warm-up call."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return median(ts)


def cpu_leg(fn, work, unit, sample):
    """Time the CPU restatement of a config on this host (oracle C quantizer
    with OpenMP, numpy/OpenBLAS fp32 matmul) and rate it in `unit`."""
    from threadpoolctl import threadpool_limits
    from oracle import oracle as O
    cores, avail = cpu_cores()
    O.lib()
    with threadpool_limits(limits=cores):
        t = time_cpu(fn)
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": round(work / t / scale, 4), "unit": unit, "cores": cores, "host_cpus_visible": avail,
            "kind": "port", "cpu_model": cpu_model(), "sample": sample + f"; median of 3 after a warm-up",
            "seconds": round(t, 4)}


def _bf16_to_f32_np(t):
    """bf16 torch tensor -> fp32 numpy (exact)."""
    import numpy as np
    import torch
    return (t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)


def cpu_quant_deq(O, x, dtype=None):
    """fp4.py:57-78 on the CPU: quantize along the last axis, dequantize."""
    c, s = O.quantize_mxfp4(x, 32, dtype)
    return O.dequantize_mxfp4(c, s)


# ----------------------------------------------------------------- GPU timing
def _time_events(fn, reps=20, warm=3):
    """Median event time of fn: a spin kernel ahead of each call keeps the GPU
    busy while the host enqueues, so no interval includes host launch time."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return median(ts)


def _time_ops(ops, reps=10, warm=2):
    """A sequence of ops run as one step: (per-op median event times, median
    step time).  The per-op times come from steps with an event between ops;
    the step time from steps with events only at their ends, since each
    event between two kernels adds a few microseconds of its own."""
    import torch
    for _ in range(warm):
        for _, f in ops:
            f()
    torch.cuda.synchronize()
    per = {name: [] for name, _ in ops}
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(ops) + 1)]
        torch.cuda._sleep(2_000_000)
        ev[0].record()
        for i, (_, f) in enumerate(ops):
            f()
            ev[i + 1].record()
        torch.cuda.synchronize()
        for i, (name, _) in enumerate(ops):
            per[name].append(ev[i].elapsed_time(ev[i + 1]))
    tot = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        e0.record()
        for _, f in ops:
            f()
        e1.record()
        torch.cuda.synchronize()
        tot.append(e0.elapsed_time(e1))
    return {k: median(v) for k, v in per.items()}, median(tot)


def _time_batch(fns, reps=10, warm=2):
    """Average launch time inside a stream: events around the calls fns[0],
    fns[1], ... back to back (callers rotate inputs larger than the 256 MB
    MALL between them, so no call finds its operands in cache), divided by
    their number; median over reps.  Unlike an event pair around one call,
    the ~3 us it takes an event to reach the GPU is spread over the batch."""
    import torch
    for _ in range(warm):
        for f in fns:
            f()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        e0.record()
        for f in fns:
            f()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) / len(fns))
    return median(ts)


def _time_loop(fn, n=50):
    """Average time of n back-to-back calls (events around the loop)."""
    import torch
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


# ----------------------------------------------------------------- main
def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path: every GPU box here has one GPU", file=sys.stderr)
        sys.exit(2)

    import torch

    from lockstep_amd import _capi, device, fp4, mxfp4_gemm

    # the reference's bench starts with require_h100() (h100.py:8-15); here
    # the kernels are gfx950 code objects
    props = device.require_gfx950()
    _capi.load()
    dev = torch.device("cuda", 0)
    n = args.size
    g = torch.Generator(device=dev).manual_seed(4001)
    A = t3(n, g, dev, torch)
    B = t3(n, g, dev, torch)
    torch.cuda.synchronize()

    # Every GPU measurement first, the CPU baselines last.  The config rows
    # run before the headline, so its warm-up starts on a GPU already under
    # load: from idle the chip first runs at its boost clock, then its power
    # management throttles it for a few milliseconds before the clock settles
    # (cfg4 steps 6-40 after idle measured 0.34-0.41 ms against 0.33 ms
    # settled), and a short warm-up alone would time that transient.
    deferred = None if args.no_cpu else []
    config_rows = run_configs(torch, dev, deferred) if not args.no_configs else None
    torch.cuda.synchronize()

    def step(ev=None):
        if ev:
            ev[0].record()
        # both operands in one launch (lsmx_quantize_mxfp4_batch): the same
        # bytes as two quantize_pack_mxfp4 calls, without a drain and a
        # ramp-up between them
        (apk, ae8), (bpk, be8) = fp4.quantize_pack_mxfp4_many((A, B), scale_layout="kmajor")
        if ev:
            ev[1].record()
        c = mxfp4_gemm.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.bfloat16)
        if ev:
            ev[2].record()
        return c

    # Per-kernel timings first (isolated launches after a spin kernel, the
    # quantizer's average launch, the reference-spelling row, the GEMM back
    # to back), then the step itself back to back (step_sustained, ~13 ms),
    # right before the headline's warm-up: the timed steps then run at the
    # step's own sustained clock, not in the power transient that follows
    # an idle period (a throttling dip after the boost) or another workload
    # (after the GEMM-only loop the clock briefly runs above the step's
    # settled value).
    qab, gm = [], []
    for _ in range(max(args.steps, 5)):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda._sleep(2_000_000)
        step(ev)
        torch.cuda.synchronize()
        qab.append(ev[0].elapsed_time(ev[1]))
        gm.append(ev[1].elapsed_time(ev[2]))
    gemm_ms = median(gm)
    quant_step_ms = median(qab)
    # the quantizer's average launch: A, B, A, B, ... back to back (each
    # operand is 256 MiB, as large as the MALL, so every launch reads HBM)
    quant_ms = _time_batch([lambda: fp4.quantize_pack_mxfp4(A, scale_layout="kmajor"),
                            lambda: fp4.quantize_pack_mxfp4(B, scale_layout="kmajor")] * 4)
    apk, ae8 = fp4.quantize_pack_mxfp4(A, scale_layout="kmajor")
    bpk, be8 = fp4.quantize_pack_mxfp4(B, scale_layout="kmajor")
    ref_spelling = None
    if not args.no_configs:
        ref_spelling = bench_cfg4_reference_spelling(torch, A, B, apk, bpk, ae8, be8)
    sustained_ms = _time_loop(lambda: mxfp4_gemm.mxfp4_gemm_packed(apk, bpk, ae8, be8), n=50)
    del apk, bpk
    step_sustained_ms = _time_loop(step, n=40)

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

    flop = 2.0 * n * n * n
    gemm_tflops = flop / (gemm_ms * 1e-3) / 1e12
    sus_tflops = flop / (sustained_ms * 1e-3) / 1e12
    q_bytes = n * n * (4 + 0.5 + 1.0 / 32)            # fp32 in, packed nibbles + E8M0 out
    quant_gbs = q_bytes / (quant_ms * 1e-3) / 1e9
    value = flop / (ms_per_step * 1e-3) / 1e12
    gemm_clock = clock_from_profiles("gemm_f4f4_mx16_kernel")

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
        "step_sustained": {"ms": round(step_sustained_ms, 4),
                           "tflops": round(flop / (step_sustained_ms * 1e-3) / 1e12, 1),
                           "how": "40 steps back to back, events around the loop, right before the warm-up"},
        "gemm_sustained": {"ms": round(sustained_ms, 4), "tflops": round(sus_tflops, 1),
                           "frac_fp4_peak": round(sus_tflops / PEAK_FP4_TFLOPS, 4),
                           "how": "50 GEMMs back to back, events around the loop"},
        "quantize": {"ms_per_operand": round(quant_ms, 4), "gbs": round(quant_gbs, 1),
                     "frac_hbm": round(quant_gbs / PEAK_HBM_GBS, 4), "bytes_per_launch": int(q_bytes),
                     "how": "8 launches back to back (A, B alternating), events around the batch",
                     "step_launch_ms": round(quant_step_ms, 4),
                     "step_launch_gbs": round(2 * q_bytes / (quant_step_ms * 1e-3) / 1e9, 1),
                     "step_launch": "the step's one launch for A and B (quantize_rows_batch_kernel), event pair "
                                    "after a spin kernel"},
        "roofline": roofline("mfma", "gemm_f4f4_mx16_kernel", gemm_tflops, PEAK_FP4_TFLOPS, "TFLOP/s",
                             traffic_from_profiles("gemm_f4f4_mx16_kernel"), gemm_clock),
        "roofline_quantize": roofline("hbm", "quantize_rows_kernel", quant_gbs, PEAK_HBM_GBS, "GB/s",
                                      traffic_from_profiles("quantize_rows_kernel")),
    }
    if args.calib:
        # plain copy of known size: 256 MiB read + 256 MiB written per launch
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).uniform_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = src.numel() * 4
        del src, dst
    del A, B
    torch.cuda.empty_cache()

    suite_lines = bench_reference_rows(torch, dev) if args.suite else None

    cfg4_cpu = None
    if not args.no_cpu:
        cfg4_cpu = cpu_cfg4(n)
        out["cpu_baseline"] = cfg4_cpu
        for leg in deferred:
            leg()
    if config_rows is not None:
        out["configs"] = config_rows
        out["configs"].insert(len(out["configs"]) - 1, {
            "workload": "cfg4 fully-FP4 GEMM 8192^3, both operands quantized on the fly (the headline)",
            "ms": round(ms_per_step, 4), "rate": round(value, 1), "unit": "TFLOP/s",
            "roofline": out["roofline"], "roofline_quantize": out["roofline_quantize"],
            "cpu_baseline": cfg4_cpu})
        out["configs"].insert(len(out["configs"]) - 1, ref_spelling)
    if suite_lines is not None:
        with open(args.suite, "w") as f:
            for ln in suite_lines:
                f.write(json.dumps(ln) + "\n")
    print(json.dumps(out), flush=True)


def bench_cfg4_reference_spelling(torch, A, B, apk, bpk, ae8, be8):
    """cfg4 through the reference's own call sequence (fp4_linear.py:36-39):
    fp4.quantize_mxfp4 (unpacked codes, fp32 scales) and fp4.pack_fp4 per
    operand, then mxfp4_gemm_packed with the fp32 scales -- which regroups
    them to K-major E8M0 on the device and runs the kernel of the headline.
    The GEMM call is timed against the headline's K-major call on the same
    codes (isolated launches, medians)."""
    from lockstep_amd import fp4, mxfp4_gemm
    n = A.shape[0]

    def quant(x):
        c, s = fp4.quantize_mxfp4(x)
        return fp4.pack_fp4(c), s

    def step():
        (pa, sa), (pb, sb) = quant(A), quant(B)
        return mxfp4_gemm.mxfp4_gemm_packed(pa, pb, sa, sb, out_dtype=torch.bfloat16)

    (pa, sa), (pb, sb) = quant(A), quant(B)
    assert torch.equal(pa, apk) and torch.equal(pb, bpk)
    gemm_ref = _time_events(lambda: mxfp4_gemm.mxfp4_gemm_packed(pa, pb, sa, sb, out_dtype=torch.bfloat16))
    gemm_km = _time_events(lambda: mxfp4_gemm.mxfp4_gemm_packed(apk, bpk, ae8, be8, out_dtype=torch.bfloat16))
    step_ms = _time_events(step, reps=10)
    flop = 2.0 * n ** 3
    return {"workload": f"cfg4 {n}^3 through the reference's spelling: quantize_mxfp4 (fp32 scales) + pack_fp4 "
                        "per operand, mxfp4_gemm_packed with fp32 scales",
            "ms": round(step_ms, 4), "rate": round(flop / step_ms / 1e9, 1), "unit": "TFLOP/s",
            "gemm_call_ms": round(gemm_ref, 4), "gemm_call_kmajor_ms": round(gemm_km, 4),
            "gemm_call_ratio": round(gemm_ref / gemm_km, 4),
            "roofline": roofline("mfma", "gemm_f4f4_mx16_kernel after the scale regroup", flop / gemm_ref / 1e9,
                                 PEAK_FP4_TFLOPS, "TFLOP/s"),
            "note": "the GEMM call includes the fp32 -> K-major E8M0 conversion of both scale tensors in one "
                    "launch (lsmx_scale_to_e8m0_batch); the promotion launch (lsmx_gemm_mx_promote) is skipped because "
                    "fp4.py tracks the quantizer's own scales as powers of two; the step adds the unpacked-code quantizer and pack_fp4 of both "
                    "operands"}


def cpu_cfg4(n):
    """cfg4 on the CPU: quantize A and B (C oracle), dequantize, fp32 A @ B^T."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(4001)
    a = (rng.standard_t(3, (n, n)) * 0.05).astype(np.float32)
    b = (rng.standard_t(3, (n, n)) * 0.05).astype(np.float32)

    def run():
        cpu_quant_deq(O, a) @ cpu_quant_deq(O, b).T
    return cpu_leg(run, 2.0 * n ** 3, "TFLOP/s",
                   f"full cfg4 ({n}x{n}x{n}): quantize A and B (C oracle, OpenMP), dequantize, fp32 A@B^T (numpy)")


# ----------------------------------------------------------------- configs
def run_configs(torch, dev, deferred=None):
    """cfg1, cfg2, cfg3 (M sweep) and cfg5 at their BASELINE shapes: GPU rate
    and roofline of the dominant kernel.  With a list `deferred`, each row's
    CPU restatement is appended to it as a closure that fills the row's
    cpu_baseline when called; it holds its inputs on the GPU and copies them
    to the host only then.  The caller runs the closures after every GPU
    measurement, so the GPU does not idle between the measurements."""
    import numpy as np
    cpu = deferred is not None

    from lockstep_amd import dual_gemm, fp4, mxfp4_gemm
    from oracle import gen
    rows = []

    # cfg1: X[256,1024] fp32, W[1024,1024] ~ N(0, 0.02); quantize W, Y = X @ deq(W)^T fp32
    x1 = gen.normal(1001, (256, 1024))
    w1 = gen.normal(1002, (1024, 1024), std=0.02)
    xt, wt = torch.from_numpy(x1).to(dev), torch.from_numpy(w1).to(dev)
    state = {}

    def c1_quant():
        state["w"] = fp4.quantize_pack_mxfp4(wt)

    def c1_gemm():
        mxfp4_gemm.mxfp4_gemm_bf16(xt, state["w"][0], state["w"][1], out_dtype=torch.float32)
    per, tot = _time_ops([("quantize", c1_quant), ("gemm", c1_gemm)], reps=20)
    fl1 = 2.0 * 256 * 1024 * 1024
    qb1 = 1024 * 1024 * (4 + 0.5 + 1 / 32)
    r = {"workload": "cfg1 fp4_linear layer: quantize W[1024,1024] + Y = X[256,1024] fp32 @ deq(W)^T, fp32 out",
         "ms": round(tot, 4), "rate": round(fl1 / tot / 1e9, 2), "unit": "TFLOP/s",
         "roofline": roofline("mfma", "gemm_xf4_kernel (fp32 X as 3 exact bf16 terms)", fl1 / per["gemm"] / 1e9,
                              PEAK_BF16_TFLOPS, "TFLOP/s"),
         "roofline_quantize": roofline("hbm", "quantize_rows_kernel", qb1 / per["quantize"] / 1e6, PEAK_HBM_GBS,
                                       "GB/s"),
         "note": "a correctness config: 0.5 GFLOP per step does not fill the GPU; the fp32 activations cost "
                 "three bf16 MFMAs per product"}
    if cpu:
        def leg1(r=r):
            from oracle import oracle as O

            def run1():
                x1 @ cpu_quant_deq(O, w1).T
            r["cpu_baseline"] = cpu_leg(run1, fl1, "TFLOP/s", "full cfg1: quantize W (C oracle), dequantize, "
                                                              "fp32 X @ W^T (numpy)")
        deferred.append(leg1)
    rows.append(r)

    # cfg2: A0, A1 bf16 [2048, 4096], W [4096, 4096] MXFP4, one dual launch
    g = torch.Generator(device=dev).manual_seed(2001)
    a0 = torch.randn((2048, 4096), device=dev, generator=g).to(torch.bfloat16)
    a1 = torch.randn((2048, 4096), device=dev, generator=g).to(torch.bfloat16)
    w2 = torch.randn((4096, 4096), device=dev, generator=g) * 0.02
    wpk, we8 = fp4.quantize_pack_mxfp4(w2)
    ms = _time_events(lambda: dual_gemm.dual_mxfp4(a0, a1, wpk, we8))
    ms2 = _time_events(lambda: (mxfp4_gemm.mxfp4_gemm_bf16(a0, wpk, we8), mxfp4_gemm.mxfp4_gemm_bf16(a1, wpk, we8)))
    fl2 = 2.0 * 2 * 2048 * 4096 * 4096
    r = {"workload": "cfg2 dual-batch bf16 x MXFP4: 2 x [2048,4096] . W[4096,4096]^T, one launch, bf16 out",
         "ms": round(ms, 4), "rate": round(fl2 / ms / 1e9, 1), "unit": "TFLOP/s",
         "roofline": roofline("mfma", "gemm_bf16f4_ring_kernel<2,...> (dual)", fl2 / ms / 1e9, PEAK_BF16_TFLOPS,
                              "TFLOP/s", traffic_from_profiles("gemm_bf16f4_ring_kernel<2")),
         "two_launch_ms": round(ms2, 4)}
    if cpu:
        def leg2(r=r, w2=w2, a0=a0, a1=a1):
            from oracle import oracle as O
            wc, ws = O.quantize_mxfp4(w2.cpu().numpy())
            A0, A1 = _bf16_to_f32_np(a0), _bf16_to_f32_np(a1)

            def run2():
                W = O.dequantize_mxfp4(wc, ws)
                A0 @ W.T
                A1 @ W.T
            r["cpu_baseline"] = cpu_leg(run2, fl2, "TFLOP/s", "full cfg2: dequantize W (C oracle), two fp32 "
                                                              "matmuls (numpy)")
        deferred.append(leg2)
    rows.append(r)
    del a0, a1, w2, wpk, we8

    # cfg3: W [14336, 4096], M sweep
    w3 = torch.randn((14336, 4096), device=dev, generator=g) * 0.02
    w3pk, w3e8 = fp4.quantize_pack_mxfp4(w3)
    # the CPU legs quantize W once, when the first of them runs
    q3 = {}
    # copies of the packed weight, rotated between launches: 16 x 31 MB is
    # twice the MALL, so every launch streams its weight from HBM
    wcopies = [(w3pk.clone(), w3e8.clone()) for _ in range(16)]
    for M in (1, 16, 128, 1024, 8192):
        a = torch.randn((M, 4096), device=dev, generator=g).to(torch.bfloat16)
        ms = _time_batch([lambda wp=wp, we=we: mxfp4_gemm.mxfp4_gemm_bf16(a, wp, we) for wp, we in wcopies],
                         reps=5 if M >= 1024 else 10)
        fl = 2.0 * M * 14336 * 4096
        by = 14336 * 4096 * (0.5 + 1 / 32) + 2 * M * 4096 + 2 * M * 14336
        kern = ("gemv_bf16f4_kernel" if M <= 1 else "gemm_bf16f4_decode_kernel" if M <= 16 else
                "gemm_bf16f4_skinny_kernel" if M <= 32 else
                "gemm_bf16f4_ring_kernel (split-K) + splitk_reduce_kernel" if M <= 256 else
                "gemm_bf16f4_ring_kernel")
        if M <= 16:
            rl = roofline("hbm", kern, by / ms / 1e6, PEAK_HBM_GBS, "GB/s")
        else:
            rl = roofline("mfma", kern, fl / ms / 1e9, PEAK_BF16_TFLOPS, "TFLOP/s")
        r = {"workload": f"cfg3 weight-only bf16 x MXFP4, M={M}, N=14336, K=4096, bf16 out", "ms": round(ms, 4),
             "rate": round(fl / ms / 1e9, 2), "unit": "TFLOP/s", "gbs": round(by / ms / 1e6, 1), "roofline": rl,
             "how": "16 launches back to back over 16 copies of W, events around the batch"}
        if cpu:
            def leg3(r=r, a=a, w3=w3, M=M, fl=fl):
                from oracle import oracle as O
                if not q3:
                    q3["c"], q3["s"] = O.quantize_mxfp4(w3.cpu().numpy())
                A = _bf16_to_f32_np(a)

                def run3():
                    A @ O.dequantize_mxfp4(q3["c"], q3["s"]).T
                r["cpu_baseline"] = cpu_leg(run3, fl, "TFLOP/s", f"full cfg3 M={M}: dequantize W (C oracle), fp32 "
                                                                 "A @ W^T (numpy)")
            deferred.append(leg3)
        rows.append(r)
        del a
    del w3, w3pk, w3e8, wcopies
    torch.cuda.empty_cache()

    rows.append(bench_cfg5(torch, dev, deferred))
    return rows


def bench_cfg5(torch, dev, deferred, T=8192, H=2048, F=8192):
    """cfg5: one MLP block (fc H->F, out F->H) forward + MXFP4 backward, timed
    op by op inside one step: the 6 f4 x f4 GEMMs (fwd, dgrad, wgrad of each
    linear, train_step.py:3-6) on operands quantized along both axes.  x, w1,
    w2 and dy are quantized in one pass each; the hidden activation h and its
    gradient dh are only ever quantized, so the GEMMs that produce them (fc
    forward, out dgrad) quantize them in their epilogue and never write the
    bf16 form (mxfp4_gemm_packed_q2d)."""
    import numpy as np

    from lockstep_amd import fp4, mxfp4_gemm
    g = torch.Generator(device=dev).manual_seed(5001)
    x = torch.randn((T, H), device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn((F, H), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((H, F), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn((T, H), device=dev, generator=g).to(torch.bfloat16)
    s = {}

    def q2(name, t):
        r = fp4.quantize_pack_mxfp4_2d(t, scale_layout="kmajor")
        s[name + "_r"], s[name + "_c"] = (r[0], r[1]), (r[2], r[3])

    def q2_many(names, ts):
        for name, r in zip(names, fp4.quantize_pack_mxfp4_2d_many(ts, scale_layout="kmajor")):
            s[name + "_r"], s[name + "_c"] = (r[0], r[1]), (r[2], r[3])

    mm = lambda a, b: mxfp4_gemm.mxfp4_gemm_packed(s[a][0], s[b][0], s[a][1], s[b][1],   # noqa: E731
                                                   out_dtype=torch.bfloat16)

    def mmq(name, a, b):
        r = mxfp4_gemm.mxfp4_gemm_packed_q2d(s[a][0], s[b][0], s[a][1], s[b][1])
        s[name + "_r"], s[name + "_c"] = (r[0], r[1]), (r[2], r[3])

    ops = [
        ("q2 x w1 w2", lambda: q2_many(("x", "w1", "w2"), (x, w1, w2))),
        ("gemm fc fwd + q2 h", lambda: mmq("h", "x_r", "w1_r")),
        ("gemm out fwd", lambda: s.__setitem__("y", mm("h_r", "w2_r"))),
        ("q2 dy", lambda: q2("dy", dy)),
        ("gemm out dgrad + q2 dh", lambda: mmq("dh", "dy_r", "w2_c")),
        ("gemm out wgrad", lambda: s.__setitem__("dw2", mm("dy_c", "h_c"))),
        ("gemm fc dgrad", lambda: s.__setitem__("dx", mm("dh_r", "w1_c"))),
        ("gemm fc wgrad", lambda: s.__setitem__("dw1", mm("dh_c", "x_c"))),
    ]
    per, tot = _time_ops(ops, reps=10)
    gemm_ms = sum(v for k, v in per.items() if k.startswith("gemm"))
    q_ms = sum(v for k, v in per.items() if k.startswith("q2"))
    fl = 6 * 2.0 * T * F * H
    # one pass per operand: 2 B read + 2 x (0.5 + 1/32) B written per element
    elems = {"x": T * H, "w1": F * H, "w2": H * F, "dy": T * H}
    qbytes = sum(elems[n] for k in per if k.startswith("q2") for n in k.split()[1:]) * (2 + 2 * (0.5 + 1 / 32))
    r = {"workload": f"cfg5 MLP block fwd + MXFP4 bwd (tokens={T}, hidden={H}, ffn={F}, bf16): 6 f4 x f4 GEMMs "
                     "(2 of them quantizing h / dh along both axes in their epilogue) + two-axis quantizations of x, w1, w2 "
                     "(one launch) and dy",
         "ms": round(tot, 4), "rate": round(fl / tot / 1e9, 1),
         "unit": "TFLOP/s", "gemm_ms": round(gemm_ms, 4), "quantize_ms": round(q_ms, 4),
         "roofline": roofline("mfma", "gemm_f4f4_mx16_kernel (6 launches)", fl / gemm_ms / 1e9, PEAK_FP4_TFLOPS,
                              "TFLOP/s"),
         "roofline_quantize": roofline("hbm", "quantize_2d_batch_kernel (x, w1, w2) + quantize_2d_kernel (dy)",
                                       qbytes / q_ms / 1e6, PEAK_HBM_GBS, "GB/s"),
         "ops_ms": {k: round(v, 4) for k, v in per.items()},
         "how": "ms: median step with events only at its ends; ops_ms: steps with an event between ops, whose "
                "sum exceeds ms by the events' own cost"}
    if deferred is not None:
        bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)   # noqa: E731
        # the bf16 h and dh the CPU leg starts from (outside the timed ops)
        h_dev, dh_dev = mm("x_r", "w1_r"), mm("dy_r", "w2_c")

        def leg5(r=r, xs=(x, w1, w2, dy), h_dev=h_dev, dh_dev=dh_dev):
            from oracle import oracle as O
            X, W1, W2, DY = (bits(t) for t in xs)
            hf, dhf = _bf16_to_f32_np(h_dev), _bf16_to_f32_np(dh_dev)

            def run5():
                qd = lambda a, d=None: cpu_quant_deq(O, a, d)   # noqa: E731
                qd(X, "bf16") @ qd(W1, "bf16").T                              # fc fwd
                qd(hf) @ qd(W2, "bf16").T                                     # out fwd
                qd(DY, "bf16") @ qd(np.ascontiguousarray(W2.T), "bf16").T     # out dgrad
                qd(np.ascontiguousarray(DY.T), "bf16") @ qd(np.ascontiguousarray(hf.T)).T   # out wgrad
                qd(dhf) @ qd(np.ascontiguousarray(W1.T), "bf16").T            # fc dgrad
                qd(np.ascontiguousarray(dhf.T)) @ qd(np.ascontiguousarray(X.T), "bf16").T   # fc wgrad
            r["cpu_baseline"] = cpu_leg(run5, fl, "TFLOP/s", "full cfg5: 12 quantizations (C oracle, transposes "
                                                             "by numpy), dequantize, 6 fp32 matmuls (numpy)")
        deferred.append(leg5)
    del s
    return r


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
    row("mxfp4_gemm_fp8 (the reference's call: N-contiguous B and fp32 scales, B read in place)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, b_f8, a_s, b_s)), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_fp8 (B passed as a view of K-contiguous rows)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, bt_f8.t(), a_s, bt_s.t())), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_fp8 (E8M0 byte scales, regrouped to K-major on the device)",
        _time_events(lambda: mg.mxfp4_gemm_fp8(a_f8, bt_f8.t(), a_e8, bt_e8.t())), fl1, PEAK_FP8_TFLOPS)
    row("mxfp4_gemm_packed (f4 x f4)", _time_events(lambda: mg.mxfp4_gemm_packed(a_pk, bt_pk, a_e8, bt_e8)),
        fl1, PEAK_FP4_TFLOPS)
    # fp32 scales that are not powers of two (the quantizer's times 1.5): the
    # conversion flags them, and after the fast kernel the promotion kernel
    # recomputes C with the reference's per-block fp32 arithmetic
    # (mxfp4_gemm.py:141-150), 2 vector-ALU operations per output per block
    a_s15, bt_s15 = a_s * 1.5, bt_s * 1.5
    ms = _time_events(lambda: mg.mxfp4_gemm_packed(a_pk, bt_pk, a_s15, bt_s15), reps=5)
    ops = 2.0 * n * n * (n // 32)
    rows.append({"config": f"ref-bench mxfp4_gemm_packed, fp32 scales that are not powers of two (flagged "
                           f"conversion + fast kernel + promotion kernel), {n}^3", "ms": ms, "tflops": fl1 / ms / 1e9,
                 "valu_gops": ops / ms / 1e6, "frac_valu": ops / ms / 1e6 / PEAK_VALU_GOPS})
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
    rows.extend(dual_numerics(torch, dev))
    return rows


def dual_numerics(torch, dev, m=256, n=256):
    """The reference bench's numerics table for the packed dual accumulator
    (bench.py:120-160): for K in {16, 32, 64, 128, 512}, random q-grid
    operands (fp4.random_codes -> codes_to_q), zero-padded to a multiple of
    64 along K, A2 scaled by 2^slot_offset(K); dual_packed accumulates A1.B1
    + 2^s A2.B2 in one fp32 accumulator and unpack_dual splits it.  Reports
    the share of outputs where both products come back exact (vs the fp64
    products), in bf16 and, when the scaled A2 is representable, e4m3.

    Every K here needs more than fp32's 24 mantissa bits (bits = 2 *
    bitlen(144 K) + 1 >= 25), so whether an output survives depends on the
    order in which its partial sums are rounded: here the MFMA's order inside
    each 64-deep K block, in the reference tl.dot's.  The rates are this
    build's measurement, not a parity claim ("parity unpinned"); the
    64-block alternation of the two products matches the reference's loop
    and is tested (tests/test_gpu_scales.py)."""
    from lockstep_amd import dual_gemm as dg
    from lockstep_amd import fp4
    torch.manual_seed(0)
    out = []

    def exact_rate(dt, q, s, ref1, ref2):
        a1, b1, b2 = q[0].to(dt), q[2].to(dt), q[3].to(dt)
        a2s = (q[1] * (2.0 ** s)).to(dt)
        acc = dg.dual_packed(a1, a2s, b1, b2)
        g1, g2 = dg.unpack_dual(acc, s)
        return ((g1.double() == ref1) & (g2.double() == ref2)).float().mean().item()

    for k in (16, 32, 64, 128, 512):
        s = dg.slot_offset(k)
        need = 2 * (144 * k).bit_length() + 1
        kp = max(64, (k + 63) // 64 * 64)
        q = []
        for sh, axis in (((m, k), 1), ((m, k), 1), ((k, n), 0), ((k, n), 0)):
            v = fp4.codes_to_q(fp4.random_codes(sh, dev)).float()
            if kp != k:
                pad = torch.zeros((m, kp - k) if axis == 1 else (kp - k, n), device=dev)
                v = torch.cat([v, pad], dim=axis)
            q.append(v.contiguous())
        ref1 = q[0].double() @ q[2].double()
        ref2 = q[1].double() @ q[3].double()
        bf = exact_rate(torch.bfloat16, q, s, ref1, ref2)
        a2s = q[1] * (2.0 ** s)
        rt = a2s.to(torch.float8_e4m3fn).float()
        enc = bool(torch.isfinite(rt).all().item() and (rt == a2s).all().item())
        f8 = exact_rate(torch.float8_e4m3fn, q, s, ref1, ref2) if enc else None
        out.append({"config": f"ref-bench dual numerics: packed accumulator, K={k}, {m}x{n}",
                    "k": k, "s": s, "bits_needed": need, "bf16_exact": bf, "fp8_encodable": enc,
                    "fp8_exact": f8, "parity": "unpinned (bits needed > 24: depends on the accumulation "
                                               "order inside a 64-deep K block)" if need > 24 else "pinned"})
    return out


if __name__ == "__main__":
    main()
