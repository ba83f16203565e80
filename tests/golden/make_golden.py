"""Write golden vectors for the MXFP4 quantizer from the reference's fp4.py.

Runs only where the reference is mounted (the build container), never on the
GPU box:  python tests/golden/make_golden.py [/root/reference]

Only fp4.quantize_mxfp4 and fp4._round_to_e2m1 are called.  Their byte-level
output as torch executes it (the float32 log2 edge of the E8M0 exponent at
fp4.py:68, NaN/Inf/-0 handling at fp4.py:50-54) is not fixed by the
reference's own tests (tests/test_fp4.py:64 accepts either exponent) or by
the mathematics, so it is recorded here as data.  Inputs come from
oracle/gen.py, whose integer-only generator reproduces them on any host; the
fixtures keep digests of full outputs plus small explicit slices.
"""

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import gen  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def edge_blocks() -> np.ndarray:
    """Blocks whose amax sits 0..50 ulps below 2^k (and just above 2^(k-1)),
    for binades across the whole fp32 range, plus a fixed ramp of smaller
    elements so the element rounding is exercised at each scale."""
    rows = []
    ramp = np.linspace(-0.9, 0.9, 31, dtype=np.float64)
    for k in [-126, -100, -99, -64, -63, -33, -32, -17, -16, -9, -8, -5, -4, -3, -2, -1, 0, 1,
              2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64, 65, 100, 127, 128]:
        top = (np.uint32(min(k + 127, 255)) << np.uint32(23)).astype(np.uint32)
        for j in list(range(0, 51, 1)) + [64, 100]:
            b = np.uint32(int(top) - 1 - j)
            amax = np.array([b], dtype=np.uint32).view(np.float32)[0]
            if not np.isfinite(amax) or amax == 0:
                continue
            blk = np.empty(32, dtype=np.float32)
            blk[0] = -amax if (j % 2) else amax
            blk[1:] = (ramp * float(amax)).astype(np.float32)
            rows.append(blk)
    return np.stack(rows)


def special_blocks() -> np.ndarray:
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = []
    base = np.linspace(-3.0, 3.0, 32, dtype=np.float32)
    r = base.copy(); r[5] = nan; rows.append(r)                       # +NaN inside
    r = base.copy(); r[7] = -nan; rows.append(r)                      # -NaN inside
    r = base.copy(); r[3] = inf; rows.append(r)                       # +Inf
    r = base.copy(); r[9] = -inf; rows.append(r)                      # -Inf
    r = base.copy(); r[3] = inf; r[4] = nan; rows.append(r)           # Inf and NaN
    rows.append(np.zeros(32, dtype=np.float32))                       # zero block
    rows.append(-np.zeros(32, dtype=np.float32))                      # -0 block
    r = np.zeros(32, dtype=np.float32); r[0] = 1.0; r[1:] = -1e-9; rows.append(r)  # -> code 8
    r = np.full(32, 1e-38, dtype=np.float32); rows.append(r)          # subnormal-ish amax
    r = np.full(32, 1e-45, dtype=np.float32); r[2] = -1e-45; rows.append(r)  # denormal amax
    r = np.full(32, 3.0e38, dtype=np.float32); r[1] = -3.4028235e38; rows.append(r)  # FLT_MAX
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], dtype=np.float32)
    r = np.concatenate([mids, -mids, mids * 0.5, -mids * 0.5]).astype(np.float32)
    rows.append(r)                                                    # ties at scale 1 and 1/2
    return np.stack(rows)


def main():
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(ref))
    import fp4  # the reference module, read from the mounted checkout

    torch.set_num_threads(8)
    out_json = {"generator": "oracle/gen.py", "torch": torch.__version__, "cases": {}}
    arrays = {}

    def record(name, x, block=32, keep_rows=2, xdtype="f32"):
        if xdtype == "bf16":
            t = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
        else:
            t = torch.from_numpy(x)
        codes, scale = fp4.quantize_mxfp4(t, block)
        c = codes.numpy().astype(np.uint8)
        s = scale.numpy().astype(np.float32)
        out_json["cases"][name] = {
            "shape": list(x.shape), "block": block, "dtype": xdtype,
            "codes_sha256": sha(c), "scale_sha256": sha(s.view(np.uint32)),
        }
        arrays[f"{name}__codes"] = c[:keep_rows] if keep_rows else c
        arrays[f"{name}__scale"] = s[:keep_rows] if keep_rows else s

    # cfg1: W [1024,1024] ~ N(0, 0.02), X [256,1024] ~ N(0, 1)  (fp4_linear.py:36-37)
    record("cfg1_W", gen.normal(1002, (1024, 1024), std=0.02))
    record("cfg1_X", gen.normal(1001, (256, 1024)))
    # cfg2/cfg3-style weight slice and bf16 activations
    record("w_slice", gen.normal(2003, (64, 4096), std=0.02))
    record("a_bf16", gen.to_bf16_bits(gen.normal(2001, (64, 4096))), xdtype="bf16")
    # cfg4: Student-t (df=3) * 0.05, along K
    record("t3_slice", gen.student_t3(4001, (64, 8192), scale=0.05))
    # block 16 (tests/test_fp4.py:54 covers both)
    record("blk16", gen.normal(7, (32, 512)), block=16)
    # rows spread over ~2^-10..2^11 as in tests/test_fp4.py:57 (exact multipliers)
    mult = np.ldexp(1.0 + (np.arange(64) % 7) / 8.0, np.arange(64) // 3 - 10)
    lg = (gen.normal(0, (64, 256)).astype(np.float64) * mult[:, None]).astype(np.float32)
    record("logspace", lg)
    # explicit corner cases, kept whole
    record("edges", edge_blocks(), keep_rows=0)
    record("special", special_blocks(), keep_rows=0)

    # _round_to_e2m1 over every bf16 bit pattern (as fp32), fp4.py:43-54
    allbf = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    rc = fp4._round_to_e2m1(torch.from_numpy(allbf.copy())).numpy().astype(np.uint8)
    arrays["round_all_bf16__codes"] = rc
    out_json["cases"]["round_all_bf16"] = {"codes_sha256": sha(rc)}

    np.savez_compressed(HERE / "fp4_golden.npz", **arrays)
    (HERE / "fp4_golden.json").write_text(json.dumps(out_json, indent=1) + "\n")
    print(f"wrote {len(arrays)} arrays, {len(out_json['cases'])} cases")


if __name__ == "__main__":
    main()
