// Shared device helpers for the gfx950 MXFP4 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lsmx.h"

#define LSMX_DEV __device__ __forceinline__
#define LSMX_HD __host__ __device__ __forceinline__

namespace lsmx {

LSMX_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
LSMX_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------- E8M0 rule
// fp4.py:68 computes e = floor(log2(max(amax, 1e-30))) - 2 with a float32
// log2.  Because log2 is rounded to float32, an amax a few ulps below 2^k has
// log2 == k exactly and takes exponent k, not k-1.  The window is
// floor(ln2 * 2^p) ulps, p = floor(log2(a)) with a = k-1 (k > 0) or -k
// (k <= 0).  These functions express that rule in integer operations on the
// bits of amax (a non-negative, non-NaN float).
LSMX_HD int e8m0_window(int k) {
    const uint64_t n_of_p = 0x582C160B05020100ull;  // p -> 0,1,2,5,11,22,44,88
    int a = k > 0 ? k - 1 : -k;
    int p = a > 1 ? 31 - __builtin_clz((unsigned)a) : 0;
    return (int)((n_of_p >> (8 * p)) & 0xFF);
}

// Unbiased scale exponent for a block with absmax bits `b` (b != 0, not NaN).
LSMX_HD int e8m0_exponent(uint32_t b) {
    if (b < 0x0DA24260u) return -102;   // amax < 1e-30f is clamped to 1e-30f
    if (b >= 0x7F800000u) return 127;   // +inf: clamp(inf - 2, -127, 127)
    int be = (int)(b >> 23);            // biased exponent, 1..254
    uint32_t thr = ((uint32_t)(be + 1) << 23) - (uint32_t)e8m0_window(be - 126);
    return (be - 127) + (b >= thr ? 1 : 0) - 2;
}

// Per-block scale decision.  amax_bits = max over the block of (bits & 0x7FFFFFFF)
// as unsigned integers, which orders finite magnitudes, puts +inf above them
// and any NaN above +inf.  Returns the E8M0 byte: 127 (scale 1) for a zero
// block, 255 for a NaN block, e + 127 otherwise.
LSMX_HD uint32_t block_e8m0(uint32_t amax_bits) {
    if (amax_bits == 0) return 127u;
    if (amax_bits > 0x7F800000u) return 255u;
    return (uint32_t)(e8m0_exponent(amax_bits) + 127);
}

// fp4.py:43-54 on one element, given the block's E8M0 byte.
//   y = |x| * 2^-e (exact: a power-of-two scaling, v_ldexp_f32)
//   magnitude = number of midpoints {0.25,0.75,1.25,1.75,2.5,3.5,5} strictly
//   below min(y, 6); for y >= 1 that is round-to-nearest, ties down, onto one
//   mantissa bit: ((bits(y) + 0x1FFFFF) >> 22) - 252, capped at 7.
// Sign: copied from x.  NaN block (e8m0 == 255): magnitude 7; the sign is the
// element's own sign if it is a NaN, else 0 (the sign of the NaN scale
// torch divides by).
LSMX_DEV uint32_t e2m1_code(uint32_t xbits, uint32_t e8m0) {
    uint32_t ax = xbits & 0x7FFFFFFFu;
    uint32_t sign = xbits >> 31;
    if (e8m0 == 255u) return 7u | ((ax > 0x7F800000u ? sign : 0u) << 3);
    float y = __builtin_amdgcn_ldexpf(u2f(ax), 127 - (int)e8m0);
    uint32_t yb = f2u(y);
    uint32_t big = min((yb + 0x1FFFFFu) >> 22, 259u) - 252u;
    uint32_t small = yb > 0x3F400000u ? 2u : (yb > 0x3E800000u ? 1u : 0u);
    uint32_t mag = yb >= 0x3F800000u ? big : small;
    return mag | (sign << 3);
}

// E8M0 byte -> fp32 scale: 2^(e - 127); byte 0 is 2^-127 (the fp32
// subnormal 0x00400000) and 0xFF is NaN.
LSMX_HD float e8m0_to_f32(uint32_t e) {
    return e == 255u ? u2f(0x7FC00000u) : (e == 0u ? u2f(0x00400000u) : u2f(e << 23));
}

// E8M0 byte of an fp32 block scale (bits b): its biased exponent when the
// scale is a positive power of two in [2^-127, 2^127], else 0xFF (E8M0 NaN).
// A scale with no E8M0 form (1.5, -2, 0, inf) thus turns the outputs that
// use it into NaN rather than being truncated to its exponent field.
LSMX_HD uint32_t f32_scale_e8m0(uint32_t b) {
    const uint32_t ex = b >> 23;  // the sign is bit 8: negative scales fail both tests
    const bool pow2 = ((b & 0x7FFFFFu) == 0u && ex >= 1u && ex <= 254u) || b == 0x00400000u;
    return pow2 ? (b == 0x00400000u ? 0u : ex) : 0xFFu;
}

// 4 nibbles (low 16 bits of p) -> 4 E4M3 bytes: magnitude by a byte permute
// against the 8-entry table {00 30 38 3C 40 44 48 4C}, sign bit 3 -> bit 7.
LSMX_DEV uint32_t fp4x4_to_e4m3x4(uint32_t p) {
    const uint32_t spread = (p & 0xF) | ((p & 0xF0) << 4) | ((p & 0xF00) << 8) | ((p & 0xF000) << 12);
    const uint32_t mag = __builtin_amdgcn_perm(0x4C484440u, 0x3C383000u, spread & 0x07070707u);
    return mag | ((spread & 0x08080808u) << 4);
}

// E2M1 code -> value (fp4.py:24).
LSMX_HD float e2m1_value(uint32_t code) {
    const float m[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    float v = m[code & 7];
    return (code & 8) ? -v : v;
}

}  // namespace lsmx
