// The MXFP4 rule of fp4.py (quantize_mxfp4 :57-72, _round_to_e2m1 :43-54)
// for blocks of 16-bit values (bf16 or fp16 widened to fp32), shared by the
// two-axis quantizer and the GEMM epilogue that quantizes its bf16 output.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsmx_common.h"

namespace lsmx {

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// Lane-wise max of two pairs of unsigned 16-bit values (v_pk_max_u16).
LSMX_DEV uint32_t pk_max16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                  __builtin_bit_cast(u16x2, b)));
}

// lsmx::block_e8m0 for a block of 16-bit values, given the fp32 bits am of
// its absmax, finite (am < 0x7F800000).  block_e8m0 raises the exponent by
// one when amax lies within 88 fp32 ulps below a power of two (the float32
// rounding of fp4.py's log2); a widened bf16 (fp16) value has its low 16
// (13) bits clear, so it is never that close, and the scale exponent is the
// biased exponent of amax minus 2, at least 25 (fp4.py's clamp of amax to
// 1e-30 = 0x0DA24260 has biased exponent 27).  A zero block has scale 1.
LSMX_DEV uint32_t block_e8m0_16(uint32_t am) {
    const uint32_t e8 = max(am >> 23, 27u) - 2u;
    return am == 0u ? 127u : e8;
}

// An element x of a 16-bit input, widened to fp32 and multiplied by
// 1 - 2^-20 (exact for the values below: x has at most 11 significant bits,
// a midpoint at most 3).  The product lies strictly between x and the next
// 16-bit value toward zero: a midpoint of E2M1 at any scale (0.25 .. 5 times
// 2^e) drops just below it, and no other value crosses one, so the
// hardware's round-to-nearest-even of the product (v_cvt_scalef32_pk_fp4_f32)
// is fp4.py's round-to-nearest with ties toward the smaller magnitude
// (fp4.py:50-53).  Zeros keep their sign and Infs stay Inf.
LSMX_DEV float tie_down16(uint32_t bits) { return u2f(bits) * u2f(0x3F7FFFF0u); }

// E2M1 codes of f[0..7] / sc (sc a power of two), f[2j] and f[2j+1] in the
// low and high nibble of byte j.
LSMX_DEV uint32_t cvt_fp4_x8(const float (&f)[8], float sc) {
    uint32_t w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, f[0], f[1], sc, 0);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[2], f[3], sc, 1);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[4], f[5], sc, 2);
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[6], f[7], sc, 3);
}

// lsmx::block_e8m0 for a block of 16-bit values with any absmax: an Inf
// block has scale 2^127 (fp4.py clamps the exponent to 127), a NaN block the
// E8M0 NaN.
LSMX_DEV uint32_t block_e8m0_16x(uint32_t am) {
    return am > 0x7F800000u ? 255u : (am == 0x7F800000u ? 254u : block_e8m0_16(am));
}

// Codes of the 8 elements f (tie_down16 of 16-bit values, NaNs as they are)
// of a block with E8M0 byte e8, Inf and NaN included: the hardware maps
// +-Inf to +-6 (code 7 with the sign); a NaN block gives magnitude 7 with
// the element's sign if the element is a NaN, else 0 (lsmx::e2m1_code).
LSMX_DEV uint32_t codes8_any(const float (&f)[8], uint32_t e8) {
    uint32_t nan_codes = 0x77777777u;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t b = f2u(f[k]);
        nan_codes |= ((b & 0x7FFFFFFFu) > 0x7F800000u ? (b >> 31) : 0u) << (4 * k + 3);
    }
    const uint32_t w = cvt_fp4_x8(f, u2f(min(e8, 254u) << 23));
    return e8 == 255u ? nan_codes : w;
}

// Element k of a 16-bit block for codes8_any: tie_down16 of its fp32 bits,
// or the NaN as it is (so that its sign survives).
LSMX_DEV float nudge_keep_nan(uint32_t b) {
    return (b & 0x7FFFFFFFu) > 0x7F800000u ? u2f(b) : tie_down16(b);
}

}  // namespace lsmx
