/*
 * mxfp4_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of lockstep's MXFP4 arithmetic, used as the checker
 * for the HIP kernels in lockstep_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product library never links
 * it and never falls back to it.
 *
 * Every function cites the reference line it restates (paths relative to the
 * reference repository root):
 *   fp4.py:20-34   tables              -> kMag, kE4M3, kQ
 *   fp4.py:43-54   _round_to_e2m1      -> orc_round_e2m1
 *   fp4.py:57-72   quantize_mxfp4      -> orc_quantize_{f32,bf16,f16}
 *   fp4.py:68      E8M0 exponent       -> orc_e8m0_exp_log2 (libm path) and
 *                                         orc_e8m0_exp_int  (integer rule used
 *                                         by the GPU kernel); the two are
 *                                         checked against each other and
 *                                         against torch.log2 in tests/
 *   fp4.py:75-78   dequantize_mxfp4    -> orc_dequantize
 *   fp4.py:91-99   pack_fp4/unpack_fp4 -> orc_pack_fp4 / orc_unpack_fp4
 *   cuda/fp4_unpack.cuh:45-61  FP4->E4M3 expansion -> orc_fp4x8_to_e4m3x8
 *   mxfp4_gemm.py:52-63, 141-150  fp32 promotion per 32-block -> orc_gemm_promote
 *
 * Parity pins (what each function is checked against) are listed in
 * tests/test_oracle.py.
 *
 * Build: oracle/Makefile  ->  oracle/liboracle.so  (gcc -O2 -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* fp4.py:20 -- code & 7 -> magnitude */
static const float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
/* fp4.py:51 -- the 7 midpoints between consecutive magnitudes */
static const float kMid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
/* fp4.py:27-29 -- code -> E4M3 byte */
static const uint8_t kE4M3[16] = {0x00, 0x30, 0x38, 0x3C, 0x40, 0x44, 0x48, 0x4C,
                                  0x80, 0xB0, 0xB8, 0xBC, 0xC0, 0xC4, 0xC8, 0xCC};

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int orc_version(void) { return 1; }

/* fp4.py:20-24: code -> value (E2M1_VALUES). */
float orc_e2m1_value(uint8_t code) {
    float v = kMag[code & 7];
    return (code & 8) ? -v : v;
}

/* fp4.py:43-54.  a = min(|q|, 6); magnitude index = number of midpoints
 * strictly below a (torch.bucketize with right=False puts a value equal to a
 * boundary in the lower bucket, so ties go to the smaller magnitude); the sign
 * bit is copied from q (torch.signbit), so -0.0 and small negatives give code 8.
 * A NaN compares false everywhere in bucketize's binary search and lands in
 * the last bucket: magnitude 7. */
uint8_t orc_round_e2m1(float q) {
    uint8_t sign = (uint8_t)(f2u(q) >> 31);
    float a = fabsf(q);
    uint8_t idx;
    if (isnan(a)) {
        idx = 7;
    } else {
        if (a > 6.0f) a = 6.0f;
        idx = 0;
        for (int i = 0; i < 7; ++i) idx += (kMid[i] < a);
    }
    return (uint8_t)(idx | (sign << 3));
}

/* fp4.py:68, libm path:  e = floor(RN_f32(log2(max(amax, 1e-30f)))) - 2,
 * clamped to [-127, 127].  log2 is evaluated in double and rounded to float,
 * which is the correctly rounded float32 log2 everywhere it matters here.
 * amax must be >= 0 and not NaN.  Returns the unbiased exponent e. */
int orc_e8m0_exp_log2(float amax) {
    float a = amax < 1e-30f ? 1e-30f : amax;
    float l = (float)log2((double)a);
    float e = floorf(l) - 2.0f;
    if (e < -127.0f) e = -127.0f;
    if (e > 127.0f) e = 127.0f;
    return (int)e;
}

/* Width of the "rounds up" window below 2^k, in float32 ulps of the binade
 * [2^(k-1), 2^k): amax values within it have RN_f32(log2(amax)) == k.  With
 * a = k-1 for k > 0 and a = -k otherwise, the window is floor(ln2 * 2^p) ulps
 * where p = floor(log2(a)) (0 for a <= 1).  tests/ check it by brute force
 * against orc_e8m0_exp_log2 for every binade. */
int orc_e8m0_window(int k) {
    static const uint8_t n_of_p[8] = {0, 1, 2, 5, 11, 22, 44, 88};
    int a = k > 0 ? k - 1 : -k;
    int p = 0;
    while ((a >> (p + 1)) != 0) ++p;
    return n_of_p[p];
}

/* The same exponent as orc_e8m0_exp_log2, from integer operations on the
 * bits of amax only.  This is the rule the GPU quantizer implements. */
int orc_e8m0_exp_int(float amax) {
    uint32_t b = f2u(amax);
    if (b < 0x0DA24260u) return -102;          /* amax < 1e-30f: clamped   */
    if (b >= 0x7F800000u) return 127;          /* +inf: clamp(inf - 2)     */
    int be = (int)(b >> 23);                   /* biased exponent 1..254   */
    int k = be - 126;                          /* amax in [2^(k-1), 2^k)   */
    uint32_t thr = ((uint32_t)(be + 1) << 23) - (uint32_t)orc_e8m0_window(k);
    return (be - 127) + (b >= thr ? 1 : 0) - 2;
}

/* One 32-or-16-element block of fp4.py:57-72.  `x` holds the block as fp32.
 * Writes `block` codes and returns the fp32 scale (2^e, 1.0 for an all-zero
 * block, NaN for a block holding a NaN).
 *
 * NaN blocks: torch.amax propagates NaN, so the scale is NaN and x / scale is
 * NaN for every element.  The quotient takes the sign of the NaN operand that
 * the x86 divide returns (the dividend when it is NaN, else the divisor), and
 * the code is 7 | sign << 3.  `nan_scale_sign` is the sign bit of the NaN
 * scale that torch produces on the host (pinned by the golden fixtures). */
static const uint32_t kNanScaleSign = 0u;

static float quant_block(const float *x, int block, uint8_t *codes, int use_int_rule) {
    float amax = 0.0f;
    int has_nan = 0;
    for (int i = 0; i < block; ++i) {
        float a = fabsf(x[i]);
        if (isnan(a)) has_nan = 1;
        else if (a > amax) amax = a;
    }
    if (has_nan) {
        for (int i = 0; i < block; ++i) {
            uint32_t s = isnan(x[i]) ? (f2u(x[i]) >> 31) : kNanScaleSign;
            codes[i] = (uint8_t)(7u | (s << 3));
        }
        return u2f(0x7FC00000u | (kNanScaleSign << 31));
    }
    float scale;
    if (amax == 0.0f) {
        scale = 1.0f;
    } else {
        int e = use_int_rule ? orc_e8m0_exp_int(amax) : orc_e8m0_exp_log2(amax);
        scale = ldexpf(1.0f, e);
    }
    for (int i = 0; i < block; ++i) codes[i] = orc_round_e2m1(x[i] / scale);
    return scale;
}

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

static float f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
    if (e == 0) {
        float v = ldexpf((float)m, -24);
        return s ? -v : v;
    }
    if (e == 31) return u2f(s | 0x7F800000u | (m << 13));
    return u2f(s | ((e + 112) << 23) | (m << 13));
}

/* Row-major quantize of x[rows, K] (row stride ldx elements) along K.
 * dtype: 0 = fp32, 1 = bf16, 2 = fp16.  codes: [rows, K] (unpacked, as
 * fp4.py returns them); scale: [rows, K/block] fp32.  rule: 0 = libm log2,
 * 1 = integer rule.  Returns 0, or -1 if K % block != 0. */
int orc_quantize(const void *x, int dtype, int64_t rows, int64_t K, int64_t ldx,
                 int block, uint8_t *codes, float *scale, int rule) {
    if (block <= 0 || block > 64 || K % block != 0) return -1;
    const int64_t nb = K / block;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float buf[64];
        for (int64_t b = 0; b < nb; ++b) {
            const int64_t base = r * ldx + b * block;
            for (int i = 0; i < block; ++i) {
                if (dtype == 0) buf[i] = ((const float *)x)[base + i];
                else if (dtype == 1) buf[i] = bf16_to_f32(((const uint16_t *)x)[base + i]);
                else buf[i] = f16_to_f32(((const uint16_t *)x)[base + i]);
            }
            scale[r * nb + b] = quant_block(buf, block, codes + r * K + b * block, rule);
        }
    }
    return 0;
}

/* fp4.py:91-94: byte i = code[2i] | code[2i+1] << 4 (even index, low nibble). */
void orc_pack_fp4(const uint8_t *codes, int64_t n_bytes, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_bytes; ++i)
        out[i] = (uint8_t)((codes[2 * i] & 0x0F) | ((codes[2 * i + 1] & 0x0F) << 4));
}

/* fp4.py:97-99 */
void orc_unpack_fp4(const uint8_t *packed, int64_t n_bytes, uint8_t *codes) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_bytes; ++i) {
        codes[2 * i] = packed[i] & 0x0F;
        codes[2 * i + 1] = packed[i] >> 4;
    }
}

/* fp4.py:75-78: value(code) * scale, exact in fp32 (scale is a power of two). */
void orc_dequantize(const uint8_t *codes, const float *scale, int64_t rows, int64_t K,
                    int block, float *out) {
    const int64_t nb = K / block;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < K; ++k)
            out[r * K + k] = orc_e2m1_value(codes[r * K + k]) * scale[r * nb + k / block];
}

/* Same as orc_dequantize, from packed nibbles and E8M0 scale bytes
 * (byte = biased exponent; 0xFF = NaN).  Output fp64, for the fp64 reference
 * GEMM of fp4.py:103-112. */
void orc_dequantize_packed_e8m0_f64(const uint8_t *packed, const uint8_t *e8m0, int64_t rows,
                                    int64_t K, double *out) {
    const int64_t nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < K; ++k) {
            uint8_t byte = packed[r * (K / 2) + k / 2];
            uint8_t code = (k & 1) ? (byte >> 4) : (byte & 0x0F);
            uint8_t s = e8m0[r * nb + k / 32];
            double sc = s == 0xFF ? NAN : ldexp(1.0, (int)s - 127);
            out[r * K + k] = (double)orc_e2m1_value(code) * sc;
        }
}

/* fp4.py:81-83 and cuda/fp4_unpack.cuh:45-61: 8 packed codes (low nibble
 * first) -> 8 E4M3 bytes, by table. */
void orc_fp4x8_to_e4m3x8(const uint32_t *in, int64_t n, uint32_t *out_lo, uint32_t *out_hi) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t p = in[i], lo = 0, hi = 0;
        for (int j = 0; j < 4; ++j) lo |= (uint32_t)kE4M3[(p >> (4 * j)) & 0xF] << (8 * j);
        for (int j = 0; j < 4; ++j) hi |= (uint32_t)kE4M3[(p >> (16 + 4 * j)) & 0xF] << (8 * j);
        out_lo[i] = lo;
        out_hi[i] = hi;
    }
}

/* mxfp4_gemm.py:52-63 (_mxfp4_gemm_fp8_kernel) and :141-150
 * (_mxfp4_gemm_packed_kernel): the K loop promotes every 32-block product to
 * the fp32 accumulator and multiplies the two fp32 scales there,
 *     p = dot(a_block, b_block);  acc += p * (sa * sb)
 * with Triton's default fp contraction making the update one fma.  The block
 * product p is exact on the E2M1 grid (|p| <= 1152 in steps of 1/4); here it
 * is summed in double and rounded to float once.  Operands are values
 * (E2M1 or E4M3, already expanded to float): A [M, K], Bt [N, K]; scale
 * (row r, block kb) of A at sa[r * sa_r + kb * sa_k], likewise sb. */
void orc_gemm_promote(const float *A, const float *Bt, const float *sa, int64_t sa_r, int64_t sa_k,
                      const float *sb, int64_t sb_r, int64_t sb_k, int64_t M, int64_t N, int64_t K,
                      float *C) {
    const int64_t nkb = K / 32;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (int64_t kb = 0; kb < nkb; ++kb) {
                double d = 0.0;
                for (int64_t k = 32 * kb; k < 32 * kb + 32; ++k) d += (double)A[m * K + k] * (double)Bt[n * K + k];
                const float p = (float)d;
                const float s = sa[m * sa_r + kb * sa_k] * sb[n * sb_r + kb * sb_k];
                acc = fmaf(p, s, acc);
            }
            C[m * N + n] = acc;
        }
}

/* Number of OpenMP threads this library will use. */
int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
