// MXFP4 quantize / pack / unpack / dequantize / E4M3-expansion kernels for gfx950.
//
// Semantics follow the reference's fp4.py (quantize_mxfp4 :57-72,
// _round_to_e2m1 :43-54, pack_fp4 :91-94, unpack_fp4 :97-99,
// dequantize_mxfp4 :75-78) and cuda/fp4_unpack.cuh:45-61 (FP4 -> E4M3).
//
// Quantize (row mode) is HBM-bound: per 32-block it reads 128 B (fp32) or
// 64 B (bf16/fp16) and writes 16 B of nibbles plus one E8M0 byte.  Each lane
// owns 16 contiguous input bytes, so every global_load_dwordx4 of a wave
// reads 1 KiB of consecutive memory; the lanes of one block (8 for fp32,
// 4 for 16-bit inputs) reduce the block absmax with DPP row operations, and
// the scale decision is all-integer (lsmx::block_e8m0).
#include "lsmx_internal.h"
#include "lsmx_q16.h"

namespace lsmx {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- helpers
template <int N>
LSMX_DEV uint32_t group_max(uint32_t v) {
    // Max over aligned groups of N lanes (N = 2, 4 or 8) via DPP.
    static_assert(N == 2 || N == 4 || N == 8 || N == 1, "group size");
    if constexpr (N >= 2)
        v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));  // xor 1
    if constexpr (N >= 4)
        v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));  // xor 2
    if constexpr (N >= 8)
        v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // half mirror
    return v;
}

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kPerVec = 4;  // elements per 16-byte vector
    LSMX_DEV static void bits(const uint4 &v, uint32_t (&b)[4]) {
        b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
    }
};
// bf16 widens to fp32 by a 16-bit shift.
struct bf16_t { uint16_t v; };
struct f16_t { uint16_t v; };
template <>
struct Elem<bf16_t> {
    static constexpr int kPerVec = 8;
    LSMX_DEV static void bits(const uint4 &v, uint32_t (&b)[8]) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b[2 * i] = w[i] << 16;
            b[2 * i + 1] = w[i] & 0xFFFF0000u;
        }
    }
};
template <>
struct Elem<f16_t> {
    static constexpr int kPerVec = 8;
    LSMX_DEV static void bits(const uint4 &v, uint32_t (&b)[8]) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b[2 * i] = f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF)));
            b[2 * i + 1] = f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16)));
        }
    }
};

template <int E>
struct CodeStore;
// 4 codes -> 2 packed bytes or 4 unpacked bytes
template <>
struct CodeStore<4> {
    LSMX_DEV static void packed(uint8_t *p, const uint32_t (&c)[4]) {
        *reinterpret_cast<uint16_t *>(p) =
            (uint16_t)(c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12));
    }
    LSMX_DEV static void unpacked(uint8_t *p, const uint32_t (&c)[4]) {
        *reinterpret_cast<uint32_t *>(p) = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    }
};
template <>
struct CodeStore<8> {
    LSMX_DEV static void packed(uint8_t *p, const uint32_t (&c)[8]) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= c[i] << (4 * i);
        *reinterpret_cast<uint32_t *>(p) = w;
    }
    LSMX_DEV static void unpacked(uint8_t *p, const uint32_t (&c)[8]) {
        uint2 w;
        w.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
        w.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
        *reinterpret_cast<uint2 *>(p) = w;
    }
};

// E codes of the finite block elements b[0..E-1] (fp32 bits) packed into
// nibbles (element i in nibble i), for the block's E8M0 byte e8 < 255.
// v_cvt_scalef32_pk_fp4_f32 converts x / 2^(e8-127) to E2M1 with round-to-
// nearest-even, saturating at 6 and copying the sign (-0 -> code 8); the low
// nibble of each byte is its first source (all measured on gfx950).  fp4.py
// rounds ties toward the smaller magnitude instead (fp4.py:50-53); the two
// differ only where x / 2^e is exactly 0.75, 1.75 or 3.5 -- there ties-to-
// even picks the larger code -- so those elements, found by comparing the
// bits of |x| with the three tie values of the block, take one code less.
template <int I, int E>
LSMX_DEV uint32_t cvt_fp4_pairs(uint32_t w, const uint32_t (&b)[E], float sc) {
    if constexpr (I < E) {
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, u2f(b[I]), u2f(b[I + 1]), sc, I / 2);  // byte I/2
        return cvt_fp4_pairs<I + 2, E>(w, b, sc);
    } else {
        return w;
    }
}

template <int E>
LSMX_DEV uint32_t e2m1_pack_hw(const uint32_t (&b)[E], uint32_t e8) {
    const float sc = u2f(e8 << 23);  // 2^(e8-127); e8 is 25..254 for a non-zero finite block, 127 for zero
    const uint32_t w = cvt_fp4_pairs<0, E>(0u, b, sc);
    // A tie has mantissa 0x400000 or 0x600000: bit 22 set, bits 0-20 clear.
    // Most waves hold no such element and skip the exact comparison.
    bool maybe_tie = false;
#pragma unroll
    for (int i = 0; i < E; ++i) maybe_tie |= (b[i] & 0x005FFFFFu) == 0x00400000u;
    if (!__any(maybe_tie)) return w;
    const uint32_t t1 = ((e8 - 1) << 23) | 0x400000u;  // 0.75 * 2^e
    const uint32_t t2 = (e8 << 23) | 0x600000u;        // 1.75 * 2^e
    const uint32_t t3 = ((e8 + 1) << 23) | 0x600000u;  // 3.5  * 2^e
    uint32_t dec = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const uint32_t ax = b[i] & 0x7FFFFFFFu;
        dec |= (ax == t1 || ax == t2 || ax == t3) ? (1u << (4 * i)) : 0u;
    }
    return w - dec;  // a tie's code magnitude is 2, 4 or 6: no borrow into the next nibble
}

// The same codes for elements that come from 16-bit inputs (bf16 / fp16,
// widened to fp32 bits).  Ties toward the smaller magnitude without any
// comparison: the hardware rounds |x| - 1 ulp (of fp32) to nearest-even
// instead of |x|.  A 16-bit value has at most 11 significant bits, so no
// input lies within 1 fp32 ulp above an E2M1 midpoint (midpoint / 2^e has at
// most 3): every midpoint rounds down, as fp4.py:50-53 does, and every other
// value lands on the same code as before.  Zeros (either sign) and infinities
// are left alone, and the scale is still decided from the unmodified amax.
LSMX_DEV uint32_t below_ulp(uint32_t b) {
    const uint32_t ax = b & 0x7FFFFFFFu;
    return (ax - 1u) < 0x7F7FFFFFu ? b - 1u : b;  // 0 < |x| < inf: one ulp toward zero
}
template <int E>
LSMX_DEV uint32_t e2m1_pack_hw16(const uint32_t (&b)[E], uint32_t e8) {
    uint32_t bd[E];
#pragma unroll
    for (int i = 0; i < E; ++i) bd[i] = below_ulp(b[i]);
    return cvt_fp4_pairs<0, E>(0u, bd, u2f(e8 << 23));
}

// The same codes from the element-by-element rule (lsmx::e2m1_code), which
// also covers a NaN block (e8 == 255).
template <int E>
LSMX_DEV uint32_t e2m1_pack_exact(const uint32_t (&b)[E], uint32_t e8) {
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) w |= e2m1_code(b[i], e8) << (4 * i);
    return w;
}

// ------------------------------------------------------- row-mode quantize
// Grid: (x = chunks of kThreads*kUnroll vectors along a row, y = rows, grid-
// strided).  One vector = 16 input bytes.
constexpr int kQThreads = 256;
constexpr int kQUnroll = 2;  // measured: 2 vectors per thread beat 1, 4 and 8 (more, shorter workgroups)

// Scale store for block kb of row r in format SFMT (LSMX_SCALE_*).
template <int SFMT>
LSMX_DEV void store_scale(void *scale, int64_t r, int64_t kb, int64_t ld_scale, uint32_t e8) {
    if constexpr (SFMT == LSMX_SCALE_F32)
        reinterpret_cast<float *>(scale)[r * ld_scale + kb] = e8m0_to_f32(e8);
    else if constexpr (SFMT == LSMX_SCALE_E8M0)
        reinterpret_cast<uint8_t *>(scale)[r * ld_scale + kb] = (uint8_t)e8;
    else  // K-major: [K/128][ld_scale rows][4]
        reinterpret_cast<uint8_t *>(scale)[((kb >> 2) * ld_scale + r) * 4 + (kb & 3)] = (uint8_t)e8;
}

// Row r of x (xr: its first element), the kQUnroll vectors of this thread
// from vector v0 on.  Every lane of the workgroup calls it for the same row
// (the block maxima and K-major scale gathers are cross-lane).
template <typename T, int BLOCK, bool PACKED, int SFMT>
LSMX_DEV void quantize_row(const T *__restrict__ xr, int64_t K, uint8_t *__restrict__ codes, int64_t ld_codes,
                           void *__restrict__ scale, int64_t ld_scale, int64_t r, int64_t v0) {
    constexpr int E = Elem<T>::kPerVec;
    constexpr int G = BLOCK / E;  // lanes per block
    const int64_t vpr = K / E;    // vectors per row
    uint4 buf[kQUnroll];
#pragma unroll
    for (int u = 0; u < kQUnroll; ++u) {
        const int64_t v = v0 + u * kQThreads;
        if (v < vpr) {
            // streaming read: each input byte is used exactly once
            const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(xr) + v);
            buf[u] = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            buf[u] = make_uint4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int u = 0; u < kQUnroll; ++u) {
        const int64_t v = v0 + u * kQThreads;
        uint32_t b[E];
        Elem<T>::bits(buf[u], b);
        uint32_t am = 0;
#pragma unroll
        for (int i = 0; i < E; ++i) am = max(am, b[i] & 0x7FFFFFFFu);
        am = group_max<G>(am);  // every lane of the block participates
        const uint32_t e8 = block_e8m0(am);
        // K-major scales: the lane holding block kb (kb % 4 == 0) gathers
        // the bytes of kb..kb+3 -- the same row's dword -- for one store.
        // Every lane takes part in the cross-lane reads.
        uint32_t e4 = 0;
        if constexpr (SFMT == LSMX_SCALE_E8M0_KMAJOR && BLOCK == 32) {
            const int l = (int)(threadIdx.x & 63);
            e4 = e8 | ((uint32_t)__builtin_amdgcn_ds_bpermute(((l + G) & 63) << 2, (int)e8) << 8) |
                 ((uint32_t)__builtin_amdgcn_ds_bpermute(((l + 2 * G) & 63) << 2, (int)e8) << 16) |
                 ((uint32_t)__builtin_amdgcn_ds_bpermute(((l + 3 * G) & 63) << 2, (int)e8) << 24);
        }
        if (v >= vpr) continue;  // whole blocks are in or out of range
        // NaN blocks are rare: any lane with one takes the whole wave
        // through the exact per-element rule
        uint32_t w;
        if (__any(e8 == 255u)) w = e2m1_pack_exact<E>(b, e8);
        else if constexpr (sizeof(T) == 2) w = e2m1_pack_hw16<E>(b, e8);
        else w = e2m1_pack_hw<E>(b, e8);
        const int64_t col = v * E;
        if constexpr (PACKED) {
            if constexpr (E == 4) *reinterpret_cast<uint16_t *>(codes + r * ld_codes + col / 2) = (uint16_t)w;
            else *reinterpret_cast<uint32_t *>(codes + r * ld_codes + col / 2) = w;
        } else {
            uint32_t c[E];
#pragma unroll
            for (int i = 0; i < E; ++i) c[i] = (w >> (4 * i)) & 0xF;
            CodeStore<E>::unpacked(codes + r * ld_codes + col, c);
        }
        if constexpr (SFMT == LSMX_SCALE_E8M0_KMAJOR && BLOCK == 32) {
            const int64_t kb = col / BLOCK;
            // vectors of a wave start on a 4-block boundary (64 lanes x E elements)
            if ((threadIdx.x % (4 * G)) == 0)
                reinterpret_cast<uint32_t *>(scale)[(kb >> 2) * ld_scale + r] = e4;
        } else {
            if ((threadIdx.x % G) == 0) store_scale<SFMT>(scale, r, col / BLOCK, ld_scale, e8);
        }
    }
}

template <typename T, int BLOCK, bool PACKED, int SFMT>
__global__ __launch_bounds__(kQThreads) void quantize_rows_kernel(
    const T *__restrict__ x, int64_t rows, int64_t K, int64_t ldx, uint8_t *__restrict__ codes,
    int64_t ld_codes, void *__restrict__ scale, int64_t ld_scale) {
    const int64_t v0 = (int64_t)blockIdx.x * (kQThreads * kQUnroll) + threadIdx.x;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y)
        quantize_row<T, BLOCK, PACKED, SFMT>(x + r * ldx, K, codes, ld_codes, scale, ld_scale, r, v0);
}

// Several tensors of one dtype and format in one launch: the rows of tensor
// k are global rows end[k - 1] .. end[k] - 1, walked grid-strided along y;
// the grid's x extent covers the longest row (workgroups past a shorter
// row's end store nothing for it).
template <typename T, int SFMT>
__global__ __launch_bounds__(kQThreads) void quantize_rows_batch_kernel(QuantBatch b) {
    const int64_t v0 = (int64_t)blockIdx.x * (kQThreads * kQUnroll) + threadIdx.x;
    const int64_t total = b.end[b.n - 1];
    int k = 0;
    for (int64_t gr = blockIdx.y; gr < total; gr += gridDim.y) {
        while (gr >= b.end[k]) ++k;   // gr < total = end[n - 1]: k stays below n
        const QuantArgs &a = b.a[k];
        const int64_t r = gr - (k ? b.end[k - 1] : 0);
        quantize_row<T, 32, true, SFMT>(reinterpret_cast<const T *>(a.x) + r * a.ldx, a.K,
                                        reinterpret_cast<uint8_t *>(a.codes), a.ld_codes, a.scale, a.ld_scale, r,
                                        v0);
    }
}

// ------------------------------------------ both axes in one pass
// x[R, C] of 16-bit elements quantized along its rows (blocks of 32
// consecutive columns, the quantize_rows_kernel result) AND along its columns
// (blocks of 32 consecutive rows, the quantize_cols_kernel result, laid out
// for x^T), reading x once.  A training step needs both forms of every
// operand it quantizes: X and W along K for the forward, W and dY along N
// for dgrad, dY and X along T for wgrad (train_step.py:3-6).
//
// One workgroup of 4 waves per 128 x 128 tile; wave w holds the tile's rows
// 32w .. 32w+31, i.e. exactly one 32-row column block, so every reduction
// stays inside the wave.  Lane l holds the 8 columns 8(l%16) .. +8 of the 8
// rows 32w + 8(l/16) + i, i = 0..7 (eight 16-byte loads; each instruction
// reads four 256-byte row segments).
//   rows:    for each of its rows a lane and the 3 other lanes of its quad
//            hold one 32-column block: DPP max, hardware FP4 conversion,
//            4 bytes of codes per lane and row (64 contiguous bytes per row
//            and instruction).
//   columns: a lane's 8 rows of a column are a quarter of its block: max
//            over them, then over the 4 lanes l, l^16, l^32, l^48 of the
//            wave; each lane then converts its 4 row pairs of every column
//            with the column's scale (one dword per column), the dwords go
//            to LDS, and after one barrier each column's 64 bytes of codes
//            (the tile's 128 rows) are written by 4 adjacent lanes.
// The kernel is bound by vector-ALU issue unless each element costs only a
// few operations, so a wave whose 32 rows hold no Inf or NaN (nearly every
// wave) takes a short path:
//   - maxima on packed 16-bit magnitudes (unsigned order of the magnitude
//     bits of a bf16 or fp16 is the order of |x|, with Inf and NaN on top);
//   - the block scale from the bits of the absmax in three integer
//     operations (block_e8m0_16);
//   - each element widened to fp32 and multiplied by 1 - 2^-20 once, then
//     converted along both axes by the hardware's round-to-nearest-even
//     (tie_down16).
// A wave with an Inf or NaN in its rows writes its outputs again with the
// full scale rule and NaN codes (q2_convert_special).  Scales are E8M0,
// row-major or K-major; R and C are multiples of 128.  The common path holds
// under 96 registers, so 5 waves share each SIMD.
namespace q2 {
constexpr int T = 128;      // tile edge
constexpr int NT = 256;     // threads (4 waves)
}  // namespace q2

template <typename T>
LSMX_DEV void bits16(uint32_t w, uint32_t &lo, uint32_t &hi) {
    if constexpr (__is_same(T, f16_t)) {
        lo = f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu)));
        hi = f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)));
    } else {
        lo = w << 16;
        hi = w & 0xFFFF0000u;
    }
}

// fp32 bits of the larger of the two 16-bit magnitudes in m.
template <typename T>
LSMX_DEV uint32_t wider_half(uint32_t m) {
    if constexpr (__is_same(T, f16_t))
        return f2u((float)__builtin_bit_cast(_Float16, (uint16_t)max(m & 0xFFFFu, m >> 16)));
    else
        return max(m << 16, m & 0xFFFF0000u);
}

// fp32 bits of 16-bit magnitude half H (0: low, 1: high) of m.
template <typename T, int H>
LSMX_DEV uint32_t half_bits(uint32_t m) {
    uint32_t lo, hi;
    bits16<T>(m, lo, hi);
    return H ? hi : lo;
}

// v_cvt_scalef32_pk_fp4_f32 into byte j of w (j a constant once unrolled).
LSMX_DEV uint32_t cvt_fp4_pair(uint32_t w, float a, float b, float sc, int j) {
    switch (j) {
        case 0: return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, sc, 0);
        case 1: return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, sc, 1);
        case 2: return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, sc, 2);
        default: return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, sc, 3);
    }
}

// The conversion of a wave's 8 x 8 elements per lane along both axes, given
// the row-block maxima am and the column maxima cmx (packed 16-bit, already
// reduced over the wave), when its rows hold no Inf or NaN.  Rows go two at
// a time: each element is widened and nudged once, converted with its row
// block's scale and, paired with the element below it, with its column
// block's scale, so only 16 widened values are live at a time.  Row codes
// and scales go to memory, column codes and scales to LDS.
template <typename T, int SFMT, bool ROWS>
LSMX_DEV void q2_convert(const u32x4 (&raw)[8], const uint32_t (&am)[8], const uint32_t (&cmx)[4],
                         uint32_t (*ccode)[17], uint32_t *cscale, int64_t r0, int64_t c0, int lane, int w,
                         uint8_t *__restrict__ codes_r, int64_t ld_cr, uint8_t *__restrict__ scale_r, int64_t ld_sr) {
    const int v = lane & 15, g = lane >> 4;
    const int rl = 32 * w + 8 * g;
    const int64_t slice = c0 / 128;
    uint32_t e8c[8], dw[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        e8c[e] = block_e8m0_16((e & 1) ? half_bits<T, 1>(cmx[e >> 1]) : half_bits<T, 0>(cmx[e >> 1]));
        dw[e] = 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float f[2][8];  // rows 2j and 2j+1, widened and nudged
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t lo, hi;
                bits16<T>(raw[2 * j + h][p], lo, hi);
                f[h][2 * p] = tie_down16(lo);
                f[h][2 * p + 1] = tie_down16(hi);
            }
            if constexpr (ROWS) {
                const int i = 2 * j + h;
                const uint32_t e8 = block_e8m0_16(am[i]);
                const int64_t r = r0 + rl + i;
                *reinterpret_cast<uint32_t *>(codes_r + r * ld_cr + (c0 + 8 * v) / 2) = cvt_fp4_x8(f[h], u2f(e8 << 23));
                if ((v & 3) == 0) {  // the quad's block byte
                    if constexpr (SFMT == LSMX_SCALE_E8M0_KMAJOR)
                        scale_r[(slice * ld_sr + r) * 4 + (v >> 2)] = (uint8_t)e8;
                    else
                        scale_r[r * ld_sr + c0 / 32 + (v >> 2)] = (uint8_t)e8;
                }
            }
        }
        // column e: rows 2j, 2j+1 into byte j (row rl in the low nibble)
#pragma unroll
        for (int e = 0; e < 8; ++e) dw[e] = cvt_fp4_pair(dw[e], f[0][e], f[1][e], u2f(e8c[e] << 23), j);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        ccode[8 * v + e][4 * w + g] = dw[e];
        if (g == 0) reinterpret_cast<uint8_t *>(cscale)[4 * (8 * v + e) + w] = (uint8_t)e8c[e];
    }
}

// The same outputs for a wave whose rows hold an Inf or NaN, with the scale
// rule and codes of block_e8m0_16x and codes8_any.  Rare: rows and columns
// are widened separately to keep its registers below the common path's.
template <typename T, int SFMT, bool ROWS>
LSMX_DEV void q2_convert_special(u32x4 (&raw)[8], const uint32_t (&am)[8], const uint32_t (&cmx)[4],
                                 uint32_t (*ccode)[17], uint32_t *cscale, int64_t r0, int64_t c0, int lane, int w,
                                 uint8_t *__restrict__ codes_r, int64_t ld_cr, uint8_t *__restrict__ scale_r,
                                 int64_t ld_sr) {
    const int v = lane & 15, g = lane >> 4;
    const int rl = 32 * w + 8 * g;
    const int64_t slice = c0 / 128;
    if constexpr (ROWS) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float f[8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t lo, hi;
                bits16<T>(raw[i][p], lo, hi);
                f[2 * p] = nudge_keep_nan(lo);
                f[2 * p + 1] = nudge_keep_nan(hi);
            }
            const uint32_t e8 = block_e8m0_16x(am[i]);
            const int64_t r = r0 + rl + i;
            *reinterpret_cast<uint32_t *>(codes_r + r * ld_cr + (c0 + 8 * v) / 2) = codes8_any(f, e8);
            if ((v & 3) == 0) {
                if constexpr (SFMT == LSMX_SCALE_E8M0_KMAJOR)
                    scale_r[(slice * ld_sr + r) * 4 + (v >> 2)] = (uint8_t)e8;
                else
                    scale_r[r * ld_sr + c0 / 32 + (v >> 2)] = (uint8_t)e8;
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(raw[i]));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t e8 = block_e8m0_16x((e & 1) ? half_bits<T, 1>(cmx[e >> 1]) : half_bits<T, 0>(cmx[e >> 1]));
        float f[8];  // this lane's 8 rows of column 8v + e
#pragma unroll
        for (int i = 0; i < 8; ++i)
            f[i] = nudge_keep_nan((e & 1) ? half_bits<T, 1>(raw[i][e >> 1]) : half_bits<T, 0>(raw[i][e >> 1]));
        ccode[8 * v + e][4 * w + g] = codes8_any(f, e8);  // row rl in the low nibble
        if (g == 0) reinterpret_cast<uint8_t *>(cscale)[4 * (8 * v + e) + w] = (uint8_t)e8;
    }
}

// Block maxima of a wave's 8 x 8 elements per lane, on packed 16-bit
// magnitudes: am[i] = fp32 bits of row i's block absmax (the quad's 32
// columns), cmx = the column maxima over the wave's 32 rows (lanes l, l^16,
// l^32, l^48), two 16-bit halves per dword.  Returns the largest am[i].
template <typename T>
LSMX_DEV uint32_t q2_maxima(const u32x4 (&raw)[8], uint32_t (&am)[8], uint32_t (&cmx)[4]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t m[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            m[p] = raw[i][p] & 0x7FFF7FFFu;
            cmx[p] = i == 0 ? m[p] : pk_max16(cmx[p], m[p]);
        }
        am[i] = group_max<4>(wider_half<T>(pk_max16(pk_max16(m[0], m[1]), pk_max16(m[2], m[3]))));
    }
    uint32_t top = am[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) top = max(top, am[i]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        cmx[p] = pk_max16(cmx[p], (uint32_t)__shfl_xor((int)cmx[p], 16, 64));
        cmx[p] = pk_max16(cmx[p], (uint32_t)__shfl_xor((int)cmx[p], 32, 64));
    }
    return top;
}

// One 128 x 128 tile of x (tile index `tile`, row-major over the tiles),
// by one workgroup of q2::NT threads.  ROWS = false: the column form only
// (lsmx_quantize_mxfp4_t of a 16-bit x).
template <typename T, int SFMT, bool ROWS>
LSMX_DEV void q2_tile(const T *__restrict__ x, int64_t R, int64_t C, int64_t ldx, uint8_t *__restrict__ codes_r,
                      int64_t ld_cr, uint8_t *__restrict__ scale_r, int64_t ld_sr, uint8_t *__restrict__ codes_c,
                      int64_t ld_cc, uint8_t *__restrict__ scale_c, int64_t ld_sc, int64_t tile) {
    static_assert(sizeof(T) == 2, "16-bit inputs");
    // [column][dword]: dword 4w + g holds the codes of tile rows 32w + 8g .. +8
    __shared__ __attribute__((aligned(16))) uint32_t ccode[q2::T][17];
    __shared__ uint32_t cscale[q2::T];

    const int64_t tiles_c = C / q2::T;
    const int64_t r0 = (tile / tiles_c) * q2::T, c0 = (tile % tiles_c) * q2::T;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int v = lane & 15, g = lane >> 4;
    const int rl = 32 * w + 8 * g;                       // first tile row of this lane

    u32x4 raw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        raw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + (r0 + rl + i) * ldx + c0 + 8 * v));

    uint32_t am[8], cmx[4];
    const uint32_t top = q2_maxima<T>(raw, am, cmx);
    q2_convert<T, SFMT, ROWS>(raw, am, cmx, ccode, cscale, r0, c0, lane, w, codes_r, ld_cr, scale_r, ld_sr);
    if (__any(top >= 0x7F800000u)) {
        // rare: an Inf or NaN in the wave's rows.  Its outputs are written
        // again with the full rules, from a second load of its words (from
        // L2), so that no register stays live for this path through the
        // common one.  The empty asm hides that the lane index and the load
        // are the ones above: otherwise the compiler keeps the first load
        // and every per-lane address of the common path for reuse here.
        int lane2 = lane;
        asm volatile("" : "+v"(lane2));
        const int rl2 = 32 * w + 8 * (lane2 >> 4);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            raw[i] = *reinterpret_cast<const u32x4 *>(x + (r0 + rl2 + i) * ldx + c0 + 8 * (lane2 & 15));
        q2_maxima<T>(raw, am, cmx);
        q2_convert_special<T, SFMT, ROWS>(raw, am, cmx, ccode, cscale, r0, c0, lane2, w, codes_r, ld_cr, scale_r,
                                          ld_sr);
    }
    __syncthreads();
    {
        // column 64k + t / 4, quarter t % 4 (16 of its 64 bytes): 4 adjacent
        // lanes write each column's 64 bytes in one instruction
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int col = 64 * k + (t >> 2), q = t & 3;
            const uint32_t *src = &ccode[col][4 * q];
            *reinterpret_cast<u32x4 *>(codes_c + (c0 + col) * ld_cc + r0 / 2 + 16 * q) =
                u32x4{src[0], src[1], src[2], src[3]};
        }
        if (t < q2::T) {
            const uint32_t e4 = cscale[t];
            if constexpr (SFMT == LSMX_SCALE_E8M0_KMAJOR)
                reinterpret_cast<uint32_t *>(scale_c)[(r0 / 128) * ld_sc + c0 + t] = e4;
            else
                *reinterpret_cast<uint32_t *>(scale_c + (c0 + t) * ld_sc + r0 / 32) = e4;
        }
    }
}

template <typename T, int SFMT, bool ROWS = true>
__global__ __launch_bounds__(q2::NT, 5) void quantize_2d_kernel(
    const T *__restrict__ x, int64_t R, int64_t C, int64_t ldx, uint8_t *__restrict__ codes_r, int64_t ld_cr,
    uint8_t *__restrict__ scale_r, int64_t ld_sr, uint8_t *__restrict__ codes_c, int64_t ld_cc,
    uint8_t *__restrict__ scale_c, int64_t ld_sc) {
    q2_tile<T, SFMT, ROWS>(x, R, C, ldx, codes_r, ld_cr, scale_r, ld_sr, codes_c, ld_cc, scale_c, ld_sc,
                           (int64_t)blockIdx.x);
}

// Several tensors in one launch: workgroup b takes tile b - end[k - 1] of
// tensor k, the first k with b < end[k] (end: running tile counts).  One
// launch keeps the memory system busy across the tensors' boundaries, where
// separate launches of a few-MB tensor each pay a ramp-up and a drain.
template <typename T, int SFMT>
__global__ __launch_bounds__(q2::NT, 5) void quantize_2d_batch_kernel(Quant2dBatch b) {
    const int64_t blk = (int64_t)blockIdx.x;
    int k = 0;
    while (k + 1 < b.n && blk >= b.end[k]) ++k;
    const Quant2dArgs &a = b.a[k];
    q2_tile<T, SFMT, true>(reinterpret_cast<const T *>(a.x), a.R, a.C, a.ldx, a.codes_r, a.ld_cr, a.scale_r, a.ld_sr,
                           a.codes_c, a.ld_cc, a.scale_c, a.ld_sc, blk - (k ? b.end[k - 1] : 0));
}

hipError_t launch_quantize_2d_batch(const Quant2dBatch &b, hipStream_t s) {
    const dim3 grid((unsigned)b.end[b.n - 1]), blk(q2::NT);
    const bool bf = b.a[0].x_dtype == LSMX_BF16, km = b.a[0].scale_fmt == LSMX_SCALE_E8M0_KMAJOR;
    if (bf && km) hipLaunchKernelGGL((quantize_2d_batch_kernel<bf16_t, LSMX_SCALE_E8M0_KMAJOR>), grid, blk, 0, s, b);
    else if (bf) hipLaunchKernelGGL((quantize_2d_batch_kernel<bf16_t, LSMX_SCALE_E8M0>), grid, blk, 0, s, b);
    else if (km) hipLaunchKernelGGL((quantize_2d_batch_kernel<f16_t, LSMX_SCALE_E8M0_KMAJOR>), grid, blk, 0, s, b);
    else hipLaunchKernelGGL((quantize_2d_batch_kernel<f16_t, LSMX_SCALE_E8M0>), grid, blk, 0, s, b);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_2d(const Quant2dArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.R / q2::T) * (a.C / q2::T))), blk(q2::NT);
#define LSMX_Q2(F)                                                                                                \
    hipLaunchKernelGGL((quantize_2d_kernel<T, F>), grid, blk, 0, s, reinterpret_cast<const T *>(a.x), a.R, a.C,  \
                       a.ldx, a.codes_r, a.ld_cr, a.scale_r, a.ld_sr, a.codes_c, a.ld_cc, a.scale_c, a.ld_sc)
    if (a.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) LSMX_Q2(LSMX_SCALE_E8M0_KMAJOR);
    else LSMX_Q2(LSMX_SCALE_E8M0);
#undef LSMX_Q2
    return hipGetLastError();
}

hipError_t launch_quantize_2d(const Quant2dArgs &a, hipStream_t s) {
    return a.x_dtype == LSMX_BF16 ? launch_2d<bf16_t>(a, s) : launch_2d<f16_t>(a, s);
}

// ------------------------------------------------- column-mode quantize
// x[K, cols]: blocks of BLOCK consecutive rows within one column.  One thread
// per (column, block); consecutive threads take consecutive columns, so every
// load instruction of a wave reads 64 consecutive elements of one row.
constexpr int kTThreads = 256;

template <typename T, int BLOCK, bool PACKED, int SFMT>
__global__ __launch_bounds__(kTThreads) void quantize_cols_kernel(
    const T *__restrict__ x, int64_t K, int64_t cols, int64_t ldx, uint8_t *__restrict__ codes,
    int64_t ld_codes, void *__restrict__ scale, int64_t ld_scale) {
    const int64_t c = (int64_t)blockIdx.x * kTThreads + threadIdx.x;
    if (c >= cols) return;
    const int64_t nkb = K / BLOCK;
    for (int64_t kb = blockIdx.y; kb < nkb; kb += gridDim.y) {
        const T *xp = x + kb * BLOCK * ldx + c;
        uint32_t b[BLOCK];
#pragma unroll
        for (int i = 0; i < BLOCK; ++i) {
            if constexpr (sizeof(T) == 4) {
                b[i] = __builtin_bit_cast(uint32_t, xp[i * ldx]);
            } else {
                const uint16_t h = __builtin_bit_cast(uint16_t, xp[i * ldx]);
                uint32_t w = (uint32_t)h;
                if constexpr (__is_same(T, f16_t))
                    b[i] = f2u((float)__builtin_bit_cast(_Float16, h));
                else
                    b[i] = w << 16;
            }
        }
        uint32_t am = 0;
#pragma unroll
        for (int i = 0; i < BLOCK; ++i) am = max(am, b[i] & 0x7FFFFFFFu);
        const uint32_t e8 = block_e8m0(am);
        uint8_t *out = codes + c * ld_codes;
        if constexpr (PACKED) {
            uint32_t w[BLOCK / 8];
#pragma unroll
            for (int j = 0; j < BLOCK / 8; ++j) {
                w[j] = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) w[j] |= e2m1_code(b[8 * j + i], e8) << (4 * i);
            }
            if constexpr (BLOCK == 32)
                *reinterpret_cast<uint4 *>(out + kb * 16) = make_uint4(w[0], w[1], w[2], w[3]);
            else
                *reinterpret_cast<uint2 *>(out + kb * 8) = make_uint2(w[0], w[1]);
        } else {
#pragma unroll
            for (int j = 0; j < BLOCK / 16; ++j) {
                uint32_t w[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    w[q] = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) w[q] |= e2m1_code(b[16 * j + 4 * q + i], e8) << (8 * i);
                }
                *reinterpret_cast<uint4 *>(out + kb * BLOCK + 16 * j) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
        store_scale<SFMT>(scale, c, kb, ld_scale, e8);
    }
}

// ---------------------------------------------------------- elementwise
template <int DT>
__global__ void round_kernel(const void *__restrict__ q, int64_t n, uint8_t *__restrict__ codes) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t b;
    if constexpr (DT == LSMX_F32) b = reinterpret_cast<const uint32_t *>(q)[i];
    else if constexpr (DT == LSMX_BF16) b = (uint32_t)reinterpret_cast<const uint16_t *>(q)[i] << 16;
    else b = f2u((float)reinterpret_cast<const _Float16 *>(q)[i]);
    codes[i] = (uint8_t)e2m1_code(b, 127u);  // scale 1, never the NaN-block path
}

__global__ void pack_kernel(const uint4 *__restrict__ codes, uint2 *__restrict__ packed, int64_t n16,
                            const uint8_t *__restrict__ codes_b, uint8_t *__restrict__ packed_b,
                            int64_t n_bytes) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) {
        const uint4 c = codes[i];  // 16 codes -> 8 bytes
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
        uint32_t o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t a = w[2 * h], b = w[2 * h + 1];
            uint32_t pa = (a & 0xF) | ((a >> 4) & 0xF0) | ((a >> 8) & 0xF00) | ((a >> 12) & 0xF000);
            uint32_t pb = (b & 0xF) | ((b >> 4) & 0xF0) | ((b >> 8) & 0xF00) | ((b >> 12) & 0xF000);
            o[h] = pa | (pb << 16);
        }
        packed[i] = make_uint2(o[0], o[1]);
    }
    // tail bytes (n_bytes not a multiple of 8)
    const int64_t t = n16 * 8 + i;
    if (i < 8 && t < n_bytes) packed_b[t] = (uint8_t)((codes_b[2 * t] & 0xF) | ((codes_b[2 * t + 1] & 0xF) << 4));
}

__global__ void unpack_kernel(const uint2 *__restrict__ packed, uint4 *__restrict__ codes, int64_t n8,
                              const uint8_t *__restrict__ packed_b, uint8_t *__restrict__ codes_b,
                              int64_t n_bytes) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n8) {
        const uint2 p = packed[i];  // 8 bytes -> 16 codes
        const uint32_t w[2] = {p.x, p.y};
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                uint32_t s = (w[h] >> (16 * q)) & 0xFFFF;  // 4 nibbles
                o[2 * h + q] = (s & 0xF) | ((s & 0xF0) << 4) | ((s & 0xF00) << 8) | ((s & 0xF000) << 12);
            }
        }
        codes[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    const int64_t t = n8 * 8 + i;
    if (i < 8 && t < n_bytes) {
        codes_b[2 * t] = packed_b[t] & 0xF;
        codes_b[2 * t + 1] = packed_b[t] >> 4;
    }
}

__global__ void fp4_to_e4m3_kernel(const uint32_t *__restrict__ in, uint2 *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const uint32_t p = in[i];
        out[i] = make_uint2(fp4x4_to_e4m3x4(p & 0xFFFF), fp4x4_to_e4m3x4(p >> 16));
    }
}

// 16-byte aligned buffers: 4 words per lane (one 16-byte load, two 16-byte
// stores), so a wave moves 1 KiB in and 2 KiB out per instruction pair.  The
// lane past the last whole quad converts the 0-3 words left over.
__global__ void fp4_to_e4m3_x4_kernel(const u32x4 *__restrict__ in, u32x4 *__restrict__ out, int64_t n) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nq = n >> 2;
    if (q < nq) {
        const u32x4 p = in[q];
        u32x4 lo, hi;
        lo.x = fp4x4_to_e4m3x4(p.x & 0xFFFF), lo.y = fp4x4_to_e4m3x4(p.x >> 16);
        lo.z = fp4x4_to_e4m3x4(p.y & 0xFFFF), lo.w = fp4x4_to_e4m3x4(p.y >> 16);
        hi.x = fp4x4_to_e4m3x4(p.z & 0xFFFF), hi.y = fp4x4_to_e4m3x4(p.z >> 16);
        hi.z = fp4x4_to_e4m3x4(p.w & 0xFFFF), hi.w = fp4x4_to_e4m3x4(p.w >> 16);
        out[2 * q] = lo;
        out[2 * q + 1] = hi;
    } else if (q == nq) {
        const uint32_t *iw = reinterpret_cast<const uint32_t *>(in);
        uint2 *ow = reinterpret_cast<uint2 *>(out);
        for (int64_t i = 4 * nq; i < n; ++i) {
            const uint32_t p = iw[i];
            ow[i] = make_uint2(fp4x4_to_e4m3x4(p & 0xFFFF), fp4x4_to_e4m3x4(p >> 16));
        }
    }
}

template <bool PACKED, bool SCALE_F32, bool OUT_BF16>
__global__ void dequant_kernel(const uint8_t *__restrict__ codes, int64_t ld_codes,
                               const void *__restrict__ scale, int64_t ld_scale, int64_t rows,
                               int64_t K, int block, void *__restrict__ out, int64_t ld_out) {
    // one thread per 8 consecutive elements of a row
    const int64_t per_row = K / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * per_row) return;
    const int64_t r = i / per_row, k0 = (i % per_row) * 8;
    uint32_t c[8];
    if constexpr (PACKED) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(codes + r * ld_codes + k0 / 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = (w >> (4 * j)) & 0xF;
    } else {
        const uint2 w = *reinterpret_cast<const uint2 *>(codes + r * ld_codes + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) { c[j] = (w.x >> (8 * j)) & 0xF; c[j + 4] = (w.y >> (8 * j)) & 0xF; }
    }
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t kb = (k0 + j) / block;
        float s;
        if constexpr (SCALE_F32) s = reinterpret_cast<const float *>(scale)[r * ld_scale + kb];
        else s = e8m0_to_f32(reinterpret_cast<const uint8_t *>(scale)[r * ld_scale + kb]);
        v[j] = e2m1_value(c[j]) * s;
    }
    if constexpr (OUT_BF16) {
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // exact: an E2M1 value times a power of two has <= 2 significant bits
            const uint32_t lo = f2u(v[2 * j]) >> 16, hi = f2u(v[2 * j + 1]) >> 16;
            o[j] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(out) + r * ld_out + k0) =
            make_uint4(o[0], o[1], o[2], o[3]);
    } else {
        float4 *o = reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + r * ld_out + k0);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// ---------------------------------------------------------------- launchers
template <typename T, int BLOCK, bool PACKED, int SF32>
static hipError_t launch_rows(const QuantArgs &a, hipStream_t s) {
    constexpr int E = Elem<T>::kPerVec;
    const int64_t vpr = a.K / E;
    const int64_t gx = (vpr + kQThreads * kQUnroll - 1) / (kQThreads * kQUnroll);
    const int64_t gy = a.rows < 65535 ? a.rows : 65535;
    hipLaunchKernelGGL((quantize_rows_kernel<T, BLOCK, PACKED, SF32>), dim3((unsigned)gx, (unsigned)gy),
                       dim3(kQThreads), 0, s, reinterpret_cast<const T *>(a.x), a.rows, a.K, a.ldx,
                       reinterpret_cast<uint8_t *>(a.codes), a.ld_codes, a.scale, a.ld_scale);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_rows_batch(const QuantBatch &b, hipStream_t s) {
    constexpr int E = Elem<T>::kPerVec;
    int64_t kmax = 0;
    for (int k = 0; k < b.n; ++k) kmax = b.a[k].K > kmax ? b.a[k].K : kmax;
    const int64_t gx = (kmax / E + kQThreads * kQUnroll - 1) / (kQThreads * kQUnroll);
    const int64_t total = b.end[b.n - 1];
    const int64_t gy = total < 65535 ? total : 65535;
    if (b.a[0].scale_fmt == LSMX_SCALE_E8M0_KMAJOR)
        hipLaunchKernelGGL((quantize_rows_batch_kernel<T, LSMX_SCALE_E8M0_KMAJOR>), dim3((unsigned)gx, (unsigned)gy),
                           dim3(kQThreads), 0, s, b);
    else
        hipLaunchKernelGGL((quantize_rows_batch_kernel<T, LSMX_SCALE_E8M0>), dim3((unsigned)gx, (unsigned)gy),
                           dim3(kQThreads), 0, s, b);
    return hipGetLastError();
}

hipError_t launch_quantize_batch(const QuantBatch &b, hipStream_t s) {
    switch (b.a[0].x_dtype) {
        case LSMX_F32: return launch_rows_batch<float>(b, s);
        case LSMX_BF16: return launch_rows_batch<bf16_t>(b, s);
        default: return launch_rows_batch<f16_t>(b, s);
    }
}

template <typename T, int BLOCK, bool PACKED, int SF32>
static hipError_t launch_cols(const QuantArgs &a, hipStream_t s) {
    // 16-bit x, 32-blocks, packed codes and E8M0 scales on whole 128 x 128
    // tiles: the column half of the two-axis kernel (one 32-row block per
    // wave, 64-byte code runs per column)
    if constexpr (sizeof(T) == 2 && BLOCK == 32 && PACKED && SF32 != LSMX_SCALE_F32) {
        const uintptr_t cp = reinterpret_cast<uintptr_t>(a.codes), sp = reinterpret_cast<uintptr_t>(a.scale);
        if (a.K % q2::T == 0 && a.rows % q2::T == 0 && a.ldx * 2 % 16 == 0 &&
            (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (cp & 15) == 0 && a.ld_codes % 16 == 0 &&
            (sp & 3) == 0 && (SF32 == LSMX_SCALE_E8M0_KMAJOR || a.ld_scale % 4 == 0)) {
            const dim3 grid((unsigned)((a.K / q2::T) * (a.rows / q2::T))), blk(q2::NT);
            hipLaunchKernelGGL((quantize_2d_kernel<T, SF32, false>), grid, blk, 0, s, reinterpret_cast<const T *>(a.x),
                               a.K, a.rows, a.ldx, nullptr, (int64_t)0, nullptr, (int64_t)0,
                               reinterpret_cast<uint8_t *>(a.codes), a.ld_codes, reinterpret_cast<uint8_t *>(a.scale),
                               a.ld_scale);
            return hipGetLastError();
        }
    }
    // a.rows = cols, a.K = K for the column mode
    const int64_t gx = (a.rows + kTThreads - 1) / kTThreads;
    const int64_t nkb = a.K / BLOCK;
    const int64_t gy = nkb < 65535 ? nkb : 65535;
    hipLaunchKernelGGL((quantize_cols_kernel<T, BLOCK, PACKED, SF32>), dim3((unsigned)gx, (unsigned)gy),
                       dim3(kTThreads), 0, s, reinterpret_cast<const T *>(a.x), a.K, a.rows, a.ldx,
                       reinterpret_cast<uint8_t *>(a.codes), a.ld_codes, a.scale, a.ld_scale);
    return hipGetLastError();
}

template <typename T, int BLOCK>
static hipError_t dispatch_fmt(const QuantArgs &a, bool cols, hipStream_t s) {
    const bool packed = a.codes_fmt == LSMX_CODES_PACKED;
#define LSMX_Q(P, F) return cols ? launch_cols<T, BLOCK, P, F>(a, s) : launch_rows<T, BLOCK, P, F>(a, s)
    if (a.scale_fmt == LSMX_SCALE_F32) {
        if (packed) LSMX_Q(true, LSMX_SCALE_F32);
        LSMX_Q(false, LSMX_SCALE_F32);
    }
    if (a.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) {
        if (packed) LSMX_Q(true, LSMX_SCALE_E8M0_KMAJOR);
        LSMX_Q(false, LSMX_SCALE_E8M0_KMAJOR);
    }
    if (packed) LSMX_Q(true, LSMX_SCALE_E8M0);
    LSMX_Q(false, LSMX_SCALE_E8M0);
#undef LSMX_Q
}

template <typename T>
static hipError_t dispatch_block(const QuantArgs &a, bool cols, hipStream_t s) {
    return a.block == 32 ? dispatch_fmt<T, 32>(a, cols, s) : dispatch_fmt<T, 16>(a, cols, s);
}

hipError_t launch_quantize(const QuantArgs &a, bool cols, hipStream_t s) {
    switch (a.x_dtype) {
        case LSMX_F32: return dispatch_block<float>(a, cols, s);
        case LSMX_BF16: return dispatch_block<bf16_t>(a, cols, s);
        default: return dispatch_block<f16_t>(a, cols, s);
    }
}

hipError_t launch_round(const void *q, int q_dtype, int64_t n, uint8_t *codes, hipStream_t s) {
    const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
    if (q_dtype == LSMX_F32) hipLaunchKernelGGL(round_kernel<LSMX_F32>, grid, blk, 0, s, q, n, codes);
    else if (q_dtype == LSMX_BF16) hipLaunchKernelGGL(round_kernel<LSMX_BF16>, grid, blk, 0, s, q, n, codes);
    else hipLaunchKernelGGL(round_kernel<LSMX_F16>, grid, blk, 0, s, q, n, codes);
    return hipGetLastError();
}

hipError_t launch_pack(const uint8_t *codes, uint8_t *packed, int64_t n_bytes, hipStream_t s) {
    const int64_t n16 = n_bytes / 8;  // groups of 16 codes
    const int64_t threads = n16 > 8 ? n16 : 8;
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const uint4 *>(codes), reinterpret_cast<uint2 *>(packed), n16,
                       codes, packed, n_bytes);
    return hipGetLastError();
}

hipError_t launch_unpack(const uint8_t *packed, uint8_t *codes, int64_t n_bytes, hipStream_t s) {
    const int64_t n8 = n_bytes / 8;
    const int64_t threads = n8 > 8 ? n8 : 8;
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const uint2 *>(packed), reinterpret_cast<uint4 *>(codes), n8,
                       packed, codes, n_bytes);
    return hipGetLastError();
}

hipError_t launch_fp4_to_e4m3(const uint32_t *in, uint32_t *out, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (((uintptr_t)in | (uintptr_t)out) % 16 == 0) {
        const int64_t lanes = (n >> 2) + 1;  // whole quads plus the tail lane
        hipLaunchKernelGGL(fp4_to_e4m3_x4_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, s,
                           reinterpret_cast<const u32x4 *>(in), reinterpret_cast<u32x4 *>(out), n);
    } else {
        hipLaunchKernelGGL(fp4_to_e4m3_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in,
                           reinterpret_cast<uint2 *>(out), n);
    }
    return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs &a, hipStream_t s) {
    const int64_t n = a.rows * (a.K / 8);
    const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
    const bool p = a.codes_fmt == LSMX_CODES_PACKED, f = a.scale_fmt == LSMX_SCALE_F32,
               b = a.out_dtype == LSMX_BF16;
#define LSMX_D(P, F, B)                                                                          \
    hipLaunchKernelGGL((dequant_kernel<P, F, B>), grid, blk, 0, s,                               \
                       reinterpret_cast<const uint8_t *>(a.codes), a.ld_codes, a.scale, a.ld_scale, \
                       a.rows, a.K, a.block, a.out, a.ld_out)
    if (p && f && b) LSMX_D(true, true, true);
    else if (p && f) LSMX_D(true, true, false);
    else if (p && b) LSMX_D(true, false, true);
    else if (p) LSMX_D(true, false, false);
    else if (f && b) LSMX_D(false, true, true);
    else if (f) LSMX_D(false, true, false);
    else if (b) LSMX_D(false, false, true);
    else LSMX_D(false, false, false);
#undef LSMX_D
    return hipGetLastError();
}

}  // namespace lsmx
