// Epilogue helpers shared by the GEMM kernels: fp32 -> bf16/fp16 stores of
// accumulator values, the in-quad 4x4 transpose that gives each lane four
// consecutive output columns, and the load-wait + barrier of the stage loops.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsmx_common.h"

namespace lsmx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with round-to-nearest-even (the reference's `acc.to(bf16)`):
// one v_cvt_pk_bf16_f32 per pair of values on gfx950.
typedef __bf16 v2bf16 __attribute__((ext_vector_type(2)));
LSMX_DEV uint32_t bf16x2(float lo, float hi) { return __builtin_bit_cast(uint32_t, v2bf16{(__bf16)lo, (__bf16)hi}); }
LSMX_DEV uint32_t bf16_rne(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f); }

LSMX_DEV uint32_t f16_bits(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f); }

template <int CT>
LSMX_DEV void store_c(void *c, int64_t idx, float v) {
    if constexpr (CT == LSMX_F32) reinterpret_cast<float *>(c)[idx] = v;
    else if constexpr (CT == LSMX_BF16) reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)bf16_rne(v);
    else reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)f16_bits(v);
}

// 4 consecutive columns of one row from one lane.
template <int CT>
LSMX_DEV void store_c4(void *c, int64_t idx, float v0, float v1, float v2, float v3) {
    if constexpr (CT == LSMX_F32) {
        *reinterpret_cast<u32x4 *>(reinterpret_cast<float *>(c) + idx) = u32x4{f2u(v0), f2u(v1), f2u(v2), f2u(v3)};
    } else if constexpr (CT == LSMX_BF16) {
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(c) + idx) =
            u32x2{bf16x2(v0, v1), bf16x2(v2, v3)};
    } else {
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(c) + idx) =
            u32x2{f16_bits(v0) | (f16_bits(v1) << 16), f16_bits(v2) | (f16_bits(v3) << 16)};
    }
}

// Value held by the lane `D` away inside each quad (D = 1: 1,0,3,2; D = 2: 2,3,0,1).
template <int D>
LSMX_DEV float quad_xor(float v) {
    constexpr int ctrl = D == 1 ? 0xB1 : 0x4E;
    // every lane of a quad is a valid source, so bound_ctrl needs no "old" value
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, true));
}

// 4x4 transpose inside each quad of lanes: on entry lane q holds x[r] =
// M[r][q] (rows r of column q); on exit x[c] = M[q][c] (columns c of row q).
// Two butterfly stages: at distance d, x[k] with bit d of k different from
// bit d of q is replaced by the partner lane's x[k ^ d].
LSMX_DEV void quad_transpose(float (&x)[4], int q) {
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float o = quad_xor<1>(x[k ^ 1]);
        y[k] = ((k ^ q) & 1) ? o : x[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float o = quad_xor<2>(y[k ^ 2]);
        x[k] = ((k ^ q) & 2) ? o : y[k];
    }
}

// Value held by the lane `D` away inside each quad, for 32-bit words.
template <int D>
LSMX_DEV uint32_t quad_xor_u(uint32_t v) {
    constexpr int ctrl = D == 1 ? 0xB1 : 0x4E;
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, true);
}

// A 4x4 block of 16-bit outputs held one column per lane of each quad
// (lane q: x[r] = M[r][q]), rounded and transposed so that lane q holds row
// q: the two words of M[q][0..3].  The values are rounded first and the
// transpose moves packed pairs: two exchanges of one word each and four byte
// permutes, instead of eight exchanges and eight selects of fp32 values.
//   1. words: lane q keeps rows {2qh, 2qh+1} (qh = q >> 1) of its column and
//      takes the same rows of column q ^ 2 from lane q ^ 2;
//   2. halves: lane q keeps row q of both columns and takes row q of columns
//      q ^ 1 and q ^ 3 from lane q ^ 1;
//   3. bytes: put the four columns of row q in order.
// The transpose of quad_pack16 on values already rounded and packed: p0 =
// rows 0 and 1, p1 = rows 2 and 3 of lane q's column.
LSMX_DEV u32x2 quad_pack16_bits(uint32_t p0, uint32_t p1, int q) {
    const bool qh = (q & 2) != 0, ql = (q & 1) != 0;
    const uint32_t t0 = qh ? p1 : p0;
    const uint32_t t1 = quad_xor_u<2>(qh ? p0 : p1);
    // v_perm_b32: selector bytes 0-3 pick bytes of the second operand, 4-7 of the first
    const uint32_t keep = __builtin_amdgcn_perm(t1, t0, ql ? 0x07060302u : 0x05040100u);
    const uint32_t recv = quad_xor_u<1>(__builtin_amdgcn_perm(t1, t0, ql ? 0x05040100u : 0x07060302u));
    // keep = (col q, col q^2), recv = (col q^1, col q^3) of row q
    const uint32_t lo = ql ? 0x01000504u : 0x05040100u, hi = lo + 0x02020202u;
    return u32x2{__builtin_amdgcn_perm(recv, keep, qh ? hi : lo), __builtin_amdgcn_perm(recv, keep, qh ? lo : hi)};
}
template <int CT>
LSMX_DEV u32x2 quad_pack16(const float (&x)[4], int q) {
    static_assert(CT == LSMX_BF16 || CT == LSMX_F16, "16-bit outputs");
    const uint32_t p0 = CT == LSMX_BF16 ? bf16x2(x[0], x[1]) : f16_bits(x[0]) | (f16_bits(x[1]) << 16);
    const uint32_t p1 = CT == LSMX_BF16 ? bf16x2(x[2], x[3]) : f16_bits(x[2]) | (f16_bits(x[3]) << 16);
    return quad_pack16_bits(p0, p1, q);
}

// Eight consecutive 16-bit columns of one row per lane, from two row groups
// of a 32 x 32 MFMA tile: x0 and x1 are a lane's accumulator values 8p .. 8p+3
// and 8p+4 .. 8p+7, i.e. rows r and r + 8 (r = 16p + 4*half + q) of column
// frow.  After quad_pack16 a lane holds 4 consecutive columns of row r (from
// x0) and of row r + 8 (from x1); lanes 4 apart then trade one of the two,
// so that a lane with (frow & 4) == 0 ends with columns (frow & ~7) .. +8 of
// row r and its partner with the same columns of row r + 8 (odd = (frow & 4)
// != 0).  One 16-byte store per lane then writes 64 contiguous bytes per
// row and 16 rows per instruction, half the instructions of 8-byte stores
// (the output burst at the end of a GEMM tile drains measurably faster).
// pack16_rows8_of takes the two quad_pack16 results.
LSMX_DEV u32x4 pack16_rows8_of(const u32x2 a0, const u32x2 a1, bool odd) {
    const uint32_t s0 = odd ? a0[0] : a1[0], s1 = odd ? a0[1] : a1[1];
    // DPP row_shl:4 reads lane + 4, row_shr:4 lane - 4 (within 16 lanes);
    // each lane uses the one that stays inside its 8-lane group
    const uint32_t l0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s0, 0x104, 0xF, 0xF, true);
    const uint32_t l1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s1, 0x104, 0xF, 0xF, true);
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s0, 0x114, 0xF, 0xF, true);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s1, 0x114, 0xF, 0xF, true);
    return odd ? u32x4{r0, r1, a1[0], a1[1]} : u32x4{a0[0], a0[1], l0, l1};
}
template <int CT>
LSMX_DEV u32x4 pack16_rows8(const float (&x0)[4], const float (&x1)[4], int q, bool odd) {
    return pack16_rows8_of(quad_pack16<CT>(x0, q), quad_pack16<CT>(x1, q), odd);
}

// quad_pack16's row stored at idx: lane q writes M[q][0..3].
template <int CT>
LSMX_DEV void store_c4_quad(void *c, int64_t idx, const float (&x)[4], int q) {
    *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(c) + idx) = quad_pack16<CT>(x, q);
}

template <int N>
LSMX_DEV void wait_vm_barrier() {
    // all of this thread's loads except the newest N have landed, then sync
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace lsmx
