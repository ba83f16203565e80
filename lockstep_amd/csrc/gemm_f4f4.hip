// Block-scaled MXFP4 x MXFP4 GEMM on gfx950's scaled MFMA.
//
//   C[m, n] = sum_kb  2^(sa[m,kb]-127) * 2^(sb[n,kb]-127) * sum_{k in kb} A[m,k] * Bt[n,k]
//
// Semantics: mxfp4_gemm.py:175-233 (_mxfp4_gemm_packed_kernel /
// mxfp4_gemm_packed) and cuda/mxfp4_mma_gemm.cu:69-184, with both operands
// K-contiguous ("TN"), packed two E2M1 codes per byte, low nibble first.
// Instead of promoting an FP8 product to fp32 every 32-block and multiplying
// by fp32 scales, v_mfma_scale_f32_32x32x64_f8f6f4 (cbsz = blgp = 4, FP4)
// applies one E8M0 scale per lane per operand inside the instruction: for
// that instruction each lane supplies the 32 codes (16 bytes) of one row and
// one 32-block, which is exactly one MX block, and the byte of the scale
// register selected by op_sel.
//
// Tiling: 256 x 256 macro tile per workgroup of 4 waves (2 x 2), each wave a
// 128 x 128 sub-tile = 4 x 4 MFMA tiles of 32 x 32 (256 fp32 accumulators per
// lane).  K advances 128 codes (64 bytes per row) per stage; two LDS stages,
// global loads for stage k+1 are issued before the MFMAs of stage k.
#include "lsmx_internal.h"

namespace lsmx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace f4 {
constexpr int BM = 256, BN = 256;
constexpr int BKB = 64;          // bytes of K per row per stage (128 codes, 4 blocks)
constexpr int NT = 256;          // threads
constexpr int WT = 128;          // wave tile edge
constexpr int GROUP_M = 4;
}  // namespace f4

// 16-byte chunk swizzle inside a 64-byte LDS row: keeps the 8 (or 16) lanes
// that a ds_read_b128 / ds_write_b128 serves per cycle on distinct banks.
LSMX_DEV int f4_swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

LSMX_DEV uint32_t bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;  // quiet NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

template <int CT>
LSMX_DEV void store_c(void *c, int64_t idx, float v) {
    if constexpr (CT == LSMX_F32) reinterpret_cast<float *>(c)[idx] = v;
    else if constexpr (CT == LSMX_BF16) reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)bf16_rne(v);
    else reinterpret_cast<_Float16 *>(c)[idx] = (_Float16)v;
}

// Map a linear workgroup id to a (tile_m, tile_n) pair.  Workgroups are
// dispatched round-robin over the 8 XCDs; the remap gives each XCD a run of
// consecutive logical tiles, and GROUP_M-row groups keep the A and B panels
// those tiles share resident in that XCD's L2.
LSMX_DEV void tile_coords(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
    const int per_group = f4::GROUP_M * tiles_n;
    const int group = pid / per_group;
    const int first_m = group * f4::GROUP_M;
    const int gsz = min(tiles_m - first_m, f4::GROUP_M);
    const int in_group = pid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

template <bool SF32>
LSMX_DEV uint32_t load_scale4(const void *s, int64_t off) {
    // 4 consecutive block scales as E8M0 bytes packed little-endian in a u32
    if constexpr (SF32) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(s) + off);
        return ((v[0] >> 23) & 0xFF) | (((v[1] >> 23) & 0xFF) << 8) | (((v[2] >> 23) & 0xFF) << 16) |
               (((v[3] >> 23) & 0xFF) << 24);
    } else {
        return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(s) + off);
    }
}

template <bool SF32, int CT>
__global__ __launch_bounds__(f4::NT, 1) void gemm_f4f4_kernel(GemmArgs g) {
    using namespace f4;
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * BKB];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * BKB];
    __shared__ uint32_t sSA[2][BM];
    __shared__ uint32_t sSB[2][BN];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (int)(g.K / 128);

    // ---- global -> register staging: 4 chunks of A and 4 of B per thread
    const uint8_t *ga[4];
    const uint8_t *gb[4];
    int lds_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = i * NT + t;
        const int row = q >> 2, c = q & 3;
        const int64_t am = min(m0 + row, g.M - 1);  // rows past M re-read row M-1, discarded later
        const int64_t bn = min(n0 + row, g.N - 1);
        ga[i] = g.a + am * g.lda + c * 16;
        gb[i] = g.b + bn * g.ldb + c * 16;
        lds_off[i] = row * BKB + ((c ^ f4_swz(row)) << 4);
    }
    const int64_t sa_row = min(m0 + t, g.M - 1) * g.ld_sa;
    const int64_t sb_row = min(n0 + t, g.N - 1) * g.ld_sb;

    u32x4 ra[4], rb[4];
    uint32_t rsa, rsb;
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] = *reinterpret_cast<const u32x4 *>(ga[i] + (int64_t)kt * BKB);
            rb[i] = *reinterpret_cast<const u32x4 *>(gb[i] + (int64_t)kt * BKB);
        }
        rsa = load_scale4<SF32>(g.sa, sa_row + (int64_t)kt * 4);
        rsb = load_scale4<SF32>(g.sb, sb_row + (int64_t)kt * 4);
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<u32x4 *>(&sA[buf][lds_off[i]]) = ra[i];
            *reinterpret_cast<u32x4 *>(&sB[buf][lds_off[i]]) = rb[i];
        }
        sSA[buf][t] = rsa;
        sSB[buf][t] = rsb;
    };

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int frow = lane & 31, half = lane >> 5;

    gload(0);
    swrite(0);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);

        uint32_t scA[4], scB[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            scA[i] = sSA[buf][wm * WT + i * 32 + frow] >> (8 * half);
            scB[i] = sSB[buf][wn * WT + i * 32 + frow] >> (8 * half);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int c = 2 * s + half;
            v8i fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ra_ = wm * WT + i * 32 + frow;
                const int rb_ = wn * WT + i * 32 + frow;
                const u32x4 va = *reinterpret_cast<const u32x4 *>(&sA[buf][ra_ * BKB + ((c ^ f4_swz(ra_)) << 4)]);
                const u32x4 vb = *reinterpret_cast<const u32x4 *>(&sB[buf][rb_ * BKB + ((c ^ f4_swz(rb_)) << 4)]);
                fa[i] = v8i{(int)va[0], (int)va[1], (int)va[2], (int)va[3], 0, 0, 0, 0};
                fb[i] = v8i{(int)vb[0], (int)vb[1], (int)vb[2], (int)vb[3], 0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (s == 0)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            fa[i], fb[j], acc[i][j], 4, 4, 0, (int)scA[i], 0, (int)scB[j]);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            fa[i], fb[j], acc[i][j], 4, 4, 2, (int)scA[i], 2, (int)scB[j]);
                }
        }
        if (kt + 1 < nk) swrite(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: acc element e of tile (i, j) sits at
    //      row = i*32 + 8*(e/4) + 4*half + e%4,  col = j*32 + frow
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + wn * WT + j * 32 + frow;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t row = m0 + wm * WT + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                if (row < g.M && col < g.N) store_c<CT>(g.c, row * g.ldc + col, acc[i][j][e]);
            }
        }
}

hipError_t launch_gemm_f4f4(const GemmArgs &g, hipStream_t s) {
    const int tiles = (int)(((g.M + f4::BM - 1) / f4::BM) * ((g.N + f4::BN - 1) / f4::BN));
    const dim3 grid(tiles), blk(f4::NT);
    const bool f = g.scale_fmt == LSMX_SCALE_F32;
#define LSMX_G(F, CT) hipLaunchKernelGGL((gemm_f4f4_kernel<F, CT>), grid, blk, 0, s, g)
    if (f) {
        if (g.c_dtype == LSMX_F32) LSMX_G(true, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_G(true, LSMX_BF16);
        else LSMX_G(true, LSMX_F16);
    } else {
        if (g.c_dtype == LSMX_F32) LSMX_G(false, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_G(false, LSMX_BF16);
        else LSMX_G(false, LSMX_F16);
    }
#undef LSMX_G
    return hipGetLastError();
}

}  // namespace lsmx
