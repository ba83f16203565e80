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
// Tiling: 256 x 256 macro tile, WGM x WGN waves (default 4 x 2, two waves per
// SIMD), each wave a (256/WGM) x (256/WGN) sub-tile of 32 x 32 MFMA tiles
// with fp32 accumulators in AGPRs.  K advances 128 codes (64 bytes per row,
// four MX blocks) per stage, two MFMA K-steps of 64.
//
// Persistent schedule: one workgroup per CU walks tiles pid, pid + grid, ...
// A ring of S stage slots in LDS is filled by direct-to-LDS loads
// (global_load_lds_dwordx4 / _dword: lane l's bytes land at M0 + l*size, no
// VGPR staging) and runs across tile boundaries, so the first stages of the
// next tile are already in flight while the current tile finishes and writes
// its output.  The loads come from inline asm with an explicit
// s_waitcnt vmcnt: the compiler cannot prove that ring slots do not alias and
// would otherwise wait for every outstanding load before each LDS read.
//
// Per stage and wave: the step-1 fragments are read while the step-0 MFMAs
// run; one s_barrier (after the stage's own reads completed and the next
// stage's loads landed) frees the slot; then the step-1 MFMAs run with the
// refill of that slot and the next stage's fragment and scale reads
// interleaved one by one between them, so the matrix core never waits on a
// burst of memory instructions.  Refills past the last stage re-load the
// workgroup's last tile (tile indices are clamped, lsmx_sched.h) into a slot
// that is never read again, which keeps the loop free of branches and the
// outstanding-load count constant.
//
// LDS layout per stage: rows of 64 bytes = four 16-byte chunks; chunk c of
// row r lives at r*64 + 16*(c ^ swz(r)), which keeps the lanes a ds_read_b128
// serves per cycle on distinct banks.  The DMA writes slots in lane order, so
// the swizzle is applied by choosing each lane's source address.
#include "lsmx_internal.h"
#include "lsmx_sched.h"

namespace lsmx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace f4 {
constexpr int BM = 256, BN = 256;
constexpr int BKB = 64;           // bytes of K per row per stage (128 codes, 4 blocks)
constexpr int GROUP_M = 4;
constexpr int TILE_B = BM * BKB;  // 16 KiB per operand per stage
}  // namespace f4

LSMX_DEV int f4_swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

LSMX_DEV uint32_t lds_u32(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Direct-to-LDS loads: lane l's bytes land at m0 + l*size.
LSMX_DEV void dma_x4(const void *g, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory");
}
LSMX_DEV void dma_x1(const void *g, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m0) : "memory");
}

LSMX_DEV uint32_t bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;  // quiet NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

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
            u32x2{bf16_rne(v0) | (bf16_rne(v1) << 16), bf16_rne(v2) | (bf16_rne(v3) << 16)};
    } else {
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(c) + idx) =
            u32x2{f16_bits(v0) | (f16_bits(v1) << 16), f16_bits(v2) | (f16_bits(v3) << 16)};
    }
}

// Value held by the lane `D` away inside each quad (D = 1: 1,0,3,2; D = 2: 2,3,0,1).
template <int D>
LSMX_DEV float quad_xor(float v) {
    constexpr int ctrl = D == 1 ? 0xB1 : 0x4E;
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
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

template <int N>
LSMX_DEV void wait_vm_barrier() {
    // all of this thread's loads except the newest N have landed, then sync
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 5) asm volatile("s_waitcnt vmcnt(5)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 10) asm volatile("s_waitcnt vmcnt(10)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 15) asm volatile("s_waitcnt vmcnt(15)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 20) asm volatile("s_waitcnt vmcnt(20)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 30) asm volatile("s_waitcnt vmcnt(30)\n\ts_barrier" ::: "memory");
    else static_assert(N < 0, "unsupported vmcnt");
}

// Scale formats (SFMT = LSMX_SCALE_*): F32 scales arrive as fp32 powers of two
// (16 bytes per row per stage) and are reduced to E8M0 bytes when read; E8M0
// row-major scales take one dword per row per stage at a stride of K/32 bytes;
// K-major E8M0 scales ([K/128][rows][4]) give the dwords of one stage for
// consecutive rows as one contiguous run -- one 64-byte request per 16 rows
// instead of one per row.
template <int SFMT, int CT, int S, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_f4f4_kernel(GemmArgs g) {
    using namespace f4;
    constexpr bool SF32 = SFMT == LSMX_SCALE_F32;
    constexpr bool SKM = SFMT == LSMX_SCALE_E8M0_KMAJOR;
    constexpr int NW = WGM * WGN;
    constexpr int NTH = 64 * NW;
    constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
    constexpr int NMF = TM * TN;               // MFMAs per K-step
    constexpr int SROW = SF32 ? 16 : 4;        // scale bytes per row per stage
    constexpr int XA = (BM * BKB / 16) / NTH;  // 16-byte DMA slots per thread per operand
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    // scale loads: with 4 waves every wave loads 64 rows of A's and of B's
    // scales; with 8 waves waves 0-3 load A's and waves 4-7 load B's.
    constexpr int L = 2 * XA + (NW == 4 ? 2 : 1);  // loads per thread per stage
    constexpr int NRD = TM + TN;                   // fragment reads per K-step
    static_assert(NMF >= L, "one refill op per MFMA at most");
    constexpr int RPM0 = (NRD + NMF - 1) / NMF;      // LDS reads per MFMA, step 0
    constexpr int RPM1 = (2 * NRD + NMF - 1) / NMF;  // LDS reads per MFMA, step 1
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sB[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sSA[S][BM * SROW];
    __shared__ __attribute__((aligned(16))) uint8_t sSB[S][BN * SROW];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nk = (int)(g.K / 128);

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 31, half = lane >> 5;
    const int rowA0 = wm * (TM * 32) + frow, rowB0 = wn * (TN * 32) + frow;

    // ---- DMA source of this thread for stage u (tile u / nk, k-step u % nk)
    int dma_row[XA], dma_c[XA];
#pragma unroll
    for (int i = 0; i < XA; ++i) {
        dma_row[i] = (i * NW + wave) * 16 + (lane >> 2);
        dma_c[i] = ((lane & 3) ^ f4_swz(dma_row[i])) * 16;
    }
    const int srow = (wave & 3) * 64 + lane;
    const bool s_is_b = NW == 8 && wave >= 4;
    const int64_t sbytes = SF32 ? 4 : 1;

    // origin of this workgroup's tile iteration ti (clamped to its real tiles)
    auto tile_of = [&](int ti, int64_t &m0, int64_t &n0) {
        int tm, tn;
        ti = imax(0, imin(ti, my_tiles - 1));
        tile_coords((int)blockIdx.x + ti * (int)gridDim.x, tiles_m, tiles_n, GROUP_M, tm, tn);
        m0 = (int64_t)tm * BM;
        n0 = (int64_t)tn * BN;
    };
    // one memory op (q = 0..L-1) of loading stage (tile origin m0/n0, k-step
    // kt) into ring slot s
    auto issue_op = [&](int64_t m0, int64_t n0, int kt, int s, int q) {
        const int64_t ko = (int64_t)kt * BKB;
        if (q < 2 * XA) {
            const int i = q >> 1;
            if ((q & 1) == 0)
                dma_x4(g.a + min(m0 + dma_row[i], g.M - 1) * g.lda + dma_c[i] + ko,
                       __builtin_amdgcn_readfirstlane(lds_u32(&sA[s][(i * NW + wave) * 1024])));
            else
                dma_x4(g.b + min(n0 + dma_row[i], g.N - 1) * g.ldb + dma_c[i] + ko,
                       __builtin_amdgcn_readfirstlane(lds_u32(&sB[s][(i * NW + wave) * 1024])));
            return;
        }
        const int soff = (wave & 3) * 64 * SROW;
        const bool to_b = NW == 4 ? (q == 2 * XA + 1) : s_is_b;
        const int64_t srow_g = to_b ? min(n0 + srow, g.N - 1) : min(m0 + srow, g.M - 1);
        const int64_t sld = to_b ? g.ld_sb : g.ld_sa;
        // byte offset of this lane's 4 (E8M0) or 16 (F32) scale bytes of stage kt
        const int64_t so = SKM ? ((int64_t)kt * sld + srow_g) * 4 : srow_g * sld * sbytes + (int64_t)kt * SROW;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(to_b ? g.sb : g.sa);
        const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_u32(to_b ? &sSB[s][soff] : &sSA[s][soff]));
        if constexpr (SF32) dma_x4(src + so, dst);
        else dma_x1(src + so, dst);
    };
    auto refill = [&](int u, int s) {  // all ops of stage u (prologue)
        int64_t m0, n0;
        tile_of(stage_tile_iter(u, nk, my_tiles), m0, n0);
#pragma unroll
        for (int q = 0; q < L; ++q) issue_op(m0, n0, u % nk, s, q);
    };

    auto scale_of = [&](const uint8_t *base, int r) -> uint32_t {
        if constexpr (SF32) {
            const u32x4 f = *reinterpret_cast<const u32x4 *>(base + r * 16);
            return ((f[0] >> 23) & 0xFF) | (((f[1] >> 23) & 0xFF) << 8) | (((f[2] >> 23) & 0xFF) << 16) |
                   (((f[3] >> 23) & 0xFF) << 24);
        } else {
            return *reinterpret_cast<const uint32_t *>(base + r * 4);
        }
    };
    // fragment read q (0..NRD-1) of K-step st from slot s: A tiles, then B tiles
    auto read_frag = [&](int s, int st, int q, v8i (&fa)[TM], v8i (&fb)[TN]) {
        const int c = 2 * st + half;
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        const uint8_t *base = q < TM ? sA[s] : sB[s];
        const u32x4 v = *reinterpret_cast<const u32x4 *>(base + r * BKB + ((c ^ f4_swz(r)) << 4));
        const v8i f = v8i{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
        if (q < TM) fa[q] = f;
        else fb[q - TM] = f;
    };
    auto read_scale = [&](int s, int q, uint32_t (&sa)[TM], uint32_t (&sb)[TN]) {
        if (q < TM) sa[q] = scale_of(sSA[s], rowA0 + q * 32) >> (8 * half);
        else sb[q - TM] = scale_of(sSB[s], rowB0 + (q - TM) * 32) >> (8 * half);
    };

    v16f acc[TM][TN];
    uint32_t scA[TM], scB[TN], nA[TM], nB[TN];
    v8i fa0[TM], fb0[TN], fa1[TM], fb1[TN];

    // ---- prologue: fill the ring, publish stage 0, read its step-0 operands
#pragma unroll
    for (int p = 0; p < S; ++p) refill(p, p);
    wait_vm_barrier<(S - 1) * L>();
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_scale(0, q, scA, scB);
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_frag(0, 0, q, fa0, fb0);

    const bool vec_c = ((reinterpret_cast<uintptr_t>(g.c) & 15) == 0) && (g.ldc % 4 == 0);
    // Stage u + S refills slot u % S.  Stages past the last one re-load the
    // workgroup's last tile (tile_of clamps), so the loads stay inside the
    // operands and land in slots that are never read again.
    int rt = S / nk, rk = S % nk;  // tile iteration and k-step of stage u + S
    int u = 0;
    for (int ti = 0; ti < my_tiles; ++ti) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

        for (int kt = 0; kt < nk; ++kt, ++u) {
            const int s = u % S;
            const int sn = (u + 1) % S;
            int64_t rm0, rn0;
            tile_of(rt, rm0, rn0);
            // step 0: MFMAs, with the step-1 fragment reads of this stage in between
#pragma unroll
            for (int idx = 0; idx < NMF; ++idx) {
                const int i = idx / TN, j = idx % TN;
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    fa0[i], fb0[j], acc[i][j], 4, 4, 0, (int)scA[i], 0, (int)scB[j]);
#pragma unroll
                for (int r = idx * RPM0; r < (idx + 1) * RPM0; ++r)
                    if (r < NRD) read_frag(s, 1, r, fa1, fb1);
                __builtin_amdgcn_sched_barrier(0);
            }
            // this wave's reads of slot s are complete; once all waves pass the
            // barrier slot s is free and stage u+1 has landed
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            wait_vm_barrier<(S - 2) * L>();
            __builtin_amdgcn_sched_barrier(0);
            // step 1: MFMAs, with the refill of slot s and the next stage's
            // scale and step-0 fragment reads in between
#pragma unroll
            for (int idx = 0; idx < NMF; ++idx) {
                const int i = idx / TN, j = idx % TN;
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    fa1[i], fb1[j], acc[i][j], 4, 4, 2, (int)scA[i], 2, (int)scB[j]);
                if (idx < L) issue_op(rm0, rn0, rk, s, idx);
#pragma unroll
                for (int r = idx * RPM1; r < (idx + 1) * RPM1; ++r) {
                    if (r < NRD) read_scale(sn, r, nA, nB);
                    else if (r < 2 * NRD) read_frag(sn, 0, r - NRD, fa0, fb0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) scA[i] = nA[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) scB[j] = nB[j];
            const bool wrap = rk + 1 == nk;
            rk = wrap ? 0 : rk + 1;
            rt += wrap ? 1 : 0;
        }

        // ---- epilogue of tile ti.  acc element e of tile (i, j) sits at
        //      row = i*32 + 8*(e/4) + 4*half + e%4,  col = j*32 + frow;
        //      a 4x4 transpose inside each quad of lanes gives every lane 4
        //      consecutive columns of one row.
        int64_t m0, n0;
        tile_of(ti, m0, n0);
        const int q = frow & 3;
        const bool full = vec_c && m0 + BM <= g.M && n0 + BN <= g.N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    float x[4] = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                  acc[i][j][4 * gq + 3]};
                    quad_transpose(x, q);
                    const int64_t row = m0 + wm * (TM * 32) + i * 32 + 8 * gq + 4 * half + q;
                    const int64_t col = n0 + wn * (TN * 32) + j * 32 + (frow & ~3);
                    if (full) {
                        store_c4<CT>(g.c, row * g.ldc + col, x[0], x[1], x[2], x[3]);
                    } else if (row < g.M) {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (col + c < g.N) store_c<CT>(g.c, row * g.ldc + col + c, x[c]);
                    }
                }
    }
    // no load may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

#ifndef LSMX_F4_STAGES
#define LSMX_F4_STAGES 4
#endif
// Default: 8 waves in a 4 x 2 grid (64 x 128 per wave), two waves per SIMD,
// so one wave's MFMAs keep the matrix core busy while the other is held by
// load back-pressure or the stage barrier (measured 8192^3: 2 x 2 waves
// 487 us, 4 x 2 waves 395 us).
#ifndef LSMX_F4_WGM
#define LSMX_F4_WGM 4
#endif
#ifndef LSMX_F4_WGN
#define LSMX_F4_WGN 2
#endif

static int num_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

hipError_t launch_gemm_f4f4(const GemmArgs &g, hipStream_t s) {
    constexpr int W = LSMX_F4_WGM, Z = LSMX_F4_WGN, SE = LSMX_F4_STAGES;
    const int tiles = (int)(((g.M + f4::BM - 1) / f4::BM) * ((g.N + f4::BN - 1) / f4::BN));
    const int grid = tiles < num_cus() ? tiles : num_cus();
    const dim3 blk(64 * W * Z);
#define LSMX_G(F, CT, S) hipLaunchKernelGGL((gemm_f4f4_kernel<F, CT, S, W, Z>), dim3(grid), blk, 0, s, g)
#define LSMX_GC(F, S)                                             \
    do {                                                          \
        if (g.c_dtype == LSMX_F32) LSMX_G(F, LSMX_F32, S);        \
        else if (g.c_dtype == LSMX_BF16) LSMX_G(F, LSMX_BF16, S); \
        else LSMX_G(F, LSMX_F16, S);                              \
    } while (0)
    if (g.scale_fmt == LSMX_SCALE_F32) LSMX_GC(LSMX_SCALE_F32, 3);  // 16-byte scale rows: one stage less
    else if (g.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) LSMX_GC(LSMX_SCALE_E8M0_KMAJOR, SE);
    else LSMX_GC(LSMX_SCALE_E8M0, SE);
#undef LSMX_GC
#undef LSMX_G
    return hipGetLastError();
}

}  // namespace lsmx
