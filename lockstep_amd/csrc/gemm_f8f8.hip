// Block-scaled E4M3 x E4M3 GEMM (the reference's mxfp4_gemm_fp8) on gfx950's
// scaled MFMA, built like the f4 x f4 kernel:
//
//   C[m, n] = sum_kb 2^(sa[m,kb]-127) * 2^(sb[n,kb]-127) * sum_{k in kb} A[m,k] * Bt[n,k]
//
// Semantics: mxfp4_gemm.py:29-87 (_mxfp4_gemm_fp8_kernel / mxfp4_gemm_fp8),
// with both operands K-contiguous E4M3 bytes and E8M0 block scales in the
// K-major layout [K/128][rows][4].  v_mfma_scale_f32_32x32x64_f8f6f4 with
// cbsz = blgp = 0 (E4M3) applies the scales inside the instruction.  Its
// 8-bit operand order (pinned on the hardware): VGPRs 0-3 of lane half h hold
// K 16h .. 16h+15 of the instruction's 32-block 0, VGPRs 4-7 hold
// K 32+16h .. of block 1, and lane half h supplies the scale of block h.
//
// Tiling: 256 x 256 per workgroup of 4 waves (2 x 2, 128 x 128 per wave, 16
// MFMA tiles with AGPR accumulators, one wave per SIMD).  A stage is 128
// bytes of every row (128 K, two MFMA K-steps, one K-major scale dword per
// row); two 64 KiB stage slots in LDS are filled by direct-to-LDS loads and
// the ring runs across tile boundaries of a persistent schedule.  K-step 0
// reads K-step 1's fragments; after one s_barrier at K-step 1 the slot is
// free, and its refill, the next stage's scales and its K-step-0 fragments
// are interleaved with K-step 1's MFMAs.
#include "lsmx_dma.h"
#include "lsmx_store.h"
#include "lsmx_internal.h"
#include "lsmx_sched.h"

namespace lsmx {

namespace f8 {
constexpr int BM = 256, BN = 256;
constexpr int WGM = 2, WGN = 2, NW = WGM * WGN, NT = 64 * NW;
constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;   // 4 x 4 tiles of 32 x 32 per wave
constexpr int NMF = TM * TN;
constexpr int BKB = 128;                  // bytes = E4M3 elements of K per row per stage
constexpr int CPR = BKB / 16;             // 16-byte chunks per row
constexpr int RPI = 64 / CPR;             // rows per load instruction
constexpr int TILE_B = BM * BKB;          // 32 KiB per operand per stage
constexpr int S = 2;                      // stage slots
constexpr int XA = TILE_B / 16 / NT;      // data loads per thread per operand per stage
constexpr int L = 2 * XA + 2;             // + one scale load each for A and B
constexpr int NRD = TM + TN;              // fragment (and scale) reads per K-step
constexpr int OPM = (L + NMF - 1) / NMF;  // refill loads per MFMA in K-step 1
constexpr int GROUP_M = 4;
LSMX_DEV int swz(int row) { return (row >> 1) & 7; }
}  // namespace f8

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f8 __attribute__((ext_vector_type(16)));

// The scaled MFMA through its LLVM intrinsic (v8i32 operands): op_sel then
// only has to be a constant after unrolling, as for the f4 x f4 kernel.
__device__ v16f8 mfma_scale_f8(v8i a, v8i b, v16f8 c, int cbsz, int blgp, int opsel_a, int scale_a, int opsel_b,
                               int scale_b) __asm("llvm.amdgcn.mfma.scale.f32.32x32x64.f8f6f4.v8i32.v8i32");

// Eight E4M3 values of one column from a [K][N] LDS tile with
// ds_read_b64_tr_b8: within each 16-lane group, lanes 2m and 2m + 1 give the
// addresses of 8 consecutive bytes each of row m (16 columns), and lane j
// receives column j of the group's 8 x 16 block, row m as its byte m (the
// lane layout was checked on the device with an in-bounds probe).
typedef int v2i_f8 __attribute__((ext_vector_type(2)));
LSMX_DEV v2i_f8 ds_read_tr8x8(const uint8_t *p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i_f8 *)(p));
}

// BNC: B arrives as the reference passes it, [K, N] E4M3 with N contiguous
// (row stride ldb bytes).  A stage of B is then 128 K-rows of 256 bytes; a
// DMA instruction carries 4 rows, LDS chunk p of row r holding source chunk
// p ^ 2 (r & 7) (the 8 rows a half-wave reads at once cover the 256-byte bank
// span), and each B fragment is four transposing reads of 8 K values.
template <int CT, bool BNC = false>
__global__ __launch_bounds__(f8::NT, 1) void gemm_f8f8_kernel(DenseArgs g) {
    using namespace f8;
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sB[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sSA[S][BM * 4];
    __shared__ __attribute__((aligned(16))) uint8_t sSB[S][BN * 4];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nk = (int)(g.K / BKB);

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 31, half = lane >> 5;
    const int rowA0 = wm * (TM * 32) + frow, rowB0 = wn * (TN * 32) + frow;

    // ---- load addressing: data load i of this lane reads row
    // (i*NW + wave)*RPI + lane/CPR of the refill tile, LDS chunk lane%CPR
    // holding source chunk (lane%CPR) ^ swz(row), so the byte offset is
    // off0 + i*step.  Descriptors end at the operand's last row.
    const int drow0 = wave * RPI + lane / CPR;
    const uint32_t offA0 = (uint32_t)(drow0 * g.lda + (((lane % CPR) ^ swz(drow0)) << 4));
    // BNC: load i of this lane reads K-row 4 (i*NW + wave) + lane/16 of the
    // stage, chunk (lane % 16) ^ 2 (row & 7) (row & 7 does not depend on i)
    const int brow0 = 4 * wave + (lane >> 4);
    const uint32_t offB0 = BNC ? (uint32_t)(brow0 * g.ldb + (((lane & 15) ^ (2 * (brow0 & 7))) << 4))
                               : (uint32_t)(drow0 * g.ldb + (((lane % CPR) ^ swz(drow0)) << 4));
    const uint32_t stepA = (uint32_t)(NW * RPI * g.lda);
    const uint32_t stepB = BNC ? (uint32_t)(4 * NW * g.ldb) : (uint32_t)(NW * RPI * g.ldb);
    // scales: every wave loads 64 rows of A's and of B's dwords per stage
    const uint32_t offS = (uint32_t)((wave * 64 + lane) * 4);
    const uint64_t sbytes_a = (uint64_t)(((g.K / 128 - 1) * g.ld_sa + g.M) * 4);
    const uint64_t sbytes_b = (uint64_t)(((g.K / 128 - 1) * g.ld_sb + g.N) * 4);

    int64_t rm0 = 0, rn0 = 0;   // origin of the refill tile
    const TileMap tmap = make_tile_map(tiles_m, tiles_n, GROUP_M);
    auto tile_of = [&](int ti, int64_t &m0, int64_t &n0) __attribute__((always_inline)) {
        int tm, tn;
        ti = imax(0, imin(ti, my_tiles - 1));
        tile_coords((int)blockIdx.x + ti * (int)gridDim.x, tmap, tm, tn);
        m0 = (int64_t)tm * BM;
        n0 = (int64_t)tn * BN;
    };
    auto set_refill_tile = [&](int ti) __attribute__((always_inline)) { tile_of(ti, rm0, rn0); };
    // buffer descriptors of k-step kt of the refill tile, in three parts.
    // 32-bit factors (the host bounds M, N and the leading dimensions below
    // 2^31 and a 256-row panel below 2^31 bytes), so every product is one
    // 32 x 32 -> 64-bit multiply.
    const uint32_t M32 = (uint32_t)g.M, N32 = (uint32_t)g.N;
    const uint32_t lda32 = (uint32_t)g.lda, ldb32 = (uint32_t)g.ldb;
    const uint32_t ldsa32 = (uint32_t)g.ld_sa, ldsb32 = (uint32_t)g.ld_sb;
    v4i_rsrc rsA, rsB, rsSA, rsSB;
    auto make_desc = [&](int part, int kt) __attribute__((always_inline)) {
        const uint32_t ko = (uint32_t)kt * BKB;
        if (part == 0) {
            const uint32_t m0 = (uint32_t)rm0, rows = min(M32 - m0, (uint32_t)BM);
            rsA = buf_rsrc(g.a0 + (uint64_t)m0 * lda32 + ko, rows * lda32 - ko);
        } else if (part == 1) {
            if constexpr (BNC) {
                // 128 K-rows per stage; the range ends at the last column of
                // the last K-row (columns past N in other rows read the next
                // row's values, whose products reach no stored output)
                const uint64_t kr = (uint64_t)kt * BKB * (uint64_t)g.ldb;
                rsB = buf_rsrc(g.b0 + (uint64_t)rn0 + kr, (uint64_t)(g.K - 1) * (uint64_t)g.ldb +
                                                                (uint64_t)(g.N - rn0) - kr);
            } else {
                const uint32_t n0 = (uint32_t)rn0, rows = min(N32 - n0, (uint32_t)BN);
                rsB = buf_rsrc(g.b0 + (uint64_t)n0 * ldb32 + ko, rows * ldb32 - ko);
            }
        } else {
            // K-major scale slice kt: rows past the operand read later slices
            // or zeros; their products only reach outputs that are not stored
            const uint64_t oa = ((uint64_t)kt * ldsa32 + (uint32_t)rm0) * 4;
            const uint64_t ob = ((uint64_t)kt * ldsb32 + (uint32_t)rn0) * 4;
            rsSA = buf_rsrc(g.sa + oa, sbytes_a - oa);
            rsSB = buf_rsrc(g.sb + ob, sbytes_b - ob);
        }
    };
    // one memory op (q = 0..L-1) of loading the refill stage into slot s
    auto issue_op = [&](int s, int q) __attribute__((always_inline)) {
        if (q < 2 * XA) {
            const int i = q >> 1;
            const uint32_t m0 = lds_u32((q & 1) ? &sB[0][0] : &sA[0][0]) + s * TILE_B + (i * NW + wave) * 1024;
            if ((q & 1) == 0) dma_x4(offA0 + i * stepA, rsA, m0);
            else dma_x4(offB0 + i * stepB, rsB, m0);
            return;
        }
        const bool to_b = q == 2 * XA + 1;
        dma_x1(offS, to_b ? rsSB : rsSA, lds_u32(to_b ? &sSB[s][wave * 256] : &sSA[s][wave * 256]));
    };

    // K-step st: lane half h supplies chunks 4st + h (block 0 part) and
    // 4st + 2 + h (block 1 part) of its row
    // BNC fragment reads: lane (group g = lane/16, j = lane % 16) of B tile
    // jt reads rows k0 + j/2 (k0 = 64 st + 16 half + {0, 8, 32, 40}: the
    // K-contiguous fragment's two 16-byte pieces) and the 8 bytes 8 (j & 1) of
    // column chunk wn*8 + jt*2 + (g & 1), which the row swizzle 2 (j/2) moves
    // to 2 ((wn*4 + jt) ^ j/2) + (g & 1); one offset per jt, the rest immediates
    const int bj8 = lane & 15, brs8 = bj8 >> 1;
    uint32_t bfo[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
        bfo[j] = (uint32_t)(half * (16 * 256) + brs8 * 256 + ((2 * ((wn * 4 + j) ^ brs8) + ((lane >> 4) & 1)) << 4) +
                            8 * (bj8 & 1));
    auto read_frag = [&](int s, int st, int q, v8i (&fa)[TM], v8i (&fb)[TN]) __attribute__((always_inline)) {
        if constexpr (BNC) {
            if (q >= TM) {
                const uint8_t *p = sB[s] + bfo[q - TM] + st * (64 * 256);
                const v2i_f8 r0 = ds_read_tr8x8(p), r1 = ds_read_tr8x8(p + 8 * 256);
                const v2i_f8 r2 = ds_read_tr8x8(p + 32 * 256), r3 = ds_read_tr8x8(p + 40 * 256);
                fb[q - TM] = v8i{r0.x, r0.y, r1.x, r1.y, r2.x, r2.y, r3.x, r3.y};
                return;
            }
        }
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        const uint8_t *base = (q < TM ? sA[s] : sB[s]) + r * BKB;
        const u32x4 lo = *reinterpret_cast<const u32x4 *>(base + (((4 * st + half) ^ swz(r)) << 4));
        const u32x4 hi = *reinterpret_cast<const u32x4 *>(base + (((4 * st + 2 + half) ^ swz(r)) << 4));
        const v8i f = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        if (q < TM) fa[q] = f;
        else fb[q - TM] = f;
    };
    // the stage's scale dword of fragment row q, shifted so that op_sel = 2*st
    // picks block 2*st + h for lane half h
    auto read_scale = [&](int s, int q, uint32_t (&sa)[TM], uint32_t (&sb)[TN]) __attribute__((always_inline)) {
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        const uint32_t v = *reinterpret_cast<const uint32_t *>((q < TM ? sSA[s] : sSB[s]) + r * 4) >> (8 * half);
        if (q < TM) sa[q] = v;
        else sb[q - TM] = v;
    };

    v16f8 acc[TM][TN];
    uint32_t scA[TM], scB[TN];
    v8i fa[2][TM], fb[2][TN];

    // ---- prologue: fill the ring, publish stage 0, read its step-0 operands
    {
        int cur = -1;
#pragma unroll
        for (int p = 0; p < S; ++p) {
            const int ti = stage_tile_iter(p, nk, my_tiles);
            if (ti != cur) {
                set_refill_tile(ti);
                cur = ti;
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) make_desc(c, p % nk);
#pragma unroll
            for (int q = 0; q < L; ++q) issue_op(p, q);
        }
    }
    wait_vm_barrier<(S - 1) * L>();
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_scale(0, q, scA, scB);
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_frag(0, 0, q, fa[0], fb[0]);

    const bool vec_c = ((reinterpret_cast<uintptr_t>(g.c0) & 15) == 0) && (g.ldc % 4 == 0);
    // Stage u + S refills slot u % S.  Stage kt of tile iteration ti
    // refills k-step kt + ra of tile ti + qa while kt + ra < nk and k-step
    // kt + ra - nk of tile ti + qa + 1 after, with qa = S / nk and
    // ra = S % nk; both tiles' coordinates are found once per tile, and each
    // stage only selects between them.  Stages past the last one re-load the
    // workgroup's last tile (tile coordinates are clamped): the loads stay
    // inside the operands and land in slots that are never read again.
    const int qa = S / nk, ra = S % nk;
    int u = 0;
    for (int ti = 0; ti < my_tiles; ++ti) {
        int tma, tna, tmb, tnb;
        tile_coords((int)blockIdx.x + imin(ti + qa, my_tiles - 1) * (int)gridDim.x, tmap, tma, tna);
        tile_coords((int)blockIdx.x + imin(ti + qa + 1, my_tiles - 1) * (int)gridDim.x, tmap, tmb, tnb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

        for (int kt = 0; kt < nk; ++kt, ++u) {
            const int s = u % S;
            const int sn = (u + 1) % S;
            const bool pb = kt + ra >= nk;
            const int rk = pb ? kt + ra - nk : kt + ra;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                if (st == 1) {
                    // this wave's reads of slot s are complete; once all waves
                    // pass the barrier slot s is free and stage u+1 has landed
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    wait_vm_barrier<(S - 2) * L>();
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int idx = 0; idx < NMF; ++idx) {
                    const int i = idx / TN, j = idx % TN;
                    acc[i][j] = mfma_scale_f8(fa[st][i], fb[st][j], acc[i][j], 0, 0, 2 * st, (int)scA[i], 2 * st,
                                              (int)scB[j]);
                    if (st == 0) {
                        // descriptors of the refill stage, one part after each
                        // of the first MFMAs so that their scalar arithmetic
                        // overlaps the matrix core; the empty asm passes rk
                        // through an SGPR so that the IR optimizer cannot
                        // hoist a part above the fence in front of it
                        if (idx < 3) {
                            __builtin_amdgcn_sched_barrier(0);
                            int k = rk;
                            asm volatile("" : "+s"(k));
                            if (idx == 0) {
                                rm0 = (int64_t)(pb ? tmb : tma) * BM;
                                rn0 = (int64_t)(pb ? tnb : tna) * BN;
                            }
                            make_desc(idx, k);
                        }
                        if (idx < NRD) read_frag(s, 1, idx, fa[1], fb[1]);
                    } else {
#pragma unroll
                        for (int o = idx * OPM; o < (idx + 1) * OPM; ++o)
                            if (o < L) issue_op(s, o);
                        if (idx < NRD) read_frag(sn, 0, idx, fa[0], fb[0]);
                        // the next stage's scales go straight into the registers
                        // whose last MFMA has just issued: scA[i] after MFMA
                        // (i, TN-1), scB[j] after MFMA (TM-1, j)
                        if (idx % TN == TN - 1) read_scale(sn, idx / TN, scA, scB);
                        if (idx >= (TM - 1) * TN) read_scale(sn, TM + idx - (TM - 1) * TN, scA, scB);
                    }
                    // keep this K-step's LDS reads here (the MFMA is a pure
                    // intrinsic: without a memory clobber the compiler may
                    // hoist later reads and keep all fragments live at once)
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }

        // ---- epilogue of tile ti: a 4x4 transpose inside each quad of lanes
        //      gives every lane 4 consecutive columns of one row
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
                    const int64_t row = m0 + wm * (TM * 32) + i * 32 + 8 * gq + 4 * half + q;
                    const int64_t col = n0 + wn * (TN * 32) + j * 32 + (frow & ~3);
                    if (full) {
                        // the fp32 transpose: the packed one (store_c4_quad)
                        // needs more registers than this kernel has left
                        quad_transpose(x, q);
                        store_c4<CT>(g.c0, row * g.ldc + col, x[0], x[1], x[2], x[3]);
                    } else {
                        // all four lanes of a quad take part in the
                        // exchanges, so the row test comes after them
                        quad_transpose(x, q);
                        if (row < g.M)
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                if (col + c < g.N) store_c<CT>(g.c0, row * g.ldc + col + c, x[c]);
                    }
                }
        // the next stage's scales and K-step-0 fragments (slot u % S landed at
        // the last barrier), read again here so that the epilogue does not
        // keep the copies read during the last K-step live
#pragma unroll
        for (int q = 0; q < NRD; ++q) read_scale(u % S, q, scA, scB);
#pragma unroll
        for (int q = 0; q < NRD; ++q) read_frag(u % S, 0, q, fa[0], fb[0]);
    }
    // no load may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

static int num_cus_f8() {
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

hipError_t launch_gemm_f8f8_kmajor(const DenseArgs &g, hipStream_t s) {
    const int tiles = (int)(((g.M + f8::BM - 1) / f8::BM) * ((g.N + f8::BN - 1) / f8::BN));
    const int grid = tiles < num_cus_f8() ? tiles : num_cus_f8();
    const dim3 blk(f8::NT);
#define LSMX_F8(CT)                                                                                   \
    do {                                                                                          \
        if (g.b_nc) hipLaunchKernelGGL((gemm_f8f8_kernel<CT, true>), dim3(grid), blk, 0, s, g);    \
        else hipLaunchKernelGGL((gemm_f8f8_kernel<CT, false>), dim3(grid), blk, 0, s, g);          \
    } while (0)
    if (g.c_dtype == LSMX_F32) LSMX_F8(LSMX_F32);
    else if (g.c_dtype == LSMX_BF16) LSMX_F8(LSMX_BF16);
    else LSMX_F8(LSMX_F16);
#undef LSMX_F8
    return hipGetLastError();
}

}  // namespace lsmx
