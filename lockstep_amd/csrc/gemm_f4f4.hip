// Block-scaled MXFP4 x MXFP4 GEMM on gfx950's scaled MFMA.
//
//   C[m, n] = sum_kb  2^(sa[m,kb]-127) * 2^(sb[n,kb]-127) * sum_{k in kb} A[m,k] * Bt[n,k]
//
// Semantics: mxfp4_gemm.py:116-174 (_mxfp4_gemm_packed_kernel /
// mxfp4_gemm_packed) and cuda/mxfp4_mma_gemm.cu:69-184, with both operands
// K-contiguous ("TN"), packed two E2M1 codes per byte, low nibble first.
// Instead of promoting an FP8 product to fp32 every 32-block and multiplying
// by fp32 scales, the scaled MFMAs (v_mfma_scale_f32_{32x32x64,16x16x128}_
// f8f6f4, cbsz = blgp = 4: FP4) apply one E8M0 scale per lane per operand
// inside the instruction: each lane supplies the 32 codes (16 bytes, four
// VGPRs) of one row and one 32-block, which is exactly one MX block, and the
// byte of its scale register selected by op_sel.
//
// Two kernels share one design: a 256 x 256 macro tile per workgroup of 8
// waves (4 x 2, each 64 x 128, two waves per SIMD) with fp32 accumulators;
// a persistent schedule, one workgroup per CU walking tiles pid, pid + grid,
// ...; and a ring of LDS stage slots filled by direct-to-LDS loads
// (buffer_load_dwordx4 ... lds: lane l's bytes land at M0 + 16 l, no VGPR
// staging) that runs across tile boundaries, so the first stages of the next
// tile are in flight while the current tile finishes and writes its output.
// The loads come from inline asm with an explicit s_waitcnt vmcnt: the
// compiler cannot prove that ring slots do not alias and would otherwise
// wait for every outstanding load before each LDS read.
//
//  * gemm_f4f4_mx16_kernel (K-major E8M0 scales, K % 256 == 0; the fast
//    path): v_mfma_scale_f32_16x16x128_f8f6f4 on 128-byte stage rows in a
//    2-slot ring of 64 KiB stages.  Whole 128-byte rows matter: the
//    direct-to-LDS path is limited by the number of L2 requests (measured:
//    19 B/clk per CU for 16 rows x 64 B per load instruction, 36 B/clk for
//    8 rows x 128 B).
//  * gemm_f4f4_kernel (fp32 or row-major E8M0 scales, or K % 256 != 0):
//    v_mfma_scale_f32_32x32x64_f8f6f4 on 64-byte stage rows in a 3- or
//    4-slot ring.
//
// Per stage and wave the MFMAs of one K-step run while the fragments of the
// next are read from LDS between them.  Once the slot has been read, one
// s_barrier (after the stage's own reads completed and the next stage's
// loads landed) frees it; the remaining MFMAs then run with the refill of
// that slot and the next stage's scale and first fragment reads
// interleaved, so the matrix core never waits on a burst of memory
// instructions.  Refills past the last stage re-load the workgroup's last
// tile (tile indices are clamped, lsmx_sched.h) into a slot that is never
// read again, which keeps the loop free of branches and the
// outstanding-load count constant.
//
// Only waves 0-3 issue the refill loads.  The two waves of a SIMD share its
// matrix core; the older one (0-3) wins issue arbitration and reaches the
// stage barrier first, so the younger one's instruction stream sets the pace
// and is kept to MFMAs and LDS reads.  The refill tile changes only in the
// last S stages of a tile, so each tile runs two stage loops ("phases") and
// the refill panels are computed between them, not per stage.
//
// LDS layout per stage: rows of 16*CPR bytes (CPR 16-byte chunks); chunk c
// of row r lives at r*16*CPR + 16*(c ^ swz(r)), which keeps the lanes a
// ds_read_b128 serves per cycle on distinct banks.  The DMA writes slots in
// lane order, so the swizzle is applied by choosing each lane's source
// address.
#include "lsmx_dma.h"
#include "lsmx_q16.h"
#include "lsmx_store.h"
#include "lsmx_internal.h"
#include "lsmx_sched.h"

namespace lsmx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The scaled MFMA with 4-VGPR operands: the FP4 form reads only 16 bytes per
// lane, and the v8i32 form of the clang builtin would hold four zero VGPRs
// per fragment.  The LLVM intrinsic is overloaded on the operand width.
__device__ v16f mfma_scale_f4(v4i a, v4i b, v16f c, int cbsz, int blgp, int opsel_a, int scale_a, int opsel_b,
                              int scale_b) __asm("llvm.amdgcn.mfma.scale.f32.32x32x64.f8f6f4.v4i32.v4i32");

// The stage barrier.  A loader wave first waits until all but its newest N
// direct-to-LDS loads have landed; the barrier then publishes every loader's
// data.  The other waves issue no loads, so they go straight to the barrier:
// their only vector-memory operations are the previous tile's C stores,
// which then stay in flight across the next tile's stages instead of
// holding the wave (vmcnt counts stores too).
template <bool LOADER, int N>
LSMX_DEV void stage_barrier() {
    if constexpr (LOADER) wait_vm_barrier<N>();
    else asm volatile("s_barrier" ::: "memory");
}

namespace f4 {
constexpr int BM = 256, BN = 256;
constexpr int GROUP_M = 4;
}  // namespace f4

// swizzle of 16-byte chunk positions in a row of CPR chunks
template <int CPR>
LSMX_DEV int f4_swz(int row) {
    if constexpr (CPR == 4) return ((row >> 1) ^ (row >> 3)) & 3;
    else return (row >> 1) & 7;
}

// Scale formats (SFMT = LSMX_SCALE_*): F32 scales arrive as fp32 powers of two
// (16 bytes per row per 128 codes) and are reduced to E8M0 bytes when read;
// E8M0 row-major scales take one dword per row per 128 codes at a stride of
// K/32 bytes; K-major E8M0 scales ([K/128][rows][4]) give the dwords of one
// 128-code slice for consecutive rows as one contiguous run -- one 64-byte
// request per 16 rows instead of one per row.
template <int SFMT, int S, int CT>
__global__ __launch_bounds__(512, 1) void gemm_f4f4_kernel(GemmArgs g) {
    using namespace f4;
    constexpr int WGM = 4, WGN = 2;            // waves: 64 x 128 each, two per SIMD
    constexpr int KS = 2;                      // MFMA K-steps per stage (64-byte rows)
    constexpr bool SF32 = SFMT == LSMX_SCALE_F32;
    constexpr bool SKM = SFMT == LSMX_SCALE_E8M0_KMAJOR;
    constexpr int NW = WGM * WGN;
    constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
    constexpr int NMF = TM * TN;               // MFMAs per K-step
    constexpr int BKB = 32 * KS;               // bytes of K per row per stage
    constexpr int CPR = BKB / 16;              // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;              // rows per DMA instruction
    constexpr int TILE_B = BM * BKB;           // bytes per operand per stage
    constexpr int NSL = KS / 2;                // 128-code scale slices per stage
    constexpr int SSL = SF32 ? 16 : 4;         // scale bytes per row per slice
    // The ring's loads are issued by waves 0-3 only ("loader waves").  With
    // 8 waves the other four run nothing but MFMAs and LDS reads: the two
    // waves of a SIMD share its matrix core, the older one (0-3) wins issue
    // arbitration and then waits at the stage barrier for the younger one,
    // so the younger one's instruction stream sets the pace and is kept
    // short.
    constexpr int NLW = 4;
    constexpr int XA = (TILE_B / 16) / (64 * NLW);  // 16-byte DMA slots per loader lane per operand
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    // scale loads: every loader wave loads 64 rows of A's and of B's scales
    constexpr int LS = 2 * NSL;
    constexpr int L = 2 * XA + LS;                   // loads per thread per stage
    constexpr int NRD = TM + TN;                     // fragment (and scale) reads per K-step / stage
    constexpr int OPM = (L + NMF - 1) / NMF;         // refill ops per MFMA, last K-step
    constexpr int RPM0 = (NRD + NMF - 1) / NMF;      // LDS reads per MFMA, other K-steps
    constexpr int RPM1 = (2 * NRD + NMF - 1) / NMF;  // LDS reads per MFMA, last K-step
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sB[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sSA[S][NSL][BM * SSL];
    __shared__ __attribute__((aligned(16))) uint8_t sSB[S][NSL][BN * SSL];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nk = (int)(g.K / (2 * BKB));

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: LDS bases stay scalar
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 31, half = lane >> 5;
    const int rowA0 = wm * (TM * 32) + frow, rowB0 = wn * (TN * 32) + frow;

    // ---- DMA addressing (loader waves).  Data load i of this lane reads row
    // (i*NLW + wave)*RPI + lane/CPR of the refill tile; the chunk swizzle of
    // those rows does not depend on i, so the byte offset is off0 + i*step.
    // Descriptors start at the refill tile's first row and K offset and end
    // at the operand's last row: rows past it read zeros.
    const int drow0 = wave * RPI + lane / CPR;
    const uint32_t offA0 = (uint32_t)(drow0 * g.lda + ((lane % CPR) ^ f4_swz<CPR>(drow0)) * 16);
    const uint32_t offB0 = (uint32_t)(drow0 * g.ldb + ((lane % CPR) ^ f4_swz<CPR>(drow0)) * 16);
    const uint32_t stepA = (uint32_t)(NLW * RPI * g.lda), stepB = (uint32_t)(NLW * RPI * g.ldb);
    const int srow = (wave & 3) * 64 + lane;
    // scale arrays: total bytes, and this lane's row offset inside a slice
    const uint64_t sbytes_a = SKM ? ((g.K / 128 - 1) * g.ld_sa + g.M) * 4
                                  : ((g.M - 1) * g.ld_sa + g.K / 32) * (SF32 ? 4 : 1);
    const uint64_t sbytes_b = SKM ? ((g.K / 128 - 1) * g.ld_sb + g.N) * 4
                                  : ((g.N - 1) * g.ld_sb + g.K / 32) * (SF32 ? 4 : 1);
    const uint32_t offSA = (uint32_t)(SKM ? srow * 4 : SF32 ? srow * g.ld_sa * 4 : srow * g.ld_sa);
    const uint32_t offSB = (uint32_t)(SKM ? srow * 4 : SF32 ? srow * g.ld_sb * 4 : srow * g.ld_sb);
    int64_t rm0 = 0, rn0 = 0;  // origin of the refill tile
    static_assert(GROUP_M <= 4, "tile_coords divides by group heights up to 4");
    const TileMap tmap = make_tile_map(tiles_m, tiles_n, GROUP_M);
    auto tile_of = [&](int ti, int64_t &m0, int64_t &n0) {
        int tm, tn;
        ti = imax(0, imin(ti, my_tiles - 1));
        tile_coords((int)blockIdx.x + ti * (int)gridDim.x, tmap, tm, tn);
        m0 = (int64_t)tm * BM;
        n0 = (int64_t)tn * BN;
    };
    // Refill panels: first byte and byte count, at k-step 0 of the refill
    // tile, of its A and B code rows and of the scale slices this wave loads,
    // and the scale bytes one stage advances.  Wave-uniform; recomputed only
    // when the refill target moves on to the next tile.
    constexpr int NSD = LS;  // scale descriptors per stage
    struct Panel {
        const uint8_t *p;
        int64_t n;
    };
    Panel pA, pB, pS[NSD];
    int64_t sstep[NSD];
#pragma unroll
    for (int r = 0; r < NSD; ++r) {
        const bool to_b = r & 1;
        const int64_t sld = to_b ? g.ld_sb : g.ld_sa;
        sstep[r] = SKM ? NSL * sld * 4 : SF32 ? NSL * 16 : NSL * 4;
    }
    auto set_refill_origin = [&](int64_t m0, int64_t n0) {
        rm0 = m0;
        rn0 = n0;
        pA = Panel{g.a + rm0 * g.lda, min(g.M - rm0, (int64_t)BM) * g.lda};
        pB = Panel{g.b + rn0 * g.ldb, min(g.N - rn0, (int64_t)BN) * g.ldb};
#pragma unroll
        for (int r = 0; r < NSD; ++r) {
            const bool to_b = r & 1;
            const int j = r >> 1;  // scale slice within the stage
            const int64_t r0 = to_b ? rn0 : rm0, sld = to_b ? g.ld_sb : g.ld_sa;
            // scalar part of this slice's address; the lane adds its row
            // offset.  Rows past the operand read other scales or zeros:
            // their products only reach outputs that are not stored.
            const int64_t sb0 = SKM ? (j * sld + r0) * 4 : SF32 ? r0 * sld * 4 + j * 16 : r0 * sld + j * 4;
            pS[r] = Panel{reinterpret_cast<const uint8_t *>(to_b ? g.sb : g.sa) + sb0,
                          (int64_t)(to_b ? sbytes_b : sbytes_a) - sb0};
        }
    };
    auto set_refill_tile = [&](int ti) {
        int64_t m0, n0;
        tile_of(ti, m0, n0);
        set_refill_origin(m0, n0);
    };
    // buffer descriptors of k-step kt of the refill tile
    v4i_rsrc rsA, rsB, rsS[NSD];
    auto make_desc_a = [&](int kt) {
        const int64_t ko = (int64_t)kt * BKB;
        rsA = buf_rsrc(pA.p + ko, (uint64_t)(pA.n - ko));
    };
    auto make_desc_b = [&](int kt) {
        const int64_t ko = (int64_t)kt * BKB;
        rsB = buf_rsrc(pB.p + ko, (uint64_t)(pB.n - ko));
    };
    auto make_desc_s = [&](int kt) {
#pragma unroll
        for (int r = 0; r < NSD; ++r) {
            const int64_t so = (int64_t)kt * sstep[r];
            rsS[r] = buf_rsrc(pS[r].p + so, (uint64_t)(pS[r].n - so));
        }
    };
    // one memory op (q = 0..L-1) of loading the refill stage into ring slot s
    auto issue_op = [&](int s, int q) {
        if (q < 2 * XA) {
            const int i = q >> 1;
            const uint32_t m0 = lds_u32((q & 1) ? &sB[0][0] : &sA[0][0]) + s * TILE_B + (i * NLW + wave) * 1024;
            if ((q & 1) == 0) dma_x4(offA0 + i * stepA, rsA, m0);
            else dma_x4(offB0 + i * stepB, rsB, m0);
            return;
        }
        const int r = q - 2 * XA;
        const bool to_b = r & 1;
        const int j = r >> 1;
        const uint32_t m0 = lds_u32(to_b ? &sSB[s][j][(wave & 3) * 64 * SSL] : &sSA[s][j][(wave & 3) * 64 * SSL]);
        if constexpr (SF32) dma_x4(to_b ? offSB : offSA, rsS[r], m0);
        else dma_x1(to_b ? offSB : offSA, rsS[r], m0);
    };

    // K positions: at K-step st, lane half h supplies 16-byte chunk 2h + st
    // of its row (blocks 2h and 2h + 1), so one scale register per fragment
    // row serves the whole stage and op_sel = st picks the block's byte.  A
    // and B use the same assignment, so the sum is unchanged.
    auto chunk_of = [&](int st) { return 2 * half + st; };
    auto read_frag = [&](int s, int st, int q, v4i (&fa)[TM], v4i (&fb)[TN]) {
        const int c = chunk_of(st);
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        const uint8_t *base = q < TM ? sA[s] : sB[s];
        const u32x4 v = *reinterpret_cast<const u32x4 *>(base + r * BKB + ((c ^ f4_swz<CPR>(r)) << 4));
        const v4i f = v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
        if (q < TM) fa[q] = f;
        else fb[q - TM] = f;
    };
    // scale register of fragment row q: the bytes of blocks chunk_of(0..KS-1)
    auto read_scale = [&](int s, int q, uint32_t (&sa)[TM], uint32_t (&sb)[TN]) {
        const uint8_t *tab = q < TM ? sSA[s][0] : sSB[s][0];
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        uint32_t v;
        if constexpr (SF32) {
            const u32x4 f = *reinterpret_cast<const u32x4 *>(tab + r * 16);
            v = (f32_scale_e8m0(f[0]) | (f32_scale_e8m0(f[1]) << 8) | (f32_scale_e8m0(f[2]) << 16) |
                 (f32_scale_e8m0(f[3]) << 24)) >> (16 * half);
        } else {
            v = *reinterpret_cast<const uint16_t *>(tab + r * 4 + 2 * half);
        }
        if (q < TM) sa[q] = v;
        else sb[q - TM] = v;
    };

    // The main loop, instantiated for loader and non-loader waves.
    auto body = [&](auto loader_c) __attribute__((always_inline)) {
    constexpr bool LOADER = decltype(loader_c)::value;
    v16f acc[TM][TN];
    uint32_t scA[TM], scB[TN], nA[TM], nB[TN];
    v4i fa[2][TM], fb[2][TN];

    // ---- prologue: fill the ring, publish stage 0, read its step-0 operands
    if constexpr (LOADER) {
        int cur = -1;
#pragma unroll
        for (int p = 0; p < S; ++p) {
            const int ti = stage_tile_iter(p, nk, my_tiles);
            if (ti != cur) {
                set_refill_tile(ti);
                cur = ti;
            }
            make_desc_a(p % nk);
            make_desc_b(p % nk);
            make_desc_s(p % nk);
#pragma unroll
            for (int q = 0; q < L; ++q) issue_op(p, q);
        }
    }
    wait_vm_barrier<(S - 1) * L>();
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_scale(0, q, scA, scB);
#pragma unroll
    for (int q = 0; q < NRD; ++q) read_frag(0, 0, q, fa[0], fb[0]);

    // full-tile stores: 16-byte aligned rows, and 8 rows of C within a
    // 32-bit byte offset of a lane's row
    const bool vec_c = ((reinterpret_cast<uintptr_t>(g.c) & 15) == 0) && (g.ldc % 4 == 0) && g.ldc < ((int64_t)1 << 26);
    // Stage u + S refills slot u % S.  Stage kt of tile iteration ti
    // refills k-step kt + ra of tile ti + qa while kt + ra < nk (phase A)
    // and k-step kt + ra - nk of tile ti + qa + 1 after (phase B), with
    // qa = S / nk and ra = S % nk; the refill panels are set once per phase,
    // outside the stage loops.  Stages past the last one re-load the
    // workgroup's last tile (tile_of clamps), so the loads stay inside the
    // operands and land in slots that are never read again.
    const int qa = S / nk, ra = S % nk;
    int u = 0;
    for (int ti = 0; ti < my_tiles; ++ti) {
        int64_t mb0 = 0, nb0 = 0;  // origin of the phase B refill tile
        if constexpr (LOADER) {
            tile_of(ti + qa + 1, mb0, nb0);
            set_refill_tile(ti + qa);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

        // one pipeline stage (stage u, ring slot u % S) whose refill loads
        // k-step rk of the current refill tile
        auto run_stage = [&](const int rk) __attribute__((always_inline)) {
            const int s = u % S;
            const int sn = (u + 1) % S;
            // Descriptors of the refill stage, built before the stage's
            // MFMAs.  The empty asm passes rk through an SGPR so that the IR
            // optimizer cannot hoist a part above the scheduling fence in
            // front of it.
            auto refill_desc_part = [&](int c) {
                int k = __builtin_amdgcn_readfirstlane(rk);
                asm volatile("" : "+s"(k));
                if (c == 0) make_desc_a(k);
                else if (c == 1) make_desc_b(k);
                else make_desc_s(k);
            };
            if constexpr (LOADER)
                for (int c = 0; c < 3; ++c) refill_desc_part(c);
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                const int fb_cur = st & 1;
                if (st == KS - 1) {
                    // this wave's reads of slot s are complete; once all waves
                    // pass the barrier slot s is free and stage u+1 has landed
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    stage_barrier<LOADER, (S - 2) * L>();
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int idx = 0; idx < NMF; ++idx) {
                    const int i = idx / TN, j = idx % TN;
                    acc[i][j] = mfma_scale_f4(fa[fb_cur][i], fb[fb_cur][j], acc[i][j], 4, 4, st, (int)scA[i], st,
                                              (int)scB[j]);
                    if (st < KS - 1) {
                        // fragments of the next K-step of this stage
#pragma unroll
                        for (int r = idx * RPM0; r < (idx + 1) * RPM0; ++r)
                            if (r < NRD) read_frag(s, st + 1, r, fa[fb_cur ^ 1], fb[fb_cur ^ 1]);
                    } else {
                        // refill of slot s, then the next stage's scales and
                        // K-step-0 fragments
#pragma unroll
                        for (int o = idx * OPM; o < (idx + 1) * OPM; ++o)
                            if (LOADER && o < L) issue_op(s, o);
#pragma unroll
                        for (int r = idx * RPM1; r < (idx + 1) * RPM1; ++r) {
                            if (r < NRD) read_scale(sn, r, nA, nB);
                            else if (r < 2 * NRD) read_frag(sn, 0, r - NRD, fa[0], fb[0]);
                        }
                    }
                    // Pin this slot's LDS reads here: the MFMA is a pure
                    // intrinsic, so without a memory clobber the optimizer
                    // may hoist every later K-step's reads to the top of the
                    // stage and keep all their fragments live at once.
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) scA[i] = nA[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) scB[j] = nB[j];
        };
        // stages kt0 .. kt1-1 of this tile, refilling k-step kt + rk_off;
        // with a 2-slot ring, pairs of stages with compile-time slots
        auto run_range = [&](int kt0, int kt1, int rk_off) __attribute__((always_inline)) {
            for (int kt = kt0; kt < kt1; ++kt, ++u) run_stage(kt + rk_off);
        };
        run_range(0, nk - ra, ra);
        if constexpr (LOADER) set_refill_origin(mb0, nb0);
        run_range(nk - ra, nk, ra - nk);

        // ---- epilogue of tile ti.  acc element e of tile (i, j) sits at
        //      row = i*32 + 8*(e/4) + 4*half + e%4,  col = j*32 + frow;
        //      a 4x4 transpose inside each quad of lanes gives every lane 4
        //      consecutive columns of one row.
        int64_t m0, n0;
        tile_of(ti, m0, n0);
        const int q = frow & 3;
        if (vec_c && m0 + BM <= g.M && n0 + BN <= g.N) {
            // Full tile: one branch for the whole tile, and each store's
            // address is a wave-uniform row pointer (scalar arithmetic) plus
            // this lane's fixed byte offset plus an immediate for column block j.
            constexpr int EB = CT == LSMX_F32 ? 4 : 2;  // bytes per output element
            const uint8_t *cw = reinterpret_cast<const uint8_t *>(g.c) +
                                ((m0 + wm * (TM * 32)) * g.ldc + n0 + wn * (TN * 32)) * EB;
            if constexpr (CT == LSMX_F32) {
                const uint32_t loff = (uint32_t)(((4 * half + q) * g.ldc + (frow & ~3)) * EB);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        uint8_t *crow = const_cast<uint8_t *>(cw) + (i * 32 + 8 * gq) * g.ldc * EB;
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            float x[4] = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                          acc[i][j][4 * gq + 3]};
                            quad_transpose(x, q);
                            *reinterpret_cast<u32x4 *>(crow + loff + j * 32 * EB) =
                                u32x4{f2u(x[0]), f2u(x[1]), f2u(x[2]), f2u(x[3])};
                        }
                    }
            } else {
                // 16 bytes per lane (pack16_rows8): rows 16p + 4*half + q
                // and +8, 8 columns at (frow & ~7)
                const bool odd = (frow & 4) != 0;
                const uint32_t loff = (uint32_t)(((4 * half + q + (odd ? 8 : 0)) * g.ldc + (frow & ~7)) * EB);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        uint8_t *crow = const_cast<uint8_t *>(cw) + (i * 32 + 16 * p) * g.ldc * EB;
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const float x0[4] = {acc[i][j][8 * p], acc[i][j][8 * p + 1], acc[i][j][8 * p + 2],
                                                 acc[i][j][8 * p + 3]};
                            const float x1[4] = {acc[i][j][8 * p + 4], acc[i][j][8 * p + 5], acc[i][j][8 * p + 6],
                                                 acc[i][j][8 * p + 7]};
                            *reinterpret_cast<u32x4 *>(crow + loff + j * 32 * EB) = pack16_rows8<CT>(x0, x1, q, odd);
                        }
                    }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        float x[4] = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                      acc[i][j][4 * gq + 3]};
                        // all four lanes of a quad take part in the exchanges,
                        // so the bounds tests come after them
                        quad_transpose(x, q);
                        const int64_t row = m0 + wm * (TM * 32) + i * 32 + 8 * gq + 4 * half + q;
                        const int64_t col = n0 + wn * (TN * 32) + j * 32 + (frow & ~3);
                        if (row < g.M)
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                if (col + c < g.N) store_c<CT>(g.c, row * g.ldc + col + c, x[c]);
                    }
        }
    }
    };
    if (NW == NLW || wave < NLW) body(BoolC<true>{});
    else body(BoolC<false>{});
    // no load may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// The same pipeline on v_mfma_scale_f32_16x16x128_f8f6f4.  Under the chip's
// power limit the 16 x 16 shape holds a higher clock at the same matrix-core
// occupancy: per FLOP it reads and writes half the accumulator registers of
// the 32 x 32 shape.  For this instruction lane 16g + r supplies 16 bytes,
// one MX block, of row r and K-group g (g = 0..3).  A stage (128 bytes of
// every row, 8 blocks) is two K-steps of 128 codes; at K-step st lane group g
// takes block 2g + st, so one scale register per fragment row (the dword of
// scale slice g >> 1, shifted right by 16 (g & 1)) serves the whole stage and
// op_sel = st picks the block's byte.  A and B use the same assignment, so
// the sum is unchanged.
//
// Per wave 64 x 128 = 4 x 8 tiles of 16 x 16.  MFMAs run column-block major
// (j outer, i inner): the 4 A fragments of a K-step stay in registers while
// the 8 B fragments stream past them, each read two column blocks ahead, so
// only a few B fragments are live at once.  In K-step 1 the B fragments of
// column blocks 2..7 are read early; once they have landed the slot is fully
// read and the stage barrier follows, before the MFMAs of column block JB.
// Those last (8 - JB) * 4 MFMAs cover the barrier, the refill of the slot
// (loader waves) and the reads of the next stage's scales and first
// fragments.  Ring, DMA addressing, schedule and loader waves are those of
// gemm_f4f4_kernel's wide path.
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ v4f mfma_scale_f4_16(v4i a, v4i b, v4f c, int cbsz, int blgp, int opsel_a, int scale_a, int opsel_b,
                                int scale_b) __asm("llvm.amdgcn.mfma.scale.f32.16x16x128.f8f6f4.v4i32.v4i32");

// ---- quantizing epilogue: both MXFP4 forms of a wave's 64 x 128 outputs,
// rounded to bf16 (cb), with the rule and K-major E8M0 layout of
// lsmx_quantize_mxfp4_2d applied to the stored bf16 C (the column form is
// the quantization of C^T along its rows).  cb[i][j][h] holds rows
// 16 i + 4 grp + 2 h (low half) and + 1 (high half) of column 16 j + r16.

// Column maxima of 32-row blocks: cam[ip][jp] = the 16-bit magnitude maxima
// of rows 32 ip .. + 32 in column 16 (2 jp) + r16 (low half) and 16 (2 jp +
// 1) + r16 (high half), the same in all four lane groups.  Returns the
// largest over the wave's columns.
LSMX_DEV uint32_t qepi_col_maxima(const uint32_t (&cb)[4][8][2], uint32_t (&cam)[2][4]) {
    uint32_t top = 0;
#pragma unroll
    for (int ip = 0; ip < 2; ++ip)
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
            uint32_t h[2];
#pragma unroll
            for (int o = 0; o < 2; ++o) {
                const int j = 2 * jp + o;
                const uint32_t m = pk_max16(pk_max16(cb[2 * ip][j][0] & 0x7FFF7FFFu, cb[2 * ip][j][1] & 0x7FFF7FFFu),
                                            pk_max16(cb[2 * ip + 1][j][0] & 0x7FFF7FFFu,
                                                     cb[2 * ip + 1][j][1] & 0x7FFF7FFFu));
                h[o] = max(m & 0xFFFFu, m >> 16);
            }
            uint32_t x = h[0] | (h[1] << 16);
            // lanes l and l ^ 32, then l and l ^ 16: each swap returns the two
            // halves of the pair, so their maximum is the pair's in every lane
            const auto s32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
            x = pk_max16(s32[0], s32[1]);
            const auto s16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
            x = pk_max16(s16[0], s16[1]);
            cam[ip][jp] = x;
            top = pk_max16(top, x);
        }
    return max(top & 0xFFFFu, top >> 16);
}

// The column codes d0 (rows 0..31) and d1 (rows 32..63) of lane r16 + 16 grp
// -- the low half of d_ip holds code bytes 16 ip + 2 grp .. + 2 of its
// column, the high half bytes 16 ip + 8 + 2 grp .. + 2 -- regrouped over the
// four lane groups so that lane group grp holds bytes 8 grp .. + 8.
LSMX_DEV u32x2 qepi_col_regroup(uint32_t d0, uint32_t d1, int grp) {
    // groups g and g + 2 trade: group g now holds the words of ip = g >> 1
    // from groups g & 1 (x) and (g & 1) + 2 (y)
    const auto xy = __builtin_amdgcn_permlane32_swap(d0, d1, false, false);
    const uint32_t x = xy[0], y = xy[1];
    const bool od = (grp & 1) != 0;
    // even groups collect the low halves (bytes 16 ip ..), odd groups the
    // high halves (16 ip + 8 ..); v_perm_b32 selector bytes 0-3 pick bytes
    // of the second operand, 4-7 of the first
    const uint32_t lo = __builtin_amdgcn_perm(y, x, 0x05040100u), hi = __builtin_amdgcn_perm(y, x, 0x07060302u);
    const uint32_t keep = od ? hi : lo, send = od ? lo : hi;
    const auto sw = __builtin_amdgcn_permlane16_swap(send, send, false, false);
    const uint32_t recv = od ? sw[0] : sw[1];       // the partner group's send
    const uint32_t first = od ? recv : keep, second = od ? keep : recv;
    return u32x2{__builtin_amdgcn_perm(second, first, 0x05040100u), __builtin_amdgcn_perm(second, first, 0x07060302u)};
}

template <bool ANY>
LSMX_DEV float qepi_nudge(uint32_t b) {
    if constexpr (ANY) return nudge_keep_nan(b);
    else return tie_down16(b);
}
template <bool ANY>
LSMX_DEV uint32_t qepi_e8(uint32_t am16) {
    if constexpr (ANY) return block_e8m0_16x(am16 << 16);
    else return block_e8m0_16(am16 << 16);
}
template <bool ANY>
LSMX_DEV uint32_t qepi_codes(const float (&f)[8], uint32_t e8) {
    if constexpr (ANY) return codes8_any(f, e8);
    else return cvt_fp4_x8(f, u2f(e8 << 23));
}

// Both forms of the wave's outputs: rows r0 .. + 64, columns c0 .. + 128 of
// C.  ANY: the wave's outputs hold an Inf or NaN (the rules of
// block_e8m0_16x and codes8_any).
template <bool ANY>
LSMX_DEV void qepi_store(const uint32_t (&cb)[4][8][2], const uint32_t (&cam)[2][4], const GemmArgs &g, int64_t r0,
                         int64_t c0, int el) {
    const int q = el & 3, grp = el >> 4, r16 = el & 15;
    const bool odd = (el & 4) != 0;
    const int cl = 16 * (odd ? 1 : 0) + 8 * ((el >> 3) & 1);
    // Store addresses: a wave-uniform base per array (scalar registers) plus
    // a 32-bit lane offset (the launcher bounds the strides), so that each
    // store costs no 64-bit address arithmetic.
    uint8_t *const ccb = g.codes_c + c0 * g.ld_cc + r0 / 2;
    const uint32_t ccl = (uint32_t)(r16 * g.ld_cc + 8 * grp);
    uint8_t *const scb = g.scale_c + ((r0 >> 7) * g.ld_sc + c0) * 4 + 2 * ((r0 >> 6) & 1);
    const uint32_t scl = (uint32_t)((16 * grp + r16) * 4);
    uint8_t *const rcb = g.codes_r + r0 * g.ld_cr + c0 / 2;
    const uint32_t rcl = (uint32_t)((4 * grp + q) * g.ld_cr + cl / 2);
    uint8_t *const rsb = g.scale_r + ((c0 >> 7) * g.ld_sr + r0) * 4;
    const uint32_t rsl = (uint32_t)((4 * grp + q) * 4);
    uint8_t *const cwb = reinterpret_cast<uint8_t *>(g.c) + (r0 * g.ldc + c0) * 2;
    const uint32_t cwl = (uint32_t)(((4 * grp + q) * g.ldc + cl) * 2);
    // ---- column form: codes_c [N][M / 2], scale_c [M / 128][N][4]
    uint32_t sp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t d[2];
#pragma unroll
        for (int ip = 0; ip < 2; ++ip) {
            const uint32_t e8 = qepi_e8<ANY>((cam[ip][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            float f[8];
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t w = cb[2 * ip + k][j][h];
                    f[4 * k + 2 * h] = qepi_nudge<ANY>(w << 16);
                    f[4 * k + 2 * h + 1] = qepi_nudge<ANY>(w & 0xFFFF0000u);
                }
            d[ip] = qepi_codes<ANY>(f, e8);
            sp[j] = ip == 0 ? e8 : sp[j] | (e8 << 8);
        }
        const u32x2 v = qepi_col_regroup(d[0], d[1], grp);
        *reinterpret_cast<u32x2 *>(ccb + j * (16 * g.ld_cc) + ccl) = v;
    }
    // the two scale bytes of column 16 j + r16 from lane group j & 3
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const uint32_t v = grp == 0 ? sp[4 * jj] : grp == 1 ? sp[4 * jj + 1] : grp == 2 ? sp[4 * jj + 2] : sp[4 * jj + 3];
        *reinterpret_cast<uint16_t *>(scb + 256 * jj + scl) = (uint16_t)v;
    }
    // ---- row form: codes_r [M][N / 2], scale_r [N / 128][M][4]; lanes hold
    // 8 consecutive columns of one row after the in-quad transpose
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t rs = 0;
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
            const u32x4 p = pack16_rows8_of(quad_pack16_bits(cb[i][2 * jp][0], cb[i][2 * jp][1], q),
                                            quad_pack16_bits(cb[i][2 * jp + 1][0], cb[i][2 * jp + 1][1], q), odd);
            if (g.c) *reinterpret_cast<u32x4 *>(cwb + i * (32 * g.ldc) + 64 * jp + cwl) = p;
            const uint32_t m = pk_max16(pk_max16(p[0] & 0x7FFF7FFFu, p[1] & 0x7FFF7FFFu),
                                        pk_max16(p[2] & 0x7FFF7FFFu, p[3] & 0x7FFF7FFFu));
            // the block's 32 columns lie in lanes l, l ^ 4, l ^ 8, l ^ 12:
            // rotations by 4 and 8 within the 16-lane row reach all four
            uint32_t am = max(m & 0xFFFFu, m >> 16);
            am = max(am, (uint32_t)__builtin_amdgcn_mov_dpp((int)am, 0x124, 0xF, 0xF, false));
            am = max(am, (uint32_t)__builtin_amdgcn_mov_dpp((int)am, 0x128, 0xF, 0xF, false));
            const uint32_t e8 = qepi_e8<ANY>(am);
            float f[8];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                f[2 * h] = qepi_nudge<ANY>(p[h] << 16);
                f[2 * h + 1] = qepi_nudge<ANY>(p[h] & 0xFFFF0000u);
            }
            *reinterpret_cast<uint32_t *>(rcb + i * (16 * g.ld_cr) + 16 * jp + rcl) = qepi_codes<ANY>(f, e8);
            rs |= e8 << (8 * jp);
        }
        if ((el & 12) == 0) *reinterpret_cast<uint32_t *>(rsb + 64 * i + rsl) = rs;
    }
}

template <int JB, int CT, bool EPI = false>
__global__ __launch_bounds__(512, 1) void gemm_f4f4_mx16_kernel(GemmArgs g) {
    using namespace f4;
    constexpr int S = 2;                             // ring slots
    constexpr int WGN = 2;                           // waves 4 x 2, 64 x 128 each
    constexpr int TM = 4, TN = 8;                    // 16 x 16 tiles per wave
    constexpr int BKB = 128, CPR = 8, RPI = 64 / CPR;
    constexpr int TILE_B = BM * BKB;                 // bytes per operand per stage
    constexpr int NSL = 2;                           // 128-code scale slices per stage
    constexpr int SLB = BM * 4 + 64;                 // slice stride: +64 B keeps lane groups 0-1 and 2-3 on other banks
    constexpr int NLW = 4;                           // loader waves
    constexpr int XA = (TILE_B / 16) / (64 * NLW);   // 16-byte DMA slots per loader lane per operand
    constexpr int L = 2 * XA + 1;                    // loads per loader lane per stage (+1: a 1 KiB scale slice)
    constexpr int NPOST = (TN - JB) * TM;            // K-step 1 MFMAs after the barrier
    static_assert(JB >= 2 && JB < TN, "barrier position");
    static_assert(BN == 256 && BM == 256, "256 x 256 tiles");
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sB[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sSA[S][NSL * SLB];
    __shared__ __attribute__((aligned(16))) uint8_t sSB[S][NSL * SLB];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nk = (int)(g.K / (2 * BKB));

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int r16 = lane & 15, grp = lane >> 4;

    // ---- DMA addressing (loader waves), as in gemm_f4f4_kernel.  Scales are
    // K-major ([K/128][rows][4]): loader wave w loads the 1 KiB slice w & 1
    // of operand (w >> 1) & 1 of the refill stage with one 16-byte DMA per
    // lane.
    const int drow0 = wave * RPI + lane / CPR;
    const uint32_t offA0 = (uint32_t)(drow0 * g.lda + ((lane % CPR) ^ f4_swz<CPR>(drow0)) * 16);
    const uint32_t offB0 = (uint32_t)(drow0 * g.ldb + ((lane % CPR) ^ f4_swz<CPR>(drow0)) * 16);
    const uint32_t stepA = (uint32_t)(NLW * RPI * g.lda), stepB = (uint32_t)(NLW * RPI * g.ldb);
    const bool s_b = (wave >> 1) & 1;                // this loader's scale operand and slice
    const int s_j = wave & 1;
    const int64_t s_ld = s_b ? g.ld_sb : g.ld_sa;
    const uint64_t s_bytes = ((g.K / 128 - 1) * s_ld + (s_b ? g.N : g.M)) * 4;
    static_assert(GROUP_M <= 4, "tile_coords divides by group heights up to 4");
    const TileMap tmap = make_tile_map(tiles_m, tiles_n, GROUP_M);
    auto tile_of = [&](int ti, int64_t &m0, int64_t &n0) {
        int tm, tn;
        ti = imax(0, imin(ti, my_tiles - 1));
        tile_coords((int)blockIdx.x + ti * (int)gridDim.x, tmap, tm, tn);
        m0 = (int64_t)tm * BM;
        n0 = (int64_t)tn * BN;
    };
    struct Panel {
        const uint8_t *p;
        int64_t n;
    };
    Panel pA, pB, pS;
    const int64_t sstep = NSL * s_ld * 4;            // scale bytes one stage advances
    auto set_refill_origin = [&](int64_t m0, int64_t n0) {
        pA = Panel{g.a + m0 * g.lda, min(g.M - m0, (int64_t)BM) * g.lda};
        pB = Panel{g.b + n0 * g.ldb, min(g.N - n0, (int64_t)BN) * g.ldb};
        // rows past the operand read other scales or zeros: their products
        // only reach outputs that are not stored
        const int64_t sb0 = (s_j * s_ld + (s_b ? n0 : m0)) * 4;
        pS = Panel{reinterpret_cast<const uint8_t *>(s_b ? g.sb : g.sa) + sb0, (int64_t)s_bytes - sb0};
    };
    auto set_refill_tile = [&](int ti) {
        int64_t m0, n0;
        tile_of(ti, m0, n0);
        set_refill_origin(m0, n0);
    };
    v4i_rsrc rsA, rsB, rsS;
    auto make_desc_a = [&](int kt) {
        const int64_t ko = (int64_t)kt * BKB;
        rsA = buf_rsrc(pA.p + ko, (uint64_t)(pA.n - ko));
    };
    auto make_desc_b = [&](int kt) {
        const int64_t ko = (int64_t)kt * BKB;
        rsB = buf_rsrc(pB.p + ko, (uint64_t)(pB.n - ko));
    };
    auto make_desc_s = [&](int kt) {
        const int64_t so = (int64_t)kt * sstep;
        rsS = buf_rsrc(pS.p + so, (uint64_t)(pS.n - so));
    };
    auto issue_op = [&](int s, int q) {
        if (q < 2 * XA) {
            const int i = q >> 1;
            const uint32_t m0 = lds_u32((q & 1) ? &sB[0][0] : &sA[0][0]) + s * TILE_B + (i * NLW + wave) * 1024;
            if ((q & 1) == 0) dma_x4_at(offA0, i, stepA, rsA, m0);
            else dma_x4_at(offB0, i, stepB, rsB, m0);
            return;
        }
        dma_x4((uint32_t)lane * 16, rsS, lds_u32(s_b ? &sSB[s][s_j * SLB] : &sSA[s][s_j * SLB]));
    };

    // ---- fragment and scale reads.  Rows of fragment q start 16 q rows
    // apart, so the chunk swizzle ((row >> 1) & 7) depends on r16 only and
    // each read is a per-lane offset plus an immediate.
    const int fA0 = (wm * 64) * BKB, fB0 = (wn * 128) * BKB;
    uint32_t loff[2];
    for (int st = 0; st < 2; ++st) loff[st] = (uint32_t)(r16 * BKB + (((2 * grp + st) ^ ((r16 >> 1) & 7)) << 4));
    // A lane reads only the two scale bytes its K-group uses (blocks 2g and
    // 2g + 1: bytes 2 (g & 1) and +1 of slice g >> 1) with a 16-bit read at a
    // per-lane byte offset; op_sel = st picks the byte.  Reading the dword
    // and shifting it would make a VALU instruction wait for every scale read
    // (measured: 245 against 223 us at 8192^3).
    const uint32_t soff = (uint32_t)((grp >> 1) * SLB + r16 * 4 + 2 * (grp & 1));
    auto rd_a = [&](int s, int st, int i) -> v4i {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(&sA[s][fA0 + i * 16 * BKB] + loff[st]);
        return v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
    };
    auto rd_b = [&](int s, int st, int j) -> v4i {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(&sB[s][fB0 + j * 16 * BKB] + loff[st]);
        return v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
    };
    auto rd_sa = [&](int s, int i) -> uint32_t {
        return *reinterpret_cast<const uint16_t *>(&sSA[s][(wm * 64 + 16 * i) * 4] + soff);
    };
    auto rd_sb = [&](int s, int j) -> uint32_t {
        return *reinterpret_cast<const uint16_t *>(&sSB[s][(wn * 128 + 16 * j) * 4] + soff);
    };

    auto body = [&](auto loader_c) __attribute__((always_inline)) {
    constexpr bool LOADER = decltype(loader_c)::value;
    v4f acc[TM][TN];
    // A scales live for the whole stage (both K-steps); a B fragment's scale
    // is read with it and lives only as long as the fragment
    uint32_t scA[TM], nA[TM], scB[TN];
    v4i fa[2][TM], fb[TN];

    // ---- prologue: fill the ring, publish stage 0, read its first operands
    if constexpr (LOADER) {
        int cur = -1;
#pragma unroll
        for (int p = 0; p < S; ++p) {
            const int ti = stage_tile_iter(p, nk, my_tiles);
            if (ti != cur) {
                set_refill_tile(ti);
                cur = ti;
            }
            make_desc_a(p % nk);
            make_desc_b(p % nk);
            make_desc_s(p % nk);
#pragma unroll
            for (int q = 0; q < L; ++q) issue_op(p, q);
        }
    }
    wait_vm_barrier<(S - 1) * L>();
#pragma unroll
    for (int i = 0; i < TM; ++i) scA[i] = rd_sa(0, i);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[0][i] = rd_a(0, 0, i);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        fb[j] = rd_b(0, 0, j);
        scB[j] = rd_sb(0, j);
    }

    const bool vec_c = ((reinterpret_cast<uintptr_t>(g.c) & 15) == 0) && (g.ldc % 4 == 0) && g.ldc < ((int64_t)1 << 26);
    const int qa = S / nk, ra = S % nk;
    int u = 0;
    for (int ti = 0; ti < my_tiles; ++ti) {
        int64_t mb0 = 0, nb0 = 0;
        if constexpr (LOADER) {
            tile_of(ti + qa + 1, mb0, nb0);
            set_refill_tile(ti + qa);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

        auto run_stage = [&](const int rk, auto slot_c) __attribute__((always_inline)) {
            constexpr int s = decltype(slot_c)::value;
            constexpr int sn = (s + 1) % S;
            auto refill_desc_part = [&](int c) {
                int k = __builtin_amdgcn_readfirstlane(rk);
                asm volatile("" : "+s"(k));
                if (c == 0) make_desc_a(k);
                else if (c == 1) make_desc_b(k);
                else make_desc_s(k);
            };
            // B fragment j of K-step st from slot sl; its scale register
            // serves both K-steps and is read with the step-0 fragment
            auto load_b = [&](int sl, int st, int j) __attribute__((always_inline)) {
                fb[j] = rd_b(sl, st, j);
                if (st == 0) scB[j] = rd_sb(sl, j);
            };
            // next-stage reads after the barrier, in the order they are
            // needed: A(0, i) with the A scales, B(0, 0..1) with theirs
            constexpr int NNEXT = 2 * TM + 2;
            auto next_read = [&](int k) {
                // 0: A0 1: B0 2: sA0 3: A1 4: sA1 5: A2 6: sA2 7: A3 8: sA3 9: B1
                if (k == 1) load_b(sn, 0, 0);
                else if (k == 9) load_b(sn, 0, 1);
                else {
                    const int i = k < 2 ? 0 : (k - 1) >> 1;
                    if (k == 0 || (k > 1 && (k & 1))) fa[0][i] = rd_a(sn, 0, i);
                    else nA[i] = rd_sa(sn, i);
                }
            };
#pragma unroll
            for (int st = 0; st < 2; ++st) {
#pragma unroll
                for (int idx = 0; idx < TM * TN; ++idx) {
                    const int j = idx / TM, i = idx % TM;
                    if (st == 1 && idx == JB * TM) {
                        // this wave's reads of slot s are complete; once all
                        // waves pass the barrier the slot is free and stage
                        // u + 1 has landed
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        stage_barrier<LOADER, (S - 2) * L>();
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    acc[i][j] = mfma_scale_f4_16(fa[st][i], fb[j], acc[i][j], 4, 4, st, (int)scA[i], st, (int)scB[j]);
                    if (st == 0) {
                        if (LOADER && idx < 3) {
                            __builtin_amdgcn_sched_barrier(0);
                            refill_desc_part(idx);
                        }
                        if (i == 0) {
                            if (j + 2 < TN) load_b(s, 0, j + 2);
                            else load_b(s, 1, j + 2 - TN);
                        }
                        if (i == 2 && j < TM) fa[1][j] = rd_a(s, 1, j);
                    } else if (idx < JB * TM) {
                        // B fragments 2..7 of K-step 1, spread over the MFMAs before the barrier
                        constexpr int NR = TN - 2;
#pragma unroll
                        for (int k = 0; k < NR; ++k)
                            if (idx == k * (JB * TM - 2) / NR) load_b(s, 1, 2 + k);
                    } else {
                        const int p = idx - JB * TM;
#pragma unroll
                        for (int k = p * NNEXT / NPOST; k < (p + 1) * NNEXT / NPOST; ++k) next_read(k);
#pragma unroll
                        for (int o = p * L / NPOST; o < (p + 1) * L / NPOST; ++o)
                            if (LOADER) issue_op(s, o);
                    }
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) scA[i] = nA[i];
        };
        auto run_range = [&](int kt0, int kt1, int rk_off) __attribute__((always_inline)) {
            int kt = kt0;
            if (kt < kt1 && (u & 1)) {
                run_stage(kt + rk_off, SlotC<1>{});
                ++kt, ++u;
            }
            for (; kt + 1 < kt1; kt += 2) {
                run_stage(kt + rk_off, SlotC<0>{});
                ++u;
                run_stage(kt + 1 + rk_off, SlotC<1>{});
                ++u;
            }
            if (kt < kt1) {
                run_stage(kt + rk_off, SlotC<0>{});
                ++u;
            }
        };
        run_range(0, nk - ra, ra);
        if constexpr (LOADER) set_refill_origin(mb0, nb0);
        run_range(nk - ra, nk, ra - nk);

        // ---- epilogue.  acc[i][j] element e sits at row 16 i + 4 grp + e,
        //      column 16 j + r16; a 4 x 4 transpose inside each quad of lanes
        //      gives every lane 4 consecutive columns of row 16 i + 4 grp + q.
        int64_t m0, n0;
        tile_of(ti, m0, n0);
        // lane-dependent epilogue values are derived here from an opaque copy
        // of the lane id: hoisted out of the tile loop they would stay live
        // (and spill) through every stage
        int el = lane;
        asm volatile("" : "+v"(el));
        const int q = el & 3, egrp = el >> 4, er16 = el & 15;
        if constexpr (EPI) {
            // whole tiles only (the launcher checks); round to bf16 first
            uint32_t cb[TM][TN][2];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    cb[i][j][0] = bf16x2(acc[i][j][0], acc[i][j][1]);
                    cb[i][j][1] = bf16x2(acc[i][j][2], acc[i][j][3]);
                }
            uint32_t cam[2][4];
            const uint32_t top = qepi_col_maxima(cb, cam);
            const int64_t r0 = m0 + wm * 64, c0 = n0 + wn * 128;
            if (__builtin_expect(__any(top >= 0x7F80u), 0)) qepi_store<true>(cb, cam, g, r0, c0, el);
            else qepi_store<false>(cb, cam, g, r0, c0, el);
        } else if (vec_c && m0 + BM <= g.M && n0 + BN <= g.N) {
            constexpr int EB = CT == LSMX_F32 ? 4 : 2;
            const uint8_t *cw = reinterpret_cast<const uint8_t *>(g.c) + ((m0 + wm * 64) * g.ldc + n0 + wn * 128) * EB;
            if constexpr (CT == LSMX_F32) {
                const uint32_t loffc = (uint32_t)(((4 * egrp + q) * g.ldc + (er16 & ~3)) * EB);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    uint8_t *crow = const_cast<uint8_t *>(cw) + (16 * i) * g.ldc * EB;
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        float x[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                        quad_transpose(x, q);
                        *reinterpret_cast<u32x4 *>(crow + loffc + j * 16 * EB) = u32x4{f2u(x[0]), f2u(x[1]), f2u(x[2]), f2u(x[3])};
                    }
                }
            } else {
                // column blocks j and j + 1 share one 16-byte store per lane
                // (pack16_rows8 with the second block in place of rows + 8):
                // lanes with bit 2 clear store 8 columns of block j, the
                // others 8 columns of block j + 1
                const bool odd = (el & 4) != 0;
                const uint32_t loffc = (uint32_t)(((4 * egrp + q) * g.ldc + (odd ? 16 : 0) + 8 * ((el >> 3) & 1)) * EB);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    uint8_t *crow = const_cast<uint8_t *>(cw) + (16 * i) * g.ldc * EB;
#pragma unroll
                    for (int jp = 0; jp < TN / 2; ++jp) {
                        const float x0[4] = {acc[i][2 * jp][0], acc[i][2 * jp][1], acc[i][2 * jp][2], acc[i][2 * jp][3]};
                        const float x1[4] = {acc[i][2 * jp + 1][0], acc[i][2 * jp + 1][1], acc[i][2 * jp + 1][2],
                                             acc[i][2 * jp + 1][3]};
                        *reinterpret_cast<u32x4 *>(crow + loffc + jp * 32 * EB) = pack16_rows8<CT>(x0, x1, q, odd);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    float x[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                    quad_transpose(x, q);
                    const int64_t row = m0 + wm * 64 + 16 * i + 4 * egrp + q;
                    const int64_t col = n0 + wn * 128 + 16 * j + (er16 & ~3);
                    if (row < g.M)
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (col + c < g.N) store_c<CT>(g.c, row * g.ldc + col + c, x[c]);
                }
        }
    }
    };
    if (wave < NLW) body(BoolC<true>{});
    else body(BoolC<false>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

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
    const int tiles = (int)(((g.M + f4::BM - 1) / f4::BM) * ((g.N + f4::BN - 1) / f4::BN));
    const int grid = tiles < num_cus() ? tiles : num_cus();
#define LSMX_GC(K, ...)                                                                        \
    do {                                                                                       \
        if (g.c_dtype == LSMX_F32) hipLaunchKernelGGL((K<__VA_ARGS__, LSMX_F32>), grid, 512, 0, s, g);   \
        else if (g.c_dtype == LSMX_BF16) hipLaunchKernelGGL((K<__VA_ARGS__, LSMX_BF16>), grid, 512, 0, s, g); \
        else hipLaunchKernelGGL((K<__VA_ARGS__, LSMX_F16>), grid, 512, 0, s, g);                 \
    } while (0)
    // K-major E8M0 scales and whole 256-code stages: the 16 x 16 x 128
    // kernel, with the stage barrier before column block 4 of its second
    // K-step.  Row-major E8M0 (one scale request per row), fp32 scales (16
    // bytes per row per 128 codes) and K % 256 != 0 run the 32 x 32 x 64
    // kernel on 64-byte stages in a 3- or 4-slot ring; the Python layer
    // regroups scales to K-major before it calls, so it always takes the
    // first path when K allows.
    if (g.K % 256 == 0 && g.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) LSMX_GC(gemm_f4f4_mx16_kernel, 4);
    else if (g.scale_fmt == LSMX_SCALE_F32) LSMX_GC(gemm_f4f4_kernel, LSMX_SCALE_F32, 3);
    else if (g.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) LSMX_GC(gemm_f4f4_kernel, LSMX_SCALE_E8M0_KMAJOR, 4);
    else LSMX_GC(gemm_f4f4_kernel, LSMX_SCALE_E8M0, 4);
#undef LSMX_GC
    return hipGetLastError();
}

hipError_t launch_gemm_f4f4_quant(const GemmArgs &g, hipStream_t s) {
    const int tiles = (int)((g.M / f4::BM) * (g.N / f4::BN));
    const int grid = tiles < num_cus() ? tiles : num_cus();
    hipLaunchKernelGGL((gemm_f4f4_mx16_kernel<4, LSMX_BF16, true>), grid, 512, 0, s, g);
    return hipGetLastError();
}

}  // namespace lsmx
