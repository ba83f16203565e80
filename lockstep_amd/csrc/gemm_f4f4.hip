// Block-scaled MXFP4 x MXFP4 GEMM on gfx950's scaled MFMA.
//
//   C[m, n] = sum_kb  2^(sa[m,kb]-127) * 2^(sb[n,kb]-127) * sum_{k in kb} A[m,k] * Bt[n,k]
//
// Semantics: mxfp4_gemm.py:116-174 (_mxfp4_gemm_packed_kernel /
// mxfp4_gemm_packed) and cuda/mxfp4_mma_gemm.cu:69-184, with both operands
// K-contiguous ("TN"), packed two E2M1 codes per byte, low nibble first.
// Instead of promoting an FP8 product to fp32 every 32-block and multiplying
// by fp32 scales, v_mfma_scale_f32_32x32x64_f8f6f4 (cbsz = blgp = 4, FP4)
// applies one E8M0 scale per lane per operand inside the instruction: for
// that instruction each lane supplies the 32 codes (16 bytes, four VGPRs) of
// one row and one 32-block, which is exactly one MX block, and the byte of
// the scale register selected by op_sel.
//
// Tiling: 256 x 256 macro tile, WGM x WGN waves (default 4 x 2, two waves per
// SIMD), each wave a (256/WGM) x (256/WGN) sub-tile of 32 x 32 MFMA tiles
// with fp32 accumulators.  A pipeline stage holds KS MFMA K-steps of 64
// codes: KS = 4 stages 128 bytes of every row (256 codes), KS = 2 stages 64.
// Whole 128-byte rows matter: the direct-to-LDS path is limited by the
// number of L2 requests, and a 64-byte row segment costs a request for half
// a cache line (measured: 19 B/clk per CU for 16 rows x 64 B per load
// instruction, 36 B/clk for 8 rows x 128 B).
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
// Per stage and wave: while the MFMAs of K-step st run, the fragments of
// K-step st + 1 are read from LDS between them.  Once the slot has been read
// (before K-step 2 with KS = 4, the last K-step with KS = 2), one s_barrier
// (after the stage's own reads completed and the next stage's loads landed)
// frees it; the remaining MFMAs then run with the refill of that slot and the
// next stage's scale and K-step-0 fragment reads interleaved, so the matrix
// core never waits on a burst of memory instructions.  Refills past the last
// stage re-load the workgroup's last tile (tile indices are clamped,
// lsmx_sched.h) into a slot that is never read again, which keeps the loop
// free of branches and the outstanding-load count constant.
//
// Only waves 0-3 issue the refill loads.  The two waves of a SIMD share its
// matrix core; the older one (0-3) wins issue arbitration and reaches the
// stage barrier first, so the younger one's instruction stream sets the pace
// and is kept to MFMAs and LDS reads.  The refill tile changes only in the
// last S stages of a tile, so each tile runs two stage loops ("phases") and
// the refill panels are computed between them, not per stage; with a 2-slot
// ring, stages run in pairs with compile-time slots, which makes every LDS
// address a loop-invariant register plus an immediate.
//
// LDS layout per stage: rows of 16*CPR bytes (CPR = 2*KS chunks of 16 bytes);
// chunk c of row r lives at r*16*CPR + 16*(c ^ swz(r)), which keeps the 16
// lanes a ds_read_b128 serves per cycle on distinct banks.  The DMA writes
// slots in lane order, so the swizzle is applied by choosing each lane's
// source address.
#include "lsmx_dma.h"
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
#ifndef LSMX_F4_NLW_WAIT
#define LSMX_F4_NLW_WAIT 0
#endif
template <bool LOADER, int N>
LSMX_DEV void stage_barrier() {
    if constexpr (LOADER || LSMX_F4_NLW_WAIT) wait_vm_barrier<N>();
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
template <int SFMT, int CT, int S, int WGM, int WGN, int KS>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_f4f4_kernel(GemmArgs g) {
    using namespace f4;
    constexpr bool SF32 = SFMT == LSMX_SCALE_F32;
    constexpr bool SKM = SFMT == LSMX_SCALE_E8M0_KMAJOR;
    constexpr int NW = WGM * WGN;
    constexpr int NTH = 64 * NW;
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
    static_assert(KS == 2 || KS == 4, "2 or 4 K-steps per stage");
    // scale loads: every loader wave loads 64 rows of A's and of B's scales
    // per slice, except for K-major E8M0 scales with KS = 4: one 1 KiB slice
    // (256 rows) per dwordx4 load, loader wave w takes operand (w >> 1) & 1,
    // slice w & 1.
    constexpr bool SX4 = SKM && KS == 4;
    constexpr int LS = SX4 ? 1 : 2 * NSL;
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
    constexpr int NSD = SX4 ? 1 : LS;  // scale descriptors per stage
    struct Panel {
        const uint8_t *p;
        int64_t n;
    };
    Panel pA, pB, pS[NSD];
    int64_t sstep[NSD];
#pragma unroll
    for (int r = 0; r < NSD; ++r) {
        const bool to_b = SX4 ? ((wave >> 1) & 1) : (r & 1);
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
            // SX4: operand (wave >> 1) & 1, slice wave & 1
            const bool to_b = SX4 ? ((wave >> 1) & 1) : (r & 1);
            const int j = SX4 ? (wave & 1) : (r >> 1);  // scale slice within the stage
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
        if constexpr (SX4) {
            const bool xb = (wave >> 1) & 1;
            const int j = wave & 1;
            dma_x4((uint32_t)lane * 16, rsS[0], lds_u32(xb ? &sSB[s][j][0] : &sSA[s][j][0]));
            return;
        }
        const int r = q - 2 * XA;
        const bool to_b = r & 1;
        const int j = r >> 1;
        const uint32_t m0 = lds_u32(to_b ? &sSB[s][j][(wave & 3) * 64 * SSL] : &sSA[s][j][(wave & 3) * 64 * SSL]);
        if constexpr (SF32) dma_x4(to_b ? offSB : offSA, rsS[SX4 ? 0 : r], m0);
        else dma_x1(to_b ? offSB : offSA, rsS[SX4 ? 0 : r], m0);
    };

    // K positions: at K-step st, lane half h supplies 16-byte chunk
    // c = (KS/2)*2*h + st of its row -- for KS = 4 the four blocks of scale
    // slice h, for KS = 2 blocks 2h and 2h+1 -- so one scale register per
    // fragment row serves the whole stage and op_sel = st picks the block's
    // byte.  A and B use the same assignment, so the sum is unchanged.
    auto chunk_of = [&](int st) { return (KS == 4 ? 4 : 2) * half + st; };
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
        const uint8_t *tab = q < TM ? sSA[s][KS == 4 ? half : 0] : sSB[s][KS == 4 ? half : 0];
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        uint32_t v;
        if constexpr (SF32) {
            const u32x4 f = *reinterpret_cast<const u32x4 *>(tab + r * 16);
            v = (f32_scale_e8m0(f[0]) | (f32_scale_e8m0(f[1]) << 8) | (f32_scale_e8m0(f[2]) << 16) |
                 (f32_scale_e8m0(f[3]) << 24)) >> (16 * half);
        } else if constexpr (KS == 4) {
            v = *reinterpret_cast<const uint32_t *>(tab + r * 4);
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
    // fragment buffers: KS = 4 keeps three K-steps' fragments at once (see the stage loop)
    v4i fa[KS == 4 ? 3 : 2][TM], fb[KS == 4 ? 3 : 2][TN];

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
        // SLOT < 0: ring slot u % S computed at run time; SLOT >= 0: the
        // caller knows u % S == SLOT, so every LDS address of the stage is a
        // loop-invariant register plus an immediate offset.
        auto run_stage = [&](const int rk, auto slot_c) __attribute__((always_inline)) {
            constexpr int SLOT = decltype(slot_c)::value;
            const int s = SLOT >= 0 ? SLOT : u % S;
            const int sn = SLOT >= 0 ? (SLOT + 1) % S : (u + 1) % S;
            // Descriptors of the refill stage.  With KS = 4 part c is built
            // after the stage's MFMA c, so that its scalar arithmetic overlaps
            // the matrix core instead of delaying the stage's first MFMA on
            // both waves of a SIMD.  The empty asm passes rk through an SGPR
            // so that the IR optimizer cannot hoist a part above the
            // scheduling fence in front of it.
            constexpr int NPART = 3;
            auto refill_desc_part = [&](int c) {
                int k = __builtin_amdgcn_readfirstlane(rk);
                asm volatile("" : "+s"(k));
                if (c == 0) make_desc_a(k);
                else if (c == 1) make_desc_b(k);
                else make_desc_s(k);
            };
            if constexpr (KS != 4 && LOADER)
                for (int c = 0; c < NPART; ++c) refill_desc_part(c);
            if constexpr (KS == 4) {
                // K-step 0 reads step 1's fragments, step 1 reads steps 2 and
                // 3's, so slot s is fully read before step 2.  The barrier
                // sits there, and the slot's refill is spread over steps 2
                // and 3 (one load per MFMA) instead of being issued in one
                // burst: a burst of direct-to-LDS loads blocks issue on every
                // wave at once and the matrix core goes idle.  Buffers: step
                // 0 -> 0, 1 -> 1, 2 -> 2, 3 -> 0 (free after step 0); the
                // next stage's step 0 is read into 1 and moved to 0.
                constexpr int BUF[4] = {0, 1, 2, 0};
                constexpr int LH = (L + 1) / 2;                  // refill ops in step 2
                constexpr int OPH = (LH + NMF - 1) / NMF;
                constexpr int RP1 = (2 * NRD + NMF - 1) / NMF;   // reads per MFMA in step 1
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    if (st == 2) {
                        // this wave's reads of slot s are complete; once all
                        // waves pass the barrier slot s is free and stage u+1
                        // has landed
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        stage_barrier<LOADER, (S - 2) * L>();
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int idx = 0; idx < NMF; ++idx) {
                        const int i = idx / TN, j = idx % TN;
                        acc[i][j] = mfma_scale_f4(fa[BUF[st]][i], fb[BUF[st]][j], acc[i][j], 4, 4, st, (int)scA[i], st,
                                                  (int)scB[j]);
                        if (st == 0) {
                            if (LOADER && idx < NPART) {
                                __builtin_amdgcn_sched_barrier(0);
                                refill_desc_part(idx);
                            }
                            if (idx < NRD) read_frag(s, 1, idx, fa[1], fb[1]);
                        } else if (st == 1) {
#pragma unroll
                            for (int r = idx * RP1; r < (idx + 1) * RP1; ++r) {
                                if (r < NRD) read_frag(s, 2, r, fa[2], fb[2]);
                                else if (r < 2 * NRD) read_frag(s, 3, r - NRD, fa[0], fb[0]);
                            }
                        } else if (st == 2) {
#pragma unroll
                            for (int o = idx * OPH; o < (idx + 1) * OPH; ++o)
                                if (LOADER && o < LH) issue_op(s, o);
                            if (idx < NRD) read_scale(sn, idx, nA, nB);
                        } else {
#pragma unroll
                            for (int o = LH + idx * OPH; o < LH + (idx + 1) * OPH; ++o)
                                if (LOADER && o < L) issue_op(s, o);
                            if (idx < NRD) read_frag(sn, 0, idx, fa[1], fb[1]);
                        }
                        // Pin this slot's LDS reads here: the MFMA is a pure
                        // intrinsic, so without a memory clobber the optimizer
                        // may hoist every later K-step's reads to the top of
                        // the stage and keep all their fragments live at once.
                        asm volatile("" ::: "memory");
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i) fa[0][i] = fa[1][i];
#pragma unroll
                for (int j = 0; j < TN; ++j) fb[0][j] = fb[1][j];
            } else {
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
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) scA[i] = nA[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) scB[j] = nB[j];
        };
        // stages kt0 .. kt1-1 of this tile, refilling k-step kt + rk_off;
        // with a 2-slot ring, pairs of stages with compile-time slots
        auto run_range = [&](int kt0, int kt1, int rk_off) __attribute__((always_inline)) {
            if constexpr (S == 2) {
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
            } else {
                for (int kt = kt0; kt < kt1; ++kt, ++u) run_stage(kt + rk_off, SlotC<-1>{});
            }
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
// K-steps per stage of the wide path (E8M0 scales, K % 256 == 0) and its ring
// depth: 4 K-steps = 128-byte rows, two 64 KiB stages.
#ifndef LSMX_F4_KS
#define LSMX_F4_KS 4
#endif
#ifndef LSMX_F4_STAGES
#define LSMX_F4_STAGES 2
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
    constexpr int W = LSMX_F4_WGM, Z = LSMX_F4_WGN;
    const int tiles = (int)(((g.M + f4::BM - 1) / f4::BM) * ((g.N + f4::BN - 1) / f4::BN));
    const int grid = tiles < num_cus() ? tiles : num_cus();
    const dim3 blk(64 * W * Z);
#define LSMX_G(F, CT, S, KS) hipLaunchKernelGGL((gemm_f4f4_kernel<F, CT, S, W, Z, KS>), dim3(grid), blk, 0, s, g)
#define LSMX_GC(F, S, KS)                                             \
    do {                                                              \
        if (g.c_dtype == LSMX_F32) LSMX_G(F, LSMX_F32, S, KS);        \
        else if (g.c_dtype == LSMX_BF16) LSMX_G(F, LSMX_BF16, S, KS); \
        else LSMX_G(F, LSMX_F16, S, KS);                              \
    } while (0)
    const bool wide = g.K % (64 * LSMX_F4_KS) == 0;
    if (g.scale_fmt == LSMX_SCALE_F32) LSMX_GC(LSMX_SCALE_F32, 3, 2);  // 16-byte scale rows: narrow stages
    else if (g.scale_fmt == LSMX_SCALE_E8M0_KMAJOR && wide) LSMX_GC(LSMX_SCALE_E8M0_KMAJOR, LSMX_F4_STAGES, LSMX_F4_KS);
    else if (g.scale_fmt == LSMX_SCALE_E8M0_KMAJOR) LSMX_GC(LSMX_SCALE_E8M0_KMAJOR, 4, 2);
    else if (wide) LSMX_GC(LSMX_SCALE_E8M0, LSMX_F4_STAGES, LSMX_F4_KS);
    else LSMX_GC(LSMX_SCALE_E8M0, 4, 2);
#undef LSMX_GC
#undef LSMX_G
    return hipGetLastError();
}

}  // namespace lsmx
