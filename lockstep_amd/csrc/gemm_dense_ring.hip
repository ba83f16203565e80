// Dense bf16 / fp16 GEMMs of dual_gemm.py on a persistent direct-to-LDS ring.
//
// Semantics (fp32 accumulate, fp32 out), both operands K-contiguous:
//   MODE 0  C0 = A0 . B0^T                      gemm          (dual_gemm.py:188-226)
//   MODE 1  C0 = A0 . B0^T + A1 . B1^T          dual_packed   (dual_gemm.py:42-72, 230-241)
//   MODE 2  C0 = A0 . B0^T,  C1 = A1 . B1^T     dual_separate (dual_gemm.py:78-110, 244-255)
// MODE 1 is one GEMM over the interleaved K (the reference pre-scales A1 on
// the host; the kernel only adds the products): 64-deep K blocks of A0.B0
// and A1.B1 alternate, in the order of the reference's loop.  MODE 2 is two GEMM problems
// in one launch: the persistent workgroups walk the tiles of both, ordered so
// that the two tiles sharing (m, n) run side by side on one XCD, so a shared
// B (b0 == b1) is read once per XCD from HBM and hit in L2 the second time.
//
// The machinery is that of the f4 x f4 kernel (gemm_f4f4.hip), without the
// block scales: a bf16/fp16 MFMA K-step of 16 elements reads 16 bytes per
// lane, like an FP4 K-step of 32 codes, so a 128-byte stage row holds four
// K-steps and the LDS layout, swizzle, DMA addressing and fragment reads are
// the same.  256 x 256 tiles, 8 waves in a 4 x 2 grid (64 x 128 per wave,
// two waves per SIMD), a 2-slot ring of 64 KiB stages filled by
// buffer_load ... lds from waves 0-3 only, one barrier per stage, refill
// panels set once per tile phase, stages in pairs with compile-time slots,
// epilogue of 16-byte fp32 stores after an in-quad transpose.
#include "lsmx_dma.h"
#include "lsmx_internal.h"
#include "lsmx_sched.h"
#include "lsmx_store.h"

namespace lsmx {

namespace dr {
constexpr int BM = 256, BN = 256;
constexpr int WGM = 4, WGN = 2, NW = WGM * WGN, NT = 64 * NW;
constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;  // 2 x 4 MFMA tiles per wave
constexpr int NMF = TM * TN;                           // MFMAs per K-step
constexpr int KS = 4;                                  // K-steps per stage
constexpr int BKB = 128;                               // bytes of every row per stage (64 elements)
constexpr int CPR = BKB / 16;                          // 16-byte chunks per row
constexpr int RPI = 64 / CPR;                          // rows per DMA instruction
constexpr int TILE_B = BM * BKB;                       // 32 KiB per operand per stage
constexpr int S = 2;                                   // ring slots
constexpr int NLW = 4;                                 // loader waves
constexpr int XA = (TILE_B / 16) / (64 * NLW);         // DMA loads per loader lane per operand (8)
constexpr int L = 2 * XA;                              // loads per loader wave per stage
constexpr int NRD = TM + TN;                           // fragment reads per K-step
constexpr int GROUP_M = 4;
LSMX_DEV int swz(int row) { return (row >> 1) & 7; }  // 16-byte chunk swizzle of a 128-byte row
}  // namespace dr

typedef int v4i_d __attribute__((ext_vector_type(4)));
typedef float v16f_d __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf_d __attribute__((ext_vector_type(8)));
typedef _Float16 v8h_d __attribute__((ext_vector_type(8)));

template <int DT>
LSMX_DEV v16f_d mfma_dense16(v4i_d a, v4i_d b, v16f_d c) {
    if constexpr (DT == LSMX_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_d, a), __builtin_bit_cast(v8bf_d, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_d, a), __builtin_bit_cast(v8h_d, b), c, 0,
                                                     0, 0);
}

template <int V>
struct DrSlot {
    static constexpr int value = V;
};
template <bool V>
struct DrLoader {
    static constexpr bool value = V;
};

// Four bf16/fp16 values of one column from a [K][N] LDS tile with
// ds_read_b64_tr_b16: within each 16-lane group, lanes 4k .. 4k + 3 give the
// addresses of 4 consecutive values of row k (8 bytes each), and lane j
// receives value j % 4 of lane 4k + j / 4's row piece as its element k, i.e.
// column j of the group's 4 x 16 block (the lane layout was checked on the
// device with an in-bounds probe).
typedef short v4s_d __attribute__((ext_vector_type(4)));
typedef int v2i_d __attribute__((ext_vector_type(2)));
LSMX_DEV v2i_d ds_read_tr16x4(const uint8_t *p) {
    const v4s_d v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_d *)(p));
    return __builtin_bit_cast(v2i_d, v);
}

// BNC: B arrives as the reference passes it, [K, N] with N contiguous (row
// stride ldb elements), instead of K-contiguous Bt [N, K].  A stage of B is
// then 64 K-rows of 512 bytes (256 columns); a DMA instruction carries two
// rows, LDS position p of row r holding source chunk p ^ 4 (r & 3) (the 4
// rows a half-wave reads at once land in 4 different 64-byte windows of the
// 256-byte bank span), and each B fragment is two transposing reads of 4 K
// values.
template <int DT, int MODE, bool BNC = false>
__global__ __launch_bounds__(dr::NT, 1) void gemm_dense_ring_kernel(DenseArgs g) {
    using namespace dr;
    constexpr int P = MODE == 2 ? 2 : 1;      // GEMM problems
    constexpr int KC = MODE == 1 ? 2 : 1;     // products per tile (MODE 1: A0.B0 and A1.B1, alternating)
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][TILE_B];
    __shared__ __attribute__((aligned(16))) uint8_t sB[S][TILE_B];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int total = P * tiles;
    const int my_tiles = (total - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nkh = (int)(g.K * 2 / BKB);     // stages per product
    const int nk = KC * nkh;                  // stages per tile

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 31, half = lane >> 5;
    const int rowA0 = wm * (TM * 32) + frow, rowB0 = wn * (TN * 32) + frow;

    // ---- DMA addressing (loader waves): data load i of this lane reads row
    // (i*NLW + wave)*RPI + lane/CPR of the refill tile, byte offset off0 + i*step.
    const int64_t lda_b = g.lda * 2, ldb_b = g.ldb * 2;
    const int drow0 = wave * RPI + lane / CPR;
    const uint32_t offA0 = (uint32_t)(drow0 * lda_b + ((lane % CPR) ^ swz(drow0)) * 16);
    // BNC: load i of this lane reads K-row 2 (i*NLW + wave) + lane/32 of the
    // stage, chunk (lane % 32) ^ 4 (row & 3) (row & 3 does not depend on i)
    const int brow0 = 2 * wave + (lane >> 5);
    const uint32_t offB0 = BNC ? (uint32_t)(brow0 * ldb_b + (((lane & 31) ^ (4 * (brow0 & 3))) << 4))
                               : (uint32_t)(drow0 * ldb_b + ((lane % CPR) ^ swz(drow0)) * 16);
    const uint32_t stepA = (uint32_t)(NLW * RPI * lda_b);
    const uint32_t stepB = BNC ? (uint32_t)(2 * NLW * ldb_b) : (uint32_t)(NLW * RPI * ldb_b);

    // Tile id -> (problem, tile row, tile column).  Workgroup ids reach the 8
    // XCDs round-robin; the remap gives each XCD a contiguous run of ids, in
    // which the two problems of MODE 2 alternate, and groups of GROUP_M tile
    // rows keep the shared panels in that XCD's L2.
    static_assert(GROUP_M <= 4, "tile_coords divides by group heights up to 4");
    const TileMap tmap = make_tile_map(tiles_m, tiles_n, GROUP_M);
    auto tile_of = [&](int ti, int &p, int64_t &m0, int64_t &n0) __attribute__((always_inline)) {
        int id = (int)blockIdx.x + imax(0, imin(ti, my_tiles - 1)) * (int)gridDim.x;
        if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
        p = P == 2 ? (id & 1) : 0;
        int tm, tn;
        group_coords(P == 2 ? id >> 1 : id, tmap, tm, tn);
        m0 = (int64_t)tm * BM;
        n0 = (int64_t)tn * BN;
    };

    // Refill panels of the refill tile: first byte and byte count of the A
    // and B rows for each K half.  Wave-uniform; set once per tile phase.
    const uint8_t *pa[KC], *pb[KC];
    int64_t na = 0, nb = 0;
    auto set_refill_tile = [&](int ti) __attribute__((always_inline)) {
        int p;
        int64_t m0, n0;
        tile_of(ti, p, m0, n0);
#pragma unroll
        for (int h = 0; h < KC; ++h) {
            const bool second = (P == 2 && p == 1) || (KC == 2 && h == 1);
            pa[h] = (second ? g.a1 : g.a0) + m0 * lda_b;
            pb[h] = (second ? g.b1 : g.b0) + (BNC ? n0 * 2 : n0 * ldb_b);
        }
        na = min(g.M - m0, (int64_t)BM) * lda_b;
        // BNC: to the last column of the last K-row; columns past N in other
        // rows read the next row's values, whose products only reach outputs
        // that are not stored
        nb = BNC ? (g.K - 1) * ldb_b + (g.N - n0) * 2 : min(g.N - n0, (int64_t)BN) * ldb_b;
    };
    v4i_rsrc rsA, rsB;
    // descriptors of stage kt of the refill tile, in two parts.  MODE 1
    // alternates the two products every 64-deep K block, as the reference's
    // loop does (dual_gemm.py:59-61): stage kt is K block kt/2 of A0.B0
    // (kt even) or of A1.B1 (kt odd).
    auto make_desc = [&](int part, int kt) __attribute__((always_inline)) {
        const int h = KC == 2 ? (kt & 1) : 0;
        const int64_t ko = (int64_t)(KC == 2 ? kt >> 1 : kt) * BKB;
        if (part == 0) rsA = buf_rsrc((h ? pa[KC - 1] : pa[0]) + ko, (uint64_t)(na - ko));
        else if constexpr (BNC) {
            const int64_t kr = (int64_t)(KC == 2 ? kt >> 1 : kt) * 64 * ldb_b;   // 64 K-rows per stage
            rsB = buf_rsrc((h ? pb[KC - 1] : pb[0]) + kr, (uint64_t)(nb - kr));
        } else rsB = buf_rsrc((h ? pb[KC - 1] : pb[0]) + ko, (uint64_t)(nb - ko));
    };
    auto issue_op = [&](int s, int q) __attribute__((always_inline)) {
        const int i = q >> 1;
        const uint32_t m0 = lds_u32((q & 1) ? &sB[0][0] : &sA[0][0]) + s * TILE_B + (i * NLW + wave) * 1024;
        if ((q & 1) == 0) dma_x4(offA0 + i * stepA, rsA, m0);
        else dma_x4(offB0 + i * stepB, rsB, m0);
    };

    // K-step st: lane half h supplies 16-byte chunk 4h + st of its row (A and
    // B alike, so the sum is unchanged)
    // BNC fragment reads: lane (group g = lane/16, j = lane % 16) of B tile
    // jt at K-step st addresses row 8 (4 half + st) + j/4 (+ 4 for the second
    // read) and columns wn*128 + jt*32 + 16 (g & 1) + 4 (j & 3) .. + 3, i.e.
    // chunk wn*16 + jt*4 + cx, cx = 2 (g & 1) + (j & 3) / 2, which the row's
    // swizzle 4 (j/4) moves to wn*16 + (jt ^ j/4)*4 + cx; all but st and the
    // read is per lane (one offset per jt)
    const int bj = lane & 15, brs = bj >> 2;
    const uint32_t bl = (uint32_t)(half * (32 * 512) + brs * 512 + ((2 * ((lane >> 4) & 1) + ((bj & 3) >> 1)) << 4) +
                                   (bj & 1) * 8 + wn * (TN * 64));
    uint32_t bjo[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) bjo[j] = bl + (uint32_t)(((j ^ brs) & 3) << 6);
    auto read_frag = [&](int s, int st, int q, v4i_d (&fa)[TM], v4i_d (&fb)[TN]) __attribute__((always_inline)) {
        if constexpr (BNC) {
            if (q >= TM) {
                const uint8_t *p = sB[s] + bjo[q - TM] + st * 4096;
                const v2i_d lo = ds_read_tr16x4(p), hi = ds_read_tr16x4(p + 4 * 512);
                fb[q - TM] = v4i_d{lo.x, lo.y, hi.x, hi.y};
                return;
            }
        }
        const int c = 4 * half + st;
        const int r = q < TM ? rowA0 + q * 32 : rowB0 + (q - TM) * 32;
        const uint8_t *base = q < TM ? sA[s] : sB[s];
        const u32x4 v = *reinterpret_cast<const u32x4 *>(base + r * BKB + ((c ^ swz(r)) << 4));
        const v4i_d f = v4i_d{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
        if (q < TM) fa[q] = f;
        else fb[q - TM] = f;
    };

    const bool vec_c = ((reinterpret_cast<uintptr_t>(g.c0) & 15) == 0) &&
                       (P == 1 || (reinterpret_cast<uintptr_t>(g.c1) & 15) == 0) && g.ldc % 4 == 0 &&
                       g.ldc < ((int64_t)1 << 25);
    const int qa = S / nk, ra = S % nk;

    auto body = [&](auto loader_c) __attribute__((always_inline)) {
        constexpr bool LOADER = decltype(loader_c)::value;
        v16f_d acc[TM][TN];
        v4i_d fa[3][TM], fb[3][TN];

        // ---- prologue: fill the ring, publish stage 0, read its step-0 fragments
        if constexpr (LOADER) {
            int cur = -1;
#pragma unroll
            for (int p = 0; p < S; ++p) {
                const int ti = stage_tile_iter(p, nk, my_tiles);
                if (ti != cur) {
                    set_refill_tile(ti);
                    cur = ti;
                }
                make_desc(0, p % nk);
                make_desc(1, p % nk);
#pragma unroll
                for (int q = 0; q < L; ++q) issue_op(p, q);
            }
        }
        wait_vm_barrier<(S - 1) * L>();
#pragma unroll
        for (int q = 0; q < NRD; ++q) read_frag(0, 0, q, fa[0], fb[0]);

        // Stage u + S refills slot u % S: stage kt of tile iteration ti
        // refills stage kt + ra of tile ti + qa while kt + ra < nk (phase A)
        // and stage kt + ra - nk of tile ti + qa + 1 after (phase B).
        int u = 0;
        for (int ti = 0; ti < my_tiles; ++ti) {
            if constexpr (LOADER) set_refill_tile(ti + qa);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

            auto run_stage = [&](const int rk, auto slot_c) __attribute__((always_inline)) {
                constexpr int s = decltype(slot_c)::value, sn = (s + 1) % S;
                constexpr int BUF[4] = {0, 1, 2, 0};
                constexpr int LH = L / 2, OPH = (LH + NMF - 1) / NMF, RP1 = (2 * NRD + NMF - 1) / NMF;
#pragma unroll
                for (int st = 0; st < KS; ++st) {
                    if (st == 2) {
                        // this wave's reads of slot s are complete; once all
                        // waves pass the barrier slot s is free and stage u+1
                        // has landed
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        wait_vm_barrier<(S - 2) * L>();
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int idx = 0; idx < NMF; ++idx) {
                        const int i = idx / TN, j = idx % TN;
                        acc[i][j] = mfma_dense16<DT>(fa[BUF[st]][i], fb[BUF[st]][j], acc[i][j]);
                        if (st == 0) {
                            if (LOADER && idx < 2) {
                                // the refill stage's descriptors, after the
                                // first MFMAs; the empty asm keeps the IR
                                // optimizer from hoisting them above the fence
                                __builtin_amdgcn_sched_barrier(0);
                                int k = __builtin_amdgcn_readfirstlane(rk);
                                asm volatile("" : "+s"(k));
                                make_desc(idx, k);
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
                        } else {
#pragma unroll
                            for (int o = LH + idx * OPH; o < LH + (idx + 1) * OPH; ++o)
                                if (LOADER && o < L) issue_op(s, o);
                            if (idx < NRD) read_frag(sn, 0, idx, fa[1], fb[1]);
                        }
                        // pin this slot's LDS reads here (the MFMA is a pure
                        // intrinsic: without a memory clobber later reads
                        // would be hoisted and all fragments kept live)
                        asm volatile("" ::: "memory");
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i) fa[0][i] = fa[1][i];
#pragma unroll
                for (int j = 0; j < TN; ++j) fb[0][j] = fb[1][j];
            };
            auto run_range = [&](int kt0, int kt1, int rk_off) __attribute__((always_inline)) {
                int kt = kt0;
                if (kt < kt1 && (u & 1)) {
                    run_stage(kt + rk_off, DrSlot<1>{});
                    ++kt, ++u;
                }
                for (; kt + 1 < kt1; kt += 2) {
                    run_stage(kt + rk_off, DrSlot<0>{});
                    ++u;
                    run_stage(kt + 1 + rk_off, DrSlot<1>{});
                    ++u;
                }
                if (kt < kt1) {
                    run_stage(kt + rk_off, DrSlot<0>{});
                    ++u;
                }
            };
            run_range(0, nk - ra, ra);
            if constexpr (LOADER) set_refill_tile(ti + qa + 1);
            run_range(nk - ra, nk, ra - nk);

            // ---- epilogue: acc element e of tile (i, j) sits at row
            //      i*32 + 8*(e/4) + 4*half + e%4, column j*32 + frow; a 4x4
            //      transpose inside each quad gives every lane 4 columns
            int p;
            int64_t m0, n0;
            tile_of(ti, p, m0, n0);
            float *c = reinterpret_cast<float *>(P == 2 && p == 1 ? g.c1 : g.c0);
            const int q = frow & 3;
            if (vec_c && m0 + BM <= g.M && n0 + BN <= g.N) {
                const float *cw = c + (m0 + wm * (TM * 32)) * g.ldc + n0 + wn * (TN * 32);
                const uint32_t loff = (uint32_t)((4 * half + q) * g.ldc + (frow & ~3));
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        float *crow = const_cast<float *>(cw) + (i * 32 + 8 * gq) * g.ldc;
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            float x[4] = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                          acc[i][j][4 * gq + 3]};
                            quad_transpose(x, q);
                            *reinterpret_cast<u32x4 *>(crow + loff + j * 32) =
                                u32x4{f2u(x[0]), f2u(x[1]), f2u(x[2]), f2u(x[3])};
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
                            // all four lanes of a quad take part in the exchanges
                            quad_transpose(x, q);
                            const int64_t row = m0 + wm * (TM * 32) + i * 32 + 8 * gq + 4 * half + q;
                            const int64_t col = n0 + wn * (TN * 32) + j * 32 + (frow & ~3);
                            if (row < g.M)
#pragma unroll
                                for (int cc = 0; cc < 4; ++cc)
                                    if (col + cc < g.N) c[row * g.ldc + col + cc] = x[cc];
                        }
            }
        }
    };
    if (wave < NLW) body(DrLoader<true>{});
    else body(DrLoader<false>{});
    // no load may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

static int num_cus_dr() {
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

bool dense_ring_ok(const DenseArgs &g, int dtype) {
    // bf16 / fp16 operands, whole 64-element stages, no split-K, 16-byte
    // aligned operand rows, 32-bit DMA offsets
    return (dtype == LSMX_BF16 || dtype == LSMX_F16) && g.k_split == g.K && g.K % 64 == 0 && g.K > 0 &&
           g.lda % 8 == 0 && g.ldb % 8 == 0 && g.lda <= ((int64_t)1 << 22) && g.ldb <= ((int64_t)1 << 22) &&
           g.c_dtype == LSMX_F32;
}

hipError_t launch_gemm_dense_ring(const DenseArgs &g, int dtype, int mode, hipStream_t s) {
    const int tiles = (int)(((g.M + dr::BM - 1) / dr::BM) * ((g.N + dr::BN - 1) / dr::BN)) * (mode == 2 ? 2 : 1);
    const int grid = tiles < num_cus_dr() ? tiles : num_cus_dr();
#define LSMX_DR(DT, MD)                                                                                  \
    do {                                                                                             \
        if (g.b_nc) hipLaunchKernelGGL((gemm_dense_ring_kernel<DT, MD, true>), dim3(grid), dim3(dr::NT), 0, s, g); \
        else hipLaunchKernelGGL((gemm_dense_ring_kernel<DT, MD>), dim3(grid), dim3(dr::NT), 0, s, g);  \
    } while (0)
    if (dtype == LSMX_BF16) {
        if (mode == 0) LSMX_DR(LSMX_BF16, 0);
        else if (mode == 1) LSMX_DR(LSMX_BF16, 1);
        else LSMX_DR(LSMX_BF16, 2);
    } else {
        if (mode == 0) LSMX_DR(LSMX_F16, 0);
        else if (mode == 1) LSMX_DR(LSMX_F16, 1);
        else LSMX_DR(LSMX_F16, 2);
    }
#undef LSMX_DR
    return hipGetLastError();
}

}  // namespace lsmx
