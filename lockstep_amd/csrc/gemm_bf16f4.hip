// Weight-only bf16 x MXFP4 GEMM and its dual-batch form, for gfx950.
//
//   single:  C[m, n]  = sum_k A[m, k]  * deq(W)[n, k]
//   dual:    C0[m, n] = sum_k A0[m, k] * deq(W)[n, k],  C1 likewise with A1
//
// Semantics: the fake-quant forward of fp4_linear.py:40 with an unquantized
// activation (deq(W) = E2M1 value * 2^e, fp4.py:75-78), and dual_gemm.py:78-110
// _dual_separate_kernel used with one shared weight (train_step.py:52-53):
// two accumulators, one launch.  deq(W) is exact in bf16 (at most two
// significant bits times a power of two inside bf16's exponent range), so
// the products are exact and only fp32 accumulation rounds.
//
// Dequantization happens in registers: each lane pulls the 16 packed bytes
// (32 codes, one MX block) of its weight column for the stage from LDS and
// turns them into 32 bf16 values with v_cvt_scalef32_pk_bf16_fp4, which
// multiplies by the block scale on the way.  The MFMA is
// v_mfma_f32_32x32x16_bf16.  Its K positions are assigned so that, across
// the four K=16 steps of a 64-wide stage, lane half h covers block h of the
// stage: the A operand for step s reads A[row][32h + 8s .. +8].  A and W use
// the same assignment, so the sum is unchanged.
//
// Tiling: 256 "A rows" x 256 weight columns per workgroup of 4 waves (2 x 2),
// 128 x 128 per wave (4 x 4 MFMA tiles).  In dual mode the 256 A rows are
// 128 rows of A0 followed by the same 128 rows of A1: one weight tile in LDS
// feeds both batches and is read from memory once per stage.
#include "lsmx_dma.h"
#include "lsmx_store.h"
#include "lsmx_internal.h"
#include "lsmx_sched.h"

namespace lsmx {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace w4 {
constexpr int BK = 64;         // K per stage
constexpr int A_ROW_B = BK * 2;    // 128 bytes of bf16 per A row per stage
constexpr int W_ROW_B = BK / 2;    // 32 bytes of codes per W row per stage
constexpr int NT = 256;
constexpr int GROUP_M = 4;
}  // namespace w4

LSMX_DEV int a_swz(int row) { return (row ^ (row >> 3)) & 7; }

LSMX_DEV uint32_t bf16_rne_w(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

template <int CT>
LSMX_DEV void store_cw(void *c, int64_t idx, float v) {
    if constexpr (CT == LSMX_F32) reinterpret_cast<float *>(c)[idx] = v;
    else if constexpr (CT == LSMX_BF16) reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)bf16_rne_w(v);
    else reinterpret_cast<_Float16 *>(c)[idx] = (_Float16)v;
}

LSMX_DEV void tile_coords_w(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
    const int per_group = w4::GROUP_M * tiles_n;
    const int group = pid / per_group;
    const int first_m = group * w4::GROUP_M;
    const int gsz = min(tiles_m - first_m, w4::GROUP_M);
    const int in_group = pid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

template <bool SF32>
LSMX_DEV uint32_t load_scale2(const void *s, int64_t off) {
    // 2 consecutive block scales as E8M0 bytes in the low 16 bits
    if constexpr (SF32) {
        const u32x2 v = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const float *>(s) + off);
        return f32_scale_e8m0(v[0]) | (f32_scale_e8m0(v[1]) << 8);
    } else {
        return *reinterpret_cast<const uint16_t *>(reinterpret_cast<const uint8_t *>(s) + off);
    }
}

LSMX_DEV float e8m0_scale_f32(uint32_t e) {
    return e == 0u ? u2f(0x00400000u) : (e == 255u ? u2f(0x7FC00000u) : u2f(e << 23));
}

// BR A rows (all batches) x BN weight columns per workgroup of 4 waves in a
// 2 x 2 grid: 256 x 256 for large M; 128 x 128 or 128 x 64 (several
// workgroups per CU) when larger tiles would leave CUs idle.
template <int NB, bool SF32, int CT, int BR, int BN>
__global__ __launch_bounds__(w4::NT, BR == 256 ? 1 : 2) void gemm_bf16f4_kernel(GemmArgs g) {
    using namespace w4;
    constexpr int RPB = BR / NB;           // A rows per batch per workgroup
    constexpr int RT = BR / 64 / NB;       // row tiles per batch per wave
    constexpr int WT = BN / 2;             // weight columns per wave
    constexpr int CTW = WT / 32;           // column tiles per wave
    constexpr int XA = BR * A_ROW_B / 16 / NT;   // A chunks per thread per stage
    constexpr int XW = BN * W_ROW_B / 16 / NT;   // W chunks per thread per stage (0 for BN = 64: threads
                                                 // t and t + 128 load the same chunk)
    static_assert(RT >= 1 && CTW >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BR * A_ROW_B];   // 2 x 32 KiB
    __shared__ __attribute__((aligned(16))) uint8_t sW[2][BN * W_ROW_B];   // 2 x 8 KiB, [half][col][16B]
    __shared__ uint32_t sS[2][BN];

    const int tiles_m = (int)((g.M + RPB - 1) / RPB), tiles_n = (int)((g.N + BN - 1) / BN);
    int tm, tn;
    tile_coords_w(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * RPB, n0 = (int64_t)tn * BN;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (int)(g.K / BK);

    // A staging: XA chunks of 16 B per thread; row = q >> 3, chunk = q & 7
    const uint8_t *ga[XA];
    int a_off[XA];
#pragma unroll
    for (int i = 0; i < XA; ++i) {
        const int q = i * NT + t;
        const int row = q >> 3, c = q & 7;
        const int b = row / RPB, r = row % RPB;
        const int64_t am = min(m0 + r, g.M - 1);
        const uint8_t *base = (NB == 2 && b == 1) ? g.a1 : g.a;
        ga[i] = base + am * g.lda * 2 + c * 16;
        a_off[i] = row * A_ROW_B + ((c ^ a_swz(row)) << 4);
    }
    // W staging: 2 chunks (one per block half) per weight row; with BN = 128
    // the 256 threads cover the 256 chunks once, with BN = 64 twice
    constexpr int XW1 = XW > 0 ? XW : 1;
    const uint8_t *gw[XW1];
    int w_off[XW1];
#pragma unroll
    for (int i = 0; i < XW1; ++i) {
        const int q = (i * NT + t) % (2 * BN);
        const int row = q >> 1, h = q & 1;
        const int64_t wn_ = min(n0 + row, g.N - 1);
        gw[i] = g.b + wn_ * g.ldb + h * 16;
        w_off[i] = h * (BN * 16) + row * 16;
    }
    // thread t < BN stages the scales of weight column t (threads past BN
    // load a clamped column and store nothing)
    const int64_t s_row = min(n0 + (t % BN), g.N - 1) * g.ld_sb;

    u32x4 ra[XA], rw[XW1];
    uint32_t rs;
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < XA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(ga[i] + (int64_t)kt * A_ROW_B);
#pragma unroll
        for (int i = 0; i < XW1; ++i) rw[i] = *reinterpret_cast<const u32x4 *>(gw[i] + (int64_t)kt * W_ROW_B);
        rs = load_scale2<SF32>(g.sb, s_row + (int64_t)kt * 2);
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XA; ++i) *reinterpret_cast<u32x4 *>(&sA[buf][a_off[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < XW1; ++i) *reinterpret_cast<u32x4 *>(&sW[buf][w_off[i]]) = rw[i];
        if (BN == NT || t < BN) sS[buf][t % BN] = rs;
    };

    v16f acc[NB][RT][CTW];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CTW; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[b][i][j][e] = 0.0f;

    const int frow = lane & 31, half = lane >> 5;

    gload(0);
    swrite(0);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);

        // dequantize this wave's CTW weight column tiles for the stage:
        // 32 codes of block `half` -> 32 bf16, 8 per K=16 step.
        v8bf fw[CTW][4];  // [col tile][step]
#pragma unroll
        for (int j = 0; j < CTW; ++j) {
            const int col = wn * WT + j * 32 + frow;
            const u32x4 pw = *reinterpret_cast<const u32x4 *>(&sW[buf][half * (BN * 16) + col * 16]);
            const float sc = e8m0_scale_f32((sS[buf][col] >> (8 * half)) & 0xFF);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw[s], sc, 0);
                const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw[s], sc, 1);
                const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw[s], sc, 2);
                const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw[s], sc, 3);
                fw[j][s] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = half * 4 + s;  // 16-byte chunk: A[row][32h + 8s .. +8]
            v8bf fa[NB][RT];
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < RT; ++i) {
                    const int row = b * RPB + wm * (RT * 32) + i * 32 + frow;
                    fa[b][i] = *reinterpret_cast<const v8bf *>(&sA[buf][row * A_ROW_B + ((c ^ a_swz(row)) << 4)]);
                }
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < RT; ++i)
#pragma unroll
                    for (int j = 0; j < CTW; ++j)
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[b][i], fw[j][s], acc[b][i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) swrite(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int b = 0; b < NB; ++b) {
        void *cb = (NB == 2 && b == 1) ? g.c1 : g.c;
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CTW; ++j) {
                const int64_t col = n0 + wn * WT + j * 32 + frow;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t row = m0 + wm * (RT * 32) + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                    if (row < g.M && col < g.N) store_cw<CT>(cb, row * g.ldc + col, acc[b][i][j][e]);
                }
            }
    }
}

// ------------------------------------------------------------------ fp32 / fp16 activations
// Weight-only GEMM with wider activations: Y = X . deq(W)^T for X in fp32
// (the fake-quant forward of fp4_linear.py:40 with an unquantized fp32
// X, deq(W) of fp4.py:75-78) or fp16.  Each activation is
// split exactly into NTERM bf16 terms, each the bf16 truncation of what the
// terms before it leave,
//     hi = tr(x),  mid = tr(x - hi),  lo = x - hi - mid     (fp32: NTERM = 3)
// (x has 24 significant bits and each term holds 8; every subtraction and
// the last term are exact; fp16's 11 bits need hi and mid only), and each
// term runs through v_mfma_f32_32x32x16_bf16 against the exact bf16 weight.
// The products are exact in fp32, so only the fp32 accumulation rounds, as
// in an fp32 matmul.  Per K-step the terms are added hi, mid, lo.
// Tile: BR rows x BN weight columns per workgroup of 4 waves, 64-deep K
// stages, the widest tile whose grid still fills the CUs: 64 x 128 or
// 64 x 64 (2 x 2 waves of 32 x BN/2), or for small outputs 32 x 32 with the
// 4 waves splitting each stage's four 16-deep K-steps (cfg1's 256 x 1024
// output is 256 such workgroups); their partial tiles are added in wave
// order through LDS at the end.  The split happens once per element, as
// the activations are staged: each thread loads its 16-byte chunks two
// stages ahead into VGPRs and, after a stage's MFMAs, writes their terms to
// a double-buffered LDS tile of NTERM bf16 planes (128 bytes per row and
// plane per stage).  The K positions are those of the bf16 kernel above: at
// K-step s lane half h supplies X[row][32h + 8s .. +8] and codes 8s .. 8s+7
// of the weight's block h of the stage.
static int num_cus_w();

namespace xf {
constexpr int BK = 64, NT = 256;
constexpr int ROW_B = BK * 2;     // bytes per row of one bf16 term plane per stage
}  // namespace xf

// The bf16 terms of x (fp32 bits xb): hi = tr(x), mid = tr(x - hi),
// lo = tr(x - hi - mid), exact for |x| >= 2^-110 (there lo is at least a
// bf16 subnormal's ulp); Inf and NaN pass through hi alone (a NaN whose
// payload lies in the low 16 bits keeps a quiet bit).
LSMX_DEV void split_bf16_terms(uint32_t xb, uint32_t &hb, uint32_t &mb, uint32_t &lb) {
    const bool special = (xb & 0x7F800000u) == 0x7F800000u;
    hb = (xb >> 16) | (special && (xb & 0xFFFFu) ? 0x40u : 0u);
    const float r1 = special ? 0.0f : u2f(xb) - u2f(hb << 16);
    mb = f2u(r1) >> 16;
    lb = f2u(r1 - u2f(mb << 16)) >> 16;
}

template <int AT, bool SF32, int CT, int BR, int BN, int KS, int KG = 1>
__global__ __launch_bounds__(xf::NT * KG, KG == 1 ? 2 : 4) void gemm_xf4_kernel(GemmArgs g) {
    using namespace xf;
    static_assert(KG == 1 || KS == 4, "K groups split the 32 x 32 tile form");
    constexpr int ES = AT == LSMX_F32 ? 4 : 2;        // activation bytes
    constexpr int NTERM = AT == LSMX_F32 ? 3 : 2;     // bf16 terms per activation
    constexpr int WM = KS == 1 ? 2 : 1, WN = KS == 1 ? 2 : 1;  // wave grid over the tile
    static_assert(WM * WN * KS == 4 && BR == 32 * WM, "4 waves: 2 x 2 tiles, or one tile split 4 ways along K");
    constexpr int CTW = BN / 32 / WN;                 // 32-column MFMA tiles per wave
    constexpr int EPC = 16 / ES;                      // activations per 16-byte source chunk (4 or 8)
    constexpr int CPR = BK / EPC;                     // source chunks per row per stage (16 or 8)
    constexpr int XA = BR * CPR / NT;                 // source chunks per thread per stage (4 or 2)
    constexpr int WCH = BN * 2;                       // 16-byte W chunks per stage
    // K group kg's activation rows are rows kg * BR .. of each term plane,
    // its W chunks and scales the kg-th part of each buffer, so that every
    // LDS address is a per-lane offset (which includes kg) plus an immediate
    __shared__ __attribute__((aligned(16))) uint8_t sX[2][NTERM][KG * BR * ROW_B];  // 2 x 3 x 8 KiB per group (fp32)
    __shared__ __attribute__((aligned(16))) uint8_t sW[2][KG * BN * 32];            // [group][half][col][16 B]
    __shared__ uint32_t sS[2][KG * BN];

    const int tiles_m = (int)((g.M + BR - 1) / BR), tiles_n = (int)((g.N + BN - 1) / BN);
    int tm, tn;
    tile_coords_w(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BR, n0 = (int64_t)tn * BN;
    // K group kg (4 waves) runs stages kg * nkg .. + nkg - 1 on its own LDS
    // buffers; the groups meet only at the workgroup barriers, which they
    // reach in step
    const int kg = __builtin_amdgcn_readfirstlane((int)threadIdx.x / NT);
    const int t = (int)threadIdx.x % NT, lane = t & 63, wave = t >> 6;
    const int wm = KS == 1 ? wave >> 1 : 0, wn = KS == 1 ? wave & 1 : 0;
    const int wk = KS == 1 ? 0 : wave;                // this wave's K-steps: wk, wk + KS, ... of each stage
    const int frow = lane & 31, half = lane >> 5;
    const int nk = (int)(g.K / BK) / KG;              // stages of this K group (the launcher keeps KG | K / BK)
    const int64_t kg0 = (int64_t)kg * nk;             // its first stage

    // source chunk q = i * NT + t: row q / CPR, activations EPC * (q % CPR)
    // .. +EPC, i.e. 2 * EPC bytes of each term plane at byte 2 * EPC * (q %
    // CPR) of the row, whose 16-byte chunk sits at chunk ^ a_swz(row)
    const uint8_t *ga[XA];
    int x_off[XA];
#pragma unroll
    for (int i = 0; i < XA; ++i) {
        const int q = i * NT + t;
        const int row = q / CPR, c = q % CPR, lrow = kg * BR + row;
        ga[i] = g.a + min(m0 + row, g.M - 1) * g.lda * ES + c * 16;
        const int pb = 2 * EPC * c;  // byte in the plane row
        x_off[i] = lrow * ROW_B + (((pb >> 4) ^ a_swz(lrow)) << 4) + (pb & 15);
    }
    const int wq = t < WCH ? t : 0;  // W chunk of this thread (threads >= WCH load none)
    const uint8_t *gw = g.b + min(n0 + (wq >> 1), g.N - 1) * g.ldb + (wq & 1) * 16;
    const int w_off = (2 * kg + (wq & 1)) * (BN * 16) + (wq >> 1) * 16;
    const int64_t s_row = min(n0 + (t % BN), g.N - 1) * g.ld_sb;

    // two register slots of staged loads: stage k lives in slot k % 2 from
    // its load (issued two stages ahead) until its terms go to LDS
    u32x4 ra[2][XA], rw[2];
    uint32_t rs[2];
    auto gload = [&](int kt, auto slot) {
        constexpr int q = decltype(slot)::value;
#pragma unroll
        for (int i = 0; i < XA; ++i) ra[q][i] = *reinterpret_cast<const u32x4 *>(ga[i] + (kg0 + kt) * BK * ES);
        if (t < WCH) rw[q] = *reinterpret_cast<const u32x4 *>(gw + (kg0 + kt) * 32);
        rs[q] = load_scale2<SF32>(g.sb, s_row + (kg0 + kt) * 2);
    };
    auto swrite = [&](int buf, auto slot) {
        constexpr int q = decltype(slot)::value;
#pragma unroll
        for (int i = 0; i < XA; ++i) {
            if constexpr (ES == 4) {
                uint32_t tb[3][4];
#pragma unroll
                for (int e = 0; e < 4; ++e) split_bf16_terms(ra[q][i][e], tb[0][e], tb[1][e], tb[2][e]);
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    *reinterpret_cast<u32x2 *>(&sX[buf][p][x_off[i]]) =
                        u32x2{tb[p][0] | (tb[p][1] << 16), tb[p][2] | (tb[p][3] << 16)};
            } else {
                uint32_t hw[4], mw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint32_t h0, m0_, l0, h1, m1, l1;
                    split_bf16_terms(f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(ra[q][i][e] & 0xFFFFu))), h0, m0_, l0);
                    split_bf16_terms(f2u((float)__builtin_bit_cast(_Float16, (uint16_t)(ra[q][i][e] >> 16))), h1, m1, l1);
                    hw[e] = h0 | (h1 << 16);
                    mw[e] = m0_ | (m1 << 16);
                }
                *reinterpret_cast<u32x4 *>(&sX[buf][0][x_off[i]]) = u32x4{hw[0], hw[1], hw[2], hw[3]};
                *reinterpret_cast<u32x4 *>(&sX[buf][1][x_off[i]]) = u32x4{mw[0], mw[1], mw[2], mw[3]};
            }
        }
        if (t < WCH) *reinterpret_cast<u32x4 *>(&sW[buf][w_off]) = rw[q];
        if (t < BN) sS[buf][kg * BN + t] = rs[q];
    };

    v16f acc[CTW];
#pragma unroll
    for (int j = 0; j < CTW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

    // stage kt from LDS buffer kt % 2; stage kt + 1 (in slot `slot`) goes
    // to the other buffer and stage kt + 3 is loaded into the freed slot
    auto step = [&](int kt, auto slot) {
        const int buf = kt & 1;
        constexpr int NS = 4 / KS;                    // K-steps of 16 per wave per stage
        v8bf fw[CTW][NS];
#pragma unroll
        for (int j = 0; j < CTW; ++j) {
            const int col = wn * (BN / WN) + j * 32 + frow;
            const u32x4 pw = *reinterpret_cast<const u32x4 *>(&sW[buf][(2 * kg + half) * (BN * 16) + col * 16]);
            const float sc = e8m0_scale_f32((sS[buf][kg * BN + col] >> (8 * half)) & 0xFF);
#pragma unroll
            for (int ss = 0; ss < NS; ++ss) {
                const uint32_t cw = KS == 1 ? pw[ss] : pw[wk];
                const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 0);
                const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 1);
                const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 2);
                const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 3);
                fw[j][ss] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
            }
        }
        const int row = kg * BR + wm * 32 + frow;
#pragma unroll
        for (int ss = 0; ss < NS; ++ss) {
            const int s = wk + KS * ss;
            v8bf fa[NTERM];
#pragma unroll
            for (int p = 0; p < NTERM; ++p)
                fa[p] = *reinterpret_cast<const v8bf *>(&sX[buf][p][row * ROW_B + (((4 * half + s) ^ a_swz(row)) << 4)]);
#pragma unroll
            for (int j = 0; j < CTW; ++j)
#pragma unroll
                for (int p = 0; p < NTERM; ++p)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[p], fw[j][ss], acc[j], 0, 0, 0);
        }
        if (kt + 1 < nk) swrite(buf ^ 1, slot);
        if (kt + 3 < nk) gload(kt + 3, slot);
        __syncthreads();
    };
    constexpr SlotC<0> S0{};
    constexpr SlotC<1> S1{};
    gload(0, S0);
    swrite(0, S0);
    if (1 < nk) gload(1, S1);
    if (2 < nk) gload(2, S0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
        step(kt, S1);                   // stage kt + 1 sits in slot 1
        if (kt + 1 < nk) step(kt + 1, S0);
    }

    if constexpr (KS > 1) {
        // waves 1 .. KG * KS - 1 (wave wk of K group kg is kg * KS + wk)
        // hand their partial tiles to wave 0 through LDS (the staging planes
        // are free after the last barrier), which adds them in that order
        constexpr int NW = KG * KS;
        const int gwv = kg * KS + wk;
        float *red = reinterpret_cast<float *>(&sX[0][0][0]);
        static_assert(CTW == 1 && (NW - 1) * 16 * 64 * 4 <= (int)sizeof(sX), "reduction buffer");
        if (gwv > 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) red[((gwv - 1) * 16 + e) * 64 + lane] = acc[0][e];
        }
        __syncthreads();
        if (gwv > 0) return;
        // one partial tile at a time (unrolled over 15 tiles, the compiler
        // would issue all 240 reads at once and spill)
#pragma nounroll
        for (int w2 = 0; w2 < NW - 1; ++w2)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[0][e] += red[(w2 * 16 + e) * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < CTW; ++j) {
        const int64_t col = n0 + wn * (BN / WN) + j * 32 + frow;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t row = m0 + wm * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
            if (row < g.M && col < g.N) store_cw<CT>(g.c, row * g.ldc + col, acc[j][e]);
        }
    }
}

hipError_t launch_gemm_xf4(const GemmArgs &g, int a_dtype, hipStream_t s) {
    // the widest tile whose grid still fills the CUs: 64 x 128, 64 x 64, or
    // 32 x 32 tiles split four ways along K
    auto tiles = [&](int br, int bn) { return ((g.M + br - 1) / br) * ((g.N + bn - 1) / bn); };
    const int cus = num_cus_w();
    // the 32 x 32 form: 4 K groups of 4 waves when the stage count allows
    // (each group runs a quarter of the stages; cfg1's 16 dependent stages
    // become 4)
    const int shape = tiles(64, 128) >= cus ? 0 : (tiles(64, 64) >= cus ? 1 : ((g.K / xf::BK) % 4 == 0 ? 3 : 2));
    const dim3 grid((unsigned)(shape == 0 ? tiles(64, 128) : shape == 1 ? tiles(64, 64) : tiles(32, 32))),
        blk(xf::NT), blk4(4 * xf::NT);
    const bool f = g.scale_fmt == LSMX_SCALE_F32;
#define LSMX_X(AT, F, CT)                                                                           \
    do {                                                                                            \
        if (shape == 0) hipLaunchKernelGGL((gemm_xf4_kernel<AT, F, CT, 64, 128, 1>), grid, blk, 0, s, g); \
        else if (shape == 1) hipLaunchKernelGGL((gemm_xf4_kernel<AT, F, CT, 64, 64, 1>), grid, blk, 0, s, g); \
        else if (shape == 3) hipLaunchKernelGGL((gemm_xf4_kernel<AT, F, CT, 32, 32, 4, 4>), grid, blk4, 0, s, g); \
        else hipLaunchKernelGGL((gemm_xf4_kernel<AT, F, CT, 32, 32, 4>), grid, blk, 0, s, g);       \
    } while (0)
#define LSMX_XC(AT, F)                                           \
    do {                                                         \
        if (g.c_dtype == LSMX_F32) LSMX_X(AT, F, LSMX_F32);      \
        else if (g.c_dtype == LSMX_BF16) LSMX_X(AT, F, LSMX_BF16); \
        else LSMX_X(AT, F, LSMX_F16);                            \
    } while (0)
    if (a_dtype == LSMX_F32) { if (f) LSMX_XC(LSMX_F32, true); else LSMX_XC(LSMX_F32, false); }
    else { if (f) LSMX_XC(LSMX_F16, true); else LSMX_XC(LSMX_F16, false); }
#undef LSMX_XC
#undef LSMX_X
    return hipGetLastError();
}

// ------------------------------------------------------------------ ring
// The large-M form: 256 "A rows" x 256 weight columns per workgroup of 8 waves
// (4 x 2, 64 x 128 per wave: two waves per SIMD, so one wave's MFMAs run
// while the other waits), a 3-slot LDS ring filled by direct-to-LDS loads
// (no VGPR staging), one barrier per 64-deep K stage.
//   - A stage is 128 bytes of every A row (64 bf16; 8 rows per load
//     instruction, chunk-swizzled) and 32 bytes of every W row (64 codes, two
//     MX blocks; 32 rows per load instruction).  Rows past the operand read
//     zeros through the buffer descriptor.
//   - At the barrier of stage u every wave has its own loads of stage u in
//     LDS and has finished stage u - 1, so the slot of stage u - 1 is free
//     and the loads of stage u + 2 go there, spread over the K-steps.
//     Stages past the end re-load the last stage (same slot pattern, no
//     branch), and the kernel waits for them before it exits.
//   - K positions: at K-step s lane half h supplies A[row][32h + 8s .. +8]
//     and the codes 8s .. 8s+7 of W's block h, so a lane dequantizes one
//     16-byte block per column tile per stage with one scale.
//   - A W load instruction covers 32 weight rows; its 1 KiB of LDS holds the
//     first 16-byte halves of those rows, then the second halves, so the 16
//     lanes a ds_read_b128 serves per cycle read 256 contiguous bytes.
//   - E8M0 block scales (row-major [N, K/32]) come 16 bytes per weight row =
//     8 stages at a time, into a 2-deep LDS buffer; the load for stages
//     8g .. 8g+7 is issued first in stage 8g - 2 (scale rows must be 16-byte
//     multiples: K % 512 == 0; fp32 scales use the VGPR-staged kernel).
namespace wr {
constexpr int BK = 64;
constexpr int NW = 8, NT = 64 * NW;
constexpr int A_ROW_B = BK * 2, W_ROW_B = BK / 2;
constexpr int GROUP_M = 4;
LSMX_DEV int swz(int row) { return (row >> 1) & 7; }
}  // namespace wr

// BR x BN tile (256 x 256 for large M; 128 x 64 and 128 x 128 for M of a few
// hundred rows, where a 256-row tile would leave most CUs idle and every CU
// streams all of A), S-slot ring.
// SPLITK: the workgroup takes K slice blockIdx % splits of its tile (g.k_split
// deep) and writes its fp32 partial tile to the workspace g.ws;
// splitk_reduce_kernel then adds the slices in slice order and stores C.
// WGM x (8 / WGM) waves: 4 x 2 (each wave a quarter of the rows and half of
// the columns) or, for 128-row tiles, 1 x 8 (each wave all rows and a 32-
// column strip, so every weight fragment is dequantized by one wave instead
// of four: the dequantization is VALU work that does not shrink with the
// tile's row count).
// NLW loader waves issue the stage loads (all 8, or waves 0-3 only: the two
// waves of a SIMD share its matrix core, the older one (0-3) wins issue
// arbitration and reaches the barrier first, so the younger one's
// instruction stream sets the stage's pace and is kept to LDS reads,
// dequantization and MFMAs).
template <bool V>
struct LoaderC {
    static constexpr bool value = V;
};
template <int NB, int CT, int BR, int BN, int S, bool SPLITK = false, int WGM = 4, int NLW = wr::NW>
__global__ __launch_bounds__(wr::NT, 1) void gemm_bf16f4_ring_kernel(GemmArgs g) {
    using namespace wr;
    constexpr int RPB = BR / NB;        // A rows per batch per workgroup
    constexpr int WGN = NW / WGM;
    constexpr int TM = BR / 32 / WGM, TN = BN / 32 / WGN;   // 32 x 32 tiles per wave
    static_assert(NB == 1 || TM * 32 <= RPB, "a wave's rows lie in one batch");
    constexpr int A_SLOT = BR * A_ROW_B, W_SLOT = BN * W_ROW_B;
    constexpr int XA = A_SLOT / 1024 / NLW;      // A load instructions per loader wave per stage
    constexpr int WW = BN / 32;                  // W load instructions per stage (32 rows each)
    constexpr int XWL = (WW + NLW - 1) / NLW;    // W loads per loader wave (some may be empty)
    constexpr int L = XA + XWL;                  // (scales: one more every 8 stages)
    constexpr int SWV = BN >= 64 ? BN / 64 : 1;  // distinct scale loads (64 rows each)
    static_assert(TM >= 1 && TN >= 1 && XA >= 1 && S >= 3 && (A_SLOT / 1024) % NLW == 0 && NLW <= NW, "tile");
    static_assert(NLW >= SWV, "every scale block needs a loader");
    // The scales of stages 8g+8 .. 8g+15 are issued first among stage 8g+6's
    // loads and first read right after the barrier of stage 8g+7 (4 slots) or
    // 8g+8 (3 slots); the wait at that barrier leaves (S - 3) L or (S - 2) L
    // loads outstanding, which covers the scale load only for these depths.
    static_assert(S == 3 || S == 4, "the scale prefetch distance assumes a 3- or 4-slot ring");
    __shared__ __attribute__((aligned(16))) uint8_t sA[S][A_SLOT];
    __shared__ __attribute__((aligned(16))) uint8_t sW[S][W_SLOT];
    __shared__ __attribute__((aligned(16))) uint8_t sS[2][BN * 16];   // [group & 1][row][16 scale bytes]
    // landing place of the loader waves' W loads past WW: they read nothing
    // (an empty buffer descriptor: every lane out of range) and write zeros
    // here, so that every loader counts the same loads
    __shared__ __attribute__((aligned(16))) uint8_t sNull[XWL * NLW > WW ? 1024 : 16];

    const int tiles_m = (int)((g.M + RPB - 1) / RPB), tiles_n = (int)((g.N + BN - 1) / BN);
    const int tile = SPLITK ? (int)blockIdx.x / g.splits : (int)blockIdx.x;
    const int split = SPLITK ? (int)blockIdx.x - tile * g.splits : 0;
    int tm, tn;
    tile_coords(tile, tiles_m, tiles_n, GROUP_M, tm, tn);
    const int64_t m0 = (int64_t)tm * RPB, n0 = (int64_t)tn * BN;
    // this workgroup's K range: [kb0, kb0 + kdepth)
    const int64_t kb0 = SPLITK ? (int64_t)split * g.k_split : 0, kdepth = SPLITK ? g.k_split : g.K;
    const int nk = (int)(kdepth / BK);

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int frow = lane & 31, half = lane >> 5;

    // ---- DMA addressing (loader waves).  A load i of loader w covers slot
    // rows (i*NLW + w)*8 .. +7: lane -> row + lane/8, LDS chunk lane%8 holding
    // source chunk (lane%8) ^ swz(row).  All 8 rows of one instruction lie in
    // one batch.
    const int64_t lda_b = g.lda * 2;
    const int arow_l = lane >> 3;
    // Per load: the first byte and byte count of its rows at K offset 0,
    // loop-invariant, so that a stage's descriptors cost a 64-bit add and
    // subtract each (the scalar unit is shared by the CU's 8 waves).
    uint32_t a_off[XA];
    const uint8_t *a_base[XA];
    uint64_t a_bytes[XA];
#pragma unroll
    for (int i = 0; i < XA; ++i) {
        const int r0 = (i * NLW + wave) * 8;           // first slot row, wave-uniform
        const int b = NB == 2 ? r0 / RPB : 0;
        const int rb = r0 - b * RPB;                    // row inside the batch tile
        const int row = r0 + arow_l;
        a_off[i] = (uint32_t)(arow_l * lda_b + (((lane & 7) ^ swz(row)) << 4));
        a_base[i] = (b ? g.a1 : g.a) + (m0 + rb) * lda_b + kb0 * 2;
        // rows left in the operand from this instruction's first row, at most 8
        const int64_t left = g.M - (m0 + rb), rows = left < 8 ? (left > 0 ? left : 0) : 8;
        a_bytes[i] = rows > 0 ? (uint64_t)((rows - 1) * lda_b + (g.K - kb0) * 2) : 0;
    }
    // W: load j of loader w covers slot rows (j*NLW + w)*32 .. +31 (when that
    // is below BN), lane -> row lane%32, 16-byte half lane/32
    const uint32_t w_off = (uint32_t)((lane & 31) * g.ldb + (lane >> 5) * 16);
    const uint8_t *w_base[XWL];
    uint64_t w_bytes[XWL];
    uint32_t w_lds[XWL], w_slot[XWL];
#pragma unroll
    for (int j = 0; j < XWL; ++j) {
        const int wi = j * NLW + wave;
        const bool real = wi < WW;
        w_base[j] = g.b + (n0 + (real ? wi : 0) * 32) * g.ldb + kb0 / 2;
        const int64_t left = real ? g.N - (n0 + wi * 32) : 0, rows = left < 32 ? (left > 0 ? left : 0) : 32;
        w_bytes[j] = rows > 0 ? (uint64_t)((rows - 1) * g.ldb + (g.K - kb0) / 2) : 0;
        w_lds[j] = real ? lds_u32(&sW[0][0]) + wi * 1024 : lds_u32(&sNull[0]);
        w_slot[j] = real ? W_SLOT : 0;
    }
    // scales: loader w loads 16 bytes of weight rows (w % SWV)*64 + lane
    // (loaders w and w + SWV write the same bytes, so every loader counts the
    // same loads)
    const int s_w = wave % SWV;
    const int64_t s_rows = g.N - n0;
    const uint8_t *s_base = reinterpret_cast<const uint8_t *>(g.sb) + n0 * g.ld_sb + kb0 / 32;
    const uint32_t s_off = (uint32_t)(((s_w * 64) + lane) * g.ld_sb);
    auto issue_scales = [&](int grp) __attribute__((always_inline)) {
        const int64_t ks = (int64_t)grp * 16;
        const int64_t rows = s_rows < BN ? s_rows : BN;
        const uint64_t bytes = (uint64_t)((rows - 1) * g.ld_sb + (g.K - kb0) / 32 - ks);
        dma_x4(s_off, buf_rsrc(s_base + ks, bytes), lds_u32(&sS[grp & 1][0]) + s_w * 1024);
    };

    auto issue = [&](int kt, int slot, int q) __attribute__((always_inline)) {
        const int64_t ko = (int64_t)kt * A_ROW_B;
        if (q < XA) {
            const uint64_t bytes = a_bytes[q] > 0 ? a_bytes[q] - (uint64_t)ko : 0;
            dma_x4(a_off[q], buf_rsrc(a_base[q] + ko, bytes),
                   lds_u32(&sA[0][0]) + slot * A_SLOT + (q * NLW + wave) * 1024);
        } else {
            const int j = q - XA;
            const int64_t kw = (int64_t)kt * W_ROW_B;
            const uint64_t bytes = w_bytes[j] > 0 ? w_bytes[j] - (uint64_t)kw : 0;
            dma_x4(w_off, buf_rsrc(w_base[j] + kw, bytes), w_lds[j] + slot * w_slot[j]);
        }
    };


    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    int rowA[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) rowA[i] = wm * (TM * 32) + i * 32 + frow;
    auto body = [&](auto loader_c) __attribute__((always_inline)) {
    constexpr bool LOADER = decltype(loader_c)::value;
    // prologue: scales of stages 0..7, stages 0 .. S-2 in flight
    if constexpr (LOADER) {
        issue_scales(0);
#pragma unroll
        for (int p = 0; p < S - 1; ++p)
#pragma unroll
            for (int q = 0; q < L; ++q) issue(p < nk ? p : nk - 1, p, q);
    }
    // A stage's head: the W blocks and scales of this lane's columns and the
    // A fragments of its first K-step; the rest of its A fragments are read
    // one K-step ahead.  With 4 or more slots the head of stage u + 1 is read
    // during the last K-step of stage u, so that a stage's MFMAs start right
    // after its barrier; that needs stage u + 1 landed at the barrier of
    // stage u, which a 3-slot ring cannot afford (measured: the wait for it
    // costs more than the head read saves), so there the head is read after
    // the barrier.
    constexpr bool AHEAD = S >= 4;
    u32x4 wblk[TN];
    uint32_t sraw[TN];
    v8bf fa0[TM];
    auto read_head = [&](int uu) __attribute__((always_inline)) {
        const int sl = uu % S;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = wn * (TN * 32) + j * 32 + frow;
            wblk[j] = *reinterpret_cast<const u32x4 *>(&sW[sl][(wn * TN + j) * 1024 + half * 512 + frow * 16]);
            sraw[j] = sS[(uu >> 3) & 1][col * 16 + 2 * (uu & 7) + half];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int r = rowA[i];
            fa0[i] = *reinterpret_cast<const v8bf *>(&sA[sl][r * A_ROW_B + (((4 * half) ^ swz(r)) << 4)]);
        }
    };
    if constexpr (AHEAD) {
        // stage 0 (and its scales) landed for every wave
        if constexpr (LOADER) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((S - 2) * L) : "memory");
        else asm volatile("s_barrier" ::: "memory");
        read_head(0);
    }
    for (int u = 0; u < nk; ++u) {
        const int slot = u % S;
        // this thread's loads of stage u + 1 (AHEAD) or u have landed (only
        // the later stages up to u + S - 2 may be outstanding, and a scale
        // load issued before the newest of them is waited for too); after
        // the barrier everyone's have, and slot (u + S - 1) % S = (u - 1) % S
        // is no longer read (a wave that issues no loads only meets the
        // barrier)
        constexpr int NOUT = (AHEAD ? S - 3 : S - 2) * L;
        if constexpr (LOADER) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NOUT) : "memory");
        else asm volatile("s_barrier" ::: "memory");
        if constexpr (!AHEAD) read_head(u);
        const int kn = u + S - 1 < nk ? u + S - 1 : nk - 1;
        const int sn = (u + S - 1) % S;
        // scales of the next group of 8 stages, first of this stage's loads
        // (the next stage's vmcnt wait then also covers it)
        if constexpr (LOADER)
            if ((u & 7) == 6 && u + 2 < nk) issue_scales((u + 2) >> 3);
        u32x4 wcur[TN];
        float sc[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            wcur[j] = wblk[j];
            sc[j] = e8m0_scale_f32(sraw[j]);
        }
        v8bf fa[2][TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = fa0[i];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v8bf fw[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const uint32_t p = wcur[j][st];
                const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[j], 0);
                const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[j], 1);
                const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[j], 2);
                const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[j], 3);
                fw[j] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
            }
            // the next K-step's A fragments, or the next stage's head (its
            // slot landed before this stage's barrier; past the last stage it
            // holds a re-load of the last stage, read and discarded)
            if (st < 3) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int r = rowA[i];
                    fa[(st + 1) & 1][i] = *reinterpret_cast<const v8bf *>(
                        &sA[slot][r * A_ROW_B + (((4 * half + st + 1) ^ swz(r)) << 4)]);
                }
            } else if constexpr (AHEAD) {
                read_head(u + 1);
            }
            // loads of stage u + S - 1, spread over the K-steps
            if constexpr (LOADER)
#pragma unroll
                for (int q = 0; q < L; ++q)
                    if ((q * 4) / L == st) issue(kn, sn, q);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[st & 1][i], fw[j], acc[i][j], 0, 0, 0);
        }
    }
    };
    if (wave < NLW) body(LoaderC<true>{});
    else body(LoaderC<false>{});
    // no load may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if constexpr (SPLITK) {
        // The K slice's partial tile goes to partial array `split` of the
        // workspace, [splits][NB][Mp][Np] fp32 with Mp, Np the tile-padded
        // sizes, so every store is in bounds; 16-byte stores of 4
        // consecutive columns after the in-quad transpose.  The reduction
        // kernel launched next on the stream adds the slices.
        const int64_t Mp = (int64_t)tiles_m * RPB, Np = (int64_t)tiles_n * BN;
        const int bq = NB == 2 ? (wm * TM * 32) / RPB : 0;
        float *pbase = g.ws + ((int64_t)split * NB + bq) * Mp * Np;
        const int64_t prow0 = m0 + wm * (TM * 32) - bq * RPB, pcol0 = n0 + wn * (TN * 32);
        const int q = frow & 3;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    float x[4] = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                                  acc[i][j][4 * gq + 3]};
                    quad_transpose(x, q);
                    const int64_t row = prow0 + i * 32 + 8 * gq + 4 * half + q;
                    // rows past M are never read by the reduction; streaming
                    // stores (the reduction kernel reads each value once)
                    if (row < g.M)
                        __builtin_nontemporal_store(u32x4{f2u(x[0]), f2u(x[1]), f2u(x[2]), f2u(x[3])},
                                                    reinterpret_cast<u32x4 *>(pbase + row * Np + pcol0 + j * 32 +
                                                                              (frow & ~3)));
                }
        return;
    }

    // epilogue: acc element e of tile (i, j) is row i*32 + 8*(e/4) + 4*half + e%4, column j*32 + frow
    const int b = NB == 2 ? (wm * TM * 32) / RPB : 0;
    void *cb = b ? g.c1 : g.c;
    const int64_t rbase = m0 + wm * (TM * 32) - b * RPB;
    const int64_t cbase = n0 + wn * (TN * 32);
    if (((reinterpret_cast<uintptr_t>(cb) & 15) == 0) && g.ldc % 4 == 0 && g.ldc < ((int64_t)1 << 26) &&
        rbase + TM * 32 <= g.M && cbase + TN * 32 <= g.N) {
        // this wave's block lies inside C: a 4x4 transpose inside each quad
        // of lanes gives every lane 4 consecutive columns of one row (fp32
        // C: one 16-byte store each); for 16-bit C lanes 4 apart then trade
        // halves so each lane stores 8 columns (pack16_rows8).  Every store
        // is a wave-uniform row pointer plus a fixed lane offset.
        constexpr int EB = CT == LSMX_F32 ? 4 : 2;
        const int q = frow & 3;
        const uint8_t *cw = reinterpret_cast<const uint8_t *>(cb) + (rbase * g.ldc + cbase) * EB;
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
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t col = cbase + j * 32 + frow;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t row = rbase + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                if (row < g.M && col < g.N) store_cw<CT>(cb, row * g.ldc + col, acc[i][j][e]);
            }
        }
}

template <int NB, int BR, int BN, int S, int WGM = 4, int NLW = wr::NW>
static hipError_t launch_ring(const GemmArgs &g, hipStream_t s) {
    constexpr int RPB = BR / NB;
    const int tiles = (int)(((g.M + RPB - 1) / RPB) * ((g.N + BN - 1) / BN));
    const dim3 grid(tiles), blk(wr::NT);
#define LSMX_R(CT) hipLaunchKernelGGL((gemm_bf16f4_ring_kernel<NB, CT, BR, BN, S, false, WGM, NLW>), grid, blk, 0, s, g)
    if (g.c_dtype == LSMX_F32) LSMX_R(LSMX_F32);
    else if (g.c_dtype == LSMX_BF16) LSMX_R(LSMX_BF16);
    else LSMX_R(LSMX_F16);
#undef LSMX_R
    return hipGetLastError();
}

// the ring kernel reads E8M0 scales 16 bytes (8 stages) at a time
static bool ring_ok(const GemmArgs &g) {
    return g.scale_fmt == LSMX_SCALE_E8M0 && g.ld_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(g.sb) & 15) == 0 &&
           g.K % 512 == 0;
}

// ------------------------------------------------------------------ skinny M
// For few activation rows (decode, M <= 32 per batch) the weight stream is the
// whole cost: N*K/2 bytes of codes against 2*M*K bytes of activations.  The
// 256-row tile above would leave most CUs idle, so this kernel spreads the
// weight over the chip instead:
//   - a workgroup owns 16*CT weight rows, its 8 waves split K: wave w takes
//     the 128-wide K chunks w, w + 8, w + 16, ...
//   - each lane loads one 16-byte MX block (32 codes) of one weight row per
//     chunk straight into registers, dequantizes it with
//     v_cvt_scalef32_pk_bf16_fp4, and feeds v_mfma_f32_16x16x32_bf16;
//   - the activation rows (MT tiles of 16, rows past M clamped) come straight
//     from global memory/L2, where they stay resident: they are tiny;
//   - the 8 partial sums are added in LDS in wave order and stored.
// K positions inside a chunk are assigned so that lane group q (lanes
// 16q..16q+15) of MFMA step s covers K = 128c + 32q + 8s .. +8 for both
// operands: one lane's 16 weight bytes are one block with one scale.
// Dual mode: virtual rows [0, M) are A0's and [M, 2M) are A1's, so the
// weight is streamed once for both batches.  The summation order of an
// output element depends on K only, so single and dual launches of the same
// M and K give identical bits.
namespace sk {
constexpr int WK = 8;  // waves per workgroup (K split)
constexpr int CHUNK = 128;
}  // namespace sk

typedef float v4f __attribute__((ext_vector_type(4)));

// MT <= 2: at most 128 VGPRs, so two workgroups (16 waves) share a CU.
template <int MT, int CT>
__global__ __launch_bounds__(64 * sk::WK, MT <= 2 ? 4 : 2) void gemm_bf16f4_skinny_kernel(GemmArgs g) {
    constexpr int U = MT == 1 ? 2 : 1;  // chunks in flight per wave
    __shared__ float red[sk::WK][MT * CT * 256];

    const int lane = threadIdx.x & 63, wk = threadIdx.x >> 6;
    const int j = lane & 15, grp = lane >> 4;
    const bool dual = g.a1 != nullptr;
    const int64_t VM = dual ? 2 * g.M : g.M;
    const int64_t nbase = (int64_t)blockIdx.x * (16 * CT);
    const bool sf32 = g.scale_fmt == LSMX_SCALE_F32;

    const uint8_t *arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int64_t v = min((int64_t)(16 * mt + j), VM - 1);
        const bool second = dual && v >= g.M;
        arow[mt] = (second ? g.a1 : g.a) + (second ? v - g.M : v) * g.lda * 2 + grp * 64;
    }
    const uint8_t *wrow[CT];
    int64_t srow[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        const int64_t n = min(nbase + 16 * ct + j, g.N - 1);
        wrow[ct] = g.b + n * g.ldb + grp * 16;
        srow[ct] = n * g.ld_sb + grp;
    }

    v4f acc[MT][CT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[mt][ct] = v4f{0.f, 0.f, 0.f, 0.f};

    const int nchunks = (int)(g.K / sk::CHUNK);
    for (int c0 = wk; c0 < nchunks; c0 += sk::WK * U) {
        u32x4 wv[U][CT], av[U][MT][4];
        uint32_t sv[U][CT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * sk::WK;
            if (c < nchunks) {
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    wv[u][ct] = *reinterpret_cast<const u32x4 *>(wrow[ct] + (int64_t)c * 64);
                    const int64_t so = srow[ct] + (int64_t)c * 4;
                    sv[u][ct] = sf32 ? f32_scale_e8m0(f2u(reinterpret_cast<const float *>(g.sb)[so]))
                                     : reinterpret_cast<const uint8_t *>(g.sb)[so];
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        av[u][mt][s] = *reinterpret_cast<const u32x4 *>(arow[mt] + (int64_t)c * 256 + s * 16);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u * sk::WK < nchunks) {
                float sc[CT];
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) sc[ct] = e8m0_scale_f32(sv[u][ct]);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    // dequantize step s of every column tile: codes 8s..8s+7 of the block
                    v8bf wf[CT];
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        const uint32_t p = wv[u][ct][s];
                        const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[ct], 0);
                        const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[ct], 1);
                        const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[ct], 2);
                        const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[ct], 3);
                        wf[ct] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const v8bf fa = __builtin_bit_cast(v8bf, av[u][mt][s]);
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct)
                            acc[mt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, wf[ct], acc[mt][ct], 0, 0, 0);
                    }
                }
            }
        }
    }

    // acc[mt][ct][r] = D[4*grp + r][j] of the 16 x 16 tile (rows: activation
    // rows of m-tile mt, columns: weight rows of col tile ct)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wk][(mt * CT + ct) * 256 + r * 64 + lane] = acc[mt][ct][r];
    __syncthreads();
    for (int p = wk; p < MT * CT; p += sk::WK) {
        const int mt = p / CT, ct = p % CT;
        const int64_t n = nbase + 16 * ct + j;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < sk::WK; ++w) v += red[w][p * 256 + r * 64 + lane];
            const int64_t vr = 16 * mt + 4 * grp + r;
            if (vr < VM && n < g.N) {
                const bool second = dual && vr >= g.M;
                void *cb = second ? g.c1 : g.c;
                const int64_t idx = (second ? vr - g.M : vr) * g.ldc + n;
                if (g.c_dtype == LSMX_F32) store_cw<LSMX_F32>(cb, idx, v);
                else if (g.c_dtype == LSMX_BF16) store_cw<LSMX_BF16>(cb, idx, v);
                else store_cw<LSMX_F16>(cb, idx, v);
            }
        }
    }
}

// ------------------------------------------------------------------ decode M
static int num_cus_w();
// Up to 16 activation rows per batch (dual: 32 virtual rows): the weight is
// read once, in whole 256-byte row pieces, with all of a workgroup's bytes in
// flight at once.
//   - a workgroup owns up to R weight rows (as many as spread the weight
//     evenly over the CUs, one workgroup each); its 8 waves split each
//     4096-deep K pass
//     into 512-deep slices (wave w: K = 512w .. 512w + 511, 256 bytes of
//     every row);
//   - at the start of a pass every wave issues its whole share: R/4 direct-
//     to-LDS loads of 4 rows x 256 contiguous bytes, the pass's E8M0 scales
//     (R rows x 128 E8M0 bytes, or 128 fp32 powers of two), and its
//     activation fragments into registers;
//     nothing is computed before they land, so a workgroup's latency is paid
//     once per pass while the other workgroups' loads keep HBM busy;
//   - lane (n, q) of MFMA step s (v_mfma_f32_16x16x32_bf16) reads 4 bytes
//     (8 codes) of weight row n: LDS chunk s of a row sits at 16 * (s ^ n),
//     which puts the 64 lanes of a ds_read_b32 on 64 distinct banks (the DMA
//     writes lanes in order, so the swizzle is applied by choosing each
//     lane's source chunk);
//   - v_cvt_scalef32_pk_bf16_fp4 expands the codes to bf16 with the block
//     scale (exact); the activation fragment of step s holds the same 8 K
//     positions (K = 32s + 8q .. +8 of the slice);
//   - the 8 waves' partial sums meet in LDS and are added in wave order.
// The summation order of an output element depends on K only, so single and
// dual launches of the same M give identical bits.
namespace dk {
constexpr int NW = 8, NT = 64 * NW;
constexpr int SLICE_K = 512;          // K per wave per pass
constexpr int PASS_K = NW * SLICE_K;  // 4096
constexpr int ROW_B = SLICE_K / 2;    // code bytes of one row per slice
constexpr int SC_ROW = PASS_K / 32;   // scale bytes of one row per pass
}  // namespace dk

// 16-byte global load from inline asm: its completion is waited for with an
// explicit s_waitcnt, which counts it together with the direct-to-LDS loads.
LSMX_DEV u32x4 gload_x4(const void *p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
    return v;
}

// E8M0 byte -> fp32 scale without branches: 2^(e - 127), with byte 0 ->
// 2^-127 (0x00400000) and byte 255 -> NaN (0x7FC00000), both of which are
// (e << 23) | 2^22.
LSMX_DEV float e8m0_scale_nb(uint32_t e) {
    const uint32_t special = ((((e + 1u) & 0xFEu) - 1u) >> 9) & 0x00400000u;
    return u2f((e << 23) | special);
}
// fp32 scale -> itself when it has an E8M0 form (a power of two in
// [2^-127, 2^127]), else NaN, without branches.
LSMX_DEV float f32_scale_nb(uint32_t b) {
    const bool ok = ((b & 0x807FFFFFu) == 0u && b - 0x00800000u <= 0x7E800000u) || b == 0x00400000u;
    return u2f(ok ? b : 0x7FC00000u);
}

// One workgroup per CU (the launcher gives each CU one share of the weight
// rows): 8 waves, two per SIMD, so up to 256 VGPRs per wave.
template <int MT, int R, int CT, bool SF32>
__global__ __launch_bounds__(dk::NT, 2) void gemm_bf16f4_decode_kernel(GemmArgs g) {
    using namespace dk;
    constexpr int TN = R / 16;                   // 16-column MFMA tiles
    constexpr int XW = R / 4;                    // weight loads per wave per pass
    constexpr int SV = SF32 ? 4 : 1;             // 16-byte scale vectors per row per slice
    static_assert(R % 16 == 0, "tile");
    __shared__ __attribute__((aligned(16))) uint8_t sW[NW][R * ROW_B];
    static_assert(sizeof(sW) >= (size_t)NW * MT * TN * 256 * 4, "reduction buffer");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n16 = lane & 15, q = lane >> 4;
    const bool dual = g.a1 != nullptr;
    const int64_t VM = dual ? 2 * g.M : g.M;
    const int64_t n0 = (int64_t)blockIdx.x * g.rows_wg;
    const int64_t nend = min(n0 + g.rows_wg, g.N);   // rows past nend read zeros

    // activation rows of this lane (rows past VM repeat the last one; their
    // outputs are not stored)
    const uint8_t *arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int64_t v = min((int64_t)(16 * mt + n16), VM - 1);
        const bool second = dual && v >= g.M;
        arow[mt] = (second ? g.a1 : g.a) + (second ? v - g.M : v) * g.lda * 2 + q * 16;
    }
    // scale rows of this lane's weight rows (rows past nend repeat the last one)
    const uint8_t *srow[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t)
        srow[t] = reinterpret_cast<const uint8_t *>(g.sb) + min(n0 + 16 * t + n16, nend - 1) * g.ld_sb * (SF32 ? 4 : 1);
    // weight load j covers rows 4j .. 4j + 3: lane l -> row 4j + l/16, LDS
    // chunk l%16 holding source chunk (l%16) ^ (row & 15)
    uint32_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        w_off[j] = (uint32_t)((lane >> 4) * g.ldb + 16 * ((lane & 15) ^ (r & 15)));
    }

    // two accumulators per tile (even and odd K-steps), so that consecutive
    // MFMAs do not wait for each other's results; added at the end
    v4f acc[MT][TN][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[mt][t][0] = acc[mt][t][1] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma nounroll
    for (int64_t kp = 0; kp < g.K; kp += PASS_K) {
        const int64_t k0 = kp + (int64_t)wave * SLICE_K;   // this wave's slice
        const bool live = k0 < g.K;                         // K % 512 == 0: whole slices
        if (kp > 0) __syncthreads();   // every wave is done with the previous pass's LDS
        if (live) {
            // The slice's 16 scales of each of this lane's weight rows and
            // its activation fragments, then its weight rows.  All are asm
            // loads counted by the explicit waits below: a compiler-visible
            // load would get a compiler wait that counts only its own loads
            // and so also waits for the weight loads issued after it.
            u32x4 sv[TN][SV];
#pragma unroll
            for (int t = 0; t < TN; ++t)
#pragma unroll
                for (int v = 0; v < SV; ++v) sv[t][v] = gload_x4(srow[t] + (k0 / 32) * (SF32 ? 4 : 1) + 16 * v);
            u32x4 af[MT][16];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int s = 0; s < 16; ++s) af[mt][s] = gload_x4(arow[mt] + (k0 + 32 * s) * 2);
#pragma unroll
            for (int j = 0; j < XW; ++j) {
                const int64_t r0 = n0 + 4 * j, left = nend - r0;
                const uint64_t bytes = left > 0 ? (uint64_t)((left - 1) * g.ldb + (g.K - k0) / 2) : 0;
                dma_x4(w_off[j & 3], buf_rsrc(g.b + r0 * g.ldb + k0 / 2, bytes),
                       lds_u32(&sW[wave][0]) + j * 1024);
            }
            // The wave reads only the LDS its own loads wrote: no barrier.
            // Column tile t's rows are loads 4t .. 4t + 3, so its MFMAs start
            // once they (and everything issued before them) have landed,
            // while the later tiles' loads are still in flight.
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * (TN - 1)) : "memory");
#pragma unroll
            for (int t = 0; t < TN; ++t)
#pragma unroll
                for (int v = 0; v < SV; ++v) asm volatile("" : "+v"(sv[t][v]));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int s = 0; s < 16; ++s) asm volatile("" : "+v"(af[mt][s]));
            // E8M0 bytes 0 and 255 need the exact conversion; any other byte
            // is 2^(e - 127) = e << 23.  Lane (n, q) tests dword q of its
            // row's 16 bytes, so the wave covers every byte once.
            bool exact = SF32;
            if constexpr (!SF32) {
                uint32_t hit = 0;
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    const uint32_t x = q == 0 ? sv[t][0].x : q == 1 ? sv[t][0].y : q == 2 ? sv[t][0].z : sv[t][0].w;
                    hit |= ((x - 0x01010101u) & ~x) | ((0xFEFEFEFEu - x) & x);   // a 00 or an FF byte
                }
                exact = __builtin_amdgcn_ballot_w64((hit & 0x80808080u) != 0u) != 0;
            }
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                if (t > 0) {
                    // nothing moves across the wait: the tile before it
                    // computes while this tile's rows land
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * (TN - 1 - t)) : "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
                float sc[16];
                if (exact) {
#pragma unroll
                    for (int s = 0; s < 16; ++s)
                        sc[s] = SF32 ? f32_scale_nb(sv[t][s >> 2][s & 3])
                                     : e8m0_scale_nb((sv[t][0][s >> 2] >> (8 * (s & 3))) & 0xFFu);
                } else {
#pragma unroll
                    for (int s = 0; s < 16; ++s) sc[s] = u2f(((sv[t][0][s >> 2] >> (8 * (s & 3))) & 0xFFu) << 23);
                }
                // the tile's 16 code words in one batch of LDS reads (one
                // latency per tile instead of one per K-step)
                uint32_t pc[16];
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    pc[s] = *reinterpret_cast<const uint32_t *>(&sW[wave][(16 * t + n16) * ROW_B + 16 * (s ^ n16) + 4 * q]);
                // dequantize four K-steps ahead of their MFMAs, into two
                // alternating register sets: an MFMA never waits for the
                // conversion just before it, and a conversion never
                // overwrites the operand of an MFMA still in flight
                v8bf wf[2][4];
                auto dequant = [&](int g4) __attribute__((always_inline)) {
#pragma unroll
                    for (int s1 = 0; s1 < 4; ++s1) {
                        const int s = 4 * g4 + s1;
                        const uint32_t p = pc[s];
                        const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[s], 0);
                        const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[s], 1);
                        const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[s], 2);
                        const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc[s], 3);
                        wf[g4 & 1][s1] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
                    }
                };
                dequant(0);
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    if (g4 < 3) dequant(g4 + 1);
#pragma unroll
                    for (int s1 = 0; s1 < 4; ++s1) {
                        const int s = 4 * g4 + s1;
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            acc[mt][t][s & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(v8bf, af[mt][s]), wf[g4 & 1][s1], acc[mt][t][s & 1], 0, 0, 0);
                    }
                }
            }
        }
    }

    // acc[mt][t][r] = D[4q + r][n16] of the 16 x 16 tile (rows: activation
    // rows of tile mt, columns: weight rows 16t ..); the 8 waves' partial
    // sums are added in wave order
    __syncthreads();
    float *red = reinterpret_cast<float *>(&sW[0][0]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[((wave * MT + mt) * TN + t) * 256 + r * 64 + lane] = acc[mt][t][0][r] + acc[mt][t][1][r];
    __syncthreads();
    for (int o = threadIdx.x; o < MT * TN * 256; o += NT) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w * MT * TN * 256 + o];
        const int p = o >> 8, e = o & 255, r = e >> 6, l = e & 63;
        const int mt = p / TN, t = p % TN;
        const int64_t vr = 16 * mt + 4 * (l >> 4) + r, n = n0 + 16 * t + (l & 15);
        if (vr < VM && n < nend) {
            const bool second = dual && vr >= g.M;
            store_cw<CT>(second ? g.c1 : g.c, (second ? vr - g.M : vr) * g.ldc + n, v);
        }
    }
}

template <int R, int MT>
static hipError_t launch_decode_r(GemmArgs g, hipStream_t s) {
    // rows per workgroup: the weight spread evenly over the CUs, in whole
    // 4-row loads, at most R
    const int64_t cus = num_cus_w(), per = (g.N + cus - 1) / cus, rows = (per + 3) / 4 * 4;
    g.rows_wg = (int)(rows > R ? R : rows < 16 ? 16 : rows);
    const dim3 grid((unsigned)((g.N + g.rows_wg - 1) / g.rows_wg)), blk(dk::NT);
    const bool f = g.scale_fmt == LSMX_SCALE_F32;
#define LSMX_D(CT, F) hipLaunchKernelGGL((gemm_bf16f4_decode_kernel<MT, R, CT, F>), grid, blk, 0, s, g)
#define LSMX_DC(F)                                                    \
    do {                                                              \
        if (g.c_dtype == LSMX_F32) LSMX_D(LSMX_F32, F);               \
        else if (g.c_dtype == LSMX_BF16) LSMX_D(LSMX_BF16, F);        \
        else LSMX_D(LSMX_F16, F);                                     \
    } while (0)
    if (f) LSMX_DC(true);
    else LSMX_DC(false);
#undef LSMX_DC
#undef LSMX_D
    return hipGetLastError();
}

// up to 16 rows per batch (2 x 16 virtual rows for the dual form)
constexpr int64_t kDecodeMaxM = 16;
// up to 16 virtual rows: 64 weight rows per workgroup; 17 .. 32 (the dual
// form): 32, so that the second activation tile's registers fit
static hipError_t launch_decode(const GemmArgs &g, hipStream_t s) {
    const int64_t vm = g.a1 ? 2 * g.M : g.M;
    return vm <= 16 ? launch_decode_r<64, 1>(g, s) : launch_decode_r<32, 2>(g, s);
}

// The decode kernel's scale loads: 16-byte aligned rows of either format
// (the same test for both, so that E8M0 bytes and fp32 powers of two of the
// same scales pick the same kernel and give the same bits).
static bool decode_ok(const GemmArgs &g) {
    return g.K % dk::SLICE_K == 0 && (reinterpret_cast<uintptr_t>(g.sb) & 15) == 0 && g.ld_sb % 16 == 0;
}

// ------------------------------------------------------------------ mid M
// 17 to 64 activation rows per batch: the decode kernel's weight layout, with
// the activations streamed instead of held.
//   - a workgroup owns the weight rows the decode kernel would give it (the
//     weight spread evenly over the CUs, at most 64 rows, four 16-row MFMA
//     tiles) and the whole K: its 8 waves split each 4096-deep pass into
//     512-deep slices, each wave's slice of every row loaded once into LDS
//     (the decode kernel's 4-row, 256-byte direct-to-LDS loads and chunk
//     swizzle) together with its 16 E8M0 scale bytes per row;
//   - the activation rows are processed in groups of 64 (4 MFMA tiles; the
//     dual form's 2M virtual rows can make two): for each 32-deep K-step of
//     its slice a wave loads the group's fragments row-contiguous (lane l:
//     16-byte piece l%4 of row l/4, so a quarter-wave touches 4 rows, not
//     16) in pairs of steps (both halves of each 128-byte line together), a
//     pair or two ahead, moves them to the MFMA layout with ds_bpermute and
//     reads the step's weight code words one step ahead of its 16
//     independent v_mfma_f32_16x16x32_bf16, dequantizing them just before
//     (v_cvt_scalef32_pk_bf16_fp4, exact); with one pass (K <= 4096) the
//     weight slice stays in LDS for every group;
//   - the 8 waves' partial sums of a group meet in a separate 32 KiB LDS
//     buffer, one activation tile at a time, and are added in wave order.
// No partial tiles go to memory and there is no second launch (the split-K
// ring's cost at these shapes).  The summation order of an output element
// depends on K only, so single and dual launches of the same M give
// identical bits.
namespace mk {
constexpr int PASS_K = 4096;                     // K per pass (all waves' slices)
constexpr int R = 64, TN = R / 16;               // weight rows (at most), 16-row MFMA tiles
constexpr int MT = 4, GROUP = 16 * MT;           // activation tiles per group, rows per group
}  // namespace mk

template <int I, int N, typename F>
LSMX_DEV void static_for(F &&f) {
    if constexpr (I < N) {
        f(SlotC<I>{});
        static_for<I + 1, N>(f);
    }
}
template <int N>
LSMX_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// NW waves (each a PASS_K / NW deep slice of K), activation step pairs
// loaded PD pairs ahead of the pair in use.
template <int NW, int PD, int CT>
__global__ __launch_bounds__(64 * NW, 1) void gemm_bf16f4_midm_kernel(GemmArgs g) {
    using namespace mk;
    constexpr int NT = 64 * NW, SLICE_K = PASS_K / NW, STEPS = SLICE_K / 32, NPAIR = STEPS / 2;
    constexpr int H = SLICE_K / 512;                // 256-byte halves of a row's slice
    constexpr int XW = (R / 4) * H;                 // weight loads per wave per pass (4 rows x 256 bytes)
    constexpr int SV = SLICE_K / 512;               // 16-byte E8M0 vectors per row per slice
    constexpr int NSLOT = 2 * (PD + 1);             // activation fragment slots (steps)
    __shared__ __attribute__((aligned(16))) uint8_t sW[NW][H][R * 256];   // 128 KiB
    __shared__ __attribute__((aligned(16))) float red[NW][TN * 256];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n16 = lane & 15, q = lane >> 4;
    const bool dual = g.a1 != nullptr;
    const int64_t VM = dual ? 2 * g.M : g.M;
    const int64_t n0 = (int64_t)blockIdx.x * g.rows_wg;
    const int64_t nend = min(n0 + g.rows_wg, g.N);   // rows past nend read zeros
    const bool one_pass = g.K <= PASS_K;

    // scale rows of this lane's weight rows (rows past nend repeat the last one)
    const uint8_t *srow[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t)
        srow[t] = reinterpret_cast<const uint8_t *>(g.sb) + min(n0 + 16 * t + n16, nend - 1) * g.ld_sb;
    // weight load (j, h) covers rows 4j .. 4j + 3, bytes 256h .. 256h + 255 of
    // their slices: lane l -> row 4j + l/16, LDS chunk l%16 holding source
    // chunk (l%16) ^ (row & 15)
    uint32_t w_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        w_off[j] = (uint32_t)((lane >> 4) * g.ldb + 16 * ((lane & 15) ^ (r & 15)));
    }
    u32x4 sv[TN][SV];
    // byte address of the lane that loaded this lane's MFMA piece
    const int src4 = 4 * (4 * n16 + q);

#pragma nounroll
    for (int64_t vg = 0; vg < VM; vg += GROUP) {
        // Activation fragments are loaded row-contiguous -- lane l reads the
        // 16-byte piece l%4 of row l/4 of the tile's 64-byte step segment, so
        // a quarter-wave touches 4 rows instead of 16 -- and moved to the MFMA
        // layout (lane (n16, q): row n16, piece q) with ds_bpermute.  Rows
        // past VM repeat the last one; their outputs are not stored.
        const uint8_t *arow[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int64_t v = min(vg + 16 * mt + (lane >> 2), VM - 1);
            const bool second = dual && v >= g.M;
            arow[mt] = (second ? g.a1 : g.a) + (second ? v - g.M : v) * g.lda * 2 + (lane & 3) * 16;
        }
        v4f acc[MT][TN];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < TN; ++t) acc[mt][t] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma nounroll
        for (int64_t kp = 0; kp < g.K; kp += PASS_K) {
            const int64_t k0 = kp + (int64_t)wave * SLICE_K;   // this wave's slice
            const bool live = k0 < g.K;                         // K % SLICE_K == 0: whole slices
            const bool load_w = vg == 0 || !one_pass;
            // every wave is done with the LDS slice it is about to overwrite
            if (load_w && kp > 0) __syncthreads();
            if (!live) continue;
            // The scales and the weight slice (when not already in LDS), then
            // the first PD + 1 pairs of steps' activation fragments: asm
            // loads, all counted by the explicit waits below, in issue order,
            // so the wait for step 0's fragments also covers the weights.
            if (load_w) {
#pragma unroll
                for (int t = 0; t < TN; ++t)
#pragma unroll
                    for (int v = 0; v < SV; ++v) sv[t][v] = gload_x4(srow[t] + k0 / 32 + 16 * v);
#pragma unroll
                for (int j = 0; j < R / 4; ++j) {
                    const int64_t r0 = n0 + 4 * j, left = nend - r0;
                    const uint64_t bytes = left > 0 ? (uint64_t)((left - 1) * g.ldb + (g.K - k0) / 2) : 0;
#pragma unroll
                    for (int h = 0; h < H; ++h)
                        dma_x4(w_off[j & 3], buf_rsrc(g.b + r0 * g.ldb + k0 / 2 + 256 * h, bytes > 256u * h ? bytes - 256u * h : 0),
                               lds_u32(&sW[wave][h][0]) + j * 1024);
                }
            }
            // Steps s and s + 1 (s even) are loaded back to back per tile, so
            // the two 64-byte halves of each 128-byte line are requested
            // together (one line fill).
            u32x4 af[NSLOT][MT];
            auto fetch2 = [&](int s) __attribute__((always_inline)) {
                const uint32_t off0 = (uint32_t)(k0 * 2) + 64u * (uint32_t)s;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    af[s % NSLOT][mt] = gload_x4(arow[mt] + off0);
                    af[(s + 1) % NSLOT][mt] = gload_x4(arow[mt] + off0 + 64);
                }
            };
            // A step's operands (the permuted activation fragments ab and the
            // weight code words pc) are prepared one step ahead, so their LDS
            // latencies overlap the previous step's MFMAs.
            auto prep = [&](int s, u32x4 (&ab)[MT], uint32_t (&pc)[TN]) __attribute__((always_inline)) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    asm volatile("" : "+v"(af[s % NSLOT][mt]));
                    const u32x4 v = af[s % NSLOT][mt];
                    ab[mt] = u32x4{(uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)v.x),
                                   (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)v.y),
                                   (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)v.z),
                                   (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)v.w)};
                }
                const int h = s >> 4, c = s & 15;
#pragma unroll
                for (int t = 0; t < TN; ++t)
                    pc[t] = *reinterpret_cast<const uint32_t *>(&sW[wave][h][(16 * t + n16) * 256 + 16 * (c ^ n16) + 4 * q]);
            };
            // Pair p (steps 2p, 2p + 1) is issued in the prologue for p <= PD,
            // else at the end of step 2(p - PD) - 1.  wait_for<s, cur>: step
            // s's fragments have landed, given the pairs issued by step cur;
            // what may stay in flight is what was issued after step s's last
            // fragment (that of tile MT - 1).
            auto wait_for = [&](auto sc, auto cc) __attribute__((always_inline)) {
                constexpr int st = decltype(sc)::value, cur = decltype(cc)::value;
                constexpr int newest = (PD + (cur + 1) / 2) < NPAIR - 1 ? PD + (cur + 1) / 2 : NPAIR - 1;
                constexpr int ahead = st % 2 == 0 ? 1 + (newest - st / 2) * 2 * MT : (newest - (st - 1) / 2) * 2 * MT;
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt<ahead>();
                __builtin_amdgcn_sched_barrier(0);
            };
#pragma unroll
            for (int p = 0; p <= PD; ++p) fetch2(2 * p);
            wait_for(SlotC<0>{}, SlotC<-1>{});
            if (load_w) {
#pragma unroll
                for (int t = 0; t < TN; ++t)
#pragma unroll
                    for (int v = 0; v < SV; ++v) asm volatile("" : "+v"(sv[t][v]));
            }
            u32x4 ab[2][MT];
            uint32_t pc[2][TN];
            prep(0, ab[0], pc[0]);
            static_for<0, STEPS>([&](auto sc) __attribute__((always_inline)) {
                constexpr int st = decltype(sc)::value;
                // the pair PD + 1 ahead of the one ending here
                if constexpr (st % 2 == 1 && (st + 1) / 2 + PD < NPAIR) fetch2(2 * ((st + 1) / 2 + PD));
                if constexpr (st + 1 < STEPS) {
                    wait_for(SlotC<st + 1>{}, SlotC<st>{});
                    prep(st + 1, ab[(st + 1) % 2], pc[(st + 1) % 2]);
                }
                // dequantize the step's weight fragments (exact, block scale applied)
                v8bf wf[TN];
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    const uint32_t pw = pc[st % 2][t];
                    const float sc8 = e8m0_scale_nb((sv[t][st >> 4][(st >> 2) & 3] >> (8 * (st & 3))) & 0xFFu);
                    const v2bf d0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw, sc8, 0);
                    const v2bf d1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw, sc8, 1);
                    const v2bf d2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw, sc8, 2);
                    const v2bf d3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(pw, sc8, 3);
                    wf[t] = v8bf{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int t = 0; t < TN; ++t)
                        acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(v8bf, ab[st % 2][mt]), wf[t], acc[mt][t], 0, 0, 0);
            });
        }

        // acc[mt][t][r] = D[4q + r][n16] of the 16 x 16 tile (rows: activation
        // rows vg + 16 mt .., columns: weight rows 16 t ..); one activation
        // tile at a time, the waves' partial sums are added in wave order
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            __syncthreads();
#pragma unroll
            for (int t = 0; t < TN; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave][t * 256 + r * 64 + lane] = acc[mt][t][r];
            __syncthreads();
            for (int o = threadIdx.x; o < TN * 256; o += NT) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < NW; ++w) v += red[w][o];
                const int t = o >> 8, e = o & 255, r = e >> 6, l = e & 63;
                const int64_t vr = vg + 16 * mt + 4 * (l >> 4) + r, n = n0 + 16 * t + (l & 15);
                if (vr < VM && n < nend) {
                    const bool second = dual && vr >= g.M;
                    store_cw<CT>(second ? g.c1 : g.c, (second ? vr - g.M : vr) * g.ldc + n, v);
                }
            }
        }
    }
}

// 8 waves with the next pair in flight: 4 waves (one per SIMD, 512
// registers) with 2 or 3 pairs in flight measured 11-16% slower at M = 32,
// 64 and 128 (cfg3's weight, one box)
constexpr int kMidNW = 8, kMidPD = 1;
template <int CT>
static void launch_midm_ct(GemmArgs g, hipStream_t s) {
    const int64_t cus = num_cus_w(), per = (g.N + cus - 1) / cus, rows = (per + 3) / 4 * 4;
    g.rows_wg = (int)(rows > mk::R ? mk::R : rows < 16 ? 16 : rows);
    const dim3 grid((unsigned)((g.N + g.rows_wg - 1) / g.rows_wg)), blk(64 * kMidNW);
    hipLaunchKernelGGL((gemm_bf16f4_midm_kernel<kMidNW, kMidPD, CT>), grid, blk, 0, s, g);
}

static hipError_t launch_midm(const GemmArgs &g, hipStream_t s) {
    if (g.c_dtype == LSMX_F32) launch_midm_ct<LSMX_F32>(g, s);
    else if (g.c_dtype == LSMX_BF16) launch_midm_ct<LSMX_BF16>(g, s);
    else launch_midm_ct<LSMX_F16>(g, s);
    return hipGetLastError();
}

// Per-batch rows the mid-M kernel takes (above the decode kernel's).  Up to
// 64 it beats the skinny and split-K kernels at cfg3's weight (M = 32: 20.3
// against 26.3 us, M = 64: 21.0 against 27.1, the dual form of M = 64: 33.5
// against 38.9); at M = 128 the activation stream through each CU's vector
// memory path makes it slower than split-K (33.5 against 29.5).
constexpr int64_t kMidMaxM = 64;
// The shape test (M, N, K only, so that the split-K workspace query agrees):
// whole 512-deep K slices, the weight spread as the decode kernel spreads it
// (at most 64 rows per workgroup) over at least one workgroup per CU.
static bool midm_shape(int64_t M, int64_t N, int64_t K) {
    const int64_t cus = num_cus_w();
    return M > kDecodeMaxM && M <= kMidMaxM && K % (mk::PASS_K / kMidNW) == 0 && N >= 16 * cus && (N + cus - 1) / cus <= mk::R;
}
// and E8M0 byte scales in 16-byte aligned rows (the decode kernel's scale loads)
static bool midm_ok(const GemmArgs &g) {
    return g.scale_fmt == LSMX_SCALE_E8M0 && decode_ok(g) && midm_shape(g.M, g.N, g.K);
}

// ------------------------------------------------------------------ GEMV
// For one or two activation rows per batch (decode) the whole cost is reading
// W once, and the matrix cores have almost nothing to do.  This kernel reads
// W with fully contiguous loads and does the arithmetic on the VALU:
//   - the activation rows are staged once per workgroup in LDS;
//   - a wave owns RPW weight rows; lane l takes the MX blocks l, l + 64,
//     l + 128, ... of every row, so each load instruction reads 1 KiB of one
//     row in one piece, and all of a wave's weight loads are issued before
//     any arithmetic;
//   - v_cvt_scalef32_pk_bf16_fp4 expands a block to 32 bf16 (exact, block
//     scale applied) and v_dot2_f32_bf16 multiplies pairs with the
//     activations;
//   - the 64 lane partial sums of each (row, activation row) are added with a
//     fixed butterfly, so the order depends on K only.
// VM is the number of virtual activation rows (M, or 2M in dual mode).
namespace gv {
// 4 waves of 2 weight rows each (1792 workgroups at N = 14336): a 14336 x
// 4096 weight streams in 8.4 us against 8.9 us for 8-wave workgroups (896),
// 9.5 us for 2-wave ones and 9.5-9.8 us with 1 or 4 rows per wave.  Of the
// 8.4 us, the dequantize-and-dot arithmetic adds ~1.2 us and the activation
// staging ~0.5 us to the 6.8 us of the loads alone (a plain 31 MB read runs
// in 6.0 us); the lane sum on the vector ALU (wave_sum_fixed) took ~0.5 us
// off the arithmetic's share
constexpr int NT = 256;
constexpr int RPW = 2;
constexpr int UB = 2;     // groups of 64 blocks per lane in flight
}  // namespace gv

// Sum over the 64 lanes, the same in every lane, in a fixed tree on the
// vector ALU: pairs (l, l ^ 1), (l, l ^ 2) of each quad (DPP quad_perm), then
// the two quads of each 8 (row_half_mirror), the two halves of each row of
// 16 (row_mirror), then rows l, l ^ 16 and halves l, l ^ 32
// (v_permlane16_swap / v_permlane32_swap).  Each step adds a pair whose two
// lanes hold the same two values, and fp32 addition commutes, so all lanes
// end with the same bits.  Through __shfl_xor (LDS permutes) the six
// dependent steps cost ~0.5 us of the M = 1 GEMV.
LSMX_DEV float wave_sum_fixed(float v) {
    v += u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0xB1, 0xF, 0xF, false));
    v += u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x4E, 0xF, 0xF, false));
    v += u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x141, 0xF, 0xF, false));
    v += u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x140, 0xF, 0xF, false));
    const auto s16 = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
    v = u2f(s16[0]) + u2f(s16[1]);
    const auto s32 = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
    return u2f(s32[0]) + u2f(s32[1]);
}

template <int VM, bool SF32, int CT>
__global__ __launch_bounds__(gv::NT) void gemv_bf16f4_kernel(GemmArgs g) {
    using namespace gv;
    extern __shared__ __attribute__((aligned(16))) uint8_t sact[];   // [VM][K] bf16
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int64_t n0 = ((int64_t)blockIdx.x * (NT / 64) + wave) * RPW;
    const int nblk = (int)(g.K / 32);
    const bool dual = g.a1 != nullptr;

    // Stage the activation rows, 16 bytes per thread per step.  Lane l reads
    // the 64 bytes of block l (+ 64 k) as four 16-byte chunks, so 16 lanes
    // of one ds_read_b128 start 64 bytes apart; chunk q of block b is stored
    // at position (q + (b >> 2)) & 3 of the block, which puts those 16 lanes
    // on 16 distinct 16-byte bank groups (without it, 4-way conflicts).
    auto apos = [](int64_t b, int q) { return b * 64 + 16 * ((q + (int)(b >> 2)) & 3); };
    const int per_row = (int)(g.K / 8);   // 16-byte chunks per row
    // K % 512 == 0 (whole 64-chunk DMA instructions per row): the rows are
    // staged by direct-to-LDS loads issued before the weight loads.  A
    // staging load through registers would have to land before its LDS
    // store, and with vmcnt counting in issue order the weight stream could
    // only start after it; a DMA needs no register, so the weight loads go
    // out behind it at once and the wave waits for the DMA alone (all but
    // the newest 4 vector-memory operations: the first block group's weight
    // and scale loads, always issued) before the barrier.  Lane l of a DMA
    // writes chunk position p = its base + l; the swizzle is applied by
    // loading into position p the chunk that apos puts there.
    const bool dma_act = per_row % 64 == 0;
    if (dma_act) {
        for (int base = 64 * wave; base < VM * per_row; base += NT) {
            const int m = base / per_row;
            const bool second = dual && m >= (int)g.M;
            const uint8_t *row = (second ? g.a1 : g.a) + (int64_t)(second ? m - g.M : m) * g.lda * 2;
            const int p = base - m * per_row + lane, bk = p >> 2, slot = p & 3;
            const uint32_t voff = (uint32_t)((4 * bk + ((slot - (bk >> 2)) & 3)) * 16);
            dma_x4(voff, buf_rsrc(row, (uint64_t)g.K * 2),
                   lds_u32(sact) + (uint32_t)((int64_t)m * g.K * 2 + (int64_t)(base - m * per_row) * 16));
        }
    } else {
        for (int i = t; i < VM * per_row; i += NT) {
            const int m = i / per_row, c = i - m * per_row;
            const bool second = dual && m >= (int)g.M;
            const uint8_t *src = (second ? g.a1 : g.a) + (int64_t)(second ? m - g.M : m) * g.lda * 2 + c * 16;
            *reinterpret_cast<u32x4 *>(sact + ((int64_t)m * g.K * 2 + apos(c >> 2, c & 3))) =
                *reinterpret_cast<const u32x4 *>(src);
        }
    }

    const uint8_t *wrow[RPW];
    const uint8_t *srow[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t n = min(n0 + r, g.N - 1);
        wrow[r] = g.b + n * g.ldb;
        srow[r] = reinterpret_cast<const uint8_t *>(g.sb) + n * g.ld_sb * (SF32 ? 4 : 1);
    }

    float acc[RPW][VM];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int m = 0; m < VM; ++m) acc[r][m] = 0.0f;

    u32x4 w[UB][RPW];
    uint32_t e[UB][RPW];
    // weight and scale loads of the UB block groups starting at b0 (blocks
    // past the row are skipped)
    auto wload = [&](int b0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int b = b0 + 64 * u;
            if (b < nblk) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wrow[r] + (int64_t)b * 16));
                    e[u][r] = SF32 ? f32_scale_e8m0(f2u(reinterpret_cast<const float *>(srow[r])[b])) : srow[r][b];
                }
            }
        }
    };
    wload(lane);       // the first weight loads are in flight across the barrier
    if (dma_act) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    __syncthreads();
    for (int b0 = lane; b0 < nblk;) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int b = b0 + 64 * u;
            if (b >= nblk) break;
            u32x4 av[VM][4];  // 32 bf16 of activation row m at K = 32b
#pragma unroll
            for (int m = 0; m < VM; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    av[m][q] = *reinterpret_cast<const u32x4 *>(sact + ((int64_t)m * g.K * 2 + apos(b, q)));
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const float sc = e8m0_scale_f32(e[u][r]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // dword q of the block: codes 8q .. 8q+7, low nibble first
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const v2bf d = p == 0 ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[u][r][q], sc, 0)
                                     : p == 1 ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[u][r][q], sc, 1)
                                     : p == 2 ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[u][r][q], sc, 2)
                                              : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[u][r][q], sc, 3);
#pragma unroll
                        for (int m = 0; m < VM; ++m) {  // activations 8q + 2p, 8q + 2p + 1 of the block
                            const u32x4 aq = av[m][q];
                            const uint32_t ap = p == 0 ? aq.x : p == 1 ? aq.y : p == 2 ? aq.z : aq.w;
                            acc[r][m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, ap), d, acc[r][m], false);
                        }
                    }
                }
            }
        }
        b0 += 64 * UB;
        if (b0 < nblk) wload(b0);
    }

#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int m = 0; m < VM; ++m) acc[r][m] = wave_sum_fixed(acc[r][m]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int64_t n = n0 + r;
            if (n >= g.N) continue;
#pragma unroll
            for (int m = 0; m < VM; ++m) {
                if (m >= (dual ? 2 * g.M : g.M)) continue;
                const bool second = dual && m >= (int)g.M;
                const int64_t idx = (int64_t)(second ? m - g.M : m) * g.ldc + n;
                store_cw<CT>(second ? g.c1 : g.c, idx, acc[r][m]);
            }
        }
    }
}

// one activation row per batch (from two rows on the decode kernel is faster)
constexpr int64_t kGemvMaxM = 1;
constexpr int64_t kGemvMaxLds = 64 * 1024;   // activation bytes staged per workgroup

static hipError_t launch_gemv(const GemmArgs &g, hipStream_t s) {
    const int vm = (int)(g.a1 ? 2 * g.M : g.M);
    const int vmt = vm == 1 ? 1 : vm == 2 ? 2 : 4;
    const size_t lds = (size_t)vmt * g.K * 2;
    const int rows_per_wg = (gv::NT / 64) * gv::RPW;
    const dim3 grid((unsigned)((g.N + rows_per_wg - 1) / rows_per_wg)), blk(gv::NT);
    const bool f = g.scale_fmt == LSMX_SCALE_F32;
#define LSMX_V(VMT, F, CT) hipLaunchKernelGGL((gemv_bf16f4_kernel<VMT, F, CT>), grid, blk, lds, s, g)
#define LSMX_VC(VMT, F)                                               \
    do {                                                              \
        if (g.c_dtype == LSMX_F32) LSMX_V(VMT, F, LSMX_F32);          \
        else if (g.c_dtype == LSMX_BF16) LSMX_V(VMT, F, LSMX_BF16);   \
        else LSMX_V(VMT, F, LSMX_F16);                                \
    } while (0)
    if (vmt == 1) { if (f) LSMX_VC(1, true); else LSMX_VC(1, false); }
    else if (vmt == 2) { if (f) LSMX_VC(2, true); else LSMX_VC(2, false); }
    else { if (f) LSMX_VC(4, true); else LSMX_VC(4, false); }
#undef LSMX_VC
#undef LSMX_V
    return hipGetLastError();
}

// up to 32 rows per batch (M = 16 against a 14336 x 4096 weight: 20 us against 34 us for the 128-row
// ring tile, whose MFMAs would be 7/8 padding; from M = 64 the ring is faster)
constexpr int64_t kSkinnyMaxM = 32;

static int num_cus_w() {
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

static hipError_t launch_skinny(const GemmArgs &g, hipStream_t s) {
    const int64_t vm = g.a1 ? 2 * g.M : g.M;
    const int mt = vm <= 16 ? 1 : vm <= 32 ? 2 : vm <= 64 ? 4 : 8;
    // two 16-row weight tiles per workgroup (the activation loads then serve
    // twice the weight bytes) while that still gives every CU a workgroup;
    // MT <= 2 keeps two workgroups resident per CU either way
    const int ct = (mt <= 4 && (g.N + 31) / 32 >= num_cus_w()) ? 2 : 1;
    const dim3 grid((unsigned)((g.N + 16 * ct - 1) / (16 * ct))), blk(64 * sk::WK);
#define LSMX_S(MT, CT) hipLaunchKernelGGL((gemm_bf16f4_skinny_kernel<MT, CT>), grid, blk, 0, s, g)
    switch (mt * 10 + ct) {
        case 11: LSMX_S(1, 1); break;
        case 12: LSMX_S(1, 2); break;
        case 21: LSMX_S(2, 1); break;
        case 22: LSMX_S(2, 2); break;
        case 41: LSMX_S(4, 1); break;
        case 42: LSMX_S(4, 2); break;
        default: LSMX_S(8, 1); break;
    }
#undef LSMX_S
    return hipGetLastError();
}

template <int NB, int BR, int BN>
static hipError_t launch_w4(const GemmArgs &g, hipStream_t s) {
    constexpr int RPB = BR / NB;
    const int tiles = (int)(((g.M + RPB - 1) / RPB) * ((g.N + BN - 1) / BN));
    const dim3 grid(tiles), blk(w4::NT);
    const bool f = g.scale_fmt == LSMX_SCALE_F32;
#define LSMX_W(F, CT) hipLaunchKernelGGL((gemm_bf16f4_kernel<NB, F, CT, BR, BN>), grid, blk, 0, s, g)
    if (f) {
        if (g.c_dtype == LSMX_F32) LSMX_W(true, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_W(true, LSMX_BF16);
        else LSMX_W(true, LSMX_F16);
    } else {
        if (g.c_dtype == LSMX_F32) LSMX_W(false, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_W(false, LSMX_BF16);
        else LSMX_W(false, LSMX_F16);
    }
#undef LSMX_W
    return hipGetLastError();
}

// the ring kernel (256 x 256 tiles) from half a wave of tiles on, else the
// largest VGPR-staged tile that still gives every CU a workgroup: 256 x 256,
// then 128 x 128, then 128 x 64 (mid M, e.g. 128 rows against 14336 columns)
template <int NB>
static hipError_t launch_w4_any(const GemmArgs &g, hipStream_t s) {
    auto tiles = [&](int br, int bn) { return ((g.M + br / NB - 1) / (br / NB)) * ((g.N + bn - 1) / bn); };
    const int64_t cus = num_cus_w();
    // the ring kernel is worth it from half a wave of 256 x 256 tiles on (M = 1024, N = 14336: 224 tiles)
    // single form whose 256 x 256 tiles leave CUs idle while 128 x 256 tiles
    // still fit in one wave of workgroups: 128-row tiles, 1 x 8 waves (each
    // all 128 rows and a 32-column strip), loads from waves 0-3.  cfg2's
    // single batch (M = 2048 against a 4096 x 4096 weight, 128 -> 256
    // workgroups) 97 -> 63 us; M = 1024 against 8192 x 4096 91 -> 62 us
    if constexpr (NB == 1)
        if (ring_ok(g) && tiles(256, 256) < cus && tiles(128, 256) <= cus &&
            2 * tiles(128, 256) > cus)
            return launch_ring<NB, 128, 256, 4, 1, 4>(g, s);
    if (ring_ok(g) && 2 * tiles(256, 256) >= cus) return launch_ring<NB, 256, 256, 3, 2, 4>(g, s);
    if (tiles(256, 256) >= cus) return launch_w4<NB, 256, 256>(g, s);
    if (tiles(128, 128) >= cus) return launch_w4<NB, 128, 128>(g, s);
    // a few hundred rows: 128 x 64 tiles through a 4-slot DMA ring (N =
    // 14336, K = 4096, M = 128: 48 -> 38 us; M = 64: 44 -> 35 us against the skinny kernel)
    if (ring_ok(g)) return launch_ring<NB, 128, 64, 4>(g, s);
    return launch_w4<NB, 128, 64>(g, s);
}

// ------------------------------------------------------------------ split-K
// A few hundred activation rows against a wide weight (M = 128, N = 14336:
// 56 output tiles of 128 x 256 for 256 CUs) leave most CUs idle with whole-K
// tiles, and narrower tiles make every CU re-read the whole activation
// panel.  Instead each output tile of 128 rows (per batch) by 256 or 128
// weight columns is cut into 2 or 4 K slices (>= 512 deep, a whole group of
// E8M0 scale loads), one workgroup each; the fp32 partial tiles meet in a
// caller-provided workspace.  Of the plans that fit one wave of workgroups,
// the one with the most workgroups wins, and among those the one with the
// fewest partial bytes: M = 128 against N = 14336 runs 112 tiles of 128 x
// 128 in 2 slices (224 workgroups, 14.7 MB of partials) rather than 56 tiles
// of 128 x 256 in 4.  The plan depends on M, N and K only (128-row tiles per
// batch in both forms), so the single and the dual launch of one M give
// identical bits.
struct SplitPlan {
    int splits, bn;
};
static SplitPlan splitk_plan(int64_t M, int64_t N, int64_t K) {
    SplitPlan best{1, 256};
    if (M <= kSkinnyMaxM || midm_shape(M, N, K)) return best;  // the GEMV, decode, mid-M and skinny kernels own these
    const int64_t mt = (M + 127) / 128, cus = num_cus_w();
    if (2 * mt * ((N + 255) / 256) > cus) return best;  // whole-K tiles fill half of the CUs
    int64_t best_wg = 0, best_bytes = 0;
    for (int bn = 256; bn >= 128; bn /= 2)
        for (int sp = 2; sp <= 4; sp *= 2) {
            const int64_t nt = (N + bn - 1) / bn, wg = mt * nt * sp, bytes = sp * nt * bn;
            if (wg > cus || K % (512 * sp) != 0) continue;
            if (wg > best_wg || (wg == best_wg && bytes < best_bytes)) {
                best = SplitPlan{sp, bn};
                best_wg = wg;
                best_bytes = bytes;
            }
        }
    return best;
}
int gemm_bf16f4_splits(int64_t M, int64_t N, int64_t K, bool /*dual*/) { return splitk_plan(M, N, K).splits; }

// Workspace: the fp32 partial tiles [splits][NB][Mp][Np] (Mp = M rounded up
// to 128 rows, Np = N rounded up to the plan's tile width).
int64_t gemm_bf16f4_workspace(int64_t M, int64_t N, int64_t K, bool dual) {
    const SplitPlan p = splitk_plan(M, N, K);
    if (p.splits < 2) return 0;
    return (int64_t)p.splits * (dual ? 2 : 1) * ((M + 127) / 128 * 128) * ((N + p.bn - 1) / p.bn * p.bn) * 4;
}

// C[b][m][n] = sum over slices s = 0, 1, ... of partial[s][b][m][n], in that
// order: 4 consecutive columns per thread, one 16-byte load per slice.  A
// workgroup covers 1024 columns of one output row: workgroup x is row
// x / cb (cb workgroups per row), so the row and batch come from scalar
// 32-bit divisions of uniform values and the loads issue at once (64-bit
// per-thread divisions put ~1 us of index arithmetic in front of them).
template <int CT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ ws, int splits, int nb,
                                                            int64_t Mp, int64_t Np, void *c0, void *c1, int64_t ldc,
                                                            int64_t M, int64_t N) {
    const uint32_t cb = (uint32_t)((Np / 4 + 255) / 256);   // workgroups per output row
    const uint32_t row = blockIdx.x / cb, b = row / (uint32_t)M;
    const int64_t m = row - b * (uint32_t)M;
    const int64_t n = ((int64_t)(blockIdx.x - row * cb) * 256 + threadIdx.x) * 4;
    if ((int)b >= nb || n >= N) return;
    const float *p = ws + (b * Mp + m) * Np + n;
    const int64_t slice = (int64_t)nb * Mp * Np;
    u32x4 v = *reinterpret_cast<const u32x4 *>(p);
    float x[4] = {u2f(v.x), u2f(v.y), u2f(v.z), u2f(v.w)};
    for (int s = 1; s < splits; ++s) {
        v = *reinterpret_cast<const u32x4 *>(p + s * slice);
        x[0] += u2f(v.x);
        x[1] += u2f(v.y);
        x[2] += u2f(v.z);
        x[3] += u2f(v.w);
    }
    void *c = b ? c1 : c0;
    const int64_t idx = m * ldc + n;
    if (n + 4 <= N && (((uintptr_t)c + idx * (CT == LSMX_F32 ? 4 : 2)) & (CT == LSMX_F32 ? 15 : 7)) == 0) {
        store_c4<CT>(c, idx, x[0], x[1], x[2], x[3]);
    } else {
        for (int k = 0; k < 4 && n + k < N; ++k) store_c<CT>(c, idx + k, x[k]);
    }
}

// Ring depth of the single form's split-K kernel (24 KiB per slot): 3 and 4
// slots time within 3% of each other for M = 64 .. 256 against a 14336 x
// 4096 weight, 4 the faster, so the loads in flight do not set its pace
// (deeper rings would need the scale loads issued earlier).  The dual form's
// 40 KiB slots fit 3.
// Wave layouts of the split-K tiles: 128 x 256 single, 1 x 8 waves (each all
// 128 rows and a 32-column strip, so each weight fragment is dequantized
// once); 128 x 128 single, 2 x 4 (64 x 32 per wave); dual (256 A rows), 4 x 2
// waves for both widths.
template <int NB, int BN>
static hipError_t launch_ring_splitk(GemmArgs g, int splits, hipStream_t s) {
    constexpr int BR = 128 * NB;
    constexpr int WGM = NB == 2 ? 4 : (BN == 256 ? 1 : 2);
    constexpr int SL = NB == 1 ? 4 : 3;
    const int64_t tiles = ((g.M + 127) / 128) * ((g.N + BN - 1) / BN);
    g.splits = splits;
    g.k_split = g.K / splits;
    const dim3 grid((unsigned)(tiles * splits)), blk(wr::NT);
    const int64_t Mp = (g.M + 127) / 128 * 128, Np = (g.N + BN - 1) / BN * BN;
    const dim3 rgrid((unsigned)(NB * g.M * ((Np / 4 + 255) / 256))), rblk(256);
#define LSMX_RS(CT)                                                                                              \
    do {                                                                                                         \
        hipLaunchKernelGGL((gemm_bf16f4_ring_kernel<NB, CT, BR, BN, SL, true, WGM>), grid, blk, 0, s, g);        \
        hipLaunchKernelGGL((splitk_reduce_kernel<CT>), rgrid, rblk, 0, s, g.ws, splits, NB, Mp, Np, g.c, g.c1, \
                           g.ldc, g.M, g.N);                                                                     \
    } while (0)
    if (g.c_dtype == LSMX_F32) LSMX_RS(LSMX_F32);
    else if (g.c_dtype == LSMX_BF16) LSMX_RS(LSMX_BF16);
    else LSMX_RS(LSMX_F16);
#undef LSMX_RS
    return hipGetLastError();
}
template <int NB>
static hipError_t launch_ring_splitk(GemmArgs g, SplitPlan p, hipStream_t s) {
    return p.bn == 256 ? launch_ring_splitk<NB, 256>(g, p.splits, s) : launch_ring_splitk<NB, 128>(g, p.splits, s);
}

hipError_t launch_gemm_bf16f4(const GemmArgs &g, hipStream_t s) {
    // the same M picks the same kernel for the single and the dual form
    // GEMV when the dual form's 2M activation rows of K bf16 fit in LDS (the
    // test depends on M and K only, so single and dual launches agree)
    if (g.M <= kGemvMaxM && 2 * g.M * g.K * 2 <= kGemvMaxLds) return launch_gemv(g, s);
    if (g.M <= kDecodeMaxM && decode_ok(g)) return launch_decode(g, s);
    if (midm_ok(g)) return launch_midm(g, s);
    if (g.M <= kSkinnyMaxM && (g.a1 ? 2 * g.M : g.M) <= 128) return launch_skinny(g, s);
    if (g.ws && ring_ok(g)) {
        const SplitPlan p = splitk_plan(g.M, g.N, g.K);
        if (p.splits > 1) return g.a1 ? launch_ring_splitk<2>(g, p, s) : launch_ring_splitk<1>(g, p, s);
    }
    return g.a1 ? launch_w4_any<2>(g, s) : launch_w4_any<1>(g, s);
}

}  // namespace lsmx
