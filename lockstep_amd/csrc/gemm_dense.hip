// Dense GEMMs with fp32 accumulation on gfx950's MFMA: the kernels behind the
// reference's dual_gemm.py family and mxfp4_gemm_fp8.
//
//   single        C  = A0 . Bt0^T                       dual_gemm.py:189-226 (gemm)
//   dual packed   C  = A0 . Bt0^T + A1 . Bt1^T  (one accumulator)
//                                                       dual_gemm.py:43-72, 230-241
//   dual separate C0 = A0 . Bt0^T,  C1 = A1 . Bt1^T      dual_gemm.py:79-110, 244-255
//   split-K       any of the above over K slices, fp32 atomic adds into a
//                 zeroed output                          dual_gemm.py:118-179, 261-289
//   fp8 scaled    C  = sum_kb sa[m,kb] sb[n,kb] (A_kb . Bt_kb), E4M3 operands,
//                 E8M0 block scales                      mxfp4_gemm.py:29-87
//
// Operands are K-contiguous: A [M, lda], Bt [N, ldb].  The reference takes B
// as [K, N] (N-contiguous); the Python layer hands a transposed copy (or the
// K-contiguous tensor B is a view of) to these kernels.
//
// Element types: bf16 and fp16 (v_mfma_f32_32x32x16_{bf16,f16}: each lane
// supplies 8 consecutive K of one row) and E4M3 (v_mfma_scale_f32_32x32x64_
// f8f6f4 with cbsz = blgp = 0: each lane supplies 16 K of each of the two
// 32-blocks, and the E8M0 scale of block lane / 32, 127 = 1.0 when unscaled).
//
// Tiling: 128 x 128 per workgroup of 4 waves (2 x 2, 64 x 64 per wave, 2 x 2
// MFMA tiles of 32 x 32).  A stage is 64 elements of K (128 bytes of a bf16
// row, 64 of an E4M3 row), staged through VGPRs into a double-buffered LDS
// tile; the next stage's global loads are in flight while this one computes.
// Rows past M or N are clamped to the last row (their outputs are not
// stored).  LDS rows are XOR-swizzled by 16-byte chunk.
#include "lsmx_internal.h"

namespace lsmx {

namespace dn {
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BKE = 64;  // tile and stage (elements of K)
constexpr int NT = 256;                       // 4 waves
constexpr int TM = 2, TN = 2;                 // 32 x 32 MFMA tiles per wave

LSMX_DEV int swz(int row, int cpr) { return (row >> 1) & (cpr - 1); }

template <int DT>
struct Ty {
    static constexpr int es = DT == LSMX_E4M3 ? 1 : 2;  // element bytes
    static constexpr int RB = BKE * es;                  // bytes per row per stage
    static constexpr int CPR = RB / 16;                  // 16-byte chunks per row
    static constexpr int KS = DT == LSMX_E4M3 ? 1 : 4;   // MFMA K-steps per stage
    static constexpr int LPT = BM * RB / 16 / NT;        // 16-byte loads per thread per operand
};

template <int DT>
LSMX_DEV v16f mma(const u32x4 (&a)[2], const u32x4 (&b)[2], v16f c, uint32_t sa, uint32_t sb) {
    if constexpr (DT == LSMX_BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[0]), __builtin_bit_cast(v8bf, b[0]), c,
                                                       0, 0, 0);
    } else if constexpr (DT == LSMX_F16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[0]), __builtin_bit_cast(v8h, b[0]), c,
                                                      0, 0, 0);
    } else {
        const v8i va = v8i{(int)a[0][0], (int)a[0][1], (int)a[0][2], (int)a[0][3],
                           (int)a[1][0], (int)a[1][1], (int)a[1][2], (int)a[1][3]};
        const v8i vb = v8i{(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3],
                           (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]};
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, vb, c, 0, 0, 0, (int)sa, 0, (int)sb);
    }
}

LSMX_DEV uint32_t bf16_bits(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f); }
LSMX_DEV uint32_t f16_bits(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f); }

template <int CT, bool ATOMIC>
LSMX_DEV void put(void *c, int64_t idx, float v) {
    if constexpr (ATOMIC) {
        __hip_atomic_fetch_add(reinterpret_cast<float *>(c) + idx, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (CT == LSMX_F32) {
        reinterpret_cast<float *>(c)[idx] = v;
    } else if constexpr (CT == LSMX_BF16) {
        reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)bf16_bits(v);
    } else {
        reinterpret_cast<uint16_t *>(c)[idx] = (uint16_t)f16_bits(v);
    }
}
}  // namespace dn

// MODE: 0 single, 1 dual packed, 2 dual separate.  SHB: the two B operands
// are one tensor (the shared-weight form, train_step.py:52-53): each B tile is
// loaded once and feeds both products.  SCALED: E8M0 block scales (E4M3
// only).  ATOMIC: split-K partial sums added into a zeroed fp32 output.
template <int DT, int MODE, bool SHB>
constexpr int dense_lds_bytes() {
    return 2 * ((MODE == 0 ? 1 : 2) + (MODE == 0 || SHB ? 1 : 2)) * dn::BM * dn::Ty<DT>::RB;
}

// two workgroups per CU while both fit in the 160 KiB of LDS
template <int DT, int MODE, bool SHB, bool SCALED, int CT, bool ATOMIC>
__global__ __launch_bounds__(dn::NT, (dense_lds_bytes<DT, MODE, SHB>() <= 80 * 1024 ? 2 : 1)) void gemm_dense_kernel(
    DenseArgs g) {
    using namespace dn;
    using T = Ty<DT>;
    constexpr int NO = MODE == 0 ? 1 : 2;      // A operands
    constexpr int NOB = SHB ? 1 : NO;          // B operands
    constexpr int NACC = MODE == 2 ? 2 : 1;    // accumulators
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][NO][BM * T::RB];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][NOB][BN * T::RB];

    const int tiles_m = (int)((g.M + BM - 1) / BM), tiles_n = (int)((g.N + BN - 1) / BN);
    int tm, tn;
    {
        // groups of 8 tile rows share B panels in L2
        const int pid = (int)blockIdx.x, per_group = 8 * tiles_n;
        const int group = pid / per_group, first = group * 8;
        const int gsz = min(tiles_m - first, 8);
        tm = first + (pid - group * per_group) % gsz;
        tn = (pid - group * per_group) / gsz;
    }
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t k_begin = (int64_t)blockIdx.y * g.k_split;
    const int nk = (int)(g.k_split / BKE);

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int frow = lane & 31, half = lane >> 5;

    // staging: load q of thread t covers 16 bytes of row (q*NT + t) / CPR
    const uint8_t *ga[NO][T::LPT], *gb[NOB][T::LPT];
    int soff[T::LPT];
#pragma unroll
    for (int q = 0; q < T::LPT; ++q) {
        const int idx = q * NT + t;
        const int row = idx / T::CPR, c = idx % T::CPR;
        soff[q] = row * T::RB + ((c ^ swz(row, T::CPR)) << 4);
        const int64_t ra = min(m0 + row, g.M - 1), rb = min(n0 + row, g.N - 1);
#pragma unroll
        for (int o = 0; o < NO; ++o) ga[o][q] = (o ? g.a1 : g.a0) + (ra * g.lda + k_begin) * T::es + c * 16;
#pragma unroll
        for (int o = 0; o < NOB; ++o) gb[o][q] = (o ? g.b1 : g.b0) + (rb * g.ldb + k_begin) * T::es + c * 16;
    }
    u32x4 ra_[NO][T::LPT], rb_[NOB][T::LPT];
    auto gload = [&](int kt) __attribute__((always_inline)) {
        const int64_t off = (int64_t)kt * T::RB;
#pragma unroll
        for (int q = 0; q < T::LPT; ++q) {
#pragma unroll
            for (int o = 0; o < NO; ++o) ra_[o][q] = *reinterpret_cast<const u32x4 *>(ga[o][q] + off);
#pragma unroll
            for (int o = 0; o < NOB; ++o) rb_[o][q] = *reinterpret_cast<const u32x4 *>(gb[o][q] + off);
        }
    };
    auto swrite = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < T::LPT; ++q) {
#pragma unroll
            for (int o = 0; o < NO; ++o) *reinterpret_cast<u32x4 *>(&sA[buf][o][soff[q]]) = ra_[o][q];
#pragma unroll
            for (int o = 0; o < NOB; ++o) *reinterpret_cast<u32x4 *>(&sB[buf][o][soff[q]]) = rb_[o][q];
        }
    };
    // fragment of K-step s for tile row r: bf16/f16 one 16-byte chunk (8
    // elements at 16s + 8h); E4M3 two chunks, elements 16h + [0, 16) of
    // 32-block 0 in VGPRs 0-3 and 32 + 16h + [0, 16) of block 1 in VGPRs 4-7
    // (the f8f6f4 MFMA's K order for 8-bit operands; lane half h carries the
    // scale of block h)
    auto frag = [&](const uint8_t *tile, int r, int s, u32x4 (&f)[2]) __attribute__((always_inline)) {
        if constexpr (DT == LSMX_E4M3) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
                f[j] = *reinterpret_cast<const u32x4 *>(tile + r * T::RB + (((2 * j + half) ^ swz(r, T::CPR)) << 4));
        } else {
            f[0] = *reinterpret_cast<const u32x4 *>(tile + r * T::RB + (((2 * s + half) ^ swz(r, T::CPR)) << 4));
        }
    };
    // E8M0 scale of block (k / 32) for a tile row: lane half h covers block 2*kt + h
    auto scale_of = [&](const uint8_t *s, int64_t ld, int64_t row, int kt) __attribute__((always_inline)) -> uint32_t {
        if constexpr (SCALED) return s[row * ld + (k_begin / 32) + 2 * kt + half];  // one byte, L2-resident
        else return 127u;
    };

    v16f acc[NACC][TM][TN];
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[a][i][j][e] = 0.0f;

    // block scales are loaded one stage ahead, with that stage's operands
    uint32_t sa[TM], sb[TN], nsa[TM], nsb[TN];
    auto sload = [&](int kt, uint32_t (&xa)[TM], uint32_t (&xb)[TN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i) xa[i] = scale_of(g.sa, g.ld_sa, min(m0 + wm * 64 + i * 32 + frow, g.M - 1), kt);
#pragma unroll
        for (int j = 0; j < TN; ++j) xb[j] = scale_of(g.sb, g.ld_sb, min(n0 + wn * 64 + j * 32 + frow, g.N - 1), kt);
    };
    gload(0);
    sload(0, sa, sb);
    swrite(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) {
            gload(kt + 1);
            sload(kt + 1, nsa, nsb);
        }
        // product by product over the 64-deep stage: in MODE 1 the stage's
        // A0.B0 block is added before its A1.B1 block, the order of the
        // reference's loop (dual_gemm.py:59-61)
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int ai = MODE == 2 ? o : 0, bi = SHB ? 0 : o;
#pragma unroll
            for (int s = 0; s < T::KS; ++s) {
                u32x4 fa[TM][2], fb[TN][2];
#pragma unroll
                for (int j = 0; j < TN; ++j) frag(sB[buf][bi], wn * 64 + j * 32 + frow, s, fb[j]);
#pragma unroll
                for (int i = 0; i < TM; ++i) frag(sA[buf][o], wm * 64 + i * 32 + frow, s, fa[i]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[ai][i][j] = mma<DT>(fa[i], fb[j], acc[ai][i][j], sa[i], sb[j]);
            }
        }
        if (kt + 1 < nk) {
            swrite(buf ^ 1);
#pragma unroll
            for (int i = 0; i < TM; ++i) sa[i] = nsa[i];
#pragma unroll
            for (int j = 0; j < TN; ++j) sb[j] = nsb[j];
        }
        __syncthreads();
    }

    // epilogue: acc element e of tile (i, j) is row i*32 + 8*(e/4) + 4*half + e%4, column j*32 + frow
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
        void *c = a ? g.c1 : g.c0;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int64_t col = n0 + wn * 64 + j * 32 + frow;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                    if (row < g.M && col < g.N) put<CT, ATOMIC>(c, row * g.ldc + col, acc[a][i][j][e]);
                }
            }
    }
}

// y[cols, ldy] = x[rows, ldx]^T through a 64 x 64 LDS tile.  Full tiles of
// 16-byte aligned rows: each thread loads 16 bytes of a row; the tile sits in
// LDS as dwords of E = 4 / sizeof(T) consecutive elements, one padding dword
// per row, so that the dword column reads below touch 64 distinct banks.  A
// thread then reads E dwords down one dword column (E consecutive rows),
// transposes that E x E block in registers (v_perm_b32) and writes one dword
// to each of E output rows; consecutive lanes take consecutive row blocks,
// so each output row receives 64 (bytes), 128 (16-bit) or 256 (32-bit)
// contiguous bytes per store instruction.  Edge tiles and unaligned operands
// go element by element.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T *__restrict__ x, int64_t rows, int64_t cols,
                                                        int64_t ldx, T *__restrict__ y, int64_t ldy, int vec) {
    constexpr int E = 4 / (int)sizeof(T);    // elements per dword
    constexpr int WPR = 64 / E;              // dwords per tile row
    constexpr int P = WPR + 1;               // padded LDS row, in dwords
    __shared__ uint32_t tile[64 * P];
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const int t = threadIdx.x;
    const bool full = vec && r0 + 64 <= rows && c0 + 64 <= cols;
    if (full) {
        for (int q = t; q < 64 * WPR / 4; q += 256) {
            const int r = q / (WPR / 4), w4 = (q % (WPR / 4)) * 4;
            const uint4 v = *reinterpret_cast<const uint4 *>(x + (r0 + r) * ldx + c0 + w4 * E);
            uint32_t *d = &tile[r * P + w4];
            d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
        }
        __syncthreads();
        for (int q = t; q < (64 / E) * WPR; q += 256) {
            const int p = q % (64 / E), w = q / (64 / E);   // rows E*p .., dword column w
            uint32_t a[E], o[E];
#pragma unroll
            for (int k = 0; k < E; ++k) a[k] = tile[(E * p + k) * P + w];
            if constexpr (E == 4) {
                // o[i] = byte i of a[0], a[1], a[2], a[3]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t sel = 0x0C0C0000u | ((uint32_t)(4 + i) << 8) | (uint32_t)i;
                    o[i] = __builtin_amdgcn_perm(a[1], a[0], sel) | (__builtin_amdgcn_perm(a[3], a[2], sel) << 16);
                }
            } else if constexpr (E == 2) {
                o[0] = __builtin_amdgcn_perm(a[1], a[0], 0x05040100u);
                o[1] = __builtin_amdgcn_perm(a[1], a[0], 0x07060302u);
            } else {
                o[0] = a[0];
            }
#pragma unroll
            for (int i = 0; i < E; ++i)
                *reinterpret_cast<uint32_t *>(y + (c0 + E * w + i) * ldy + r0 + E * p) = o[i];
        }
        return;
    }
    // element by element through a [64][65] view of the same LDS
    T *te = reinterpret_cast<T *>(tile);
    constexpr int PE = 65;
    static_assert(64 * PE * sizeof(T) <= sizeof(tile), "edge-tile view fits");
    for (int q = t; q < 64 * 64; q += 256) {
        const int r = q / 64, cc = q % 64;
        if (r0 + r < rows && c0 + cc < cols) te[r * PE + cc] = x[(r0 + r) * ldx + c0 + cc];
    }
    __syncthreads();
    for (int q = t; q < 64 * 64; q += 256) {
        const int oc = q / 64, rr = q % 64;   // output row oc = input column, element rr
        if (c0 + oc < cols && r0 + rr < rows) y[(c0 + oc) * ldy + r0 + rr] = te[rr * PE + oc];
    }
}

// E8M0 bytes of fp32 power-of-two scales (their exponent field).  Element
// (r, c) of s is the scale of (output row r, block c), or of (block r, output
// row c) with LSMX_E8M0_IN_T; the output is row-major [out rows, ldo] or,
// with LSMX_E8M0_OUT_KMAJOR, K-major [blocks/4, ldo, 4].  The quantizer's
// scales 2^e, e in [-127, 127], convert exactly (2^-127 is the subnormal
// 0x00400000 -> 0).  A scale that is not a positive power of two in that
// range has no E8M0 form: it becomes 0xFF, E8M0's NaN, so every output that
// depends on it is NaN rather than silently wrong.
__global__ void scale_to_e8m0_kernel(const float *__restrict__ s, int64_t rows, int64_t cols, int64_t lds,
                                     int layout, uint8_t *__restrict__ out, int64_t ldo) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i - r * cols;
    const uint8_t e = (uint8_t)f32_scale_e8m0(f2u(s[r * lds + c]));
    const bool tin = layout & LSMX_E8M0_IN_T;
    const int64_t orow = tin ? c : r, blk = tin ? r : c;
    if (layout & LSMX_E8M0_OUT_KMAJOR) out[((blk >> 2) * ldo + orow) * 4 + (blk & 3)] = e;
    else out[orow * ldo + blk] = e;
}

// The K-major output four blocks at a time: thread i converts blocks 4g ..
// 4g+3 of output row o (o = i mod orows, g = i / orows) and writes their
// dword, so that consecutive threads write consecutive dwords (and, for
// transposed input, read consecutive floats).  The number of blocks is a
// multiple of 4.
__global__ void scale_to_e8m0_km4_kernel(const float *__restrict__ s, int64_t orows, int64_t groups, int64_t lds,
                                         bool tin, uint8_t *__restrict__ out, int64_t ldo, bool out4) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= orows * groups) return;
    const int64_t g = i / orows, o = i - g * orows;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t blk = 4 * g + k;
        w |= f32_scale_e8m0(f2u(tin ? s[blk * lds + o] : s[o * lds + blk])) << (8 * k);
    }
    uint8_t *d = out + (g * ldo + o) * 4;
    if (out4) {
        *reinterpret_cast<uint32_t *>(d) = w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = (uint8_t)(w >> (8 * k));
    }
}

// Row-major fp32 scales [orows, 4 * groups] -> K-major E8M0 dwords
// [groups][orows] through an LDS tile of 64 rows x 16 dword groups: the
// reads are 256 contiguous bytes of a row per 16 threads and the writes 64
// consecutive dwords of a group per 64 threads (the direct mapping above
// read each row's 16 bytes from a different thread 64 rows apart and ran at
// 1.3 TB/s).
__global__ __launch_bounds__(256) void scale_to_e8m0_km4_tiled_kernel(const float *__restrict__ s, int64_t orows,
                                                                      int64_t groups, int64_t lds,
                                                                      uint8_t *__restrict__ out, int64_t ldo) {
    __shared__ uint32_t tile[16][65];
    const int t = threadIdx.x;
    const int64_t o0 = (int64_t)blockIdx.x * 64, g0 = (int64_t)blockIdx.y * 16;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t, r = idx >> 4, gi = idx & 15;
        const int64_t o = o0 + r, gr = g0 + gi;
        if (o < orows && gr < groups) {
            const float4 v = *reinterpret_cast<const float4 *>(s + o * lds + 4 * gr);
            tile[gi][r] = f32_scale_e8m0(f2u(v.x)) | (f32_scale_e8m0(f2u(v.y)) << 8) |
                          (f32_scale_e8m0(f2u(v.z)) << 16) | (f32_scale_e8m0(f2u(v.w)) << 24);
        }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t, gi = idx >> 6, r = idx & 63;
        const int64_t o = o0 + r, gr = g0 + gi;
        if (o < orows && gr < groups) *reinterpret_cast<uint32_t *>(out + (gr * ldo + o) * 4) = tile[gi][r];
    }
}

// Up to four fp32 scale tensors -> K-major E8M0 dwords in one launch (the A
// and B scales of one GEMM call).  A workgroup converts 64 output rows x 16
// four-block groups of one tensor through a dword tile in LDS (one padding
// dword per group row): row-major input with 16-byte rows is read as in
// scale_to_e8m0_km4_tiled_kernel (four blocks per float4, 256 contiguous
// bytes per 16 threads); [blocks, rows] input (tin) one float per thread, 64
// consecutive rows of a block per wave, each lane writing a byte of its own
// dword.  The stores are 64 consecutive dwords of a group.  A scale with no
// E8M0 form becomes 0xFF as above and, unless it is a NaN (which E8M0 has,
// with the same effect on every output that uses it), makes the wave that
// met it write the caller's epoch to the flag (one store per wave), which
// the promotion GEMM that follows checks.
__global__ __launch_bounds__(256) void scale_to_e8m0_batch_kernel(E8m0Batch b) {
    __shared__ uint32_t tile[16][65];
    const int64_t blk = (int64_t)blockIdx.x;
    int k = 0;
    while (k + 1 < b.n && blk >= b.end[k]) ++k;
    const E8m0Item &it = b.it[k];
    const int64_t local = blk - (k ? b.end[k - 1] : 0);
    const int64_t tiles_o = (it.orows + 63) / 64;
    const int64_t o0 = (local % tiles_o) * 64, g0 = (local / tiles_o) * 16;
    const int t = threadIdx.x;
    bool bad = false;
    if (it.tin) {
        uint8_t *tb = reinterpret_cast<uint8_t *>(tile);
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const int q = i * 256 + t, r = q & 63, c = q >> 6;  // out row, block in tile
            const int64_t o = o0 + r, bk = 4 * g0 + c;
            if (o < it.orows && bk < 4 * it.groups) {
                const uint32_t x = f2u(it.s[bk * it.lds + o]), e = f32_scale_e8m0(x);
                bad |= e == 0xFFu && (x & 0x7FFFFFFFu) <= 0x7F800000u;
                tb[((c >> 2) * 65 + r) * 4 + (c & 3)] = (uint8_t)e;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = i * 256 + t, r = q >> 4, gi = q & 15;
            const int64_t o = o0 + r, gr = g0 + gi;
            if (o < it.orows && gr < it.groups) {
                uint32_t x[4];
                if (it.vec4) {
                    const float4 v = *reinterpret_cast<const float4 *>(it.s + o * it.lds + 4 * gr);
                    x[0] = f2u(v.x), x[1] = f2u(v.y), x[2] = f2u(v.z), x[3] = f2u(v.w);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[j] = f2u(it.s[o * it.lds + 4 * gr + j]);
                }
                uint32_t w = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t e = f32_scale_e8m0(x[j]);
                    bad |= e == 0xFFu && (x[j] & 0x7FFFFFFFu) <= 0x7F800000u;
                    w |= e << (8 * j);
                }
                tile[gi][r] = w;
            }
        }
    }
    if (b.flag) {
        const uint64_t m = __ballot(bad);
        if (m && (t & 63) == __builtin_ctzll(m)) *b.flag = b.epoch;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = i * 256 + t, gi = q >> 6, r = q & 63;
        const int64_t o = o0 + r, gr = g0 + gi;
        if (o < it.orows && gr < it.groups) *reinterpret_cast<uint32_t *>(it.out + (gr * it.ldo + o) * 4) = tile[gi][r];
    }
}

hipError_t launch_scale_to_e8m0_batch(const E8m0Batch &b, hipStream_t s) {
    hipLaunchKernelGGL(scale_to_e8m0_batch_kernel, dim3((unsigned)b.end[b.n - 1]), dim3(256), 0, s, b);
    return hipGetLastError();
}

template <int DT, int MODE, bool SHB, bool SCALED, int CT, bool ATOMIC>
static void launch_d(const DenseArgs &g, hipStream_t s) {
    const int tiles = (int)(((g.M + dn::BM - 1) / dn::BM) * ((g.N + dn::BN - 1) / dn::BN));
    const int splits = (int)(g.K / g.k_split);
    hipLaunchKernelGGL((gemm_dense_kernel<DT, MODE, SHB, SCALED, CT, ATOMIC>), dim3(tiles, splits), dim3(dn::NT), 0,
                       s, g);
}

template <int DT, int MODE, bool SHB>
static void launch_mode(const DenseArgs &g, hipStream_t s) {
    if (g.k_split != g.K) launch_d<DT, MODE, SHB, false, LSMX_F32, true>(g, s);
    else launch_d<DT, MODE, SHB, false, LSMX_F32, false>(g, s);
}

hipError_t launch_gemm_dense(const DenseArgs &g, int dtype, int mode, hipStream_t s) {
    const bool shb = mode != 0 && g.b0 == g.b1;
#define LSMX_DM(DT)                                                      \
    do {                                                                 \
        if (mode == 0) launch_mode<DT, 0, false>(g, s);                  \
        else if (mode == 1 && shb) launch_mode<DT, 1, true>(g, s);       \
        else if (mode == 1) launch_mode<DT, 1, false>(g, s);             \
        else if (shb) launch_mode<DT, 2, true>(g, s);                    \
        else launch_mode<DT, 2, false>(g, s);                            \
    } while (0)
    if (dtype == LSMX_BF16) LSMX_DM(LSMX_BF16);
    else if (dtype == LSMX_F16) LSMX_DM(LSMX_F16);
    else LSMX_DM(LSMX_E4M3);
#undef LSMX_DM
    return hipGetLastError();
}

hipError_t launch_gemm_f8f8_scaled(const DenseArgs &g, hipStream_t s) {
    if (g.c_dtype == LSMX_F32) launch_d<LSMX_E4M3, 0, false, true, LSMX_F32, false>(g, s);
    else if (g.c_dtype == LSMX_BF16) launch_d<LSMX_E4M3, 0, false, true, LSMX_BF16, false>(g, s);
    else launch_d<LSMX_E4M3, 0, false, true, LSMX_F16, false>(g, s);
    return hipGetLastError();
}

hipError_t launch_transpose(const void *x, int elem_bytes, int64_t rows, int64_t cols, int64_t ldx, void *y,
                            int64_t ldy, hipStream_t s) {
    const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64)), blk(256);
    const int vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                    (ldx * elem_bytes) % 16 == 0 && (ldy * elem_bytes) % 16 == 0;
    if (elem_bytes == 1)
        hipLaunchKernelGGL(transpose_kernel<uint8_t>, grid, blk, 0, s, reinterpret_cast<const uint8_t *>(x), rows, cols,
                           ldx, reinterpret_cast<uint8_t *>(y), ldy, vec);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, blk, 0, s, reinterpret_cast<const uint16_t *>(x), rows,
                           cols, ldx, reinterpret_cast<uint16_t *>(y), ldy, vec);
    else
        hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, blk, 0, s, reinterpret_cast<const uint32_t *>(x), rows,
                           cols, ldx, reinterpret_cast<uint32_t *>(y), ldy, vec);
    return hipGetLastError();
}

hipError_t launch_scale_to_e8m0(const float *sc, int64_t rows, int64_t cols, int64_t lds, int layout, uint8_t *out,
                                int64_t ldo, hipStream_t s) {
    if (layout & LSMX_E8M0_OUT_KMAJOR) {
        const bool tin = layout & LSMX_E8M0_IN_T;
        const int64_t orows = tin ? cols : rows, groups = (tin ? rows : cols) / 4, n = orows * groups;
        const bool out4 = (reinterpret_cast<uintptr_t>(out) & 3) == 0;
        if (!tin && out4 && (reinterpret_cast<uintptr_t>(sc) & 15) == 0 && lds % 4 == 0) {
            const dim3 grid((unsigned)((orows + 63) / 64), (unsigned)((groups + 15) / 16));
            hipLaunchKernelGGL(scale_to_e8m0_km4_tiled_kernel, grid, dim3(256), 0, s, sc, orows, groups, lds, out, ldo);
            return hipGetLastError();
        }
        hipLaunchKernelGGL(scale_to_e8m0_km4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sc, orows,
                           groups, lds, tin, out, ldo, (reinterpret_cast<uintptr_t>(out) & 3) == 0);
        return hipGetLastError();
    }
    const int64_t n = rows * cols;
    hipLaunchKernelGGL(scale_to_e8m0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sc, rows, cols, lds,
                       layout, out, ldo);
    return hipGetLastError();
}

}  // namespace lsmx
