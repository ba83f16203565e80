// The reference's promotion arithmetic for block scales of any fp32 value:
//
//   acc = 0;  for kb in blocks:  acc = fma(p_kb, sa[m,kb] * sb[n,kb], acc)
//   p_kb = sum_{k in 32-block kb} A[m,k] * Bt[n,k]        (fp32, exact on the E2M1 grid)
//
// mxfp4_gemm.py:52-63 (_mxfp4_gemm_fp8_kernel) and :141-150
// (_mxfp4_gemm_packed_kernel) promote every 32-block product to an fp32
// accumulator and multiply the two fp32 scales there; Triton contracts
// `acc += p * s` to one fma (its default fp fusion).  The fast GEMMs apply
// E8M0 exponents inside the scaled MFMA instead, which is the same
// arithmetic only while every scale is a power of two in [2^-127, 2^127];
// this kernel runs the other cases (1.5, 0, -2, inf, NaN ...), in the
// reference's order, block after block.
//
// Work: one v_mfma_f32_16x16x32_fp8_fp8 per 16 x 16 output tile and 32-block
// (A and Bt as E4M3; packed FP4 codes are expanded exactly to E4M3 as they
// are stored to LDS, one byte permute per 4 codes), then per output element
// one fp32 multiply (sa * sb) and one fma into the accumulator: the vector
// ALU, not the matrix core, bounds it (2 VALU per output per 32-block).
//
// Tiling: 128 x 128 per workgroup of 4 waves (2 x 2, 64 x 64 per wave, 4 x 4
// MFMA tiles).  Chunks of 8 blocks (256 K) of both operands and their
// scales go through registers into LDS between two barriers (two workgroups
// per CU, so one computes while the other loads); rows past M or N are
// clamped for the loads and not stored.  Persistent workgroups walk the
// tiles.  With a flag, every workgroup first
// compares *flag with the caller's epoch and returns when they differ, so a
// launch that follows the fast GEMM costs one load when all scales were
// powers of two (the scale conversion writes the epoch when one is not).
//
// BNC (E4M3 only): B arrives as the reference passes b_fp8, [K, N] with N
// contiguous (row stride ldb bytes).  A chunk of B is then 256 K-rows of the
// tile's 128 columns in LDS (row stride RSN), and each MFMA operand (8 K
// positions of one column per lane) comes from one transposing LDS read
// (ds_read_b64_tr_b8): in each 16-lane group, lanes 2m and 2m + 1 address the
// two 8-byte halves of K-row m and lane j receives column j.  Same products,
// same order, same bits as on the transposed B.
#include "lsmx_store.h"
#include "lsmx_internal.h"

namespace lsmx {

namespace pm {
constexpr int BM = 128, BN = 128, NT = 256;
constexpr int KC = 8;  // 32-blocks per chunk
}  // namespace pm

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool F4>
struct PmOp {
    static constexpr int CB = (F4 ? 16 : 32) * pm::KC;   // bytes of a row per chunk in memory
    static constexpr int RS = 32 * pm::KC + 16;           // LDS row stride (E4M3 bytes): rows 4 banks apart
    static constexpr int PPR = CB / 16;                    // 16-byte pieces per row
    static constexpr int PT = pm::BM * PPR / pm::NT;       // pieces per thread per operand
    static constexpr int RSN = pm::BN + 16;                // BNC: LDS stride of a K-row of B
};

typedef int v2i_pm __attribute__((ext_vector_type(2)));

LSMX_DEV uint64_t ds_read_tr8(const uint8_t *p) {
    return __builtin_bit_cast(
        uint64_t, __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i_pm *)(p)));
}

// 8 packed FP4 codes (code j in bits 4j .. 4j+3) -> 8 E4M3 bytes, the even
// codes first (x: codes 0, 2, 4, 6; y: 1, 3, 5, 7): the magnitude by a byte
// permute against {00 30 38 3C 40 44 48 4C}, the sign bit 3 -> bit 7.  A
// block product does not depend on the order of its K positions as long as
// both operands use the same one.
LSMX_DEV u32x2 fp4x8_to_e4m3x8_eo(uint32_t p) {
    const uint32_t ev = p & 0x0F0F0F0Fu, od = (p >> 4) & 0x0F0F0F0Fu;
    const uint32_t me = __builtin_amdgcn_perm(0x4C484440u, 0x3C383000u, ev & 0x07070707u);
    const uint32_t mo = __builtin_amdgcn_perm(0x4C484440u, 0x3C383000u, od & 0x07070707u);
    return u32x2{me | ((ev << 4) & 0x80808080u), mo | ((od << 4) & 0x80808080u)};
}

template <bool F4, int CT, bool BNC = false>
__global__ __launch_bounds__(pm::NT, 2) void gemm_promote_kernel(PromoteArgs g) {
    using O = PmOp<F4>;
    static_assert(!(BNC && F4), "N-contiguous B is an E4M3 form");
    if (g.flag && *g.flag != g.epoch) return;
    __shared__ __align__(16) uint8_t la[pm::BM * O::RS];
    __shared__ __align__(16) uint8_t lb[BNC ? pm::KC * 32 * O::RSN : pm::BN * O::RS];
    __shared__ __align__(16) float lsa[pm::KC][pm::BM];
    __shared__ __align__(16) float lsb[pm::KC][pm::BN];

    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6), wm = w >> 1, wn = w & 1;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int64_t tn = (g.N + pm::BN - 1) / pm::BN, tiles = ((g.M + pm::BM - 1) / pm::BM) * tn;
    const int nkb = (int)(g.K / 32), nch = (nkb + pm::KC - 1) / pm::KC;
    // Loads through buffer descriptors: a lane whose offset lies at or past a
    // descriptor's byte count reads zeros, and the launcher keeps every
    // offset below 2^31.  Thread t loads PT consecutive 16-byte pieces of
    // row t * PT / PPR of each operand (one offset register, the pieces at
    // immediate offsets); rows past M or N and K past the operand land in
    // LDS rows and columns that no output reads.
    const int lda = (int)g.lda, ldb = (int)g.ldb;
    const int ar0 = t * O::PT / O::PPR, ac0 = (t * O::PT % O::PPR) * 16;
    // coalesced scale loads: consecutive threads walk the axis with the
    // smaller stride (blocks of a row, or rows of a block); element
    // q = i * NT + t is (row q / KC, block q % KC) or (row q % BM, block q / BM)
    const bool sa_byrow = g.sa_k <= g.sa_r, sb_byrow = g.sb_k <= g.sb_r;
    const int sar = (int)g.sa_r, sak = (int)g.sa_k, sbr = (int)g.sb_r, sbk = (int)g.sb_k;
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void *)g.sa, 0, g.sa_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc((void *)g.sb, 0, g.sb_bytes, 0x00020000);

    for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int64_t m0 = (tile / tn) * pm::BM, n0 = (tile % tn) * pm::BN;
        const __amdgpu_buffer_rsrc_t ra_ = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(g.a + m0 * g.lda), 0, (int)min((g.M - m0) * g.lda, (int64_t)0x7FFFFFFF), 0x00020000);
        const __amdgpu_buffer_rsrc_t rb_ = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(g.b + n0 * g.ldb), 0, (int)min((g.N - n0) * g.ldb, (int64_t)0x7FFFFFFF), 0x00020000);
        u32x4 ra[O::PT], rb[O::PT];
        float rsa_[4], rsb_[4];
        auto load = [&](int ch) {
            const int oa = ar0 * lda + ac0 + ch * O::CB, ob = ar0 * ldb + ac0 + ch * O::CB;
#pragma unroll
            for (int i = 0; i < O::PT; ++i) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra_, oa + 16 * i, 0, 0);
            if constexpr (BNC) {
                // K-rows ch * 256 + t / 8 + 32 i, bytes 16 (t % 8) .. of the
                // tile's columns, through a descriptor based at the chunk's
                // first row that ends after column N - 1 of row K - 1: rows
                // past K read zeros (their blocks are not used), columns past
                // N (N % 16 == 0) land in LDS columns no output reads
                const int64_t k0 = (int64_t)ch * (pm::KC * 32);
                const __amdgpu_buffer_rsrc_t rbc = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)(g.b + k0 * g.ldb + n0), 0,
                    (int)min((g.K - 1 - k0) * g.ldb + (g.N - n0), (int64_t)0x7FFFFFFF), 0x00020000);
                const int ob_n = (t >> 3) * ldb + (t & 7) * 16;
#pragma unroll
                for (int i = 0; i < O::PT; ++i)
                    rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rbc, ob_n, i * 32 * ldb, 0);
            } else {
#pragma unroll
                for (int i = 0; i < O::PT; ++i) rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb_, ob + 16 * i, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = i * pm::NT + t;
                const int sa_o = sa_byrow ? ((int)m0 + q / pm::KC) * sar + (ch * pm::KC + q % pm::KC) * sak
                                          : ((int)m0 + q % pm::BM) * sar + (ch * pm::KC + q / pm::BM) * sak;
                const int sb_o = sb_byrow ? ((int)n0 + q / pm::KC) * sbr + (ch * pm::KC + q % pm::KC) * sbk
                                          : ((int)n0 + q % pm::BN) * sbr + (ch * pm::KC + q / pm::BN) * sbk;
                rsa_[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsa, 4 * sa_o, 0, 0));
                rsb_[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsb, 4 * sb_o, 0, 0));
            }
        };
        auto stash = [&]() {
#pragma unroll
            for (int i = 0; i < O::PT; ++i) {
                if constexpr (F4) {
                    // a 16-byte piece is one 32-code block: 32 E4M3 bytes in LDS
                    const int o = ar0 * O::RS + 2 * ac0 + 32 * i;
                    const u32x2 a0 = fp4x8_to_e4m3x8_eo(ra[i].x), a1 = fp4x8_to_e4m3x8_eo(ra[i].y);
                    const u32x2 a2 = fp4x8_to_e4m3x8_eo(ra[i].z), a3 = fp4x8_to_e4m3x8_eo(ra[i].w);
                    const u32x2 b0 = fp4x8_to_e4m3x8_eo(rb[i].x), b1 = fp4x8_to_e4m3x8_eo(rb[i].y);
                    const u32x2 b2 = fp4x8_to_e4m3x8_eo(rb[i].z), b3 = fp4x8_to_e4m3x8_eo(rb[i].w);
                    *reinterpret_cast<u32x4 *>(la + o) = u32x4{a0.x, a0.y, a1.x, a1.y};
                    *reinterpret_cast<u32x4 *>(la + o + 16) = u32x4{a2.x, a2.y, a3.x, a3.y};
                    *reinterpret_cast<u32x4 *>(lb + o) = u32x4{b0.x, b0.y, b1.x, b1.y};
                    *reinterpret_cast<u32x4 *>(lb + o + 16) = u32x4{b2.x, b2.y, b3.x, b3.y};
                } else {
                    *reinterpret_cast<u32x4 *>(la + ar0 * O::RS + ac0 + 16 * i) = ra[i];
                    if constexpr (BNC)
                        *reinterpret_cast<u32x4 *>(lb + ((t >> 3) + 32 * i) * O::RSN + (t & 7) * 16) = rb[i];
                    else
                        *reinterpret_cast<u32x4 *>(lb + ar0 * O::RS + ac0 + 16 * i) = rb[i];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = i * pm::NT + t;
                lsa[sa_byrow ? (q % pm::KC) : (q / pm::BM)][sa_byrow ? (q / pm::KC) : (q % pm::BM)] = rsa_[i];
                lsb[sb_byrow ? (q % pm::KC) : (q / pm::BN)][sb_byrow ? (q / pm::KC) : (q % pm::BN)] = rsb_[i];
            }
        };

        f32x4 acc[4][4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (int ch = 0; ch < nch; ++ch) {
            load(ch);
            __syncthreads();  // the previous chunk's LDS reads are done
            stash();
            __syncthreads();
            const int nb = min(pm::KC, nkb - ch * pm::KC);
            for (int j = 0; j < nb; ++j) {
                uint64_t af[4], bf[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    const int ar = wm * 64 + x * 16 + r16, br = wn * 64 + x * 16 + r16;
                    af[x] = *reinterpret_cast<const uint64_t *>(la + ar * O::RS + j * 32 + g4 * 8);
                    if constexpr (BNC)
                        bf[x] = ds_read_tr8(lb + (j * 32 + g4 * 8 + (r16 >> 1)) * O::RSN + wn * 64 + x * 16 +
                                            8 * (r16 & 1));
                    else
                        bf[x] = *reinterpret_cast<const uint64_t *>(lb + br * O::RS + j * 32 + g4 * 8);
                }
                f32x4 sa4[4];
                float sb1[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    sa4[x] = *reinterpret_cast<const f32x4 *>(&lsa[j][wm * 64 + x * 16 + g4 * 4]);
                    sb1[x] = lsb[j][wn * 64 + x * 16 + r16];
                }
                // the products of row tile mi + 1 run on the matrix core while
                // the vector ALU promotes those of row tile mi
                f32x4 p[2][4];
                auto products = [&](auto mc) {
                    constexpr int mi = decltype(mc)::value;
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
                        p[mi & 1][ni] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
                            (long)af[mi], (long)bf[ni], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                };
                auto promote = [&](auto mc) {
                    constexpr int mi = decltype(mc)::value;
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        const f32x4 q = p[mi & 1][ni];
                        acc[mi][ni].x = __builtin_fmaf(q.x, sa4[mi].x * sb1[ni], acc[mi][ni].x);
                        acc[mi][ni].y = __builtin_fmaf(q.y, sa4[mi].y * sb1[ni], acc[mi][ni].y);
                        acc[mi][ni].z = __builtin_fmaf(q.z, sa4[mi].z * sb1[ni], acc[mi][ni].z);
                        acc[mi][ni].w = __builtin_fmaf(q.w, sa4[mi].w * sb1[ni], acc[mi][ni].w);
                    }
                };
                products(SlotC<0>{});
                products(SlotC<1>{});
                __builtin_amdgcn_sched_barrier(0);
                promote(SlotC<0>{});
                products(SlotC<2>{});
                __builtin_amdgcn_sched_barrier(0);
                promote(SlotC<1>{});
                products(SlotC<3>{});
                __builtin_amdgcn_sched_barrier(0);
                promote(SlotC<2>{});
                promote(SlotC<3>{});
            }
        }

        // lane (r16, g4) of MFMA tile (mi, ni) holds rows 4 g4 .. 4 g4 + 3 of
        // column r16
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int64_t col = n0 + wn * 64 + ni * 16 + r16;
                const int64_t row = m0 + wm * 64 + mi * 16 + g4 * 4;
                if (col >= g.N) continue;
                const float v[4] = {acc[mi][ni].x, acc[mi][ni].y, acc[mi][ni].z, acc[mi][ni].w};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (row + i < g.M) store_c<CT>(g.c, (row + i) * g.ldc + col, v[i]);
            }
        __syncthreads();  // the last chunk's LDS reads are done before the next tile's stash
    }
}

hipError_t launch_gemm_promote(const PromoteArgs &g, bool fp4, hipStream_t s) {
    const int64_t tiles = ((g.M + pm::BM - 1) / pm::BM) * ((g.N + pm::BN - 1) / pm::BN);
    const dim3 grid((unsigned)min(tiles, (int64_t)1024)), blk(pm::NT);
#define LSMX_PM(F, CT) hipLaunchKernelGGL((gemm_promote_kernel<F, CT>), grid, blk, 0, s, g)
#define LSMX_PMN(CT) hipLaunchKernelGGL((gemm_promote_kernel<false, CT, true>), grid, blk, 0, s, g)
    if (g.b_nc) {
        if (g.c_dtype == LSMX_F32) LSMX_PMN(LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_PMN(LSMX_BF16);
        else LSMX_PMN(LSMX_F16);
    } else if (fp4) {
        if (g.c_dtype == LSMX_F32) LSMX_PM(true, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_PM(true, LSMX_BF16);
        else LSMX_PM(true, LSMX_F16);
    } else {
        if (g.c_dtype == LSMX_F32) LSMX_PM(false, LSMX_F32);
        else if (g.c_dtype == LSMX_BF16) LSMX_PM(false, LSMX_BF16);
        else LSMX_PM(false, LSMX_F16);
    }
#undef LSMX_PM
#undef LSMX_PMN
    return hipGetLastError();
}

}  // namespace lsmx
