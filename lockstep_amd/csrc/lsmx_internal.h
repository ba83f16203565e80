// Internal launcher interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include "lsmx_common.h"

namespace lsmx {

// Compile-time arguments passed to the generic lambdas of the pipelined
// kernels: a ring or register slot, a loader wave or not.
template <int V>
struct SlotC {
    static constexpr int value = V;
};
template <bool V>
struct BoolC {
    static constexpr bool value = V;
};

struct QuantArgs {
    const void *x;
    int x_dtype;
    int64_t rows;  // rows (row mode) or columns (column mode)
    int64_t K;
    int64_t ldx;
    int block;
    void *codes;
    int codes_fmt;
    int64_t ld_codes;
    void *scale;
    int scale_fmt;
    int64_t ld_scale;
};

// Quantization of a 16-bit x[R, C] along both axes in one pass: the row
// form (codes_r [R, ld_cr], scale_r) and the column form laid out for x^T
// (codes_c [C, ld_cc], scale_c); packed codes, E8M0 scales (row-major or
// K-major, the same format for both).
struct Quant2dArgs {
    const void *x;
    int x_dtype;
    int64_t R, C, ldx;
    uint8_t *codes_r;
    int64_t ld_cr;
    uint8_t *scale_r;
    int64_t ld_sr;
    uint8_t *codes_c;
    int64_t ld_cc;
    uint8_t *scale_c;
    int64_t ld_sc;
    int scale_fmt;
};

// Up to kQBatch tensors of one dtype and scale format quantized along their
// rows by one launch (packed codes, 32-blocks, E8M0 scales); end[k] = rows of
// tensors 0 .. k.
constexpr int kQBatch = 8;
struct QuantBatch {
    QuantArgs a[kQBatch];
    int64_t end[kQBatch];
    int n;
};

// Up to kQ2Batch tensors of one dtype and scale format quantized by one
// launch; end[k] = tiles of tensors 0 .. k.
constexpr int kQ2Batch = 8;
struct Quant2dBatch {
    Quant2dArgs a[kQ2Batch];
    int64_t end[kQ2Batch];
    int n;
};

struct DequantArgs {
    const void *codes;
    int codes_fmt;
    int64_t ld_codes;
    const void *scale;
    int scale_fmt;
    int64_t ld_scale;
    int64_t rows, K;
    int block;
    void *out;
    int out_dtype;
    int64_t ld_out;
};

struct GemmArgs {
    const uint8_t *a;  // packed A [M, lda] (f4f4) or bf16 A [M, lda] (bf16f4)
    const uint8_t *a1; // second activation batch (dual), else null
    int64_t lda;
    const void *sa;    // A scales (f4f4 only)
    int64_t ld_sa;
    const uint8_t *b;  // packed Bt / W [N, ldb]
    int64_t ldb;
    const void *sb;
    int64_t ld_sb;
    int scale_fmt;
    void *c;
    void *c1;          // second output (dual)
    int c_dtype;
    int64_t ldc;
    int64_t M, N, K;
    // split-K (weight-only ring kernel): K slices of k_split, fp32 partial
    // tiles in the workspace ws
    int splits = 1;
    int64_t k_split = 0;
    float *ws = nullptr;
    // decode-shape weight-only kernel: weight rows per workgroup
    int rows_wg = 0;
    // f4 x f4 GEMM with a quantizing epilogue: both MXFP4 forms of the
    // bf16-rounded C with K-major E8M0 scales, as lsmx_quantize_mxfp4_2d
    // writes them (c optional)
    uint8_t *codes_r = nullptr;
    int64_t ld_cr = 0;
    uint8_t *scale_r = nullptr;
    int64_t ld_sr = 0;
    uint8_t *codes_c = nullptr;
    int64_t ld_cc = 0;
    uint8_t *scale_c = nullptr;
    int64_t ld_sc = 0;
};

struct DenseArgs {
    const uint8_t *a0, *a1;  // [M, lda] K-contiguous
    int64_t lda;
    const uint8_t *b0, *b1;  // Bt [N, ldb] K-contiguous
    int64_t ldb;
    const uint8_t *sa, *sb;  // E8M0 [rows, ld] (scaled E4M3 only)
    int64_t ld_sa, ld_sb;
    void *c0, *c1;
    int c_dtype;
    int64_t ldc;
    int64_t M, N, K;
    int64_t k_split;         // K per split (== K without split-K)
    int b_nc;                // 1: b0, b1 are B [K, ldb] N-contiguous (bf16/fp16 ring kernel only)
};

// The reference's promotion arithmetic for fp32 block scales of any value
// (gemm_promote.hip): A [M, lda] and Bt [N, ldb] as packed FP4 codes or E4M3
// bytes, scale (r, kb) of A at sa[r * sa_r + kb * sa_k] (likewise sb).  With
// a flag the launch does nothing unless *flag == epoch.
struct PromoteArgs {
    const uint8_t *a;
    int64_t lda;
    const uint8_t *b;
    int64_t ldb;
    const float *sa;
    int64_t sa_r, sa_k;
    const float *sb;
    int64_t sb_r, sb_k;
    int sa_bytes, sb_bytes;  // extents of the scale tensors (loads past them read 0)
    void *c;
    int c_dtype;
    int64_t ldc;
    int64_t M, N, K;
    const uint64_t *flag;
    uint64_t epoch;
    int b_nc;  // 1: b is B [K, ldb] N-contiguous E4M3 (else Bt [N, ldb])
};

// Up to kE8Batch fp32 scale tensors converted to K-major E8M0 in one launch;
// end[k] = workgroups of tensors 0 .. k.  When a scale has no E8M0 form the
// launch writes epoch to *flag (if flag is not null).
constexpr int kE8Batch = 4;
struct E8m0Item {
    const float *s;
    int64_t orows, groups, lds;  // out rows, 4-block groups, stride of s
    int tin;                     // s is [blocks, out rows] (else [out rows, blocks])
    int vec4;                    // row-major with 16-byte rows: float4 loads
    uint8_t *out;
    int64_t ldo;
};
struct E8m0Batch {
    E8m0Item it[kE8Batch];
    int64_t end[kE8Batch];
    int n;
    uint64_t *flag;
    uint64_t epoch;
};

hipError_t launch_quantize(const QuantArgs &a, bool cols, hipStream_t s);
hipError_t launch_quantize_2d(const Quant2dArgs &a, hipStream_t s);
hipError_t launch_quantize_2d_batch(const Quant2dBatch &b, hipStream_t s);
hipError_t launch_quantize_batch(const QuantBatch &b, hipStream_t s);
hipError_t launch_round(const void *q, int q_dtype, int64_t n, uint8_t *codes, hipStream_t s);
hipError_t launch_pack(const uint8_t *codes, uint8_t *packed, int64_t n_bytes, hipStream_t s);
hipError_t launch_unpack(const uint8_t *packed, uint8_t *codes, int64_t n_bytes, hipStream_t s);
hipError_t launch_fp4_to_e4m3(const uint32_t *in, uint32_t *out, int64_t n, hipStream_t s);
hipError_t launch_dequant(const DequantArgs &a, hipStream_t s);
hipError_t launch_gemm_f4f4(const GemmArgs &g, hipStream_t s);
hipError_t launch_gemm_f4f4_quant(const GemmArgs &g, hipStream_t s);
hipError_t launch_gemm_bf16f4(const GemmArgs &g, hipStream_t s);
hipError_t launch_gemm_xf4(const GemmArgs &g, int a_dtype, hipStream_t s);
// split count the weight-only GEMM uses at this shape when given a workspace
// (1: no split), and the workspace bytes that needs (partials + counters)
int gemm_bf16f4_splits(int64_t M, int64_t N, int64_t K, bool dual);
int64_t gemm_bf16f4_workspace(int64_t M, int64_t N, int64_t K, bool dual);
hipError_t launch_gemm_dense(const DenseArgs &g, int dtype, int mode, hipStream_t s);
bool dense_ring_ok(const DenseArgs &g, int dtype);
hipError_t launch_gemm_dense_ring(const DenseArgs &g, int dtype, int mode, hipStream_t s);
hipError_t launch_gemm_f8f8_scaled(const DenseArgs &g, hipStream_t s);
hipError_t launch_gemm_f8f8_kmajor(const DenseArgs &g, hipStream_t s);
hipError_t launch_transpose(const void *x, int elem_bytes, int64_t rows, int64_t cols, int64_t ldx, void *y,
                            int64_t ldy, hipStream_t s);
hipError_t launch_scale_to_e8m0(const float *sc, int64_t rows, int64_t cols, int64_t lds, int layout, uint8_t *out,
                                int64_t ldo, hipStream_t s);
hipError_t launch_scale_to_e8m0_batch(const E8m0Batch &b, hipStream_t s);
hipError_t launch_gemm_promote(const PromoteArgs &g, bool fp4, hipStream_t s);

}  // namespace lsmx
