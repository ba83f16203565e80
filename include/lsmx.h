/*
 * lsmx.h -- C ABI of the MI355X (gfx950) MXFP4 library, liblsmx.so.
 *
 * MXFP4 = E2M1 4-bit elements with one E8M0 (power-of-two) scale per 32
 * consecutive elements along the contraction axis K; two elements per byte,
 * the even-indexed element in the low nibble.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; sizes, leading dimensions (ld*) and
 *     offsets are in ELEMENTS of the pointed-to type (bytes for packed codes
 *     and E8M0 scales).  Row-major, unit stride along the last axis.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Every call is
 *     asynchronous and stream-ordered; none synchronizes the device.
 *   - The library never allocates device memory.
 *   - Return value: LSMX_OK (0) or a negative LSMX_ERR_* code; the message
 *     for the calling thread is in lsmx_last_error().
 *
 * Reference interfaces replaced (paths relative to the lockstep checkout):
 * each declaration cites the Python/Triton/CUDA function whose semantics it
 * implements.
 */
#ifndef LSMX_H
#define LSMX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define LSMX_OK 0
#define LSMX_ERR_SHAPE -1   /* a size or block that the reference asserts against */
#define LSMX_ERR_ALIGN -2   /* pointer or leading dimension misaligned            */
#define LSMX_ERR_DTYPE -3   /* unsupported element type or format                 */
#define LSMX_ERR_DEVICE -4  /* no device, or the current device is not gfx950     */
#define LSMX_ERR_LAUNCH -5  /* the HIP runtime rejected a kernel launch           */
#define LSMX_ERR_ARG -6     /* null pointer or otherwise invalid argument         */

/* element types */
#define LSMX_F32 0
#define LSMX_BF16 1
#define LSMX_F16 2
#define LSMX_E4M3 3  /* FP8 E4M3 (torch.float8_e4m3fn): dense GEMM operands only */

/* code formats */
#define LSMX_CODES_PACKED 0    /* [rows, K/2] bytes, even element in the low nibble */
#define LSMX_CODES_UNPACKED 1  /* [rows, K] bytes, one code (0..15) per byte         */

/* scale formats */
#define LSMX_SCALE_E8M0 0  /* one byte per block: biased exponent, 0xFF = NaN        */
#define LSMX_SCALE_F32 1   /* one fp32 per block holding the power of two (fp4.py)   */
/* E8M0 bytes grouped by 128-element K slices: byte (kb/4, row, kb%4) of a
 * [K/128][ld_scale][4] array, ld_scale >= rows.  The GEMMs read the four
 * scales of one K slice for consecutive rows as one contiguous run.  Same
 * byte count as LSMX_SCALE_E8M0; requires K % 128 == 0. */
#define LSMX_SCALE_E8M0_KMAJOR 2

/* Library version string, e.g. "lsmx 0.1.0 gfx950". */
const char *lsmx_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *lsmx_last_error(void);

/* LSMX_OK if the current HIP device is a gfx950 (MI355X class) GPU.
 * Replaces the device guard of h100.py:8-15 / fp4_linear.py:19. */
int lsmx_device_check(void);

/* MXFP4 quantization of x[rows, K] along K.
 * Replaces fp4.py:57-72 quantize_mxfp4 (codes + fp32 scale, UNPACKED) and,
 * with LSMX_CODES_PACKED, the fused quantize_mxfp4 + pack_fp4 of
 * fp4_linear.py:36-39 / fp4.py:91-94.
 *   x_dtype   LSMX_F32 | LSMX_BF16 | LSMX_F16; ldx >= K (elements).
 *   block     32 or 16 (K % block == 0, as fp4.py:65 asserts).
 *   codes     [rows, ld_codes] bytes; ld_codes >= K/2 (PACKED) or K (UNPACKED).
 *   scale     [rows, ld_scale] E8M0 bytes or fp32; ld_scale >= K/block.
 * Scale exponent: floor(RN_f32(log2(max(amax, 1e-30)))) - 2, clamped to
 * [-127, 127]; 1.0 for an all-zero block; NaN (0xFF) for a block with a NaN.
 * Rounding: to nearest with ties toward the smaller magnitude, clip at 6,
 * sign copied from the input (-0 -> code 8), exactly as fp4.py:43-54. */
int lsmx_quantize_mxfp4(const void *x, int x_dtype, int64_t rows, int64_t K, int64_t ldx,
                        int block, void *codes, int codes_fmt, int64_t ld_codes, void *scale,
                        int scale_fmt, int64_t ld_scale, void *stream);

/* One tensor of lsmx_quantize_mxfp4_batch: the arguments of
 * lsmx_quantize_mxfp4 for it (block 32, packed codes). */
typedef struct {
    const void *x;
    int64_t rows, K, ldx;
    void *codes;
    int64_t ld_codes;
    void *scale;
    int64_t ld_scale;
} lsmx_q_item;

/* lsmx_quantize_mxfp4 (block 32, LSMX_CODES_PACKED, E8M0 scales row-major
 * or K-major) of n <= 8 tensors of one dtype and scale format in one launch,
 * with the same outputs bit for bit.  The fully-FP4 GEMM step quantizes both
 * of its operands before the product (fp4_linear.py:36-39: X and W); one
 * launch streams both without a drain and a ramp-up between them.  items is
 * host memory, read before the call returns; the same checks as
 * lsmx_quantize_mxfp4 apply to each tensor. */
int lsmx_quantize_mxfp4_batch(const lsmx_q_item *items, int n, int x_dtype, int scale_fmt, void *stream);

/* The same quantizer along the OTHER axis: x[K, cols] (ldx >= cols) is
 * quantized in blocks of `block` consecutive ROWS, and the outputs are laid
 * out for x^T: codes [cols, ld_codes], scale [cols, ld_scale].
 * Equivalent to fp4.py:57-72 applied to x.t().contiguous() (the requantization
 * of a transposed operand, as bench.py:161 does for B). */
int lsmx_quantize_mxfp4_t(const void *x, int x_dtype, int64_t K, int64_t cols, int64_t ldx,
                          int block, void *codes, int codes_fmt, int64_t ld_codes, void *scale,
                          int scale_fmt, int64_t ld_scale, void *stream);

/* Both of the above from ONE read of x: x[rows, cols] (bf16 or fp16,
 * ldx >= cols) quantized along its rows -- codes_r [rows, ld_codes_r] packed,
 * scale_r -- and along its columns -- codes_c [cols, ld_codes_c] packed,
 * scale_c, laid out for x^T -- with E8M0 scales, row-major or K-major
 * (scale_fmt; the same for both; K-major ld_scale_r >= rows, ld_scale_c >=
 * cols).  Bit-identical to lsmx_quantize_mxfp4 and lsmx_quantize_mxfp4_t
 * with block 32 (fp4.py:57-72 on x and on x.t().contiguous()).  A training
 * step needs both forms of each operand it quantizes (train_step.py:3-6:
 * X and W along K for fprop, W and dY along N for dgrad, dY and X along T
 * for wgrad); this reads each once.  rows, cols % 128 == 0. */
int lsmx_quantize_mxfp4_2d(const void *x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx, uint8_t *codes_r,
                           int64_t ld_codes_r, uint8_t *scale_r, int64_t ld_scale_r, uint8_t *codes_c,
                           int64_t ld_codes_c, uint8_t *scale_c, int64_t ld_scale_c, int scale_fmt, void *stream);

/* One tensor of lsmx_quantize_mxfp4_2d_batch: the arguments of
 * lsmx_quantize_mxfp4_2d for it. */
typedef struct {
    const void *x;
    int64_t rows, cols, ldx;
    uint8_t *codes_r;
    int64_t ld_codes_r;
    uint8_t *scale_r;
    int64_t ld_scale_r;
    uint8_t *codes_c;
    int64_t ld_codes_c;
    uint8_t *scale_c;
    int64_t ld_scale_c;
} lsmx_q2d_item;

/* lsmx_quantize_mxfp4_2d of n <= 8 tensors of one dtype and scale format in
 * one launch, with the same outputs bit for bit.  The tensors a training
 * step quantizes at its start (the activation and the weights of each
 * linear, train_step.py:3-6) are a few MB each; one launch keeps the memory
 * system streaming across them instead of ramping up and draining per
 * tensor.  items is host memory, read before the call returns. */
int lsmx_quantize_mxfp4_2d_batch(const lsmx_q2d_item *items, int n, int x_dtype, int scale_fmt,
                                 void *stream);

/* fp4.py:43-54 _round_to_e2m1: codes[i] = E2M1 code of q[i] (scale 1):
 * nearest, ties toward the smaller magnitude, clip at 6, sign copied, NaN -> 7.
 * q_dtype LSMX_F32 | LSMX_BF16 | LSMX_F16; n elements, one code byte each. */
int lsmx_round_e2m1(const void *q, int q_dtype, int64_t n, uint8_t *codes, void *stream);

/* fp4.py:91-94 pack_fp4: n_bytes output bytes from 2*n_bytes codes. */
int lsmx_pack_fp4(const uint8_t *codes, uint8_t *packed, int64_t n_bytes, void *stream);

/* fp4.py:97-99 unpack_fp4: 2*n_bytes codes from n_bytes packed bytes. */
int lsmx_unpack_fp4(const uint8_t *packed, uint8_t *codes, int64_t n_bytes, void *stream);

/* fp4.py:75-78 dequantize_mxfp4: out[r, k] = value(code[r, k]) * scale[r, k/block],
 * out_dtype LSMX_F32 | LSMX_BF16 (exact in both: the scale is a power of two). */
int lsmx_dequantize_mxfp4(const void *codes, int codes_fmt, int64_t ld_codes, const void *scale,
                          int scale_fmt, int64_t ld_scale, int64_t rows, int64_t K, int block,
                          void *out, int out_dtype, int64_t ld_out, void *stream);

/* fp4.py:81-83 codes_to_e4m3 / cuda/fp4_unpack.cuh:52-55 fp4x8_to_e4m3x8 /
 * cuda/mxfp4_mma_gemm.cu:187-195 unpack_kernel: each input word of 8 packed
 * codes becomes 8 E4M3 bytes, out[2i] = codes 0..3, out[2i+1] = codes 4..7. */
int lsmx_fp4_to_e4m3(const uint32_t *in, uint32_t *out, int64_t n_words, void *stream);

/* Block-scaled FP4 x FP4 GEMM:  C[M, N] = sum_kb sa[m,kb] sb[n,kb] (A_kb . Bt_kb).
 * Replaces mxfp4_gemm.py:161-174 mxfp4_gemm_packed / _mxfp4_gemm_packed_kernel
 * (mxfp4_gemm.py:116-158) and cuda/mxfp4_mma_gemm.cu:69-184.
 *   a_pk  [M, lda] bytes (lda >= K/2),   a_scale [M, ld_sa] (E8M0 or fp32)
 *   bt_pk [N, ldb] bytes (ldb >= K/2),   b_scale [N, ld_sb]
 *   c     [M, ldc] of c_dtype (LSMX_F32 | LSMX_BF16 | LSMX_F16), fp32 accumulate.
 *   K % 128 == 0 (mxfp4_gemm.py:166); any M, N >= 1; lda, ldb and the
 *   row-major scale rows (in bytes) below 2^24.
 * fp32 scales are the powers of two fp4.py produces.  A scale with no E8M0
 * form (not a positive power of two in [2^-127, 2^127]) is taken as E8M0
 * NaN here: the outputs that use it are NaN, where the reference's fp32
 * multiply (mxfp4_gemm.py:148-150) would scale by it; for any fp32 scale,
 * convert with lsmx_scale_to_e8m0_batch (flag, epoch), call this with the
 * K-major bytes and follow with lsmx_gemm_mx_promote (flag, epoch), as
 * mxfp4_gemm.mxfp4_gemm_packed does.  E8M0 byte 0 is 2^-127.  K-major E8M0 scales with K % 256 == 0 run the fastest kernel
 * (16 x 16 x 128 scaled MFMA on 256-code stages); the other formats and K
 * % 256 != 0 run a 32 x 32 x 64 kernel on 128-code stages.  Every format of
 * the same scales gives the same bits. */
int lsmx_gemm_f4f4(const uint8_t *a_pk, int64_t lda, const void *a_scale, int64_t ld_sa,
                   const uint8_t *bt_pk, int64_t ldb, const void *b_scale, int64_t ld_sb,
                   int scale_fmt, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                   int64_t K, void *stream);

/* lsmx_gemm_f4f4 (K-major E8M0 scales) whose epilogue quantizes its output:
 * C = A . Bt^T rounded to bf16 is written as both MXFP4 forms that
 * lsmx_quantize_mxfp4_2d(C, LSMX_SCALE_E8M0_KMAJOR) would write from the
 * stored bf16 C, bit for bit -- the row form (codes_r [M, ld_codes_r] with
 * scale_r [N/128][ld_scale_r][4]) and the column form laid out for C^T
 * (codes_c [N, ld_codes_c], scale_c [M/128][ld_scale_c][4]) -- and, when c
 * is not NULL, as the bf16 C [M, ldc] itself.  It replaces a GEMM followed by
 * quantize_mxfp4 (fp4.py:57-72) of its output along both axes: between two
 * linear layers trained in MXFP4, the hidden activation H and its gradient
 * dH each feed one GEMM along rows and one along columns (the three GEMMs per
 * linear of train_step.py:3-6), so the bf16 H and dH need never be stored
 * or read back.  M, N, K multiples of 256; packed A and
 * Bt rows 16-byte aligned below 2^24 bytes; K-major input scales; row
 * codes 4-byte, column codes 8-byte aligned rows; scales 4-byte aligned;
 * c rows 16-byte aligned. */
int lsmx_gemm_f4f4_quant(const uint8_t *a_pk, int64_t lda, const void *a_scale, int64_t ld_sa,
                         const uint8_t *bt_pk, int64_t ldb, const void *b_scale, int64_t ld_sb,
                         void *c, int64_t ldc, uint8_t *codes_r, int64_t ld_codes_r,
                         uint8_t *scale_r, int64_t ld_scale_r, uint8_t *codes_c,
                         int64_t ld_codes_c, uint8_t *scale_c, int64_t ld_scale_c, int64_t M,
                         int64_t N, int64_t K, void *stream);

/* Weight-only GEMM, bf16 activations x MXFP4 weight:
 *   C[M, N] = A[M, K] . deq(W)[N, K]^T, fp32 accumulate.
 * Replaces the forward of fp4_linear.py:34-40 for an unquantized activation
 * (the fake-quant F.linear on dequantized weights) at LLM MLP shapes.
 *   a [M, lda] bf16;  w_pk [N, ldw] bytes;  w_scale [N, ld_sw] E8M0 or fp32
 *   (fp32 scales with no E8M0 form give NaN outputs, as lsmx_gemm_f4f4).
 *   c [M, ldc] of c_dtype.  K % 128 == 0; lda, ldw < 2^27, scale rows
 *   (in bytes) < 2^24. */
int lsmx_gemm_bf16f4(const void *a, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                     const void *w_scale, int64_t ld_sw, int scale_fmt, void *c, int c_dtype,
                     int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream);

/* Workspace bytes the split-K form of the bf16 x MXFP4 GEMM below needs at
 * this shape (single form: dual = 0, dual-batch form: dual = 1), or 0 when
 * the library does not split this shape.  It splits K in 2 or 4 slices when
 * the whole-K 128 x 256 output tiles would fill less than half of the CUs
 * (a few hundred activation rows against a wide weight, e.g. M = 128
 * against N = 14336: 128 x 128 tiles in 2 slices).  The answer depends on
 * M, N and K only, but the split itself runs only for E8M0 scales whose rows
 * are 16-byte aligned with a stride that is a multiple of 16 bytes; other
 * scales (fp32, or E8M0 rows of another alignment) run the whole-K kernels
 * and leave a given workspace unused, with other bits than the split form
 * (same tolerance).  The Python layer converts fp32 weight scales to E8M0
 * bytes first, so both forms of a weight take the same kernels there. */
int64_t lsmx_gemm_bf16f4_workspace(int64_t M, int64_t N, int64_t K, int dual);

/* lsmx_gemm_bf16f4 (a1 = c1 = NULL) or lsmx_gemm_dual_bf16f4 (both set)
 * with a caller-provided device workspace, which lets the library split K
 * (lsmx_gemm_bf16f4_workspace): each K slice of a 128-row output tile is
 * one workgroup that writes an fp32 partial tile to the workspace, and a
 * second kernel on the same stream adds the slices in slice order (a fixed
 * order: repeated calls, and the single and dual forms, give identical
 * bits).  The same sums as the reference's split-K GEMM (dual_gemm.py:
 * 117-179) without its atomics.  Workspace: 16-byte aligned, at least the
 * bytes lsmx_gemm_bf16f4_workspace returns, no initial contents required;
 * calls that share a workspace must be stream-ordered.  A NULL workspace,
 * or a shape the library does not split, runs the whole-K kernels. */
int lsmx_gemm_bf16f4_ws(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                        const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, void *workspace, int64_t workspace_bytes, void *stream);

/* lsmx_gemm_bf16f4_ws without the workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same kernels and the same bits as lsmx_gemm_bf16f4_ws with a workspace;
 * the split-K partial tiles go to a fixed 64 MiB device array of the library
 * instead (one per GPU, held from the first call on that GPU until the process
 * ends; its device address is looked up once per GPU on that first call).
 * A shape whose split-K partials need more is rejected with LSMX_ERR_SHAPE
 * (on a 256-CU gfx950 none does).  The call allocates nothing.  Every call
 * on one GPU shares the array: calls that overlap on one GPU (different
 * streams, or host threads without stream ordering) race. */
int lsmx_gemm_bf16f4_noalloc(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                             const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream);

/* Weight-only GEMM for any activation type: C[M, N] = A[M, K] . deq(W)^T.
 * Replaces the reference's fp32 fake-quant product, Y = X @ dequantize_mxfp4(W)^T
 * (fp4.py:75-78 inside fp4_linear.py:40's fake-quant F.linear, with X left
 * unquantized), which the reference computes in fp32 on the CPU.
 *   a_dtype LSMX_BF16: the same kernels as lsmx_gemm_bf16f4.
 *   a_dtype LSMX_F32 | LSMX_F16: each activation is split exactly into three
 *   (fp32) or two (fp16) bf16 terms, each multiplied with the exact bf16
 *   weight on the MFMA: exact products, fp32 accumulation -- the arithmetic
 *   of an fp32 matmul, without narrowing X to bf16 (exact for |x| >= 2^-110).
 *   a [M, lda] of a_dtype with 16-byte aligned rows; other arguments as
 *   lsmx_gemm_bf16f4. */
int lsmx_gemm_wonly_f4(const void *a, int a_dtype, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                       const void *w_scale, int64_t ld_sw, int scale_fmt, void *c, int c_dtype, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, void *stream);

/* Dual-batch weight-only GEMM: C0 = A0 . deq(W)^T and C1 = A1 . deq(W)^T in
 * ONE launch, each W tile loaded and dequantized once for both batches.
 * Replaces dual_gemm.py:244-255 dual_separate(a1, a2, b, b) as used with a
 * shared weight (train_step.py:52-53), with W in MXFP4.
 *   a0, a1 [M, lda] bf16; c0, c1 [M, ldc]; other arguments as lsmx_gemm_bf16f4. */
int lsmx_gemm_dual_bf16f4(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk,
                          int64_t ldw, const void *w_scale, int64_t ld_sw, int scale_fmt,
                          void *c0, void *c1, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                          int64_t K, void *stream);

/* Dense GEMM with fp32 accumulation and fp32 output, operands K-contiguous:
 *   a0, a1 [M, lda] and bt0, bt1 [N, ldb] of dtype LSMX_BF16 | LSMX_F16 | LSMX_E4M3.
 *   mode 0: c0 = a0 . bt0^T                       dual_gemm.py:189-226 gemm
 *   mode 1: c0 = a0 . bt0^T + a1 . bt1^T          dual_gemm.py:43-72, 230-241 dual_packed
 *           (one accumulator; the caller pre-scales a1 by 2^s as the reference does;
 *           64-deep K blocks of the two products alternate, as in its loop)
 *   mode 2: c0 = a0 . bt0^T,  c1 = a1 . bt1^T     dual_gemm.py:79-110, 244-255 dual_separate
 * splits > 1: K is cut into `splits` equal slices whose partial sums are added
 * into c0 (and c1) with fp32 atomics, so the outputs must hold zeros on entry
 * (dual_gemm.py:118-179, 261-289 splitk_packed / splitk_separate; the order of
 * the additions, hence the last bits, varies from run to run as there).
 * The reference takes B as [K, N]; pass its transpose (lsmx_transpose).
 * K % (64 * splits) == 0 (dual_gemm.py:219, 265); rows 16-byte aligned. */
int lsmx_gemm_dense(const void *a0, const void *a1, int64_t lda, const void *bt0, const void *bt1, int64_t ldb,
                    int dtype, int mode, float *c0, float *c1, int64_t ldc, int64_t M, int64_t N, int64_t K,
                    int splits, void *stream);

/* lsmx_gemm_dense (bf16 / fp16, no split-K) with B as the reference passes
 * it: b0, b1 [K, ldb] N-contiguous (dual_gemm.py:188-289 take b [K, N]), so
 * no transpose is needed.  The kernel reads B rows of 256 columns into LDS
 * and forms each MFMA operand with transposing LDS reads (ds_read_b64_tr_b16);
 * same sums in the same order as lsmx_gemm_dense on the transposed B, so the
 * same bits.  K % 64 == 0, N % 8 == 0; lda >= K, ldb >= N, both <= 2^22;
 * rows 16-byte aligned. */
int lsmx_gemm_dense_nb(const void *a0, const void *a1, int64_t lda, const void *b0, const void *b1, int64_t ldb,
                       int dtype, int mode, float *c0, float *c1, int64_t ldc, int64_t M, int64_t N, int64_t K,
                       void *stream);

/* MXFP4 GEMM on E4M3 operands holding E2M1 values, with E8M0 block scales:
 *   C[M, N] = sum_kb 2^(sa[m,kb]-127) 2^(sb[n,kb]-127) (A_kb . Bt_kb)
 * Replaces mxfp4_gemm.py:74-87 mxfp4_gemm_fp8 / _mxfp4_gemm_fp8_kernel
 * (mxfp4_gemm.py:29-71), which promotes each 32-block product to fp32 and
 * multiplies fp32 scales; here the scaled MFMA applies the exponents.
 *   a [M, lda] and bt [N, ldb] E4M3 bytes (K-contiguous; the reference's
 *   b_fp8 [K, N] transposed); scale_fmt LSMX_SCALE_E8M0: a_e8m0 [M, ld_sa],
 *   b_e8m0 [N, ld_sb] bytes, or LSMX_SCALE_E8M0_KMAJOR (the fast path):
 *   [K/128, ld_sa, 4] and [K/128, ld_sb, 4] with ld_sa >= M, ld_sb >= N
 *   (lsmx_scale_to_e8m0 of fp4.py's fp32 power-of-two scales);
 *   c [M, ldc] of c_dtype (LSMX_F32 | LSMX_BF16 | LSMX_F16).  K % 128 == 0
 *   (mxfp4_gemm.py:78).  fp32 scales that are not powers of two take the
 *   lsmx_scale_to_e8m0_batch + lsmx_gemm_mx_promote sequence described at
 *   lsmx_gemm_f4f4 (op_fmt LSMX_E4M3). */
int lsmx_gemm_f8f8(const uint8_t *a, int64_t lda, const uint8_t *a_e8m0, int64_t ld_sa, const uint8_t *bt,
                   int64_t ldb, const uint8_t *b_e8m0, int64_t ld_sb, int scale_fmt, void *c, int c_dtype,
                   int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream);

/* lsmx_gemm_f8f8 with K-major E8M0 scales and B as the reference passes it:
 * b [K, ldb] E4M3, N-contiguous (mxfp4_gemm.py:74-87 takes b_fp8 [K, N]), so
 * no transpose is needed; b_e8m0 is K-major [K/128][ld_sb][4] over B's
 * columns.  The kernel forms each MFMA operand with transposing LDS reads
 * (ds_read_b64_tr_b8); same sums in the same order as lsmx_gemm_f8f8 on the
 * transposed B, so the same bits.  K % 128 == 0, N % 16 == 0; ldb >= N;
 * lda, ldb <= (2^31 - 1) / 256; rows 16-byte aligned.  fp32 scales that may
 * not be powers of two: follow with lsmx_gemm_mx_promote on the same b
 * (op_fmt LSMX_E4M3 | LSMX_B_NCONTIG). */
int lsmx_gemm_f8f8_nb(const uint8_t *a, int64_t lda, const uint8_t *a_e8m0, int64_t ld_sa, const uint8_t *b,
                      int64_t ldb, const uint8_t *b_e8m0, int64_t ld_sb, void *c, int c_dtype, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, void *stream);

/* y[cols, ldy] = x[rows, ldx]^T for elements of elem_bytes = 1, 2 or 4 bytes.
 * Lays out the reference's N-contiguous B operands ([K, N], dual_gemm.py:
 * 189-289, mxfp4_gemm.py:29-87) K-contiguous for the kernels above. */
int lsmx_transpose(const void *x, int elem_bytes, int64_t rows, int64_t cols, int64_t ldx, void *y, int64_t ldy,
                   void *stream);

/* E8M0 bytes of fp32 power-of-two scales (their exponent field), the exact
 * inverse of fp4.py:61-69's 2^e.  s is [rows, cols] (stride lds) of scales
 * of (output row, block) pairs, or with LSMX_E8M0_IN_T in `layout` of
 * (block, output row) pairs (mxfp4_gemm.py:79's b_scale [K/32, N]).  The
 * output is row-major [out rows, ldo], or with LSMX_E8M0_OUT_KMAJOR the
 * K-major [blocks/4, ldo, 4] (blocks % 4 == 0, ldo >= out rows) that the
 * GEMMs stream fastest.  A scale that is not a power of two in
 * [2^-127, 2^127] has no E8M0 form and becomes 0xFF (E8M0 NaN), so the
 * outputs that use it are NaN. */
#define LSMX_E8M0_IN_T 1
#define LSMX_E8M0_OUT_KMAJOR 2
int lsmx_scale_to_e8m0(const float *s, int64_t rows, int64_t cols, int64_t lds, int layout, uint8_t *out,
                       int64_t ldo, void *stream);

/* lsmx_scale_to_e8m0 with K-major output for up to 4 fp32 scale tensors in
 * one launch (the A and B scales of one GEMM call: mxfp4_gemm.py:161-174's
 * and :74-87's fp32 scales, regrouped for the fast kernels), and a test for
 * the scales the fast kernels cannot apply: when any scale is neither a
 * power of two in [2^-127, 2^127] nor a NaN (1.5, 0, -2, inf ...; a NaN
 * scale is E8M0 0xFF, NaN in every output that uses it, as the reference's
 * multiply makes it) and flag is not NULL, the launch writes epoch to *flag
 * (8-byte aligned device memory); otherwise it leaves *flag as it was.  A caller picks an epoch it
 * has never used with that flag, so no earlier content can equal it, and
 * passes flag and epoch to lsmx_gemm_mx_promote after the fast GEMM. */
typedef struct {
    const float *s;   /* [rows, cols], row stride lds (elements)           */
    int64_t rows, cols, lds;
    int layout;       /* 0 or LSMX_E8M0_IN_T; the output is always K-major */
    uint8_t *out;     /* [blocks/4][ldo][4], 4-byte aligned, ldo >= out rows */
    int64_t ldo;
} lsmx_e8m0_item;
int lsmx_scale_to_e8m0_batch(const lsmx_e8m0_item *items, int n, uint64_t *flag, uint64_t epoch,
                             void *stream);

/* The reference's own arithmetic for fp32 block scales of any value:
 *   acc = 0;  for kb in 0 .. K/32-1:  acc = fma(p_kb, a_scale[m,kb] * b_scale[n,kb], acc)
 *   p_kb = the 32-block product of A[m, :] and Bt[n, :] (fp32; exact on the E2M1 grid)
 *   C[m, n] = acc rounded to c_dtype
 * Replaces the promotion step of mxfp4_gemm.py:141-150 (_mxfp4_gemm_packed_
 * kernel, op_fmt LSMX_CODES_PACKED: a [M, lda] and bt [N, ldb] packed FP4
 * bytes) and mxfp4_gemm.py:52-63 (_mxfp4_gemm_fp8_kernel, op_fmt
 * LSMX_E4M3: E4M3 bytes, bt = the reference's b_fp8 [K, N] transposed), with
 * Triton's fma contraction of `acc += p * (sa * sb)`.  Scale (row r, block
 * kb) of A is a_scale[r * sa_row + kb * sa_blk], likewise b_scale (the
 * reference's b_scale [K/32, N] of mxfp4_gemm_fp8 has sb_row = 1, sb_blk =
 * N).  K % 128 == 0; operand rows 16-byte aligned; c [M, ldc] of c_dtype
 * (LSMX_F32 | LSMX_BF16 | LSMX_F16).  With flag NULL it always computes.
 * Otherwise the launch does nothing unless *flag == epoch: call
 * lsmx_scale_to_e8m0_batch(flag, epoch), then lsmx_gemm_f4f4 / lsmx_gemm_f8f8
 * on its E8M0 bytes, then this on the same C, and a call whose scales are all
 * powers of two costs one early-exit launch while the others get every
 * output recomputed by this kernel.  Vector-ALU bound (2 fp32 operations per
 * output per 32-block): a fallback, not a fast path.
 * op_fmt LSMX_E4M3 | LSMX_B_NCONTIG: bt is instead the reference's b_fp8
 * itself, [K, ldb] E4M3 with N contiguous (N % 16 == 0, ldb >= N; the
 * lsmx_gemm_f8f8_nb form), read with transposing LDS loads: same bits. */
#define LSMX_B_NCONTIG 0x10
int lsmx_gemm_mx_promote(const uint8_t *a, int64_t lda, const float *a_scale, int64_t sa_row, int64_t sa_blk,
                         const uint8_t *bt, int64_t ldb, const float *b_scale, int64_t sb_row, int64_t sb_blk,
                         int op_fmt, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K,
                         const uint64_t *flag, uint64_t epoch, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LSMX_H */
