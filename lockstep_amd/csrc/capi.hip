// C ABI of liblsmx.so: argument validation, device guard, error reporting,
// and dispatch to the kernel launchers.  Declarations and reference
// citations: include/lsmx.h.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>

#include "lsmx_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

// Per-device cache of the architecture check (0 = unknown, 1 = gfx950, 2 = other).
constexpr int kMaxDev = 64;
int g_arch_ok[kMaxDev] = {0};
std::mutex g_arch_mu;

int device_guard() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0) return fail(LSMX_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    if (dev >= kMaxDev) return fail(LSMX_ERR_DEVICE, "device index %d out of range", dev);
    int ok = g_arch_ok[dev];
    if (ok == 0) {
        std::lock_guard<std::mutex> lk(g_arch_mu);
        hipDeviceProp_t p;
        e = hipGetDeviceProperties(&p, dev);
        if (e != hipSuccess) return fail(LSMX_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
        ok = strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
        g_arch_ok[dev] = ok;
        if (ok != 1) return fail(LSMX_ERR_DEVICE, "needs a gfx950 (MI355X) GPU: found %s", p.gcnArchName);
    }
    if (ok != 1) return fail(LSMX_ERR_DEVICE, "needs a gfx950 (MI355X) GPU on device %d", dev);
    return LSMX_OK;
}

int launched(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(LSMX_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return LSMX_OK;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int elem_size(int dt) { return dt == LSMX_F32 ? 4 : 2; }

// Split-K scratch of lsmx_gemm_bf16f4_noalloc: the largest partial-tile
// workspace the library asks for on a 256-CU gfx950 (4 K slices x 2 batches
// x 256 tiles' worth of 128 x 256 fp32 partials = 64 MiB; the single form
// needs at most half).
constexpr int64_t kScratchBytes = (int64_t)64 << 20;

}  // namespace

// One copy per device, loaded with this file's code object and held until
// the process ends.  Host code never passes `scratch` itself to a kernel
// (on the host it names a stand-in, not device memory): it uses the device
// address that scratch_of looks up.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::atomic<void *> g_scratch[kMaxDev];
std::mutex g_scratch_mu;

// The device address of `scratch` on the device `stream` runs on: looked up
// with hipGetSymbolAddress once per device, with that device current.
int scratch_of(void *stream, void **out) {
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0) return fail(LSMX_ERR_DEVICE, "scratch: no device for the stream: %s", hipGetErrorString(e));
    if (dev >= kMaxDev) return fail(LSMX_ERR_DEVICE, "scratch: device index %d out of range", dev);
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            int cur = -1;
            if ((e = hipGetDevice(&cur)) != hipSuccess) return fail(LSMX_ERR_DEVICE, "scratch: %s", hipGetErrorString(e));
            if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
                return fail(LSMX_ERR_DEVICE, "scratch: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            const hipError_t e2 = cur != dev ? hipSetDevice(cur) : hipSuccess;
            if (e != hipSuccess || !p)
                return fail(LSMX_ERR_DEVICE, "scratch: hipGetSymbolAddress on device %d: %s", dev, hipGetErrorString(e));
            if (e2 != hipSuccess) return fail(LSMX_ERR_DEVICE, "scratch: hipSetDevice(%d): %s", cur, hipGetErrorString(e2));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return LSMX_OK;
}

}  // namespace

extern "C" {

const char *lsmx_version(void) { return "lsmx 0.1.0 gfx950"; }

const char *lsmx_last_error(void) { return g_err; }

int lsmx_device_check(void) { return device_guard(); }

// The argument checks of lsmx_quantize_mxfp4(_t) and of each tensor of
// lsmx_quantize_mxfp4_batch.
static int check_quant(const char *fn, const void *x, int x_dtype, int64_t rows, int64_t K, int64_t ldx, int block,
                       const void *codes, int codes_fmt, int64_t ld_codes, const void *scale, int scale_fmt,
                       int64_t ld_scale, bool cols) {
    if (!x || !codes || !scale) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (x_dtype != LSMX_F32 && x_dtype != LSMX_BF16 && x_dtype != LSMX_F16)
        return fail(LSMX_ERR_DTYPE, "%s: x_dtype %d unsupported", fn, x_dtype);
    if (codes_fmt != LSMX_CODES_PACKED && codes_fmt != LSMX_CODES_UNPACKED)
        return fail(LSMX_ERR_DTYPE, "%s: codes_fmt %d unsupported", fn, codes_fmt);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_F32 && scale_fmt != LSMX_SCALE_E8M0_KMAJOR)
        return fail(LSMX_ERR_DTYPE, "%s: scale_fmt %d unsupported", fn, scale_fmt);
    if (block != 32 && block != 16) return fail(LSMX_ERR_SHAPE, "%s: block must be 16 or 32, got %d", fn, block);
    if (scale_fmt == LSMX_SCALE_E8M0_KMAJOR && (block != 32 || K % 128 != 0))
        return fail(LSMX_ERR_SHAPE, "%s: K-major E8M0 scales need block 32 and K %% 128 == 0", fn);
    if (rows < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % block != 0) return fail(LSMX_ERR_SHAPE, "K=%lld must be a multiple of block=%d", (long long)K, block);
    const int64_t lead = cols ? rows : K;  // the contiguous extent of x
    if (ldx < lead) return fail(LSMX_ERR_SHAPE, "%s: ldx %lld < %lld", fn, (long long)ldx, (long long)lead);
    const int64_t code_w = codes_fmt == LSMX_CODES_PACKED ? K / 2 : K;
    if (ld_codes < code_w) return fail(LSMX_ERR_SHAPE, "%s: ld_codes %lld < %lld", fn, (long long)ld_codes, (long long)code_w);
    if (scale_fmt == LSMX_SCALE_E8M0_KMAJOR ? ld_scale < rows : ld_scale < K / block)
        return fail(LSMX_ERR_SHAPE, "%s: ld_scale too small", fn);
    const int es = elem_size(x_dtype);
    if (!cols) {
        // each lane reads 16 B of a row and writes 2..8 B of codes
        const int vec_el = 16 / es;
        const int code_b = (codes_fmt == LSMX_CODES_PACKED ? vec_el / 2 : vec_el);
        if (!aligned(x, 16) || (ldx * es) % 16) return fail(LSMX_ERR_ALIGN, "%s: x rows must be 16-byte aligned", fn);
        if (!aligned(codes, code_b) || ld_codes % code_b) return fail(LSMX_ERR_ALIGN, "%s: codes rows must be %d-byte aligned", fn, code_b);
    } else {
        if (!aligned(x, es)) return fail(LSMX_ERR_ALIGN, "%s: x misaligned", fn);
        const int code_b = codes_fmt == LSMX_CODES_PACKED ? block / 2 : 16;
        if (!aligned(codes, code_b) || ld_codes % code_b) return fail(LSMX_ERR_ALIGN, "%s: codes rows must be %d-byte aligned", fn, code_b);
    }
    if ((scale_fmt == LSMX_SCALE_F32 || scale_fmt == LSMX_SCALE_E8M0_KMAJOR) && !aligned(scale, 4))
        return fail(LSMX_ERR_ALIGN, "%s: fp32 and K-major scales must be 4-byte aligned", fn);
    return LSMX_OK;
}

static int quantize_common(const void *x, int x_dtype, int64_t rows, int64_t K, int64_t ldx, int block,
                           void *codes, int codes_fmt, int64_t ld_codes, void *scale, int scale_fmt,
                           int64_t ld_scale, void *stream, bool cols) {
    const char *fn = cols ? "lsmx_quantize_mxfp4_t" : "lsmx_quantize_mxfp4";
    if (int r = check_quant(fn, x, x_dtype, rows, K, ldx, block, codes, codes_fmt, ld_codes, scale, scale_fmt,
                            ld_scale, cols))
        return r;
    if (int r = device_guard()) return r;
    if (rows == 0 || K == 0) return LSMX_OK;
    lsmx::QuantArgs a{x, x_dtype, rows, K, ldx, block, codes, codes_fmt, ld_codes, scale, scale_fmt, ld_scale};
    return launched(lsmx::launch_quantize(a, cols, (hipStream_t)stream), fn);
}

int lsmx_quantize_mxfp4(const void *x, int x_dtype, int64_t rows, int64_t K, int64_t ldx, int block,
                        void *codes, int codes_fmt, int64_t ld_codes, void *scale, int scale_fmt,
                        int64_t ld_scale, void *stream) {
    return quantize_common(x, x_dtype, rows, K, ldx, block, codes, codes_fmt, ld_codes, scale, scale_fmt,
                           ld_scale, stream, false);
}

int lsmx_quantize_mxfp4_t(const void *x, int x_dtype, int64_t K, int64_t cols, int64_t ldx, int block,
                          void *codes, int codes_fmt, int64_t ld_codes, void *scale, int scale_fmt,
                          int64_t ld_scale, void *stream) {
    return quantize_common(x, x_dtype, cols, K, ldx, block, codes, codes_fmt, ld_codes, scale, scale_fmt,
                           ld_scale, stream, true);
}

int lsmx_quantize_mxfp4_batch(const lsmx_q_item *items, int n, int x_dtype, int scale_fmt, void *stream) {
    const char *fn = "lsmx_quantize_mxfp4_batch";
    if (!items) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (n < 0 || n > lsmx::kQBatch) return fail(LSMX_ERR_SHAPE, "%s: n must be 0 .. %d", fn, lsmx::kQBatch);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_E8M0_KMAJOR)
        return fail(LSMX_ERR_DTYPE, "%s: scale_fmt must be E8M0 or K-major E8M0", fn);
    lsmx::QuantBatch b{};
    int64_t rows = 0;
    for (int k = 0; k < n; ++k) {
        const lsmx_q_item &it = items[k];
        if (int r = check_quant(fn, it.x, x_dtype, it.rows, it.K, it.ldx, 32, it.codes, LSMX_CODES_PACKED,
                                it.ld_codes, it.scale, scale_fmt, it.ld_scale, false))
            return r;
        if (it.rows == 0 || it.K == 0) continue;   // empty tensors take no row of the grid
        b.a[b.n] = lsmx::QuantArgs{it.x, x_dtype, it.rows, it.K, it.ldx, 32, it.codes, LSMX_CODES_PACKED,
                                   it.ld_codes, it.scale, scale_fmt, it.ld_scale};
        rows += it.rows;
        b.end[b.n++] = rows;
    }
    if (int r = device_guard()) return r;
    if (b.n == 0) return LSMX_OK;
    return launched(lsmx::launch_quantize_batch(b, (hipStream_t)stream), fn);
}

// The argument checks of one tensor of lsmx_quantize_mxfp4_2d(_batch).
static int check_q2d(const char *fn, const void *x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
                     const uint8_t *codes_r, int64_t ld_codes_r, const uint8_t *scale_r, int64_t ld_scale_r,
                     const uint8_t *codes_c, int64_t ld_codes_c, const uint8_t *scale_c, int64_t ld_scale_c,
                     int scale_fmt) {
    if (!x || !codes_r || !scale_r || !codes_c || !scale_c) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (x_dtype != LSMX_BF16 && x_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: x_dtype must be bf16 or fp16", fn);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_E8M0_KMAJOR)
        return fail(LSMX_ERR_DTYPE, "%s: scale_fmt must be E8M0 or K-major E8M0", fn);
    if (rows < 0 || cols < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (rows % 128 || cols % 128) return fail(LSMX_ERR_SHAPE, "%s: rows and cols must be multiples of 128", fn);
    const bool km = scale_fmt == LSMX_SCALE_E8M0_KMAJOR;
    if (ldx < cols || ld_codes_r < cols / 2 || ld_codes_c < rows / 2 || ld_scale_r < (km ? rows : cols / 32) ||
        ld_scale_c < (km ? cols : rows / 32))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!aligned(x, 16) || (ldx * 2) % 16) return fail(LSMX_ERR_ALIGN, "%s: x rows must be 16-byte aligned", fn);
    if (!aligned(codes_r, 4) || ld_codes_r % 4 || !aligned(codes_c, 16) || ld_codes_c % 16)
        return fail(LSMX_ERR_ALIGN, "%s: row codes need 4-byte, column codes 16-byte aligned rows", fn);
    if (!aligned(scale_r, 4) || !aligned(scale_c, 4) || (!km && (ld_scale_r % 4 || ld_scale_c % 4)))
        return fail(LSMX_ERR_ALIGN, "%s: scales must be 4-byte aligned", fn);
    if ((rows / 128) * (cols / 128) > 0x7FFFFFFF) return fail(LSMX_ERR_SHAPE, "%s: too many tiles", fn);
    return LSMX_OK;
}

int lsmx_quantize_mxfp4_2d(const void *x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx, uint8_t *codes_r,
                           int64_t ld_codes_r, uint8_t *scale_r, int64_t ld_scale_r, uint8_t *codes_c,
                           int64_t ld_codes_c, uint8_t *scale_c, int64_t ld_scale_c, int scale_fmt, void *stream) {
    const char *fn = "lsmx_quantize_mxfp4_2d";
    if (int r = check_q2d(fn, x, x_dtype, rows, cols, ldx, codes_r, ld_codes_r, scale_r, ld_scale_r, codes_c,
                          ld_codes_c, scale_c, ld_scale_c, scale_fmt))
        return r;
    if (int r = device_guard()) return r;
    if (rows == 0 || cols == 0) return LSMX_OK;
    lsmx::Quant2dArgs a{x, x_dtype, rows, cols, ldx, codes_r, ld_codes_r, scale_r, ld_scale_r,
                        codes_c, ld_codes_c, scale_c, ld_scale_c, scale_fmt};
    return launched(lsmx::launch_quantize_2d(a, (hipStream_t)stream), fn);
}

int lsmx_quantize_mxfp4_2d_batch(const lsmx_q2d_item *items, int n, int x_dtype, int scale_fmt, void *stream) {
    const char *fn = "lsmx_quantize_mxfp4_2d_batch";
    if (!items) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (n < 0 || n > lsmx::kQ2Batch) return fail(LSMX_ERR_SHAPE, "%s: n must be 0 .. %d", fn, lsmx::kQ2Batch);
    lsmx::Quant2dBatch b{};
    int64_t tiles = 0;
    for (int k = 0; k < n; ++k) {
        const lsmx_q2d_item &it = items[k];
        if (int r = check_q2d(fn, it.x, x_dtype, it.rows, it.cols, it.ldx, it.codes_r, it.ld_codes_r, it.scale_r,
                              it.ld_scale_r, it.codes_c, it.ld_codes_c, it.scale_c, it.ld_scale_c, scale_fmt))
            return r;
        const int64_t t = (it.rows / 128) * (it.cols / 128);
        if (t == 0) continue;                      // empty tensors take no workgroup
        if (tiles + t > 0x7FFFFFFF) return fail(LSMX_ERR_SHAPE, "%s: too many tiles", fn);
        b.a[b.n] = lsmx::Quant2dArgs{it.x, x_dtype, it.rows, it.cols, it.ldx, it.codes_r, it.ld_codes_r,
                                     it.scale_r, it.ld_scale_r, it.codes_c, it.ld_codes_c, it.scale_c,
                                     it.ld_scale_c, scale_fmt};
        tiles += t;
        b.end[b.n++] = tiles;
    }
    if (int r = device_guard()) return r;
    if (b.n == 0) return LSMX_OK;
    return launched(lsmx::launch_quantize_2d_batch(b, (hipStream_t)stream), fn);
}

int lsmx_round_e2m1(const void *q, int q_dtype, int64_t n, uint8_t *codes, void *stream) {
    if (!q || !codes) return fail(LSMX_ERR_ARG, "lsmx_round_e2m1: null pointer");
    if (q_dtype != LSMX_F32 && q_dtype != LSMX_BF16 && q_dtype != LSMX_F16)
        return fail(LSMX_ERR_DTYPE, "lsmx_round_e2m1: q_dtype %d unsupported", q_dtype);
    if (n < 0) return fail(LSMX_ERR_SHAPE, "lsmx_round_e2m1: negative size");
    if (!aligned(q, elem_size(q_dtype))) return fail(LSMX_ERR_ALIGN, "lsmx_round_e2m1: q misaligned");
    if (int r = device_guard()) return r;
    if (n == 0) return LSMX_OK;
    return launched(lsmx::launch_round(q, q_dtype, n, codes, (hipStream_t)stream), "lsmx_round_e2m1");
}

int lsmx_pack_fp4(const uint8_t *codes, uint8_t *packed, int64_t n_bytes, void *stream) {
    if (!codes || !packed) return fail(LSMX_ERR_ARG, "lsmx_pack_fp4: null pointer");
    if (n_bytes < 0) return fail(LSMX_ERR_SHAPE, "lsmx_pack_fp4: negative size");
    if (!aligned(codes, 16) || !aligned(packed, 8)) return fail(LSMX_ERR_ALIGN, "lsmx_pack_fp4: codes need 16-byte, packed 8-byte alignment");
    if (int r = device_guard()) return r;
    if (n_bytes == 0) return LSMX_OK;
    return launched(lsmx::launch_pack(codes, packed, n_bytes, (hipStream_t)stream), "lsmx_pack_fp4");
}

int lsmx_unpack_fp4(const uint8_t *packed, uint8_t *codes, int64_t n_bytes, void *stream) {
    if (!codes || !packed) return fail(LSMX_ERR_ARG, "lsmx_unpack_fp4: null pointer");
    if (n_bytes < 0) return fail(LSMX_ERR_SHAPE, "lsmx_unpack_fp4: negative size");
    if (!aligned(codes, 16) || !aligned(packed, 8)) return fail(LSMX_ERR_ALIGN, "lsmx_unpack_fp4: codes need 16-byte, packed 8-byte alignment");
    if (int r = device_guard()) return r;
    if (n_bytes == 0) return LSMX_OK;
    return launched(lsmx::launch_unpack(packed, codes, n_bytes, (hipStream_t)stream), "lsmx_unpack_fp4");
}

int lsmx_dequantize_mxfp4(const void *codes, int codes_fmt, int64_t ld_codes, const void *scale, int scale_fmt,
                          int64_t ld_scale, int64_t rows, int64_t K, int block, void *out, int out_dtype,
                          int64_t ld_out, void *stream) {
    const char *fn = "lsmx_dequantize_mxfp4";
    if (!codes || !scale || !out) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (codes_fmt != LSMX_CODES_PACKED && codes_fmt != LSMX_CODES_UNPACKED) return fail(LSMX_ERR_DTYPE, "%s: codes_fmt", fn);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_F32) return fail(LSMX_ERR_DTYPE, "%s: scale_fmt", fn);
    if (out_dtype != LSMX_F32 && out_dtype != LSMX_BF16) return fail(LSMX_ERR_DTYPE, "%s: out_dtype", fn);
    if (block != 32 && block != 16) return fail(LSMX_ERR_SHAPE, "%s: block must be 16 or 32", fn);
    if (rows < 0 || K < 0 || K % block) return fail(LSMX_ERR_SHAPE, "K=%lld must be a multiple of block=%d", (long long)K, block);
    const int cb = codes_fmt == LSMX_CODES_PACKED ? 4 : 8;
    if (!aligned(codes, cb) || ld_codes % cb) return fail(LSMX_ERR_ALIGN, "%s: codes rows misaligned", fn);
    const int ob = out_dtype == LSMX_F32 ? 4 : 2;
    if (!aligned(out, 16) || (ld_out * ob) % 16) return fail(LSMX_ERR_ALIGN, "%s: out rows must be 16-byte aligned", fn);
    if (scale_fmt == LSMX_SCALE_F32 && !aligned(scale, 4)) return fail(LSMX_ERR_ALIGN, "%s: scale misaligned", fn);
    if (int r = device_guard()) return r;
    if (rows == 0 || K == 0) return LSMX_OK;
    lsmx::DequantArgs a{codes, codes_fmt, ld_codes, scale, scale_fmt, ld_scale, rows, K, block, out, out_dtype, ld_out};
    return launched(lsmx::launch_dequant(a, (hipStream_t)stream), fn);
}

int lsmx_fp4_to_e4m3(const uint32_t *in, uint32_t *out, int64_t n_words, void *stream) {
    if (!in || !out) return fail(LSMX_ERR_ARG, "lsmx_fp4_to_e4m3: null pointer");
    if (n_words < 0) return fail(LSMX_ERR_SHAPE, "lsmx_fp4_to_e4m3: negative size");
    if (!aligned(in, 4) || !aligned(out, 8)) return fail(LSMX_ERR_ALIGN, "lsmx_fp4_to_e4m3: misaligned");
    if (int r = device_guard()) return r;
    if (n_words == 0) return LSMX_OK;
    return launched(lsmx::launch_fp4_to_e4m3(in, out, n_words, (hipStream_t)stream), "lsmx_fp4_to_e4m3");
}

static int check_scale(const char *fn, const void *s, int64_t ld, int fmt, int per_stage, int64_t rows,
                       int64_t K) {
    if (fmt == LSMX_SCALE_E8M0_KMAJOR) {
        // [K/128][ld][4]: one dword per row per 128-K slice
        if (!aligned(s, 4)) return fail(LSMX_ERR_ALIGN, "%s: K-major scales must be 4-byte aligned", fn);
        if (ld < rows) return fail(LSMX_ERR_SHAPE, "%s: K-major scale row stride %lld < %lld", fn, (long long)ld, (long long)rows);
        if (K % 128) return fail(LSMX_ERR_SHAPE, "%s: K-major scales need K %% 128 == 0", fn);
        return LSMX_OK;
    }
    if (ld < K / 32) return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    // the GEMMs read `per_stage` consecutive scales with one aligned load
    const int bytes = per_stage * (fmt == LSMX_SCALE_F32 ? 4 : 1);
    if (!aligned(s, bytes) || (ld * (fmt == LSMX_SCALE_F32 ? 4 : 1)) % bytes)
        return fail(LSMX_ERR_ALIGN, "%s: scale rows must be %d-byte aligned", fn, bytes);
    return LSMX_OK;
}

int lsmx_gemm_f4f4(const uint8_t *a_pk, int64_t lda, const void *a_scale, int64_t ld_sa, const uint8_t *bt_pk,
                   int64_t ldb, const void *b_scale, int64_t ld_sb, int scale_fmt, void *c, int c_dtype,
                   int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
    const char *fn = "lsmx_gemm_f4f4";
    if (!a_pk || !a_scale || !bt_pk || !b_scale || !c) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_F32 && scale_fmt != LSMX_SCALE_E8M0_KMAJOR)
        return fail(LSMX_ERR_DTYPE, "%s: scale_fmt", fn);
    if (c_dtype != LSMX_F32 && c_dtype != LSMX_BF16 && c_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: c_dtype", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 128 != 0) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 128 (max BLOCK_K)");
    if (M > (int64_t)1 << 30 || N > (int64_t)1 << 30) return fail(LSMX_ERR_SHAPE, "%s: M, N must be < 2^30", fn);
    if (lda < K / 2 || ldb < K / 2 || ldc < N) return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!aligned(a_pk, 16) || !aligned(bt_pk, 16) || lda % 16 || ldb % 16)
        return fail(LSMX_ERR_ALIGN, "%s: packed rows must be 16-byte aligned", fn);
    if (int r = check_scale(fn, a_scale, ld_sa, scale_fmt, 4, M, K)) return r;
    if (int r = check_scale(fn, b_scale, ld_sb, scale_fmt, 4, N, K)) return r;
    // the kernel's per-lane buffer offsets are 32-bit: up to 256 rows of
    // codes, and of row-major scales, past a descriptor's base
    const int64_t sbw = scale_fmt == LSMX_SCALE_F32 ? 4 : 1;
    if (lda >= ((int64_t)1 << 24) || ldb >= ((int64_t)1 << 24) ||
        (scale_fmt != LSMX_SCALE_E8M0_KMAJOR && (ld_sa * sbw >= ((int64_t)1 << 24) || ld_sb * sbw >= ((int64_t)1 << 24))))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit load offsets", fn);
    if (!aligned(c, c_dtype == LSMX_F32 ? 4 : 2)) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::GemmArgs g{a_pk, nullptr, lda, a_scale, ld_sa, bt_pk, ldb, b_scale, ld_sb, scale_fmt, c, nullptr,
                     c_dtype, ldc, M, N, K};
    return launched(lsmx::launch_gemm_f4f4(g, (hipStream_t)stream), fn);
}

int lsmx_gemm_f4f4_quant(const uint8_t *a_pk, int64_t lda, const void *a_scale, int64_t ld_sa, const uint8_t *bt_pk,
                         int64_t ldb, const void *b_scale, int64_t ld_sb, void *c, int64_t ldc, uint8_t *codes_r,
                         int64_t ld_codes_r, uint8_t *scale_r, int64_t ld_scale_r, uint8_t *codes_c,
                         int64_t ld_codes_c, uint8_t *scale_c, int64_t ld_scale_c, int64_t M, int64_t N, int64_t K,
                         void *stream) {
    const char *fn = "lsmx_gemm_f4f4_quant";
    if (!a_pk || !a_scale || !bt_pk || !b_scale || !codes_r || !scale_r || !codes_c || !scale_c)
        return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (M % 256 || N % 256 || K % 256)
        return fail(LSMX_ERR_SHAPE, "%s: M, N and K must be multiples of 256 (whole output tiles and stages)", fn);
    if (M > (int64_t)1 << 30 || N > (int64_t)1 << 30) return fail(LSMX_ERR_SHAPE, "%s: M, N must be < 2^30", fn);
    if (lda < K / 2 || ldb < K / 2 || (c && ldc < N) || ld_codes_r < N / 2 || ld_codes_c < M / 2 ||
        ld_scale_r < M || ld_scale_c < N)
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!aligned(a_pk, 16) || !aligned(bt_pk, 16) || lda % 16 || ldb % 16)
        return fail(LSMX_ERR_ALIGN, "%s: packed rows must be 16-byte aligned", fn);
    if (int r = check_scale(fn, a_scale, ld_sa, LSMX_SCALE_E8M0_KMAJOR, 4, M, K)) return r;
    if (int r = check_scale(fn, b_scale, ld_sb, LSMX_SCALE_E8M0_KMAJOR, 4, N, K)) return r;
    if (lda >= ((int64_t)1 << 24) || ldb >= ((int64_t)1 << 24))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit load offsets", fn);
    // the epilogue's per-lane store offsets are 32-bit: 16 rows of codes
    // (and of C) past a wave-uniform base
    if (ld_codes_r >= ((int64_t)1 << 27) || ld_codes_c >= ((int64_t)1 << 27) || (c && ldc >= ((int64_t)1 << 26)))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit store offsets", fn);
    if (c && (!aligned(c, 16) || (ldc * 2) % 16)) return fail(LSMX_ERR_ALIGN, "%s: c rows must be 16-byte aligned", fn);
    if (!aligned(codes_r, 4) || ld_codes_r % 4 || !aligned(codes_c, 8) || ld_codes_c % 8)
        return fail(LSMX_ERR_ALIGN, "%s: row codes need 4-byte, column codes 8-byte aligned rows", fn);
    if (!aligned(scale_r, 4) || !aligned(scale_c, 4)) return fail(LSMX_ERR_ALIGN, "%s: scales must be 4-byte aligned", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::GemmArgs g{a_pk, nullptr, lda, a_scale, ld_sa, bt_pk, ldb, b_scale, ld_sb, LSMX_SCALE_E8M0_KMAJOR, c,
                     nullptr, LSMX_BF16, ldc, M, N, K};
    g.codes_r = codes_r;
    g.ld_cr = ld_codes_r;
    g.scale_r = scale_r;
    g.ld_sr = ld_scale_r;
    g.codes_c = codes_c;
    g.ld_cc = ld_codes_c;
    g.scale_c = scale_c;
    g.ld_sc = ld_scale_c;
    return launched(lsmx::launch_gemm_f4f4_quant(g, (hipStream_t)stream), fn);
}

static int rows16(const void *p, int64_t ld, int es) { return aligned(p, 16) && (ld * es) % 16 == 0; }

int lsmx_gemm_dense(const void *a0, const void *a1, int64_t lda, const void *bt0, const void *bt1, int64_t ldb,
                    int dtype, int mode, float *c0, float *c1, int64_t ldc, int64_t M, int64_t N, int64_t K,
                    int splits, void *stream) {
    const char *fn = "lsmx_gemm_dense";
    if (dtype != LSMX_BF16 && dtype != LSMX_F16 && dtype != LSMX_E4M3)
        return fail(LSMX_ERR_DTYPE, "%s: dtype must be bf16, fp16 or e4m3", fn);
    if (mode < 0 || mode > 2) return fail(LSMX_ERR_ARG, "%s: mode must be 0, 1 or 2", fn);
    if (!a0 || !bt0 || !c0 || (mode && (!a1 || !bt1)) || (mode == 2 && !c1))
        return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 64) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 64 (max BLOCK_K); zero-pad if shorter");
    if (splits < 1 || K % (64 * (int64_t)splits)) return fail(LSMX_ERR_SHAPE, "K must divide splits*BK");
    if (splits > 65535) return fail(LSMX_ERR_SHAPE, "%s: at most 65535 splits", fn);
    if (((M + 127) / 128) * ((N + 127) / 128) > 0x7FFFFFFF)
        return fail(LSMX_ERR_SHAPE, "%s: more than 2^31 - 1 output tiles", fn);
    if (lda < K || ldb < K || ldc < N) return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    const int es = dtype == LSMX_E4M3 ? 1 : 2;
    if (!rows16(a0, lda, es) || !rows16(bt0, ldb, es) || (mode && (!rows16(a1, lda, es) || !rows16(bt1, ldb, es))))
        return fail(LSMX_ERR_ALIGN, "%s: operand rows must be 16-byte aligned", fn);
    if (!aligned(c0, 4) || (c1 && !aligned(c1, 4))) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::DenseArgs g{reinterpret_cast<const uint8_t *>(a0), reinterpret_cast<const uint8_t *>(a1), lda,
                      reinterpret_cast<const uint8_t *>(bt0), reinterpret_cast<const uint8_t *>(bt1), ldb,
                      nullptr, nullptr, 0, 0, c0, c1, LSMX_F32, ldc, M, N, K, K / splits};
    if (lsmx::dense_ring_ok(g, dtype)) return launched(lsmx::launch_gemm_dense_ring(g, dtype, mode, (hipStream_t)stream), fn);
    return launched(lsmx::launch_gemm_dense(g, dtype, mode, (hipStream_t)stream), fn);
}

int lsmx_gemm_f8f8_nb(const uint8_t *a, int64_t lda, const uint8_t *a_e8m0, int64_t ld_sa, const uint8_t *b,
                      int64_t ldb, const uint8_t *b_e8m0, int64_t ld_sb, void *c, int c_dtype, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, void *stream) {
    const char *fn = "lsmx_gemm_f8f8_nb";
    if (!a || !a_e8m0 || !b || !b_e8m0 || !c) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (c_dtype != LSMX_F32 && c_dtype != LSMX_BF16 && c_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: c_dtype", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 128) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 128 (max BLOCK_K)");
    // whole 16-byte pieces of every B row (see lsmx_gemm_dense_nb)
    if (N % 16) return fail(LSMX_ERR_SHAPE, "%s: N must be a multiple of 16", fn);
    if (lda < K || ldb < N || ldc < N || ld_sa < M || ld_sb < N)
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!rows16(a, lda, 1) || !rows16(b, ldb, 1)) return fail(LSMX_ERR_ALIGN, "%s: operand rows must be 16-byte aligned", fn);
    if (!aligned(a_e8m0, 4) || !aligned(b_e8m0, 4)) return fail(LSMX_ERR_ALIGN, "%s: K-major scales must be 4-byte aligned", fn);
    if (!aligned(c, c_dtype == LSMX_F32 ? 4 : 2)) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (lda > 0x7FFFFFFF / 256 || ldb > 0x7FFFFFFF / 256)
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit load offsets", fn);
    if (M > 0x7FFFFFFF || N > 0x7FFFFFFF || ld_sa > 0x7FFFFFFF || ld_sb > 0x7FFFFFFF ||
        ((M + 255) / 256) * ((N + 255) / 256) > 0x7FFFFFFF)
        return fail(LSMX_ERR_SHAPE, "%s: M, N and scale leading dimensions must be below 2^31", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::DenseArgs g{a, nullptr, lda, b, nullptr, ldb, a_e8m0, b_e8m0, ld_sa, ld_sb, c, nullptr, c_dtype, ldc,
                      M, N, K, K, 1};
    return launched(lsmx::launch_gemm_f8f8_kmajor(g, (hipStream_t)stream), fn);
}

int lsmx_gemm_dense_nb(const void *a0, const void *a1, int64_t lda, const void *b0, const void *b1, int64_t ldb,
                       int dtype, int mode, float *c0, float *c1, int64_t ldc, int64_t M, int64_t N, int64_t K,
                       void *stream) {
    const char *fn = "lsmx_gemm_dense_nb";
    if (dtype != LSMX_BF16 && dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: dtype must be bf16 or fp16", fn);
    if (mode < 0 || mode > 2) return fail(LSMX_ERR_ARG, "%s: mode must be 0, 1 or 2", fn);
    if (!a0 || !b0 || !c0 || (mode && (!a1 || !b1)) || (mode == 2 && !c1))
        return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 64) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 64 (max BLOCK_K); zero-pad if shorter");
    // whole 16-byte pieces of every B row: the last row's loads stop at its
    // N-th column, and a piece cut there would read as zeros
    if (N % 8) return fail(LSMX_ERR_SHAPE, "%s: N must be a multiple of 8", fn);
    if (((M + 255) / 256) * ((N + 255) / 256) > 0x3FFFFFFF)
        return fail(LSMX_ERR_SHAPE, "%s: too many output tiles", fn);
    if (lda < K || ldb < N || ldc < N) return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (lda > ((int64_t)1 << 22) || ldb > ((int64_t)1 << 22))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimensions above 2^22 elements", fn);
    if (!rows16(a0, lda, 2) || !rows16(b0, ldb, 2) || (mode && (!rows16(a1, lda, 2) || !rows16(b1, ldb, 2))))
        return fail(LSMX_ERR_ALIGN, "%s: operand rows must be 16-byte aligned", fn);
    if (!aligned(c0, 4) || (c1 && !aligned(c1, 4))) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::DenseArgs g{reinterpret_cast<const uint8_t *>(a0), reinterpret_cast<const uint8_t *>(a1), lda,
                      reinterpret_cast<const uint8_t *>(b0), reinterpret_cast<const uint8_t *>(b1), ldb,
                      nullptr, nullptr, 0, 0, c0, c1, LSMX_F32, ldc, M, N, K, K, 1};
    return launched(lsmx::launch_gemm_dense_ring(g, dtype, mode, (hipStream_t)stream), fn);
}

int lsmx_gemm_f8f8(const uint8_t *a, int64_t lda, const uint8_t *a_e8m0, int64_t ld_sa, const uint8_t *bt,
                   int64_t ldb, const uint8_t *b_e8m0, int64_t ld_sb, int scale_fmt, void *c, int c_dtype,
                   int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
    const char *fn = "lsmx_gemm_f8f8";
    if (!a || !a_e8m0 || !bt || !b_e8m0 || !c) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (c_dtype != LSMX_F32 && c_dtype != LSMX_BF16 && c_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: c_dtype", fn);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_E8M0_KMAJOR)
        return fail(LSMX_ERR_DTYPE, "%s: scale_fmt must be E8M0 or K-major E8M0", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 128) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 128 (max BLOCK_K)");
    if (((M + 127) / 128) * ((N + 127) / 128) > 0x7FFFFFFF)
        return fail(LSMX_ERR_SHAPE, "%s: more than 2^31 - 1 output tiles", fn);
    const bool km = scale_fmt == LSMX_SCALE_E8M0_KMAJOR;
    if (lda < K || ldb < K || ldc < N || ld_sa < (km ? M : K / 32) || ld_sb < (km ? N : K / 32))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!rows16(a, lda, 1) || !rows16(bt, ldb, 1)) return fail(LSMX_ERR_ALIGN, "%s: operand rows must be 16-byte aligned", fn);
    if (km && (!aligned(a_e8m0, 4) || !aligned(b_e8m0, 4))) return fail(LSMX_ERR_ALIGN, "%s: K-major scales must be 4-byte aligned", fn);
    if (!aligned(c, c_dtype == LSMX_F32 ? 4 : 2)) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (km && (lda > 0x7FFFFFFF / 256 || ldb > 0x7FFFFFFF / 256))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit load offsets", fn);
    if (km && (M > 0x7FFFFFFF || N > 0x7FFFFFFF || ld_sa > 0x7FFFFFFF || ld_sb > 0x7FFFFFFF))
        return fail(LSMX_ERR_SHAPE, "%s: M, N and scale leading dimensions must be below 2^31", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::DenseArgs g{a, nullptr, lda, bt, nullptr, ldb, a_e8m0, b_e8m0, ld_sa, ld_sb, c, nullptr, c_dtype, ldc,
                      M, N, K, K};
    if (km) return launched(lsmx::launch_gemm_f8f8_kmajor(g, (hipStream_t)stream), fn);
    return launched(lsmx::launch_gemm_f8f8_scaled(g, (hipStream_t)stream), fn);
}

int lsmx_transpose(const void *x, int elem_bytes, int64_t rows, int64_t cols, int64_t ldx, void *y, int64_t ldy,
                   void *stream) {
    const char *fn = "lsmx_transpose";
    if (!x || !y) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) return fail(LSMX_ERR_DTYPE, "%s: elem_bytes", fn);
    if (rows < 0 || cols < 0 || ldx < cols || ldy < rows) return fail(LSMX_ERR_SHAPE, "%s: bad shape", fn);
    if (!aligned(x, elem_bytes) || !aligned(y, elem_bytes)) return fail(LSMX_ERR_ALIGN, "%s: misaligned", fn);
    if (rows > (int64_t)65535 * 64 || cols > (int64_t)0x7FFFFFFF * 64) return fail(LSMX_ERR_SHAPE, "%s: too large", fn);
    if (int r = device_guard()) return r;
    if (rows == 0 || cols == 0) return LSMX_OK;
    return launched(lsmx::launch_transpose(x, elem_bytes, rows, cols, ldx, y, ldy, (hipStream_t)stream), fn);
}

int lsmx_scale_to_e8m0(const float *s, int64_t rows, int64_t cols, int64_t lds, int layout, uint8_t *out,
                       int64_t ldo, void *stream) {
    const char *fn = "lsmx_scale_to_e8m0";
    if (!s || !out) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (layout & ~(LSMX_E8M0_IN_T | LSMX_E8M0_OUT_KMAJOR)) return fail(LSMX_ERR_ARG, "%s: layout", fn);
    const bool tin = layout & LSMX_E8M0_IN_T, km = layout & LSMX_E8M0_OUT_KMAJOR;
    const int64_t orows = tin ? cols : rows, blocks = tin ? rows : cols;
    if (rows < 0 || cols < 0 || lds < cols || ldo < (km ? orows : blocks)) return fail(LSMX_ERR_SHAPE, "%s: bad shape", fn);
    if (km && blocks % 4) return fail(LSMX_ERR_SHAPE, "%s: K-major output needs a multiple of 4 blocks", fn);
    if (!aligned(s, 4)) return fail(LSMX_ERR_ALIGN, "%s: misaligned", fn);
    if (rows > 0 && cols > ((int64_t)1 << 38) / rows) return fail(LSMX_ERR_SHAPE, "%s: too large", fn);
    if (int r = device_guard()) return r;
    if (rows == 0 || cols == 0) return LSMX_OK;
    return launched(lsmx::launch_scale_to_e8m0(s, rows, cols, lds, layout, out, ldo, (hipStream_t)stream), fn);
}

int lsmx_scale_to_e8m0_batch(const lsmx_e8m0_item *items, int n, uint64_t *flag, uint64_t epoch, void *stream) {
    const char *fn = "lsmx_scale_to_e8m0_batch";
    if (!items && n) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (n < 0 || n > lsmx::kE8Batch) return fail(LSMX_ERR_SHAPE, "%s: n must be 0 .. %d", fn, lsmx::kE8Batch);
    if (flag && !aligned(flag, 8)) return fail(LSMX_ERR_ALIGN, "%s: flag must be 8-byte aligned", fn);
    lsmx::E8m0Batch b{};
    int64_t wgs = 0;
    for (int k = 0; k < n; ++k) {
        const lsmx_e8m0_item &it = items[k];
        if ((!it.s || !it.out) && it.rows && it.cols) return fail(LSMX_ERR_ARG, "%s: null pointer in item %d", fn, k);
        if (it.layout & ~LSMX_E8M0_IN_T)
            return fail(LSMX_ERR_ARG, "%s: item %d layout must be 0 or LSMX_E8M0_IN_T (the output is K-major)", fn, k);
        const bool tin = it.layout & LSMX_E8M0_IN_T;
        const int64_t orows = tin ? it.cols : it.rows, blocks = tin ? it.rows : it.cols;
        if (it.rows < 0 || it.cols < 0 || it.lds < it.cols || it.ldo < orows)
            return fail(LSMX_ERR_SHAPE, "%s: item %d: bad shape", fn, k);
        if (blocks % 4) return fail(LSMX_ERR_SHAPE, "%s: item %d: K-major output needs a multiple of 4 blocks", fn, k);
        if (!aligned(it.s, 4) || !aligned(it.out, 4)) return fail(LSMX_ERR_ALIGN, "%s: item %d misaligned", fn, k);
        if (it.rows > 0 && it.cols > ((int64_t)1 << 38) / it.rows) return fail(LSMX_ERR_SHAPE, "%s: item %d too large", fn, k);
        const int64_t w = ((orows + 63) / 64) * ((blocks / 4 + 15) / 16);
        if (w == 0) continue;  // empty tensors take no workgroup
        if (wgs + w > 0x7FFFFFFF) return fail(LSMX_ERR_SHAPE, "%s: too many workgroups", fn);
        const int vec4 = !tin && aligned(it.s, 16) && it.lds % 4 == 0;
        b.it[b.n] = lsmx::E8m0Item{it.s, orows, blocks / 4, it.lds, (int)tin, vec4, it.out, it.ldo};
        wgs += w;
        b.end[b.n++] = wgs;
    }
    b.flag = flag;
    b.epoch = epoch;
    if (int r = device_guard()) return r;
    if (b.n == 0) return LSMX_OK;
    return launched(lsmx::launch_scale_to_e8m0_batch(b, (hipStream_t)stream), fn);
}

int lsmx_gemm_mx_promote(const uint8_t *a, int64_t lda, const float *a_scale, int64_t sa_row, int64_t sa_blk,
                         const uint8_t *bt, int64_t ldb, const float *b_scale, int64_t sb_row, int64_t sb_blk,
                         int op_fmt, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K,
                         const uint64_t *flag, uint64_t epoch, void *stream) {
    const char *fn = "lsmx_gemm_mx_promote";
    if (!a || !a_scale || !bt || !b_scale || !c) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    const int b_nc = (op_fmt & LSMX_B_NCONTIG) ? 1 : 0;
    op_fmt &= ~LSMX_B_NCONTIG;
    if (op_fmt != LSMX_CODES_PACKED && op_fmt != LSMX_E4M3)
        return fail(LSMX_ERR_DTYPE, "%s: op_fmt must be LSMX_CODES_PACKED or LSMX_E4M3", fn);
    if (b_nc && op_fmt != LSMX_E4M3) return fail(LSMX_ERR_DTYPE, "%s: LSMX_B_NCONTIG needs LSMX_E4M3", fn);
    if (b_nc && N % 16) return fail(LSMX_ERR_SHAPE, "%s: N must be a multiple of 16 for N-contiguous B", fn);
    if (c_dtype != LSMX_F32 && c_dtype != LSMX_BF16 && c_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: c_dtype", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 128) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 128 (max BLOCK_K)");
    const int64_t kbytes = op_fmt == LSMX_CODES_PACKED ? K / 2 : K;
    if (lda < kbytes || ldb < (b_nc ? N : kbytes) || ldc < N)
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (sa_row < 0 || sa_blk < 0 || sb_row < 0 || sb_blk < 0) return fail(LSMX_ERR_SHAPE, "%s: negative scale stride", fn);
    if (!aligned(a, 16) || !aligned(bt, 16) || lda % 16 || ldb % 16)
        return fail(LSMX_ERR_ALIGN, "%s: operand rows must be 16-byte aligned", fn);
    if (!aligned(a_scale, 4) || !aligned(b_scale, 4) || !aligned(c, elem_size(c_dtype)) || (flag && !aligned(flag, 8)))
        return fail(LSMX_ERR_ALIGN, "%s: misaligned scale, output or flag", fn);
    // the kernel forms every load offset in 32 bits, over rows up to a
    // tile past M or N and blocks up to a chunk past K
    const int64_t lim = (int64_t)1 << 31, nkb = K / 32;
    if (128 * lda + kbytes + 256 >= lim || (b_nc ? 256 * ldb + 256 : 128 * ldb + kbytes + 256) >= lim)
        return fail(LSMX_ERR_SHAPE, "%s: operand rows of %lld / %lld bytes are too long", fn, (long long)lda,
                    (long long)ldb);
    if (M + 128 > lim / 4 || N + 128 > lim / 4 || 4 * ((M + 128) * sa_row + (nkb + 8) * sa_blk) >= lim ||
        4 * ((N + 128) * sb_row + (nkb + 8) * sb_blk) >= lim)
        return fail(LSMX_ERR_SHAPE, "%s: scale tensors span 2^31 bytes or more", fn);
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    const int sa_bytes = nkb ? (int)(4 * ((M - 1) * sa_row + (nkb - 1) * sa_blk + 1)) : 0;
    const int sb_bytes = nkb ? (int)(4 * ((N - 1) * sb_row + (nkb - 1) * sb_blk + 1)) : 0;
    lsmx::PromoteArgs g{a, lda, bt, ldb, a_scale, sa_row, sa_blk, b_scale, sb_row, sb_blk, sa_bytes, sb_bytes,
                        c, c_dtype, ldc, M, N, K, flag, epoch, b_nc};
    return launched(lsmx::launch_gemm_promote(g, op_fmt == LSMX_CODES_PACKED, (hipStream_t)stream), fn);
}

static int w4_common(const char *fn, const void *a0, const void *a1, int a_dtype, int64_t lda, const uint8_t *w_pk,
                     int64_t ldw, const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype,
                     int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream, void *ws = nullptr,
                     int64_t ws_bytes = 0) {
    if (!a0 || !w_pk || !w_scale || !c0) return fail(LSMX_ERR_ARG, "%s: null pointer", fn);
    if (a_dtype != LSMX_BF16 && a_dtype != LSMX_F32 && a_dtype != LSMX_F16)
        return fail(LSMX_ERR_DTYPE, "%s: a_dtype %d unsupported", fn, a_dtype);
    if (a1 && a_dtype != LSMX_BF16) return fail(LSMX_ERR_DTYPE, "%s: the dual form takes bf16 activations", fn);
    if (scale_fmt != LSMX_SCALE_E8M0 && scale_fmt != LSMX_SCALE_F32) return fail(LSMX_ERR_DTYPE, "%s: scale_fmt", fn);
    if (c_dtype != LSMX_F32 && c_dtype != LSMX_BF16 && c_dtype != LSMX_F16) return fail(LSMX_ERR_DTYPE, "%s: c_dtype", fn);
    if (M < 0 || N < 0 || K < 0) return fail(LSMX_ERR_SHAPE, "%s: negative size", fn);
    if (K % 128 != 0) return fail(LSMX_ERR_SHAPE, "K must be a multiple of 128 (max BLOCK_K)");
    if (M > (int64_t)1 << 30 || N > (int64_t)1 << 30) return fail(LSMX_ERR_SHAPE, "%s: M, N must be < 2^30", fn);
    if (lda < K || ldw < K / 2 || ldc < N) return fail(LSMX_ERR_SHAPE, "%s: leading dimension too small", fn);
    if (!aligned(a0, 16) || (a1 && !aligned(a1, 16)) || (lda * elem_size(a_dtype)) % 16)
        return fail(LSMX_ERR_ALIGN, "%s: activation rows must be 16-byte aligned", fn);
    if (!aligned(w_pk, 16) || ldw % 16) return fail(LSMX_ERR_ALIGN, "%s: packed weight rows must be 16-byte aligned", fn);
    if (scale_fmt == LSMX_SCALE_E8M0_KMAJOR) return fail(LSMX_ERR_DTYPE, "%s: K-major scales are not supported here", fn);
    if (int r = check_scale(fn, w_scale, ld_sw, scale_fmt, 2, N, K)) return r;
    // 32-bit per-lane buffer offsets: 8 activation rows, 32 weight rows and
    // 256 rows of scales past a descriptor's base
    if (lda >= ((int64_t)1 << 27) || ldw >= ((int64_t)1 << 27) ||
        ld_sw * (scale_fmt == LSMX_SCALE_F32 ? 4 : 1) >= ((int64_t)1 << 24))
        return fail(LSMX_ERR_SHAPE, "%s: leading dimension too large for 32-bit load offsets", fn);
    const int cb = c_dtype == LSMX_F32 ? 4 : 2;
    if (!aligned(c0, cb) || (c1 && !aligned(c1, cb))) return fail(LSMX_ERR_ALIGN, "%s: c misaligned", fn);
    if (ws) {
        const int64_t need = lsmx::gemm_bf16f4_workspace(M, N, K, a1 != nullptr);
        if (ws_bytes < need)
            return fail(LSMX_ERR_ARG, "%s: workspace of %lld bytes, this shape needs %lld", fn, (long long)ws_bytes,
                        (long long)need);
        if (!aligned(ws, 16)) return fail(LSMX_ERR_ALIGN, "%s: workspace must be 16-byte aligned", fn);
    }
    if (int r = device_guard()) return r;
    if (M == 0 || N == 0) return LSMX_OK;
    if (K == 0) return fail(LSMX_ERR_SHAPE, "%s: K == 0", fn);
    lsmx::GemmArgs g{reinterpret_cast<const uint8_t *>(a0), reinterpret_cast<const uint8_t *>(a1), lda, nullptr, 0,
                     w_pk, ldw, w_scale, ld_sw, scale_fmt, c0, c1, c_dtype, ldc, M, N, K};
    g.ws = reinterpret_cast<float *>(ws);
    if (a_dtype != LSMX_BF16) return launched(lsmx::launch_gemm_xf4(g, a_dtype, (hipStream_t)stream), fn);
    return launched(lsmx::launch_gemm_bf16f4(g, (hipStream_t)stream), fn);
}

int lsmx_gemm_bf16f4(const void *a, int64_t lda, const uint8_t *w_pk, int64_t ldw, const void *w_scale, int64_t ld_sw,
                     int scale_fmt, void *c, int c_dtype, int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
    return w4_common("lsmx_gemm_bf16f4", a, nullptr, LSMX_BF16, lda, w_pk, ldw, w_scale, ld_sw, scale_fmt, c, nullptr, c_dtype,
                     ldc, M, N, K, stream);
}

int lsmx_gemm_dual_bf16f4(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                          const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype,
                          int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
    if (!a1 || !c1) return fail(LSMX_ERR_ARG, "lsmx_gemm_dual_bf16f4: null pointer");
    return w4_common("lsmx_gemm_dual_bf16f4", a0, a1, LSMX_BF16, lda, w_pk, ldw, w_scale, ld_sw, scale_fmt, c0, c1, c_dtype,
                     ldc, M, N, K, stream);
}

int64_t lsmx_gemm_bf16f4_workspace(int64_t M, int64_t N, int64_t K, int dual) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
    return lsmx::gemm_bf16f4_workspace(M, N, K, dual != 0);
}

int lsmx_gemm_bf16f4_ws(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                        const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, void *workspace, int64_t workspace_bytes, void *stream) {
    if ((a1 == nullptr) != (c1 == nullptr)) return fail(LSMX_ERR_ARG, "lsmx_gemm_bf16f4_ws: a1 and c1 go together");
    return w4_common("lsmx_gemm_bf16f4_ws", a0, a1, LSMX_BF16, lda, w_pk, ldw, w_scale, ld_sw, scale_fmt, c0, c1,
                     c_dtype, ldc, M, N, K, stream, workspace, workspace_bytes);
}

int lsmx_gemm_bf16f4_noalloc(const void *a0, const void *a1, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                             const void *w_scale, int64_t ld_sw, int scale_fmt, void *c0, void *c1, int c_dtype,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream) {
    const char *fn = "lsmx_gemm_bf16f4_noalloc";
    if ((a1 == nullptr) != (c1 == nullptr)) return fail(LSMX_ERR_ARG, "%s: a1 and c1 go together", fn);
    // the split-K partial tiles this shape needs (0: whole-K kernels, no
    // scratch); w4_common validates everything else before any launch
    int64_t need = 0;
    if (M > 0 && N > 0 && K > 0 && K % 128 == 0 && M <= ((int64_t)1 << 30) && N <= ((int64_t)1 << 30))
        need = lsmx::gemm_bf16f4_workspace(M, N, K, a1 != nullptr);
    if (need > kScratchBytes)
        return fail(LSMX_ERR_SHAPE, "%s: this shape needs %lld bytes of split-K scratch; the fixed scratch holds %lld",
                    fn, (long long)need, (long long)kScratchBytes);
    void *ws = nullptr;
    if (need > 0) {
        if (int r = device_guard()) return r;
        if (int r = scratch_of(stream, &ws)) return r;
    }
    return w4_common(fn, a0, a1, LSMX_BF16, lda, w_pk, ldw, w_scale, ld_sw, scale_fmt, c0, c1, c_dtype, ldc, M, N, K,
                     stream, ws, ws ? kScratchBytes : 0);
}

int lsmx_gemm_wonly_f4(const void *a, int a_dtype, int64_t lda, const uint8_t *w_pk, int64_t ldw,
                       const void *w_scale, int64_t ld_sw, int scale_fmt, void *c, int c_dtype, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, void *stream) {
    return w4_common("lsmx_gemm_wonly_f4", a, nullptr, a_dtype, lda, w_pk, ldw, w_scale, ld_sw, scale_fmt, c, nullptr,
                     c_dtype, ldc, M, N, K, stream);
}

}  // extern "C"
