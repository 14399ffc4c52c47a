// rxq4_capi.hip -- the C ABI (include/rxq4.h) over the gfx950 launchers.
//
// Each entry point validates its arguments on the host, then enqueues on the
// caller's stream.  No entry point synchronises or falls back to the CPU: a
// call either launches the HIP kernels or returns a non-success status with
// the reason in rxq4_last_error().  The only allocation is the split
// launches' workspace, once per (device, stream) (runtime.cpp).
#include "rxq4.h"

#include <stdarg.h>

#include <atomic>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "launch.h"
#include "status.h"

namespace {
thread_local char g_last_error[256] = "";
}  // namespace

namespace rxq4 {

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int set_ok() {
    g_last_error[0] = '\0';
    return RXQ4_STATUS_SUCCESS;
}

}  // namespace rxq4

namespace {

using rxq4::set_error;

int ok() { return rxq4::set_ok(); }

int from_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return ok();
    if (e == hipErrorOutOfMemory)  // rxq4::Scratch::get, or the workspace allocation
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                         "%s: the fp32 split partials do not fit the scratch / workspace (%s)",
                         what, hipGetErrorString(e));
    return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: HIP error %s", what, hipGetErrorString(e));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool kquant_type(int t) { return t == RXQ4_GGML_TYPE_Q5_K || t == RXQ4_GGML_TYPE_Q6_K; }

// Weight alignment each format's kernels need: Q4_K / Q5_K blocks are read
// with 16-byte loads; Q6_K's 210-byte blocks are only 2-byte aligned in a
// tensor, and its kernels read every field with dword-aligned loads from the
// dword at or below the row and realign (so any row slice is accepted).
bool weights_aligned(const void *w, int ggml_type) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    return ggml_type == RXQ4_GGML_TYPE_Q6_K ? (a & 1u) == 0 : (a & 15u) == 0;
}

// Checks shared by every weight-streaming entry point.
int check_common(const char *fn, const void *w, int ggml_type, int K) {
    if (ggml_type != RXQ4_GGML_TYPE_Q4_K && !kquant_type(ggml_type))
        return set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT,
                    "%s: ggml_type %d not supported (Q4_K = 12, Q5_K = 13, Q6_K = 14)", fn,
                    ggml_type);
    if (K <= 0 || K % 256 != 0 || K > RXQ4_MAX_K)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                    "%s: K=%d must be a positive multiple of 256 and <= %d", fn, K, RXQ4_MAX_K);
    if (!w) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null weight pointer", fn);
    if (!weights_aligned(w, ggml_type))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                         "%s: weights must be %d-byte aligned for ggml_type %d", fn,
                         ggml_type == RXQ4_GGML_TYPE_Q6_K ? 2 : 16, ggml_type);
    return RXQ4_STATUS_SUCCESS;
}

// Last check before a launch (the only one that queries the HIP runtime).
int check_device(const char *fn) {
    if (!rxq4::device_info().arch_ok)
        return set_error(RXQ4_STATUS_UNSUPPORTED_DEVICE, "%s: current device is not gfx950", fn);
    return RXQ4_STATUS_SUCCESS;
}

int check_x(const char *fn, const void *x) {
    if (!x) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null x", fn);
    if (!aligned16(x)) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: x must be 16-byte aligned", fn);
    return RXQ4_STATUS_SUCCESS;
}

int gemv_single(const char *fn, void *y, const void *w, int ggml_type, const void *x,
                const void *residual, int M, int K, int epi, void *stream) {
    int s = check_common(fn, w, ggml_type, K);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if ((s = check_x(fn, x)) != RXQ4_STATUS_SUCCESS) return s;
    if (M < 0) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: M=%d < 0", fn, M);
    if (M == 0) return ok();
    if (!y) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null y", fn);
    if (epi == rxq4::kEpiAdd && !residual)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null residual", fn);
    if ((s = check_device(fn)) != RXQ4_STATUS_SUCCESS) return s;
    const rxq4::GemvRange range{static_cast<const uint8_t *>(w), y,
                                static_cast<const uint16_t *>(residual), M};
    if (kquant_type(ggml_type))
        return from_hip(rxq4::launch_kq_gemv(ggml_type, range, static_cast<const uint16_t *>(x),
                                             K, epi, static_cast<hipStream_t>(stream)),
                        fn);
    rxq4::GemvParams p{};
    p.r[0] = range;
    p.n_ranges = 1;
    p.total_rows = M;
    p.x = static_cast<const uint16_t *>(x);
    p.nb = K / 256;
    return from_hip(rxq4::launch_gemv(p, epi, static_cast<hipStream_t>(stream)), fn);
}

}  // namespace

extern "C" {

int rxq4_gemv_f16(void *y, const void *w, int ggml_type, const void *x, int M, int K,
                  void *stream) {
    return gemv_single("rxq4_gemv_f16", y, w, ggml_type, x, nullptr, M, K, rxq4::kEpiF16,
                       stream);
}

int rxq4_gemv_f32(float *y, const void *w, int ggml_type, const void *x, int M, int K,
                  void *stream) {
    return gemv_single("rxq4_gemv_f32", y, w, ggml_type, x, nullptr, M, K, rxq4::kEpiF32,
                       stream);
}

int rxq4_gemv_add_f16(void *y, const void *w, int ggml_type, const void *x,
                      const void *residual, int M, int K, void *stream) {
    return gemv_single("rxq4_gemv_add_f16", y, w, ggml_type, x, residual, M, K,
                       rxq4::kEpiAdd, stream);
}

int rxq4_gemv_multi_f16(const rxq4_rows *ranges, int n_ranges, const void *x, int K,
                        void *stream) {
    const char *fn = "rxq4_gemv_multi_f16";
    if (!ranges || n_ranges < 1 || n_ranges > 3)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: n_ranges=%d must be 1..3", fn, n_ranges);
    // All-Q4_K ranges take the Q4_K kernels; any Q5_K / Q6_K range makes the
    // whole call one mixed-type launch (as the reference's mixed Q4/Q4/Q6
    // triple, q4_gemm.cu:1157-1206).
    rxq4::GemvParams p{};
    rxq4::GemvRange kq[3];
    int kq_type[3];
    int n_live = 0;
    bool any_kq = false;
    int64_t total = 0;
    for (int i = 0; i < n_ranges; ++i) {
        const rxq4_rows &r = ranges[i];
        int s = check_common(fn, r.w, r.ggml_type, K);
        if (s != RXQ4_STATUS_SUCCESS) return s;
        if (r.M < 0) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: range %d M=%d < 0", fn, i, r.M);
        if (r.M > 0 && !r.y) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: range %d null y", fn, i);
        const rxq4::GemvRange g{static_cast<const uint8_t *>(r.w), r.y, nullptr, r.M};
        any_kq = any_kq || kquant_type(r.ggml_type);
        if (r.M > 0) {
            kq[n_live] = g;
            kq_type[n_live++] = r.ggml_type;
        }
        p.r[p.n_ranges++] = g;
        total += r.M;
    }
    int s = check_x(fn, x);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (total > 0x7FFFFFFF) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: too many rows", fn);
    if (total == 0) return ok();
    if ((s = check_device(fn)) != RXQ4_STATUS_SUCCESS) return s;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (any_kq) return from_hip(rxq4::launch_kq_multi(kq, kq_type, n_live, xx, K, st), fn);
    p.total_rows = (int)total;
    p.x = xx;
    p.nb = K / 256;
    return from_hip(rxq4::launch_gemv(p, rxq4::kEpiF16, st), fn);
}

}  // extern "C"

namespace {

// The GEMM routing shared by rxq4_gemm and rxq4_gemm_noalloc; split launches
// keep their partials in `sc`.
int gemm_impl(const char *fn, void *y, int y_dtype, const void *w, int ggml_type, const void *x,
              int x_dtype, int M, int N, int K, void *stream, const rxq4::Scratch &sc) {
    int s = check_common(fn, w, ggml_type, K);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if ((s = check_x(fn, x)) != RXQ4_STATUS_SUCCESS) return s;
    if (M < 0 || N < 0) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: M=%d N=%d", fn, M, N);
    if (M == 0 || N == 0) return ok();
    if (!y) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null y", fn);
    const bool f16_ok = x_dtype == RXQ4_DTYPE_F16 &&
                        (y_dtype == RXQ4_DTYPE_F16 || y_dtype == RXQ4_DTYPE_F32);
    const bool bf16_ok = x_dtype == RXQ4_DTYPE_BF16 &&
                         (y_dtype == RXQ4_DTYPE_BF16 || y_dtype == RXQ4_DTYPE_F32);
    if (!f16_ok && !bf16_ok)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: unsupported dtypes x=%d y=%d", fn,
                    x_dtype, y_dtype);
    if ((s = check_device(fn)) != RXQ4_STATUS_SUCCESS) return s;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (N == 1 && x_dtype == RXQ4_DTYPE_F16) {
        // One token is the decode GEMV (reference q4_gemm.cu:1714-1717).
        return gemv_single(fn, y, w, ggml_type, x, nullptr, M, K,
                           y_dtype == RXQ4_DTYPE_F32 ? rxq4::kEpiF32 : rxq4::kEpiF16, stream);
    }
    hipError_t e;
    if (kquant_type(ggml_type) && N <= rxq4::kMaxSmallBatch)
        e = rxq4::launch_kq_tokens(ggml_type, y, y_dtype, static_cast<const uint8_t *>(w), x,
                                   x_dtype, M, N, K, st);
    else if (kquant_type(ggml_type))
        e = rxq4::launch_gemm(ggml_type, y, y_dtype, static_cast<const uint8_t *>(w), x, x_dtype,
                              M, N, K, st, sc);
    else if (N <= rxq4::kMaxRegTokens && x_dtype == RXQ4_DTYPE_F16 &&
             (rxq4::tuning().multi_token_gemv > 0 ||
              (rxq4::tuning().multi_token_gemv < 0 && rxq4::gemv_multi_token_preferred(N, M, K))) &&
             rxq4::gemv_multi_token_fits(N, K))
        // 2 (or 3) fp16 tokens: the decode GEMV with every token's activations
        // in registers (one weight read, the nibble decode shared by the tokens)
        e = rxq4::launch_gemv_multi_token(y, y_dtype, static_cast<const uint8_t *>(w),
                                          static_cast<const uint16_t *>(x), M, N, K, st);
    else if (N <= rxq4::kMaxSmallBatch)
        e = rxq4::launch_gemv_tokens(y, y_dtype, static_cast<const uint8_t *>(w), x, x_dtype, M,
                                     N, K, st, sc);
    else
        e = rxq4::launch_gemm(12, y, y_dtype, static_cast<const uint8_t *>(w), x, x_dtype, M, N, K,
                              st, sc);
    return from_hip(e, fn);
}

}  // namespace

extern "C" {

int rxq4_gemm(void *y, int y_dtype, const void *w, int ggml_type, const void *x, int x_dtype,
              int M, int N, int K, void *stream) {
    return gemm_impl("rxq4_gemm", y, y_dtype, w, ggml_type, x, x_dtype, M, N, K, stream,
                     rxq4::Scratch{});
}

}  // extern "C"

// ------------------------------------------------------ rxq4_gemm_noalloc
// The split partials of rxq4_gemm_noalloc live in this file-scope array:
// each device holds its own copy (kNoAllocScratchBytes), made when the HIP
// runtime loads this file's code object on it (at the first
// hipGetSymbolAddress below) and held until the process ends.  Host code
// never uses the array's name as an address: the device address is taken
// once per device with hipGetSymbolAddress and kept in g_scratch_addr.
namespace {

constexpr size_t kNoAllocScratchBytes = rxq4::kWorkspaceBytes;  // 48 MiB
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];
std::atomic<float *> g_scratch_addr[kMaxDevices];

hipError_t scratch_address(float **p) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    float *a = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (!a) {
        // The first call may come while the caller's stream is being captured
        // (the entry point is for graph capture): the lookup is not part of
        // any graph, so it runs with this thread's capture mode relaxed.
        void *q = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        if ((e = hipThreadExchangeStreamCaptureMode(&mode)) != hipSuccess) return e;
        e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
        hipStreamCaptureMode back = mode;
        (void)hipThreadExchangeStreamCaptureMode(&back);
        if (e != hipSuccess) return e;
        a = static_cast<float *>(q);
        g_scratch_addr[dev].store(a, std::memory_order_release);
    }
    *p = a;
    return hipSuccess;
}

}  // namespace

extern "C" {

int rxq4_gemm_noalloc(void *y, int y_dtype, const void *w, int ggml_type, const void *x,
                      int x_dtype, int M, int N, int K, void *stream) {
    const char *fn = "rxq4_gemm_noalloc";
    float *sp = nullptr;
    const hipError_t e = scratch_address(&sp);
    if (e != hipSuccess) return from_hip(e, fn);
    return gemm_impl(fn, y, y_dtype, w, ggml_type, x, x_dtype, M, N, K, stream,
                     rxq4::Scratch{sp, kNoAllocScratchBytes});
}

int rxq4_gemm_f16(void *y, const void *w, int ggml_type, const void *x, int M, int N, int K,
                  void *stream) {
    return rxq4_gemm(y, RXQ4_DTYPE_F16, w, ggml_type, x, RXQ4_DTYPE_F16, M, N, K, stream);
}

int rxq4_embed_row_f16(void *dst, const void *w, int ggml_type, int token_id, int hidden_dim,
                       void *stream) {
    const char *fn = "rxq4_embed_row_f16";
    // Order of checks as the reference (q4_gemm.cu:2079-2105): shape first,
    // then the weight pointer, then the type.
    if (hidden_dim <= 0 || hidden_dim % 256 != 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: hidden_dim=%d", fn, hidden_dim);
    if (!w) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null weights", fn);
    // Q4_K and Q6_K, as the reference (q4_gemm.cu:2089-2106).
    if (ggml_type != RXQ4_GGML_TYPE_Q4_K && ggml_type != RXQ4_GGML_TYPE_Q6_K)
        return set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT, "%s: ggml_type %d", fn, ggml_type);
    if (!weights_aligned(w, ggml_type) || !dst || !aligned16(dst))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                         "%s: misaligned weights (Q4_K 16 bytes, Q6_K 2) or dst (16 bytes)", fn);
    if (!rxq4::device_info().arch_ok)
        return set_error(RXQ4_STATUS_UNSUPPORTED_DEVICE, "%s: current device is not gfx950", fn);
    const auto launch = ggml_type == RXQ4_GGML_TYPE_Q6_K ? rxq4::launch_kq_embed : rxq4::launch_embed;
    return from_hip(launch(static_cast<uint16_t *>(dst), static_cast<const uint8_t *>(w), nullptr,
                           token_id, 0, 1, hidden_dim, static_cast<hipStream_t>(stream)),
                    fn);
}

int rxq4_embed_rows_f16(void *dst, const void *w, int ggml_type, int64_t n_vocab,
                        const int32_t *ids, int n_ids, int hidden_dim, void *stream) {
    const char *fn = "rxq4_embed_rows_f16";
    if (hidden_dim <= 0 || hidden_dim % 256 != 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: hidden_dim=%d", fn, hidden_dim);
    if (!w) return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null weights", fn);
    if (ggml_type != RXQ4_GGML_TYPE_Q4_K && ggml_type != RXQ4_GGML_TYPE_Q6_K)
        return set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT, "%s: ggml_type %d", fn, ggml_type);
    if (n_ids < 0 || n_vocab < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: n_ids=%d n_vocab=%lld", fn, n_ids,
                    (long long)n_vocab);
    if (n_ids == 0) return ok();
    if (!ids || !dst || !weights_aligned(w, ggml_type) || !aligned16(dst))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null/misaligned pointer", fn);
    if (!rxq4::device_info().arch_ok)
        return set_error(RXQ4_STATUS_UNSUPPORTED_DEVICE, "%s: current device is not gfx950", fn);
    const auto launch = ggml_type == RXQ4_GGML_TYPE_Q6_K ? rxq4::launch_kq_embed : rxq4::launch_embed;
    return from_hip(launch(static_cast<uint16_t *>(dst), static_cast<const uint8_t *>(w), ids, 0,
                           n_vocab, n_ids, hidden_dim, static_cast<hipStream_t>(stream)),
                    fn);
}

int rxq4_quantize_q4k(void *dst, const float *src, int64_t n_rows, int K, void *stream) {
    const char *fn = "rxq4_quantize_q4k";
    if (K <= 0 || K % 256 != 0 || n_rows < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: K=%d n_rows=%lld", fn, K,
                    (long long)n_rows);
    if (n_rows == 0) return ok();
    if (!dst || !src || !aligned16(dst) || !aligned16(src))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null/misaligned pointer", fn);
    if (!rxq4::device_info().arch_ok)
        return set_error(RXQ4_STATUS_UNSUPPORTED_DEVICE, "%s: current device is not gfx950", fn);
    return from_hip(rxq4::launch_quantize(static_cast<uint8_t *>(dst), src, n_rows * (K / 256),
                                          static_cast<hipStream_t>(stream)),
                    fn);
}

int rxq4_quantize(void *dst, int ggml_type, const float *src, int64_t n_rows, int K,
                  void *stream) {
    const char *fn = "rxq4_quantize";
    if (ggml_type != RXQ4_GGML_TYPE_Q4_K && !kquant_type(ggml_type))
        return set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT,
                         "%s: ggml_type %d not supported (Q4_K = 12, Q5_K = 13, Q6_K = 14)", fn,
                         ggml_type);
    if (K <= 0 || K % 256 != 0 || n_rows < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: K=%d n_rows=%lld", fn, K,
                         (long long)n_rows);
    if (n_rows == 0) return ok();
    if (!dst || !src || !aligned16(src))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null or misaligned src", fn);
    const uintptr_t need = ggml_type == RXQ4_GGML_TYPE_Q6_K ? 1u : 15u;
    if ((reinterpret_cast<uintptr_t>(dst) & need) != 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: dst must be %d-byte aligned", fn,
                         (int)need + 1);
    if (n_rows > INT64_MAX / (K / 256))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: too many rows", fn);
    if (!rxq4::device_info().arch_ok)
        return set_error(RXQ4_STATUS_UNSUPPORTED_DEVICE, "%s: current device is not gfx950", fn);
    return from_hip(rxq4::launch_quantize_ggml(ggml_type, static_cast<uint8_t *>(dst), src,
                                               n_rows * (K / 256), static_cast<hipStream_t>(stream)),
                    fn);
}

}  // extern "C"

namespace {

int attention(const char *fn, void *out, const void *q, const void *k, const void *v,
              int n_heads, int n_kv, int head_dim, int n_tok, int seq0, float scale, int kv_int8,
              const float *ks, const float *vs, void *stream) {
    if (n_heads == 0 || n_tok == 0) return ok();
    if (n_heads < 0 || n_kv <= 0 || n_heads % n_kv != 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                    "%s: n_heads=%d must be a positive multiple of n_kv_heads=%d", fn, n_heads,
                    n_kv);
    const int align = kv_int8 ? 16 : 8;
    if (head_dim <= 0 || head_dim > 256 || head_dim % align != 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                    "%s: head_dim=%d must be a multiple of %d and <= 256", fn, head_dim, align);
    if (n_tok < 0 || seq0 < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: negative length", fn);
    if (!out || !q || !aligned16(out) || !aligned16(q))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: q/out null or not 16-byte aligned", fn);
    if (seq0 + n_tok - 1 > 0 && (!k || !v || !aligned16(k) || !aligned16(v)))
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: k/v null or not 16-byte aligned", fn);
    int s = check_device(fn);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    return from_hip(rxq4::launch_attention(static_cast<uint16_t *>(out),
                                           static_cast<const uint16_t *>(q), k, v,
                                           kv_int8 ? ks : nullptr, kv_int8 ? vs : nullptr, n_heads,
                                           n_kv, head_dim, n_tok, seq0, scale, kv_int8 ? 1 : 0,
                                           static_cast<hipStream_t>(stream)),
                    fn);
}

}  // namespace

extern "C" {

int rxq4_attention_decode_f16(void *out, const void *q, const void *k_cache,
                              const void *v_cache, int n_heads, int n_kv_heads, int head_dim,
                              int seq_len, float scale, int kv_int8, const float *k_scales,
                              const float *v_scales, void *stream) {
    if (seq_len < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "rxq4_attention_decode_f16: seq_len=%d",
                    seq_len);
    return attention("rxq4_attention_decode_f16", out, q, k_cache, v_cache, n_heads, n_kv_heads,
                     head_dim, 1, seq_len, scale, kv_int8, k_scales, v_scales, stream);
}

int rxq4_attention_prefill_f16(void *out, const void *q, const void *k_cache,
                               const void *v_cache, int n_heads, int n_kv_heads, int head_dim,
                               int N, int start_pos, float scale, int kv_int8,
                               const float *k_scales, const float *v_scales, void *stream) {
    if (N < 0 || start_pos < 0)
        return set_error(RXQ4_STATUS_INVALID_ARGUMENT, "rxq4_attention_prefill_f16: N=%d start_pos=%d",
                    N, start_pos);
    return attention("rxq4_attention_prefill_f16", out, q, k_cache, v_cache, n_heads, n_kv_heads,
                     head_dim, N, start_pos + 1, scale, kv_int8, k_scales, v_scales, stream);
}

const void *rxq4_resolve_weights(const void *w, const void *w_device) {
    if (w_device) return w_device;
    if (!w) return nullptr;
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof(attr));
    if (hipPointerGetAttributes(&attr, w) != hipSuccess) {
        (void)hipGetLastError();  // ordinary host pointers report an error here
        return nullptr;
    }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) return w;
    return nullptr;
}

int rxq4_reserve_workspace(void *stream) {
    float *ws = nullptr;
    return from_hip(rxq4::stream_workspace(static_cast<hipStream_t>(stream), &ws),
                    "rxq4_reserve_workspace");
}

int rxq4_release_workspace(void *stream) {
    int released = 0;
    return from_hip(rxq4::release_stream_workspace(static_cast<hipStream_t>(stream), &released),
                    "rxq4_release_workspace");
}

const char *rxq4_version(void) { return "rxq4 0.1.0 gfx950"; }

const char *rxq4_last_error(void) { return g_last_error; }

}  // extern "C"
