// seam.cpp -- reflex::infer::kernels::* over the C ABI of include/rxq4.h.
//
// Mirrors the host layer of the reference (src/kernels/q4_gemm.cu:1707-2115):
// resolve each weight pointer (the `weights_device` alias wins, else the
// runtime's pointer attributes; q4_gemm.cu:111-135), then launch on the
// caller's stream.
//
// Host path, as the reference's (q4_gemm.cu:1886-1899, 1916-1947, 1963-1966,
// 1986-1991, 1994-2016, 1735-1739): when a weight pointer resolves to no
// GPU-visible address, or JLLM_FAST_GEMV=0, the GEMV family computes on the
// CPU (rxq4_host_gemv): wait for the stream, copy x (and the residual) to
// the host, compute, copy y back.  Pair and triple take the host path per
// range, the batched GEMM per token.  It is reached only through these two
// conditions: a GPU launch that fails returns its status, it never falls back
// to the host.
//
// Other differences, all deliberate:
//   * ggml types other than Q4_K/Q5_K/Q6_K (12/13/14) return
//     UnsupportedQuantFormat, where the reference zero-fills y;
//   * K must be a multiple of 256 (the reference assumes it silently);
//   * the CUDA variant switches (JLLM_Q4K_UINT32_LOADS, JLLM_MMQ_Q4K,
//     JLLM_GEMV_ROWS) have no meaning here and are ignored.
// JLLM_DEBUG_KERNELS (non-zero) prints the first outputs and inputs of the
// first three gemv_quant calls after synchronising the stream, as the
// reference (q4_gemm.cu:47-53, 1863-1881, 1901-1912); calls made while the
// stream is being captured are not synchronised and print nothing.
#include "seam.h"

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "rxq4.h"
#include "status.h"

namespace reflex::infer::kernels {
namespace {

Status to_status(int s) { return static_cast<Status>(s); }

bool fast_gemv() {
    static const bool on = [] {
        const char* v = std::getenv("JLLM_FAST_GEMV");
        return !v || std::strcmp(v, "0") != 0;
    }();
    return on;
}

bool debug_kernels() {
    static const bool on = [] {
        const char* v = std::getenv("JLLM_DEBUG_KERNELS");
        return v && std::strcmp(v, "0") != 0;
    }();
    return on;
}

void warn_once(std::atomic<bool>& flag, const char* what) {
    if (!flag.exchange(true, std::memory_order_relaxed)) std::fprintf(stderr, "%s\n", what);
}

Status finish(int s, const char* who) {
    if (s != RXQ4_STATUS_SUCCESS) {
        static std::atomic<int> reported{0};
        if (reported.fetch_add(1, std::memory_order_relaxed) < 8)
            std::fprintf(stderr, "[rxq4] %s failed: %s\n", who, rxq4_last_error());
    }
    return to_status(s);
}

// The pointer the kernels read, or nullptr when the host path must run
// (no GPU-visible address, or the GPU GEMV switched off).
const void* gpu_weights(const void* w, const void* w_device) {
    if (!fast_gemv()) return nullptr;
    return rxq4_resolve_weights(w, w_device);
}

bool capturing(void* stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return cs != hipStreamCaptureStatusNone;
}

// The host path of one GEMV (y fp16 or fp32, optional fp16 residual).
int host_gemv(void* y, int y_dtype, const void* w, int type, const void* x,
              const void* residual, int M, int K, void* stream) {
    static std::atomic<bool> noted{false};
    warn_once(noted, fast_gemv()
                         ? "[rxq4] weights not GPU-visible (host memory, no weights_device "
                           "alias): computing the GEMV on the CPU"
                         : "[rxq4] JLLM_FAST_GEMV=0: computing the GEMV family on the CPU");
    if (M <= 0) return RXQ4_STATUS_SUCCESS;
    // validate before touching the stream or copying (M = 0 checks the rest)
    int s = rxq4_host_gemv(nullptr, y_dtype, w, type, nullptr, nullptr, 0, K);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    const char* fn = "host GEMV";
    if (!y || !x || !w) return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (capturing(stream))
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                               "%s: cannot run while the stream is being captured", fn);
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    if (hipPointerGetAttributes(&attr, w) == hipSuccess) {
        if (attr.type == hipMemoryTypeDevice)
            return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                                   "%s: weights are device memory, not readable on the host", fn);
    } else {
        (void)hipGetLastError();  // ordinary host memory reports an error here
    }
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    std::vector<uint16_t> hx(K), hres(residual ? M : 0);
    const size_t ybytes = (size_t)M * (y_dtype == RXQ4_DTYPE_F32 ? 4 : 2);
    std::vector<unsigned char> hy(ybytes);
    if (e == hipSuccess) e = hipMemcpy(hx.data(), x, (size_t)K * 2, hipMemcpyDefault);
    if (e == hipSuccess && residual) e = hipMemcpy(hres.data(), residual, (size_t)M * 2, hipMemcpyDefault);
    if (e != hipSuccess)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: %s", fn, hipGetErrorString(e));
    s = rxq4_host_gemv(hy.data(), y_dtype, w, type, hx.data(), residual ? hres.data() : nullptr,
                       M, K);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if ((e = hipMemcpy(y, hy.data(), ybytes, hipMemcpyDefault)) != hipSuccess)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: %s", fn, hipGetErrorString(e));
    return RXQ4_STATUS_SUCCESS;
}

float half_bits_to_float(uint16_t h) {
    // exact; only for the debug print
    const int e = (h >> 10) & 31, m = h & 1023;
    float v = e == 0 ? std::ldexp((float)m, -24)
              : e == 31 ? (m ? NAN : INFINITY)
                        : std::ldexp((float)(m + 1024), e - 25);
    return (h & 0x8000) ? -v : v;
}

// JLLM_DEBUG_KERNELS: first outputs and inputs of the first three calls.
void debug_print(const char* tag, const GemvQuantArgs& a) {
    static std::atomic<int> count{0};
    if (!debug_kernels() || a.M <= 0 || capturing(a.stream)) return;
    const int n = count.fetch_add(1, std::memory_order_relaxed);
    if (n >= 3) return;
    if (hipStreamSynchronize(static_cast<hipStream_t>(a.stream)) != hipSuccess) {
        std::fprintf(stderr, "[%s #%d] execution failed: %s\n", tag, n,
                     hipGetErrorString(hipGetLastError()));
        return;
    }
    uint16_t hy[8] = {}, hx[8] = {};
    const int ny = a.M < 8 ? a.M : 8, nx = a.K < 8 ? a.K : 8;
    if (hipMemcpy(hy, a.y, ny * 2, hipMemcpyDefault) != hipSuccess ||
        hipMemcpy(hx, a.x, nx * 2, hipMemcpyDefault) != hipSuccess)
        return;
    std::fprintf(stderr, "[%s #%d] type=%d M=%d K=%d out: ", tag, n, a.ggml_type, a.M, a.K);
    for (int i = 0; i < ny; ++i) std::fprintf(stderr, "%.4f ", half_bits_to_float(hy[i]));
    std::fprintf(stderr, " | in: ");
    for (int i = 0; i < nx; ++i) std::fprintf(stderr, "%.4f ", half_bits_to_float(hx[i]));
    std::fprintf(stderr, "\n");
}

}  // namespace

Status gemv_quant(const GemvQuantArgs& a) {
    const void* w = gpu_weights(a.weights, a.weights_device);
    Status s;
    if (w || a.M <= 0) {
        s = finish(rxq4_gemv_f16(a.y, w, a.ggml_type, a.x, a.M, a.K, a.stream), "gemv_quant");
        if (s == Status::Success) debug_print("GEMV-GPU", a);
    } else {
        s = finish(host_gemv(a.y, RXQ4_DTYPE_F16, a.weights, a.ggml_type, a.x, nullptr, a.M, a.K,
                             a.stream),
                   "gemv_quant");
        if (s == Status::Success) debug_print("GEMV", a);
    }
    return s;
}

Status gemv_quant_add(const GemvQuantAddArgs& a) {
    const void* w = gpu_weights(a.weights, a.weights_device);
    if (w || a.M <= 0)
        return finish(rxq4_gemv_add_f16(a.y, w, a.ggml_type, a.x, a.residual, a.M, a.K, a.stream),
                      "gemv_quant_add");
    return finish(host_gemv(a.y, RXQ4_DTYPE_F16, a.weights, a.ggml_type, a.x, a.residual, a.M,
                            a.K, a.stream),
                  "gemv_quant_add");
}

namespace {

// Pair / triple: one launch when every range is GPU-visible, else range by
// range (GPU ranges as single GEMVs, the rest on the host), as the
// reference's per-range fallback (q4_gemm.cu:1963-1966, 1986-1991).
Status gemv_multi(const rxq4_rows* host, const void* const* dev_alias, int n, const void* x,
                  int K, void* stream, const char* who) {
    rxq4_rows r[3];
    bool all_gpu = true;
    for (int i = 0; i < n; ++i) {
        r[i] = host[i];
        r[i].w = gpu_weights(host[i].w, dev_alias[i]);
        if (!r[i].w && r[i].M > 0) all_gpu = false;
    }
    if (all_gpu) return finish(rxq4_gemv_multi_f16(r, n, x, K, stream), who);
    for (int i = 0; i < n; ++i) {
        int s;
        if (r[i].w || r[i].M <= 0)
            s = rxq4_gemv_f16(r[i].y, r[i].w, r[i].ggml_type, x, r[i].M, K, stream);
        else
            s = host_gemv(r[i].y, RXQ4_DTYPE_F16, host[i].w, host[i].ggml_type, x, nullptr,
                          host[i].M, K, stream);
        if (s != RXQ4_STATUS_SUCCESS) return finish(s, who);
    }
    return Status::Success;
}

}  // namespace

Status gemv_quant_pair(const GemvQuantPairArgs& a) {
    const rxq4_rows r[2] = {{a.y0, a.weights0, a.ggml_type0, a.M0},
                            {a.y1, a.weights1, a.ggml_type1, a.M1}};
    const void* alias[2] = {a.weights0_device, a.weights1_device};
    return gemv_multi(r, alias, 2, a.x, a.K, a.stream, "gemv_quant_pair");
}

Status gemv_quant_triple(const GemvQuantTripleArgs& a) {
    const rxq4_rows r[3] = {{a.y0, a.weights0, a.ggml_type0, a.M0},
                            {a.y1, a.weights1, a.ggml_type1, a.M1},
                            {a.y2, a.weights2, a.ggml_type2, a.M2}};
    const void* alias[3] = {a.weights0_device, a.weights1_device, a.weights2_device};
    return gemv_multi(r, alias, 3, a.x, a.K, a.stream, "gemv_quant_triple");
}

Status gemm_quant_batched(const GemmQuantBatchedArgs& a) {
    // Empty shapes are a no-op (reference q4_gemm.cu:1713).
    if (a.N <= 0 || a.M <= 0 || a.K <= 0) return Status::Success;
    if (a.N == 1) {  // the decode GEMV (q4_gemm.cu:1714-1717)
        GemvQuantArgs g{};
        g.y = a.y;
        g.weights = a.weights;
        g.weights_device = a.weights_device;
        g.ggml_type = a.ggml_type;
        g.x = a.x;
        g.M = a.M;
        g.K = a.K;
        g.stream = a.stream;
        return kernels::gemv_quant(g);
    }
    const void* w = gpu_weights(a.weights, a.weights_device);
    if (w)
        return finish(rxq4_gemm_f16(a.y, w, a.ggml_type, a.x, a.M, a.N, a.K, a.stream),
                      "gemm_quant_batched");
    // per-token host GEMVs (q4_gemm.cu:1735-1739)
    for (int t = 0; t < a.N; ++t) {
        const int s = host_gemv(static_cast<uint16_t*>(a.y) + (size_t)t * a.M, RXQ4_DTYPE_F16,
                                a.weights, a.ggml_type,
                                static_cast<const uint16_t*>(a.x) + (size_t)t * a.K, nullptr, a.M,
                                a.K, a.stream);
        if (s != RXQ4_STATUS_SUCCESS) return finish(s, "gemm_quant_batched");
    }
    return Status::Success;
}

Status gemv_quant_f32(const GemvQuantF32Args& a) {
    const void* w = gpu_weights(a.weights, a.weights_device);
    if (w || a.M <= 0)
        return finish(rxq4_gemv_f32(a.y, w, a.ggml_type, a.x, a.M, a.K, a.stream),
                      "gemv_quant_f32");
    return finish(host_gemv(a.y, RXQ4_DTYPE_F32, a.weights, a.ggml_type, a.x, nullptr, a.M, a.K,
                            a.stream),
                  "gemv_quant_f32");
}

Status dequant_embedding_row(const DequantEmbeddingRowArgs& a) {
    // Check order of the reference (q4_gemm.cu:2079-2105); host-only tables
    // are InvalidArgument there too (no CPU embedding path).
    if (a.hidden_dim <= 0 || a.hidden_dim % 256 != 0) return Status::InvalidArgument;
    const void* w = rxq4_resolve_weights(a.weights, a.weights_device);
    if (!w) return Status::InvalidArgument;
    return finish(rxq4_embed_row_f16(a.dst, w, a.ggml_type, a.token_id, a.hidden_dim, a.stream),
                  "dequant_embedding_row");
}

// Attention (reference attention.cu:432-466): the caches and q are device
// pointers; no pointer resolution.
Status flash_attention_decode(const AttentionDecodeArgs& a) {
    return finish(rxq4_attention_decode_f16(a.output, a.q, a.k_cache, a.v_cache, a.n_heads,
                                            a.n_kv_heads, a.head_dim, a.seq_len, a.scale,
                                            a.kv_int8 ? 1 : 0, a.k_scales, a.v_scales, a.stream),
                  "flash_attention_decode");
}

Status flash_attention_prefill_batched(const AttentionPrefillBatchedArgs& a) {
    return finish(rxq4_attention_prefill_f16(a.output, a.q, a.k_cache, a.v_cache, a.n_heads,
                                             a.n_kv_heads, a.head_dim, a.N, a.start_pos, a.scale,
                                             a.kv_int8 ? 1 : 0, a.k_scales, a.v_scales, a.stream),
                  "flash_attention_prefill_batched");
}

}  // namespace reflex::infer::kernels
