// seam.cpp -- reflex::infer::kernels::* over the C ABI of include/rxq4.h.
//
// Mirrors the host layer of the reference (src/kernels/q4_gemm.cu:1707-2115):
// resolve each weight pointer (the `weights_device` alias wins, else the
// runtime's pointer attributes; q4_gemm.cu:111-135), then launch on the
// caller's stream.  Differences, all deliberate and in the direction of
// failing loudly instead of computing on the host:
//   * there is no CPU fallback: host-only weights (no GPU-visible alias) and
//     launch errors return InvalidArgument with a one-time stderr message,
//     where the reference would run gemv_quant_cpu;
//   * ggml types other than Q4_K/Q5_K/Q6_K (12/13/14) return
//     UnsupportedQuantFormat, where the reference zero-fills y;
//   * K must be a multiple of 256 (the reference assumes it silently);
//   * JLLM_FAST_GEMV=0, which selects the reference's CPU path, is reported
//     once and ignored; the CUDA variant switches (JLLM_Q4K_UINT32_LOADS,
//     JLLM_MMQ_Q4K, JLLM_GEMV_ROWS) have no meaning here and are ignored.
#include "seam.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "rxq4.h"

namespace reflex::infer::kernels {
namespace {

Status to_status(int s) { return static_cast<Status>(s); }

void warn_once(std::atomic<bool>& flag, const char* what) {
    if (!flag.exchange(true, std::memory_order_relaxed)) std::fprintf(stderr, "%s\n", what);
}

void note_fast_gemv_flag() {
    static std::atomic<bool> noted{false};
    const char* v = std::getenv("JLLM_FAST_GEMV");
    if (v && std::strcmp(v, "0") == 0)
        warn_once(noted,
                  "[rxq4] JLLM_FAST_GEMV=0 ignored: the MI355X build has no CPU GEMV path");
}

const void* resolve_or_warn(const void* w, const void* w_device, const char* who) {
    const void* dev = rxq4_resolve_weights(w, w_device);
    if (!dev && w) {
        static std::atomic<bool> warned{false};
        (void)who;
        warn_once(warned,
                  "[rxq4] GPU-visible weight pointer unavailable (host-only memory and no "
                  "weights_device alias); returning InvalidArgument");
    }
    return dev;
}

Status finish(int s, const char* who) {
    if (s != RXQ4_STATUS_SUCCESS) {
        static std::atomic<int> reported{0};
        if (reported.fetch_add(1, std::memory_order_relaxed) < 8)
            std::fprintf(stderr, "[rxq4] %s failed: %s\n", who, rxq4_last_error());
    }
    return to_status(s);
}

}  // namespace

Status gemv_quant(const GemvQuantArgs& a) {
    note_fast_gemv_flag();
    const void* w = resolve_or_warn(a.weights, a.weights_device, "gemv_quant");
    if (!w && a.M > 0) return Status::InvalidArgument;
    return finish(rxq4_gemv_f16(a.y, w, a.ggml_type, a.x, a.M, a.K, a.stream), "gemv_quant");
}

Status gemv_quant_add(const GemvQuantAddArgs& a) {
    note_fast_gemv_flag();
    const void* w = resolve_or_warn(a.weights, a.weights_device, "gemv_quant_add");
    if (!w && a.M > 0) return Status::InvalidArgument;
    return finish(rxq4_gemv_add_f16(a.y, w, a.ggml_type, a.x, a.residual, a.M, a.K, a.stream),
                  "gemv_quant_add");
}

Status gemv_quant_pair(const GemvQuantPairArgs& a) {
    note_fast_gemv_flag();
    rxq4_rows r[2] = {
        {a.y0, resolve_or_warn(a.weights0, a.weights0_device, "gemv_quant_pair"), a.ggml_type0,
         a.M0},
        {a.y1, resolve_or_warn(a.weights1, a.weights1_device, "gemv_quant_pair"), a.ggml_type1,
         a.M1},
    };
    for (const auto& x : r)
        if (!x.w && x.M > 0) return Status::InvalidArgument;
    return finish(rxq4_gemv_multi_f16(r, 2, a.x, a.K, a.stream), "gemv_quant_pair");
}

Status gemv_quant_triple(const GemvQuantTripleArgs& a) {
    note_fast_gemv_flag();
    rxq4_rows r[3] = {
        {a.y0, resolve_or_warn(a.weights0, a.weights0_device, "gemv_quant_triple"),
         a.ggml_type0, a.M0},
        {a.y1, resolve_or_warn(a.weights1, a.weights1_device, "gemv_quant_triple"),
         a.ggml_type1, a.M1},
        {a.y2, resolve_or_warn(a.weights2, a.weights2_device, "gemv_quant_triple"),
         a.ggml_type2, a.M2},
    };
    for (const auto& x : r)
        if (!x.w && x.M > 0) return Status::InvalidArgument;
    return finish(rxq4_gemv_multi_f16(r, 3, a.x, a.K, a.stream), "gemv_quant_triple");
}

Status gemm_quant_batched(const GemmQuantBatchedArgs& a) {
    // Empty shapes are a no-op (reference q4_gemm.cu:1713).
    if (a.N <= 0 || a.M <= 0 || a.K <= 0) return Status::Success;
    note_fast_gemv_flag();
    const void* w = resolve_or_warn(a.weights, a.weights_device, "gemm_quant_batched");
    if (!w) return Status::InvalidArgument;
    return finish(rxq4_gemm_f16(a.y, w, a.ggml_type, a.x, a.M, a.N, a.K, a.stream),
                  "gemm_quant_batched");
}

Status gemv_quant_f32(const GemvQuantF32Args& a) {
    note_fast_gemv_flag();
    const void* w = resolve_or_warn(a.weights, a.weights_device, "gemv_quant_f32");
    if (!w && a.M > 0) return Status::InvalidArgument;
    return finish(rxq4_gemv_f32(a.y, w, a.ggml_type, a.x, a.M, a.K, a.stream), "gemv_quant_f32");
}

Status dequant_embedding_row(const DequantEmbeddingRowArgs& a) {
    // Check order of the reference (q4_gemm.cu:2079-2105).
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
