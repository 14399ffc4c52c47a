/*
 * rxq4.h -- C ABI of the MI355X (gfx950) Q4_K weight-path library.
 *
 * Plain C: pointers, sizes and int status codes, no C++ or torch types.  The
 * first seven entry points replace, one for one, the kernel-layer functions
 * that reflex-infer's dispatcher binds (reference
 * src/kernels/kernel_entrypoints.h:7-13, defined in src/kernels/q4_gemm.cu);
 * the C++ API of include/reflex/infer.h is implemented on top of them.  The
 * entry points marked NEW have no reference counterpart: they expose work
 * the reference API cannot express (bf16 GEMM, batched embedding gather,
 * small-batch decode, the quantiser used to build inputs).
 *
 * Conventions for every entry point:
 *   - `w` is a DEVICE pointer to raw GGML blocks of `ggml_type`: Q4_K (12,
 *     144 bytes per 256 weights), Q5_K (13, 176 bytes) or Q6_K (14, 210
 *     bytes); rows of K/256 blocks, row-major, the base 16-byte aligned.
 *     The embedding entry points take Q4_K and Q6_K, as the reference.
 *     Pointer resolution of host/mmap pointers happens above this layer
 *     (rxq4_resolve_weights).
 *   - fp16/bf16 buffers are raw 16-bit patterns; x must be 16-byte aligned.
 *   - K must be a positive multiple of 256 and at most RXQ4_MAX_K.
 *   - `stream` is a hipStream_t (NULL = null stream).  Calls only enqueue
 *     work; no entry point but rxq4_release_workspace synchronises the
 *     device or the stream.  The one allocation is the fp32 workspace of the
 *     split launches (split-K GEMM with few output tiles, small-batch
 *     products on long rows, decode attention over long sequences): 48 MiB
 *     per (device, stream), made by the first such launch on that stream,
 *     never resized, and kept until rxq4_release_workspace(stream) frees it,
 *     so a HIP graph captured on a stream stays valid whatever runs later,
 *     and launches on different streams never share it.  hipStreamPerThread
 *     names a different stream in every thread, so its workspace is kept per
 *     (device, thread).  That first allocation is also legal while the
 *     stream is being captured.
 *   - x must be 16-byte aligned (the one alignment rule the reference does
 *     not have).  Weight blocks need the alignment of their format: Q4_K
 *     and Q5_K 16 bytes, Q6_K 2 bytes (its 210-byte blocks; a row slice of a
 *     Q6_K tensor is accepted wherever it starts).
 *   - The return value is a reflex::infer::Status value (RXQ4_STATUS_*).
 *     On an error nothing is launched; rxq4_last_error() says why.
 */
#ifndef RXQ4_H
#define RXQ4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Values of reflex::infer::Status (reference include/reflex/infer.h:16-23). */
#define RXQ4_STATUS_SUCCESS 0
#define RXQ4_STATUS_UNSUPPORTED_DEVICE 1
#define RXQ4_STATUS_UNSUPPORTED_MODEL 2
#define RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT 3
#define RXQ4_STATUS_INVALID_ARGUMENT 4
#define RXQ4_STATUS_NOT_IMPLEMENTED 5

#define RXQ4_GGML_TYPE_Q4_K 12
#define RXQ4_GGML_TYPE_Q5_K 13
#define RXQ4_GGML_TYPE_Q6_K 14
#define RXQ4_MAX_K 65536

/* Element types for the typed GEMM entry point. */
#define RXQ4_DTYPE_F32 0
#define RXQ4_DTYPE_F16 1
#define RXQ4_DTYPE_BF16 2

/* One output range of a multi-matrix GEMV sharing one x (pair = 2, triple = 3). */
typedef struct rxq4_rows {
    void *y;           /* fp16 [M] */
    const void *w;     /* device blocks of ggml_type [M x K/256] */
    int ggml_type;
    int M;
} rxq4_rows;

/* y[M] fp16 = RNE(W[M x K] . x[K]), fp32 accumulation.
 * Replaces kernels::gemv_quant (reference q4_gemm.cu:2031-2036, 1856-1914). */
int rxq4_gemv_f16(void *y, const void *w, int ggml_type, const void *x, int M, int K,
                  void *stream);

/* y[M] fp16 = RNE(float(RNE(W . x)) + float(residual)); y may equal residual.
 * Replaces kernels::gemv_quant_add (reference q4_gemm.cu:2038-2045, 755-779). */
int rxq4_gemv_add_f16(void *y, const void *w, int ggml_type, const void *x,
                      const void *residual, int M, int K, void *stream);

/* 1..3 independent GEMVs sharing x, one launch (ranges may mix Q4_K, Q5_K
 * and Q6_K).
 * Replaces kernels::gemv_quant_pair (reference q4_gemm.cu:2047-2056) with
 * n_ranges = 2 and kernels::gemv_quant_triple (q4_gemm.cu:2058-2069) with 3. */
int rxq4_gemv_multi_f16(const rxq4_rows *ranges, int n_ranges, const void *x, int K,
                        void *stream);

/* y[M] fp32 = W . x (logits).
 * Replaces kernels::gemv_quant_f32 (reference q4_gemm.cu:2071-2076, 491-507). */
int rxq4_gemv_f32(float *y, const void *w, int ggml_type, const void *x, int M, int K,
                  void *stream);

/* y[N x M] fp16 (token-major) = x[N x K] fp16 . W^T.  N == 1 is the GEMV;
 * for Q4_K, N <= 4 runs the decode GEMV with every token's activations in
 * registers (per token bit-identical to the GEMV), N <= 16 the multi-token
 * MFMA kernel, larger N the MFMA GEMM; Q5_K / Q6_K run their multi-token
 * MFMA kernel up to N = 16 and the same GEMM above.
 * Replaces kernels::gemm_quant_batched (reference q4_gemm.cu:2023-2029,
 * 1707-1740). */
int rxq4_gemm_f16(void *y, const void *w, int ggml_type, const void *x, int M, int N,
                  int K, void *stream);

/* dst[hidden] fp16 = dequant(W[token_id, :]), bit-exact.
 * Replaces kernels::dequant_embedding_row (reference q4_gemm.cu:2078-2115).
 * Like the reference, token_id is not range-checked (no vocab size given). */
int rxq4_embed_row_f16(void *dst, const void *w, int ggml_type, int token_id,
                       int hidden_dim, void *stream);

/* NEW.  Typed GEMM: y[N x M] (y_dtype) = x[N x K] (x_dtype) . W^T.
 * Supported: x F16 -> y F16|F32, x BF16 -> y BF16|F32.  Weight tiles are
 * dequantised to the x type, products accumulate in fp32. */
int rxq4_gemm(void *y, int y_dtype, const void *w, int ggml_type, const void *x,
              int x_dtype, int M, int N, int K, void *stream);

/* NEW.  rxq4_gemm with no allocation: same arguments, routing, kernels and
 * results, but the fp32 partials of its split launches live in a fixed
 * 48 MiB device array of the library (one per device, made by the HIP
 * runtime when the entry point is first called on that device and held
 * until the process ends) instead of the stream's workspace, so no call ever allocates device
 * memory (no hipMalloc/hipFree/allocating library call).  No counterpart in
 * the reference; it is for callers that cannot allocate: code under HIP graph
 * capture, serving loops, harnesses that forbid allocation.  No shape is
 * refused for the array's size: the launchers shrink their split counts so
 * that the partials fit it (the same counts as rxq4_gemm, whose workspace has
 * the same size, so the results are identical).  The array keeps the last call's
 * contents and every call on a device shares it: calls that overlap on one
 * device (two streams, or two threads) race and must be serialised by the
 * caller. */
int rxq4_gemm_noalloc(void *y, int y_dtype, const void *w, int ggml_type, const void *x,
                      int x_dtype, int M, int N, int K, void *stream);

/* NEW.  Batched gather: dst[i, :] fp16 = dequant(W[ids[i], :]) for i < n_ids.
 * ids is a device int32 array; ids outside [0, n_vocab) give a zero row. */
int rxq4_embed_rows_f16(void *dst, const void *w, int ggml_type, int64_t n_vocab,
                        const int32_t *ids, int n_ids, int hidden_dim, void *stream);

/* NEW.  Quantise fp32 rows [n_rows x K] (device) to Q4_K blocks (device)
 * with a plain per-sub-block min/max fit (fast; not ggml's search). */
int rxq4_quantize_q4k(void *dst, const float *src, int64_t n_rows, int K, void *stream);

/* NEW.  Quantise fp32 rows [n_rows x K] (device, 16-byte aligned) to blocks
 * of ggml_type 12 (Q4_K), 13 (Q5_K) or 14 (Q6_K) (device; 16-byte aligned,
 * Q6_K 2-byte) with ggml's reference quantisers, byte for byte what
 * llama.cpp's quantize_row_q{4,5,6}_K_ref write without an importance
 * matrix (ggml-quants.c), so synthetic weights match real GGUF files
 * statistically.  No reference counterpart: the reference ships no
 * quantiser and reads these formats (q4_gemm.cu:147-171). */
int rxq4_quantize(void *dst, int ggml_type, const float *src, int64_t n_rows, int K,
                  void *stream);

/* out[n_heads x head_dim] fp16 = attention of one query token over KV
 * positions [0, seq_len): per head h (KV head h / (n_heads / n_kv_heads)),
 * softmax(scale * q.K^T) V with fp32 softmax.  k_cache / v_cache are
 * [pos][n_kv_heads][head_dim], fp16, or int8 when kv_int8 != 0 with optional
 * per-(position, KV head) fp32 scales k_scales / v_scales [pos][n_kv_heads]
 * (NULL = 1).  head_dim a multiple of 8 (int8: 16), at most 256; n_heads a
 * multiple of n_kv_heads.  Decode splits long sequences over the stream's
 * workspace described above.
 * Replaces kernels::flash_attention_decode (reference attention.cu:450-466,
 * 41-173). */
int rxq4_attention_decode_f16(void *out, const void *q, const void *k_cache,
                              const void *v_cache, int n_heads, int n_kv_heads, int head_dim,
                              int seq_len, float scale, int kv_int8, const float *k_scales,
                              const float *v_scales, void *stream);

/* Prefill: N query tokens q[N x n_heads x head_dim]; token t attends to
 * positions [0, start_pos + t + 1) of the caches (causal).
 * Replaces kernels::flash_attention_prefill_batched (reference
 * attention.cu:432-448, 180-290). */
int rxq4_attention_prefill_f16(void *out, const void *q, const void *k_cache,
                               const void *v_cache, int n_heads, int n_kv_heads, int head_dim,
                               int N, int start_pos, float scale, int kv_int8,
                               const float *k_scales, const float *v_scales, void *stream);

/* The reference's host GEMV (gemv_quant_cpu, q4_gemm.cu:1742-1854, with its
 * callers' output rounding: fp16 at 1898, fp32 at 2016, the residual's
 * double rounding at 1941-1945), on HOST pointers only: y[M] = W[M x K] . x[K]
 * for Q4_K / Q5_K / Q6_K blocks `w`, fp16 x; y_dtype F32 or F16; a non-NULL
 * fp16 `residual` (F16 only) gives y = RNE(float(RNE(acc)) + residual).  One
 * fp32 accumulator per row in the reference's element order, bit for bit its
 * result.  The C++ API runs it for weights the GPU cannot read (no
 * weights_device alias and host-only memory) and under JLLM_FAST_GEMV=0, as
 * the reference does (q4_gemm.cu:1886-1899, 1916-1947, 1994-2016); no GPU
 * launch ever falls back to it. */
int rxq4_host_gemv(void *y, int y_dtype, const void *w, int ggml_type, const void *x,
                   const void *residual, int M, int K);

/* Number of rxq4_host_gemv computations so far in this process. */
long long rxq4_host_gemv_calls(void);

/* NEW.  Allocates the split launches' workspace for `stream` on the
 * current device now, so that no later call on that stream allocates
 * (optional; no reference counterpart, the reference splits nothing). */
int rxq4_reserve_workspace(void *stream);

/* NEW.  Synchronises `stream` and frees its workspace on the current device
 * (for hipStreamPerThread: the calling thread's); Success also when it has
 * none.  For callers that create streams per request and would otherwise
 * keep 48 MiB per stream.  A graph captured with split launches on that
 * stream must not be replayed afterwards (its partials would point at
 * freed memory); the next split launch on the stream allocates again.  No
 * reference counterpart. */
int rxq4_release_workspace(void *stream);

/* Pointer resolution of the reference (q4_gemm.cu:111-135): returns
 * w_device if non-NULL, else w if the HIP runtime reports it as device or
 * managed memory, else NULL (host-only memory cannot be read by the kernels). */
const void *rxq4_resolve_weights(const void *w, const void *w_device);

/* Library version and the reason for the last non-success status on the
 * calling thread ("" if none). */
const char *rxq4_version(void);
const char *rxq4_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
