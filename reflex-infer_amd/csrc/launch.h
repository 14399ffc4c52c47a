// launch.h -- host-side launchers of the gfx950 kernels (internal; the public
// surface is the C ABI in include/rxq4.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rxq4 {

// The fp32 workspace of the split launches (split-K partials, attention
// chunks): kWorkspaceBytes per (device, stream) (per (device, thread) for
// hipStreamPerThread), allocated by the first split launch on that stream,
// never resized, freed only by release_stream_workspace.  Launchers choose
// split counts whose partials fit in it.
constexpr size_t kWorkspaceBytes = size_t(48) << 20;
hipError_t stream_workspace(hipStream_t stream, float **ws);
// Synchronises `stream` and frees its workspace (*released = 1), or does
// nothing if it has none (*released = 0).
hipError_t release_stream_workspace(hipStream_t stream, int *released);

// Where a split launch keeps its fp32 partials: `ptr` (device memory of
// `bytes` bytes, supplied by the caller) or, when ptr is null, the stream's
// workspace above.
struct Scratch {
    float *ptr = nullptr;
    size_t bytes = 0;
    size_t capacity() const { return ptr ? bytes : kWorkspaceBytes; }
    // `need` bytes of it; launchers size their splits to fit, so a request
    // beyond the capacity is refused (no launch) rather than overrun
    hipError_t get(hipStream_t st, size_t need, float **p) const {
        if (need > capacity()) return hipErrorOutOfMemory;
        if (ptr) {
            *p = ptr;
            return hipSuccess;
        }
        return stream_workspace(st, p);
    }
};
int workspace_count();  // buffers allocated so far (all devices and streams)

enum Epilogue : int { kEpiF16 = 0, kEpiF32 = 1, kEpiAdd = 2 };

// One output range of a (multi-)GEMV: rows of `w` produce y[0 .. rows).
struct GemvRange {
    const uint8_t *w;
    void *y;
    const uint16_t *res;  // fp16 residual, kEpiAdd only
    int rows;
};

// Work is cut into "units" (a wave of the register kernel, a workgroup of the
// split kernel); every unit belongs to exactly one range, so the range is
// uniform across the unit.  Units [unit_start[i], unit_start[i+1]) serve
// range i.
struct GemvParams {
    GemvRange r[3];
    int n_ranges;
    int total_rows;
    const uint16_t *x;   // fp16 [K], 16-byte aligned
    int nb;              // Q4_K blocks per row = K / 256
    int per_unit;        // steps per wave (register kernel) / rows per workgroup (split)
    int unit_start[3];   // first unit of ranges 1..2 in [1], [2]; [0] = 0
    int total_units;
    int n_tok;           // tokens (1..kMaxRegTokens): x[t*K], y[t*y_stride + row]; one range if > 1
    int y_stride;
};

// Token counts the decode GEMV kernels take in one pass (one weight read).
constexpr int kMaxRegTokens = 4;

// Multi-token decode GEMV, 2 <= n_tok <= kMaxRegTokens, fp16 x [n_tok x K],
// y fp16 or fp32 [n_tok x M] (token-major).
hipError_t launch_gemv_multi_token(void *y, int y_dtype, const uint8_t *w, const uint16_t *x,
                                   int M, int n_tok, int K, hipStream_t stream);
// Whether launch_gemv_multi_token takes n_tok tokens of length K: rows of
// K/256 <= 16 blocks keep x in registers; longer rows stage every token's x
// in LDS (n_tok * K/256 * 576 bytes, at most 160 KiB).
bool gemv_multi_token_fits(int n_tok, int K);
// Whether n_tok tokens on M rows of length K run faster on the multi-token
// GEMV than on the MFMA small-batch kernel (measured crossover).
bool gemv_multi_token_preferred(int n_tok, int M, int K);

struct DeviceInfo {
    int cu_count;
    int arch_ok;  // 1 if the current device is gfx950
};

// Cached properties of the current device.
const DeviceInfo &device_info();

// Launch a GEMV over 1..3 ranges with the given epilogue.  Shapes were
// validated by the caller.  Returns hipSuccess or the launch error.
hipError_t launch_gemv(GemvParams p, int epilogue, hipStream_t stream);

// Multi-token GEMV for 2 <= n_tok <= kMaxSmallBatch tokens:
// y[t*M + row] (fp16 or fp32) = W[row] . x[t].
constexpr int kMaxSmallBatch = 16;
hipError_t launch_gemv_tokens(void *y, int y_dtype, const uint8_t *w, const void *x,
                              int x_dtype, int M, int n_tok, int K, hipStream_t stream,
                              const Scratch &sc = Scratch{});

// MFMA GEMM: y[N x M] = x[N x K] . dequant(W)^T for Q4_K (12), Q5_K (13)
// or Q6_K (14) weights, with x/weight tiles of the x type (fp16 or bf16) and
// fp32 accumulation; y fp32/fp16/bf16.
hipError_t launch_gemm(int ggml_type, void *y, int y_dtype, const uint8_t *w, const void *x,
                       int x_dtype, int M, int N, int K, hipStream_t stream,
                       const Scratch &sc = Scratch{});

// Embedding rows: dst[i, :] = fp16(dequant(W[id_i, :])).  ids == nullptr means
// the single row token_id (no range check, as in the reference).
hipError_t launch_embed(uint16_t *dst, const uint8_t *w, const int32_t *ids, int token_id,
                        int64_t n_vocab, int n_ids, int K, hipStream_t stream);

// Q5_K (13) / Q6_K (14) GEMV of one range with the given epilogue.
hipError_t launch_kq_gemv(int ggml_type, const GemvRange &r, const uint16_t *x, int K,
                          int epilogue, hipStream_t stream);

// 1..3 ranges of any of Q4_K / Q5_K / Q6_K sharing x, fp16 out, one launch.
hipError_t launch_kq_multi(const GemvRange *ranges, const int *types, int n_ranges,
                           const uint16_t *x, int K, hipStream_t stream);

// Q5_K / Q6_K multi-token product for any N >= 1 (16-token chunks).
hipError_t launch_kq_tokens(int ggml_type, void *y, int y_dtype, const uint8_t *w, const void *x,
                            int x_dtype, int M, int N, int K, hipStream_t stream);

// Q6_K embedding rows (as launch_embed).
hipError_t launch_kq_embed(uint16_t *dst, const uint8_t *w, const int32_t *ids, int token_id,
                           int64_t n_vocab, int n_ids, int K, hipStream_t stream);


// Tuning overrides from the environment, read once per process (for sweeps;
// 0 / true = the launchers' defaults):
//   RXQ4_GEMM_SPLITS, RXQ4_GEMV_WAVES_PER_CU, RXQ4_GEMV_LDS_WAVES_PER_CU,
//   RXQ4_ATTN_SPLIT (cap on decode chunks), RXQ4_ATTN_MFMA=0 (VALU prefill),
//   RXQ4_MULTI_TOKEN_GEMV=0 (2..4 tokens on the MFMA small-batch kernel),
//   RXQ4_GEMM_TM=128|256 (the GEMM's token tile),
//   RXQ4_GEMM_ORDER=1|2 (the GEMM's unit order: row-major | token-major),
//   RXQ4_GEMM_NW=4|8 (the GEMM's waves per workgroup: 128- or 256-row tiles),
//   RXQ4_TOKENS_WAVES=4|6|8 (waves of the LDS small-batch kernel's workgroups),
//   RXQ4_TOKENS_LDS_SPLIT=n (its K split on long rows),
//   RXQ4_GEMV_STREAM=0|n (one-token register GEMV: 0 the register kernel,
//   n the streamed kernel's long groups from n steps per wave, default 32).
struct Tuning {
    int gemm_splits = 0;
    int gemv_waves_per_cu = 0;
    int gemv_lds_waves_per_cu = 0;
    int attn_split = 0;
    bool attn_mfma = true;
    int multi_token_gemv = -1;  // 2..4 tokens on the multi-token GEMV: -1 measured crossover, 0 never, 1 always
    int gemm_tm = 0;
    int gemm_order = 0;
    int gemm_mixed = 0;  // > 0: mixed token tiles with this many whole areas per XCD
    int tokens_waves = 0;
    int tokens_lds_split = 0;
    int gemm_nw = 0;  // 4 | 8: force the GEMM's four- or eight-wave workgroup
    int gemv_stream = 0;  // -1 register kernel, n > 0 long stream groups from n steps, 0 default
};
const Tuning &tuning();

// Attention for n_tok query tokens; token t sees positions [0, seq0 + t).
// Decode is n_tok = 1, seq0 = seq_len; prefill seq0 = start_pos + 1.
hipError_t launch_attention(uint16_t *out, const uint16_t *q, const void *k, const void *v,
                            const float *ks, const float *vs, int n_heads, int n_kv,
                            int head_dim, int n_tok, int seq0, float scale, int kv_int8,
                            hipStream_t stream);

// fp32 rows -> Q4_K blocks (min/max quantiser).
hipError_t launch_quantize(uint8_t *dst, const float *src, int64_t n_blocks,
                           hipStream_t stream);

// fp32 rows -> blocks of ggml_type 12/13/14 with ggml's reference quantisers.
hipError_t launch_quantize_ggml(int ggml_type, uint8_t *dst, const float *src, int64_t n_blocks,
                                hipStream_t stream);

}  // namespace rxq4
