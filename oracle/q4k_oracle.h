/*
 * q4k_oracle.h -- CPU restatement of reflex-infer's Q4_K weight path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, the smoke() check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load the
 * library built from this file, and only as the checker or the timed CPU
 * baseline.  The shipped library never calls into it.
 *
 * Every function names the reference lines (src/kernels/q4_gemm.cu in
 * FastCrest/reflex-infer) whose arithmetic it restates.  Build flags are
 * -O2 -ffp-contract=off without -ffast-math / -march, which keeps every fp32
 * operation a separately rounded IEEE-754 binary32 operation, exactly as the
 * reference's gcc host build on baseline x86-64 (no FMA) evaluates them.
 *
 * Pinning status (what independent check fixes each function) is written in
 * the header comment of q4k_oracle.c.
 */
#ifndef RXQ4_ORACLE_H
#define RXQ4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_BLOCK_BYTES 144
#define ORC_Q5K_BYTES 176
#define ORC_Q6K_BYTES 210

/* fp16 bits -> fp32, host branch of raw_fp16_to_float (q4_gemm.cu:177-188). */
float orc_fp16_to_f32(uint16_t h);
/* fp32 -> fp16 bits, round-to-nearest-even (the semantics of __float2half). */
uint16_t orc_f32_to_fp16(float f);
/* fp32 -> bf16 bits, round-to-nearest-even; NaN stays NaN (quiet). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);

/* 6-bit scale/min of sub-block j in [0,8) (q4_gemm.cu:192-202). */
void orc_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *mn);
/* Inverse of orc_get_scale_min_k4: packs 8 (sc, mn) pairs into 12 bytes. */
void orc_pack_scale_min_k4(const uint8_t *sc, const uint8_t *mn, uint8_t *scales);

/* Dequantise rows [row0, row0+n_rows) of a Q4_K matrix with K columns.
 * Element mapping and arithmetic of dequant_embedding_q4k_kernel
 * (q4_gemm.cu:545-572): w = d*sc*q - dmin*m in fp32. */
void orc_dequant_rows_f32(const void *W, int64_t row0, int64_t n_rows, int K, float *out);
/* Same, rounded to fp16 bits (q4_gemm.cu:571 __float2half). */
void orc_dequant_rows_f16(const void *W, int64_t row0, int64_t n_rows, int K, uint16_t *out);
/* Same, rounded to bf16 bits (the operand rounding of the bf16 MFMA GEMM). */
void orc_dequant_rows_bf16(const void *W, int64_t row0, int64_t n_rows, int K, uint16_t *out);
/* Gather: out[i, :] = dequant_f16(W[ids[i], :]); ids outside [0, n_rows)
 * give a zero row (the product kernel's documented behaviour). */
void orc_embed_rows_f16(const void *W, int64_t n_rows, int K, const int32_t *ids,
                        int64_t n_ids, uint16_t *out);

/* gemv_quant_cpu, Q4_K branch (q4_gemm.cu:1742-1784, store 1850): one fp32
 * accumulator per row, blocks in order, per 64-element group the 32 low
 * nibbles then the 32 high nibbles.  x is fp16 bits, y fp32.  Rows
 * [row0, row0+n_rows) only; y is indexed from 0. */
void orc_gemv_f32(const void *W, const uint16_t *x, int64_t row0, int64_t n_rows, int K,
                  float *y);
/* Multi-threaded driver of orc_gemv_f32 (rows split across threads; every
 * row is bit-identical to the single-threaded result). */
void orc_gemv_f32_mt(const void *W, const uint16_t *x, int64_t M, int K, float *y,
                     int n_threads);
/* fp16 output: y16 = RNE(gemv) (q4_gemm.cu:1898). */
void orc_gemv_f16(const void *W, const uint16_t *x, int64_t M, int K, uint16_t *y);
/* residual add: y16 = RNE(float(RNE(gemv)) + float(res)) (q4_gemm.cu:1941-1945). */
void orc_gemv_add_f16(const void *W, const uint16_t *x, const uint16_t *res, int64_t M,
                      int K, uint16_t *y);
/* Prefill GEMM as the reference's per-token fallback (q4_gemm.cu:1735-1739):
 * y[t*M + row] = RNE(gemv(x[t*K : (t+1)*K]))[row]; also the fp32 values. */
void orc_gemm_tokens_f32(const void *W, const uint16_t *x, int64_t M, int64_t N, int K,
                         float *y);

/* fp64 reference for tolerance checks: y[row] = sum_k w32[row,k] * x[k],
 * accumulated in double, with w32 the exact fp32 dequantised weight and x
 * given as fp32 values (already rounded to whatever operand type is used). */
/* Q5_K (ggml type 13) and Q6_K (14), kquant_oracle.c; type 12 forwards to
 * the Q4_K functions above. */
int orc_block_bytes(int ggml_type);
void orc_kq_dequant_rows_f32(const void *W, int type, int64_t row0, int64_t n_rows, int K,
                             float *out);
void orc_kq_embed_rows_f16(const void *W, int type, int64_t n_rows, int K, const int32_t *ids,
                           int64_t n_ids, uint16_t *out);
void orc_kq_gemv_f32(const void *W, int type, const uint16_t *x, int64_t row0, int64_t n_rows,
                     int K, float *y);
void orc_kq_gemm_f64(const void *W, int type, const float *x, int64_t M, int64_t N, int K,
                     int wkind, double *y);

/* Decode / prefill attention, attn_oracle.c.  q fp16 bits [n_heads x
 * head_dim] (prefill: [n_tok x ...]); k, v fp16 bits or int8 [pos x n_kv x
 * head_dim]; out fp32. */
void orc_attn_decode_f32(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                         int head_dim, int seq_len, float scale, int kv_int8, const float *ks,
                         const float *vs, float *out);
void orc_attn_prefill_f32(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                          int head_dim, int n_tok, int start_pos, float scale, int kv_int8,
                          const float *ks, const float *vs, float *out);
void orc_attn_decode_f64(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                         int head_dim, int seq_len, double scale, int kv_int8, const float *ks,
                         const float *vs, double *out);

void orc_gemv_f64(const void *W, const float *x, int64_t M, int K, double *y);
/* fp64 GEMM over operands rounded like the MFMA kernels: wr = round(w32) to
 * fp16 (wkind=0) or bf16 (wkind=1); x given as fp32 values [N x K];
 * y[t*M + row] = sum_k wr * x (double). */
void orc_gemm_f64(const void *W, const float *x, int64_t M, int64_t N, int K, int wkind,
                  double *y);

/* The build's own fp32 -> Q4_K quantiser (the reference ships none).  Per
 * 32-element sub-block: offset mo = max(0, -min), span s = (max + mo) / 15;
 * d = fp16(max s / 63), dmin = fp16(max mo / 63); sc = clamp(rint(s / d)),
 * m = clamp(rint(mo / dmin)); q = clamp(rint((v + dmin*m) / (d*sc)), 0, 15).
 * Only correctly rounded IEEE operations, so the HIP quantiser reproduces it
 * bit for bit. */
void orc_quantize_rows(const float *src, int64_t n_rows, int K, void *dst);

/* ggml's reference K-quant quantisers (ggml_quant_oracle.c): fp32 rows
 * [n_rows x K] -> blocks of type 12 (Q4_K), 13 (Q5_K) or 14 (Q6_K).
 * Returns 0, or -1 for another type or K % 256 != 0. */
int orc_quantize_ggml(int type, const float *src, int64_t n_rows, int K, void *dst);

#ifdef __cplusplus
}
#endif
#endif
