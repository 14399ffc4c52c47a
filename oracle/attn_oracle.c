/*
 * attn_oracle.c -- CPU restatement of reflex-infer's decode / prefill
 * attention (src/kernels/attention.cu of FastCrest/reflex-infer).
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE (see q4k_oracle.h).
 *
 * orc_attn_decode_f32 follows the reference CPU path (attention.cu:379-424):
 * per head, kv_head = head / (n_heads / n_kv_heads); score = (sum_d q*k) *
 * scale with one fp32 accumulator in d order; max; p = expf(score - max);
 * sum in position order; inv_sum = sum > 0 ? 1/sum : 0; out[d] = sum_pos
 * (p * inv_sum) * v.  The CPU path has no int8 KV; for it the element values
 * of the GPU kernels are used (attention.cu:88-96, 146-154): k = int8 *
 * k_scales[pos * n_kv_heads + kv_head] (scale 1 when k_scales is NULL),
 * likewise v.  Prefill (attention.cu:182-195): query token t attends to
 * positions [0, start_pos + t + 1).
 *
 * What pins it (tests/test_oracle_attn.py): seq_len 1 returns v[0] exactly;
 * equal keys or q = 0 give the mean of v; the fp64 softmax bound; heads of
 * one GQA group with equal q agree and take their group's K/V; int8 KV with
 * power-of-two scales equals the fp16 path on the same values; prefill is
 * causal (keys past a token's range do not change it) and equals decode at
 * seq_len start_pos + t + 1.
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "q4k_oracle.h"

static float kv_value(const void *cache, int kv_int8, const float *scales, int64_t pos,
                      int n_kv, int kvh, int head_dim, int d) {
    const int64_t idx = (pos * n_kv + kvh) * (int64_t)head_dim + d;
    if (kv_int8) {
        const float s = scales ? scales[pos * n_kv + kvh] : 1.0f;
        return (float)((const int8_t *)cache)[idx] * s;
    }
    return orc_fp16_to_f32(((const uint16_t *)cache)[idx]);
}

void orc_attn_decode_f32(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                         int head_dim, int seq_len, float scale, int kv_int8, const float *ks,
                         const float *vs, float *out) {
    const int gqa = n_heads / n_kv;
    float *scores = (float *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(float));
    for (int head = 0; head < n_heads; ++head) {
        const int kvh = head / gqa;
        const uint16_t *qh = q + (int64_t)head * head_dim;
        float max_score = -FLT_MAX;
        for (int pos = 0; pos < seq_len; ++pos) {
            float dot = 0.0f;
            for (int d = 0; d < head_dim; ++d)
                dot += orc_fp16_to_f32(qh[d]) * kv_value(k, kv_int8, ks, pos, n_kv, kvh, head_dim, d);
            const float score = dot * scale;
            scores[pos] = score;
            if (score > max_score) max_score = score;
        }
        float sum = 0.0f;
        for (int pos = 0; pos < seq_len; ++pos) {
            const float p = expf(scores[pos] - max_score);
            scores[pos] = p;
            sum += p;
        }
        const float inv_sum = (sum > 0.0f) ? (1.0f / sum) : 0.0f;
        for (int d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (int pos = 0; pos < seq_len; ++pos)
                acc += scores[pos] * inv_sum * kv_value(v, kv_int8, vs, pos, n_kv, kvh, head_dim, d);
            out[(int64_t)head * head_dim + d] = acc;
        }
    }
    free(scores);
}

void orc_attn_prefill_f32(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                          int head_dim, int n_tok, int start_pos, float scale, int kv_int8,
                          const float *ks, const float *vs, float *out) {
    const int64_t q_dim = (int64_t)n_heads * head_dim;
    for (int t = 0; t < n_tok; ++t)
        orc_attn_decode_f32(q + t * q_dim, k, v, n_heads, n_kv, head_dim, start_pos + t + 1, scale,
                            kv_int8, ks, vs, out + t * q_dim);
}

/* The same attention in fp64 (softmax and sums), for error bounds. */
void orc_attn_decode_f64(const uint16_t *q, const void *k, const void *v, int n_heads, int n_kv,
                         int head_dim, int seq_len, double scale, int kv_int8, const float *ks,
                         const float *vs, double *out) {
    const int gqa = n_heads / n_kv;
    double *scores = (double *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(double));
    for (int head = 0; head < n_heads; ++head) {
        const int kvh = head / gqa;
        const uint16_t *qh = q + (int64_t)head * head_dim;
        double mx = -INFINITY;
        for (int pos = 0; pos < seq_len; ++pos) {
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d)
                dot += (double)orc_fp16_to_f32(qh[d]) *
                       (double)kv_value(k, kv_int8, ks, pos, n_kv, kvh, head_dim, d);
            scores[pos] = dot * scale;
            if (scores[pos] > mx) mx = scores[pos];
        }
        double sum = 0.0;
        for (int pos = 0; pos < seq_len; ++pos) {
            scores[pos] = exp(scores[pos] - mx);
            sum += scores[pos];
        }
        for (int d = 0; d < head_dim; ++d) {
            double acc = 0.0;
            for (int pos = 0; pos < seq_len; ++pos)
                acc += scores[pos] * (double)kv_value(v, kv_int8, vs, pos, n_kv, kvh, head_dim, d);
            out[(int64_t)head * head_dim + d] = sum > 0.0 ? acc / sum : 0.0;
        }
    }
    free(scores);
}
