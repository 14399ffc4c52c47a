/*
 * kquant_oracle.c -- CPU restatement of reflex-infer's Q5_K and Q6_K weight
 * formats (ggml types 13 and 14), the widening of the Q4_K path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE (see q4k_oracle.h).  Reference file
 * for every citation: src/kernels/q4_gemm.cu of FastCrest/reflex-infer.
 *
 * What pins each function (tests/test_oracle.py):
 *   orc_kq_dequant_rows_f32  closed forms through a numpy packer written from
 *                            the GGML block description (every q, scale, min
 *                            and high bit placed by index, then read back as
 *                            d*sc*(q-32) resp. d*sc*q - dmin*m), exhaustive
 *                            6-bit / 5-bit q values, negative and subnormal d
 *   orc_kq_gemv_f32          one-hot x (an exact dequantised column, which
 *                            ties the CPU loop's element order to the
 *                            embedding kernel's), integer-valued operands
 *                            (exact dot), the fp64 bound, and type 12 equal
 *                            to orc_gemv_f32
 *   orc_kq_embed_rows_f16    RNE of the pinned dequant (numpy float16)
 *   orc_kq_gemm_f64          numpy float64 matmul on the dequantised matrix
 * No golden vector from the reference exists for these formats (its tests
 * do not cover the quantised path).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "q4k_oracle.h"

typedef struct {
    uint16_t d_raw;
    uint16_t dmin_raw;
    uint8_t scales[12];
    uint8_t qh[ORC_QK_K / 8];
    uint8_t qs[ORC_QK_K / 2];
} orc_block_q5;

typedef struct {
    uint8_t ql[ORC_QK_K / 2];
    uint8_t qh[ORC_QK_K / 4];
    int8_t scales[ORC_QK_K / 16];
    uint8_t d_lo, d_hi; /* uint16 d at offset 208, unaligned in a packed row */
} orc_block_q6;

_Static_assert(sizeof(orc_block_q5) == ORC_Q5K_BYTES, "Q5_K block is 176 bytes");
_Static_assert(sizeof(orc_block_q6) == ORC_Q6K_BYTES, "Q6_K block is 210 bytes");

int orc_block_bytes(int ggml_type) {
    switch (ggml_type) {
        case 12: return ORC_BLOCK_BYTES;
        case 13: return ORC_Q5K_BYTES;
        case 14: return ORC_Q6K_BYTES;
        default: return 0;
    }
}

static const uint8_t *block_at(const void *W, int type, int64_t row, int K, int b) {
    return (const uint8_t *)W + (row * (int64_t)(K / ORC_QK_K) + b) * orc_block_bytes(type);
}

static float q6_d(const orc_block_q6 *blk) {
    return orc_fp16_to_f32((uint16_t)(blk->d_lo | (blk->d_hi << 8)));
}

/* q4_gemm.cu:574-616 (dequant_embedding_q6k_kernel): element i of a block ->
 * half = i/128, quarter = (i%128)/32, lane = i%32; q from the low (quarters
 * 0, 1) or high (2, 3) nibble of ql[64*half + lane (+32 for quarters 1, 3)]
 * and bits 2*quarter.. of qh[32*half + lane]; scale scales[8*half + lane/16 +
 * 2*quarter]; val = d * scale * (q - 32), left to right in fp32. */
static void dequant_q6_block(const orc_block_q6 *blk, float *out) {
    const float d = q6_d(blk);
    for (int i = 0; i < ORC_QK_K; ++i) {
        const int half = i >> 7;
        const int local = i & 127;
        const int lane = local & 31;
        const int quarter = local >> 5;
        const uint8_t *ql = blk->ql + half * 64;
        const uint8_t *qh = blk->qh + half * 32;
        const int8_t *sc = blk->scales + half * 8;
        const int is = lane >> 4;
        const int lo = (quarter & 1) ? ql[lane + 32] : ql[lane];
        const int nib = (quarter & 2) ? (lo >> 4) : (lo & 0x0F);
        const int qv = nib | (((qh[lane] >> (2 * quarter)) & 3) << 4);
        const int scale = sc[is + 2 * quarter];
        out[i] = d * (float)scale * (float)(qv - 32);
    }
}

/* Q5_K element i, as the CPU loop forms it (q4_gemm.cu:1785-1816):
 * il = i/64; low nibble of qs[32*il + i%32] for i%64 < 32 (sub-block 2*il,
 * high bit qh[i%32] & (1 << 2*il)), else high nibble (sub-block 2*il+1,
 * bit 2*il+1); w = (dall*sc) * q - dmin*m with q = nibble + 16*bit. */
static void dequant_q5_block(const orc_block_q5 *blk, float *out) {
    const float dall = orc_fp16_to_f32(blk->d_raw);
    const float dmin = orc_fp16_to_f32(blk->dmin_raw);
    for (int i = 0; i < ORC_QK_K; ++i) {
        const int il = i >> 6;
        const int hi = (i & 63) >= 32;
        const int l = i & 31;
        uint8_t sc, mn;
        orc_get_scale_min_k4(2 * il + hi, blk->scales, &sc, &mn);
        const float d1 = dall * sc;
        const float dm1 = dmin * mn;
        const uint8_t q = blk->qs[32 * il + l];
        const int nib = hi ? (q >> 4) : (q & 0x0F);
        const int bit = (blk->qh[l] >> (2 * il + hi)) & 1;
        out[i] = d1 * (nib + (bit ? 16 : 0)) - dm1;
    }
}

void orc_kq_dequant_rows_f32(const void *W, int type, int64_t row0, int64_t n_rows, int K,
                             float *out) {
    const int nb = K / ORC_QK_K;
    if (type == 12) {
        orc_dequant_rows_f32(W, row0, n_rows, K, out);
        return;
    }
    for (int64_t r = 0; r < n_rows; ++r)
        for (int b = 0; b < nb; ++b) {
            const uint8_t *p = block_at(W, type, row0 + r, K, b);
            float *o = out + r * K + (int64_t)b * ORC_QK_K;
            if (type == 13)
                dequant_q5_block((const orc_block_q5 *)p, o);
            else
                dequant_q6_block((const orc_block_q6 *)p, o);
        }
}

void orc_kq_embed_rows_f16(const void *W, int type, int64_t n_rows, int K, const int32_t *ids,
                           int64_t n_ids, uint16_t *out) {
    float *tmp = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t i = 0; i < n_ids; ++i) {
        const int64_t id = ids[i];
        if (id < 0 || id >= n_rows) {
            memset(out + i * K, 0, (size_t)K * sizeof(uint16_t));
            continue;
        }
        orc_kq_dequant_rows_f32(W, type, id, 1, K, tmp);
        for (int k = 0; k < K; ++k) out[i * K + k] = orc_f32_to_fp16(tmp[k]);
    }
    free(tmp);
}

/* gemv_quant_cpu, Q5_K branch (q4_gemm.cu:1785-1816) and Q6_K branch
 * (1817-1846): one fp32 accumulator per row, terms in the reference's order
 * (Q6_K interleaves k, k+32, k+64, k+96 for each l). */
void orc_kq_gemv_f32(const void *W, int type, const uint16_t *x, int64_t row0, int64_t n_rows,
                     int K, float *y) {
    if (type == 12) {
        orc_gemv_f32(W, x, row0, n_rows, K, y);
        return;
    }
    const int n_blocks = K / ORC_QK_K;
    float *xf = (float *)malloc((size_t)K * sizeof(float));
    for (int k = 0; k < K; ++k) xf[k] = orc_fp16_to_f32(x[k]);
    for (int64_t r = 0; r < n_rows; ++r) {
        float acc = 0.0f;
        for (int b = 0; b < n_blocks; ++b) {
            const uint8_t *p = block_at(W, type, row0 + r, K, b);
            if (type == 13) {
                const orc_block_q5 *blk = (const orc_block_q5 *)p;
                const float dall = orc_fp16_to_f32(blk->d_raw);
                const float dmin = orc_fp16_to_f32(blk->dmin_raw);
                const uint8_t *ql = blk->qs;
                const uint8_t *qh = blk->qh;
                uint8_t u1 = 1, u2 = 2;
                int is = 0;
                int k = b * ORC_QK_K;
                for (int j = 0; j < ORC_QK_K; j += 64) {
                    uint8_t sc1, m1, sc2, m2;
                    orc_get_scale_min_k4(is + 0, blk->scales, &sc1, &m1);
                    orc_get_scale_min_k4(is + 1, blk->scales, &sc2, &m2);
                    const float d1 = dall * sc1;
                    const float dm1 = dmin * m1;
                    const float d2 = dall * sc2;
                    const float dm2 = dmin * m2;
                    for (int l = 0; l < 32; ++l) {
                        const float w = d1 * ((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - dm1;
                        acc += w * xf[k + l];
                    }
                    for (int l = 0; l < 32; ++l) {
                        const float w = d2 * ((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - dm2;
                        acc += w * xf[k + 32 + l];
                    }
                    ql += 32;
                    is += 2;
                    u1 = (uint8_t)(u1 << 2);
                    u2 = (uint8_t)(u2 << 2);
                    k += 64;
                }
            } else {
                const orc_block_q6 *blk = (const orc_block_q6 *)p;
                const float d = q6_d(blk);
                const uint8_t *ql = blk->ql;
                const uint8_t *qh = blk->qh;
                const int8_t *sc = blk->scales;
                const int k_base = b * ORC_QK_K;
                for (int n = 0; n < ORC_QK_K; n += 128) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        const int k = k_base + n + l;
                        acc += d * (float)sc[is + 0] * (float)q1 * xf[k + 0];
                        acc += d * (float)sc[is + 2] * (float)q2 * xf[k + 32];
                        acc += d * (float)sc[is + 4] * (float)q3 * xf[k + 64];
                        acc += d * (float)sc[is + 6] * (float)q4 * xf[k + 96];
                    }
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
        }
        y[r] = acc;
    }
    free(xf);
}

/* fp64 GEMM on the dequantised matrix with the weights rounded to the MFMA
 * operand type first: wkind 0 = fp16, 1 = bf16, -1 = no rounding. */
void orc_kq_gemm_f64(const void *W, int type, const float *x, int64_t M, int64_t N, int K,
                     int wkind, double *y) {
    float *w = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < M; ++r) {
        orc_kq_dequant_rows_f32(W, type, r, 1, K, w);
        if (wkind >= 0)
            for (int k = 0; k < K; ++k)
                w[k] = wkind ? orc_bf16_to_f32(orc_f32_to_bf16(w[k]))
                             : orc_fp16_to_f32(orc_f32_to_fp16(w[k]));
        for (int64_t t = 0; t < N; ++t) {
            const float *xt = x + t * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)w[k] * (double)xt[k];
            y[t * M + r] = acc;
        }
    }
    free(w);
}
