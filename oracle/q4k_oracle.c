/*
 * q4k_oracle.c -- CPU restatement of reflex-infer's Q4_K weight path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE (see q4k_oracle.h).  Reference file
 * for every citation: src/kernels/q4_gemm.cu of FastCrest/reflex-infer.  The
 * reference .cu file cannot be compiled here (it includes <cuda_runtime.h>
 * and no CUDA toolkit exists), so its CPU path is restated, not linked.
 *
 * What pins each function (tests/test_oracle.py):
 *   orc_fp16_to_f32        all 65536 patterns vs numpy's float16 decoder
 *   orc_f32_to_fp16        2^24 strided + boundary + random patterns vs numpy
 *   orc_f32_to_bf16        random + boundary patterns vs torch's RNE bf16 cast
 *   orc_get_scale_min_k4   exhaustive 64x64 per sub-block through the packer,
 *                          and an independent bit-field description of the
 *                          GGML 12-byte layout written in numpy
 *   orc_dequant_rows_*     closed forms (d=0, dmin=0, sc=m=0, q=15 ...),
 *                          subnormal/negative d, and a vectorised numpy
 *                          dequantiser written from the format description
 *   orc_gemv_f32           one-hot x (returns one dequantised column exactly),
 *                          integer-valued operands (exact dot), fp64 bound,
 *                          and a pure-Python float32 loop on tiny shapes
 *   orc_gemv_add_f16       double rounding checked against numpy float16 ops
 *   orc_gemm_tokens_f32    equals per-token orc_gemv_f32 (its definition) and
 *                          the fp64 bound
 *   orc_gemv_f64/gemm_f64  numpy float64 matmul on the dequantised matrix
 *   orc_quantize_rows      round trip |v - dq(q(v))| bound, packing
 *                          invariants, idempotence on representable inputs
 * Parity of these functions with the reference's own execution is unpinned
 * only in one respect: the reference ships no fixtures or tests for this
 * path, so no golden vector from the reference exists to check against.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    uint16_t d_raw;
    uint16_t dmin_raw;
    uint8_t scales[12];
    uint8_t qs[ORC_QK_K / 2];
} orc_block;

_Static_assert(sizeof(orc_block) == ORC_BLOCK_BYTES, "Q4_K block is 144 bytes");

/* q4_gemm.cu:177-188 */
float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t expo = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    float r;
    if (expo == 0) {
        r = ldexpf((float)mant, -24);
    } else if (expo == 31) {
        r = mant ? NAN : INFINITY;
    } else {
        r = ldexpf((float)(mant + 1024u), (int)expo - 25);
    }
    return sign ? -r : r;
}

uint16_t orc_f32_to_fp16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) {                 /* NaN: keep top payload bits, quiet */
        return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    }
    if (a >= 0x477FF000u) {                /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (a >= 0x38800000u) {                /* normal fp16 range, >= 2^-14 */
        uint32_t r = a - 0x38000000u;      /* exponent bias 127 -> 15 */
        r += 0xFFFu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    if (a <= 0x33000000u) {                /* <= 2^-25: rounds to (signed) zero */
        return (uint16_t)sign;
    }
    /* fp16 subnormal: result = RNE(|f| / 2^-24) */
    const uint32_t e = a >> 23;
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t s = 126u - e;           /* 14..24 */
    uint32_t m = mant >> s;
    const uint32_t rem = mant & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1u);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint16_t)(sign | m);
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* q4_gemm.cu:192-202 */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

void orc_pack_scale_min_k4(const uint8_t *sc, const uint8_t *mn, uint8_t *s) {
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

static const orc_block *row_blocks(const void *W, int64_t row, int K) {
    return (const orc_block *)W + row * (int64_t)(K / ORC_QK_K);
}

/* q4_gemm.cu:545-572: element i of a block -> il = i/64, sub-block
 * is = 2*il + (i%64 >= 32), q byte qs[32*il + i%32], low or high nibble;
 * val = dall * sc * q - dmin * m (fp32, left to right). */
static void dequant_block_f32(const orc_block *blk, float *out) {
    const float dall = orc_fp16_to_f32(blk->d_raw);
    const float dmin = orc_fp16_to_f32(blk->dmin_raw);
    for (int i = 0; i < ORC_QK_K; ++i) {
        const int il = i >> 6;
        const int lane64 = i & 63;
        const int lane32 = lane64 & 31;
        const int is = 2 * il + (lane64 >= 32);
        uint8_t sc, mn;
        orc_get_scale_min_k4(is, blk->scales, &sc, &mn);
        const uint8_t q = blk->qs[32 * il + lane32];
        const int qv = (lane64 < 32) ? (q & 0x0F) : (q >> 4);
        out[i] = dall * (float)sc * (float)qv - dmin * (float)mn;
    }
}

void orc_dequant_rows_f32(const void *W, int64_t row0, int64_t n_rows, int K, float *out) {
    const int nb = K / ORC_QK_K;
    for (int64_t r = 0; r < n_rows; ++r) {
        const orc_block *rb = row_blocks(W, row0 + r, K);
        for (int b = 0; b < nb; ++b) dequant_block_f32(&rb[b], out + r * K + (int64_t)b * ORC_QK_K);
    }
}

void orc_dequant_rows_f16(const void *W, int64_t row0, int64_t n_rows, int K, uint16_t *out) {
    float tmp[ORC_QK_K];
    const int nb = K / ORC_QK_K;
    for (int64_t r = 0; r < n_rows; ++r) {
        const orc_block *rb = row_blocks(W, row0 + r, K);
        for (int b = 0; b < nb; ++b) {
            dequant_block_f32(&rb[b], tmp);
            for (int i = 0; i < ORC_QK_K; ++i)
                out[r * K + (int64_t)b * ORC_QK_K + i] = orc_f32_to_fp16(tmp[i]);
        }
    }
}

void orc_dequant_rows_bf16(const void *W, int64_t row0, int64_t n_rows, int K, uint16_t *out) {
    float tmp[ORC_QK_K];
    const int nb = K / ORC_QK_K;
    for (int64_t r = 0; r < n_rows; ++r) {
        const orc_block *rb = row_blocks(W, row0 + r, K);
        for (int b = 0; b < nb; ++b) {
            dequant_block_f32(&rb[b], tmp);
            for (int i = 0; i < ORC_QK_K; ++i)
                out[r * K + (int64_t)b * ORC_QK_K + i] = orc_f32_to_bf16(tmp[i]);
        }
    }
}

void orc_embed_rows_f16(const void *W, int64_t n_rows, int K, const int32_t *ids,
                        int64_t n_ids, uint16_t *out) {
    for (int64_t i = 0; i < n_ids; ++i) {
        const int64_t id = ids[i];
        if (id < 0 || id >= n_rows) {
            memset(out + i * K, 0, (size_t)K * sizeof(uint16_t));
        } else {
            orc_dequant_rows_f16(W, id, 1, K, out + i * K);
        }
    }
}

/* gemv_quant_cpu, Q4_K branch: q4_gemm.cu:1750-1784, result store 1850. */
void orc_gemv_f32(const void *W, const uint16_t *x, int64_t row0, int64_t n_rows, int K,
                  float *y) {
    const int n_blocks = K / ORC_QK_K;
    /* x converted once up front: the conversion is exact, so this only saves
     * the per-element decode the reference repeats inside the loop. */
    float *xf = (float *)malloc((size_t)K * sizeof(float));
    for (int k = 0; k < K; ++k) xf[k] = orc_fp16_to_f32(x[k]);
    for (int64_t r = 0; r < n_rows; ++r) {
        float acc = 0.0f;
        const orc_block *rb = row_blocks(W, row0 + r, K);
        for (int b = 0; b < n_blocks; ++b) {
            const orc_block *blk = &rb[b];
            const float dall = orc_fp16_to_f32(blk->d_raw);
            const float dmin = orc_fp16_to_f32(blk->dmin_raw);
            const uint8_t *q = blk->qs;
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
                for (int l = 0; l < 32; ++l)
                    acc += (d1 * (q[l] & 0xF) - dm1) * xf[k + l];
                for (int l = 0; l < 32; ++l)
                    acc += (d2 * (q[l] >> 4) - dm2) * xf[k + 32 + l];
                q += 32;
                is += 2;
                k += 64;
            }
        }
        y[r] = acc;
    }
    free(xf);
}

typedef struct {
    const void *W;
    const uint16_t *x;
    int64_t row0, n_rows;
    int K;
    float *y;
} gemv_job;

static void *gemv_worker(void *arg) {
    gemv_job *j = (gemv_job *)arg;
    orc_gemv_f32(j->W, j->x, j->row0, j->n_rows, j->K, j->y + j->row0);
    return NULL;
}

void orc_gemv_f32_mt(const void *W, const uint16_t *x, int64_t M, int K, float *y,
                     int n_threads) {
    if (n_threads <= 1 || M < 2 * n_threads) {
        orc_gemv_f32(W, x, 0, M, K, y);
        return;
    }
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    gemv_job jobs[256];
    const int64_t per = (M + n_threads - 1) / n_threads;
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
        const int64_t r0 = (int64_t)t * per;
        if (r0 >= M) break;
        jobs[t] = (gemv_job){W, x, r0, (r0 + per > M) ? (M - r0) : per, K, y};
        if (pthread_create(&th[t], NULL, gemv_worker, &jobs[t]) != 0) {
            gemv_worker(&jobs[t]);
            th[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t)
        if (th[t]) pthread_join(th[t], NULL);
}

void orc_gemv_f16(const void *W, const uint16_t *x, int64_t M, int K, uint16_t *y) {
    float *tmp = (float *)malloc((size_t)M * sizeof(float));
    orc_gemv_f32(W, x, 0, M, K, tmp);
    for (int64_t i = 0; i < M; ++i) y[i] = orc_f32_to_fp16(tmp[i]);
    free(tmp);
}

void orc_gemv_add_f16(const void *W, const uint16_t *x, const uint16_t *res, int64_t M,
                      int K, uint16_t *y) {
    float *tmp = (float *)malloc((size_t)M * sizeof(float));
    orc_gemv_f32(W, x, 0, M, K, tmp);
    for (int64_t i = 0; i < M; ++i) {
        const uint16_t projected = orc_f32_to_fp16(tmp[i]);
        y[i] = orc_f32_to_fp16(orc_fp16_to_f32(projected) + orc_fp16_to_f32(res[i]));
    }
    free(tmp);
}

void orc_gemm_tokens_f32(const void *W, const uint16_t *x, int64_t M, int64_t N, int K,
                         float *y) {
    for (int64_t t = 0; t < N; ++t) orc_gemv_f32(W, x + t * K, 0, M, K, y + t * M);
}

void orc_gemv_f64(const void *W, const float *x, int64_t M, int K, double *y) {
    float *w = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < M; ++r) {
        orc_dequant_rows_f32(W, r, 1, K, w);
        double acc = 0.0;
        for (int k = 0; k < K; ++k) acc += (double)w[k] * (double)x[k];
        y[r] = acc;
    }
    free(w);
}

void orc_gemm_f64(const void *W, const float *x, int64_t M, int64_t N, int K, int wkind,
                  double *y) {
    float *w = (float *)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < M; ++r) {
        orc_dequant_rows_f32(W, r, 1, K, w);
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

static float clampf_(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* The build's own quantiser; see q4k_oracle.h.  Every step is a correctly
 * rounded IEEE operation (min/max, +, *, /, rint), evaluated in the same
 * order as the HIP quantiser. */
static void quantize_block(const float *v, orc_block *blk) {
    float span[8], off[8];
    float max_span = 0.0f, max_off = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float lo = v[32 * j], hi = v[32 * j];
        for (int i = 1; i < 32; ++i) {
            const float t = v[32 * j + i];
            lo = t < lo ? t : lo;
            hi = t > hi ? t : hi;
        }
        const float mo = lo < 0.0f ? -lo : 0.0f;
        const float top = hi > 0.0f ? hi : 0.0f;
        span[j] = (top + mo) / 15.0f;
        off[j] = mo;
        max_span = span[j] > max_span ? span[j] : max_span;
        max_off = mo > max_off ? mo : max_off;
    }
    const uint16_t d_raw = orc_f32_to_fp16(max_span / 63.0f);
    const uint16_t dmin_raw = orc_f32_to_fp16(max_off / 63.0f);
    const float d = orc_fp16_to_f32(d_raw);
    const float dmin = orc_fp16_to_f32(dmin_raw);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = (uint8_t)(d > 0.0f ? clampf_(rintf(span[j] / d), 0.0f, 63.0f) : 0.0f);
        mn[j] = (uint8_t)(dmin > 0.0f ? clampf_(rintf(off[j] / dmin), 0.0f, 63.0f) : 0.0f);
    }
    blk->d_raw = d_raw;
    blk->dmin_raw = dmin_raw;
    orc_pack_scale_min_k4(sc, mn, blk->scales);
    uint8_t q[ORC_QK_K];
    for (int j = 0; j < 8; ++j) {
        const float step = d * (float)sc[j];
        const float bias = dmin * (float)mn[j];
        for (int i = 0; i < 32; ++i) {
            float qv = 0.0f;
            if (step > 0.0f) qv = clampf_(rintf((v[32 * j + i] + bias) / step), 0.0f, 15.0f);
            q[32 * j + i] = (uint8_t)qv;
        }
    }
    for (int il = 0; il < 4; ++il)
        for (int l = 0; l < 32; ++l)
            blk->qs[32 * il + l] = (uint8_t)(q[64 * il + l] | (q[64 * il + 32 + l] << 4));
}

void orc_quantize_rows(const float *src, int64_t n_rows, int K, void *dst) {
    const int nb = K / ORC_QK_K;
    orc_block *out = (orc_block *)dst;
    for (int64_t r = 0; r < n_rows; ++r)
        for (int b = 0; b < nb; ++b)
            quantize_block(src + r * K + (int64_t)b * ORC_QK_K, &out[r * nb + b]);
}
