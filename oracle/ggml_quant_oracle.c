/*
 * ggml_quant_oracle.c -- CPU restatement of ggml's reference K-quant
 * quantisers (Q4_K, Q5_K, Q6_K), the algorithm llama.cpp uses to write GGUF
 * files when no importance matrix is given.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE (see q4k_oracle.h).  The reference
 * (FastCrest/reflex-infer) ships no quantiser; the Q4_K/Q5_K/Q6_K formats it
 * reads are ggml's (reference q4_gemm.cu:2, 147-171).  Third-party source
 * followed, not vendored in the reference and absent here: llama.cpp
 * ggml/src/ggml-quants.c (2024-2025 releases) -- nearest_int,
 * make_qkx2_quants, make_qx_quants, quantize_row_q4_K_ref,
 * quantize_row_q5_K_ref, quantize_row_q6_K_ref.  The steps and their
 * evaluation order are kept because the GPU quantiser must reproduce these
 * bytes exactly; the code is written for this build.
 *
 * Parity with ggml itself is UNPINNED (no ggml, no llama.cpp, no GGUF file
 * written by them is available here).  What pins it (tests/test_oracle_quant.py):
 * the closed-form error of the least-squares fit (the returned scale/min
 * minimise the weighted error over the final codes), the search never
 * being worse than the plain min/max codes, exact packing round trips through
 * the dequantisers, degenerate blocks (all-equal, all-zero, one non-zero,
 * positive-only), and error statistics on Gaussian data.
 */
#include <math.h>
#include <string.h>

#include "q4k_oracle.h"

/* ggml's nearest_int: add 1.5 * 2^23 and read the low mantissa bits (round to
 * nearest even for |v| < 2^22; what it returns beyond that is kept too). */
static int nearest_int_(float v) {
    const float t = v + 12582912.0f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007FFFFF) - 0x00400000;
}

static int imin_(int a, int b) { return a < b ? a : b; }
static int imax_(int a, int b) { return a > b ? a : b; }

/* make_qkx2_quants (use_mad = false): codes L[i] in [0, nmax] for
 * x ~ scale * L - the_min, searched over nstep + 1 trial inverse scales
 * with a weighted least-squares refit of (scale, min) per trial. */
static float make_qkx2_(int n, int nmax, const float *x, const float *w, uint8_t *L,
                        float *the_min, float rmin, float rdelta, int nstep) {
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        L[i] = (uint8_t)imax_(0, imin_(nmax, nearest_int_(iscale * (x[i] - mn))));
        float diff = scale * L[i] + mn - x[i];
        diff = diff * diff;
        best += w[i] * diff;
    }
    uint8_t Laux[32];
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            const int l = imax_(0, imin_(nmax, nearest_int_(iscale * (x[i] - mn))));
            Laux[i] = (uint8_t)l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                err += w[i] * diff;
            }
            if (err < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = err;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

/* make_qx_quants with rmse_type = 1 (weights x^2), no importance weights:
 * signed codes L[i] - nmax in [-nmax, nmax - 1], x ~ scale * (L - nmax). */
static float make_qx_(int n, int nmax, const float *x, uint8_t *L) {
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = imax_(-nmax, imin_(nmax - 1, nearest_int_(iscale * x[i])));
        L[i] = (uint8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = imax_(-nmax, imin_(nmax - 1, nearest_int_(iscale * x[i])));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                const int l = nearest_int_(iscale * x[i]);
                L[i] = (uint8_t)(nmax + imax_(-nmax, imin_(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* quantize_row_q4_K_ref / quantize_row_q5_K_ref for one 256-value block:
 * nmax 15 (Q4_K) or 31 (Q5_K). */
static void quantize_qk_block(const float *x, uint8_t *out, int five) {
    const int nmax = five ? 31 : 15;
    uint8_t L[ORC_QK_K];
    float scales[8], mins[8], w[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = five ? make_qkx2_(32, nmax, x + 32 * j, w, L + 32 * j, &mins[j], -0.5f, 0.1f, 15)
                         : make_qkx2_(32, nmax, x + 32 * j, w, L + 32 * j, &mins[j], -1.0f, 0.1f, 20);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        const uint8_t ls = (uint8_t)nearest_int_(inv_scale * scales[j]);
        const uint8_t lm = (uint8_t)nearest_int_(inv_min * mins[j]);
        sc[j] = ls < 63 ? ls : 63;
        m[j] = lm < 63 ? lm : 63;
    }
    const uint16_t d_raw = orc_f32_to_fp16(max_scale / 63.0f);
    const uint16_t dmin_raw = orc_f32_to_fp16(max_min / 63.0f);
    memcpy(out, &d_raw, 2);
    memcpy(out + 2, &dmin_raw, 2);
    orc_pack_scale_min_k4(sc, m, out + 4);
    for (int j = 0; j < 8; ++j) {
        const float d = orc_fp16_to_f32(d_raw) * sc[j];
        if (!d) continue;
        const float dm = orc_fp16_to_f32(dmin_raw) * m[j];
        for (int i = 0; i < 32; ++i) {
            const int l = nearest_int_((x[32 * j + i] + dm) / d);
            L[32 * j + i] = (uint8_t)imax_(0, imin_(nmax, l));
        }
    }
    if (!five) {
        uint8_t *qs = out + 16;
        for (int il = 0; il < 4; ++il)
            for (int l = 0; l < 32; ++l)
                qs[32 * il + l] = (uint8_t)(L[64 * il + l] | (L[64 * il + 32 + l] << 4));
        return;
    }
    uint8_t *qh = out + 16, *qs = out + 48;
    memset(qh, 0, 32);
    for (int il = 0; il < 4; ++il)
        for (int l = 0; l < 32; ++l) {
            const int lo = L[64 * il + l], hi = L[64 * il + 32 + l];
            qh[l] |= (uint8_t)(((lo >> 4) << (2 * il)) | ((hi >> 4) << (2 * il + 1)));
            qs[32 * il + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
        }
}

/* quantize_row_q6_K_ref for one block. */
static void quantize_q6_block(const float *x, uint8_t *out) {
    uint8_t L[ORC_QK_K];
    float scales[16];
    float max_scale = 0, max_abs = 0;
    for (int ib = 0; ib < 16; ++ib) {
        const float s = make_qx_(16, 32, x + 16 * ib, L + 16 * ib);
        scales[ib] = s;
        if (fabsf(s) > max_abs) {
            max_abs = fabsf(s);
            max_scale = s;
        }
    }
    memset(out, 0, ORC_Q6K_BYTES);
    if (max_abs < 1e-15f) return;  /* all-zero block: d = +0 */
    const float iscale = -128.0f / max_scale;
    const uint16_t d_raw = orc_f32_to_fp16(1 / iscale);
    int8_t *sc = (int8_t *)(out + 192);
    for (int ib = 0; ib < 16; ++ib) sc[ib] = (int8_t)imin_(127, nearest_int_(iscale * scales[ib]));
    memcpy(out + 208, &d_raw, 2);
    for (int j = 0; j < 16; ++j) {
        const float d = orc_fp16_to_f32(d_raw) * sc[j];
        if (!d) continue;
        for (int i = 0; i < 16; ++i) {
            const int l = nearest_int_(x[16 * j + i] / d);
            L[16 * j + i] = (uint8_t)(imax_(-32, imin_(31, l)) + 32);
        }
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int h = 0; h < 2; ++h)
        for (int l = 0; l < 32; ++l) {
            const uint8_t *q = L + 128 * h + l;
            ql[64 * h + l] = (uint8_t)((q[0] & 15) | ((q[64] & 15) << 4));
            ql[64 * h + 32 + l] = (uint8_t)((q[32] & 15) | ((q[96] & 15) << 4));
            qh[32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[32] >> 4) << 2) | ((q[64] >> 4) << 4) |
                                       ((q[96] >> 4) << 6));
        }
}

int orc_quantize_ggml(int type, const float *src, int64_t n_rows, int K, void *dst) {
    const int bytes = orc_block_bytes(type);
    if (bytes == 0 || K % ORC_QK_K != 0) return -1;
    const int64_t nb = (int64_t)n_rows * (K / ORC_QK_K);
    uint8_t *out = (uint8_t *)dst;
    for (int64_t b = 0; b < nb; ++b) {
        const float *x = src + b * ORC_QK_K;
        if (type == 14)
            quantize_q6_block(x, out + b * bytes);
        else
            quantize_qk_block(x, out + b * bytes, type == 13);
    }
    return 0;
}
