// host_gemv.cpp -- the GEMV on the CPU, for weights the GPU cannot read.
//
// reflex-infer computes on the host when a weight pointer resolves to no
// GPU-visible address (host-only memory and no `weights_device` alias) or
// when JLLM_FAST_GEMV=0 (reference q4_gemm.cu:1886-1899, 1916-1947,
// 1994-2016); its loop is gemv_quant_cpu (q4_gemm.cu:1742-1854).  This is
// that computation: one fp32 accumulator per row, the elements of a row in
// the reference's order, every product and sum a separately rounded fp32
// operation (the file is built with -ffp-contract=off), so each output is
// bit for bit what the reference's host build computes.
//   Q4_K (q4_gemm.cu:1756-1784): per block, per quant group g = 0..3, the
//     32 low nibbles of qs[32g..32g+31] (sub-block 2g) then the 32 high
//     nibbles (sub-block 2g+1); w = (d*sc)*q - dmin*m, acc += w * x.
//   Q5_K (1785-1815): the same with the fifth bit from qh, bit pair 2g/2g+1.
//   Q6_K (1816-1846): per 128-weight half, l = 0..31, the four weights
//     l, l+32, l+64, l+96: acc += ((d*sc)*(q-32)) * x.
// Rows are independent, so they are spread over threads without changing
// any result.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "rxq4.h"
#include "status.h"

namespace {

// fp16 bits -> fp32, exact (IEEE binary16; NaN payloads kept).
float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {  // subnormal: m * 2^-24, exact in fp32
        const float v = std::ldexp(static_cast<float>(m), -24);
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// fp32 -> fp16 bits, round to nearest even (overflow to infinity).
uint16_t float_to_half(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u | static_cast<uint16_t>((a >> 13) & 0x1FFu);  // NaN
    if (a >= 0x47800000u) return sign | 0x7C00u;  // >= 65536 (and infinity)
    if (a >= 0x38800000u) {                       // normal fp16 range (carry may give inf)
        const uint32_t r = a - 0x38000000u;
        uint32_t h = r >> 13;
        const uint32_t rem = r & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return sign | static_cast<uint16_t>(h);
    }
    const uint32_t e = a >> 23;
    if (e == 0) return sign;  // fp32 subnormals are far below half an fp16 ulp
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t s = 126u - e;  // the value is m * 2^-s fp16 subnormal units, s >= 14
    if (s >= 32) return sign;
    uint32_t q = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u);
    const uint32_t halfway = 1u << (s - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return sign | static_cast<uint16_t>(q);
}

uint16_t load_u16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

// The 6-bit (scale, min) of sub-block j of a Q4_K / Q5_K block's 12 packed
// bytes: j < 4 in the low six bits of bytes j and j+4; j >= 4 split between
// the nibbles of byte j+4 and the top two bits of bytes j-4 and j.
void scale_min(const uint8_t *s, int j, float &sc, float &mn) {
    uint32_t a, b;
    if (j < 4) {
        a = s[j] & 63u;
        b = s[j + 4] & 63u;
    } else {
        a = (s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4);
        b = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    sc = static_cast<float>(a);
    mn = static_cast<float>(b);
}

// One row of Q4_K (144-byte blocks) or Q5_K (176-byte blocks).
template <bool Q5>
float row_q4q5(const uint8_t *row, int nb, const float *xf) {
    constexpr int kBytes = Q5 ? 176 : 144;
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * kBytes;
        const float d = half_to_float(load_u16(blk));
        const float dmin = half_to_float(load_u16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qh = blk + 16;                   // Q5_K only
        const uint8_t *qs = blk + (Q5 ? 48 : 16);
        const float *xb = xf + (size_t)b * 256;
        for (int g = 0; g < 4; ++g) {
            float sc_lo, m_lo, sc_hi, m_hi;
            scale_min(scales, 2 * g, sc_lo, m_lo);
            scale_min(scales, 2 * g + 1, sc_hi, m_hi);
            const float d_lo = d * sc_lo, dm_lo = dmin * m_lo;
            const float d_hi = d * sc_hi, dm_hi = dmin * m_hi;
            const uint8_t *q = qs + 32 * g;
            const float *xg = xb + 64 * g;
            for (int l = 0; l < 32; ++l) {
                int v = q[l] & 15;
                if (Q5 && ((qh[l] >> (2 * g)) & 1)) v += 16;
                const float w = d_lo * static_cast<float>(v) - dm_lo;
                acc = acc + w * xg[l];
            }
            for (int l = 0; l < 32; ++l) {
                int v = q[l] >> 4;
                if (Q5 && ((qh[l] >> (2 * g + 1)) & 1)) v += 16;
                const float w = d_hi * static_cast<float>(v) - dm_hi;
                acc = acc + w * xg[32 + l];
            }
        }
    }
    return acc;
}

// One row of Q6_K (210-byte blocks: ql[128], qh[64], int8 scales[16], d).
float row_q6(const uint8_t *row, int nb, const float *xf) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * 210;
        const float d = half_to_float(load_u16(blk + 208));
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
        for (int h = 0; h < 2; ++h) {
            const uint8_t *ql = blk + 64 * h;
            const uint8_t *qh = blk + 128 + 32 * h;
            const int8_t *s = sc + 8 * h;
            const float *xh = xf + (size_t)b * 256 + 128 * h;
            for (int l = 0; l < 32; ++l) {
                const int t = l / 16;
                const int lo0 = ql[l] & 15, lo1 = ql[l + 32] & 15;
                const int hi0 = ql[l] >> 4, hi1 = ql[l + 32] >> 4;
                const int qv[4] = {(lo0 | (((qh[l] >> 0) & 3) << 4)) - 32,
                                   (lo1 | (((qh[l] >> 2) & 3) << 4)) - 32,
                                   (hi0 | (((qh[l] >> 4) & 3) << 4)) - 32,
                                   (hi1 | (((qh[l] >> 6) & 3) << 4)) - 32};
                for (int r = 0; r < 4; ++r) {
                    const float w = d * static_cast<float>(s[t + 2 * r]) * static_cast<float>(qv[r]);
                    acc = acc + w * xh[l + 32 * r];
                }
            }
        }
    }
    return acc;
}

std::atomic<long long> g_calls{0};

}  // namespace

extern "C" {

int rxq4_host_gemv(void *y, int y_dtype, const void *w, int ggml_type, const void *x,
                   const void *residual, int M, int K) {
    const char *fn = "rxq4_host_gemv";
    if (ggml_type != RXQ4_GGML_TYPE_Q4_K && ggml_type != RXQ4_GGML_TYPE_Q5_K &&
        ggml_type != RXQ4_GGML_TYPE_Q6_K)
        return rxq4::set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT, "%s: ggml_type %d", fn,
                               ggml_type);
    if (K <= 0 || K % 256 != 0 || K > RXQ4_MAX_K || M < 0)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: M=%d K=%d", fn, M, K);
    if (y_dtype != RXQ4_DTYPE_F32 && y_dtype != RXQ4_DTYPE_F16)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: y_dtype %d", fn, y_dtype);
    if (residual && y_dtype != RXQ4_DTYPE_F16)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: residual needs fp16 y", fn);
    if (M == 0) return rxq4::set_ok();
    if (!y || !w || !x) return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null pointer", fn);
    g_calls.fetch_add(1, std::memory_order_relaxed);

    const int nb = K / 256;
    const size_t row_bytes = (size_t)nb * (ggml_type == RXQ4_GGML_TYPE_Q4_K   ? 144
                                           : ggml_type == RXQ4_GGML_TYPE_Q5_K ? 176
                                                                              : 210);
    std::vector<float> xf(K);
    const uint16_t *xh = static_cast<const uint16_t *>(x);
    for (int k = 0; k < K; ++k) xf[k] = half_to_float(xh[k]);
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const uint16_t *res = static_cast<const uint16_t *>(residual);

    auto rows = [&](int r0, int r1) {
        for (int r = r0; r < r1; ++r) {
            const uint8_t *row = wb + (size_t)r * row_bytes;
            const float acc = ggml_type == RXQ4_GGML_TYPE_Q4_K   ? row_q4q5<false>(row, nb, xf.data())
                              : ggml_type == RXQ4_GGML_TYPE_Q5_K ? row_q4q5<true>(row, nb, xf.data())
                                                                 : row_q6(row, nb, xf.data());
            if (y_dtype == RXQ4_DTYPE_F32) {
                static_cast<float *>(y)[r] = acc;
            } else if (!res) {
                static_cast<uint16_t *>(y)[r] = float_to_half(acc);
            } else {  // y = half(half(acc) + residual) (q4_gemm.cu:1941-1945)
                const float proj = half_to_float(float_to_half(acc));
                static_cast<uint16_t *>(y)[r] = float_to_half(proj + half_to_float(res[r]));
            }
        }
    };
    // Rows split over threads (per-row results do not depend on it).
    const long long work = (long long)M * K;
    int threads = (int)std::min<unsigned>(std::max(1u, std::thread::hardware_concurrency()), 16u);
    if (work < (1 << 22)) threads = 1;
    threads = std::min(threads, M);
    if (threads <= 1) {
        rows(0, M);
    } else {
        std::vector<std::thread> pool;
        const int per = (M + threads - 1) / threads;
        for (int t = 0; t < threads; ++t) {
            const int r0 = t * per, r1 = std::min(M, r0 + per);
            if (r0 < r1) pool.emplace_back(rows, r0, r1);
        }
        for (auto &th : pool) th.join();
    }
    return rxq4::set_ok();
}

long long rxq4_host_gemv_calls(void) { return g_calls.load(std::memory_order_relaxed); }

}  // extern "C"
