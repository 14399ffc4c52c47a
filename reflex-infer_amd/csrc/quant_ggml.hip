// quant_ggml.hip -- ggml-compatible K-quant quantisers (Q4_K, Q5_K, Q6_K) for
// gfx950: fp32 rows -> the bytes ggml's reference quantisers write when no
// importance matrix is given (llama.cpp ggml/src/ggml-quants.c:
// quantize_row_q{4,5,6}_K_ref over make_qkx2_quants / make_qx_quants), so
// synthetic weights carry the statistics of real GGUF files.  The reference
// ships no quantiser; it reads these formats (q4_gemm.cu:147-171).
//
// Mapping: one lane per sub-block (32 values for Q4_K/Q5_K, 16 for Q6_K), so
// every sum runs over its sub-block sequentially in ggml's order; a block's
// lanes are consecutive (8 or 16) and combine their scales with shuffles.
// Codes go through LDS to be packed.  Every fp32 step is a separately rounded
// IEEE operation (contraction off; division and square root correctly
// rounded), so the bytes equal the CPU restatement's bit for bit.
#include "launch.h"
#include "q4k_device.h"

#pragma clang fp contract(off)

namespace rxq4 {

namespace {

// ggml's nearest_int: 1.5 * 2^23 added, low mantissa bits read (round to
// nearest even for |v| < 2^22).
__device__ __forceinline__ int nearest_int(float v) {
    const float t = v + 12582912.0f;
    return (__builtin_bit_cast(int, t) & 0x007FFFFF) - 0x00400000;
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// make_qkx2_quants (squared error) over this lane's 32 values: codes in
// [0, NMAX], returns the scale and writes -min.
template <int NMAX, int NSTEP>
__device__ float make_qkx2(const float (&x)[32], const float (&w)[32], int (&L)[32],
                           float *the_min, float rmin, float rdelta) {
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        mn = x[i] < mn ? x[i] : mn;
        mx = x[i] > mx ? x[i] : mx;
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = (float)NMAX / (mx - mn);
    float scale = 1.0f / iscale;
    float best = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        L[i] = clampi(nearest_int(iscale * (x[i] - mn)), 0, NMAX);
        float diff = scale * (float)L[i] + mn - x[i];
        diff = diff * diff;
        best += w[i] * diff;
    }
#pragma unroll 1
    for (int is = 0; is <= NSTEP; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)NMAX) / (mx - mn);
        int La[32];
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            La[i] = clampi(nearest_int(iscale * (x[i] - mn)), 0, NMAX);
            const float l = (float)La[i];
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
            float err = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                float diff = this_scale * (float)La[i] + this_min - x[i];
                diff = diff * diff;
                err += w[i] * diff;
            }
            if (err < best) {
#pragma unroll
                for (int i = 0; i < 32; ++i) L[i] = La[i];
                best = err;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

// make_qx_quants, rmse_type 1, over this lane's 16 values: codes
// L - 32 in [-32, 31].
__device__ float make_qx32(const float (&x)[16], int (&L)[16]) {
    float mx = 0.0f, amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -32.0f / mx;
    float sumlx = 0.0f, suml2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int l = clampi(nearest_int(iscale * x[i]), -32, 31);
        L[i] = l + 32;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
#pragma unroll 1
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(32.0f + 0.1f * (float)is) / mx;
        sumlx = suml2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int l = clampi(nearest_int(iscale * x[i]), -32, 31);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) L[i] = 32 + clampi(nearest_int(iscale * x[i]), -32, 31);
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) {
        const float t = __shfl_xor(v, o, 64);
        v = t > v ? t : v;
    }
    return v;
}

// Q4_K (FIVE = false) / Q5_K blocks: 8 lanes per block, 32 blocks per
// 256-thread workgroup.  Every lane reaches the barrier.
template <bool FIVE>
__global__ __launch_bounds__(256) void quantize_qk_kernel(uint8_t *__restrict__ dst,
                                                          const float *__restrict__ src,
                                                          int64_t n_blocks) {
    constexpr int NMAX = FIVE ? 31 : 15;
    constexpr int BYTES = FIVE ? 176 : 144;
    __shared__ uint32_t codes[32][64];  // 256 codes of each block, 4 per dword
    const int tid = threadIdx.x;
    const int j = tid & 7;        // sub-block
    const int lb = tid >> 3;      // block within the workgroup
    const int64_t blk = (int64_t)blockIdx.x * 32 + lb;
    const bool live = blk < n_blocks;
    const float *xs = src + (live ? blk : 0) * kQK + 32 * j;
    float x[32], w[32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(xs + i);
        x[i] = v.x; x[i + 1] = v.y; x[i + 2] = v.z; x[i + 3] = v.w;
    }
    float sum_x2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) sum_x2 += x[i] * x[i];
    const float av_x = sqrtf(sum_x2 / 32.0f);
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = av_x + fabsf(x[i]);
    int L[32];
    float mmin;
    const float scale = FIVE ? make_qkx2<NMAX, 15>(x, w, L, &mmin, -0.5f, 0.1f)
                             : make_qkx2<NMAX, 20>(x, w, L, &mmin, -1.0f, 0.1f);
    // max over the block, starting from 0 as ggml does
    const float max_scale = group_max<8>(scale > 0.0f ? scale : 0.0f);
    const float max_min = group_max<8>(mmin > 0.0f ? mmin : 0.0f);
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    const uint32_t ls = min((uint32_t)(uint8_t)nearest_int(inv_scale * scale), 63u);
    const uint32_t lm = min((uint32_t)(uint8_t)nearest_int(inv_min * mmin), 63u);
    const uint16_t d_raw = f32_to_f16_bits(max_scale / 63.0f);
    const uint16_t dmin_raw = f32_to_f16_bits(max_min / 63.0f);
    const float d = f16_bits_to_f32(d_raw) * (float)ls;
    if (d != 0.0f) {
        const float dm = f16_bits_to_f32(dmin_raw) * (float)lm;
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = clampi(nearest_int((x[i] + dm) / d), 0, NMAX);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        codes[lb][8 * j + i] = (uint32_t)L[4 * i] | ((uint32_t)L[4 * i + 1] << 8) |
                               ((uint32_t)L[4 * i + 2] << 16) | ((uint32_t)L[4 * i + 3] << 24);
    // the eight (sc, m) pairs of the block, for its header
    uint32_t sc[8], mn[8];
    const int g0 = (tid & 63) & ~7;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        sc[s] = __shfl(ls, g0 + s, 64);
        mn[s] = __shfl(lm, g0 + s, 64);
    }
    __syncthreads();
    if (!live) return;
    uint8_t *out = dst + blk * BYTES;
    const uint32_t *cb = codes[lb];
    // qs: lane j packs bytes [16j, 16j + 16): group il = j / 2, l = 16 (j & 1) + [0, 16)
    // byte qs[32 il + l] = code[64 il + l] | code[64 il + 32 + l] << 4
    {
        const int il = j >> 1, l0 = 16 * (j & 1);
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = cb[(64 * il + l0) / 4 + k], hi = cb[(64 * il + 32 + l0) / 4 + k];
            q[k] = (lo & 0x0F0F0F0Fu) | ((hi & 0x0F0F0F0Fu) << 4);
        }
        *reinterpret_cast<u32x4 *>(out + (FIVE ? 48 : 16) + 16 * j) = u32x4{q[0], q[1], q[2], q[3]};
    }
    if (FIVE && j < 2) {
        // qh[l], l = 16 j + [0, 16): bit 2 il + hi = bit 4 of code[64 il + 32 hi + l]
        uint32_t h[4] = {0, 0, 0, 0};
#pragma unroll
        for (int il = 0; il < 4; ++il)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = cb[(64 * il + 16 * j) / 4 + k];
                const uint32_t hi = cb[(64 * il + 32 + 16 * j) / 4 + k];
                h[k] |= ((lo >> 4) & 0x01010101u) << (2 * il);
                h[k] |= ((hi >> 4) & 0x01010101u) << (2 * il + 1);
            }
        *reinterpret_cast<u32x4 *>(out + 16 + 16 * j) = u32x4{h[0], h[1], h[2], h[3]};
    }
    if (j == 0) {
        uint32_t words[3] = {0, 0, 0};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t b0 = (sc[s] & 63u) | ((sc[s + 4] >> 4) << 6);
            const uint32_t b4 = (mn[s] & 63u) | ((mn[s + 4] >> 4) << 6);
            const uint32_t b8 = (sc[s + 4] & 0xFu) | ((mn[s + 4] & 0xFu) << 4);
            words[0] |= b0 << (8 * s);
            words[1] |= b4 << (8 * s);
            words[2] |= b8 << (8 * s);
        }
        *reinterpret_cast<u32x4 *>(out) =
            u32x4{(uint32_t)d_raw | ((uint32_t)dmin_raw << 16), words[0], words[1], words[2]};
    }
}

// Q6_K blocks: 16 lanes per block (16-value sub-blocks), 16 blocks per
// workgroup.  Blocks are 210 bytes, so every store is 2 bytes wide.
__global__ __launch_bounds__(256) void quantize_q6_kernel(uint8_t *__restrict__ dst,
                                                         const float *__restrict__ src,
                                                         int64_t n_blocks) {
    __shared__ uint32_t codes[16][64];
    const int tid = threadIdx.x;
    const int ib = tid & 15;
    const int lb = tid >> 4;
    const int64_t blk = (int64_t)blockIdx.x * 16 + lb;
    const bool live = blk < n_blocks;
    const float *xs = src + (live ? blk : 0) * kQK + 16 * ib;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(xs + i);
        x[i] = v.x; x[i + 1] = v.y; x[i + 2] = v.z; x[i + 3] = v.w;
    }
    int L[16];
    const float scale = make_qx32(x, L);
    // the scale of largest magnitude, the lowest sub-block on ties (ggml's
    // strict '>' over ib = 0..15, starting from 0)
    float best_abs = fabsf(scale), best = scale;
    int best_ib = ib;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        const float ta = __shfl_xor(best_abs, o, 64), tb = __shfl_xor(best, o, 64);
        const int ti = __shfl_xor(best_ib, o, 64);
        if (ta > best_abs || (ta == best_abs && ti < best_ib)) {
            best_abs = ta;
            best = tb;
            best_ib = ti;
        }
    }
    const bool zero_block = !(best_abs >= 1e-15f);
    const float iscale = -128.0f / best;
    const uint16_t d_raw = zero_block ? (uint16_t)0 : f32_to_f16_bits(1.0f / iscale);
    const int sc = zero_block ? 0 : min(127, nearest_int(iscale * scale));
    const float d = f16_bits_to_f32(d_raw) * (float)sc;
    if (d != 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = clampi(nearest_int(x[i] / d), -32, 31) + 32;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        codes[lb][4 * ib + i] = (uint32_t)L[4 * i] | ((uint32_t)L[4 * i + 1] << 8) |
                                ((uint32_t)L[4 * i + 2] << 16) | ((uint32_t)L[4 * i + 3] << 24);
    const uint32_t sc_next = __shfl_down((uint32_t)sc & 0xFFu, 1, 64);
    __syncthreads();
    if (!live) return;
    uint16_t *out = reinterpret_cast<uint16_t *>(dst + blk * 210);
    const uint32_t *cb = codes[lb];
    if (zero_block) {
        // ggml writes an all-zero block
#pragma unroll
        for (int k = ib; k < 105; k += 16) out[k] = 0;
        return;
    }
    // ql: lane ib packs bytes [8 ib, 8 ib + 8); byte 64 h + 32 s + l
    // (l < 32) = code[128 h + 32 s + l] & 15 | (code[128 h + 32 s + 64 + l] & 15) << 4
    {
        const int h = ib >> 3, s = (ib >> 2) & 1, l0 = 8 * (ib & 3);
        const int base = 128 * h + 32 * s + l0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t lo = cb[base / 4 + k], hi = cb[(base + 64) / 4 + k];
            const uint32_t v = (lo & 0x0F0F0F0Fu) | ((hi & 0x0F0F0F0Fu) << 4);
            out[4 * ib + 2 * k] = (uint16_t)v;
            out[4 * ib + 2 * k + 1] = (uint16_t)(v >> 16);
        }
    }
    // qh: lane ib packs bytes [4 ib, 4 ib + 4) of qh[64]: byte 32 h + l
    // = sum_j (code[128 h + 32 j + l] >> 4) << 2 j
    {
        const int h = ib >> 3, l0 = 4 * (ib & 7);
        uint32_t v = 0;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) v |= ((cb[(128 * h + 32 * jj + l0) / 4] >> 4) & 0x03030303u) << (2 * jj);
        out[64 + 2 * ib] = (uint16_t)v;
        out[64 + 2 * ib + 1] = (uint16_t)(v >> 16);
    }
    // int8 scales at byte 192 (pairs by even lanes), d at byte 208
    if ((ib & 1) == 0) out[96 + ib / 2] = (uint16_t)(((uint32_t)sc & 0xFFu) | (sc_next << 8));
    if (ib == 0) out[104] = d_raw;
}

}  // namespace

hipError_t launch_quantize_ggml(int ggml_type, uint8_t *dst, const float *src, int64_t n_blocks,
                                hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    const int per = ggml_type == 14 ? 16 : 32;
    const int64_t grid = (n_blocks + per - 1) / per;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
    switch (ggml_type) {
        case 12: quantize_qk_kernel<false><<<(unsigned)grid, 256, 0, st>>>(dst, src, n_blocks); break;
        case 13: quantize_qk_kernel<true><<<(unsigned)grid, 256, 0, st>>>(dst, src, n_blocks); break;
        case 14: quantize_q6_kernel<<<(unsigned)grid, 256, 0, st>>>(dst, src, n_blocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rxq4
