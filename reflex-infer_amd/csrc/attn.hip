// attn.hip -- decode and prefill attention for gfx950 (fp16 or int8 KV cache).
//
// Replaces flash_attention_decode_kernel / flash_attention_prefill_batched_kernel
// (reference src/kernels/attention.cu:41-173, 180-290): per query head h
// (KV head h / (n_heads / n_kv_heads)), out = softmax(scale * q.K^T) V over
// positions [0, seq_len), fp32 softmax and accumulation, fp16 out.  Prefill
// token t sees positions [0, start_pos + t + 1).  int8 caches hold
// int8 * k_scales[pos * n_kv_heads + kv_head] (scale 1 when NULL).
//
// A workgroup (4 waves) takes one KV head, up to 8 of its query heads, one
// token and one chunk of positions, so each K/V row is read once for the
// whole GQA group.  Positions are walked in tiles of 256 with an online
// softmax:
//   scores  a thread per position: its K row (16-byte loads) against the
//           group's q (fp32 in LDS, read as broadcasts);
//   softmax 32 threads per head: tile max, rescale factor, exp and sum;
//   P.V     a thread per fp16 pair of dims and per quarter of the tile (V rows
//           read 256 bytes per wave per position), partials added across the
//           4 waves through LDS at the end.
// Decode splits the positions over enough workgroups to fill the chip; each
// writes (max, sum, unnormalised output) to a workspace and a second launch
// combines the chunks in chunk order (results do not depend on scheduling).
#include <math.h>

#include <algorithm>

#include "launch.h"
#include "q4k_device.h"

namespace rxq4 {

constexpr int kAttnTile = 256;
constexpr int kAttnMaxHeads = 8;   // query heads per workgroup
constexpr int kAttnMaxDim = 256;

struct AttnParams {
    uint16_t *out;         // fp16 [n_tok][n_heads][head_dim]
    const uint16_t *q;     // fp16 [n_tok][n_heads][head_dim]
    const void *k, *v;     // fp16 or int8 [pos][n_kv][head_dim]
    const float *ks, *vs;  // int8 scales [pos][n_kv] or null
    float *ws;             // [n_heads][n_chunks][head_dim + 2] when n_chunks > 1
    int n_heads, n_kv, head_dim, group, hpw, n_hg;
    int seq0;              // positions of token 0 (decode: seq_len)
    int chunk, n_chunks;
    float scale;
    int kv_int8;
};

__global__ __launch_bounds__(256) void attn_kernel(AttnParams p) {
    __shared__ float qf[kAttnMaxHeads][kAttnMaxDim];
    __shared__ float sc[kAttnMaxHeads][kAttnTile];
    __shared__ float stat[3][kAttnMaxHeads];  // running max, running sum, rescale
    __shared__ float red[4][kAttnMaxHeads][kAttnMaxDim];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wq = tid >> 6;
    const int c = blockIdx.x % p.n_chunks;
    const int g = blockIdx.x / p.n_chunks;
    const int kvh = g / p.n_hg;
    const int h0 = kvh * p.group + (g % p.n_hg) * p.hpw;
    const int nh = min(p.hpw, kvh * p.group + p.group - h0);
    const int t = blockIdx.y;
    const int seq = p.seq0 + t;
    const int beg = c * p.chunk;
    const int end = min(seq, beg + p.chunk);
    const int hd = p.head_dim;
    const int64_t q_dim = (int64_t)p.n_heads * hd;

    for (int i = tid; i < nh * hd; i += 256)
        qf[i / hd][i % hd] = f16_bits_to_f32(p.q[t * q_dim + (int64_t)h0 * hd + i]);
    if (tid < kAttnMaxHeads) {
        stat[0][tid] = -INFINITY;
        stat[1][tid] = 0.0f;
    }
    // P.V: this thread's fp16 dim pairs (pp, pp + 64) for the quarter wq.
    const int npairs = hd >> 1;
    float acc[kAttnMaxHeads][2][2];
#pragma unroll
    for (int h = 0; h < kAttnMaxHeads; ++h)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[h][j][0] = acc[h][j][1] = 0.0f;
    __syncthreads();

    const int64_t row_stride = (int64_t)p.n_kv * hd;  // elements per position
    for (int p0 = beg; p0 < end; p0 += kAttnTile) {
        // Scores: thread tid = position p0 + tid.
        {
            const int pos = p0 + tid;
            float dot[kAttnMaxHeads];
#pragma unroll
            for (int h = 0; h < kAttnMaxHeads; ++h) dot[h] = 0.0f;
            if (pos < end) {
                const int64_t base = pos * row_stride + (int64_t)kvh * hd;
                if (!p.kv_int8) {
                    const u32x4 *kr = reinterpret_cast<const u32x4 *>(
                        static_cast<const uint16_t *>(p.k) + base);
                    for (int d8 = 0; d8 < hd / 8; ++d8) {
                        const u32x4 w = kr[d8];
                        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
                        float kf[8];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            kf[2 * i] = f16_bits_to_f32(wv[i] & 0xFFFFu);
                            kf[2 * i + 1] = f16_bits_to_f32(wv[i] >> 16);
                        }
#pragma unroll
                        for (int h = 0; h < kAttnMaxHeads; ++h) {
                            if (h < nh) {
#pragma unroll
                                for (int i = 0; i < 8; ++i) dot[h] += qf[h][8 * d8 + i] * kf[i];
                            }
                        }
                    }
                } else {
                    const u32x4 *kr = reinterpret_cast<const u32x4 *>(
                        static_cast<const int8_t *>(p.k) + base);
                    for (int d16 = 0; d16 < hd / 16; ++d16) {
                        const u32x4 w = kr[d16];
                        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
                        float kf[16];
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            kf[i] = (float)(int8_t)(uint8_t)(wv[i >> 2] >> (8 * (i & 3)));
#pragma unroll
                        for (int h = 0; h < kAttnMaxHeads; ++h) {
                            if (h < nh) {
#pragma unroll
                                for (int i = 0; i < 16; ++i) dot[h] += qf[h][16 * d16 + i] * kf[i];
                            }
                        }
                    }
                    const float s = p.ks ? p.ks[(int64_t)pos * p.n_kv + kvh] : 1.0f;
#pragma unroll
                    for (int h = 0; h < kAttnMaxHeads; ++h) dot[h] *= s;
                }
            }
#pragma unroll
            for (int h = 0; h < kAttnMaxHeads; ++h)
                if (h < nh) sc[h][tid] = pos < end ? dot[h] * p.scale : -INFINITY;
        }
        __syncthreads();
        // Online softmax: 32 threads per head.
        {
            const int h = tid >> 5, l32 = tid & 31;
            if (h < nh) {
                float mx = -INFINITY;
                for (int j = l32; j < kAttnTile; j += 32) mx = fmaxf(mx, sc[h][j]);
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
                const float m_old = stat[0][h];
                const float m_new = fmaxf(m_old, mx);
                // m_new is finite: the tile holds at least one position.
                const float corr = expf(m_old - m_new);  // 0 while m_old = -inf
                float sum = 0.0f;
                for (int j = l32; j < kAttnTile; j += 32) {
                    const float e = expf(sc[h][j] - m_new);  // 0 for positions past the end
                    sum += e;
                    const int pos = p0 + j;
                    sc[h][j] = (p.kv_int8 && p.vs && pos < end)
                                   ? e * p.vs[(int64_t)pos * p.n_kv + kvh]
                                   : e;
                }
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 32);
                // The 32 threads of a head are in one wave: their reads of
                // stat above precede this write.
                if (l32 == 0) {
                    stat[0][h] = m_new;
                    stat[1][h] = stat[1][h] * corr + sum;
                    stat[2][h] = corr;
                }
            }
        }
        __syncthreads();
        // P.V over this thread's quarter of the tile.
        {
            const int q0 = p0 + wq * 64;
            const int q1 = min(end, q0 + 64);
#pragma unroll
            for (int h = 0; h < kAttnMaxHeads; ++h) {
                if (h < nh) {
                    const float corr = stat[2][h];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[h][j][0] *= corr;
                        acc[h][j][1] *= corr;
                    }
                }
            }
            for (int pos = q0; pos < q1; ++pos) {
                const int64_t base = pos * row_stride + (int64_t)kvh * hd;
                float vf[2][2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int pp = lane + 64 * j;
                    vf[j][0] = vf[j][1] = 0.0f;
                    if (pp < npairs) {
                        if (!p.kv_int8) {
                            const uint32_t w =
                                reinterpret_cast<const uint32_t *>(
                                    static_cast<const uint16_t *>(p.v) + base)[pp];
                            vf[j][0] = f16_bits_to_f32(w & 0xFFFFu);
                            vf[j][1] = f16_bits_to_f32(w >> 16);
                        } else {
                            const uint16_t w = reinterpret_cast<const uint16_t *>(
                                static_cast<const int8_t *>(p.v) + base)[pp];
                            vf[j][0] = (float)(int8_t)(uint8_t)(w & 0xFFu);
                            vf[j][1] = (float)(int8_t)(uint8_t)(w >> 8);
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < kAttnMaxHeads; ++h) {
                    if (h < nh) {
                        const float pr = sc[h][pos - p0];
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            acc[h][j][0] += pr * vf[j][0];
                            acc[h][j][1] += pr * vf[j][1];
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    // Add the four quarters.
#pragma unroll
    for (int h = 0; h < kAttnMaxHeads; ++h)
        if (h < nh)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int pp = lane + 64 * j;
                if (pp < npairs) {
                    red[wq][h][2 * pp] = acc[h][j][0];
                    red[wq][h][2 * pp + 1] = acc[h][j][1];
                }
            }
    __syncthreads();
    for (int i = tid; i < nh * hd; i += 256) {
        const int h = i / hd, d = i % hd;
        const float o = red[0][h][d] + red[1][h][d] + red[2][h][d] + red[3][h][d];
        if (p.n_chunks == 1) {
            const float l = stat[1][h];
            p.out[t * q_dim + (int64_t)(h0 + h) * hd + d] = f32_to_f16_bits(l > 0.0f ? o * (1.0f / l) : 0.0f);
        } else {
            float *w = p.ws + ((int64_t)(h0 + h) * p.n_chunks + c) * (hd + 2);
            w[d] = o;
            if (d == 0) {
                w[hd] = stat[0][h];
                w[hd + 1] = stat[1][h];
            }
        }
    }
}

// Chunk combine (decode): out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
    const int h = blockIdx.x;
    const int hd = p.head_dim;
    const float *w = p.ws + (int64_t)h * p.n_chunks * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < p.n_chunks; ++c) M = fmaxf(M, w[c * (hd + 2) + hd]);
    float L = 0.0f;
    for (int c = 0; c < p.n_chunks; ++c)
        L += expf(w[c * (hd + 2) + hd] - M) * w[c * (hd + 2) + hd + 1];
    for (int d = threadIdx.x; d < hd; d += 256) {
        float o = 0.0f;
        for (int c = 0; c < p.n_chunks; ++c)
            o += expf(w[c * (hd + 2) + hd] - M) * w[c * (hd + 2) + d];
        p.out[(int64_t)h * hd + d] = f32_to_f16_bits(L > 0.0f ? o * (1.0f / L) : 0.0f);
    }
}

hipError_t launch_attention(uint16_t *out, const uint16_t *q, const void *k, const void *v,
                            const float *ks, const float *vs, int n_heads, int n_kv,
                            int head_dim, int n_tok, int seq0, float scale, int kv_int8,
                            hipStream_t st) {
    AttnParams p{};
    p.out = out;
    p.q = q;
    p.k = k;
    p.v = v;
    p.ks = ks;
    p.vs = vs;
    p.n_heads = n_heads;
    p.n_kv = n_kv;
    p.head_dim = head_dim;
    p.group = n_heads / n_kv;
    p.hpw = std::min(p.group, kAttnMaxHeads);
    p.n_hg = (p.group + p.hpw - 1) / p.hpw;
    p.seq0 = seq0;
    p.scale = scale;
    p.kv_int8 = kv_int8;
    const int units = n_kv * p.n_hg;
    p.n_chunks = 1;
    p.chunk = seq0 + n_tok;  // whole sequence
    if (n_tok == 1 && seq0 > kAttnTile) {
        // Decode: split the positions so that about 2 workgroups per CU run.
        const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
        const int want = std::max(1, std::min(64, (2 * cus + units - 1) / units));
        int chunk = (seq0 + want - 1) / want;
        chunk = (chunk + kAttnTile - 1) / kAttnTile * kAttnTile;
        p.chunk = chunk;
        p.n_chunks = (seq0 + chunk - 1) / chunk;
        if (p.n_chunks > 1) {
            const size_t bytes = (size_t)n_heads * p.n_chunks * (head_dim + 2) * sizeof(float);
            const hipError_t e = device_workspace(bytes, &p.ws);
            if (e != hipSuccess) return e;
        }
    }
    if (n_tok > 65535) return hipErrorInvalidValue;  // grid.y
    const dim3 grid(units * p.n_chunks, n_tok);
    attn_kernel<<<grid, 256, 0, st>>>(p);
    if (p.n_chunks > 1) attn_combine_kernel<<<n_heads, 256, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace rxq4
