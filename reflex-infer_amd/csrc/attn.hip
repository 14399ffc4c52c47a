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
// whole GQA group.  Positions are walked in tiles of 64 with an online
// softmax (short tiles keep the serial latency of a workgroup low; decode
// spreads a sequence over about four workgroups per CU):
//   scores  16 lanes per position, 8 dims a lane (q of the group's heads
//           in registers), the lanes' partial dots summed with DPP row
//           rotations; the 16 positions of a lane group are loaded first;
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

constexpr int kAttnTile = 64;
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

// Sum over the 16 lanes of a DPP row (every lane gets the sum).
template <int CTRL>
__device__ __forceinline__ float row_ror_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v = row_ror_add<0x128>(v);  // row_ror:8
    v = row_ror_add<0x124>(v);  // row_ror:4
    v = row_ror_add<0x122>(v);  // row_ror:2
    return row_ror_add<0x121>(v);  // row_ror:1
}

// LDS hand-off between the waves of a workgroup: this wave's LDS accesses
// complete, then the barrier.  Unlike __syncthreads it leaves global loads in
// flight, so the next tile's K/V prefetch survives the softmax barriers.
__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Scale 1 for int8 caches without scale arrays: read with stride 0.
__device__ const float g_attn_one = 1.0f;

constexpr int kAttnPPG = kAttnTile / 16;  // score positions per lane group

// The raw K/V bytes (and int8 scales) one thread needs for one 64-position
// tile; loaded one tile ahead of the arithmetic.
template <int CPL, bool I8>
struct KvTile {
    u32x4 k[kAttnPPG][CPL];  // 8 dims: fp16 16 bytes, int8 8 bytes (.x, .y)
    uint32_t v[16][CPL];     // a dim pair of 16 positions: fp16 dword, int8 ushort
    float ks[kAttnPPG];      // int8: K scale of the score positions
    float vs[2];             // int8: V scale of the softmax positions
};

// CPL = 8-dim chunks per lane (1: head_dim <= 128, 2: <= 256); HPW = query
// heads per workgroup, a power of two (q is zero for heads past the group,
// whose results are not stored), so every head loop is unrolled without
// branches; I8 = int8 cache.
template <int CPL, int HPW, bool I8>
__global__ __launch_bounds__(256) void attn_kernel(AttnParams p) {
    constexpr int MAXH = HPW;
    constexpr int PPG = kAttnPPG;
    __shared__ float sc[2][kAttnMaxHeads][kAttnTile];  // double-buffered by tile
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
    constexpr int esz = I8 ? 1 : 2;  // bytes per K/V element

    if (end <= beg) {  // no positions (seq_len 0): zeros; uniform, before any barrier
        for (int i = tid; i < nh * hd; i += 256)
            p.out[t * q_dim + (int64_t)h0 * hd + i] = 0;
        return;
    }

    // Scores layout: lane group grp (16 lanes) takes positions grp + 16 i;
    // lane sub holds dims 8 (sub + 16 j), j < cpl.
    const int sub = tid & 15, grp = tid >> 4;
    const int n8 = hd >> 3;  // 8-dim chunks per row
    const int npairs = hd >> 1;
    const int64_t row_stride = (int64_t)p.n_kv * hd * esz;  // bytes per position
    const uint8_t *kb = static_cast<const uint8_t *>(p.k) + (int64_t)kvh * hd * esz;
    const uint8_t *vb = static_cast<const uint8_t *>(p.v) + (int64_t)kvh * hd * esz;
    const float *ksp = p.ks ? p.ks + kvh : &g_attn_one;
    const float *vsp = p.vs ? p.vs + kvh : &g_attn_one;
    const int s_stride = p.ks ? p.n_kv : 0, v_stride = p.vs ? p.n_kv : 0;
    const int sm_h = tid >> 5, l32 = tid & 31;  // softmax: 32 threads per head

    // Loads of one tile, all unconditional: positions past the end re-read
    // the last valid row (their results are discarded), so the compiler's
    // vmcnt bookkeeping stays exact and a prefetch never stalls a barrier.
    auto load_tile = [&](int p0, KvTile<CPL, I8> &T) {
#pragma unroll
        for (int i = 0; i < PPG; ++i) {
            const int pos = min(p0 + grp + 16 * i, end - 1);
            const uint8_t *row = kb + pos * row_stride;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int ch = min(sub + 16 * j, n8 - 1);
                if (I8) {
                    const u32x2 w = reinterpret_cast<const u32x2 *>(row)[ch];
                    T.k[i][j] = u32x4{w.x, w.y, 0u, 0u};
                } else {
                    T.k[i][j] = reinterpret_cast<const u32x4 *>(row)[ch];
                }
            }
            if (I8) T.ks[i] = ksp[(int64_t)pos * s_stride];
        }
        const int q0 = p0 + wq * (kAttnTile / 4);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int pos = min(q0 + i, end - 1);
            const uint8_t *row = vb + pos * row_stride;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int pp = min(lane + 64 * j, npairs - 1);
                T.v[i][j] = I8 ? (uint32_t)reinterpret_cast<const uint16_t *>(row)[pp]
                               : reinterpret_cast<const uint32_t *>(row)[pp];
            }
        }
        if (I8) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                T.vs[jj] = vsp[(int64_t)min(p0 + l32 + 32 * jj, end - 1) * v_stride];
        }
    };

    KvTile<CPL, I8> A, B;
    load_tile(beg, A);

    // q of the group's heads (16-byte loads, clamped; zero past the group).
    float qr[CPL][MAXH][8];
    {
        u32x4 qraw[CPL][MAXH];
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int h = 0; h < MAXH; ++h) {
                const int ch = min(sub + 16 * j, n8 - 1);
                const int hh = min(h, nh - 1);
                qraw[j][h] = *reinterpret_cast<const u32x4 *>(
                    p.q + t * q_dim + (int64_t)(h0 + hh) * hd + 8 * ch);
            }
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int h = 0; h < MAXH; ++h) {
                const bool ok = h < nh && sub + 16 * j < n8;
                const uint32_t w[4] = {qraw[j][h].x, qraw[j][h].y, qraw[j][h].z, qraw[j][h].w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qr[j][h][e] = ok ? f16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) : 0.0f;
            }
    }
    if (tid < kAttnMaxHeads) {
        stat[0][tid] = -INFINITY;
        stat[1][tid] = 0.0f;
    }
    // P.V: this thread's fp16 dim pairs (pp, pp + 64) for the quarter wq.
    float acc[MAXH][CPL][2];
#pragma unroll
    for (int h = 0; h < MAXH; ++h)
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[h][j][0] = acc[h][j][1] = 0.0f;

    auto process = [&](int p0, const KvTile<CPL, I8> &T, int buf) {
        // Scores.
#pragma unroll
        for (int i = 0; i < PPG; ++i) {
            const int pos = p0 + grp + 16 * i;
            float kf[CPL][8];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t wv[4] = {T.k[i][j].x, T.k[i][j].y, T.k[i][j].z, T.k[i][j].w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    kf[j][e] = I8 ? (float)(int8_t)(uint8_t)(wv[e >> 2] >> (8 * (e & 3)))
                                  : f16_bits_to_f32((wv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            }
#pragma unroll
            for (int h = 0; h < MAXH; ++h) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < CPL; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e) d += qr[j][h][e] * kf[j][e];
                d = row16_sum(d);
                if (sub == 0)
                    sc[buf][h][grp + 16 * i] =
                        pos < end ? d * (I8 ? T.ks[i] : 1.0f) * p.scale : -INFINITY;
            }
        }
        lds_sync();
        // Online softmax: 32 threads per head.
        if (sm_h < HPW) {
            float mx = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) mx = fmaxf(mx, sc[buf][sm_h][l32 + 32 * jj]);
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
            const float m_old = stat[0][sm_h];
            const float m_new = fmaxf(m_old, mx);
            // m_new is finite: the tile holds at least one position.
            const float corr = expf(m_old - m_new);  // 0 while m_old = -inf
            float sum = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = l32 + 32 * jj;
                const float e = expf(sc[buf][sm_h][j] - m_new);  // 0 past the end
                sum += e;
                sc[buf][sm_h][j] = I8 && p0 + j < end ? e * T.vs[jj] : e;
            }
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 32);
            // The 32 threads of a head are in one wave: their reads of stat
            // above precede this write.
            if (l32 == 0) {
                stat[0][sm_h] = m_new;
                stat[1][sm_h] = stat[1][sm_h] * corr + sum;
                stat[2][sm_h] = corr;
            }
        }
        lds_sync();
        // P.V over this thread's quarter of the tile (positions past q1
        // weigh 0).  The next tile's scores write the other sc buffer, and
        // its softmax (which rewrites stat) follows a barrier every wave
        // reaches only after this loop, so no third barrier is needed.
        const int q0 = p0 + wq * (kAttnTile / 4);
        const int q1 = min(end, q0 + kAttnTile / 4);
#pragma unroll
        for (int h = 0; h < MAXH; ++h) {
            const float corr = stat[2][h];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                acc[h][j][0] *= corr;
                acc[h][j][1] *= corr;
            }
        }
        float vf[16][CPL][2];
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t w = T.v[i][j];
                if (I8) {
                    vf[i][j][0] = (float)(int8_t)(uint8_t)(w & 0xFFu);
                    vf[i][j][1] = (float)(int8_t)(uint8_t)((w >> 8) & 0xFFu);
                } else {
                    vf[i][j][0] = f16_bits_to_f32(w & 0xFFFFu);
                    vf[i][j][1] = f16_bits_to_f32(w >> 16);
                }
            }
#pragma unroll
        for (int h = 0; h < MAXH; ++h) {
            const float4 *pr4 = reinterpret_cast<const float4 *>(&sc[buf][h][q0 - p0]);
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const float4 pr = pr4[i4];
                const float prs[4] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * i4 + e;
                    const float w = q0 + i < q1 ? prs[e] : 0.0f;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        acc[h][j][0] += w * vf[i][j][0];
                        acc[h][j][1] += w * vf[i][j][1];
                    }
                }
            }
        }
    };

    // Two tiles in flight: the next tile's loads go out before this tile's
    // arithmetic (the one past the end re-reads the last row: cache hits).
    for (int p0 = beg;;) {
        load_tile(p0 + kAttnTile, B);
        process(p0, A, 0);
        p0 += kAttnTile;
        if (p0 >= end) break;
        load_tile(p0 + kAttnTile, A);
        process(p0, B, 1);
        p0 += kAttnTile;
        if (p0 >= end) break;
    }

    // Add the four quarters.
#pragma unroll
    for (int h = 0; h < MAXH; ++h)
        if (h < nh)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int pp = lane + 64 * j;
                if (pp < npairs) {
                    red[wq][h][2 * pp] = acc[h][j][0];
                    red[wq][h][2 * pp + 1] = acc[h][j][1];
                }
            }
    lds_sync();
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
// Workgroup (head, 64-dim slice); every load is issued before the barrier:
// the first wave's chunk statistics and each wave's chunks w, w+4, .. for its
// lane's dim.  The first wave forms the weights; the four partial sums are
// added in wave order (results do not depend on scheduling).
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
    __shared__ float wgt[64];
    __shared__ float inv_l;
    __shared__ float part[4][64];
    const int hd = p.head_dim;
    const int n_sl = (hd + 63) / 64;
    const int h = blockIdx.x / n_sl;
    const int d0 = (blockIdx.x % n_sl) * 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int d = min(d0 + lane, hd - 1);
    const float *w = p.ws + (int64_t)h * p.n_chunks * (hd + 2);
    float a[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = w[min(wv + 4 * i, p.n_chunks - 1) * (hd + 2) + d];
    float m = -INFINITY, l = 0.0f;
    if (wv == 0) {
        const int cc = min(lane, p.n_chunks - 1);
        m = w[cc * (hd + 2) + hd];
        l = w[cc * (hd + 2) + hd + 1];
    }
    if (wv == 0) {
        const bool ok = lane < p.n_chunks;
        if (!ok) m = -INFINITY;
        float M = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float e = ok ? expf(m - M) : 0.0f;
        wgt[lane] = e;
        const float el = ok ? e * l : 0.0f;
        float L = 0.0f;
        for (int cc = 0; cc < p.n_chunks; ++cc) L += __shfl(el, cc, 64);  // chunk order
        if (lane == 0) inv_l = L > 0.0f ? 1.0f / L : 0.0f;
    }
    lds_sync();
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int cc = wv + 4 * i;
        o += (cc < p.n_chunks ? wgt[cc] : 0.0f) * a[i];
    }
    part[wv][lane] = o;
    lds_sync();
    if (tid < 64 && d0 + tid < hd) {
        const float s = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
        p.out[(int64_t)h * hd + d0 + tid] = f32_to_f16_bits(s * inv_l);
    }
}

template <bool I8>
static void launch_attn_t(const AttnParams &p, dim3 grid, int hp2, bool wide, hipStream_t st) {
    if (wide) {
        if (hp2 == 1) attn_kernel<2, 1, I8><<<grid, 256, 0, st>>>(p);
        else if (hp2 == 2) attn_kernel<2, 2, I8><<<grid, 256, 0, st>>>(p);
        else attn_kernel<2, 4, I8><<<grid, 256, 0, st>>>(p);
    } else {
        if (hp2 == 1) attn_kernel<1, 1, I8><<<grid, 256, 0, st>>>(p);
        else if (hp2 == 2) attn_kernel<1, 2, I8><<<grid, 256, 0, st>>>(p);
        else if (hp2 == 4) attn_kernel<1, 4, I8><<<grid, 256, 0, st>>>(p);
        else attn_kernel<1, 8, I8><<<grid, 256, 0, st>>>(p);
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
    // q of the workgroup's heads sits in registers: 8 heads up to 128 dims,
    // 4 beyond.
    p.hpw = std::min(p.group, head_dim > 128 ? kAttnMaxHeads / 2 : kAttnMaxHeads);
    p.n_hg = (p.group + p.hpw - 1) / p.hpw;
    p.seq0 = seq0;
    p.scale = scale;
    p.kv_int8 = kv_int8;
    const int units = n_kv * p.n_hg;
    p.n_chunks = 1;
    p.chunk = seq0 + n_tok;  // whole sequence
    if (n_tok == 1 && seq0 > kAttnTile) {
        // Decode: split the positions so that about 4 workgroups per CU run.
        const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
        const int want = std::max(1, std::min(64, (4 * cus + units - 1) / units));
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
    // hpw rounded up to a power of two selects the instance.
    const int hp2 = p.hpw <= 1 ? 1 : p.hpw <= 2 ? 2 : p.hpw <= 4 ? 4 : 8;
    if (kv_int8)
        launch_attn_t<true>(p, grid, hp2, head_dim > 128, st);
    else
        launch_attn_t<false>(p, grid, hp2, head_dim > 128, st);
    if (p.n_chunks > 1)
        attn_combine_kernel<<<n_heads * ((head_dim + 63) / 64), 256, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace rxq4
