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
#include <stdlib.h>

#include <algorithm>

#include "launch.h"
#include "mfma_util.h"
#include "q4k_device.h"

namespace rxq4 {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

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

    // q of the group's heads (16-byte loads, clamped; zero past the group),
    // issued ahead of the first tile so that it lands first.
    float qr[CPL][MAXH][8];
    KvTile<CPL, I8> A, B;
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
        load_tile(beg, A);
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
            mx = butterfly_max<32>(mx);  // the head's 32 lanes are all active
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
            sum = butterfly_sum<32>(sum);  // the __shfl_xor butterfly's values, on the VALU
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
    // A chunk of one tile (most decode splits) has nothing to prefetch.
    if (end - beg <= kAttnTile) {
        process(beg, A, 0);
    } else {
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
// lane's dim.  The first wave forms the weights; all sums use fixed orders
// (a butterfly for the denominator, chunks w, w+4, .. per wave, then the
// waves in order), so results do not depend on scheduling.
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
        // max over the 64 lanes (exact in any order), no LDS instruction
        const float M = butterfly_max<64>(m);
        const float e = ok ? expf(m - M) : 0.0f;
        wgt[lane] = e;
        // Butterfly sum: a fixed association (every lane gets the same
        // value), so the result does not depend on scheduling.  Partners
        // lane ^ 1, ^ 2, ^ 4, ^ 8, ^ 16, ^ 32 in that order, on the VALU:
        // quad permutations, then the half-row mirror and row_ror:8 (after
        // the smaller steps they reach lanes holding the partner's value),
        // then the row swaps; each step adds the same two values in the same
        // order as a shuffle butterfly would.
        float L = ok ? e * l : 0.0f;
        L = dpp_row_add<0xB1>(L);   // quad_perm [1,0,3,2]
        L = dpp_row_add<0x4E>(L);   // quad_perm [2,3,0,1]
        L = dpp_row_add<0x141>(L);  // row_half_mirror
        L = dpp_row_add<0x128>(L);  // row_ror:8
        L = sum_xor_rows<16>(L);
        L = sum_xor_rows<32>(L);
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

// ---------------------------------------------------------------------------
// Prefill on the matrix cores (head_dim 64 or 128).  A workgroup takes one
// KV head, HB of its query heads and two half blocks of TPB / 2 consecutive
// tokens (TPB = 4 * (16 / HB)), an early one and the mirror late one, so
// every workgroup has about the same share of the causal triangle; wave w
// of each of two 4-wave groups owns 16 "query rows" (token, head) =
// (16 / HB tokens) x (HB heads), all sharing the KV head (waves 0, 1 the
// early half block, 2, 3 the late one).  Group q takes the
// KV tiles 2j + q (its own LDS buffers), so two waves share each SIMD and one
// wave's softmax and staging overlap the other's MFMAs (the query rows alone
// give one wave per SIMD: 1024 waves at 512 tokens x 32 heads); at the end
// group 1 hands its (m, l, O) to group 0 through LDS, which merges the two
// online softmaxes and writes the rows.
// Per 64-position tile, staged in LDS (K and V row-major, 16-byte writes)
// with the next tile's global loads in flight during this tile's arithmetic:
//   S^T = K . Q^T   v_mfma_f32_16x16x32_f16: src0 = 16 positions x 32 dims
//                   of K (LDS), src1 = Q^T (registers); lane l ends up with
//                   positions 4 (l/16) + i of query row l % 16;
//   online softmax  per query row (lane l % 16): the four lane groups
//                   combine with two shuffles; exp2 of log2e-scaled scores;
//   O^T += V^T . P^T the same MFMA with src0 = 16 dims x 32 positions of V^T
//                   (two ds_read_tr16_b64 of the row-major V, each a 4 x 16
//                   block transposed across a 16-lane group) and src1 = P^T
//                   straight from the score registers
//                   (the k order of a lane group is its positions
//                   {4g + i, 16 + 4g + i}, in both operands).  P is split
//                   into fp16 hi + lo parts (two MFMAs), so the products
//                   keep ~22 bits of the fp32 probabilities.
// Causal: query row (t, h) sees positions [0, start + t]; rows of a tile
// past that get probability 0 (rows with nothing visible yet keep m = -inf).
// Launch bounds: two resident workgroups of the one-group form per CU (LDS
// allows two), which caps a wave at 256 registers; uncapped, the compiler
// spread the one-group kernel over AGPRs with ~320 accvgpr moves per two
// tiles (2048 tokens 129 -> 119 us with the cap).
template <int HD, int HB, bool I8, int G>
__global__ __launch_bounds__(256 * G, 2 / G) void attn_prefill_mfma(AttnParams p, int start, int n_tok) {
    constexpr int TPW = 16 / HB;       // tokens per wave
    constexpr int TPB = 4 * TPW;       // tokens per workgroup
    // V is stored row-major with 16-byte writes and read transposed
    // (ds_read_tr16_b64); threads writing V^T with 8-byte writes instead
    // measured slower (512 tokens 18.45 against 17.2 us, 2048 tokens 119
    // against 111 us).
    constexpr int KROW = HD + 8;       // LDS K row (fp16), padded: 16 rows of a fragment read hit 64 banks
    constexpr int VROW = HD + 16;      // LDS V row (fp16), padded: 8 rows of a transposed read hit 64 banks
    constexpr int KCH = HD / 8;        // 8-dim chunks per row
    constexpr int NST = kAttnTile * KCH / 256;  // staged chunks per thread (K and V each)
    constexpr int VSZ = kAttnTile * VROW;
    __shared__ __attribute__((aligned(16))) uint16_t ktg[G][2][kAttnTile * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t vtg[G][2][VSZ];
    __shared__ float kscg[G][2][kAttnTile], vscg[G][2][kAttnTile];
    static_assert(2 * kAttnTile * KROW * 2 >= 256 * (HD / 4 + 2) * 4, "merge buffer fits");

    const int q = G == 1 ? 0 : threadIdx.x >> 8;  // group: KV tiles G*j + q
    const int tid = threadIdx.x & 255, lane = tid & 63, w = tid >> 6;
    uint16_t (*kt)[kAttnTile * KROW] = ktg[q];
    uint16_t (*vt)[VSZ] = vtg[q];
    float (*ksc)[kAttnTile] = kscg[q];
    float (*vsc)[kAttnTile] = vscg[q];
    const int r = lane & 15, g = lane >> 4;
    // Token half blocks of HPB tokens (two waves of a group); workgroup pr
    // pairs half block pr (waves 0, 1) with half block n_hbs - 1 - pr
    // (waves 2, 3), so every workgroup sees about the same number of
    // visible (query row, position) pairs: the causal triangle is balanced
    // over the CUs instead of one CU taking the last block's every tile.
    // With an odd count the middle half block pairs with itself and waves
    // 2, 3 compute nothing.
    constexpr int HPB = TPB / 2;
    const int n_hbs = (n_tok + HPB - 1) / HPB;
    const int n_pair = (n_hbs + 1) / 2;
    const int pr = (int)(blockIdx.x % n_pair);
    const int hbk = blockIdx.x / n_pair;
    const int n_hb = p.group / HB;
    const int kvh = hbk / n_hb;
    const int h = kvh * p.group + (hbk % n_hb) * HB + (r % HB);
    const int long_hb = n_hbs - 1 - pr;
    const int my_hb = w < 2 ? pr : long_hb;
    const bool dup = w >= 2 && long_hb == pr;
    const int t = my_hb * HPB + (w & 1) * TPW + r / HB;
    const bool row_ok = t < n_tok && !dup;
    const int tc = min(t, n_tok - 1);
    const int qpos = start + tc;  // last visible position of this query row
    // the wave's rows see positions [0, wave_end) at most (none when dup);
    // the workgroup stages tiles up to the long half block's pos_end
    const int wave_end = dup ? 0 : start + min(n_tok, (my_hb + 1) * HPB);
    const int blk_first = start + my_hb * HPB;  // first query position of the wave's half block
    const int pos_end = start + min(n_tok, (long_hb + 1) * HPB);
    const int n_tiles = (pos_end + kAttnTile - 1) / kAttnTile;
    constexpr int esz = I8 ? 1 : 2;
    const int64_t row_stride = (int64_t)p.n_kv * HD * esz;
    const uint8_t *kb = static_cast<const uint8_t *>(p.k) + (int64_t)kvh * HD * esz;
    const uint8_t *vb = static_cast<const uint8_t *>(p.v) + (int64_t)kvh * HD * esz;
    const float *ksp = p.ks ? p.ks + kvh : &g_attn_one;
    const float *vsp = p.vs ? p.vs + kvh : &g_attn_one;
    const int s_stride = p.ks ? p.n_kv : 0, v_stride = p.vs ? p.n_kv : 0;

    // Q^T fragments: dims 32 ks + 8 g .. + 8 of query row r.
    u32x4 qf[HD / 32];
    {
        const uint16_t *qrow = p.q + ((int64_t)tc * p.n_heads + h) * HD;
#pragma unroll
        for (int ks = 0; ks < HD / 32; ++ks)
            qf[ks] = *reinterpret_cast<const u32x4 *>(qrow + 32 * ks + 8 * g);
    }

    // Staging registers, a ring of two tiles (tile j in set j & 1, loaded
    // two iterations before it is used): K and V chunks row-major (16 lanes
    // per row: coalesced).
    struct Stage {
        u32x4 k[NST], vr[NST];
        float ks, vs;
    };
    // Byte offsets of the thread's staging loads within a tile (row p - p0
    // of the tile at (p - p0) * row_stride): the loads go through buffer
    // resources based at the tile's first row and bounded at pos_end, so
    // rows past the block's last visible position read zeros (their
    // scores are masked) and no 64-bit address is formed per load.
    int koff[NST];
#pragma unroll
    for (int j = 0; j < NST; ++j) {
        const int id = tid + 256 * j;
        koff[j] = (int)((id / KCH) * row_stride) + (id % KCH) * 8 * esz;
    }
    auto load_tile = [&](int p0, Stage &S) {
        // past the last tile (clamped prefetches that are never used): no rows
        // (the values are wave-uniform; readfirstlane keeps the descriptors
        // in scalar registers instead of a per-lane waterfall loop)
        const int bytes = __builtin_amdgcn_readfirstlane(
            (int)(max(0, min(pos_end - p0, kAttnTile)) * row_stride));
        const int64_t tile_off = (int64_t)p0 * row_stride;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)tile_off);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(tile_off >> 32));
        const int64_t toff = (int64_t)(((uint64_t)hi << 32) | lo);
        const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb + toff, bytes);
        const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vb + toff, bytes);
#pragma unroll
        for (int j = 0; j < NST; ++j) {
            if (I8) {
                const u32x2 a = buffer_load8(krs, koff[j]);
                S.k[j] = u32x4{a.x, a.y, 0u, 0u};
            } else {
                S.k[j] = buffer_load16(krs, koff[j]);
            }
            if (I8) {
                const u32x2 b = buffer_load8(vrs, koff[j]);
                S.vr[j] = u32x4{b.x, b.y, 0u, 0u};
            } else {
                S.vr[j] = buffer_load16(vrs, koff[j]);
            }
        }
        if (I8 && tid < kAttnTile) {
            const int pos = min(p0 + tid, pos_end - 1);
            S.ks = ksp[(int64_t)pos * s_stride];
            S.vs = vsp[(int64_t)pos * v_stride];
        }
    };
    // 8 int8 (bytes of .x, .y) as 8 fp16 (exact).
    auto i8_to_f16 = [](u32x4 v) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t wd = e < 2 ? v.x : v.y;
            const int sh = 16 * (e & 1);
            o[e] = pack2<RXQ4_DTYPE_F16>((float)(int8_t)(uint8_t)(wd >> sh),
                                         (float)(int8_t)(uint8_t)(wd >> (sh + 8)));
        }
        return u32x4{o[0], o[1], o[2], o[3]};
    };
    auto store_tile = [&](int b, const Stage &S) {
#pragma unroll
        for (int j = 0; j < NST; ++j) {
            const int id = tid + 256 * j;
            const u32x4 kv = I8 ? i8_to_f16(S.k[j]) : S.k[j];
            const u32x4 vv = I8 ? i8_to_f16(S.vr[j]) : S.vr[j];
            *reinterpret_cast<u32x4 *>(&kt[b][(id / KCH) * KROW + 8 * (id % KCH)]) = kv;
            *reinterpret_cast<u32x4 *>(&vt[b][(id / KCH) * VROW + 8 * (id % KCH)]) = vv;
        }
        if (I8 && tid < kAttnTile) {
            ksc[b][tid] = S.ks;
            vsc[b][tid] = S.vs;
        }
    };

    f32x4 o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const float sl2 = p.scale * 1.4426950408889634f;  // scores in log2 units

    // The group's tile j (KV tile 2j + q) is in LDS buffer j & 1 during
    // iteration j; tile j + 1 in registers, stored at its end; tile j + 2
    // loaded at its start.  Both groups run n_iter iterations (the barriers
    // are the workgroup's): group 1 has one tile fewer when n_tiles is odd,
    // and loads past a group's tiles are clamped re-reads that are never
    // stored or computed.
    const int n_j = (n_tiles - q + G - 1) / G;   // tiles of this group
    const int n_iter = (n_tiles + G - 1) / G;    // iterations of every group
    auto tile_p0 = [&](int j) { return (G * j + q) * kAttnTile; };
    Stage R0, R1;
    load_tile(tile_p0(0), R0);
    load_tile(tile_p0(1), R1);
    store_tile(0, R0);
    lds_sync();
    auto compute_tile = [&](int it, int b) {
        const int p0 = it * kAttnTile;
        // a tile past the wave's visible positions changes nothing (all its
        // probabilities are 0 and the rescale factor 1): skipped (uniform)
        if (p0 >= wave_end) return;
        // S^T for the 4 sub-tiles of 16 positions; the causal mask only on
        // tiles that reach past the block's first token (uniform: every
        // other tile is visible to all of the workgroup's rows).
        float sv[4][4];
        auto scores = [&](bool mask) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < HD / 32; ++ks) {
                    const u32x4 a = *reinterpret_cast<const u32x4 *>(
                        &kt[b][(16 * st + r) * KROW + 32 * ks + 8 * g]);
                    acc = mfma<RXQ4_DTYPE_F16>(a, qf[ks], acc);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int pp = 16 * st + 4 * g + i;
                    const float s = acc[i] * sl2 * (I8 ? ksc[b][pp] : 1.0f);
                    sv[st][i] = !mask || p0 + pp <= qpos ? s : -INFINITY;
                }
            }
        };
        if (p0 + kAttnTile - 1 <= blk_first)
            scores(false);
        else
            scores(true);
        float mx = -INFINITY;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[st][i]);
        mx = max_xor_rows<16>(mx);
        mx = max_xor_rows<32>(mx);
        const float m_new = fmaxf(m, mx);
        const bool live = m_new != -INFINITY;  // something visible so far
        const float corr = live ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
        // masked scores are -inf and exp2(-inf) = 0; rows with nothing
        // visible yet subtract 0 instead of -inf
        const float m_use = live ? m_new : 0.0f;
        float sum = 0.0f;
        uint32_t ph[2][4], pl[2][4];  // P^T hi / lo operands per 32-position k step
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                float e0 = __builtin_amdgcn_exp2f(sv[st][i] - m_use);
                float e1 = __builtin_amdgcn_exp2f(sv[st][i + 1] - m_use);
                sum += e0;
                sum += e1;
                if (I8) {
                    e0 *= vsc[b][16 * st + 4 * g + i];
                    e1 *= vsc[b][16 * st + 4 * g + i + 1];
                }
                const uint32_t hi = pack2<RXQ4_DTYPE_F16>(e0, e1);
                // lo = RNE_f16(e - f32(hi)): e - f32(hi) is exact in fp32,
                // so one fma_mix per half (e * 1 - hi, rounded once to fp16)
                // gives what fp32 subtraction and conversion give
                uint32_t lo;
                asm volatile("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]"
                             : "=v"(lo) : "v"(e0), "v"(hi));
                asm volatile("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
                             : "+v"(lo) : "v"(e1), "v"(hi));
                // k order of lane group g in step ks2: sub-tile 2 ks2 then 2 ks2 + 1
                ph[st >> 1][2 * (st & 1) + (i >> 1)] = hi;
                pl[st >> 1][2 * (st & 1) + (i >> 1)] = lo;
            }
        sum = sum_xor_rows<16>(sum);
        sum = sum_xor_rows<32>(sum);
        l = l * corr + sum;
        m = m_new;
        // O^T = corr * O^T + V^T . P^T
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            o[dt] *= corr;
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2) {
                // V^T operand: dim 16 dt + r, positions {32 ks2 + 4 g + i,
                // 32 ks2 + 16 + 4 g + i}
                // lane 4e + c of a 16-lane group supplies dims 16 dt + 4c .. +3
                // of position 32 ks2 + 4 g + e; lane r receives dim 16 dt + r
                // of the four positions
                const uint16_t *vp =
                    &vt[b][(32 * ks2 + 4 * g + (r >> 2)) * VROW + 16 * dt + 4 * (r & 3)];
                const u32x2 v0 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                               (__attribute__((address_space(3))) v4i16 *)vp));
                const u32x2 v1 = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                               (__attribute__((address_space(3))) v4i16 *)(vp + 16 * VROW)));
                const u32x4 a = u32x4{v0.x, v0.y, v1.x, v1.y};
                o[dt] = mfma<RXQ4_DTYPE_F16>(a, u32x4{ph[ks2][0], ph[ks2][1], ph[ks2][2], ph[ks2][3]}, o[dt]);
                o[dt] = mfma<RXQ4_DTYPE_F16>(a, u32x4{pl[ks2][0], pl[ks2][1], pl[ks2][2], pl[ks2][3]}, o[dt]);
            }
        }
    };
    for (int j = 0; j < n_iter; j += 2) {
        load_tile(tile_p0(j + 2), R0);  // past the end: clamped re-reads, not stored
        if (j < n_j) compute_tile(G * j + q, 0);
        if (j + 1 < n_j) store_tile(1, R1);  // uniform in the group
        lds_sync();
        if (j + 1 >= n_iter) break;          // uniform in the workgroup
        load_tile(tile_p0(j + 3), R1);
        if (j + 1 < n_j) compute_tile(G * (j + 1) + q, 1);
        if (j + 2 < n_j) store_tile(0, R0);
        lds_sync();
    }
    // Merge: group 1 writes its (O, m, l) per thread, group 0 adds them to
    // its own with the usual rescaling (scores are in log2 units).
    float *mb = reinterpret_cast<float *>(&ktg[G - 1][0][0]);
    constexpr int NO = HD / 4;  // O values per thread
    if (G == 2 && q == 1) {
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mb[(4 * dt + i) * 256 + tid] = o[dt][i];
        mb[NO * 256 + tid] = m;
        mb[(NO + 1) * 256 + tid] = l;
    }
    if (G == 2) lds_sync();
    if (q == 1) return;
    if (G == 2) {
        const float m1 = mb[NO * 256 + tid], l1 = mb[(NO + 1) * 256 + tid];
        const float mm = fmaxf(m, m1);
        const bool live = mm != -INFINITY;
        const float c0 = live ? __builtin_amdgcn_exp2f(m - mm) : 0.0f;
        const float c1 = live ? __builtin_amdgcn_exp2f(m1 - mm) : 0.0f;
        l = l * c0 + l1 * c1;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][i] = o[dt][i] * c0 + mb[(4 * dt + i) * 256 + tid] * c1;
    }
    if (row_ok) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t *orow = p.out + ((int64_t)t * p.n_heads + h) * HD;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            const uint32_t a = pack2<RXQ4_DTYPE_F16>(o[dt][0] * inv, o[dt][1] * inv);
            const uint32_t c = pack2<RXQ4_DTYPE_F16>(o[dt][2] * inv, o[dt][3] * inv);
            *reinterpret_cast<u32x2 *>(orow + 16 * dt + 4 * g) = u32x2{a, c};
        }
    }
}

// ---------------------------------------------------------------------------
// Decode on the matrix cores (one token, head_dim 64 / 128, GQA group <= 16).
// A workgroup takes one KV head, all its query heads (the columns of a 16x16
// MFMA tile; columns past the group multiply zero q) and one chunk of
// positions.  Wave w takes positions 16w .. 16w+15 of every 64-position tile
// of the chunk with its own online softmax; the four waves merge at the end.
//   S^T = K . Q^T   v_mfma_f32_16x16x32_f16: src0 = 16 positions x 32 dims of
//                   K straight from memory (16 bytes a lane), src1 = Q^T;
//                   lane l gets positions 4(l/16) + i of head l%16;
//   softmax         per head (lane column l%16), exp2 of log2e-scaled scores;
//   O^T += V^T.P^T  v_mfma_f32_16x16x16_f16: src0 = 16 dims x 16 positions of
//                   V^T by one ds_read_tr16_b64 of the wave's 16 V rows
//                   (staged in its own LDS rows), src1 = P^T as the score
//                   registers hold it (k = positions 4(l/16) + i); P as fp16
//                   hi + lo parts, as in the prefill kernel.
// The loads of up to four tiles go out before their arithmetic (one memory
// round trip per workgroup for chunks of up to 256 positions); they go
// through buffer resources based at each tile and bounded at the chunk's
// end, so positions past it read zeros (their scores are masked).  Partials
// use the VALU kernel's workspace format (o unnormalised, m in natural-log
// units, l) for attn_combine_kernel, or the output directly when the chunk
// is the whole sequence.
// Launch bounds: at least two workgroups per CU, i.e. at most 256 registers
// a wave; uncapped the compiler moved values through AGPRs (336 accvgpr
// moves in the head_dim 128 kernel).
template <int HD, bool I8>
__global__ __launch_bounds__(256, 2) void attn_decode_mfma(AttnParams p) {
    constexpr int KS = HD / 32;        // k-steps of the scores
    constexpr int DT = HD / 16;        // 16-dim tiles of O
    constexpr int VROW = HD + 16;      // LDS V row (fp16), padded
    constexpr int CH = HD / 8;         // 8-dim chunks per V row
    constexpr int NV = 16 * CH / 64;   // V chunks per lane and tile
    constexpr int NB = 4;              // tiles whose loads are in flight together
    constexpr int esz = I8 ? 1 : 2;
    constexpr int NM = DT * 4 + 2;     // merge values per lane: O, m, l
    __shared__ __attribute__((aligned(16))) uint16_t vl[4][16 * VROW];
    __shared__ float mg[4][NM][64];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int c = blockIdx.x % p.n_chunks;
    const int kvh = blockIdx.x / p.n_chunks;
    const int h0 = kvh * p.group;
    const int beg = c * p.chunk;
    const int end = min(p.seq0, beg + p.chunk);
    const int64_t row_stride = (int64_t)p.n_kv * HD * esz;
    const uint8_t *kb = static_cast<const uint8_t *>(p.k) + (int64_t)kvh * HD * esz;
    const uint8_t *vb = static_cast<const uint8_t *>(p.v) + (int64_t)kvh * HD * esz;
    const float *ksp = p.ks ? p.ks + kvh : &g_attn_one;
    const float *vsp = p.vs ? p.vs + kvh : &g_attn_one;
    const int s_stride = p.ks ? p.n_kv : 0, v_stride = p.vs ? p.n_kv : 0;
    const float sl2 = p.scale * 1.4426950408889634f;  // scores in log2 units

    // Q^T: column r = head h0 + r (zero past the group), dims 32 ks + 8 g .. + 7.
    u32x4 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        qf[ks] = r < p.group ? *reinterpret_cast<const u32x4 *>(p.q + (int64_t)(h0 + r) * HD + 32 * ks + 8 * g)
                             : u32x4{0u, 0u, 0u, 0u};
    // Byte offsets within a tile: the K fragment (position 16 w + r, dims
    // 32 ks + 8 g) and the lane's V chunks (row id / CH, chunk id % CH).
    const int kfo = (int)((16 * w + r) * row_stride) + 8 * g * esz;
    int vfo[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int id = lane + 64 * j;
        vfo[j] = (int)((16 * w + id / CH) * row_stride) + (id % CH) * 8 * esz;
    }
    // 8 int8 (bytes of .x, .y) as 8 fp16 (exact).
    auto i8_to_f16 = [](u32x2 v) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t wd = e < 2 ? v.x : v.y;
            const int sh = 16 * (e & 1);
            o[e] = pack2<RXQ4_DTYPE_F16>((float)(int8_t)(uint8_t)(wd >> sh),
                                         (float)(int8_t)(uint8_t)(wd >> (sh + 8)));
        }
        return u32x4{o[0], o[1], o[2], o[3]};
    };

    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const int n_tiles = (end - beg + kAttnTile - 1) / kAttnTile;  // 0 for an empty sequence

    for (int j0 = 0; j0 < n_tiles; j0 += NB) {
        u32x4 kf[NB][KS], vr[NB][NV];
        float ksc[NB][4], vsc[NB][4];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int p0 = beg + kAttnTile * (j0 + b);
            // tile base and bound as wave-uniform values (scalar descriptors)
            const int bytes = __builtin_amdgcn_readfirstlane(
                (int)(max(0, min(end - p0, kAttnTile)) * row_stride));
            const int64_t toff = (int64_t)p0 * row_stride;
            const uint32_t tlo = __builtin_amdgcn_readfirstlane((uint32_t)toff);
            const uint32_t thi = __builtin_amdgcn_readfirstlane((uint32_t)(toff >> 32));
            const int64_t to = (int64_t)(((uint64_t)thi << 32) | tlo);
            const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb + to, bytes);
            const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vb + to, bytes);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kf[b][ks] = I8 ? i8_to_f16(buffer_load8(krs, kfo + 32 * ks))
                               : buffer_load16(krs, kfo + 64 * ks);
#pragma unroll
            for (int j = 0; j < NV; ++j)
                vr[b][j] = I8 ? i8_to_f16(buffer_load8(vrs, vfo[j])) : buffer_load16(vrs, vfo[j]);
            if (I8) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int pos = min(p0 + 16 * w + 4 * g + i, end - 1);
                    ksc[b][i] = ksp[(int64_t)pos * s_stride];
                    vsc[b][i] = vsp[(int64_t)pos * v_stride];
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (j0 + b >= n_tiles) break;  // uniform
            const int p0 = beg + kAttnTile * (j0 + b);
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) acc = mfma<RXQ4_DTYPE_F16>(kf[b][ks], qf[ks], acc);
            float sv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = acc[i] * sl2 * (I8 ? ksc[b][i] : 1.0f);
                sv[i] = p0 + 16 * w + 4 * g + i < end ? s : -INFINITY;
            }
            float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            mx = max_xor_rows<16>(mx);
            mx = max_xor_rows<32>(mx);
            const float m_new = fmaxf(m, mx);
            const bool live = m_new != -INFINITY;
            const float corr = live ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
            const float m_use = live ? m_new : 0.0f;  // masked scores are -inf: exp2 gives 0
            float e[4], sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                e[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
                sum += e[i];
                if (I8) e[i] *= vsc[b][i];
            }
            sum = sum_xor_rows<16>(sum);
            sum = sum_xor_rows<32>(sum);
            l = l * corr + sum;
            m = m_new;
            // P^T hi / lo (lo = RNE_f16(e - f32(hi)), exact difference, one rounding)
            const uint32_t h01 = pack2<RXQ4_DTYPE_F16>(e[0], e[1]);
            const uint32_t h23 = pack2<RXQ4_DTYPE_F16>(e[2], e[3]);
            uint32_t l01, l23;
            asm volatile("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(l01) : "v"(e[0]), "v"(h01));
            asm volatile("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
                         : "+v"(l01) : "v"(e[1]), "v"(h01));
            asm volatile("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(l23) : "v"(e[2]), "v"(h23));
            asm volatile("v_fma_mixhi_f16 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
                         : "+v"(l23) : "v"(e[3]), "v"(h23));
            const f16x4 ph = __builtin_bit_cast(f16x4, u32x2{h01, h23});
            const f16x4 pl = __builtin_bit_cast(f16x4, u32x2{l01, l23});
            // the wave's V rows of this tile into its LDS rows (the wave's
            // own earlier reads of them are ahead in its LDS queue)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int id = lane + 64 * j;
                *reinterpret_cast<u32x4 *>(&vl[w][(id / CH) * VROW + 8 * (id % CH)]) = vr[b][j];
            }
            // O^T = corr O^T + V^T . P^T; lane r of group g supplies dims
            // 16 dt + 4 (r & 3) .. + 3 of position 4 g + r / 4 and receives
            // dim 16 dt + r of positions 4 g .. 4 g + 3
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const f16x4 a = __builtin_bit_cast(
                    f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16 *)
                                                                   &vl[w][(4 * g + (r >> 2)) * VROW + 16 * dt + 4 * (r & 3)]));
                o[dt] *= corr;
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pl, o[dt], 0, 0, 0);
            }
        }
    }

    // Merge the four waves: lane l of every wave holds head r, dims
    // 16 dt + 4 g + i; wave w merges dims of tiles dt = w, w + 4, ...
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mg[w][4 * dt + i][lane] = o[dt][i];
    mg[w][NM - 2][lane] = m;
    mg[w][NM - 1][lane] = l;
    __syncthreads();
    float mw[4], M = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        mw[v] = mg[v][NM - 2][lane];
        M = fmaxf(M, mw[v]);
    }
    float cw[4], L = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        cw[v] = M != -INFINITY ? __builtin_amdgcn_exp2f(mw[v] - M) : 0.0f;
        L += mg[v][NM - 1][lane] * cw[v];
    }
    const bool col_ok = r < p.group;
    const int h = h0 + r;
    float *wp = p.ws + ((int64_t)h * p.n_chunks + c) * (HD + 2);
#pragma unroll
    for (int dt = w; dt < DT; dt += 4) {
        float ov[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) s += mg[v][4 * dt + i][lane] * cw[v];
            ov[i] = s;
        }
        if (!col_ok) continue;
        const int d = 16 * dt + 4 * g;
        if (p.n_chunks == 1) {
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
            const uint32_t a = pack2<RXQ4_DTYPE_F16>(ov[0] * inv, ov[1] * inv);
            const uint32_t b = pack2<RXQ4_DTYPE_F16>(ov[2] * inv, ov[3] * inv);
            *reinterpret_cast<u32x2 *>(p.out + (int64_t)h * HD + d) = u32x2{a, b};
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) wp[d + i] = ov[i];
        }
    }
    if (p.n_chunks > 1 && col_ok && w == 0 && g == 0) {
        wp[HD] = M * 0.6931471805599453f;  // natural-log units, as the VALU kernel's
        wp[HD + 1] = L;
    }
}

template <int HD, bool I8, int G>
static void launch_prefill_g(unsigned grid, int hb, const AttnParams &p, int start, int n_tok,
                             hipStream_t st) {
    switch (hb) {
        case 1: attn_prefill_mfma<HD, 1, I8, G><<<grid, 256 * G, 0, st>>>(p, start, n_tok); break;
        case 2: attn_prefill_mfma<HD, 2, I8, G><<<grid, 256 * G, 0, st>>>(p, start, n_tok); break;
        case 4: attn_prefill_mfma<HD, 4, I8, G><<<grid, 256 * G, 0, st>>>(p, start, n_tok); break;
        case 8: attn_prefill_mfma<HD, 8, I8, G><<<grid, 256 * G, 0, st>>>(p, start, n_tok); break;
        default: attn_prefill_mfma<HD, 16, I8, G><<<grid, 256 * G, 0, st>>>(p, start, n_tok); break;
    }
}

// Two wave groups per workgroup (KV tiles split between them) while the
// query rows give at most one wave per SIMD; more rows fill the SIMDs with
// one group and keep the LDS of two workgroups per CU (512 tokens x 32
// heads: 18.9 -> 17.1 us with two groups; 2048 tokens: 138.6 us with one,
// 145.0 with two).
template <int HD, bool I8>
static void launch_prefill_hd(const AttnParams &p, int hb, int start, int n_tok, hipStream_t st) {
    const int units = p.n_kv * (p.group / hb);
    const int tpb = 4 * (16 / hb);
    const unsigned grid = (unsigned)(units * ((n_tok + tpb - 1) / tpb));
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    if ((int64_t)grid * 4 <= 4 * cus)
        launch_prefill_g<HD, I8, 2>(grid, hb, p, start, n_tok, st);
    else
        launch_prefill_g<HD, I8, 1>(grid, hb, p, start, n_tok, st);
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
    // decode on the matrix cores: one workgroup per KV head takes all of its
    // query heads (the 16 columns of an MFMA tile)
    const bool mfma_decode = n_tok == 1 && (head_dim == 64 || head_dim == 128) &&
                             p.group <= 16 && tuning().attn_mfma;
    const int units = mfma_decode ? n_kv : n_kv * p.n_hg;
    p.n_chunks = 1;
    p.chunk = seq0 + n_tok;  // whole sequence
    if (n_tok == 1 && seq0 > kAttnTile) {
        // Decode: split the positions so that about 4 workgroups per CU run.
        const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
        int cap = tuning().attn_split ? std::min(64, tuning().attn_split) : 64;
        // the chunk partials (n_heads x chunks x (head_dim + 2) fp32) must fit the workspace
        const size_t per_chunk = (size_t)n_heads * (head_dim + 2) * sizeof(float);
        cap = (int)std::min<size_t>(cap, std::max<size_t>(1, kWorkspaceBytes / per_chunk));
        int want = std::max(1, std::min(cap, (4 * cus + units - 1) / units));
        // the MFMA kernel does best with at least two tiles a chunk (32 / 64
        // chunks at 4096 positions: 10.55 / 11.1 us; 16384: 20.65 / 20.1)
        if (mfma_decode) want = std::max(1, std::min(want, (seq0 + 2 * kAttnTile - 1) / (2 * kAttnTile)));
        int chunk = (seq0 + want - 1) / want;
        chunk = (chunk + kAttnTile - 1) / kAttnTile * kAttnTile;
        p.chunk = chunk;
        p.n_chunks = (seq0 + chunk - 1) / chunk;
        if (p.n_chunks > 1) {
            const hipError_t e =
                Scratch{}.get(st, per_chunk * p.n_chunks, &p.ws);
            if (e != hipSuccess) return e;
        }
    }
    if (n_tok > 1 && (head_dim == 64 || head_dim == 128) && tuning().attn_mfma) {
        // Prefill on the matrix cores; HB = the largest power of two <= 16
        // dividing the GQA group.
        int hb = 1;
        while (hb < 16 && p.group % (2 * hb) == 0) hb *= 2;
        const int start = seq0 - 1;
        const int64_t blocks = (int64_t)n_kv * (p.group / hb) * ((n_tok + 4 * (16 / hb) - 1) / (4 * (16 / hb)));
        if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
        if (head_dim == 64) {
            if (kv_int8) launch_prefill_hd<64, true>(p, hb, start, n_tok, st);
            else launch_prefill_hd<64, false>(p, hb, start, n_tok, st);
        } else {
            if (kv_int8) launch_prefill_hd<128, true>(p, hb, start, n_tok, st);
            else launch_prefill_hd<128, false>(p, hb, start, n_tok, st);
        }
        return hipGetLastError();
    }
    if (mfma_decode) {
        const unsigned grid = (unsigned)(n_kv * p.n_chunks);
        if (head_dim == 64) {
            if (kv_int8) attn_decode_mfma<64, true><<<grid, 256, 0, st>>>(p);
            else attn_decode_mfma<64, false><<<grid, 256, 0, st>>>(p);
        } else {
            if (kv_int8) attn_decode_mfma<128, true><<<grid, 256, 0, st>>>(p);
            else attn_decode_mfma<128, false><<<grid, 256, 0, st>>>(p);
        }
        if (p.n_chunks > 1)
            attn_combine_kernel<<<n_heads * ((head_dim + 63) / 64), 256, 0, st>>>(p);
        return hipGetLastError();
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
