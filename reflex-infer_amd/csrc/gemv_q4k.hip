// gemv_q4k.hip -- Q4_K decode GEMV for gfx950 (MI355X).
//
// Replaces the reference's decode GEMV family (q4_gemm.cu:204-323 dot
// helpers, 437-507 single-output kernels, 755-890 add/pair/triple kernels).
// Design, per 64-weight "slot" = (block b, 32-byte quant group il):
//   * a lane owns one slot of a row: it loads the block header (16 B) and the
//     slot's 32 quant bytes (2 x 16 B) with 128-bit loads; consecutive lanes
//     own consecutive slots, so a wave streams whole rows;
//   * the lane's 64 activations live in VGPRs for the whole kernel, stored as
//     fp16 pairs permuted to match the nibble layout, together with their sum;
//   * nibbles become fp16 with one v_and_or_b32 per pair: (q & 0x000F000F) |
//     0x64006400 is the fp16 pair (1024 + q_a, 1024 + q_b); high nibbles are
//     used in place as 1024 + 16 q.  v_dot2_f32_f16 multiplies pairs into an
//     fp32 accumulator seeded with -1024 * sum(x), so the bias cancels;
//   * per slot: y += d*sc_lo*S_lo - dmin*m_lo*sum_lo + (d*sc_hi/16)*S_hi -
//     dmin*m_hi*sum_hi, i.e. the reference's w = d*sc*q - dmin*m factored
//     over the sub-block;
//   * the lanes of a row are summed with DPP row rotations and broadcasts;
//   * loads for the next batch of rows are issued before the current batch is
//     computed (two register buffers), so memory and VALU overlap per wave.
// Work: ~1.6 VALU ops per weight, under the ~2.8 ops/weight that 8 TB/s of
// 4.5-bit weights leaves on 256 CUs.  Bytes per launch: rows*K/256*144 +
// K*2 + rows*out_bytes (+ rows*2 residual).
#include "launch.h"
#include "q4k_device.h"
#include "rxq4.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace rxq4 {

// The 64 activations of one slot, as fp16 pairs in nibble order, plus sums.
struct XSlot {
    uint32_t p[32];
    float bias_lo, bias_hi;  // -1024 * sum
    float sx_lo, sx_hi;      // sum of the 32 low-nibble / high-nibble activations
};

// The slot (b, il) of x: elements b*256 + 64*il + [0, 64), as 8 x 16 bytes
// (low-nibble half first).
__device__ __forceinline__ void load_x_raw(const uint16_t *__restrict__ x, int b, int il,
                                           u32x4 raw[8]) {
    const uint16_t *base = x + b * kQK + 64 * il;
#pragma unroll
    for (int i = 0; i < 8; ++i) raw[i] = load16(base + 8 * i);
}

// Permute a raw slot into pairs and sums.  For quant dword k (bytes 4k..4k+3
// of the group) the pairs are
//   p[4k+0] = (x_lo[4k],   x_lo[4k+2])   p[4k+1] = (x_lo[4k+1], x_lo[4k+3])
//   p[4k+2] = (x_hi[4k],   x_hi[4k+2])   p[4k+3] = (x_hi[4k+1], x_hi[4k+3])
// matching (q & 0x000F000F) and ((q >> 8) & 0x000F000F) (and 0x00F000F0).
// Pairs are byte permutes; the sums are dot products with (1, 1) (exact
// products, fp32 accumulation).
__device__ __forceinline__ void x_slot_from_raw(const u32x4 raw[8], XSlot &s) {
    uint32_t xl[16], xh[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 lo = raw[i], hi = raw[4 + i];
        xl[4 * i + 0] = lo.x; xl[4 * i + 1] = lo.y; xl[4 * i + 2] = lo.z; xl[4 * i + 3] = lo.w;
        xh[4 * i + 0] = hi.x; xh[4 * i + 1] = hi.y; xh[4 * i + 2] = hi.z; xh[4 * i + 3] = hi.w;
    }
    const half2_t ones = as_half2(0x3C003C00u);
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        s.p[4 * k + 0] = __builtin_amdgcn_perm(xl[2 * k + 1], xl[2 * k], 0x05040100u);
        s.p[4 * k + 1] = __builtin_amdgcn_perm(xl[2 * k + 1], xl[2 * k], 0x07060302u);
        s.p[4 * k + 2] = __builtin_amdgcn_perm(xh[2 * k + 1], xh[2 * k], 0x05040100u);
        s.p[4 * k + 3] = __builtin_amdgcn_perm(xh[2 * k + 1], xh[2 * k], 0x07060302u);
        sl = __builtin_amdgcn_fdot2(as_half2(xl[2 * k]), ones, sl, false);
        sh = __builtin_amdgcn_fdot2(as_half2(xh[2 * k]), ones, sh, false);
        sl = __builtin_amdgcn_fdot2(as_half2(xl[2 * k + 1]), ones, sl, false);
        sh = __builtin_amdgcn_fdot2(as_half2(xh[2 * k + 1]), ones, sh, false);
    }
    s.sx_lo = sl;
    s.sx_hi = sh;
    s.bias_lo = -1024.0f * sl;
    s.bias_hi = -1024.0f * sh;
}

// Lane-constant parts of the scale decode for quant group il.  With
// s0/s1/s2 the scale dwords (bytes 0-3, 4-7, 8-11 of the 12 scale bytes) and
// h = 16*(il & 1):
//   il < 2:  sc = (s0 >> h) & 0x3F3F,  m = (s1 >> h) & 0x3F3F
//   il >= 2: sc = (s2 >> h) & 0x0F0F | (s0 >> (h+2)) & 0x3030,
//            m  = (s2 >> (h+4)) & 0x0F0F | (s1 >> (h+2)) & 0x3030
// i.e. sc = (s0 >> shA) & mA | (s2 >> h) & mC, m = (s1 >> shA) & mA |
// (s2 >> (h+4)) & mC with the constants below; byte 0 / byte 1 of sc, m are
// the pairs of sub-blocks 2*il and 2*il+1 (get_scale_min_k4, q4_gemm.cu:192-202).
struct ScaleDecode {
    uint32_t shA, shC, shC4, mA, mC;
};

__device__ __forceinline__ ScaleDecode scale_decode_for(int il) {
    const uint32_t h = (uint32_t)(il & 1) << 4;
    const bool upper = il >= 2;
    return ScaleDecode{h + (upper ? 2u : 0u), h, h + 4u, upper ? 0x3030u : 0x3F3Fu,
                       upper ? 0x0F0Fu : 0u};
}

// v_and_or_b32 with the mask in an SGPR and the magic in a VGPR (a VOP3 may
// read one scalar operand, so the compiler cannot fuse two literal constants).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(magic));
    return r;
}

// Raw dot products of one quant group (32 bytes q0, q1) with its slot of x:
// acc_lo += sum (1024 + q_lo) x_lo, acc_hi += sum (1024 + 16 q_hi) x_hi.
__device__ __forceinline__ void group_dot(u32x4 q0, u32x4 q1, const XSlot &s, uint32_t magic,
                                          float &acc_lo, float &acc_hi) {
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        // the four pairs first: a dot product right behind the VALU op that
        // wrote its operand costs a wait state on gfx950
        const uint32_t v = q[k], v8 = q[k] >> 8;
        const uint32_t w0 = and_or(v, 0x000F000Fu, magic);
        const uint32_t w1 = and_or(v8, 0x000F000Fu, magic);
        const uint32_t w2 = and_or(v, 0x00F000F0u, magic);
        const uint32_t w3 = and_or(v8, 0x00F000F0u, magic);
        acc_lo = __builtin_amdgcn_fdot2(as_half2(w0), as_half2(s.p[4 * k + 0]), acc_lo, false);
        acc_hi = __builtin_amdgcn_fdot2(as_half2(w2), as_half2(s.p[4 * k + 2]), acc_hi, false);
        acc_lo = __builtin_amdgcn_fdot2(as_half2(w1), as_half2(s.p[4 * k + 1]), acc_lo, false);
        acc_hi = __builtin_amdgcn_fdot2(as_half2(w3), as_half2(s.p[4 * k + 3]), acc_hi, false);
    }
}

// group_dot for NT tokens: the nibble pairs are formed once and multiplied
// into every token's accumulators.
template <int NT>
__device__ __forceinline__ void group_dot_nt(u32x4 q0, u32x4 q1, const XSlot *s, uint32_t magic,
                                             float *acc_lo, float *acc_hi) {
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = q[k], v8 = q[k] >> 8;
        const uint32_t w0 = and_or(v, 0x000F000Fu, magic);
        const uint32_t w1 = and_or(v8, 0x000F000Fu, magic);
        const uint32_t w2 = and_or(v, 0x00F000F0u, magic);
        const uint32_t w3 = and_or(v8, 0x00F000F0u, magic);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            acc_lo[t] = __builtin_amdgcn_fdot2(as_half2(w0), as_half2(s[t].p[4 * k + 0]), acc_lo[t], false);
            acc_hi[t] = __builtin_amdgcn_fdot2(as_half2(w2), as_half2(s[t].p[4 * k + 2]), acc_hi[t], false);
            acc_lo[t] = __builtin_amdgcn_fdot2(as_half2(w1), as_half2(s[t].p[4 * k + 1]), acc_lo[t], false);
            acc_hi[t] = __builtin_amdgcn_fdot2(as_half2(w3), as_half2(s[t].p[4 * k + 3]), acc_hi[t], false);
        }
    }
}

// Partial dot products of one slot of one row with NT tokens' activations.
template <int NT>
__device__ __forceinline__ void slot_dot_nt(u32x4 hdr, u32x4 q0, u32x4 q1, const XSlot *s,
                                            const ScaleDecode &sd, uint32_t magic, float *out) {
    const float d = f16_bits_to_f32(hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    const uint32_t sc = ((hdr.y >> sd.shA) & sd.mA) | ((hdr.w >> sd.shC) & sd.mC);
    const uint32_t mn = ((hdr.z >> sd.shA) & sd.mA) | ((hdr.w >> sd.shC4) & sd.mC);
    float acc_lo[NT], acc_hi[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc_lo[t] = s[t].bias_lo;
        acc_hi[t] = s[t].bias_hi;
    }
    group_dot_nt<NT>(q0, q1, s, magic, acc_lo, acc_hi);
    const float d_lo = d * (float)(sc & 0xFFu);
    const float d_hi = (d * 0.0625f) * (float)((sc >> 8) & 0xFFu);
    const float m_lo = dmin * (float)(mn & 0xFFu);
    const float m_hi = dmin * (float)((mn >> 8) & 0xFFu);
#pragma unroll
    for (int t = 0; t < NT; ++t)
        out[t] = d_lo * acc_lo[t] - m_lo * s[t].sx_lo + (d_hi * acc_hi[t] - m_hi * s[t].sx_hi);
}

// Partial dot product of one slot of one row.
__device__ __forceinline__ float slot_dot(u32x4 hdr, u32x4 q0, u32x4 q1, const XSlot &s,
                                          const ScaleDecode &sd, uint32_t magic) {
    const float d = f16_bits_to_f32(hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    const uint32_t sc = ((hdr.y >> sd.shA) & sd.mA) | ((hdr.w >> sd.shC) & sd.mC);
    const uint32_t mn = ((hdr.z >> sd.shA) & sd.mA) | ((hdr.w >> sd.shC4) & sd.mC);
    float acc_lo = s.bias_lo, acc_hi = s.bias_hi;
    group_dot(q0, q1, s, magic, acc_lo, acc_hi);
    const float d_lo = d * (float)(sc & 0xFFu);
    const float d_hi = (d * 0.0625f) * (float)((sc >> 8) & 0xFFu);
    const float m_lo = dmin * (float)(mn & 0xFFu);
    const float m_hi = dmin * (float)((mn >> 8) & 0xFFu);
    return d_lo * acc_lo - m_lo * s.sx_lo + (d_hi * acc_hi - m_hi * s.sx_hi);
}

// DPP control words (GFX9): quad_perm = 0x00-0xFF, row_ror:n = 0x120 + n,
// row_half_mirror = 0x141, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                  0xF, false);
    return v + __builtin_bit_cast(float, moved);
}

// Sum over aligned groups of W lanes (W in {2, 4, 8, 16, 32, 64}).  The full
// sum is valid in lane W-1 of every group (and in every lane of the group for
// W <= 16).
template <int W>
__device__ __forceinline__ float lane_group_sum(float v) {
    if (W >= 16) {
        v = dpp_add<0x128, 0xF>(v);  // row_ror:8
        v = dpp_add<0x124, 0xF>(v);  // row_ror:4
        v = dpp_add<0x122, 0xF>(v);  // row_ror:2
        v = dpp_add<0x121, 0xF>(v);  // row_ror:1
        if (W >= 32) v = dpp_add<0x142, 0xA>(v);  // rows 1, 3 += last lane of rows 0, 2
        if (W >= 64) v = dpp_add<0x143, 0xC>(v);  // rows 2, 3 += lane 31
    } else {
        v = dpp_add<0xB1, 0xF>(v);                // quad_perm [1,0,3,2]
        if (W >= 4) v = dpp_add<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
        if (W >= 8) v = dpp_add<0x141, 0xF>(v);   // row_half_mirror
    }
    return v;
}

// One output range, copied out of the kernel parameter block field by field
// so that picking a range is a scalar select, never an indexed load from a
// stack copy of the parameters.
struct Range {
    const uint8_t *w;
    void *y;
    const uint16_t *res;
    int rows;
    int first_unit;
    int n_units;
};

__device__ __forceinline__ Range range_of_unit(const GemvParams &p, int unit) {
    const uint8_t *w0 = p.r[0].w, *w1 = p.r[1].w, *w2 = p.r[2].w;
    void *y0 = p.r[0].y, *y1 = p.r[1].y, *y2 = p.r[2].y;
    const uint16_t *r0 = p.r[0].res, *r1 = p.r[1].res, *r2 = p.r[2].res;
    const int m0 = p.r[0].rows, m1 = p.r[1].rows, m2 = p.r[2].rows;
    const int u1 = p.unit_start[1], u2 = p.unit_start[2];
    const int ri = (p.n_ranges > 1 && unit >= u1) ? ((p.n_ranges > 2 && unit >= u2) ? 2 : 1) : 0;
    Range r;
    r.w = ri == 0 ? w0 : (ri == 1 ? w1 : w2);
    r.y = ri == 0 ? y0 : (ri == 1 ? y1 : y2);
    r.res = ri == 0 ? r0 : (ri == 1 ? r1 : r2);
    r.rows = ri == 0 ? m0 : (ri == 1 ? m1 : m2);
    r.first_unit = ri == 0 ? 0 : (ri == 1 ? u1 : u2);
    r.n_units = (ri == 0 ? u1 : (ri == 1 ? u2 : p.total_units)) - r.first_unit;
    return r;
}

// `res` is the fp16 residual of the row (kEpiAdd), loaded with the weights;
// `yoff` the output offset of the token (multi-token calls).
template <int EPI>
__device__ __forceinline__ void store_row(const Range &r, int row, float v, uint32_t res,
                                          int64_t yoff = 0) {
    if (EPI == kEpiF32) {
        static_cast<float *>(r.y)[yoff + row] = v;
    } else if (EPI == kEpiF16) {
        static_cast<uint16_t *>(r.y)[yoff + row] = f32_to_f16_bits(v);
    } else {
        // q4_gemm.cu:774-777: round the projection, add the residual, round.
        const float projected = f16_bits_to_f32(f32_to_f16_bits(v));
        static_cast<uint16_t *>(r.y)[row] = f32_to_f16_bits(projected + f16_bits_to_f32(res));
    }
}

__device__ __forceinline__ uint32_t magic_vgpr() {
    uint32_t m;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
    return m;
}

// U items of weights in flight: header, the slot's 32 quant bytes and, for
// kEpiAdd, the fp16 residual of the item's row.
template <int U>
struct Batch {
    u32x4 h[U], a[U], c[U];
    uint32_t r[U];
};

// ---------------------------------------------------------------------------
// Register kernel: a lane owns one slot (64 weights: quant group il of block
// b) of a row; a row has LPR = 4*nb <= 64 slots (nb in {1,2,4,8,16}), so a
// wave covers RPS = 64/LPR rows per step and each lane's slot never changes;
// its 64 activations stay in VGPRs.  Wave w serves the contiguous steps
// [t0, t1) of one range, at most 256 rows (per_unit * RPS <= 256).
//   * x (K <= 4096 fp16) is copied into LDS once per workgroup with one
//     direct-to-LDS load per thread and round, ahead of the weights; each
//     lane then reads its slot from LDS.
//   * Two batches of U steps are issued right behind x, so a wave with at
//     most 2U steps makes a single memory round trip; longer waves refill
//     each buffer as soon as it has been consumed.
//   * Row results collect in LDS and leave in coalesced stores of 64 rows;
//     the residuals (kEpiAdd) of the first 64 were fetched up front.
constexpr int kRegMaxK = 4096;
constexpr int kRegMaxRows = 256;

template <int LPR, int EPI, int U, int NT>
__global__ __launch_bounds__(256) void gemv_reg_kernel(GemvParams p) {
    constexpr int RPS = 64 / LPR;
    __shared__ __attribute__((aligned(16))) uint16_t xsh[NT][kRegMaxK];
    __shared__ float outs[NT][4][kRegMaxRows];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = blockIdx.x * 4 + wv;
    const bool active = wave < p.total_units;
    const Range rg = range_of_unit(p, active ? wave : 0);
    const int n_steps = (rg.rows + RPS - 1) / RPS;
    const int t0 = active ? (wave - rg.first_unit) * p.per_unit : 0;
    const int t1 = active ? min(t0 + p.per_unit, n_steps) : 0;
    const int row0 = t0 * RPS;
    const int last = rg.rows - 1;

    const int slot = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int b = slot >> 2, il = slot & 3;
    const uint32_t row_bytes = (uint32_t)p.nb * kBlockBytes;
    const uint32_t hdr_off = (uint32_t)b * kBlockBytes;
    const uint32_t q_off = hdr_off + 16u + 32u * (uint32_t)il;

    // x -> LDS: chunk c (16 bytes) of thread c + 256*round, per token;
    // chunks past K read the next token's x or, past the last, zeros (the
    // staged positions past K are never read).
    const int x_bytes = p.nb * kQK * 2;
    const __amdgpu_buffer_rsrc_t xrsrc = make_rsrc(p.x, NT * x_bytes);
    constexpr int kXRounds = (RPS == 1) ? 2 : 1;  // K = 4096 only with LPR = 64
#pragma unroll
    for (int tk = 0; tk < NT; ++tk)
#pragma unroll
        for (int r = 0; r < kXRounds; ++r)
            buffer_to_lds16(xrsrc, &xsh[tk][(256 * r + 64 * wv) * 8],
                            tk * x_bytes + (256 * r + tid) * 16);
    __builtin_amdgcn_sched_barrier(0);  // the counted loads below stay behind the copies

    // Weights.  Steps past t1 reload step t1-1 (inactive waves: step 0; L2
    // hits, results discarded): the loads stay unconditional, so the
    // compiler's vmcnt waits count them exactly.
    auto load = [&](int t, Batch<U> &bt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ts = max(0, min(t0 + t + u, t1 - 1));
            // uniform part: first row of the step; lane part: sub-row, clamped
            const uint8_t *base = rg.w + (int64_t)(ts * RPS) * row_bytes;
            const uint32_t lrow = (uint32_t)min(sub, last - ts * RPS) * row_bytes;
            bt.h[u] = load16(base + (lrow + hdr_off));
            bt.a[u] = load16(base + (lrow + q_off));
            bt.c[u] = load16(base + (lrow + q_off + 16u));
        }
    };
    Batch<U> A, B;
    load(0, A);
    load(U, B);
    // residual of row row0 + lane (kEpiAdd)
    uint32_t res = 0;
    if (EPI == kEpiAdd) res = rg.res[min(row0 + lane, last)];
    constexpr int kWeightLoads = 2 * U * 3 + (EPI == kEpiAdd ? 1 : 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kWeightLoads>();  // this wave's x copies have landed
    lds_barrier();               // ... and every other wave's

    XSlot xs[NT];
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) {
        u32x4 xraw[8];
        const u32x4 *xs16 = reinterpret_cast<const u32x4 *>(xsh[tk]) + b * 32 + il * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) xraw[i] = xs16[i];
        x_slot_from_raw(xraw, xs[tk]);
    }
    const ScaleDecode sd = scale_decode_for(il);
    const uint32_t magic = magic_vgpr();
    const int n = t1 - t0;
    auto compute = [&](int t, const Batch<U> &bt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (t + u < n) {  // uniform
                float v[NT];
                if (NT == 1)
                    v[0] = slot_dot(bt.h[u], bt.a[u], bt.c[u], xs[0], sd, magic);
                else
                    slot_dot_nt<NT>(bt.h[u], bt.a[u], bt.c[u], xs, sd, magic, v);
#pragma unroll
                for (int tk = 0; tk < NT; ++tk) {
                    const float r = lane_group_sum<LPR>(v[tk]);
                    if (slot == LPR - 1) outs[tk][wv][(t + u) * RPS + sub] = r;
                }
            }
        }
    };

    // Steady state: A holds steps [t, t+U), B [t+U, t+2U), both in flight;
    // each is refilled right after it has been consumed.  The refills are
    // unconditional, so the loop entry and back edge have the same loads
    // outstanding in the same order (exact vmcnt waits).  The tail computes
    // the last <= 2U steps with no loads behind them.
    int t = 0;
    for (; t + 2 * U < n; t += 2 * U) {
        compute(t, A);
        load(t + 2 * U, A);
        compute(t + U, B);
        load(t + 3 * U, B);
    }
    compute(t, A);
    compute(t + U, B);

    // Coalesced stores of the wave's rows (same-wave LDS traffic is in
    // order, so the results written above are visible here).
    const int rows = min(n * RPS, rg.rows - row0);
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) {
        const int64_t yoff = (int64_t)tk * p.y_stride;
        if (lane < rows) store_row<EPI>(rg, row0 + lane, outs[tk][wv][lane], res, yoff);
        for (int r = 64; r < rows; r += 64) {
            const int row = row0 + r + lane;
            if (r + lane < rows)
                store_row<EPI>(rg, row, outs[tk][wv][r + lane], EPI == kEpiAdd ? rg.res[row] : 0u,
                               yoff);
        }
    }
}

// ---------------------------------------------------------------------------
// Streamed register kernel (one token, the register kernel's lane mapping
// and arithmetic).  A step of a wave is 64 slots = 16 blocks = 2304
// contiguous bytes, and a wave's steps are contiguous, so a group of G steps
// arrives by ceil(G * 2304 / 1024) direct-to-LDS 16-byte loads per lane,
// each covering up to 1 KB contiguous (whole 128-byte lines, marked
// nontemporal), into a per-wave ring of NBUF group buffers in LDS; each lane
// then reads its slot's header and quants from there.  Loads past the group,
// past the wave's last step or past the range take an offset beyond the
// buffer resource (no memory access, zeros into LDS), so a wave reads
// exactly its own rows and every load is issued unconditionally (exact
// vmcnt waits).  Against the register kernel (graph replay, alternating
// runs on one box, identical outputs):
//   * waves of 32 steps or more (the LM head [151936 x 2048], 74 steps):
//     3-step groups x 2 buffers, 33.5 -> 30.1-30.5 us; 2 x 3 30.2-30.6,
//     2 x 4 or 4 x 2 (18 KB in flight) 31.0-31.4, 2 x 2 31.4-32.0, 1-step
//     groups 32.0-33.0; without the nontemporal bit 35.2-35.5; with 8 waves
//     per CU 31.2-31.4; groups dealt round-robin over the range's waves
//     (rows stored per step) 35.6-37.2.  With the next group's LDS reads
//     issued before this group's arithmetic (below), 1-step groups x 5
//     buffers against 3 x 2: LM head 30.1-30.2 -> 28.9-29.8, [151936 x
//     1024] 16.9 -> 16.5-16.6, [65536 x 2048] 14.8 -> 14.4, [100000 x 2048]
//     add 21.2-21.4 -> 20.7-20.8 us (1 x 4 / 1 x 6 / 2 x 4 / 2 x 5: LM head
//     30.1 / 29.4-29.8 / 30.3-30.6 / 30.6-30.9);
//   * shorter waves: 1-step groups x 3 buffers, QKV triple 3.36 -> 2.82,
//     O add 3.19 -> 2.60, gate+up pair 6.85 -> 6.59 us (x 2 buffers: 2.79,
//     2.57, 7.70; 1 x 4: 2.87, 2.71, 6.54; 3 x 2: gate+up 7.2; 6 or 8
//     waves per CU slower on QKV);
//   * of those, waves of 4 steps or more (gate+up: 11) issue the next
//     group's LDS reads before this group's arithmetic, with 4 buffers:
//     gate+up 6.55-6.86 -> 6.26-6.28 us; with 3 buffers 6.91-6.96; QKV (2
//     steps) and O (1) ran slower with it (2.92 / 2.71-2.76).
constexpr int kStepBytes = 64 * 36;
// waves of at least this many steps take the long-group configuration
constexpr int kStreamMinSteps = 32;
constexpr int kStreamLongSteps = 1, kStreamLongBufs = 5;
constexpr int kStreamShortSteps = 1, kStreamShortBufs = 3;
// waves of kStreamMidSteps .. kStreamMinSteps-1 steps: 1-step groups x 4
// buffers, the next group's LDS reads issued before this group's arithmetic
constexpr int kStreamMidSteps = 4;
constexpr int kStreamMidBufs = 4;

template <int G>
struct StreamGeometry {
    static constexpr int kGroupBytes = G * kStepBytes;
    static constexpr int kLoads = (kGroupBytes + 1023) / 1024;
    static constexpr int kBufBytes = kLoads * 1024;  // a group's LDS buffer
};
// dynamic LDS per workgroup (4 waves)
template <int G, int NBUF>
constexpr size_t stream_lds() {
    return (size_t)4 * NBUF * StreamGeometry<G>::kBufBytes;
}

// f(integral_constant<int, I>) for I = B .. E-1, unrolled.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

template <int LPR, int EPI, int G, int NBUF, int NT, bool PF>
__global__ __launch_bounds__(256) void gemv_stream_kernel(GemvParams p) {
    constexpr int RPS = 64 / LPR;
    constexpr int kStreamSteps = G;
    constexpr int kStreamGroupBytes = StreamGeometry<G>::kGroupBytes;
    constexpr int kStreamLoads = StreamGeometry<G>::kLoads;
    constexpr int kStreamBufBytes = StreamGeometry<G>::kBufBytes;
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    __shared__ __attribute__((aligned(16))) uint16_t xsh[NT][kRegMaxK];
    __shared__ float outs[NT][4][kRegMaxRows];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = blockIdx.x * 4 + wv;
    const bool active = wave < p.total_units;
    const Range rg = range_of_unit(p, active ? wave : 0);
    const int n_steps = (rg.rows + RPS - 1) / RPS;
    const int t0 = active ? (wave - rg.first_unit) * p.per_unit : 0;
    const int t1 = active ? min(t0 + p.per_unit, n_steps) : 0;
    const int row0 = t0 * RPS;
    const int last = rg.rows - 1;
    const int slot = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int il = slot & 3;
    const int b = slot >> 2;

    // x of NT tokens (token tk at x + tk * K) -> LDS, as the register kernel
    const int x_bytes = p.nb * kQK * 2;
    const __amdgpu_buffer_rsrc_t xrsrc = make_rsrc(p.x, NT * x_bytes);
    constexpr int kXRounds = (RPS == 1) ? 2 : 1;
#pragma unroll
    for (int tk = 0; tk < NT; ++tk)
#pragma unroll
        for (int r = 0; r < kXRounds; ++r)
            buffer_to_lds16(xrsrc, &xsh[tk][(256 * r + 64 * wv) * 8], tk * x_bytes + (256 * r + tid) * 16);
    uint32_t res = 0;
    if (EPI == kEpiAdd) res = rg.res[min(row0 + lane, last)];
    __builtin_amdgcn_sched_barrier(0);

    // The range's bytes (the host checks that they fit a buffer resource);
    // the wave's own bytes end at step t1.
    const uint32_t row_bytes = (uint32_t)p.nb * kBlockBytes;
    const __amdgpu_buffer_rsrc_t wrsrc = make_rsrc(rg.w, (int)((uint32_t)rg.rows * row_bytes));
    const int end = t1 * kStepBytes;
    uint8_t *my = ring + wv * (NBUF * kStreamBufBytes);
    const int n = t1 - t0;
    const int n_groups = (n + kStreamSteps - 1) / kStreamSteps;
    auto load = [&](int g, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kStreamLoads; ++j) {
            const int off = (t0 * kStepBytes + g * kStreamGroupBytes) + j * 1024 + lane * 16;
            const bool mine = j * 1024 + lane * 16 < kStreamGroupBytes && off < end;
            buffer_to_lds16_nt(wrsrc, my + buf * kStreamBufBytes + j * 1024,
                               mine ? off : 0x7FFFFFF0);
        }
    };
#pragma unroll
    for (int i = 0; i < NBUF; ++i) load(i, i);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<NBUF * kStreamLoads>();  // this wave's x copies (and residual) have landed
    lds_barrier();                      // ... and every other wave's

    XSlot xs[NT];
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) {
        u32x4 xraw[8];
        const u32x4 *xs16 = reinterpret_cast<const u32x4 *>(xsh[tk]) + b * 32 + il * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) xraw[i] = xs16[i];
        x_slot_from_raw(xraw, xs[tk]);
    }
    const ScaleDecode sd = scale_decode_for(il);
    const uint32_t magic = magic_vgpr();
    // lane's slot in a step: block lane / 4 of the step, quant group lane & 3
    const int hdr_lds = (lane >> 2) * kBlockBytes;
    const int q_lds = hdr_lds + 16 + 32 * (lane & 3);
    // A group's LDS reads (3 per step), then its steps; `full` groups (all
    // steps the wave's) skip the per-step test.
    struct GroupRegs {
        u32x4 h[kStreamSteps], q0[kStreamSteps], q1[kStreamSteps];
    };
    auto read = [&](int buf, GroupRegs &R) __attribute__((always_inline)) {
        const uint8_t *gb = my + buf * kStreamBufBytes;
#pragma unroll
        for (int s = 0; s < kStreamSteps; ++s) {
            const uint8_t *sb = gb + s * kStepBytes;
            R.h[s] = *reinterpret_cast<const u32x4 *>(sb + hdr_lds);
            R.q0[s] = *reinterpret_cast<const u32x4 *>(sb + q_lds);
            R.q1[s] = *reinterpret_cast<const u32x4 *>(sb + q_lds + 16);
        }
    };
    auto compute = [&](int g, const GroupRegs &R, auto full) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < kStreamSteps; ++s) {
            const int t = g * kStreamSteps + s;
            if (decltype(full)::value || t < n) {  // uniform
                float v[NT];
                if (NT == 1)
                    v[0] = slot_dot(R.h[s], R.q0[s], R.q1[s], xs[0], sd, magic);
                else
                    slot_dot_nt<NT>(R.h[s], R.q0[s], R.q1[s], xs, sd, magic, v);
#pragma unroll
                for (int tk = 0; tk < NT; ++tk) {
                    const float r = lane_group_sum<LPR>(v[tk]);
                    if (slot == LPR - 1) outs[tk][wv][t * RPS + sub] = r;
                }
            }
        }
    };
    using Full = std::integral_constant<bool, true>;
    using Tail = std::integral_constant<bool, false>;

    int g = 0;
    if constexpr (!PF) {
        // Steady state: groups g .. g+NBUF-1 in flight, group g+i in buffer
        // i; each buffer is refilled once its group has been read (the
        // reads' values are used before the refill is issued).  The tail
        // computes the last NBUF groups with no loads behind them.
        for (; g + NBUF < n_groups; g += NBUF) {
            static_for<0, NBUF>([&](auto i) __attribute__((always_inline)) {
                constexpr int I = decltype(i)::value;
                wait_vmcnt<(NBUF - 1) * kStreamLoads>();
                GroupRegs R;
                read(I, R);
                compute(g + I, R, Full{});
                __builtin_amdgcn_sched_barrier(0);
                load(g + I + NBUF, I);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        static_for<0, NBUF>([&](auto i) __attribute__((always_inline)) {
            constexpr int I = decltype(i)::value;
            wait_vmcnt<(NBUF - 1 - I) * kStreamLoads>();
            GroupRegs R;
            read(I, R);
            compute(g + I, R, Tail{});
        });
    } else {
        // The same, with the next group's LDS reads issued before this
        // group's arithmetic (the LDS latency hides behind it): before
        // group g+i is computed, group g+i+1 must have landed, so
        // NBUF-2 groups are in flight during the arithmetic.
        static_assert(NBUF >= 3, "a group in flight behind the prefetched one");
        GroupRegs cur;
        wait_vmcnt<(NBUF - 1) * kStreamLoads>();
        read(0, cur);
        for (; g + NBUF < n_groups; g += NBUF) {
            static_for<0, NBUF>([&](auto i) __attribute__((always_inline)) {
                constexpr int I = decltype(i)::value;
                wait_vmcnt<(NBUF - 2) * kStreamLoads>();
                GroupRegs nxt;
                read((I + 1) % NBUF, nxt);
                compute(g + I, cur, Full{});
                __builtin_amdgcn_sched_barrier(0);
                load(g + I + NBUF, I);
                __builtin_amdgcn_sched_barrier(0);
                cur = nxt;
            });
        }
        static_for<0, NBUF>([&](auto i) __attribute__((always_inline)) {
            constexpr int I = decltype(i)::value;
            GroupRegs nxt;
            if constexpr (I + 1 < NBUF) {
                wait_vmcnt<(NBUF - 2 - I) * kStreamLoads>();
                read(I + 1, nxt);
            }
            compute(g + I, cur, Tail{});
            if constexpr (I + 1 < NBUF) cur = nxt;
        });
    }

    const int rows = min(n * RPS, rg.rows - row0);
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) {
        const int64_t yoff = (int64_t)tk * p.y_stride;
        if (lane < rows) store_row<EPI>(rg, row0 + lane, outs[tk][wv][lane], res, yoff);
        for (int r = 64; r < rows; r += 64) {
            const int row = row0 + r + lane;
            if (r + lane < rows)
                store_row<EPI>(rg, row, outs[tk][wv][r + lane], EPI == kEpiAdd ? rg.res[row] : 0u, yoff);
        }
    }
}

// ---------------------------------------------------------------------------
// LDS kernel for rows with more than 64 slots (any K): the workgroup stages
// x once in LDS in the same permuted-pair layout (36 dwords per slot), and
// each wave owns whole rows, walking a row's slots 64 at a time
// (J = ceil(4*nb/64) items per row).  Two batches of U items (and the
// residuals of their rows) are issued right after the first round of x
// loads, so the staging overlaps the weight round trip; each buffer is
// refilled as soon as it has been consumed.  The row's lanes are summed once per row.  No
// barrier after the staging barrier.
constexpr int kLdsSlotWords = 36;
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int EPI, int U, int NT>
__global__ __launch_bounds__(256) void gemv_lds_kernel(GemvParams p) {
    extern __shared__ uint32_t xlds[];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_slots = 4 * p.nb;
    const int J = (n_slots + 63) >> 6;
    const int wave = blockIdx.x * 4 + wv;
    const bool active = wave < p.total_units;
    const Range rg = range_of_unit(p, active ? wave : 0);
    const int r0 = (wave - rg.first_unit) * p.per_unit;
    const int r1 = active ? min(r0 + p.per_unit, rg.rows) : r0;
    const int n_items = (r1 > r0 ? r1 - r0 : 0) * J;
    const uint32_t row_bytes = (uint32_t)p.nb * kBlockBytes;

    // Items are walked in order by two cursors (loads run up to two batches
    // ahead of the arithmetic): item (row, j) covers slots [64j, 64j+64).
    // Items past the end reload the last row (inactive waves: row 0 of the
    // range) and are discarded: the loads stay unconditional, so the
    // compiler's vmcnt waits count them exactly.
    int ld_row = r0, ld_j = 0;
    auto load = [&](Batch<U> &bt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = max(0, min(ld_row, r1 - 1));
            const int slot = min(64 * ld_j + lane, n_slots - 1);
            const uint8_t *blk = rg.w + (int64_t)row * row_bytes + (slot >> 2) * kBlockBytes;
            bt.h[u] = load16(blk);
            bt.a[u] = load16(blk + 16 + 32 * (slot & 3));
            bt.c[u] = load16(blk + 32 + 32 * (slot & 3));
            if (EPI == kEpiAdd) bt.r[u] = rg.res[row];
            if (++ld_j == J) { ld_j = 0; ++ld_row; }
        }
    };
    // Stage x, one slot per thread and round (token tk's slots follow token
    // tk - 1's); the first round's loads go out before the weights (vector
    // loads complete in order).
    const int K = 256 * p.nb;
    auto stage = [&](int s, const u32x4 raw[8]) {
        XSlot xs;
        x_slot_from_raw(raw, xs);
        uint32_t *dst = xlds + s * kLdsSlotWords;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            *reinterpret_cast<u32x4 *>(dst + 4 * k) =
                u32x4{xs.p[4 * k], xs.p[4 * k + 1], xs.p[4 * k + 2], xs.p[4 * k + 3]};
        *reinterpret_cast<f32x4v *>(dst + 32) = f32x4v{xs.bias_lo, xs.bias_hi, xs.sx_lo, xs.sx_hi};
    };
    const int s_first = threadIdx.x;
    const int s_load = min(s_first, n_slots - 1);
    u32x4 xraw[NT][8];
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) load_x_raw(p.x + (int64_t)tk * K, s_load >> 2, s_load & 3, xraw[tk]);
    __builtin_amdgcn_sched_barrier(0);
    Batch<U> A, B;
    load(A);
    load(B);
    __builtin_amdgcn_sched_barrier(0);
    if (s_first < n_slots) {
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) stage(tk * n_slots + s_first, xraw[tk]);
    }
    for (int s = s_first + blockDim.x; s < n_slots; s += blockDim.x) {
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) {
            load_x_raw(p.x + (int64_t)tk * K, s >> 2, s & 3, xraw[0]);
            stage(tk * n_slots + s, xraw[0]);
        }
    }
    __syncthreads();
    if (n_items == 0) return;

    const uint32_t magic = magic_vgpr();
    float acc[NT];
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) acc[tk] = 0.0f;
    int cp_item = 0, cp_row = r0, cp_j = 0;
    auto compute = [&](const Batch<U> &bt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (cp_item < n_items) {  // uniform
                const int slot = 64 * cp_j + lane;
                const bool valid = slot < n_slots;
                const int sl = valid ? slot : 0;
                XSlot xs[NT];
#pragma unroll
                for (int tk = 0; tk < NT; ++tk) {
                    const uint32_t *src = xlds + (tk * n_slots + sl) * kLdsSlotWords;
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const u32x4 v = *reinterpret_cast<const u32x4 *>(src + 4 * k);
                        xs[tk].p[4 * k] = v.x; xs[tk].p[4 * k + 1] = v.y;
                        xs[tk].p[4 * k + 2] = v.z; xs[tk].p[4 * k + 3] = v.w;
                    }
                    const f32x4v t = *reinterpret_cast<const f32x4v *>(src + 32);
                    xs[tk].bias_lo = t[0];
                    xs[tk].bias_hi = t[1];
                    xs[tk].sx_lo = t[2];
                    xs[tk].sx_hi = t[3];
                }
                const ScaleDecode sd = scale_decode_for(sl & 3);
                float v[NT];
                if (NT == 1)
                    v[0] = slot_dot(bt.h[u], bt.a[u], bt.c[u], xs[0], sd, magic);
                else
                    slot_dot_nt<NT>(bt.h[u], bt.a[u], bt.c[u], xs, sd, magic, v);
#pragma unroll
                for (int tk = 0; tk < NT; ++tk) acc[tk] += valid ? v[tk] : 0.0f;
                ++cp_item;
                if (++cp_j == J) {
#pragma unroll
                    for (int tk = 0; tk < NT; ++tk) {
                        const float total = lane_group_sum<64>(acc[tk]);
                        if (lane == 63)
                            store_row<EPI>(rg, cp_row, total, bt.r[u], (int64_t)tk * p.y_stride);
                        acc[tk] = 0.0f;
                    }
                    cp_j = 0;
                    ++cp_row;
                }
            }
        }
    };
    // Steady state with unconditional refills, then the last <= 2U items
    // (the register kernel's scheme: exact vmcnt waits).
    int i = 0;
    for (; i + 2 * U < n_items; i += 2 * U) {
        compute(A);
        load(A);
        compute(B);
        load(B);
    }
    compute(A);
    compute(B);
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 16].
__device__ __forceinline__ void wait_vmcnt_upto16(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 7: wait_vmcnt<7>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;
        case 10: wait_vmcnt<10>(); break;
        case 11: wait_vmcnt<11>(); break;
        case 12: wait_vmcnt<12>(); break;
        case 13: wait_vmcnt<13>(); break;
        case 14: wait_vmcnt<14>(); break;
        case 15: wait_vmcnt<15>(); break;
        default: wait_vmcnt<16>(); break;
    }
}

// ---------------------------------------------------------------------------
// Streamed LDS kernel (one token, rows of more than 64 slots, the LDS
// kernel's lane mapping and arithmetic), for waves whose rows fit 16 KB
// (down [2048 x 11008]: 2 rows of 6192 B).  A wave's rows are contiguous,
// so all of its weight bytes arrive by 16 unconditional direct-to-LDS
// 16-byte loads per lane (each covering 1 KB contiguous, marked
// nontemporal; loads past the wave's rows take an offset beyond the buffer
// resource), issued before x is staged; each row waits only for the loads
// that hold it, then reads its slots from LDS.  The residuals (kEpiAdd) of
// the wave's rows are prefetched one per lane.
constexpr int kLdsStreamWaveBytes = 16384;  // largest per-wave buffer
// waves per workgroup: x is staged once per 8 waves (down, one row a wave,
// one workgroup per CU: 5.50 us against 5.78-5.84 with two 4-wave
// workgroups per CU; the decode chain 632 against 645 us)
constexpr int kLdsStreamWaves = 8;

template <int EPI, int WB, int NT>
__global__ __launch_bounds__(64 * kLdsStreamWaves) void gemv_lds_stream_kernel(GemvParams p) {
    static_assert(WB % 1024 == 0 && WB <= kLdsStreamWaveBytes, "whole 1 KB loads, at most 16");
    constexpr int kLdsStreamLoads = WB / 1024;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int n_slots = 4 * p.nb;
    const int J = (n_slots + 63) / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = blockIdx.x * kLdsStreamWaves + wv;
    const bool active = wave < p.total_units;
    const Range rg = range_of_unit(p, active ? wave : 0);
    const int r0 = active ? (wave - rg.first_unit) * p.per_unit : 0;
    const int r1 = active ? min(r0 + p.per_unit, rg.rows) : 0;
    const int n_rows = r1 - r0;
    const uint32_t row_bytes = (uint32_t)p.nb * kBlockBytes;
    uint8_t *ring = smem + wv * WB;
    uint32_t *xlds = reinterpret_cast<uint32_t *>(smem + kLdsStreamWaves * WB);

    // x, first round (slot tid of every token; token tk's slots follow
    // token tk - 1's in LDS), and the residuals of the wave's rows
    const int K = 256 * p.nb;
    const int s_first = tid;
    const int s_load = min(s_first, n_slots - 1);
    u32x4 xraw[NT][8];
#pragma unroll
    for (int tk = 0; tk < NT; ++tk) load_x_raw(p.x + (int64_t)tk * K, s_load >> 2, s_load & 3, xraw[tk]);
    uint32_t res = 0;
    if (EPI == kEpiAdd) res = rg.res[min(r0 + min(lane, max(n_rows - 1, 0)), rg.rows - 1)];
    __builtin_amdgcn_sched_barrier(0);
    // the wave's weight bytes [r0, r1) x row_bytes (the host checks that the
    // range fits a buffer resource and the rows 16 KB)
    const __amdgpu_buffer_rsrc_t wrsrc = make_rsrc(rg.w, (int)((uint32_t)rg.rows * row_bytes));
    const int wbeg = r0 * (int)row_bytes, wend = r1 * (int)row_bytes;
#pragma unroll
    for (int j = 0; j < kLdsStreamLoads; ++j) {
        const int off = wbeg + j * 1024 + lane * 16;
        buffer_to_lds16_nt(wrsrc, ring + j * 1024, off < wend ? off : 0x7FFFFFF0);
    }
    __builtin_amdgcn_sched_barrier(0);

    auto stage = [&](int s, const u32x4 raw[8]) {
        XSlot xs;
        x_slot_from_raw(raw, xs);
        uint32_t *dst = xlds + s * kLdsSlotWords;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            *reinterpret_cast<u32x4 *>(dst + 4 * k) =
                u32x4{xs.p[4 * k], xs.p[4 * k + 1], xs.p[4 * k + 2], xs.p[4 * k + 3]};
        *reinterpret_cast<f32x4v *>(dst + 32) = f32x4v{xs.bias_lo, xs.bias_hi, xs.sx_lo, xs.sx_hi};
    };
    if (s_first < n_slots) {
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) stage(tk * n_slots + s_first, xraw[tk]);
    }
    for (int s = s_first + blockDim.x; s < n_slots; s += blockDim.x) {
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) {
            load_x_raw(p.x + (int64_t)tk * K, s >> 2, s & 3, xraw[0]);
            stage(tk * n_slots + s, xraw[0]);
        }
    }
    // the staged x is visible to every wave; no wait on the weight loads
    // here (__syncthreads would wait for them: its fence counts the loads
    // into LDS), each wave waits for its own below
    wait_lgkmcnt0();
    lds_barrier();
    if (n_rows <= 0) return;

    const uint32_t magic = magic_vgpr();
    for (int k = 0; k < n_rows; ++k) {  // uniform
        const uint8_t *rowp = ring + k * row_bytes;
        float acc[NT];
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) acc[tk] = 0.0f;
        for (int j = 0; j < J; ++j) {
            // item j of row k ends at byte k * row_bytes + min(64 (j+1), n_slots) / 4
            // blocks: the first `need` loads hold it
            const uint32_t item_end = (uint32_t)k * row_bytes + (uint32_t)min(16 * (j + 1), p.nb) * kBlockBytes;
            wait_vmcnt_upto16(kLdsStreamLoads - min(kLdsStreamLoads, (int)((item_end + 1023) / 1024)));
            const int slot = 64 * j + lane;
            const bool valid = slot < n_slots;
            const int sl = valid ? slot : 0;
            XSlot xs[NT];
#pragma unroll
            for (int tk = 0; tk < NT; ++tk) {
                const uint32_t *src = xlds + (tk * n_slots + sl) * kLdsSlotWords;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(src + 4 * q);
                    xs[tk].p[4 * q] = v.x; xs[tk].p[4 * q + 1] = v.y;
                    xs[tk].p[4 * q + 2] = v.z; xs[tk].p[4 * q + 3] = v.w;
                }
                const f32x4v t = *reinterpret_cast<const f32x4v *>(src + 32);
                xs[tk].bias_lo = t[0];
                xs[tk].bias_hi = t[1];
                xs[tk].sx_lo = t[2];
                xs[tk].sx_hi = t[3];
            }
            const uint8_t *blk = rowp + (sl >> 2) * kBlockBytes;
            const u32x4 h = *reinterpret_cast<const u32x4 *>(blk);
            const u32x4 q0 = *reinterpret_cast<const u32x4 *>(blk + 16 + 32 * (sl & 3));
            const u32x4 q1 = *reinterpret_cast<const u32x4 *>(blk + 32 + 32 * (sl & 3));
            float v[NT];
            if (NT == 1)
                v[0] = slot_dot(h, q0, q1, xs[0], scale_decode_for(sl & 3), magic);
            else
                slot_dot_nt<NT>(h, q0, q1, xs, scale_decode_for(sl & 3), magic, v);
#pragma unroll
            for (int tk = 0; tk < NT; ++tk) acc[tk] += valid ? v[tk] : 0.0f;
        }
        const uint32_t rres = EPI == kEpiAdd ? (uint32_t)__builtin_amdgcn_readlane((int)res, k) : 0u;
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) {
            const float total = lane_group_sum<64>(acc[tk]);
            if (lane == 63) store_row<EPI>(rg, r0 + k, total, rres, (int64_t)tk * p.y_stride);
        }
    }
}

const DeviceInfo &device_info() {
    static thread_local int cached_dev = -1;
    static thread_local DeviceInfo info{0, 0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (dev != cached_dev) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
            info.cu_count = prop.multiProcessorCount;
            info.arch_ok = (strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 0;
        } else {
            info.cu_count = 256;
            info.arch_ok = 0;
        }
        cached_dev = dev;
    }
    return info;
}

// Cut each range into units of `per_unit` items (an item is `rows_per_item`
// rows); returns the unit count.  Units never straddle two ranges.
static int assign_units(GemvParams &p, int rows_per_item, int per_unit) {
    int units = 0;
    p.unit_start[0] = 0;
    for (int i = 0; i < p.n_ranges; ++i) {
        if (i > 0) p.unit_start[i] = units;
        const int items = (p.r[i].rows + rows_per_item - 1) / rows_per_item;
        units += (items + per_unit - 1) / per_unit;
    }
    for (int i = p.n_ranges; i < 3; ++i) p.unit_start[i] = units;
    p.per_unit = per_unit;
    p.total_units = units;
    return units;
}

// Steps per load batch of the register kernel (two batches are in flight).
#ifndef RXQ4_GEMV_BATCH
#define RXQ4_GEMV_BATCH 2
#endif
constexpr int kRegBatch = RXQ4_GEMV_BATCH;


// Whether every range of a one-token launch fits a buffer resource with room
// for the streamed kernel's out-of-range offset.
static bool stream_fits(const GemvParams &p) {
    const int64_t row_bytes = (int64_t)p.nb * kBlockBytes;
    for (int i = 0; i < p.n_ranges; ++i)
        if ((int64_t)p.r[i].rows * row_bytes > 0x7FFF0000LL) return false;
    return true;
}

template <int LPR, int EPI, int G, int NBUF, int NT, bool PF>
static hipError_t launch_stream_g(const GemvParams &p, int grid, hipStream_t st) {
    constexpr size_t lds = stream_lds<G, NBUF>();
    // the dynamic LDS limit, raised once per device (devices 0..63)
    static std::atomic<uint64_t> raised{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(raised.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_stream_kernel<LPR, EPI, G, NBUF, NT, PF>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        raised.fetch_or(bit, std::memory_order_acq_rel);
    }
    gemv_stream_kernel<LPR, EPI, G, NBUF, NT, PF><<<grid, 256, lds, st>>>(p);
    return hipSuccess;
}

template <int EPI, int WB, int NT>
static hipError_t launch_lds_stream_wb(const GemvParams &p, int grid, size_t x_lds, hipStream_t st) {
    // the dynamic LDS limit (160 KB), raised once per device (devices 0..63)
    static std::atomic<uint64_t> raised{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(raised.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_lds_stream_kernel<EPI, WB, NT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        raised.fetch_or(bit, std::memory_order_acq_rel);
    }
    gemv_lds_stream_kernel<EPI, WB, NT><<<grid, 64 * kLdsStreamWaves, (size_t)kLdsStreamWaves * WB + x_lds,
                                          st>>>(p);
    return hipGetLastError();
}

// Wave buffers of 8 KB where a wave's rows fit them, else 16 KB; `grid`
// counts workgroups of kLdsStreamWaves waves.
static size_t lds_stream_bytes(int64_t wave_bytes, size_t x_lds) {
    return (size_t)kLdsStreamWaves * (wave_bytes <= 8192 ? 8192 : 16384) + x_lds;
}

template <int EPI, int NT>
static hipError_t launch_lds_stream(const GemvParams &p, int grid, int64_t wave_bytes,
                                    size_t x_lds, hipStream_t st) {
    if (wave_bytes <= 8192) return launch_lds_stream_wb<EPI, 8192, NT>(p, grid, x_lds, st);
    return launch_lds_stream_wb<EPI, 16384, NT>(p, grid, x_lds, st);
}

template <int LPR, int EPI, int NT>
static hipError_t launch_stream(const GemvParams &p, int grid, int long_from, hipStream_t st) {
    if (p.per_unit >= long_from)
        return launch_stream_g<LPR, EPI, kStreamLongSteps, kStreamLongBufs, NT, true>(p, grid, st);
    if (p.per_unit >= kStreamMidSteps)
        return launch_stream_g<LPR, EPI, kStreamShortSteps, kStreamMidBufs, NT, true>(p, grid, st);
    return launch_stream_g<LPR, EPI, kStreamShortSteps, kStreamShortBufs, NT, false>(p, grid, st);
}

template <int LPR, int EPI, int NT>
static hipError_t launch_reg(const GemvParams &p, int grid, hipStream_t st) {
    // RXQ4_GEMV_STREAM: 0 the register kernel, n > 0 the long-wave configuration from n
    // steps per wave (default kStreamMinSteps)
    // one token and 2-4 tokens alike (gate+up [22016 x 2048] at 2 / 3
    // tokens: 8.14 -> 7.87, 9.80 -> 9.49 us)
    if (tuning().gemv_stream >= 0 && stream_fits(p))
        return launch_stream<LPR, EPI, NT>(p, grid, tuning().gemv_stream > 0 ? tuning().gemv_stream : kStreamMinSteps, st);
    gemv_reg_kernel<LPR, EPI, kRegBatch, NT><<<grid, 256, 0, st>>>(p);
    return hipSuccess;
}

template <int EPI, int NT>
static hipError_t launch_gemv_epi(GemvParams p, hipStream_t st) {
    const int slots = 4 * p.nb;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    if (slots <= 64 && (64 % slots) == 0) {
        // Register kernel: aim for `waves_per_cu` waves per CU over the launch.
        const int rps = 64 / slots;
        const int64_t steps = (p.total_rows + rps - 1) / rps;
        const int64_t target = (int64_t)cus * (tuning().gemv_waves_per_cu ? tuning().gemv_waves_per_cu : 4);
        int per_wave = (int)((steps + target - 1) / target);
        per_wave = std::max(1, std::min(per_wave, kRegMaxRows / rps));
        const int waves = assign_units(p, rps, per_wave);
        const int grid = (waves + 3) / 4;
        hipError_t e;
        switch (slots) {
            case 4: e = launch_reg<4, EPI, NT>(p, grid, st); break;
            case 8: e = launch_reg<8, EPI, NT>(p, grid, st); break;
            case 16: e = launch_reg<16, EPI, NT>(p, grid, st); break;
            case 32: e = launch_reg<32, EPI, NT>(p, grid, st); break;
            default: e = launch_reg<64, EPI, NT>(p, grid, st); break;
        }
        if (e != hipSuccess) return e;
    } else {
        // LDS kernels: whole rows per wave, `waves_per_cu` waves per CU (8
        // for the streamed kernel, 4 for the register-load kernel: down
        // [2048 x 11008] in the decode chain of 36 layers, 633 against 660
        // us per step streamed; 5.6 us for the register-load kernel at 4,
        // which 8 waves per CU did not improve).
        const size_t lds = (size_t)NT * slots * kLdsSlotWords * sizeof(uint32_t);
        if (lds > 160 * 1024) return hipErrorInvalidValue;
        auto rows_per_wave = [&](int waves_per_cu) {
            const int64_t target = (int64_t)cus * (tuning().gemv_lds_waves_per_cu ? tuning().gemv_lds_waves_per_cu : waves_per_cu);
            return (int)std::max<int64_t>(1, (p.total_rows + target - 1) / target);
        };
        const int per_wave_s = rows_per_wave(8);
        const int64_t wave_bytes = (int64_t)per_wave_s * p.nb * kBlockBytes;
        if (tuning().gemv_stream >= 0 && wave_bytes <= kLdsStreamWaveBytes &&
            lds_stream_bytes(wave_bytes, lds) <= 160 * 1024 && stream_fits(p)) {
            const int waves = assign_units(p, 1, per_wave_s);
            return launch_lds_stream<EPI, NT>(p, (waves + kLdsStreamWaves - 1) / kLdsStreamWaves,
                                          wave_bytes, lds, st);
        }
        const int per_wave = rows_per_wave(4);
        const int waves = assign_units(p, 1, per_wave);
        const int grid = (waves + 3) / 4;
        if (lds > 64 * 1024) {
            const hipError_t e = hipFuncSetAttribute(
                reinterpret_cast<const void *>(&gemv_lds_kernel<EPI, 2, NT>),
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        gemv_lds_kernel<EPI, 2, NT><<<grid, 256, lds, st>>>(p);
    }
    return hipGetLastError();
}

hipError_t launch_gemv(GemvParams p, int epilogue, hipStream_t st) {
    p.n_tok = 1;
    p.y_stride = 0;
    switch (epilogue) {
        case kEpiF16: return launch_gemv_epi<kEpiF16, 1>(p, st);
        case kEpiF32: return launch_gemv_epi<kEpiF32, 1>(p, st);
        case kEpiAdd: return launch_gemv_epi<kEpiAdd, 1>(p, st);
        default: return hipErrorInvalidValue;
    }
}

template <int EPI>
static hipError_t launch_multi_epi(GemvParams &p, int n_tok, hipStream_t st) {
    switch (n_tok) {
        case 2: return launch_gemv_epi<EPI, 2>(p, st);
        case 3: return launch_gemv_epi<EPI, 3>(p, st);
        default: return launch_gemv_epi<EPI, 4>(p, st);
    }
}

// 2 tokens: the multi-token GEMV.  3: it too for at least 4 MiB of weights
// (streamed multi-token GEMV against the MFMA small-batch kernel: gate+up
// [22016 x 2048] 9.4-9.8 against 10.8-10.9 us, down [2048 x 11008] 8.8
// against 9.4-9.5, [5632 x 2048] 5.0 against 5.6), else the MFMA kernel
// ([2560 x 2048] 4.55 against 4.21, [2048 x 2048] 4.12-4.18 against
// 4.14-4.24).  4: the MFMA kernel (gate+up 11.2 against 10.5-10.6 us, down
// 11.1 against 9.2-9.4).  Graph replay, distinct weights.
bool gemv_multi_token_preferred(int n_tok, int M, int K) {
    return n_tok == 2 || (n_tok == 3 && (int64_t)M * (K / 256) * kBlockBytes >= ((int64_t)4 << 20));
}

bool gemv_multi_token_fits(int n_tok, int K) {
    const int slots = 4 * (K / 256);
    if (slots <= 64 && (64 % slots) == 0) return true;
    return (size_t)n_tok * slots * kLdsSlotWords * sizeof(uint32_t) <= 160 * 1024;
}

hipError_t launch_gemv_multi_token(void *y, int y_dtype, const uint8_t *w, const uint16_t *x,
                                   int M, int n_tok, int K, hipStream_t st) {
    if (n_tok < 2 || n_tok > kMaxRegTokens) return hipErrorInvalidValue;
    GemvParams p{};
    p.r[0] = GemvRange{w, y, nullptr, M};
    p.n_ranges = 1;
    p.total_rows = M;
    p.x = x;
    p.nb = K / 256;
    p.n_tok = n_tok;
    p.y_stride = M;
    return y_dtype == RXQ4_DTYPE_F32 ? launch_multi_epi<kEpiF32>(p, n_tok, st)
                                     : launch_multi_epi<kEpiF16>(p, n_tok, st);
}

}  // namespace rxq4
