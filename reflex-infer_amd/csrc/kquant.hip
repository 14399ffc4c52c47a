// kquant.hip -- Q5_K (ggml type 13) and Q6_K (type 14) weights on gfx950:
// decode GEMV (fp16 / fp32 / residual-add outputs), Q6_K embedding rows and
// the small-batch (2..16 token) product; more tokens run the MFMA GEMM of
// gemm_q4k.hip with the Q5_K / Q6_K format policies.  Replaces the
// reference's Q5_K/Q6_K kernels
// (q4_gemm.cu:325-405 dot_q5k_row / dot_q6k_row, 473-489 and 527-543 the
// GEMVs, 574-616 the Q6_K embedding, 1358-1480 the batched kernels).
//
// Block formats (GGML):
//   Q5_K, 176 B: d fp16 @0, dmin fp16 @2, scales[12] @4 (the Q4_K 6-bit
//     packing), qh[32] @16, qs[128] @48.  Weight 64*il + 32*hi + l: nibble hi
//     of qs[32*il + l], fifth bit 2*il + hi of qh[l]; sub-block 2*il + hi;
//     w = d*sc*q - dmin*m.
//   Q6_K, 210 B: ql[128] @0, qh[64] @128, int8 scales[16] @192, d fp16 @208.
//     Weight 128*h + 32*j + l: nibble j>>1 of ql[64*h + 32*(j&1) + l], bits
//     2*j.. of qh[32*h + l]; scale scales[(128*h + 32*j + l) / 16];
//     w = d*sc*(q - 32).
// 210-byte blocks are only 2-byte aligned, so every Q6_K field is read with
// dword-aligned buffer loads and shifted into place with v_alignbyte.  All
// weight reads go through buffer resources bounded at the rows a wave owns:
// reads past them return zeros, which the kernels use for the rows and
// slots beyond the matrix.
//
// GEMV.  A lane owns a 64-weight slot (Q5_K: quant group il of a block;
// Q6_K: (h, s) = four runs of 16, k = 128h + 32j + 16s + i).  The workgroup
// stages x in LDS as fp16 plus fp32 sums of every 16-element run.  Quant
// values become fp16 1024+q with one v_perm per pair (byte q under a 0x64
// high byte), v_dot2_f32_f16 multiplies them with the x pairs into an fp32
// accumulator seeded with -(1024 + bias) * sum(x), so
//   Q6_K: y += d*sc_j * sum((q - 32) x)       (bias 32)
//   Q5_K: y += d*sc * sum(q x) - dmin*m * sum(x)
// Rows with 4*K/256 <= 64 slots (K <= 4096, power-of-two block counts) are
// packed 64/slots rows per wave step; longer rows take one wave per row.
#include <algorithm>
#include <type_traits>

#include "launch.h"
#include "mfma_util.h"
#include "q4k_device.h"

namespace rxq4 {

template <int T>
struct KqFormat;
template <>
struct KqFormat<12> {
    static constexpr int kBytes = 144;
};
template <>
struct KqFormat<13> {
    static constexpr int kBytes = 176;
};
template <>
struct KqFormat<14> {
    static constexpr int kBytes = 210;
};

// 16 bytes at an even byte offset: the aligned 16 bytes at off & ~3 plus the
// next dword (20 bytes cover the 16 wanted ones).
struct Raw16 {
    u32x4 v;
    uint32_t e;
};

__device__ __forceinline__ Raw16 load_raw16(__amdgpu_buffer_rsrc_t rs, int off) {
    const int a = off & ~3;
    return Raw16{buffer_load16(rs, a), buffer_load4(rs, a + 16)};
}

// Buffer resource over `bytes` bytes at p, based at the dword boundary at or
// below p (a Q6_K row starts on a 2-byte boundary when K/256 is odd):
// field offsets are taken relative to the returned base, i.e. plus `ex`.
struct RowRes {
    __amdgpu_buffer_rsrc_t rs;
    int ex;
};

__device__ __forceinline__ RowRes row_rsrc(const uint8_t *p, int bytes) {
    const int ex = (int)(reinterpret_cast<uintptr_t>(p) & 3);
    return RowRes{make_rsrc(p - ex, bytes + ex), ex};
}

// The fp16 d of a Q6_K block (2-byte load: a dword could reach past the
// last block, where the bounded resource would return zero for it).
__device__ __forceinline__ float q6_d(__amdgpu_buffer_rsrc_t rs, int boff) {
    return f16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rs, boff + 208, 0, 0));
}

// Signed scale byte `idx` (0..3) of the dword w.
__device__ __forceinline__ float scale_byte(uint32_t w, int idx) {
    return (float)((int)(w << (24 - 8 * idx)) >> 24);
}

__device__ __forceinline__ u32x4 realign16(const Raw16 &w, int r) {
    return u32x4{align_bytes(w.v.y, w.v.x, r), align_bytes(w.v.z, w.v.y, r),
                 align_bytes(w.v.w, w.v.z, r), align_bytes(w.e, w.v.w, r)};
}

// fp16 pair (1024 + byte0, 1024 + byte1) resp. bytes 2, 3 of q.
__device__ __forceinline__ uint32_t magic_lo(uint32_t q) {
    return __builtin_amdgcn_perm(0x64646464u, q, 0x04010400u);
}
__device__ __forceinline__ uint32_t magic_hi(uint32_t q) {
    return __builtin_amdgcn_perm(0x64646464u, q, 0x04030402u);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_half2(a), as_half2(b), c, false);
}

// x in LDS: fp16 [K] followed by fp32 sums of each 16-element run [K/16].
// Sum over aligned groups of `slots` lanes (uniform; a power of two, at most
// 64): the __shfl_xor butterfly, on the VALU (butterfly_sum, bit-identical)
// for groups of 32 and 64.
__device__ __forceinline__ float kq_row_sum(float v, int slots) {
    if (slots == 64) return butterfly_sum<64>(v);
    if (slots == 32) return butterfly_sum<32>(v);
    for (int q = slots >> 1; q > 0; q >>= 1) v += __shfl_xor(v, q, 64);
    return v;
}

struct XLds {
    const u32x4 *x;   // 8 fp16 per element
    const float *sum;
};

// ---------------------------------------------------------------- Q6_K slot
struct Q6Raw {
    Raw16 a, b, h, s;  // ql (j = 0/2), ql (j = 1/3), qh, scales
    float d;
};

__device__ __forceinline__ void q6_load(__amdgpu_buffer_rsrc_t rs, int boff, int h, int s,
                                        Q6Raw &o) {
    o.a = load_raw16(rs, boff + 64 * h + 16 * s);
    o.b = load_raw16(rs, boff + 64 * h + 32 + 16 * s);
    o.h = load_raw16(rs, boff + 128 + 32 * h + 16 * s);
    o.s = load_raw16(rs, boff + 192);
    o.d = q6_d(rs, boff);
}

// Quant bytes of run j for weights 4m..4m+3 of the lane's 16-run.
__device__ __forceinline__ uint32_t q6_bytes(uint32_t a, uint32_t b, uint32_t hb, int j) {
    switch (j) {
        case 0: return (a & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4);
        case 1: return (b & 0x0F0F0F0Fu) | ((hb & 0x0C0C0C0Cu) << 2);
        case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u);
        default: return ((b >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u);
    }
}

// Dot product of the lane's Q6_K slot (block at k0, half h, sixteenth s)
// with x.  r = byte misalignment of the block (0 or 2).
__device__ __forceinline__ float q6_slot_dot(const Q6Raw &w, int r, int h, int s, int k0,
                                             const XLds &xl) {
    const u32x4 A = realign16(w.a, r), B = realign16(w.b, r), H = realign16(w.h, r);
    const u32x4 S = realign16(w.s, r);
    const float d = w.d;
    // scales 8h + 2j + s: bytes s, s+2 of dword 2h (j = 0, 1), of 2h+1 (j = 2, 3)
    const uint32_t s01 = h ? S.z : S.x, s23 = h ? S.w : S.y;
    float y = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int xi = (k0 + 128 * h + 32 * j + 16 * s) >> 3;  // u32x4 index of the run
        const u32x4 x0 = xl.x[xi], x1 = xl.x[xi + 1];
        const float sc = scale_byte(j < 2 ? s01 : s23, 2 * (j & 1) + s);
        float acc = -1056.0f * xl.sum[xi >> 1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t q = q6_bytes(A[m], B[m], H[m], j);
            acc = dot2(magic_lo(q), xw[2 * m], acc);
            acc = dot2(magic_hi(q), xw[2 * m + 1], acc);
        }
        y += d * sc * acc;
    }
    return y;
}

// ---------------------------------------------------------------- Q5_K slot
struct Q5Raw {
    u32x4 hdr, qh0, qh1, qs0, qs1;
};

__device__ __forceinline__ void q5_load(__amdgpu_buffer_rsrc_t rs, int boff, int il, Q5Raw &o) {
    o.hdr = buffer_load16(rs, boff);
    o.qh0 = buffer_load16(rs, boff + 16);
    o.qh1 = buffer_load16(rs, boff + 32);
    o.qs0 = buffer_load16(rs, boff + 48 + 32 * il);
    o.qs1 = buffer_load16(rs, boff + 64 + 32 * il);
}

__device__ __forceinline__ float q5_slot_dot(const Q5Raw &w, int il, int k0, const XLds &xl) {
    const float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(w.hdr.x >> 16);
    uint32_t sc, mn;
    scale_pair(w.hdr.y, w.hdr.z, w.hdr.w, il, &sc, &mn);
    const int xl0 = (k0 + 64 * il) >> 3, xh0 = xl0 + 4;  // u32x4 index of the low / high run
    const float s_lo = xl.sum[xl0 >> 1] + xl.sum[(xl0 >> 1) + 1];
    const float s_hi = xl.sum[xh0 >> 1] + xl.sum[(xh0 >> 1) + 1];
    float acc_lo = -1024.0f * s_lo, acc_hi = -1024.0f * s_hi;
    const uint32_t qs[8] = {w.qs0.x, w.qs0.y, w.qs0.z, w.qs0.w, w.qs1.x, w.qs1.y, w.qs1.z, w.qs1.w};
    const uint32_t qh[8] = {w.qh0.x, w.qh0.y, w.qh0.z, w.qh0.w, w.qh1.x, w.qh1.y, w.qh1.z, w.qh1.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {  // 8 weights per u32x4 of x
        const u32x4 xlo = xl.x[xl0 + c], xhi = xl.x[xh0 + c];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int m = 2 * c + h2;
            const uint32_t L = qs[m], Hb = qh[m];
            const uint32_t qlo = (L & 0x0F0F0F0Fu) | (((Hb >> (2 * il)) & 0x01010101u) << 4);
            const uint32_t qhi =
                ((L >> 4) & 0x0F0F0F0Fu) | (((Hb >> (2 * il + 1)) & 0x01010101u) << 4);
            acc_lo = dot2(magic_lo(qlo), xlo[2 * h2], acc_lo);
            acc_lo = dot2(magic_hi(qlo), xlo[2 * h2 + 1], acc_lo);
            acc_hi = dot2(magic_lo(qhi), xhi[2 * h2], acc_hi);
            acc_hi = dot2(magic_hi(qhi), xhi[2 * h2 + 1], acc_hi);
        }
    }
    return d * (float)(sc & 0xFFu) * acc_lo - dmin * (float)(mn & 0xFFu) * s_lo +
           d * (float)(sc >> 8) * acc_hi - dmin * (float)(mn >> 8) * s_hi;
}

// ---------------------------------------------------------------- Q4_K slot
// (only for mixed-type multi-range launches; all-Q4_K work uses gemv_q4k.hip)
struct Q4Raw {
    u32x4 hdr, qs0, qs1;
};

__device__ __forceinline__ void q4_load(__amdgpu_buffer_rsrc_t rs, int boff, int il, Q4Raw &o) {
    o.hdr = buffer_load16(rs, boff);
    o.qs0 = buffer_load16(rs, boff + 16 + 32 * il);
    o.qs1 = buffer_load16(rs, boff + 32 + 32 * il);
}

__device__ __forceinline__ float q4_slot_dot(const Q4Raw &w, int il, int k0, const XLds &xl) {
    const float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(w.hdr.x >> 16);
    uint32_t sc, mn;
    scale_pair(w.hdr.y, w.hdr.z, w.hdr.w, il, &sc, &mn);
    const int xl0 = (k0 + 64 * il) >> 3, xh0 = xl0 + 4;
    const float s_lo = xl.sum[xl0 >> 1] + xl.sum[(xl0 >> 1) + 1];
    const float s_hi = xl.sum[xh0 >> 1] + xl.sum[(xh0 >> 1) + 1];
    float acc_lo = -1024.0f * s_lo, acc_hi = -1024.0f * s_hi;
    const uint32_t qs[8] = {w.qs0.x, w.qs0.y, w.qs0.z, w.qs0.w, w.qs1.x, w.qs1.y, w.qs1.z, w.qs1.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 xlo = xl.x[xl0 + c], xhi = xl.x[xh0 + c];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const uint32_t L = qs[2 * c + h2];
            const uint32_t qlo = L & 0x0F0F0F0Fu, qhi = (L >> 4) & 0x0F0F0F0Fu;
            acc_lo = dot2(magic_lo(qlo), xlo[2 * h2], acc_lo);
            acc_lo = dot2(magic_hi(qlo), xlo[2 * h2 + 1], acc_lo);
            acc_hi = dot2(magic_lo(qhi), xhi[2 * h2], acc_hi);
            acc_hi = dot2(magic_hi(qhi), xhi[2 * h2 + 1], acc_hi);
        }
    }
    return d * (float)(sc & 0xFFu) * acc_lo - dmin * (float)(mn & 0xFFu) * s_lo +
           d * (float)(sc >> 8) * acc_hi - dmin * (float)(mn >> 8) * s_hi;
}

// ---------------------------------------------------------------- GEMV
struct KqGemvParams {
    const uint8_t *w;
    void *y;
    const uint16_t *res;
    const uint16_t *x;
    int M, K, nb, row_bytes;
    int slots;     // 4 * nb
    int rows_per;  // rows per wave step (64 / slots) or 0: one row per step
    int n_units;   // wave steps (packed rows) or rows
};

template <int T>
struct Slot {
    using Raw = typename std::conditional<
        T == 14, Q6Raw, typename std::conditional<T == 13, Q5Raw, Q4Raw>::type>::type;
    Raw raw;
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int boff, int u) {
        if constexpr (T == 14)
            q6_load(rs, boff, u >> 1, u & 1, raw);
        else if constexpr (T == 13)
            q5_load(rs, boff, u, raw);
        else
            q4_load(rs, boff, u, raw);
    }
    // k0 = first weight of the block (clamped to a real block for x reads).
    __device__ __forceinline__ float dot(int boff, int u, int k0, const XLds &xl) const {
        if constexpr (T == 14)
            return q6_slot_dot(raw, boff & 3, u >> 1, u & 1, k0, xl);
        else if constexpr (T == 13)
            return q5_slot_dot(raw, u, k0, xl);
        else
            return q4_slot_dot(raw, u, k0, xl);
    }
};

// res: the row's residual (fp16 bits, kEpiAdd), fetched with the row's
// weights so that the store waits for no further load.
template <int EPI>
__device__ __forceinline__ void kq_store(const KqGemvParams &p, int row, float v, uint32_t res) {
    if (EPI == kEpiF32) {
        static_cast<float *>(p.y)[row] = v;
    } else if (EPI == kEpiF16) {
        static_cast<uint16_t *>(p.y)[row] = f32_to_f16_bits(v);
    } else {
        // q4_gemm.cu:774-777: round the projection, add the residual, round.
        const float projected = f16_bits_to_f32(f32_to_f16_bits(v));
        static_cast<uint16_t *>(p.y)[row] = f32_to_f16_bits(projected + f16_bits_to_f32(res));
    }
}

// Residual of `row` (clamped to the matrix) for kEpiAdd, else 0.
template <int EPI>
__device__ __forceinline__ uint32_t kq_res(const KqGemvParams &p, int row) {
    return EPI == kEpiAdd ? p.res[min(row, p.M - 1)] : 0u;
}

// PACKED: rows of at most 64 slots packed into wave steps (p.rows_per > 0);
// else one row per wave.  Two instances, so that each path gets its own
// register allocation.
template <int T, int EPI, bool PACKED>
__global__ __launch_bounds__(256) void kq_gemv_kernel(KqGemvParams p) {
    constexpr int BYTES = KqFormat<T>::kBytes;
    extern __shared__ u32x4 kq_smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int n_waves = gridDim.x * 4;
    const int wave_g = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(tid >> 6);
    const XLds xl{kq_smem, reinterpret_cast<const float *>(kq_smem + (p.K >> 3))};
    auto stage_x = [&]() {
        // x (fp16) and the fp32 sums of its 16-element runs.
        u32x4 *xs = kq_smem;
        float *sums = reinterpret_cast<float *>(kq_smem + (p.K >> 3));
        const u32x4 *xg = reinterpret_cast<const u32x4 *>(p.x);
        for (int r = tid; r < (p.K >> 4); r += 256) {
            const u32x4 a = xg[2 * r], b = xg[2 * r + 1];
            xs[2 * r] = a;
            xs[2 * r + 1] = b;
            const uint32_t w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s += f16_bits_to_f32(w8[i] & 0xFFFFu);
                s += f16_bits_to_f32(w8[i] >> 16);
            }
            sums[r] = s;
        }
        __syncthreads();
    };
    if constexpr (PACKED) {
        // slots = 64 / rows_per lanes per row; the wave takes the steps
        // wave_g + k * n_waves.  Two steps are in flight at all times: step
        // k + 2 is issued as soon as step k has been computed.  Steps past
        // the last reload the last one (L2 hits, nothing stored), so every
        // load is unconditional and the compiler's vmcnt waits count exactly.
        const int sub = lane / p.slots;
        const int slot = lane - sub * p.slots;
        const int b = slot >> 2, u = slot & 3;
        const int boff = sub * p.row_bytes + b * BYTES;
        struct Step {
            Slot<T> s;
            RowRes r;
            int r0, n;
            uint32_t res;
        };
        auto load = [&](int st, Step &o) {
            const int sc = min(st, p.n_units - 1);
            o.r0 = sc * p.rows_per;
            const int rows = min(p.rows_per, p.M - o.r0);
            o.n = st < p.n_units ? rows : 0;
            o.r = row_rsrc(p.w + (int64_t)o.r0 * p.row_bytes, rows * p.row_bytes);
            o.s.load(o.r.rs, o.r.ex + boff, u);
            o.res = kq_res<EPI>(p, o.r0 + sub);
        };
        auto finish = [&](const Step &o) {
            float v = o.s.dot(o.r.ex + boff, u, b * 256, xl);
            v = kq_row_sum(v, p.slots);
            if (slot == 0 && sub < o.n) kq_store<EPI>(p, o.r0 + sub, v, o.res);
        };
        stage_x();
        if (wave_g < p.n_units) {
            Step A, B;
            int st = wave_g;
            load(st, A);
            load(st + n_waves, B);
            for (; st + 2 * n_waves < p.n_units; st += 2 * n_waves) {
                finish(A);
                load(st + 2 * n_waves, A);
                finish(B);
                load(st + 3 * n_waves, B);
            }
            finish(A);
            finish(B);
        }
    } else {
        // One row per wave, its slots 64 at a time, two rounds per load batch
        // (slots past the row read zeros, d = 0; their x reads are clamped
        // to the last block).
        const int n_iter = (p.slots + 63) >> 6;
        stage_x();
        for (int row = wave_g; row < p.M; row += n_waves) {
            const RowRes rr = row_rsrc(p.w + (int64_t)row * p.row_bytes, p.row_bytes);
            const uint32_t res = kq_res<EPI>(p, row);
            float v = 0.0f;
            for (int c = 0; c < n_iter; c += 2) {
                const int s0 = 64 * c + lane, s1 = s0 + 64;
                const int b0 = s0 >> 2, b1 = s1 >> 2;
                const int o0 = rr.ex + b0 * BYTES, o1 = rr.ex + b1 * BYTES;
                Slot<T> A, B;
                A.load(rr.rs, o0, s0 & 3);
                B.load(rr.rs, o1, s1 & 3);
                v += A.dot(o0, s0 & 3, min(b0, p.nb - 1) * 256, xl);
                if (c + 1 < n_iter) v += B.dot(o1, s1 & 3, min(b1, p.nb - 1) * 256, xl);
            }
            v = butterfly_sum<64>(v);
            if (lane == 0) kq_store<EPI>(p, row, v, res);
        }
    }
}

// Mixed-type multi-range GEMV (pair / triple with a Q5_K or Q6_K range, e.g.
// the Q4_K q, k + Q6_K v projection): one launch and one x staging for all
// ranges.  A wave walks units (wave steps or rows) across the ranges; each
// unit belongs to one range, so its type is uniform and dispatched per unit.
struct KqMultiRange {
    const uint8_t *w;
    uint16_t *y;
    int type, M, row_bytes, unit0;  // unit0: first global unit of the range
};

struct KqMultiParams {
    KqMultiRange r[3];
    int n_ranges;
    const uint16_t *x;
    int K, nb, slots, rows_per, n_units;
};

template <int T>
__device__ __forceinline__ void kq_multi_unit(const KqMultiParams &p, const KqMultiRange &r,
                                              int lu, int lane, const XLds &xl) {
    constexpr int BYTES = KqFormat<T>::kBytes;
    if (p.rows_per > 0) {
        const int sub = lane / p.slots, slot = lane - sub * p.slots;
        const int r0 = lu * p.rows_per;
        const int n = min(p.rows_per, r.M - r0);
        const RowRes rr = row_rsrc(r.w + (int64_t)r0 * r.row_bytes, n * r.row_bytes);
        const int b = slot >> 2, u = slot & 3;
        const int boff = rr.ex + sub * r.row_bytes + b * BYTES;
        Slot<T> S;
        S.load(rr.rs, boff, u);
        float v = S.dot(boff, u, b * 256, xl);
        v = kq_row_sum(v, p.slots);
        if (slot == 0 && sub < n) r.y[r0 + sub] = f32_to_f16_bits(v);
    } else {
        const RowRes rr = row_rsrc(r.w + (int64_t)lu * r.row_bytes, r.row_bytes);
        const int n_iter = (p.slots + 63) >> 6;
        float v = 0.0f;
        for (int c = 0; c < n_iter; c += 2) {
            const int s0 = 64 * c + lane, s1 = s0 + 64;
            const int b0 = s0 >> 2, b1 = s1 >> 2;
            const int o0 = rr.ex + b0 * BYTES, o1 = rr.ex + b1 * BYTES;
            Slot<T> A, B;
            A.load(rr.rs, o0, s0 & 3);
            B.load(rr.rs, o1, s1 & 3);
            v += A.dot(o0, s0 & 3, min(b0, p.nb - 1) * 256, xl);
            if (c + 1 < n_iter) v += B.dot(o1, s1 & 3, min(b1, p.nb - 1) * 256, xl);
        }
        v = butterfly_sum<64>(v);
        if (lane == 0) r.y[lu] = f32_to_f16_bits(v);
    }
}

// The units of wave u0 and its successors u0 + n_waves, ...; each unit's
// type is dispatched.
__device__ __forceinline__ void kq_multi_units(const KqMultiParams &p, int u0, int lane,
                                               const XLds &xl) {
    const int n_waves = gridDim.x * 4;
    for (int u = u0; u < p.n_units; u += n_waves) {
        const int ri = (p.n_ranges > 1 && u >= p.r[1].unit0) + (p.n_ranges > 2 && u >= p.r[2].unit0);
        const KqMultiRange &r = p.r[ri];
        const int lu = u - r.unit0;
        switch (r.type) {
            case 12: kq_multi_unit<12>(p, r, lu, lane, xl); break;
            case 13: kq_multi_unit<13>(p, r, lu, lane, xl); break;
            default: kq_multi_unit<14>(p, r, lu, lane, xl); break;
        }
    }
}

// Packed rows, K <= 4096 (one x run of 16 per thread): the wave's first
// unit (type T) loads its weights right behind the thread's x run, x is
// staged and a barrier that waits for LDS only follows, so the weights stay
// in flight across the staging (loads complete in order: x first).  The
// unit's arithmetic and the staged x are those of kq_multi_unit.
template <int T>
__device__ __forceinline__ void kq_multi_first_packed(const KqMultiParams &p, int u0, int uc,
                                                      int ri, int tid, int lane, u32x4 *xs,
                                                      float *sums, const XLds &xl) {
    constexpr int BYTES = KqFormat<T>::kBytes;
    const int n_runs = p.K >> 4;
    const int rx = min(tid, n_runs - 1);
    const u32x4 *xg = reinterpret_cast<const u32x4 *>(p.x);
    const u32x4 xa = xg[2 * rx], xb = xg[2 * rx + 1];
    __builtin_amdgcn_sched_barrier(0);
    const KqMultiRange &r = p.r[ri];
    const int lu = uc - r.unit0;
    const int sub = lane / p.slots, slot = lane - sub * p.slots;
    const int r0 = lu * p.rows_per;
    const int n = min(p.rows_per, r.M - r0);
    const RowRes rr = row_rsrc(r.w + (int64_t)r0 * r.row_bytes, n * r.row_bytes);
    const int b = slot >> 2, u = slot & 3;
    const int boff = rr.ex + sub * r.row_bytes + b * BYTES;
    Slot<T> S;
    S.load(rr.rs, boff, u);
    __builtin_amdgcn_sched_barrier(0);
    if (tid < n_runs) {
        xs[2 * tid] = xa;
        xs[2 * tid + 1] = xb;
        const uint32_t w8[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        float sx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sx += f16_bits_to_f32(w8[i] & 0xFFFFu);
            sx += f16_bits_to_f32(w8[i] >> 16);
        }
        sums[tid] = sx;
    }
    wait_lgkmcnt0();
    lds_barrier();
    if (u0 < p.n_units) {
        float v = S.dot(boff, u, b * 256, xl);
        v = kq_row_sum(v, p.slots);
        if (slot == 0 && sub < n) r.y[r0 + sub] = f32_to_f16_bits(v);
    }
    kq_multi_units(p, u0 + gridDim.x * 4, lane, xl);
}

__global__ __launch_bounds__(256) void kq_multi_kernel(KqMultiParams p) {
    extern __shared__ u32x4 kq_smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int u0 = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(tid >> 6);
    if (p.rows_per > 0 && (p.K >> 4) <= 256) {
        u32x4 *xs = kq_smem;
        float *sums = reinterpret_cast<float *>(kq_smem + (p.K >> 3));
        const XLds xl{kq_smem, sums};
        const int uc = min(u0, p.n_units - 1);
        const int ri = (p.n_ranges > 1 && uc >= p.r[1].unit0) + (p.n_ranges > 2 && uc >= p.r[2].unit0);
        switch (p.r[ri].type) {
            case 12: kq_multi_first_packed<12>(p, u0, uc, ri, tid, lane, xs, sums, xl); break;
            case 13: kq_multi_first_packed<13>(p, u0, uc, ri, tid, lane, xs, sums, xl); break;
            default: kq_multi_first_packed<14>(p, u0, uc, ri, tid, lane, xs, sums, xl); break;
        }
        return;
    }
    {
        u32x4 *xs = kq_smem;
        float *sums = reinterpret_cast<float *>(kq_smem + (p.K >> 3));
        const u32x4 *xg = reinterpret_cast<const u32x4 *>(p.x);
        for (int r = tid; r < (p.K >> 4); r += 256) {
            const u32x4 a = xg[2 * r], b = xg[2 * r + 1];
            xs[2 * r] = a;
            xs[2 * r + 1] = b;
            const uint32_t w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s += f16_bits_to_f32(w8[i] & 0xFFFFu);
                s += f16_bits_to_f32(w8[i] >> 16);
            }
            sums[r] = s;
        }
    }
    __syncthreads();
    const XLds xl{kq_smem, reinterpret_cast<const float *>(kq_smem + (p.K >> 3))};
    kq_multi_units(p, u0, lane, xl);
}

template <int T, int EPI, bool PACKED>
static hipError_t launch_kq_gemv_p(const KqGemvParams &p, hipStream_t st) {
    const size_t lds = (size_t)p.K * 2 + (size_t)(p.K / 16) * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    // at most 3 workgroups (12 waves) per CU: the Q6_K LM head [151936 x
    // 2048] took 50.1-51.0 us with 3, 53.8-54.0 with 4, 55.6-57.1 with 5-6
    // and 58.5 with 2 (alternating runs on one box); down (one wave per row,
    // 512 workgroups) is below every cap
    constexpr size_t kWgPerCu = 3;
    const int wg_per_cu = (int)std::max<size_t>(1, std::min<size_t>(kWgPerCu, (160 * 1024) / lds));
    const int want = (p.n_units + 3) / 4;
    const int grid = std::max(1, std::min(want, cus * wg_per_cu));
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_gemv_kernel<T, EPI, PACKED>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
    }
    kq_gemv_kernel<T, EPI, PACKED><<<grid, 256, lds, st>>>(p);
    return hipGetLastError();
}

template <int T, int EPI>
static hipError_t launch_kq_gemv_t(const KqGemvParams &p, hipStream_t st) {
    return p.rows_per > 0 ? launch_kq_gemv_p<T, EPI, true>(p, st)
                          : launch_kq_gemv_p<T, EPI, false>(p, st);
}

hipError_t launch_kq_gemv(int ggml_type, const GemvRange &r, const uint16_t *x, int K,
                          int epilogue, hipStream_t st) {
    KqGemvParams p{};
    p.w = r.w;
    p.y = r.y;
    p.res = r.res;
    p.x = x;
    p.M = r.rows;
    p.K = K;
    p.nb = K / 256;
    p.row_bytes = p.nb * (ggml_type == 14 ? KqFormat<14>::kBytes : KqFormat<13>::kBytes);
    p.slots = 4 * p.nb;
    p.rows_per = (p.slots <= 64 && 64 % p.slots == 0) ? 64 / p.slots : 0;
    p.n_units = p.rows_per ? (p.M + p.rows_per - 1) / p.rows_per : p.M;
    if (p.M <= 0) return hipSuccess;
    if ((int64_t)p.rows_per * p.row_bytes > 0x7FFFFFFF) return hipErrorInvalidValue;
#define RXQ4_KQ_EPI(T)                                                   \
    switch (epilogue) {                                                  \
        case kEpiF16: return launch_kq_gemv_t<T, kEpiF16>(p, st);        \
        case kEpiF32: return launch_kq_gemv_t<T, kEpiF32>(p, st);        \
        case kEpiAdd: return launch_kq_gemv_t<T, kEpiAdd>(p, st);        \
        default: return hipErrorInvalidValue;                            \
    }
    if (ggml_type == 14) {
        RXQ4_KQ_EPI(14)
    }
    if (ggml_type == 13) {
        RXQ4_KQ_EPI(13)
    }
#undef RXQ4_KQ_EPI
    return hipErrorInvalidValue;
}

hipError_t launch_kq_multi(const GemvRange *ranges, const int *types, int n_ranges,
                           const uint16_t *x, int K, hipStream_t st) {
    KqMultiParams p{};
    p.x = x;
    p.K = K;
    p.nb = K / 256;
    p.slots = 4 * p.nb;
    p.rows_per = (p.slots <= 64 && 64 % p.slots == 0) ? 64 / p.slots : 0;
    int units = 0;
    for (int i = 0; i < n_ranges; ++i) {
        const int t = types[i];
        const int bytes = t == 14 ? 210 : t == 13 ? 176 : 144;
        p.r[p.n_ranges] = KqMultiRange{ranges[i].w, static_cast<uint16_t *>(ranges[i].y), t,
                                       ranges[i].rows, p.nb * bytes, units};
        if ((int64_t)(p.rows_per ? p.rows_per : 1) * p.nb * bytes > 0x7FFFFFFF)
            return hipErrorInvalidValue;
        units += p.rows_per ? (ranges[i].rows + p.rows_per - 1) / p.rows_per : ranges[i].rows;
        ++p.n_ranges;
    }
    p.n_units = units;
    if (units == 0) return hipSuccess;
    const size_t lds = (size_t)K * 2 + (size_t)(K / 16) * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    const int wg_per_cu = (int)std::max<size_t>(1, std::min<size_t>(4, (160 * 1024) / lds));
    const int grid = std::max(1, std::min((units + 3) / 4, cus * wg_per_cu));
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_multi_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
    }
    kq_multi_kernel<<<grid, 256, lds, st>>>(p);
    return hipGetLastError();
}

// ---------------------------------------------------------------- embedding
// Q6_K rows (reference dequant_embedding_q6k_kernel, q4_gemm.cu:574-616): a
// thread writes 8 consecutive outputs of one row with one 16-byte store;
// w = d*sc*(q - 32) is exact in fp32, so the fp16 result is bit-identical.
// Nontemporal stores, as the Q4_K gather.  kUniform (K a multiple of
// 1024): a row's K/16 threads are whole waves, so the row index, the id (a
// scalar load) and the row's buffer resource are wave-uniform; otherwise the
// resource comes from a per-lane id and every buffer load runs in a
// readfirstlane loop over the wave's distinct rows.
template <bool kBatched, bool kUniform>
__global__ __launch_bounds__(256) void embed_q6k_kernel(uint16_t *__restrict__ dst,
                                                        const uint8_t *__restrict__ w,
                                                        const int32_t *__restrict__ ids,
                                                        int token_id, int64_t n_vocab, int n_ids,
                                                        int K) {
    constexpr int BYTES = KqFormat<14>::kBytes;
    const int per_row = K >> 4;  // 16-value sub-blocks (one int8 scale each)
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int64_t i;
    if (kUniform) {
        const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4u + (threadIdx.x >> 6)));
        i = (int64_t)(wave / (uint32_t)(per_row >> 6));
    } else {
        i = t / per_row;
    }
    const int c = (int)(t - i * per_row);
    if (i >= n_ids) return;
    u32x4 *out = reinterpret_cast<u32x4 *>(dst + i * K + c * 16);
    int64_t id = token_id;
    if (kBatched) {
        id = ids[i];
        if (id < 0 || id >= n_vocab) {
            store16_nt(out, u32x4{0, 0, 0, 0});
            store16_nt(out + 1, u32x4{0, 0, 0, 0});
            return;
        }
    }
    const int nb = K >> 8;
    const int row_bytes = nb * BYTES;
    const RowRes rr = row_rsrc(w + id * row_bytes, row_bytes);
    const __amdgpu_buffer_rsrc_t rs = rr.rs;
    const int e0 = c * 16;
    const int boff = rr.ex + (e0 >> 8) * BYTES;
    const int pos = e0 & 255;
    const int h = pos >> 7, j = (pos >> 5) & 3, l0 = pos & 31;
    const int r = boff & 3;
    const u32x4 ql = realign16(load_raw16(rs, boff + 64 * h + 32 * (j & 1) + l0), r);
    const u32x4 qh = realign16(load_raw16(rs, boff + 128 + 32 * h + l0), r);
    const u32x4 S = realign16(load_raw16(rs, boff + 192), r);
    const float d = q6_d(rs, boff);
    // scale 8h + 2j + l0/16: dword 2h + (j >> 1), byte 2(j & 1) + l0/16
    const uint32_t sw = h ? ((j & 2) ? S.w : S.z) : ((j & 2) ? S.y : S.x);
    const float ds = d * scale_byte(sw, 2 * (j & 1) + (l0 >> 4));
    uint32_t packed[8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        // ql word m holds weights 4m..4m+3 of this thread in nibble j>>1,
        // qh word m their high bits at 2j.
        const uint32_t lo = ((j & 2) ? (ql[m] >> 4) : ql[m]) & 0x0F0F0F0Fu;
        const uint32_t hb = ((qh[m] >> (2 * j)) & 0x03030303u) << 4;
        const uint32_t q = lo | hb;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float v0 = ds * (float)((int)((q >> (16 * e)) & 0xFFu) - 32);
            float v1 = ds * (float)((int)((q >> (16 * e + 8)) & 0xFFu) - 32);
            // Keep the product and the fp16 rounding apart: fused into
            // v_fma_mix with a +0 addend, a -0 product (q = 32, d*sc < 0)
            // would come out +0 where the reference writes -0.
            asm volatile("" : "+v"(v0), "+v"(v1));
            packed[2 * m + e] = (uint32_t)f32_to_f16_bits(v0) | ((uint32_t)f32_to_f16_bits(v1) << 16);
        }
    }
    store16_nt(out, u32x4{packed[0], packed[1], packed[2], packed[3]});
    store16_nt(out + 1, u32x4{packed[4], packed[5], packed[6], packed[7]});
}

hipError_t launch_kq_embed(uint16_t *dst, const uint8_t *w, const int32_t *ids, int token_id,
                           int64_t n_vocab, int n_ids, int K, hipStream_t st) {
    const int64_t threads = (int64_t)n_ids * (K / 16);
    const int64_t grid = (threads + 255) / 256;
    // the uniform kernel forms the wave index blockIdx.x * 4 + w in 32 bits
    if (grid > (int64_t)1 << 30) return hipErrorInvalidValue;
    const bool uniform = (K / 16) % 64 == 0;
    if (ids) {
        if (uniform)
            embed_q6k_kernel<true, true><<<(unsigned)grid, 256, 0, st>>>(dst, w, ids, 0, n_vocab, n_ids, K);
        else
            embed_q6k_kernel<true, false><<<(unsigned)grid, 256, 0, st>>>(dst, w, ids, 0, n_vocab, n_ids, K);
    } else if (uniform) {
        embed_q6k_kernel<false, true><<<(unsigned)grid, 256, 0, st>>>(dst, w, nullptr, token_id, 0, 1, K);
    } else {
        embed_q6k_kernel<false, false><<<(unsigned)grid, 256, 0, st>>>(dst, w, nullptr, token_id, 0, 1, K);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- GEMM
// Small-batch product y[N x M] = x[N x K] . dequant(W)^T for Q5_K/Q6_K:
// a workgroup of 4 waves owns 16*RT weight rows x 16 tokens (grid.y walks
// the token chunks); the blocks of K are dealt to the waves round-robin and the
// partial tiles added in wave order through LDS.  Per 32-k step a lane
// dequantises the 8 weights of its MFMA src0 fragment (row l%16, k 8*(l/16)..)
// in fp32 -- Q6_K d*sc*(q-32) exact, Q5_K (d*sc)*q - dmin*m with one
// rounding, as the reference -- then rounds them to the x type.  x rows past
// N read zeros through a bounded buffer resource.
template <int T, int XT>
__device__ __forceinline__ void kq_fragments(__amdgpu_buffer_rsrc_t rs, int boff, int g,
                                             u32x4 *a) {
    if constexpr (T == 14) {
        const int r = boff & 3;
        const Raw16 sraw = load_raw16(rs, boff + 192);
        const float d = q6_d(rs, boff);
        // ql bytes 8g.. of the four 32-byte quarter rows, qh bytes 8g.. of the two halves.
        u32x4 ql[2][2], qh[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            ql[h][0] = realign16(load_raw16(rs, boff + 64 * h + 8 * g), r);
            ql[h][1] = realign16(load_raw16(rs, boff + 64 * h + 32 + 8 * g), r);
            qh[h] = realign16(load_raw16(rs, boff + 128 + 32 * h + 8 * g), r);
        }
        const u32x4 S = realign16(sraw, r);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int h = t >> 2, j = t & 3;
            // scale 8h + 2j + g/2: dword 2h + (j >> 1), byte 2(j & 1) + g/2
            const float ds = d * scale_byte(S[2 * h + (j >> 1)], 2 * (j & 1) + (g >> 1));
            uint32_t o[4];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint32_t src = ql[h][j & 1][m];
                const uint32_t lo = ((j & 2) ? (src >> 4) : src) & 0x0F0F0F0Fu;
                const uint32_t q = lo | (((qh[h][m] >> (2 * j)) & 0x03030303u) << 4);
                o[2 * m] = pack2<XT>(ds * (float)((int)(q & 0xFFu) - 32),
                                     ds * (float)((int)((q >> 8) & 0xFFu) - 32));
                o[2 * m + 1] = pack2<XT>(ds * (float)((int)((q >> 16) & 0xFFu) - 32),
                                         ds * (float)((int)(q >> 24) - 32));
            }
            a[t] = u32x4{o[0], o[1], o[2], o[3]};
        }
    } else {
        const u32x4 hdr = buffer_load16(rs, boff);
        const u32x2 qh = buffer_load8(rs, boff + 16 + 8 * g);
        u32x2 qs[4];
#pragma unroll
        for (int il = 0; il < 4; ++il) qs[il] = buffer_load8(rs, boff + 48 + 32 * il + 8 * g);
        const float d = f16_bits_to_f32(hdr.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int il = t >> 1, hi = t & 1;
            uint32_t sc, mn;
            scale_one(hdr.y, hdr.z, hdr.w, t, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            uint32_t o[4];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint32_t lo = (hi ? (qs[il][m] >> 4) : qs[il][m]) & 0x0F0F0F0Fu;
                const uint32_t q = lo | (((qh[m] >> (2 * il + hi)) & 0x01010101u) << 4);
                o[2 * m] = pack2<XT>(ds * (float)(q & 0xFFu) - dm, ds * (float)((q >> 8) & 0xFFu) - dm);
                o[2 * m + 1] =
                    pack2<XT>(ds * (float)((q >> 16) & 0xFFu) - dm, ds * (float)(q >> 24) - dm);
            }
            a[t] = u32x4{o[0], o[1], o[2], o[3]};
        }
    }
}

template <int T, int XT, int YT, int RT, int TT>
__global__ __launch_bounds__(256) void kq_tokens_kernel(void *__restrict__ y,
                                                        const uint8_t *__restrict__ w,
                                                        const uint16_t *__restrict__ x, int M,
                                                        int N, int K) {
    constexpr int BYTES = KqFormat<T>::kBytes;
    constexpr int NF = RT * TT;  // 16 x 16 output fragments per wave
    __shared__ f32x4 part[4][NF][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 15, g = lane >> 4;
    const int nb = K >> 8;
    const int row_bytes = nb * BYTES;
    const int row0 = blockIdx.x * 16 * RT;
    const int tok0 = blockIdx.y * 16 * TT;
    const int n_rows = min(16 * RT, M - row0), n_tok = min(16 * TT, N - tok0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w + (int64_t)row0 * row_bytes, n_rows * row_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + (int64_t)tok0 * K, n_tok * K * 2);
    f32x4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K blocks round-robin over the 4 waves; each block's RT weight
    // fragments are dequantised once and used for all TT token fragments.
    for (int b = wave; b < nb; b += 4) {
        u32x4 a[RT][8];
#pragma unroll
        for (int r = 0; r < RT; ++r)
            kq_fragments<T, XT>(rs, (16 * r + li) * row_bytes + b * BYTES, g, a[r]);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            u32x4 bx[8];
            const int xoff = (16 * t + li) * K * 2 + 16 * g + 2 * 256 * b;
#pragma unroll
            for (int k = 0; k < 8; ++k) bx[k] = buffer_load16(xr, xoff + 2 * 32 * k);
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[r][t] = mfma<XT>(a[r][k], bx[k], acc[r][t]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) part[wave][r * TT + t][lane] = acc[r][t];
    __syncthreads();
    // Fragment f is reduced (waves in order) and stored by wave f % 4.
    for (int f = wave; f < NF; f += 4) {
        const int r = f / TT, t = f % TT;
        f32x4 s = part[0][f][lane];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            const f32x4 o = part[j][f][lane];
            s = f32x4{s[0] + o[0], s[1] + o[1], s[2] + o[2], s[3] + o[3]};
        }
        const int tok = 16 * t + li;
        if (tok < n_tok) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = 16 * r + 4 * g + q;
                if (row < n_rows) store_out<YT>(y, (int64_t)(tok0 + tok) * M + row0 + row, s[q]);
            }
        }
    }
}

template <int T, int XT, int YT, int RT, int TT>
static void launch_kq_tok(dim3 grid, void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                          int K, hipStream_t st) {
    kq_tokens_kernel<T, XT, YT, RT, TT><<<grid, 256, 0, st>>>(y, w, x, M, N, K);
}

// Small batches (the C ABI sends more than 16 tokens to the eight-wave GEMM
// of gemm_q4k.hip): one 16-token fragment per workgroup (grid.y walks the
// 16-token chunks), 32 rows when that still gives a workgroup per CU.
template <int T, int XT, int YT>
static hipError_t launch_kq_tokens_xy(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                      int K, hipStream_t st) {
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    const int chunks = (N + 15) / 16;
    const int rt = (int64_t)((M + 31) / 32) * chunks >= cus ? 2 : 1;
    const dim3 grid((M + 16 * rt - 1) / (16 * rt), chunks);
    if (grid.y > 65535) return hipErrorInvalidValue;
    if (rt == 2) launch_kq_tok<T, XT, YT, 2, 1>(grid, y, w, x, M, N, K, st);
    else launch_kq_tok<T, XT, YT, 1, 1>(grid, y, w, x, M, N, K, st);
    return hipGetLastError();
}

template <int T>
static hipError_t launch_kq_tokens_t(void *y, int y_dtype, const uint8_t *w, const void *x,
                                     int x_dtype, int M, int N, int K, hipStream_t st) {
    const int64_t row_bytes = (int64_t)(K / 256) * KqFormat<T>::kBytes;
    if (row_bytes * 32 > 0x7FFFFFFF || (int64_t)128 * K * 2 > 0x7FFFFFFF) return hipErrorInvalidValue;
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            return launch_kq_tokens_xy<T, RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16>(y, w, xx, M, N, K, st);
        return launch_kq_tokens_xy<T, RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st);
    }
    if (y_dtype == RXQ4_DTYPE_F16)
        return launch_kq_tokens_xy<T, RXQ4_DTYPE_F16, RXQ4_DTYPE_F16>(y, w, xx, M, N, K, st);
    return launch_kq_tokens_xy<T, RXQ4_DTYPE_F16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st);
}

hipError_t launch_kq_tokens(int ggml_type, void *y, int y_dtype, const uint8_t *w, const void *x,
                            int x_dtype, int M, int N, int K, hipStream_t st) {
    if (ggml_type == 14) return launch_kq_tokens_t<14>(y, y_dtype, w, x, x_dtype, M, N, K, st);
    if (ggml_type == 13) return launch_kq_tokens_t<13>(y, y_dtype, w, x, x_dtype, M, N, K, st);
    return hipErrorInvalidValue;
}

}  // namespace rxq4
