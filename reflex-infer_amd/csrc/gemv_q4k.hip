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
//   * rows are reduced across their lanes with cross-lane adds.
// Work: ~1.5 VALU ops per weight, under the ~2.8 ops/weight that 8 TB/s of
// 4.5-bit weights leaves on 256 CUs.  Bytes per launch: rows*K/256*144 +
// K*2 + rows*out_bytes (+ rows*2 residual).
#include "launch.h"
#include "q4k_device.h"

#include <stdlib.h>
#include <string.h>

namespace rxq4 {

// The 64 activations of one slot, as fp16 pairs in nibble order, plus sums.
struct XSlot {
    uint32_t p[32];
    float bias_lo, bias_hi;  // -1024 * sum
    float sx_lo, sx_hi;      // sum of the 32 low-nibble / high-nibble activations
};

// Load the slot (b, il) of x: elements b*256 + 64*il + [0, 64).  For quant
// dword k (bytes 4k..4k+3 of the group) the pairs are
//   p[4k+0] = (x_lo[4k],   x_lo[4k+2])   p[4k+1] = (x_lo[4k+1], x_lo[4k+3])
//   p[4k+2] = (x_hi[4k],   x_hi[4k+2])   p[4k+3] = (x_hi[4k+1], x_hi[4k+3])
// matching (q & 0x000F000F) and ((q >> 8) & 0x000F000F) (and 0x00F000F0).
__device__ __forceinline__ void load_x_slot(const uint16_t *__restrict__ x, int b, int il,
                                            bool valid, XSlot &s) {
    uint32_t xl[16], xh[16];
    if (valid) {
        const uint16_t *base = x + b * kQK + 64 * il;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 lo = load16(base + 8 * i);
            const u32x4 hi = load16(base + 32 + 8 * i);
            xl[4 * i + 0] = lo.x; xl[4 * i + 1] = lo.y; xl[4 * i + 2] = lo.z; xl[4 * i + 3] = lo.w;
            xh[4 * i + 0] = hi.x; xh[4 * i + 1] = hi.y; xh[4 * i + 2] = hi.z; xh[4 * i + 3] = hi.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) { xl[i] = 0; xh[i] = 0; }
    }
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t a = xl[2 * k], c = xl[2 * k + 1];
        s.p[4 * k + 0] = (a & 0xFFFFu) | (c << 16);
        s.p[4 * k + 1] = (a >> 16) | (c & 0xFFFF0000u);
        const uint32_t e = xh[2 * k], f = xh[2 * k + 1];
        s.p[4 * k + 2] = (e & 0xFFFFu) | (f << 16);
        s.p[4 * k + 3] = (e >> 16) | (f & 0xFFFF0000u);
        sl += f16_bits_to_f32(a) + f16_bits_to_f32(a >> 16) + f16_bits_to_f32(c) +
              f16_bits_to_f32(c >> 16);
        sh += f16_bits_to_f32(e) + f16_bits_to_f32(e >> 16) + f16_bits_to_f32(f) +
              f16_bits_to_f32(f >> 16);
    }
    s.sx_lo = sl;
    s.sx_hi = sh;
    s.bias_lo = -1024.0f * sl;
    s.bias_hi = -1024.0f * sh;
}

// Partial dot product of one slot of one row.
__device__ __forceinline__ float slot_dot(u32x4 hdr, u32x4 q0, u32x4 q1, const XSlot &s,
                                          int il) {
    const float d = f16_bits_to_f32(hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    uint32_t sc, mn;
    scale_pair(hdr.y, hdr.z, hdr.w, il, &sc, &mn);
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float acc_lo = s.bias_lo, acc_hi = s.bias_hi;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = q[k], v8 = q[k] >> 8;
        acc_lo = __builtin_amdgcn_fdot2(as_half2((v & 0x000F000Fu) | 0x64006400u),
                                        as_half2(s.p[4 * k + 0]), acc_lo, false);
        acc_lo = __builtin_amdgcn_fdot2(as_half2((v8 & 0x000F000Fu) | 0x64006400u),
                                        as_half2(s.p[4 * k + 1]), acc_lo, false);
        acc_hi = __builtin_amdgcn_fdot2(as_half2((v & 0x00F000F0u) | 0x64006400u),
                                        as_half2(s.p[4 * k + 2]), acc_hi, false);
        acc_hi = __builtin_amdgcn_fdot2(as_half2((v8 & 0x00F000F0u) | 0x64006400u),
                                        as_half2(s.p[4 * k + 3]), acc_hi, false);
    }
    const float d_lo = d * (float)(sc & 0xFFu);
    const float d_hi = d * (float)(sc >> 8) * 0.0625f;
    const float m_lo = dmin * (float)(mn & 0xFFu);
    const float m_hi = dmin * (float)(mn >> 8);
    return d_lo * acc_lo - m_lo * s.sx_lo + (d_hi * acc_hi - m_hi * s.sx_hi);
}

// The (up to three) output ranges as plain values.  Kernels copy them out of
// the parameter block field by field so that selecting a range is a register
// select, never an indexed load from a stack copy of the parameters.
struct Ranges {
    const uint8_t *w0, *w1, *w2;
    void *y0, *y1, *y2;
    const uint16_t *r0, *r1, *r2;
    int m0, m1, n;
};

__device__ __forceinline__ Ranges ranges_of(const GemvParams &p) {
    return Ranges{p.r[0].w, p.r[1].w, p.r[2].w, p.r[0].y, p.r[1].y, p.r[2].y,
                  p.r[0].res, p.r[1].res, p.r[2].res, p.r[0].rows, p.r[1].rows, p.n_ranges};
}

// Row -> (range, local row).  Ranges are concatenated in order.
__device__ __forceinline__ int locate(const Ranges &g, int row, int *local) {
    int ri = 0;
    if (g.n > 1 && row >= g.m0) {
        row -= g.m0;
        ri = 1;
        if (g.n > 2 && row >= g.m1) {
            row -= g.m1;
            ri = 2;
        }
    }
    *local = row;
    return ri;
}

__device__ __forceinline__ const uint8_t *range_w(const Ranges &g, int ri) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(g.w0), b = reinterpret_cast<uintptr_t>(g.w1),
                    c = reinterpret_cast<uintptr_t>(g.w2);
    return reinterpret_cast<const uint8_t *>(ri == 0 ? a : (ri == 1 ? b : c));
}

template <int EPI>
__device__ __forceinline__ void store_row(const Ranges &g, int ri, int local, float v) {
    const uintptr_t ya = reinterpret_cast<uintptr_t>(g.y0), yb = reinterpret_cast<uintptr_t>(g.y1),
                    yc = reinterpret_cast<uintptr_t>(g.y2);
    void *y = reinterpret_cast<void *>(ri == 0 ? ya : (ri == 1 ? yb : yc));
    if (EPI == kEpiF32) {
        static_cast<float *>(y)[local] = v;
    } else if (EPI == kEpiF16) {
        static_cast<uint16_t *>(y)[local] = f32_to_f16_bits(v);
    } else {
        const uintptr_t ra = reinterpret_cast<uintptr_t>(g.r0), rb = reinterpret_cast<uintptr_t>(g.r1),
                        rc = reinterpret_cast<uintptr_t>(g.r2);
        const uint16_t *res = reinterpret_cast<const uint16_t *>(ri == 0 ? ra : (ri == 1 ? rb : rc));
        const float projected = f16_bits_to_f32(f32_to_f16_bits(v));
        static_cast<uint16_t *>(y)[local] =
            f32_to_f16_bits(projected + f16_bits_to_f32(res[local]));
    }
}

// Register kernel: a row has LPR = 4*nb <= 64 slots (nb in {1,2,4,8,16}), so
// a wave covers 64/LPR rows per step and each lane's slot never changes.
// Wave w owns rows [w*rows_per_unit, (w+1)*rows_per_unit); U steps of loads
// are issued before any arithmetic.
template <int LPR, int EPI, int U>
__global__ __launch_bounds__(256) void gemv_reg_kernel(GemvParams p) {
    constexpr int RPS = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int row_begin = wave * p.rows_per_unit;
    if (row_begin >= p.total_rows) return;
    const int row_end = min(row_begin + p.rows_per_unit, p.total_rows);
    const int slot = lane & (LPR - 1);
    const int sub = lane / LPR;
    const int b = slot >> 2, il = slot & 3;
    const Ranges rg = ranges_of(p);

    XSlot xs;
    load_x_slot(p.x, b, il, true, xs);
    const int64_t row_bytes = (int64_t)p.nb * kBlockBytes;
    const int slot_off = b * kBlockBytes;

    for (int r0 = row_begin; r0 < row_end; r0 += RPS * U) {
        u32x4 h[U], a[U], c[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = min(r0 + u * RPS + sub, row_end - 1);
            int local;
            const int ri = locate(rg, row, &local);
            const uint8_t *blk = range_w(rg, ri) + local * row_bytes + slot_off;
            h[u] = load16(blk);
            a[u] = load16(blk + 16 + 32 * il);
            c[u] = load16(blk + 32 + 32 * il);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v = slot_dot(h[u], a[u], c[u], xs, il);
            v = group_sum<LPR>(v);
            const int row = r0 + u * RPS + sub;
            if (slot == 0 && row < row_end) {
                int local;
                const int ri = locate(rg, row, &local);
                store_row<EPI>(rg, ri, local, v);
            }
        }
    }
}

// Split kernel for rows with more than 64 slots: a workgroup of J waves covers
// one row, wave j holding slots [64j, 64j+64) in registers; per row the J
// wave sums meet in LDS and are added in wave order.  Workgroup g owns rows
// [g*rows_per_unit, (g+1)*rows_per_unit), U rows per round.
constexpr int kMaxSplitWaves = 16;

template <int EPI, int U>
__global__ __launch_bounds__(1024) void gemv_split_kernel(GemvParams p) {
    __shared__ float part[2][kMaxSplitWaves][U];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int n_waves = blockDim.x >> 6;
    const int slot = wv * 64 + lane;
    const bool valid = slot < 4 * p.nb;
    const int b = slot >> 2, il = slot & 3;
    const int row_begin = blockIdx.x * p.rows_per_unit;
    const int row_end = min(row_begin + p.rows_per_unit, p.total_rows);
    const Ranges rg = ranges_of(p);

    XSlot xs;
    load_x_slot(p.x, b, il, valid, xs);
    const int64_t row_bytes = (int64_t)p.nb * kBlockBytes;
    const int slot_off = b * kBlockBytes;

    int buf = 0;
    for (int r0 = row_begin; r0 < row_end; r0 += U, buf ^= 1) {
        u32x4 h[U], a[U], c[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (valid) {
                const int row = min(r0 + u, row_end - 1);
                int local;
                const int ri = locate(rg, row, &local);
                const uint8_t *blk = range_w(rg, ri) + local * row_bytes + slot_off;
                h[u] = load16(blk);
                a[u] = load16(blk + 16 + 32 * il);
                c[u] = load16(blk + 32 + 32 * il);
            } else {
                h[u] = u32x4{0, 0, 0, 0};
                a[u] = h[u];
                c[u] = h[u];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v = valid ? slot_dot(h[u], a[u], c[u], xs, il) : 0.0f;
            v = group_sum<64>(v);
            if (lane == 0) part[buf][wv][u] = v;
        }
        __syncthreads();
        if (wv == 0 && lane < U) {
            const int row = r0 + lane;
            if (row < row_end) {
                float s = 0.0f;
                for (int j = 0; j < n_waves; ++j) s += part[buf][j][lane];
                int local;
                const int ri = locate(rg, row, &local);
                store_row<EPI>(rg, ri, local, s);
            }
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

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

template <int LPR, int EPI>
static void launch_reg(const GemvParams &p, int grid, hipStream_t st) {
    gemv_reg_kernel<LPR, EPI, 4><<<grid, 256, 0, st>>>(p);
}

template <int EPI>
static hipError_t launch_gemv_epi(GemvParams p, hipStream_t st) {
    const int slots = 4 * p.nb;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    if (slots <= 64 && (64 % slots) == 0) {
        // Register kernel.  Aim for `waves_per_cu` resident waves per CU.
        const int rps = 64 / slots;
        const int waves_per_cu = env_int("RXQ4_GEMV_WAVES_PER_CU", 8);
        const int64_t steps = (p.total_rows + rps - 1) / rps;
        const int64_t target = (int64_t)cus * (waves_per_cu > 0 ? waves_per_cu : 8);
        int64_t steps_per_wave = (steps + target - 1) / target;
        if (steps_per_wave < 1) steps_per_wave = 1;
        p.rows_per_unit = (int)(steps_per_wave * rps);
        const int64_t waves = (p.total_rows + p.rows_per_unit - 1) / p.rows_per_unit;
        const int grid = (int)((waves + 3) / 4);
        switch (slots) {
            case 4: launch_reg<4, EPI>(p, grid, st); break;
            case 8: launch_reg<8, EPI>(p, grid, st); break;
            case 16: launch_reg<16, EPI>(p, grid, st); break;
            case 32: launch_reg<32, EPI>(p, grid, st); break;
            default: launch_reg<64, EPI>(p, grid, st); break;
        }
    } else {
        const int j = (slots + 63) / 64;
        if (j > kMaxSplitWaves) return hipErrorInvalidValue;
        constexpr int U = 4;
        const int groups_per_cu = env_int("RXQ4_GEMV_GROUPS_PER_CU", 16 / j > 1 ? 16 / j : 1);
        const int64_t target = (int64_t)cus * (groups_per_cu > 0 ? groups_per_cu : 1);
        int64_t rounds = ((int64_t)p.total_rows + U * target - 1) / (U * target);
        if (rounds < 1) rounds = 1;
        p.rows_per_unit = (int)(rounds * U);
        const int grid = (p.total_rows + p.rows_per_unit - 1) / p.rows_per_unit;
        gemv_split_kernel<EPI, U><<<grid, 64 * j, 0, st>>>(p);
    }
    return hipGetLastError();
}

hipError_t launch_gemv(GemvParams p, int epilogue, hipStream_t st) {
    switch (epilogue) {
        case kEpiF16: return launch_gemv_epi<kEpiF16>(p, st);
        case kEpiF32: return launch_gemv_epi<kEpiF32>(p, st);
        case kEpiAdd: return launch_gemv_epi<kEpiAdd>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rxq4
