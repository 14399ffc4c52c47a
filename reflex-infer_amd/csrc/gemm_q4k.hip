// gemm_q4k.hip -- Q4_K prefill GEMM and small-batch decode on gfx950 MFMA.
//
// Replaces the reference's batched path (q4_gemm.cu:1297-1356 scalar kernel,
// 1482-1636 mma.sync MMQ kernel, 1638-1740 host chunking).  The reference
// re-streams W once per 20-token chunk; here every launch reads W once per
// token tile of 16*TF tokens.
//
// Math: y[tok, row] = sum_k x[tok, k] * w[row, k] with w = d*sc*q - dmin*m
// rounded once to fp32 and then (RNE) to the operand type of x (fp16 or
// bf16), products accumulated in fp32 by v_mfma_f32_16x16x32_{f16,bf16}:
//   src0 (16 x 32) = weight rows, lane l holds row l%16, k = 8*(l/16) .. +8
//   src1 (32 x 16) = tokens,      lane l holds token l%16, same k
//   dst  (16 x 16) lane l holds rows 4*(l/16) + r (r < 4) of token l%16.
// A lane's 8 consecutive k of one sub-block are 8 quant bytes' low nibbles;
// the same 8 bytes' high nibbles are the same k of the next sub-block, so one
// 8-byte load feeds two MFMA k-steps.
//
// GEMM kernel: workgroup = 4 waves; wave w owns 64 weight rows (4 fragments)
// and all 16*TF tokens of the workgroup's token tile.  The x tile (16*TF
// tokens x 64 k) is staged in LDS, double buffered, and read by all 4 waves;
// weights are dequantised straight into MFMA operand registers, so no wave
// dequantises another wave's rows.  Flops per launch: 2*N*M*K.
#include "launch.h"
#include "q4k_device.h"
#include "rxq4.h"

namespace rxq4 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int XT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if (XT == RXQ4_DTYPE_BF16)
        return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
    return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

// Eight weights from the low (hi = false) or high nibbles of bytes v0, v1.
template <int XT>
__device__ __forceinline__ u32x4 dequant8(uint32_t v0, uint32_t v1, bool hi, float dsc,
                                          float dm) {
    const uint32_t m0 = hi ? (v0 >> 4) & 0x0F0F0F0Fu : v0 & 0x0F0F0F0Fu;
    const uint32_t m1 = hi ? (v1 >> 4) & 0x0F0F0F0Fu : v1 & 0x0F0F0F0Fu;
    float w[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        w[t] = dsc * (float)((m0 >> (8 * t)) & 0xFFu) - dm;
        w[4 + t] = dsc * (float)((m1 >> (8 * t)) & 0xFFu) - dm;
    }
    return u32x4{pack2<XT>(w[0], w[1]), pack2<XT>(w[2], w[3]), pack2<XT>(w[4], w[5]),
                 pack2<XT>(w[6], w[7])};
}

template <int XT>
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    if (XT == RXQ4_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int YT>
__device__ __forceinline__ void store_out(void *y, int64_t idx, float v) {
    if (YT == RXQ4_DTYPE_F32)
        static_cast<float *>(y)[idx] = v;
    else if (YT == RXQ4_DTYPE_F16)
        static_cast<uint16_t *>(y)[idx] = f32_to_f16_bits(v);
    else
        static_cast<uint16_t *>(y)[idx] = f32_to_bf16_bits(v);
}

// Per-lane scale state of one weight row in one super-block.
struct RowScales {
    float d, dmin;
    uint32_t s0, s1, s2;
};

__device__ __forceinline__ RowScales row_scales(u32x4 h) {
    return RowScales{f16_bits_to_f32(h.x & 0xFFFFu), f16_bits_to_f32(h.x >> 16), h.y, h.z, h.w};
}

// ---------------------------------------------------------------------------
// Tiled GEMM.
constexpr int kGemmWaves = 4;
constexpr int kRowsPerWave = 64;   // 4 MFMA row fragments
constexpr int kRowsPerWg = kGemmWaves * kRowsPerWave;
constexpr int kXStride = 72;       // halves per token row in LDS (64 k + 8 pad)

template <int XT, int YT, int TF>
__global__ __launch_bounds__(256) void gemm_kernel(void *__restrict__ y,
                                                   const uint8_t *__restrict__ w,
                                                   const uint16_t *__restrict__ x, int M, int N,
                                                   int K) {
    constexpr int TM = 16 * TF;            // tokens per workgroup
    constexpr int XCHUNKS = TM * 8 / 256;  // 16-byte x chunks per thread per stage
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][TM * kXStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 15;   // row within fragment / token within fragment
    const int g = lane >> 4;    // k group of 8
    const int nb = K >> 8;
    const int64_t row_bytes = (int64_t)nb * kBlockBytes;
    const int row_base = blockIdx.x * kRowsPerWg + wave * kRowsPerWave;
    const int tok_base = blockIdx.y * TM;

    const uint8_t *wrow[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        const int r = min(row_base + 16 * f + li, M - 1);
        wrow[f] = w + r * row_bytes;
    }

    // x tile loader: chunk c -> token c/8, 8 halves at k offset 8*(c%8).
    u32x4 xr[XCHUNKS];
    auto load_x = [&](int stage) {
        const int k0 = stage * 64;
#pragma unroll
        for (int i = 0; i < XCHUNKS; ++i) {
            const int c = tid + 256 * i;
            const int t = tok_base + (c >> 3);
            if (t < N)
                xr[i] = load16(x + (int64_t)t * K + k0 + 8 * (c & 7));
            else
                xr[i] = u32x4{0, 0, 0, 0};
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XCHUNKS; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<u32x4 *>(&xs[buf][(c >> 3) * kXStride + 8 * (c & 7)]) = xr[i];
        }
    };

    f32x4 acc[4][TF];
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int t = 0; t < TF; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int stages = nb * 4;
    u32x4 hdr[4];
    u32x2 q8[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        hdr[f] = load16(wrow[f]);
        q8[f] = *reinterpret_cast<const u32x2 *>(wrow[f] + 16 + 8 * g);
    }
    load_x(0);
    store_x(0);
    __syncthreads();

    for (int s = 0; s < stages; ++s) {
        const int buf = s & 1;
        const int sb = s >> 2, il = s & 3;
        // Prefetch the next stage's x and quant bytes.
        u32x4 hdr_next[4];
        u32x2 q8_next[4];
        const bool more = s + 1 < stages;
        if (more) {
            load_x(s + 1);
            const int sbn = (s + 1) >> 2, iln = (s + 1) & 3;
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const uint8_t *blk = wrow[f] + sbn * kBlockBytes;
                if (iln == 0) hdr_next[f] = load16(blk);
                q8_next[f] = *reinterpret_cast<const u32x2 *>(blk + 16 + 32 * iln + 8 * g);
            }
        }
        // Dequantise this stage's 4 row fragments x 2 k-steps.
        u32x4 a_lo[4], a_hi[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const RowScales rs = row_scales(hdr[f]);
            uint32_t sc, mn;
            scale_pair(rs.s0, rs.s1, rs.s2, il, &sc, &mn);
            const float dsc_lo = rs.d * (float)(sc & 0xFFu), dm_lo = rs.dmin * (float)(mn & 0xFFu);
            const float dsc_hi = rs.d * (float)(sc >> 8), dm_hi = rs.dmin * (float)(mn >> 8);
            a_lo[f] = dequant8<XT>(q8[f].x, q8[f].y, false, dsc_lo, dm_lo);
            a_hi[f] = dequant8<XT>(q8[f].x, q8[f].y, true, dsc_hi, dm_hi);
        }
        const uint16_t *xb = xs[buf];
#pragma unroll
        for (int t = 0; t < TF; ++t) {
            const u32x4 b_lo =
                *reinterpret_cast<const u32x4 *>(&xb[(16 * t + li) * kXStride + 8 * g]);
            const u32x4 b_hi =
                *reinterpret_cast<const u32x4 *>(&xb[(16 * t + li) * kXStride + 32 + 8 * g]);
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                acc[f][t] = mfma<XT>(a_lo[f], b_lo, acc[f][t]);
                acc[f][t] = mfma<XT>(a_hi[f], b_hi, acc[f][t]);
            }
        }
        (void)sb;
        if (more) {
            store_x(buf ^ 1);
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                if (((s + 1) & 3) == 0) hdr[f] = hdr_next[f];
                q8[f] = q8_next[f];
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds rows row_base + 16f + 4g + r of token tok_base + 16t + li.
#pragma unroll
    for (int t = 0; t < TF; ++t) {
        const int tok = tok_base + 16 * t + li;
        if (tok >= N) continue;
#pragma unroll
        for (int f = 0; f < 4; ++f) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row_base + 16 * f + 4 * g + r;
                if (row < M) store_out<YT>(y, (int64_t)tok * M + row, acc[f][t][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Small batch (2..16 tokens): one 16-row x 16-token output fragment per
// workgroup, the K super-blocks split over 4 waves, x fragments read straight
// from global memory (the whole x is a few KB and stays in L2), partial sums
// added in wave order through LDS.
template <int XT, int YT>
__global__ __launch_bounds__(256) void gemv_tokens_kernel(void *__restrict__ y,
                                                          const uint8_t *__restrict__ w,
                                                          const uint16_t *__restrict__ x, int M,
                                                          int N, int K) {
    __shared__ f32x4 part[4][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 15;
    const int g = lane >> 4;
    const int nb = K >> 8;
    const int row0 = blockIdx.x * 16;
    const int64_t row_bytes = (int64_t)nb * kBlockBytes;
    const uint8_t *wr = w + min(row0 + li, M - 1) * row_bytes;
    const bool tok_ok = li < N;
    const uint16_t *xt = x + (int64_t)(tok_ok ? li : 0) * K;

    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sb = wave; sb < nb; sb += 4) {
        const uint8_t *blk = wr + sb * kBlockBytes;
        const RowScales rs = row_scales(load16(blk));
        u32x2 q[4];
        u32x4 b[8];
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            q[il] = *reinterpret_cast<const u32x2 *>(blk + 16 + 32 * il + 8 * g);
            const int k0 = sb * 256 + 64 * il + 8 * g;
            b[2 * il] = tok_ok ? load16(xt + k0) : u32x4{0, 0, 0, 0};
            b[2 * il + 1] = tok_ok ? load16(xt + k0 + 32) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            uint32_t sc, mn;
            scale_pair(rs.s0, rs.s1, rs.s2, il, &sc, &mn);
            const u32x4 a_lo = dequant8<XT>(q[il].x, q[il].y, false, rs.d * (float)(sc & 0xFFu),
                                            rs.dmin * (float)(mn & 0xFFu));
            const u32x4 a_hi = dequant8<XT>(q[il].x, q[il].y, true, rs.d * (float)(sc >> 8),
                                            rs.dmin * (float)(mn >> 8));
            acc = mfma<XT>(a_lo, b[2 * il], acc);
            acc = mfma<XT>(a_hi, b[2 * il + 1], acc);
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        f32x4 s = part[0][lane];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            const f32x4 o = part[j][lane];
            s = f32x4{s[0] + o[0], s[1] + o[1], s[2] + o[2], s[3] + o[3]};
        }
        if (tok_ok) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + 4 * g + r;
                if (row < M) store_out<YT>(y, (int64_t)li * M + row, s[r]);
            }
        }
    }
}

template <int XT, int YT>
static hipError_t launch_gemm_t(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                int K, hipStream_t st) {
    constexpr int TF = 8;  // 128 tokens per workgroup
    const dim3 grid((M + kRowsPerWg - 1) / kRowsPerWg, (N + 16 * TF - 1) / (16 * TF));
    gemm_kernel<XT, YT, TF><<<grid, 256, 0, st>>>(y, w, x, M, N, K);
    return hipGetLastError();
}

hipError_t launch_gemm(void *y, int y_dtype, const uint8_t *w, const void *x, int x_dtype,
                       int M, int N, int K, hipStream_t st) {
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            return launch_gemm_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16>(y, w, xx, M, N, K, st);
        return launch_gemm_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st);
    }
    if (y_dtype == RXQ4_DTYPE_F16)
        return launch_gemm_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F16>(y, w, xx, M, N, K, st);
    return launch_gemm_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st);
}

hipError_t launch_gemv_tokens(void *y, int y_dtype, const uint8_t *w, const void *x,
                              int x_dtype, int M, int n_tok, int K, hipStream_t st) {
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    const int grid = (M + 15) / 16;
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            gemv_tokens_kernel<RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16><<<grid, 256, 0, st>>>(y, w, xx, M, n_tok, K);
        else
            gemv_tokens_kernel<RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32><<<grid, 256, 0, st>>>(y, w, xx, M, n_tok, K);
    } else {
        if (y_dtype == RXQ4_DTYPE_F16)
            gemv_tokens_kernel<RXQ4_DTYPE_F16, RXQ4_DTYPE_F16><<<grid, 256, 0, st>>>(y, w, xx, M, n_tok, K);
        else
            gemv_tokens_kernel<RXQ4_DTYPE_F16, RXQ4_DTYPE_F32><<<grid, 256, 0, st>>>(y, w, xx, M, n_tok, K);
    }
    return hipGetLastError();
}

}  // namespace rxq4
