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
// tokens x 64 k) is staged in LDS, in a ring of 4 stages, and read by all 4 waves;
// weights are dequantised straight into MFMA operand registers, so no wave
// dequantises another wave's rows.  Flops per launch: 2*N*M*K.
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "launch.h"
#include "q4k_device.h"
#include "rxq4.h"

namespace rxq4 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> one packed pair, RNE (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
template <int XT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if (XT == RXQ4_DTYPE_BF16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// v & mask as an opaque value, so that the byte extracts below stay
// v_cvt_f32_ubyte{0..3} instead of being folded into bit-field extracts.
__device__ __forceinline__ uint32_t mask_opaque(uint32_t v, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(mask), "v"(v));
    return r;
}

// Four weights from the four bytes of m (each a nibble value, or 16 x a
// nibble value when `scale` carries the factor 1/16): w = scale*b - dm.
// The products are exact, so each w has the single fp32 rounding of the
// reference formula d*sc*q - dmin*m.
template <int XT>
__device__ __forceinline__ void dequant4(uint32_t m, float scale, float dm, uint32_t *out) {
    const float w0 = scale * (float)(m & 0xFFu) - dm;
    const float w1 = scale * (float)((m >> 8) & 0xFFu) - dm;
    const float w2 = scale * (float)((m >> 16) & 0xFFu) - dm;
    const float w3 = scale * (float)(m >> 24) - dm;
    out[0] = pack2<XT>(w0, w1);
    out[1] = pack2<XT>(w2, w3);
}

// Eight weights from the low (hi = false) or high nibbles of bytes v0, v1.
// High nibbles are used in place (16*q) with dsc/16, an exact rescaling.
template <int XT>
__device__ __forceinline__ u32x4 dequant8(uint32_t v0, uint32_t v1, bool hi, float dsc,
                                          float dm) {
    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const float scale = hi ? dsc * 0.0625f : dsc;
    uint32_t o[4];
    dequant4<XT>(mask_opaque(v0, mask), scale, dm, o);
    dequant4<XT>(mask_opaque(v1, mask), scale, dm, o + 2);
    return u32x4{o[0], o[1], o[2], o[3]};
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
//
// Workgroup = 4 waves; wave w owns 64 weight rows (4 MFMA row fragments) and
// all TM = 16*TF tokens of the workgroup tile (256 rows x TM tokens).  K is
// walked in stages of 64 (one 32-byte quant group il of a super-block = two
// sub-blocks = two MFMA k-steps):
//   * activations: each stage's TM x 64 tile is copied global -> LDS by the
//     gfx950 direct-to-LDS loads (buffer_load_dwordx4 ... lds) into a ring
//     of 4 stage buffers, 3 stages ahead (issued right after the stage
//     barrier, when every wave has finished reading the buffer being
//     refilled).  Token t's 16-byte chunk c sits at position c ^ (t & 7) of
//     the token's 128-byte row, so the fragment reads
//     (16 tokens x 16 bytes per k-group) hit distinct banks;
//   * weights: each lane loads the 8 quant bytes of its fragment row three
//     stages ahead (the block header two stages ahead) and dequantises them
//     straight into MFMA operand registers, one stage ahead of use: the
//     dequantisation of stage s+1 (VALU) is written between the MFMAs of
//     stage s, one (fragment, half) per token fragment, so the two pipes
//     overlap;
//   * per stage: wait until this stage's copies have landed (vmcnt), one
//     workgroup barrier, refill the freed buffer, then 2 x 4 x TF MFMAs.
// The vmcnt bound is static: every stage issues the same loads (beyond the
// last stage they repeat the last stage's addresses into buffers that are
// never read), so "all but the two most recent stages' loads are done"
// is the constant kStageLoads*2 (+4 where one of them fetched a header).
// Split-K (splits > 1): each workgroup covers a range of super-blocks and
// writes its fp32 tile to a workspace; a second launch (gemm_reduce_kernel)
// adds the splits in split order and writes the output, so results do not
// depend on scheduling.  The kernel boundary between the two launches is the
// only synchronisation (no atomics, fences or spinning).
constexpr int kGemmWaves = 4;
constexpr int kRowsPerWave = 64;
constexpr int kRowsPerWg = kGemmWaves * kRowsPerWave;
constexpr int kRing = 4;

struct GemmParams {
    void *y;
    const uint8_t *w;
    const uint16_t *x;
    float *ws;      // split-K partial tiles [tile][split][TF*4][256 threads] float4
    int M, N, K, nb;
    int row_tiles, tok_tiles, splits, sb_per_split;
    int total_units, units_per_xcd;
};

template <int YT>
__device__ __forceinline__ void store4(void *y, int64_t idx, f32x4 v, bool vec_ok, int valid) {
    if (vec_ok) {
        if (YT == RXQ4_DTYPE_F32) {
            *reinterpret_cast<f32x4 *>(static_cast<float *>(y) + idx) = v;
        } else {
            uint32_t lo, hi;
            if (YT == RXQ4_DTYPE_F16) {
                lo = f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
                hi = f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
            } else {
                lo = f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
                hi = f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
            }
            *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(y) + idx) = u32x2{lo, hi};
        }
    } else {
        for (int r = 0; r < valid; ++r) store_out<YT>(y, idx + r, v[r]);
    }
}

template <int XT, int YT, int TF>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    constexpr int TM = 16 * TF;
    constexpr int kXLoads = TM / 32;           // 1 KB direct-to-LDS loads per wave per stage
    constexpr int kStageLoads = kXLoads + 4;   // + 4 quant-byte loads
    __shared__ __attribute__((aligned(1024))) uint8_t xs[kRing][TM * 128];

    const int L = blockIdx.x;
    const int V = (L % 8) * p.units_per_xcd + L / 8;  // consecutive units share an XCD
    if (V >= p.total_units) return;
    const int tok_tile = V % p.tok_tiles;
    const int rest = V / p.tok_tiles;
    const int row_tile = rest % p.row_tiles;
    const int split = rest / p.row_tiles;
    const int tile = row_tile * p.tok_tiles + tok_tile;
    const int sb0 = split * p.sb_per_split;
    const int nsb = min(p.nb, sb0 + p.sb_per_split) - sb0;
    const int n_stages = 4 * nsb;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int K = p.K;
    const int64_t row_bytes = (int64_t)p.nb * kBlockBytes;
    const int row_base = row_tile * kRowsPerWg + wave * kRowsPerWave;
    const int tok_base = tok_tile * TM;

    const uint8_t *wrow[4];
#pragma unroll
    for (int f = 0; f < 4; ++f)
        wrow[f] = p.w + (int64_t)min(row_base + 16 * f + li, p.M - 1) * row_bytes + sb0 * kBlockBytes;

    // Direct-to-LDS copy of stage s (clamped to the last stage), as MUBUF
    // buffer_load_dwordx4 ... lds over the workgroup's token rows (byte
    // offsets < TM*K*2 <= 16 MiB).  The MUBUF form keeps the compiler's
    // vmcnt bookkeeping for the register loads below exact; with the FLAT
    // form (global_load_lds) it waits for vmcnt(0) at every use.
    const int ctok = lane >> 3;                 // token within a 1 KB chunk
    const int cpos = (lane & 7) ^ ctok;         // global 16-byte chunk this lane fetches
    const __amdgpu_buffer_rsrc_t xrsrc =
        make_rsrc(p.x + (int64_t)tok_base * K, min(TM, p.N - tok_base) * K * 2);
    int xoff[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
        const int tok = min(8 * (wave + 4 * i) + ctok, p.N - 1 - tok_base);
        xoff[i] = (tok * K + 8 * cpos) * 2;
    }
    auto issue_x = [&](int s) {
        const int st = min(s, n_stages - 1);
        const int k0b = (sb0 * 4 + st) * 128;   // byte offset of the stage's 64 k
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int jc = wave + 4 * i;        // 1 KB chunk = 8 tokens
            buffer_to_lds16(xrsrc, &xs[s % kRing][jc * 1024], xoff[i] + k0b);
        }
    };
    auto load_q = [&](int s, u32x2 *q) {
        const int st = min(s, n_stages - 1);
        const int off = (st >> 2) * kBlockBytes + 16 + 32 * (st & 3) + 8 * g;
#pragma unroll
        for (int f = 0; f < 4; ++f) q[f] = *reinterpret_cast<const u32x2 *>(wrow[f] + off);
    };
    auto load_h = [&](int sbi, u32x4 *h) {
        const int sbc = min(sbi, nsb - 1);
#pragma unroll
        for (int f = 0; f < 4; ++f) h[f] = load16(wrow[f] + sbc * kBlockBytes);
    };

    f32x4 acc[4][TF];
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int t = 0; t < TF; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x2 q[4][4];      // quant bytes of stages s .. s+3 (ring by s % 4)
    u32x4 hcur[4], hnext[4];
    u32x4 a[2][8];      // dequantised operands of stages s (a[s&1]) and s+1: [f] lo, [4+f] hi

    // Operands of stage st (quant group il of the super-block whose headers
    // are h) into a[buf].
    auto dequant_stage = [&](const u32x2 *qs, const u32x4 *h, int il, u32x4 *out) {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const RowScales rs = row_scales(h[f]);
            uint32_t sc, mn;
            scale_pair(rs.s0, rs.s1, rs.s2, il, &sc, &mn);
            out[f] = dequant8<XT>(qs[f].x, qs[f].y, false, rs.d * (float)(sc & 0xFFu),
                                  rs.dmin * (float)(mn & 0xFFu));
            out[4 + f] = dequant8<XT>(qs[f].x, qs[f].y, true, rs.d * (float)(sc >> 8),
                                      rs.dmin * (float)(mn >> 8));
        }
    };

    // Prologue: stages 0..2 in flight, operands of stage 0 ready.
    issue_x(0);
    load_q(0, q[0]);
    load_h(0, hcur);
    issue_x(1);
    load_q(1, q[1]);
    issue_x(2);
    load_q(2, q[2]);
    dequant_stage(q[0], hcur, 0, a[0]);

    for (int sbi = 0; sbi < nsb; ++sbi) {
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            const int s = 4 * sbi + il;
            // Copies of stage s have landed once at most the two later
            // stages' loads are outstanding; then every wave is past stage
            // s-1, so buffer (s+3) % 4 may be refilled.
            if (il >= 2)
                wait_vmcnt<2 * kStageLoads + 4>();
            else
                wait_vmcnt<2 * kStageLoads>();
            lds_barrier();
            issue_x(s + 3);
            load_q(s + 3, q[(il + 3) & 3]);
            if (il == 1) load_h(sbi + 1, hnext);

            // MFMAs of stage s interleaved with the dequantisation of stage
            // s+1 (the next quant group, or group 0 of the next super-block).
            const u32x4 *acur = a[il & 1];
            u32x4 *anext = a[(il + 1) & 1];
            const u32x4 *hn = il == 3 ? hnext : hcur;
            const u32x2 *qn = q[(il + 1) & 3];
            const uint8_t *xb = xs[s % kRing];
#pragma unroll
            for (int t = 0; t < TF; ++t) {
                const int tt = 16 * t + li;
                const u32x4 b_lo =
                    *reinterpret_cast<const u32x4 *>(xb + tt * 128 + (((g) ^ (tt & 7)) << 4));
                const u32x4 b_hi =
                    *reinterpret_cast<const u32x4 *>(xb + tt * 128 + (((4 + g) ^ (tt & 7)) << 4));
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    acc[f][t] = mfma<XT>(acur[f], b_lo, acc[f][t]);
                    acc[f][t] = mfma<XT>(acur[4 + f], b_hi, acc[f][t]);
                }
                if (TF == 8) {
                    // one (fragment, half) of the next stage per token fragment
                    const int f = t >> 1;
                    const RowScales rs = row_scales(hn[f]);
                    uint32_t sc, mn;
                    scale_pair(rs.s0, rs.s1, rs.s2, (il + 1) & 3, &sc, &mn);
                    if ((t & 1) == 0)
                        anext[f] = dequant8<XT>(qn[f].x, qn[f].y, false, rs.d * (float)(sc & 0xFFu),
                                                rs.dmin * (float)(mn & 0xFFu));
                    else
                        anext[4 + f] = dequant8<XT>(qn[f].x, qn[f].y, true, rs.d * (float)(sc >> 8),
                                                    rs.dmin * (float)(mn >> 8));
                }
            }
            if (TF != 8) dequant_stage(qn, hn, (il + 1) & 3, anext);
            if (il == 3) {
#pragma unroll
                for (int f = 0; f < 4; ++f) hcur[f] = hnext[f];
            }
        }
    }
    wait_vmcnt<0>();  // trailing clamped copies must land before the workgroup exits

    if (p.splits > 1) {
        f32x4 *part = reinterpret_cast<f32x4 *>(p.ws) +
                      ((int64_t)(tile * p.splits + split) * (4 * TF)) * 256 + tid;
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int t = 0; t < TF; ++t) part[(f * TF + t) * 256] = acc[f][t];
        return;
    }
    const bool vec_ok = (p.M & 3) == 0;
    // lane holds rows row_base + 16f + 4g + r of token tok_base + 16t + li
#pragma unroll
    for (int t = 0; t < TF; ++t) {
        const int tok = tok_base + 16 * t + li;
        if (tok >= p.N) continue;
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int row = row_base + 16 * f + 4 * g;
            if (row >= p.M) continue;
            const int valid = min(4, p.M - row);
            store4<YT>(p.y, (int64_t)tok * p.M + row, acc[f][t], vec_ok && valid == 4, valid);
        }
    }
}

// Split-K reduction: block (tile, f*TF+t) sums the splits of one fragment
// set of the tile in split order; thread tid holds the same element positions
// as thread tid of the GEMM workgroups.
template <int YT, int TF>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
    constexpr int TM = 16 * TF;
    const int tid = threadIdx.x;
    const int tile = blockIdx.x / (4 * TF);
    const int ft = blockIdx.x % (4 * TF);
    const int f = ft / TF, t = ft % TF;
    const int row_tile = tile / p.tok_tiles, tok_tile = tile % p.tok_tiles;
    const int lane = tid & 63, wave = tid >> 6;
    const int tok = tok_tile * TM + 16 * t + (lane & 15);
    const int row = row_tile * kRowsPerWg + wave * kRowsPerWave + 16 * f + 4 * (lane >> 4);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.ws) +
                       ((int64_t)tile * p.splits * (4 * TF) + ft) * 256 + tid;
    f32x4 sum = src[0];
    for (int sp = 1; sp < p.splits; ++sp) {
        const f32x4 v = src[(int64_t)sp * (4 * TF) * 256];
        sum = f32x4{sum[0] + v[0], sum[1] + v[1], sum[2] + v[2], sum[3] + v[3]};
    }
    if (tok >= p.N || row >= p.M) return;
    const int valid = min(4, p.M - row);
    store4<YT>(p.y, (int64_t)tok * p.M + row, sum, (p.M & 3) == 0 && valid == 4, valid);
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

// Split-K workspace: one allocation per device on first use, grown on demand
// (never freed).  Split-K calls that overlap on one device share it.
struct SplitWorkspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};
static std::mutex g_ws_mutex;
static SplitWorkspace g_ws[64];

static hipError_t split_workspace(size_t bytes, float **ws) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    SplitWorkspace &w = g_ws[dev];
    if (w.bytes < bytes) {
        if (w.ptr) {
            if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        void *p = nullptr;
        if ((e = hipMalloc(&p, bytes)) != hipSuccess) return e;
        w.ptr = p;
        w.bytes = bytes;
    }
    *ws = static_cast<float *>(w.ptr);
    return hipSuccess;
}

static int env_or(const char *name, int dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    const int r = atoi(v);
    return r > 0 ? r : dflt;
}

template <int XT, int YT>
static hipError_t launch_gemm_t(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                int K, hipStream_t st) {
    constexpr int TF = 8;  // 128 tokens per workgroup
    constexpr int TM = 16 * TF;
    GemmParams p{};
    p.y = y;
    p.w = w;
    p.x = x;
    p.M = M;
    p.N = N;
    p.K = K;
    p.nb = K / 256;
    p.row_tiles = (M + kRowsPerWg - 1) / kRowsPerWg;
    p.tok_tiles = (N + TM - 1) / TM;
    const int tiles = p.row_tiles * p.tok_tiles;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    // Split K to the nearest whole number of launch waves over the CUs
    // (cus / tiles rounded), keeping >= 2 super-blocks a split: 128 tiles on
    // 256 CUs split 2, 172 tiles do not split.
    int splits = std::max(1, (cus + tiles / 2) / tiles);
    splits = std::min(splits, std::max(1, p.nb / 2));
    splits = env_or("RXQ4_GEMM_SPLITS", splits);
    splits = std::max(1, std::min(splits, p.nb));
    p.sb_per_split = (p.nb + splits - 1) / splits;
    splits = (p.nb + p.sb_per_split - 1) / p.sb_per_split;  // no empty splits
    p.splits = splits;
    if (splits > 1) {
        const size_t part = (size_t)tiles * splits * TM * kRowsPerWg * sizeof(float);
        hipError_t e = split_workspace(part, &p.ws);
        if (e != hipSuccess) return e;
    }
    p.total_units = tiles * splits;
    p.units_per_xcd = (p.total_units + 7) / 8;
    gemm_kernel<XT, YT, TF><<<8 * p.units_per_xcd, 256, 0, st>>>(p);
    if (splits > 1) gemm_reduce_kernel<YT, TF><<<tiles * 4 * TF, 256, 0, st>>>(p);
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
