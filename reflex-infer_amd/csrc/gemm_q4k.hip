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
// tokens x 64 k) is staged in LDS, in a ring of 5 stages, and read by all 4 waves;
// weights are dequantised straight into MFMA operand registers, so no wave
// dequantises another wave's rows.  Flops per launch: 2*N*M*K.
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "launch.h"
#include "mfma_util.h"
#include "q4k_device.h"
#include "rxq4.h"

namespace rxq4 {

// Two fp32 values from bytes 2*word, 2*word+1 of m.  Each byte is a nibble
// value q in [0, 15]; read as an FP8 E4M3 (OCP) pattern it is exactly
// q * 2^-9 (subnormal for q < 8), so v_cvt_pk_f32_fp8 turns two nibbles
// into exact floats with one instruction.
template <bool WORD>
__device__ __forceinline__ f32x2 nibbles_f32(uint32_t m) {
    return __builtin_amdgcn_cvt_pk_f32_fp8((int)m, WORD);
}

// Four weights from the four nibble bytes of m: w = scale512 * (q * 2^-9)
// - dm with scale512 = d*sc*512, i.e. d*sc*q - dmin*m with the single fp32
// rounding of the reference (the product is exact), then RNE to the operand
// type.
template <int XT>
__device__ __forceinline__ void dequant4(uint32_t m, float scale512, float dm, uint32_t *out) {
    const f32x2 f01 = nibbles_f32<false>(m), f23 = nibbles_f32<true>(m);
    out[0] = pack2<XT>(scale512 * f01[0] - dm, scale512 * f01[1] - dm);
    out[1] = pack2<XT>(scale512 * f23[0] - dm, scale512 * f23[1] - dm);
}

// Nibble bytes of v: low nibbles (hi = false) or high nibbles.
__device__ __forceinline__ uint32_t nibble_bytes(uint32_t v, bool hi) {
    return (hi ? (v >> 4) : v) & 0x0F0F0F0Fu;
}

// Eight weights from the low (hi = false) or high nibbles of bytes v0, v1.
template <int XT>
__device__ __forceinline__ u32x4 dequant8(uint32_t v0, uint32_t v1, bool hi, float scale512,
                                          float dm) {
    uint32_t o[4];
    dequant4<XT>(nibble_bytes(v0, hi), scale512, dm, o);
    dequant4<XT>(nibble_bytes(v1, hi), scale512, dm, o + 2);
    return u32x4{o[0], o[1], o[2], o[3]};
}

// Scales of one weight row for quant group il: sub-block 2il (low nibbles)
// and 2il+1 (high nibbles), each times 512 for dequant4.
struct GroupScales {
    float lo, hi, dm_lo, dm_hi;
};

__device__ __forceinline__ GroupScales group_scales(u32x4 h, int il) {
    const float d = f16_bits_to_f32(h.x & 0xFFFFu), dmin = f16_bits_to_f32(h.x >> 16);
    uint32_t sc, mn;
    scale_pair(h.y, h.z, h.w, il, &sc, &mn);
    const float d512 = d * 512.0f;
    return GroupScales{d512 * (float)(sc & 0xFFu), d512 * (float)(sc >> 8),
                       dmin * (float)(mn & 0xFFu), dmin * (float)(mn >> 8)};
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
//     of 5 stage buffers, 4 stages ahead (issued right after the stage
//     barrier, when every wave has finished reading the buffer being
//     refilled).  Token t's 16-byte chunk c sits at position c ^ (t & 7) of
//     the token's 128-byte row, so the fragment reads (16 tokens x 16 bytes
//     per k-group) hit distinct banks;
//   * weights: each lane loads the 8 quant bytes of its fragment row four
//     stages ahead (the block header three stages ahead) and dequantises
//     them straight into MFMA operand registers, one stage ahead of use: the
//     dequantisation of stage s+1 (VALU) is written between the MFMAs of
//     stage s, one (fragment, half) per token fragment, so the two pipes
//     overlap.  The prefetch depth is set by latency: with loads two stages
//     ahead the kernel waited on memory at every stage;
//   * per stage: wait until this stage's copies have landed (vmcnt), one
//     workgroup barrier, refill the freed buffer, then 2 x 4 x TF MFMAs.
// The vmcnt bound is static: every stage issues the same loads (beyond the
// last stage they repeat the last stage's addresses into buffers that are
// never read), so the loads issued after stage s's copies are always its
// own quant bytes, three later stages and one header batch: 3*kXLoads + 20.
// Split-K (splits > 1): each workgroup covers a range of super-blocks and
// writes its fp32 tile to a workspace; a second launch (gemm_reduce_kernel)
// adds the splits in split order and writes the output, so results do not
// depend on scheduling.  The kernel boundary between the two launches is the
// only synchronisation (no atomics, fences or spinning).
constexpr int kGemmWaves = 4;
constexpr int kRowsPerWave = 64;
constexpr int kRowsPerWg = kGemmWaves * kRowsPerWave;
constexpr int kRing = 5;

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

// 32x32x16 MFMA (fp32 accumulate) with operands of the x type.  Lane l:
// src0 = row l%32, 8 k values in slot 8*(l/32); src1 = token l%32, same k
// slot; dst element i = row 8*(i/4) + 4*(l/32) + i%4 of token l%32.
template <int XT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if (XT == RXQ4_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Output position of accumulator element i of (row fragment rf, token
// fragment tf) held by lane `lane` of wave `wave` in tile (row_tile,
// tok_tile): rows row..row+3 (j = i/4) of token tok.
struct OutPos {
    int row, tok;
};

template <int TF>
__device__ __forceinline__ OutPos out_pos(int row_tile, int tok_tile, int wave, int lane, int rf,
                                          int tf, int j) {
    return OutPos{row_tile * kRowsPerWg + wave * kRowsPerWave + 32 * rf + 8 * j + 4 * (lane >> 5),
                  tok_tile * 16 * TF + 32 * tf + (lane & 31)};
}

template <int XT, int YT, int TF>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    static_assert(TF == 8, "the stage body is written for 4 token fragments of 32");
    constexpr int TM = 16 * TF;                // 128 tokens
    constexpr int NT = TM / 32;                // 32-token fragments
    constexpr int kXLoads = TM / 32;           // 1 KB direct-to-LDS loads per wave per stage
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
    const int lr = lane & 31;   // row (A) / token (B) within a 32-fragment
    const int h = lane >> 5;    // k slot: bytes 16h .. 16h+15 of each 32-byte quant group
    const int K = p.K;
    const int64_t row_bytes = (int64_t)p.nb * kBlockBytes;
    const int row_base = row_tile * kRowsPerWg + wave * kRowsPerWave;
    const int tok_base = tok_tile * TM;

    const uint8_t *wrow[2];
#pragma unroll
    for (int rf = 0; rf < 2; ++rf)
        wrow[rf] = p.w + (int64_t)min(row_base + 32 * rf + lr, p.M - 1) * row_bytes + sb0 * kBlockBytes;

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
    // The lane's 16 quant bytes of stage s for both row fragments.
    auto load_q = [&](int s, u32x4 *q) {
        const int st = min(s, n_stages - 1);
        const int off = (st >> 2) * kBlockBytes + 16 + 32 * (st & 3) + 16 * h;
#pragma unroll
        for (int rf = 0; rf < 2; ++rf) q[rf] = load16(wrow[rf] + off);
    };
    auto load_h = [&](int sbi, u32x4 *hd) {
        const int sbc = min(sbi, nsb - 1);
#pragma unroll
        for (int rf = 0; rf < 2; ++rf) hd[rf] = load16(wrow[rf] + sbc * kBlockBytes);
    };

    f32x16 acc[2][NT];
#pragma unroll
    for (int rf = 0; rf < 2; ++rf)
#pragma unroll
        for (int tf = 0; tf < NT; ++tf) acc[rf][tf] = f32x16{};

    u32x4 q[4][2];      // quant bytes of stages s .. s+3 (ring by s % 4), per row fragment
    u32x4 hcur[2], hnext[2];
    // Dequantised operands of stages s (a[s&1]) and s+1: [rf][k-step]
    // with k-steps 0: low nibbles of bytes 0-7, 1: low nibbles of bytes
    // 8-15, 2: high nibbles of bytes 0-7, 3: high nibbles of bytes 8-15 (the
    // two sub-blocks of the quant group, 8 k each per lane).
    u32x4 a[2][2][4];

    auto dequant_stage = [&](const u32x4 *qs, const u32x4 *hd, int il, u32x4 (*out)[4]) {
#pragma unroll
        for (int rf = 0; rf < 2; ++rf) {
            const GroupScales g = group_scales(hd[rf], il);
            out[rf][0] = dequant8<XT>(qs[rf].x, qs[rf].y, false, g.lo, g.dm_lo);
            out[rf][1] = dequant8<XT>(qs[rf].z, qs[rf].w, false, g.lo, g.dm_lo);
            out[rf][2] = dequant8<XT>(qs[rf].x, qs[rf].y, true, g.hi, g.dm_hi);
            out[rf][3] = dequant8<XT>(qs[rf].z, qs[rf].w, true, g.hi, g.dm_hi);
        }
    };

    // B fragments of token fragment tf of stage st, k-steps as for A: chunk
    // (16 bytes = 8 k) 2h + step of the low sub-block, 4 + 2h + step of the
    // high one, from ring buffer st % kRing (chunk c of token t sits at
    // position c ^ (t & 7)).
    auto read_b = [&](int st, int tf, u32x4 *b4) {
        const uint8_t *xb = xs[st % kRing];
        const int tt = 32 * tf + lr;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c = (k >> 1) * 4 + 2 * h + (k & 1);
            b4[k] = *reinterpret_cast<const u32x4 *>(xb + tt * 128 + ((c ^ (tt & 7)) << 4));
        }
    };
    u32x4 bf[2][NT][4];  // B fragments of stages s (bf[s&1]) and s+1

    // Prologue: the loads of stages 0..3 in the order the loop issues them
    // (stage k's copies, its quant bytes, the header every 4th stage), the
    // operands of stage 0, then its B fragments once its copies have landed.
    // (sched_barrier pins the issue order the static vmcnt bounds count on.)
    constexpr int kQLoads = 2, kHLoads = 2;
    issue_x(0);
    __builtin_amdgcn_sched_barrier(0);
    load_q(0, q[0]);
    load_h(0, hcur);
    issue_x(1);
    __builtin_amdgcn_sched_barrier(0);
    load_q(1, q[1]);
    issue_x(2);
    __builtin_amdgcn_sched_barrier(0);
    load_q(2, q[2]);
    issue_x(3);
    __builtin_amdgcn_sched_barrier(0);
    load_q(3, q[3]);
    dequant_stage(q[0], hcur, 0, a[0]);
    // loads after stage 0's copies: 4 quant batches, 3 copy batches, 1 header batch
    wait_vmcnt<3 * kXLoads + 4 * kQLoads + kHLoads>();
    lds_barrier();
#pragma unroll
    for (int tf = 0; tf < NT; ++tf) read_b(0, tf, bf[0][tf]);

    for (int sbi = 0; sbi < nsb; ++sbi) {
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            const int s = 4 * sbi + il;
            // Loads run 4 stages ahead: copies of stage s+4 into ring buffer
            // (s+4) % 5, quant bytes of stage s+4 into q[il] (it held stage
            // s, consumed during stage s-1), and at il == 0 the next
            // super-block's headers.  Stage s's B fragments were read during
            // stage s-1; this stage reads stage s+1's, so it waits for the
            // copies of stage s+1: the loads issued after them are its quant
            // bytes, two later stages and, unless il == 0, one header batch.
            // After the barrier every wave has its stage s+1 copies and is
            // past stage s-1, whose buffer is refilled.
            if (il == 0)
                wait_vmcnt<2 * kXLoads + 3 * kQLoads>();
            else
                wait_vmcnt<2 * kXLoads + 3 * kQLoads + kHLoads>();
            lds_barrier();
            // The previous stage's reads of this stage's B fragments are
            // long done; saying so up front keeps the compiler from waiting
            // inside the MFMA stream on LDS reads issued in this stage (the
            // LDS counter completes in order).
            wait_lgkmcnt0();
            issue_x(s + 4);
            __builtin_amdgcn_sched_barrier(0);
            load_q(s + 4, q[il]);
            if (il == 0) load_h(sbi + 1, hnext);

            // 32 MFMAs of stage s (k-step major: 8 independent accumulators
            // between dependent ones), each followed by a quarter of one
            // 8-weight operand of stage s+1 (the next quant group, or group 0
            // of the next super-block; ~5 VALU ops) and, every other MFMA, one
            // read of stage s+1's B fragments.  A wave issues in order, so
            // this one-to-one pattern is what lets the VALU and LDS work run
            // while the matrix core works on the preceding MFMA (32 cycles);
            // sched_barrier keeps the order.
            u32x4 (*acur)[4] = a[il & 1];
            u32x4 (*anext)[4] = a[(il + 1) & 1];
            const u32x4 *hn = il == 3 ? hnext : hcur;
            const u32x4 *qn = q[(il + 1) & 3];
            GroupScales gs[2];  // scales of stage s+1
#pragma unroll
            for (int rf = 0; rf < 2; ++rf) gs[rf] = group_scales(hn[rf], (il + 1) & 3);
            u32x4 (*bc)[4] = bf[il & 1];
            u32x4 (*bn)[4] = bf[(il + 1) & 1];
            const uint8_t *xnb = xs[(s + 1) % kRing];
            uint32_t m0 = 0, m1 = 0, o0 = 0, o1 = 0, o2 = 0, o3 = 0;
#pragma unroll
            for (int idx = 0; idx < 32; ++idx) {
                const int k = idx >> 3, tf = (idx >> 1) & 3, rf = idx & 1;
                acc[rf][tf] = mfma32<XT>(acur[rf][k], bc[tf][k], acc[rf][tf]);
                __builtin_amdgcn_sched_barrier(0);
                // operand op = (rf2, k2) of stage s+1, piece idx % 4
                const int op = idx >> 2, rf2 = op >> 2, k2 = op & 3, piece = idx & 3;
                const bool hi = k2 >= 2;
                const float sc = hi ? gs[rf2].hi : gs[rf2].lo;
                const float dm = hi ? gs[rf2].dm_hi : gs[rf2].dm_lo;
                if (piece == 0) {
                    m0 = nibble_bytes((k2 & 1) ? qn[rf2].z : qn[rf2].x, hi);
                    const f32x2 f = nibbles_f32<false>(m0);
                    o0 = pack2<XT>(sc * f[0] - dm, sc * f[1] - dm);
                } else if (piece == 1) {
                    const f32x2 f = nibbles_f32<true>(m0);
                    o1 = pack2<XT>(sc * f[0] - dm, sc * f[1] - dm);
                } else if (piece == 2) {
                    m1 = nibble_bytes((k2 & 1) ? qn[rf2].w : qn[rf2].y, hi);
                    const f32x2 f = nibbles_f32<false>(m1);
                    o2 = pack2<XT>(sc * f[0] - dm, sc * f[1] - dm);
                } else {
                    const f32x2 f = nibbles_f32<true>(m1);
                    o3 = pack2<XT>(sc * f[0] - dm, sc * f[1] - dm);
                    anext[rf2][k2] = u32x4{o0, o1, o2, o3};
                }
                if ((idx & 1) == 0) {
                    // B fragment r = idx / 2 of stage s+1: token fragment r / 4, k-step r % 4
                    const int r = idx >> 1, tf2 = r >> 2, kk = r & 3;
                    const int tt = 32 * tf2 + lr;
                    const int c = (kk >> 1) * 4 + 2 * h + (kk & 1);
                    bn[tf2][kk] = *reinterpret_cast<const u32x4 *>(xnb + tt * 128 + ((c ^ (tt & 7)) << 4));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (il == 3) {
#pragma unroll
                for (int rf = 0; rf < 2; ++rf) hcur[rf] = hnext[rf];
            }
        }
    }
    wait_vmcnt<0>();  // trailing clamped copies must land before the workgroup exits

    if (p.splits > 1) {
        // partial tile: per thread 2 x NT x 4 float4 in (rf, tf, j) order
        f32x4 *part = reinterpret_cast<f32x4 *>(p.ws) +
                      ((int64_t)(tile * p.splits + split) * (8 * NT)) * 256 + tid;
#pragma unroll
        for (int rf = 0; rf < 2; ++rf)
#pragma unroll
            for (int tf = 0; tf < NT; ++tf)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    part[((rf * NT + tf) * 4 + j) * 256] =
                        f32x4{acc[rf][tf][4 * j], acc[rf][tf][4 * j + 1], acc[rf][tf][4 * j + 2],
                              acc[rf][tf][4 * j + 3]};
        return;
    }
    const bool vec_ok = (p.M & 3) == 0;
#pragma unroll
    for (int rf = 0; rf < 2; ++rf)
#pragma unroll
        for (int tf = 0; tf < NT; ++tf)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const OutPos o = out_pos<TF>(row_tile, tok_tile, wave, lane, rf, tf, j);
                if (o.tok >= p.N || o.row >= p.M) continue;
                const int valid = min(4, p.M - o.row);
                store4<YT>(p.y, (int64_t)o.tok * p.M + o.row,
                           f32x4{acc[rf][tf][4 * j], acc[rf][tf][4 * j + 1], acc[rf][tf][4 * j + 2],
                                 acc[rf][tf][4 * j + 3]},
                           vec_ok && valid == 4, valid);
            }
}

// Split-K reduction: block (tile, e) with e = (rf*NT + tf)*4 + j sums the
// splits of one float4 of every thread of the tile in split order; thread
// tid holds the positions of thread tid of the GEMM workgroups.
template <int YT, int TF>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
    constexpr int NT = TF / 2;
    constexpr int E = 8 * NT;  // float4 per thread
    const int tid = threadIdx.x;
    const int tile = blockIdx.x / E;
    const int e = blockIdx.x % E;
    const int rf = e / (4 * NT), tf = (e / 4) % NT, j = e % 4;
    const int row_tile = tile / p.tok_tiles, tok_tile = tile % p.tok_tiles;
    const OutPos o = out_pos<TF>(row_tile, tok_tile, tid >> 6, tid & 63, rf, tf, j);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.ws) +
                       ((int64_t)tile * p.splits * E + e) * 256 + tid;
    f32x4 sum = src[0];
    for (int sp = 1; sp < p.splits; ++sp) {
        const f32x4 v = src[(int64_t)sp * E * 256];
        sum = f32x4{sum[0] + v[0], sum[1] + v[1], sum[2] + v[2], sum[3] + v[3]};
    }
    if (o.tok >= p.N || o.row >= p.M) return;
    const int valid = min(4, p.M - o.row);
    store4<YT>(p.y, (int64_t)o.tok * p.M + o.row, sum, (p.M & 3) == 0 && valid == 4, valid);
}

// ---------------------------------------------------------------------------
// Small batch (2..16 tokens): a workgroup of KW waves owns 16*RT weight rows
// x 16 tokens.  The K super-blocks are dealt to the waves round-robin (wave
// w: w, w+KW, ...); each wave computes RT 16x16 fragments with
// v_mfma_f32_16x16x32 (A = 16 weight rows, B = the 16 tokens), so one x
// fragment serves RT row tiles.  Each wave keeps two super-blocks of weights
// and x in flight (loads unconditional, clamped to the last super-block, so
// the compiler's vmcnt waits stay exact).  x is read through a buffer
// resource bounded at N*K elements: the lanes of tokens >= N read past it and
// get zeros without touching memory.  Partial sums are added in wave order
// through LDS.
template <int XT, int YT, int RT, int KW>
__global__ __launch_bounds__(KW * 64) void gemv_tokens_kernel(
    void *__restrict__ y, const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, int M,
    int N, int K) {
    __shared__ f32x4 part[KW][RT][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int nb = K >> 8;
    const int row0 = blockIdx.x * 16 * RT;
    const int64_t row_bytes = (int64_t)nb * kBlockBytes;
    const uint8_t *wr[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) wr[t] = w + min(row0 + 16 * t + li, M - 1) * row_bytes;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, N * K * 2);
    const int xoff = li * K * 2 + 16 * g;  // bytes; >= N*K*2 for tokens >= N
    const int n_w = wave < nb ? (nb - 1 - wave) / KW + 1 : 0;  // super-blocks of this wave

    struct Sb {
        u32x4 hdr[RT];
        u32x2 q[RT][4];
        u32x4 b[8];
    };
    auto load = [&](int i, Sb &o) {
        const int sb = min(wave + i * KW, nb - 1);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint8_t *blk = wr[t] + sb * kBlockBytes;
            o.hdr[t] = load16(blk);
#pragma unroll
            for (int il = 0; il < 4; ++il)
                o.q[t][il] = *reinterpret_cast<const u32x2 *>(blk + 16 + 32 * il + 8 * g);
        }
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            const int off = xoff + 2 * (sb * 256 + 64 * il);
            o.b[2 * il] = buffer_load16(xr, off);
            o.b[2 * il + 1] = buffer_load16(xr, off + 64);
        }
    };
    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Sb &o) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int il = 0; il < 4; ++il) {
                const GroupScales gsc = group_scales(o.hdr[t], il);
                const u32x4 a_lo =
                    dequant8<XT>(o.q[t][il].x, o.q[t][il].y, false, gsc.lo, gsc.dm_lo);
                const u32x4 a_hi =
                    dequant8<XT>(o.q[t][il].x, o.q[t][il].y, true, gsc.hi, gsc.dm_hi);
                acc[t] = mfma<XT>(a_lo, o.b[2 * il], acc[t]);
                acc[t] = mfma<XT>(a_hi, o.b[2 * il + 1], acc[t]);
            }
        }
    };
    Sb A, B;
    load(0, A);
    load(1, B);
    int i = 0;
    for (; i + 2 < n_w; i += 2) {
        compute(A);
        load(i + 2, A);
        compute(B);
        load(i + 3, B);
    }
    if (i < n_w) compute(A);
    if (i + 1 < n_w) compute(B);

#pragma unroll
    for (int t = 0; t < RT; ++t) part[wave][t][lane] = acc[t];
    __syncthreads();
    for (int t = wave; t < RT; t += KW) {
        f32x4 sum = part[0][t][lane];
#pragma unroll
        for (int j = 1; j < KW; ++j) {
            const f32x4 o = part[j][t][lane];
            sum = f32x4{sum[0] + o[0], sum[1] + o[1], sum[2] + o[2], sum[3] + o[3]};
        }
        if (li < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + 16 * t + 4 * g + r;
                if (row < M) store_out<YT>(y, (int64_t)li * M + row, sum[r]);
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

hipError_t device_workspace(size_t bytes, float **ws) {
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
        hipError_t e = device_workspace(part, &p.ws);
        if (e != hipSuccess) return e;
    }
    p.total_units = tiles * splits;
    p.units_per_xcd = (p.total_units + 7) / 8;
    gemm_kernel<XT, YT, TF><<<8 * p.units_per_xcd, 256, 0, st>>>(p);
    if (splits > 1) gemm_reduce_kernel<YT, TF><<<tiles * 4 * TF, 256, 0, st>>>(p);  // 4*TF = 8*NT float4 per thread
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

template <int XT, int YT>
static void launch_tokens_t(void *y, const uint8_t *w, const uint16_t *x, int M, int n_tok,
                            int K, hipStream_t st) {
    // Four waves split K.  Two row tiles per wave halve the x traffic per
    // weight byte and pay off once there are enough of them to give about
    // four waves per CU (1024 waves); a measured sweep of 1/2/4 row tiles and
    // 1/2/4/8 waves on gate+up [22016 x 2048], down [2048 x 11008] and QKV
    // [2560 x 2048] at 2..16 tokens put these two shapes first.
    constexpr int kWaves = 4;
    const int t2 = (M + 31) / 32;
    if (t2 * kWaves >= 1024)
        gemv_tokens_kernel<XT, YT, 2, kWaves><<<t2, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K);
    else
        gemv_tokens_kernel<XT, YT, 1, kWaves>
            <<<(M + 15) / 16, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K);
}

hipError_t launch_gemv_tokens(void *y, int y_dtype, const uint8_t *w, const void *x,
                              int x_dtype, int M, int n_tok, int K, hipStream_t st) {
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            launch_tokens_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16>(y, w, xx, M, n_tok, K, st);
        else
            launch_tokens_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32>(y, w, xx, M, n_tok, K, st);
    } else {
        if (y_dtype == RXQ4_DTYPE_F16)
            launch_tokens_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F16>(y, w, xx, M, n_tok, K, st);
        else
            launch_tokens_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F32>(y, w, xx, M, n_tok, K, st);
    }
    return hipGetLastError();
}

}  // namespace rxq4
