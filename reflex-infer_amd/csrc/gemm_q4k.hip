// gemm_q4k.hip -- Q4_K prefill GEMM and small-batch decode on gfx950 MFMA.
//
// Replaces the reference's batched path (q4_gemm.cu:1297-1356 scalar kernel,
// 1482-1636 mma.sync MMQ kernel, 1638-1740 host chunking).  The reference
// re-streams W once per 20-token chunk; here every launch reads W once per
// token tile of 128 tokens.
//
// Math: y[tok, row] = sum_k x[tok, k] * w[row, k] with w = d*sc*q - dmin*m
// rounded once to fp32 and then (RNE) to the operand type of x (fp16 or
// bf16), products accumulated in fp32 by MFMA: v_mfma_f32_32x32x16 in the
// GEMM (weight rows as src0, tokens as src1), v_mfma_f32_16x16x32 in the
// small-batch kernel.  A lane's 8 consecutive k of one sub-block are 8 quant
// bytes' low nibbles; the same 8 bytes' high nibbles are the same k of the
// next sub-block, so one load feeds two MFMA k-steps.  Flops per launch:
// 2*N*M*K.
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "launch.h"
#include "gemm_util.h"
#include "mfma_util.h"
#include "q4k_device.h"
#include "rxq4.h"

namespace rxq4 {

// ---------------------------------------------------------------------------
// Tiled GEMM.
//
// Workgroup = 8 waves, tile = 256 weight rows x 128 tokens; wave w owns 32
// rows (one 32-row MFMA fragment) and all 128 tokens (four 32-token
// fragments).  Two waves share each SIMD, so one wave's dequantisation
// (VALU) issues while the other's MFMAs run: measured on gfx950, a single
// wave hides only about half of its own VALU work behind its MFMAs, while a
// second wave's VALU work hides almost entirely.  At ~160 VGPRs a wave fits
// the 256-register budget of two waves per SIMD, and every weight is still
// dequantised once per workgroup.  K is walked in stages of 64 (one 32-byte
// quant group il of a super-block = two sub-blocks = four MFMA k-steps):
//   * activations: each stage's 128 x 64 tile is copied global -> LDS by the
//     gfx950 direct-to-LDS loads (buffer_load_dwordx4 ... lds) into a ring
//     of 4 stage buffers, 3 stages ahead (issued right after the stage
//     barrier, when every wave has finished reading the buffer being
//     refilled).  With 4 buffers and the stage loop unrolled by 4, every
//     buffer address is a compile-time offset (a ring of 5 cost a divide by
//     5 and an address add per LDS access).  Token t's 16-byte chunk c sits
//     at position c ^ ((t >> 1) & 7) of the token's 128-byte row: a 16-lane
//     group of a
//     fragment read (16 consecutive tokens, one chunk each) then covers all
//     64 LDS banks once (with c ^ (t & 7), tokens t and t + 8 collided;
//     measured 2.9M bank-conflict cycles against 0.8M LDS-active cycles);
//   * B fragments (16 per wave per stage, 1 KB each) stream from LDS through
//     a ring of 8 registers, read kLook MFMAs ahead (the last ones of a
//     stage read the next stage's buffer).  That is 128 KB of LDS reads per
//     stage and CU, a small part of the gfx950 LDS bandwidth;
//   * weights: each lane loads the 16 quant bytes of its row three stages
//     ahead (the next block header at the start of a super-block) and
//     dequantises them straight into MFMA operand registers, one stage
//     ahead of use: the
//     dequantisation of stage s+1 (VALU) is written between the MFMAs of
//     stage s, a quarter operand per MFMA;
//   * per stage: wait until the next stage's copies have landed (vmcnt),
//     one workgroup barrier, refill the freed buffer, then 16 MFMAs.
// The vmcnt bound is static: every stage issues the same loads (beyond the
// last stage they repeat the last stage's addresses into buffers that are
// never read), so the count of loads issued after a given stage's copies
// is fixed.
// Output: 16-bit tiles are staged through LDS as [token][row], so 32 lanes
// write one token's 512 contiguous bytes (the MFMA layout, 4 rows of one
// token per lane, would scatter 8-byte pieces over 32 tokens; measured 5.6 us
// of 38.6 us for the m = 512 [11008 x 2048] GEMM written that way).
// Split-K (splits > 1): each workgroup covers a range of super-blocks and
// writes its fp32 tile to a workspace; a second launch (gemm_reduce_kernel)
// adds the splits in split order and writes the output, so results do not
// depend on scheduling.  The kernel boundary between the two launches is the
// only synchronisation (no atomics, fences or spinning).
constexpr int kRowsPerWg = 256;  // rows of the eight-wave workgroup
constexpr int kRing = 4;  // LDS stage buffers; stage s uses buffer s % 4

struct GemmParams {
    void *y;
    const uint8_t *w;
    const uint16_t *x;
    float *ws;      // split-K partial tiles [tile][split][16][512 threads] float4
    int M, N, K, nb;
    int row_tiles, tok_tiles, splits, sb_per_split;
    int total_units, units_per_xcd;
    int tok_major;    // unit order (see gemm_kernel)
    int big_per_xcd;  // gemm_mixed_kernel: whole areas per XCD
};

constexpr int kW8Rows = 32;                       // weight rows per wave
// staged output of an NW-wave workgroup (32 * NW rows): bytes per token
template <int NW>
constexpr int out_pitch() { return 64 * NW + 16; }

// ---------------------------------------------------------------------------
// Weight formats of the GEMM.  A stage is 64 weights of every row; lane
// (row lr, half h) dequantises 32 of them into four 8-weight MFMA operands
// (k-steps kk = 0..3), a quarter operand ("piece" p = 0..3, weights 2p and
// 2p+1) per MFMA of the previous stage.  chunk(kk, h) is the 8-element x
// chunk (0..7) of the stage that k-step kk of half h multiplies; the stage's
// x elements are k0 + stage_elem(st) + chunk_elem(c) + 0..7.  Every weight is
// rounded once to fp32 (one fma of the reference's factors) and then to the
// x type.
template <int T>
struct GemmFmt;

// Q4_K (144 B): stage g of a super-block = quant group g (sub-blocks 2g and
// 2g+1); half h holds qs bytes 16h..16h+15 of the group, k-step kk the low
// (kk < 2) or high nibbles of bytes 8*(kk & 1)..+7.  Nibbles convert through
// the FP8 trick (dequant4): w = (512*d*sc) * (q * 2^-9) - dmin*m.
template <>
struct GemmFmt<12> {
    static constexpr int kBytes = 144, kQLoads = 1, kHLoads = 1;
    struct Stage {
        u32x4 q;
    };
    struct Sb {
        u32x4 h;
    };
    struct Loader {
        const uint8_t *row;  // the lane's row at the first super-block
        int nsb, h;
        // super-block indices clamp to the last one: loads past the end stay in the row
        __device__ int blk(int sb) const { return min(sb, nsb - 1); }
        __device__ Stage stage(int sb, int g) const {
            return {load16(row + blk(sb) * kBytes + 16 + 32 * g + 16 * h)};
        }
        __device__ Sb header(int sb) const { return {load16(row + blk(sb) * kBytes)}; }
    };
    using Scales = GroupScales;
    __device__ static Scales scales(const Sb &b, int g) { return group_scales(b.h, g); }
    __device__ static void prepare(Stage &, const Sb &) {}
    __device__ static int chunk(int kk, int h) { return (kk >> 1) * 4 + 2 * h + (kk & 1); }
    __device__ static int chunk_elem(int c) { return 8 * c; }
    __device__ static int stage_elem(int st) { return 64 * st; }
    struct Piece {
        uint32_t m, o[3];
    };
    template <int XT>
    __device__ static void piece(int kk, int p, int g, const Stage &s, const Sb &, const Scales &gs,
                                 Piece &st, u32x4 &out) {
        const bool hi = kk >= 2;
        const float sc = hi ? gs.hi : gs.lo;
        const float dm = hi ? gs.dm_hi : gs.dm_lo;
        if ((p & 1) == 0) st.m = nibble_bytes(p == 0 ? ((kk & 1) ? s.q.z : s.q.x)
                                                     : ((kk & 1) ? s.q.w : s.q.y), hi);
        const f32x2 f = (p & 1) ? nibbles_f32<true>(st.m) : nibbles_f32<false>(st.m);
        const uint32_t o = pack2<XT>(sc * f[0] - dm, sc * f[1] - dm);
        if (p < 3) st.o[p] = o;
        else out = u32x4{st.o[0], st.o[1], st.o[2], o};
    }
};

// Byte b (0..3) of v as fp32 (v_cvt_f32_ubyte<b>).
__device__ __forceinline__ float byte_f32(uint32_t v, int b) {
    return (float)((v >> (8 * b)) & 0xFFu);
}

// Q5_K (176 B): the Q4_K layout of qs (@48) and scales, plus the fifth bit
// 2g + hi of qh[l] (@16); half h keeps qh bytes 16h..16h+15 with the
// super-block header.  q = nibble | bit << 4 (0..31) converts with
// v_cvt_f32_ubyte: w = (d*sc) * q - dmin*m.
template <>
struct GemmFmt<13> {
    static constexpr int kBytes = 176, kQLoads = 1, kHLoads = 2;
    struct Stage {
        u32x4 q;
    };
    struct Sb {
        u32x4 h, qh;
    };
    struct Loader {
        const uint8_t *row;
        int nsb, h;
        __device__ int blk(int sb) const { return min(sb, nsb - 1); }
        __device__ Stage stage(int sb, int g) const {
            return {load16(row + blk(sb) * kBytes + 48 + 32 * g + 16 * h)};
        }
        __device__ Sb header(int sb) const {
            const uint8_t *b = row + blk(sb) * kBytes;
            return {load16(b), load16(b + 16 + 16 * h)};
        }
    };
    struct Scales {
        float lo, hi, dm_lo, dm_hi;
    };
    __device__ static Scales scales(const Sb &b, int g) {
        const float d = f16_bits_to_f32(b.h.x & 0xFFFFu), dmin = f16_bits_to_f32(b.h.x >> 16);
        uint32_t sc, mn;
        scale_pair(b.h.y, b.h.z, b.h.w, g, &sc, &mn);
        return Scales{d * (float)(sc & 0xFFu), d * (float)(sc >> 8), dmin * (float)(mn & 0xFFu),
                      dmin * (float)(mn >> 8)};
    }
    __device__ static void prepare(Stage &, const Sb &) {}
    __device__ static int chunk(int kk, int h) { return GemmFmt<12>::chunk(kk, h); }
    __device__ static int chunk_elem(int c) { return 8 * c; }
    __device__ static int stage_elem(int st) { return 64 * st; }
    struct Piece {
        uint32_t m, o[3];
    };
    template <int XT>
    __device__ static void piece(int kk, int p, int g, const Stage &s, const Sb &b,
                                 const Scales &gs, Piece &st, u32x4 &out) {
        const int hi = kk >> 1, dw = 2 * (kk & 1) + (p >> 1);
        const float sc = hi ? gs.hi : gs.lo;
        const float dm = hi ? gs.dm_hi : gs.dm_lo;
        if ((p & 1) == 0) {
            const uint32_t lo = (s.q[dw] >> (4 * hi)) & 0x0F0F0F0Fu;
            st.m = lo | (((b.qh[dw] >> (2 * g + hi)) & 0x01010101u) << 4);
        }
        const int e = 2 * (p & 1);
        const uint32_t o = pack2<XT>(sc * byte_f32(st.m, e) - dm, sc * byte_f32(st.m, e + 1) - dm);
        if (p < 3) st.o[p] = o;
        else out = u32x4{st.o[0], st.o[1], st.o[2], o};
    }
};

// Q6_K (210 B, only 2-byte aligned): stage g of a super-block = half
// n = g / 2 (128 weights), run lh = g % 2; its 64 weights are
// 128n + 32m + 16lh + (0..15) for m = 0..3, k-step kk = m, and half h takes
// l = 16lh + 8h + (0..7): ql bytes 64n + 16lh + 8h (m = 0 low nibbles, m = 2
// high) and 64n + 32 + 16lh + 8h (m = 1, 3), qh bytes 128 + 32n + 16lh + 8h
// (bits 2m, 2m+1), scale sc[8n + 2m + lh].  The fields are read with
// dword-aligned buffer loads (bounded to the wave's rows: rows past the
// matrix read zeros) and realigned by the lane's byte offset r (0 or 2),
// fixed per super-block.  q (0..63) converts with v_cvt_f32_ubyte:
// w = (d*sc) * q - 32*(d*sc) = d*sc*(q - 32) exactly as the reference.
template <>
struct GemmFmt<14> {
    static constexpr int kBytes = 210, kQLoads = 3, kHLoads = 3;
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    struct Stage {
        u32x3 a, b, qh;    // raw dwords of ql (m = 0, 2), ql (m = 1, 3), qh
        u32x2 ra, rb, rh;  // realigned 8 bytes of each (prepare)
    };
    struct Sb {
        u32x4 sc;      // raw dwords of the 16 scale bytes (+ 4 below)
        uint32_t sce;  // dword after sc
        uint32_t d;    // fp16 d in the low half
        int r;         // byte offset of the lane's block fields in the dwords
    };
    struct Loader {
        __amdgpu_buffer_rsrc_t rs;  // the wave's rows from the first super-block, dword-aligned
        int base;                   // byte offset of the lane's row in rs
        int nsb, h;
        __device__ int block(int sb) const { return base + min(sb, nsb - 1) * kBytes; }
        __device__ Stage stage(int sb, int g) const {
            const int o = block(sb), n = g >> 1, lh = g & 1, f = 16 * lh + 8 * h;
            const int oa = (o + 64 * n + f) & ~3, ob = (o + 64 * n + 32 + f) & ~3,
                      oh = (o + 128 + 32 * n + f) & ~3;
            Stage s;
            s.a = __builtin_amdgcn_raw_buffer_load_b96(rs, oa, 0, 0);
            s.b = __builtin_amdgcn_raw_buffer_load_b96(rs, ob, 0, 0);
            s.qh = __builtin_amdgcn_raw_buffer_load_b96(rs, oh, 0, 0);
            return s;
        }
        __device__ Sb header(int sb) const {
            const int o = block(sb);
            Sb b;
            b.sc = buffer_load16(rs, (o + 192) & ~3);
            b.sce = buffer_load4(rs, ((o + 192) & ~3) + 16);
            // 2-byte load: a dword could reach past the last block
            b.d = __builtin_amdgcn_raw_buffer_load_b16(rs, o + 208, 0, 0);
            b.r = o & 3;
            return b;
        }
    };
    struct Scales {
        float ds[4], off[4];
    };
    __device__ static Scales scales(const Sb &b, int g) {
        const int n = g >> 1, lh = g & 1;
        const float d = f16_bits_to_f32(b.d & 0xFFFFu);
        const uint32_t w[5] = {b.sc.x, b.sc.y, b.sc.z, b.sc.w, b.sce};
        // scale bytes 8n .. 8n+7: realigned dwords 2n, 2n+1
        const uint32_t S[2] = {align_bytes(w[2 * n + 1], w[2 * n], b.r),
                               align_bytes(w[2 * n + 2], w[2 * n + 1], b.r)};
        Scales s;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int sh = 8 * (2 * (m & 1) + lh);  // byte 2m + lh of the 8
            s.ds[m] = d * (float)((int)(S[m >> 1] << (24 - sh)) >> 24);
            s.off[m] = -32.0f * s.ds[m];
        }
        return s;
    }
    __device__ static u32x2 realign8(u32x3 v, int r) {
        return u32x2{align_bytes(v.y, v.x, r), align_bytes(v.z, v.y, r)};
    }
    __device__ static void prepare(Stage &s, const Sb &b) {
        s.ra = realign8(s.a, b.r);
        s.rb = realign8(s.b, b.r);
        s.rh = realign8(s.qh, b.r);
    }
    __device__ static int chunk(int kk, int h) { return 2 * kk + h; }
    __device__ static int chunk_elem(int c) { return 32 * (c >> 1) + 8 * (c & 1); }
    __device__ static int stage_elem(int st) {
        return 256 * (st >> 2) + 128 * ((st >> 1) & 1) + 16 * (st & 1);
    }
    struct Piece {
        uint32_t m, o[3];
    };
    template <int XT>
    __device__ static void piece(int kk, int p, int, const Stage &s, const Sb &, const Scales &gs,
                                 Piece &st, u32x4 &out) {
        const int dw = p >> 1;
        if ((p & 1) == 0) {
            const uint32_t ql = (kk & 1) ? s.rb[dw] : s.ra[dw];
            const uint32_t lo = (ql >> (4 * (kk >> 1))) & 0x0F0F0F0Fu;
            st.m = lo | (((s.rh[dw] >> (2 * kk)) & 0x03030303u) << 4);
        }
        const int e = 2 * (p & 1);
        const float ds = gs.ds[kk], off = gs.off[kk];
        const uint32_t o = pack2<XT>(ds * byte_f32(st.m, e) + off, ds * byte_f32(st.m, e + 1) + off);
        if (p < 3) st.o[p] = o;
        else out = u32x4{st.o[0], st.o[1], st.o[2], o};
    }
};

// LDS of one workgroup: the x ring, reused for the staged output tile.
template <int TM, int NW = 8>
constexpr int gemm_lds_bytes() {
    return TM * out_pitch<NW>() > kRing * TM * 128 ? TM * out_pitch<NW>() : kRing * TM * 128;
}

// One output tile of an NW-wave workgroup (NW = 8: two waves per SIMD; 4:
// one): rows [32 * NW * row_tile, +32 * NW) x tokens [TM * tok_tile, +TM)
// over super-blocks [split * sb_per_split, +sb_per_split).
template <int T, int XT, int YT, int TM, int NW = 8>
__device__ __forceinline__ void gemm_tile(const GemmParams &p, uint8_t *lds, int split,
                                          int row_tile, int tok_tile) {
    using F = GemmFmt<T>;
    // TM tokens per workgroup tile (128 or 256)
    constexpr int NT = TM / 32;      // 32-token fragments per wave
    constexpr int MPS = 4 * NT;      // MFMAs per stage and wave
    constexpr int RPW = 32 * NW;     // weight rows per workgroup
    constexpr int THREADS = 64 * NW;
    constexpr int kOutPitch = out_pitch<NW>();
    constexpr int kXLoads = TM / (8 * NW); // 1 KB direct-to-LDS copies per wave per stage
    constexpr int kQLoads = F::kQLoads, kHLoads = F::kHLoads;
    constexpr int kLook = 6;         // B fragments are read kLook MFMAs before use
    constexpr int kBufBytes = TM * 128;                        // one stage of x
    const int tile = row_tile * p.tok_tiles + tok_tile;
    const int sb0 = split * p.sb_per_split;
    const int nsb = min(p.nb, sb0 + p.sb_per_split) - sb0;
    const int n_stages = 4 * nsb;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31;   // row (A) / token (B) within a 32-fragment
    const int h = lane >> 5;    // half of the stage's weights of the row
    const int K = p.K;
    const int64_t row_bytes = (int64_t)p.nb * F::kBytes;
    const int row_base = row_tile * RPW + wave * kW8Rows;
    const int tok_base = tok_tile * TM;

    typename F::Loader ld;
    if constexpr (T == 14) {
        // buffer resource over the wave's rows (none past the matrix) from
        // super-block sb0, based at the dword at or below its first byte
        const uint8_t *first = p.w + (int64_t)row_base * row_bytes + sb0 * F::kBytes;
        const int ex = (int)(reinterpret_cast<uintptr_t>(first) & 3);
        const int rows = max(0, min(kW8Rows, p.M - row_base));
        const int64_t span = rows ? (rows - 1) * row_bytes + (p.nb - sb0) * F::kBytes : 0;
        ld.rs = make_rsrc(first - ex, (int)(span + ex));
        ld.base = (int)(lr * row_bytes) + ex;
    } else {
        ld.row = p.w + (int64_t)min(row_base + lr, p.M - 1) * row_bytes + sb0 * F::kBytes;
    }
    ld.nsb = nsb;
    ld.h = h;

    // Direct-to-LDS copies of the x tile: TM / 8 chunks of 1 KB (8 tokens)
    // per stage, chunks wave + NW * i (tokens 8*chunk + lane/8); chunk c of
    // token t at c ^ ((t >> 1) & 7), and (t >> 1) & 7 = 4*(wave & 1) + lane/16
    // (NW is even, so chunk parity is wave parity).
    const int ctok = lane >> 3;
    const int cpos = (lane & 7) ^ ((4 * (wave & 1) + (ctok >> 1)) & 7);
    const __amdgpu_buffer_rsrc_t xrsrc =
        make_rsrc(p.x + (int64_t)tok_base * K, min(TM, p.N - tok_base) * K * 2);
    int xoff[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
        const int tok = min(8 * (wave + NW * i) + ctok, p.N - 1 - tok_base);
        xoff[i] = (tok * K + F::chunk_elem(cpos)) * 2;
    }
    // Stage s's copies (clamped to the last stage) into ring buffer s % 4;
    // the stage's k offset is the wave-uniform soffset of the load.
    auto issue_x = [&](int buf, int s) {
        const int k0b = (sb0 * 256 + F::stage_elem(min(s, n_stages - 1))) * 2;
#pragma unroll
        for (int i = 0; i < kXLoads; ++i)
            buffer_to_lds16(xrsrc, lds + buf * kBufBytes + (wave + NW * i) * 1024, xoff[i], k0b);
    };

    // Per-lane byte offset of B fragment (k-step k, token fragment 0) in a
    // ring buffer: token lr, chunk c = chunk(k, h) at c ^ ((lr >> 1) & 7);
    // token fragment tf adds 4096*tf.
    int boff[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) boff[k] = lr * 128 + ((F::chunk(k, h) ^ ((lr >> 1) & 7)) << 4);
    // MFMA n of a stage (n < MPS): k-step n / NT, token fragment n % NT.
    auto read_b = [&](int buf, int n) {
        return *reinterpret_cast<const u32x4 *>(lds + buf * kBufBytes + 4096 * (n % NT) +
                                                boff[n / NT]);
    };

    f32x16 acc[NT];
#pragma unroll
    for (int tf = 0; tf < NT; ++tf) acc[tf] = f32x16{};

    typename F::Stage q[4];   // weights of stages s .. s+3 (ring by s % 4)
    typename F::Sb hcur, hnext;  // per-super-block data, current and next
    u32x4 a[2][4];            // A operands of stages s (a[s&1]) and s+1, per k-step
    u32x4 bq[8];              // B fragment ring, slot = MFMA sequence number % 8

    // Prologue: loads of stages 0..2 in loop order, stage 0's operands, then
    // its first kLook B fragments once its copies have landed.
    issue_x(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    q[0] = ld.stage(0, 0);
    hcur = ld.header(0);
    issue_x(1, 1);
    __builtin_amdgcn_sched_barrier(0);
    q[1] = ld.stage(0, 1);
    issue_x(2, 2);
    __builtin_amdgcn_sched_barrier(0);
    q[2] = ld.stage(0, 2);
    {
        F::prepare(q[0], hcur);
        const typename F::Scales g = F::scales(hcur, 0);
        typename F::Piece pc;
#pragma unroll
        for (int n = 0; n < 16; ++n)
            F::template piece<XT>(n >> 2, n & 3, 0, q[0], hcur, g, pc, a[0][n >> 2]);
    }
    wait_vmcnt<2 * kXLoads + 3 * kQLoads + kHLoads>();
    lds_barrier();
#pragma unroll
    for (int n = 0; n < kLook; ++n) bq[n] = read_b(0, n);

    for (int sbi = 0; sbi < nsb; ++sbi) {
#pragma unroll
        for (int il = 0; il < 4; ++il) {
            const int s = 4 * sbi + il;
            // Copies and weights run 3 stages ahead (ring buffer and q slot
            // (s+3) % 4 held stage s-1, finished during stage s-1), the next
            // super-block's data is issued at il == 0.  Wait for stage s+1's
            // copies (read from MFMA MPS - kLook of this stage on): the loads
            // issued after them are its weights, stage s+2's copies and
            // weights and, at il == 1 and 2, the super-block data.  After the
            // barrier every wave is past stage s-1, whose buffer is refilled.
            if (il == 1 || il == 2)
                wait_vmcnt<kXLoads + 2 * kQLoads + kHLoads>();
            else
                wait_vmcnt<kXLoads + 2 * kQLoads>();
            lds_barrier();
            issue_x((il + 3) & 3, s + 3);
            __builtin_amdgcn_sched_barrier(0);
            q[(il + 3) & 3] = ld.stage(sbi + ((il + 3) >> 2), (il + 3) & 3);
            if (il == 0) hnext = ld.header(sbi + 1);

            // MPS MFMAs of stage s; one of every MPS / 16 is followed by a
            // quarter of one 8-weight A operand of stage s+1, and each by one
            // B fragment read kLook MFMAs ahead (into stage s+1 for the last
            // kLook).  The compiler's own interleave of this stream measured
            // 1-3% faster than one pinned with sched_barrier.
            const u32x4 *acur = a[il & 1];
            u32x4 *anext = a[(il + 1) & 1];
            const typename F::Sb &hn = il == 3 ? hnext : hcur;
            typename F::Stage &qn = q[(il + 1) & 3];
            F::prepare(qn, hn);
            const typename F::Scales gs = F::scales(hn, (il + 1) & 3);
            typename F::Piece pc;
#pragma unroll
            for (int n = 0; n < MPS; ++n) {
                const int k = n / NT, tf = n % NT;
                acc[tf] = mfma32<XT>(acur[k], bq[n & 7], acc[tf]);
                if (n % (MPS / 16) == 0) {
                    const int pi = n / (MPS / 16);  // piece pi & 3 of k-step pi >> 2
                    F::template piece<XT>(pi >> 2, pi & 3, (il + 1) & 3, qn, hn, gs, pc,
                                          anext[pi >> 2]);
                }
                const int nr = n + kLook;
                bq[nr & 7] = nr < MPS ? read_b(il, nr) : read_b((il + 1) & 3, nr - MPS);
            }
            if (il == 3) hcur = hnext;
        }
    }
    // The trailing clamped copies and look-ahead reads must finish before
    // the ring is reused or the workgroup exits.
    wait_vmcnt<0>();
    wait_lgkmcnt0();

    if (p.splits > 1) {
        // partial tile: per thread NT x 4 float4 in (tf, j) order
        f32x4 *part = reinterpret_cast<f32x4 *>(p.ws) +
                      ((int64_t)(tile * p.splits + split) * (4 * NT)) * THREADS + tid;
#pragma unroll
        for (int tf = 0; tf < NT; ++tf)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                part[(tf * 4 + j) * THREADS] = f32x4{acc[tf][4 * j], acc[tf][4 * j + 1],
                                                 acc[tf][4 * j + 2], acc[tf][4 * j + 3]};
        return;
    }
    if (YT != RXQ4_DTYPE_F32 && (p.M & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0) {
        // Stage the tile as [token][RPW rows] (16-bit) in the ring, then
        // write 16 bytes per lane: RPW / 8 lanes cover one token's rows.
        lds_barrier();  // every wave is done reading the ring
        uint8_t *ot = lds;
#pragma unroll
        for (int tf = 0; tf < NT; ++tf)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 32 * tf + lr, r = wave * kW8Rows + 8 * j + 4 * h;
                uint32_t lo, hi;
                if (YT == RXQ4_DTYPE_F16) {
                    lo = f32_to_f16_bits(acc[tf][4 * j]) |
                         ((uint32_t)f32_to_f16_bits(acc[tf][4 * j + 1]) << 16);
                    hi = f32_to_f16_bits(acc[tf][4 * j + 2]) |
                         ((uint32_t)f32_to_f16_bits(acc[tf][4 * j + 3]) << 16);
                } else {
                    lo = f32_to_bf16_bits(acc[tf][4 * j]) |
                         ((uint32_t)f32_to_bf16_bits(acc[tf][4 * j + 1]) << 16);
                    hi = f32_to_bf16_bits(acc[tf][4 * j + 2]) |
                         ((uint32_t)f32_to_bf16_bits(acc[tf][4 * j + 3]) << 16);
                }
                *reinterpret_cast<u32x2 *>(ot + t * kOutPitch + r * 2) = u32x2{lo, hi};
            }
        wait_lgkmcnt0();
        lds_barrier();
        const int row0 = row_tile * RPW;
        constexpr int LPT = RPW / 8;  // lanes per token
#pragma unroll
        for (int i = 0; i < TM * LPT / THREADS; ++i) {
            const int id = tid + THREADS * i, t = id / LPT, c = id % LPT;
            const int tok = tok_base + t, row = row0 + 8 * c;
            if (tok < p.N && row < p.M)  // M % 8 == 0: all 8 rows are in range
                *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(p.y) + (int64_t)tok * p.M + row) =
                    *reinterpret_cast<const u32x4 *>(ot + t * kOutPitch + c * 16);
        }
        return;
    }
    // 4 outputs per store need M % 4 == 0 and a 16-byte aligned y (any
    // y alignment the element size allows is accepted: then element stores)
    const bool vec_ok = (p.M & 3) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0;
#pragma unroll
    for (int tf = 0; tf < NT; ++tf)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = row_base + 8 * j + 4 * h, tok = tok_base + 32 * tf + lr;
            if (tok >= p.N || row >= p.M) continue;
            const int valid = min(4, p.M - row);
            store4<YT>(p.y, (int64_t)tok * p.M + row,
                       f32x4{acc[tf][4 * j], acc[tf][4 * j + 1], acc[tf][4 * j + 2],
                             acc[tf][4 * j + 3]},
                       vec_ok && valid == 4, valid);
        }
}

template <int T, int XT, int YT, int TM, int NW = 8>
__global__ __launch_bounds__(64 * NW) void gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[gemm_lds_bytes<TM, NW>()];
    const int L = blockIdx.x;
    const int V = (L % 8) * p.units_per_xcd + L / 8;  // consecutive units share an XCD
    if (V >= p.total_units) return;
    // Unit order.  Row-major, V = (row_tile * tok_tiles + tok_tile) * splits
    // + split: an XCD holds all token tiles and splits of its row tiles, so
    // it reads their weights once and every XCD reads all of x.
    // Token-major, V = (tok_tile * splits + split) * row_tiles + row_tile:
    // an XCD holds all row tiles of a few (token tile, split) pairs, so it
    // reads only their part of x and the weights once per token tile.  The
    // launcher takes the order with less L2 fill traffic (8 x-reads + the
    // weights against x + one weight read per token tile).
    int split, row_tile, tok_tile;
    if (p.tok_major) {
        row_tile = V % p.row_tiles;
        const int r = V / p.row_tiles;
        split = r % p.splits;
        tok_tile = r / p.splits;
    } else {
        split = V % p.splits;
        const int t = V / p.splits;
        row_tile = t / p.tok_tiles;
        tok_tile = t % p.tok_tiles;
    }
    gemm_tile<T, XT, YT, TM, NW>(p, lds, split, row_tile, tok_tile);
}

// Mixed token tiles for GEMMs that fill the CUs between one and two times
// with 256-token tiles.  The units are the 256-token tiles ("areas", no K
// split), dealt to the XCDs in runs of units_per_xcd as in gemm_kernel.
// Workgroup j of an XCD (block 8j + xcd) takes the XCD's area j whole while
// j < big_per_xcd (one per CU: the first round), and the later areas as two
// 128-token halves, which the CUs take as the whole tiles finish.  Every
// output element sums the same products in the same order as either kernel
// alone.
template <int T, int XT, int YT>
__global__ __launch_bounds__(512) void gemm_mixed_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[gemm_lds_bytes<256>()];
    const int L = blockIdx.x;
    const int xcd = L % 8, j = L / 8;
    const int first = xcd * p.units_per_xcd;
    const int end = min(p.total_units, first + p.units_per_xcd);
    const bool whole = j < p.big_per_xcd;
    const int u = whole ? j : p.big_per_xcd + ((j - p.big_per_xcd) >> 1);
    const int V = first + u;
    if (V >= end) return;
    int row_tile, tok_tile;
    if (p.tok_major) {
        row_tile = V % p.row_tiles;
        tok_tile = V / p.row_tiles;
    } else {
        row_tile = V / p.tok_tiles;
        tok_tile = V % p.tok_tiles;
    }
    if (whole) {
        gemm_tile<T, XT, YT, 256>(p, lds, 0, row_tile, tok_tile);
    } else {
        const int t128 = 2 * tok_tile + ((j - p.big_per_xcd) & 1);
        if (t128 * 128 >= p.N) return;  // the second half of a partial last area
        gemm_tile<T, XT, YT, 128>(p, lds, 0, row_tile, t128);
    }
}

// Split-K reduction for gemm_kernel: block (tile, e), e = tf*4 + j, sums
// float4 e of every thread of the tile over the splits in split order.
template <int YT, int TM, int NW = 8>
__global__ __launch_bounds__(64 * NW) void gemm_reduce_kernel(GemmParams p) {
    constexpr int E = 4 * (TM / 32);  // float4 per thread
    constexpr int THREADS = 64 * NW;
    const int tid = threadIdx.x;
    // Block b runs on XCD b % 8 and reduces tiles whose first split ran on
    // that XCD in the row-major unit order (units [x * units_per_xcd,
    // (x + 1) * units_per_xcd)); in the token-major order the same blocks
    // cover every tile once, without that locality.
    const int xcd = blockIdx.x % 8, jj = blockIdx.x / 8;
    const int t0 = (xcd * p.units_per_xcd + p.splits - 1) / p.splits;
    const int t1 = ((xcd + 1) * p.units_per_xcd + p.splits - 1) / p.splits;
    const int tile = t0 + jj / E;
    const int e = jj % E;
    if (tile >= t1 || tile >= p.row_tiles * p.tok_tiles) return;
    const int tf = e / 4, j = e % 4;
    const int row_tile = tile / p.tok_tiles, tok_tile = tile % p.tok_tiles;
    const int lane = tid & 63, wave = tid >> 6;
    const int row = row_tile * 32 * NW + wave * kW8Rows + 8 * j + 4 * (lane >> 5);
    const int tok = tok_tile * TM + 32 * tf + (lane & 31);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.ws) +
                       ((int64_t)tile * p.splits * E + e) * THREADS + tid;
    // Up to 8 splits' loads are in flight before the first add (a loop of
    // dependent load-add steps waits out one memory latency per split); the
    // adds stay in split order.
    f32x4 sum = src[0];
    for (int sp0 = 1; sp0 < p.splits; sp0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (sp0 + i < p.splits) v[i] = src[(int64_t)(sp0 + i) * E * THREADS];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (sp0 + i < p.splits)
                sum = f32x4{sum[0] + v[i][0], sum[1] + v[i][1], sum[2] + v[i][2], sum[3] + v[i][3]};
    }
    if (tok >= p.N || row >= p.M) return;
    const int valid = min(4, p.M - row);
    const bool vec_ok = (p.M & 3) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0;
    store4<YT>(p.y, (int64_t)tok * p.M + row, sum, vec_ok && valid == 4, valid);
}

// ---------------------------------------------------------------------------
// Small batch (2..16 tokens): a workgroup of KW waves owns 16*RT weight rows
// x 16 tokens.  The K super-blocks are dealt to the waves round-robin (wave
// w: w, w+KW, ...); each wave computes RT 16x16 fragments with
// v_mfma_f32_16x16x32 (A = 16 weight rows, B = the 16 tokens), so one x
// fragment serves RT row tiles.  Two weight layouts (WIDE):
//   * WIDE (up to 8 tokens): lane (row li, group g) loads the 32 qs bytes of
//     quant group g with two 16-byte loads and needs only that group's
//     scales; k-step s (0..7) gives it nibble s / 4 of bytes 8*(s % 4) .. +7,
//     i.e. elements 64g + 32*(s/4) + 8*(s%4) + e, and the x fragment of the
//     step is read at those elements (four 16-byte pieces per token);
//   * otherwise lane g loads bytes 8g .. 8g+7 of every quant group (four
//     8-byte loads) and the x fragments are 64-byte runs per token.
// On 36 distinct gate+up layers the wide loads took m = 8 from 14.7 to
// 12.9 us, while m = 16, where all 16 token lanes read x, lost to the
// scattered x pieces (down 16.2 -> 19.3 us).  Each wave keeps two super-blocks of weights and x
// in flight (loads unconditional, clamped to the last super-block, so the
// compiler's vmcnt waits stay exact).  x is read through a buffer resource
// bounded at N*K elements: the lanes of tokens >= N read past it and get
// zeros without touching memory.  Partial sums are added in wave order
// through LDS.
template <int XT, int YT, int RT, int KW, bool WIDE>
__global__ __launch_bounds__(KW * 64) void gemv_tokens_kernel(
    void *__restrict__ y, const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, int M,
    int N, int K, float *__restrict__ ws, int sb_per_split) {
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
    // bytes; >= N*K*2 for tokens >= N
    const int xoff = li * K * 2 + (WIDE ? 128 * g : 16 * g);
    // Super-blocks [sb_lo, sb_hi) of K split blockIdx.y (all of K without a
    // split), dealt to the waves round-robin.
    const int sb_lo = blockIdx.y * sb_per_split, sb_hi = min(nb, sb_lo + sb_per_split);
    const int n_sb = sb_hi - sb_lo;
    const int n_w = wave < n_sb ? (n_sb - 1 - wave) / KW + 1 : 0;  // super-blocks of this wave

    // x element of k-step s (0..7) for this lane's group g, relative to the
    // super-block: WIDE 64g + 32*(s/4) + 8*(s%4); otherwise 64*(s/2) +
    // 32*(s%2) + 8g (quant group s/2, nibble s%2, bytes 8g .. 8g+7).
    auto x_elem = [](int s) { return WIDE ? 32 * (s >> 2) + 8 * (s & 3) : 64 * (s >> 1) + 32 * (s & 1); };
    struct Sb {
        u32x4 hdr[RT];
        u32x4 qw[RT][2];  // WIDE: qs bytes 32g .. 32g+31
        u32x2 q[RT][4];   // otherwise: bytes 32il + 8g .. +7 of quant group il
        u32x4 b[8];
    };
    auto load = [&](int i, Sb &o) {
        const int sb = min(sb_lo + wave + i * KW, sb_hi - 1);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint8_t *blk = wr[t] + sb * kBlockBytes;
            o.hdr[t] = load16(blk);
            if (WIDE) {
                o.qw[t][0] = load16(blk + 16 + 32 * g);
                o.qw[t][1] = load16(blk + 32 + 32 * g);
            } else {
#pragma unroll
                for (int il = 0; il < 4; ++il)
                    o.q[t][il] = *reinterpret_cast<const u32x2 *>(blk + 16 + 32 * il + 8 * g);
            }
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) o.b[s] = buffer_load16(xr, xoff + 2 * (sb * 256 + x_elem(s)));
    };
    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Sb &o) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            if (WIDE) {
                const GroupScales gsc = group_scales(o.hdr[t], g);
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const u32x4 &w = o.qw[t][(s >> 1) & 1];
                    const bool hi = s >= 4;
                    const u32x4 a = dequant8<XT>((s & 1) ? w.z : w.x, (s & 1) ? w.w : w.y, hi,
                                                 hi ? gsc.hi : gsc.lo, hi ? gsc.dm_hi : gsc.dm_lo);
                    acc[t] = mfma<XT>(a, o.b[s], acc[t]);
                }
            } else {
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
                if (row >= M) continue;
                if (ws)  // split K: fp32 partial [split][token][row]
                    ws[((int64_t)blockIdx.y * N + li) * M + row] = sum[r];
                else
                    store_out<YT>(y, (int64_t)li * M + row, sum[r]);
            }
        }
    }
}

// Small batch with x staged in LDS, for matrices with at least one 64-row
// workgroup per CU (gate+up): the W waves split rows (16*RT each, all of K)
// and share each super-block's x tile (16 tokens x 512 bytes), copied once
// per workgroup by direct-to-LDS loads into a ring of 3 buffers, 2
// super-blocks ahead.  Chunk c (16 bytes) of token t sits at c ^ (t & 15),
// so a 16-lane fragment read covers the 64 banks once.  Weights use the
// 16-byte (WIDE) layout of gemv_tokens_kernel.  Against gemv_tokens_kernel
// (x fragments from L2 per wave) on 36 distinct gate+up layers: m = 16
// 17.0 -> 13.3 us, m = 8 13.2 -> 12.8 us; down (32 such workgroups, K split
// needed) stays on gemv_tokens_kernel.
template <int XT, int YT, int RT, int W>
__global__ __launch_bounds__(W * 64) void gemv_tokens_lds_kernel(
    void *__restrict__ y, const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, int M,
    int N, int K, float *__restrict__ ws, int sb_per_split) {
    constexpr int D = 2;             // super-blocks in flight per wave
    constexpr int kBuf = D + 1;
    // x copy instructions per wave and super-block: the tile is 8 copies of
    // 1 KB; with W not dividing 8 the copies j >= 8 repeat copy j % 8 (the
    // same bytes to the same place), so every wave issues kXc copies and the
    // vmcnt waits below stay exact
    constexpr int kXc = (8 + W - 1) / W;
    __shared__ __attribute__((aligned(1024))) uint8_t xs[kBuf][16 * 512];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int nb = K >> 8;
    // super-blocks [sb_lo, sb_lo + n_sb) of K split blockIdx.y (all of K
    // without a split)
    const int sb_lo = blockIdx.y * sb_per_split;
    const int n_sb = min(nb, sb_lo + sb_per_split) - sb_lo;
    const int row0 = (blockIdx.x * W + wave) * 16 * RT;
    const int64_t row_bytes = (int64_t)nb * kBlockBytes;
    const uint8_t *wr[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) wr[t] = w + min(row0 + 16 * t + li, M - 1) * row_bytes;

    // x copies: instruction u of wave w covers tokens 2j, 2j + 1 (j = (w +
    // W*u) % 8); lane i: token 2j + i/32 (clamped to N - 1), LDS chunk i % 32.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, N * K * 2);
    int xoff[kXc];
#pragma unroll
    for (int u = 0; u < kXc; ++u) {
        const int t = 2 * ((wave + W * u) & 7) + (lane >> 5), p = lane & 31;
        xoff[u] = (min(t, N - 1) * K + 8 * (p ^ (t & 15))) * 2;
    }
    // Super-blocks past the end are still loaded, from one fixed line (the
    // first 512 B of x, the first block of w), so that every step issues the
    // same number of loads and all vmcnt waits stay exact (a branch around
    // the loads made the compiler's waits drain the prefetch: 9.7 -> 8.0 us
    // at m = 5 on [16384 x 2048]); their copies land in a ring buffer no
    // step reads again.
    auto issue_x = [&](int i) {
        const bool live = i < n_sb;  // uniform
        uint8_t *dst = xs[i % kBuf];
#pragma unroll
        for (int u = 0; u < kXc; ++u)
            buffer_to_lds16(xr, dst + ((wave + W * u) & 7) * 1024, live ? xoff[u] : 16 * (lane & 31),
                            live ? (sb_lo + i) * 512 : 0);
    };
    struct Sb {
        u32x4 hdr[RT];
        u32x4 qw[RT][2];
    };
    auto load = [&](int i, Sb &o) {
        const bool live = i < n_sb;  // uniform
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint8_t *blk = live ? wr[t] + (sb_lo + i) * kBlockBytes : w;
            o.hdr[t] = load16(blk);
            o.qw[t][0] = load16(blk + 16 + 32 * g);
            o.qw[t][1] = load16(blk + 32 + 32 * g);
        }
    };
    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Sb &o, int i) {
        const uint8_t *xb = xs[i % kBuf] + li * 512;
        u32x4 b[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int c = 8 * g + 4 * (s >> 2) + (s & 3);  // chunk of elements 64g + 32(s/4) + 8(s%4)
            b[s] = *reinterpret_cast<const u32x4 *>(xb + 16 * (c ^ li));
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const GroupScales gsc = group_scales(o.hdr[t], g);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const u32x4 &q = o.qw[t][(s >> 1) & 1];
                const bool hi = s >= 4;
                const u32x4 a = dequant8<XT>((s & 1) ? q.z : q.x, (s & 1) ? q.w : q.y, hi,
                                             hi ? gsc.hi : gsc.lo, hi ? gsc.dm_hi : gsc.dm_lo);
                acc[t] = mfma<XT>(a, b[s], acc[t]);
            }
        }
    };
    // Per step i: this wave's copies of super-block i have landed once the
    // loads issued after them (its weights, then copies and weights of the
    // D - 1 super-blocks after it: 3*RT + (D-1)*(3*RT + kXc)) are at most
    // outstanding; the barrier makes all W waves' copies visible and says
    // every wave is done with buffer (i - 1) % (D + 1), which the copies of
    // i + D refill.  Steps past n_sb (the last round) only load.
    auto step = [&](int i, Sb &S) {
        wait_vmcnt<3 * RT + (D - 1) * (3 * RT + kXc)>();
        lds_barrier();
        issue_x(i + D);
        if (i < n_sb) compute(S, i);  // uniform
        load(i + D, S);
    };
    Sb S[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue_x(j);
        load(j, S[j]);
    }
    for (int i0 = 0; i0 < n_sb; i0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) step(i0 + j, S[j]);
    }
    wait_vmcnt<0>();  // trailing copies must land before the workgroup exits

#pragma unroll
    for (int t = 0; t < RT; ++t) {
        if (li >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 16 * t + 4 * g + r;
            if (row >= M) continue;
            if (ws)  // split K: fp32 partial [split][token][row]
                ws[((int64_t)blockIdx.y * N + li) * M + row] = acc[t][r];
            else
                store_out<YT>(y, (int64_t)li * M + row, acc[t][r]);
        }
    }
}

// y[i] = sum over the K splits, in split order, of the partials ws[split][i]
// (i over N x M, token-major).
template <int YT>
__global__ __launch_bounds__(256) void tokens_reduce_kernel(void *__restrict__ y,
                                                            const float *__restrict__ ws,
                                                            int64_t n, int splits) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    // up to 8 splits' loads in flight before the adds (in split order)
    float s = ws[i];
    for (int k0 = 1; k0 < splits; k0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (k0 + j < splits) v[j] = ws[(int64_t)(k0 + j) * n + i];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (k0 + j < splits) s += v[j];
    }
    store_out<YT>(y, i, s);
}

template <int T, int XT, int YT, int TM, int NW = 8>
static hipError_t launch_gemm_t(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                int K, hipStream_t st, const Scratch &sc) {
    constexpr int RPW = 32 * NW, THREADS = 64 * NW;
    // 32-bit buffer offsets: the x tile, and a wave's 32 rows of Q6_K weights
    const int64_t row_bytes = (int64_t)(K / 256) * GemmFmt<T>::kBytes;
    if ((int64_t)TM * K * 2 > 0x7FFFFFFF || (T == 14 && row_bytes * kW8Rows > 0x7FFFFFFF))
        return hipErrorInvalidValue;
    GemmParams p{};
    p.y = y;
    p.w = w;
    p.x = x;
    p.M = M;
    p.N = N;
    p.K = K;
    p.nb = K / 256;
    p.row_tiles = (M + RPW - 1) / RPW;
    p.tok_tiles = (N + TM - 1) / TM;
    const int tiles = p.row_tiles * p.tok_tiles;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    // Split K into as many parts as keep every unit resident at once (one
    // workgroup per CU: tiles * splits <= CUs), at least 2 super-blocks a
    // split: 32 tiles on 256 CUs split 8, 86 split 2, 172 do not split.
    int splits = std::max(1, cus / tiles);
    splits = std::min(splits, std::max(1, p.nb / 2));
    if (tuning().gemm_splits) splits = tuning().gemm_splits;
    // the fp32 partials (one TM x 256 tile per unit) must fit the scratch
    const size_t unit_bytes = (size_t)TM * RPW * sizeof(float);
    splits = (int)std::min<size_t>(splits, std::max<size_t>(1, sc.capacity() / (unit_bytes * tiles)));
    splits = std::max(1, std::min(splits, p.nb));
    p.sb_per_split = (p.nb + splits - 1) / splits;
    splits = (p.nb + p.sb_per_split - 1) / p.sb_per_split;  // no empty splits
    p.splits = splits;
    if (splits > 1) {
        hipError_t e = sc.get(st, unit_bytes * tiles * splits, &p.ws);
        if (e != hipSuccess) return e;
    }
    p.total_units = tiles * splits;
    p.units_per_xcd = (p.total_units + 7) / 8;
    const double x_bytes = 2.0 * N * K, w_bytes = (double)M * row_bytes;
    p.tok_major = tuning().gemm_order ? tuning().gemm_order == 2
                                      : x_bytes + p.tok_tiles * w_bytes < 8 * x_bytes + w_bytes;
    gemm_kernel<T, XT, YT, TM, NW><<<8 * p.units_per_xcd, THREADS, 0, st>>>(p);
    if (splits > 1) {  // 4 * TM / 32 float4 per thread; at most units_per_xcd / splits + 1 tiles per XCD
        constexpr int E = 4 * (TM / 32);
        gemm_reduce_kernel<YT, TM, NW>
            <<<8 * E * ((p.units_per_xcd + splits - 1) / splits + 1), THREADS, 0, st>>>(p);
    }
    return hipGetLastError();
}

// One round of 256-token tiles (one workgroup per CU) against one of
// 128-token tiles: measured ~1.6x for twice the work ([11008 x 2048] on one
// box: 54-60 us against 35-37 us).
constexpr int kBigTileCost = 16, kHalfTileCost = 10;

// Mixed token tiles (gemm_mixed_kernel): areas of 256 tokens dealt to the
// XCDs, the first big_per_xcd of each run whole, the rest as 128-token
// halves.  Q4_K/Q5_K only, no K split (it is taken with at least one
// 128-token tile per CU).
template <int T, int XT, int YT>
static hipError_t launch_gemm_mixed(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                   int K, int big_per_xcd, hipStream_t st) {
    if ((int64_t)256 * K * 2 > 0x7FFFFFFF) return hipErrorInvalidValue;
    GemmParams p{};
    p.y = y;
    p.w = w;
    p.x = x;
    p.M = M;
    p.N = N;
    p.K = K;
    p.nb = K / 256;
    p.row_tiles = (M + kRowsPerWg - 1) / kRowsPerWg;
    p.tok_tiles = (N + 255) / 256;
    p.splits = 1;
    p.sb_per_split = p.nb;
    p.total_units = p.row_tiles * p.tok_tiles;
    p.units_per_xcd = (p.total_units + 7) / 8;
    p.big_per_xcd = std::min(big_per_xcd, p.units_per_xcd);
    const double x_bytes = 2.0 * N * K, w_bytes = (double)M * (K / 256) * GemmFmt<T>::kBytes;
    p.tok_major = tuning().gemm_order ? tuning().gemm_order == 2
                                      : x_bytes + p.tok_tiles * w_bytes < 8 * x_bytes + w_bytes;
    const int per_xcd = p.big_per_xcd + 2 * (p.units_per_xcd - p.big_per_xcd);
    gemm_mixed_kernel<T, XT, YT><<<8 * per_xcd, 512, 0, st>>>(p);
    return hipGetLastError();
}

// Token tile.  256 tokens per workgroup halve the dequantisation per MFMA
// (each wave's 32 dequantised rows feed 8 token fragments) for ~1.6x the
// time of a 128-token tile.  With at least one 128-token tile per CU the
// launcher estimates, per XCD, the time of R rounds of whole 256-token
// tiles followed by the remaining areas as 128-token halves (R = 0: the
// 128-token kernel; every area whole: the 256-token kernel; else the mixed
// kernel), and takes the fastest: m = 1024 on [11008 x 2048] (22 areas per
// XCD of 32 CUs) one round of 256; m = 2048 (43 areas) one round of 256
// and 22 halves against 3 rounds of 128 or 2 of 256; m = 4096 three rounds
// of 256.  With fewer 128-token tiles than CUs the 128-token tile and its
// K splits win (the 256-token partials double the split traffic).  Q6_K
// keeps 128 (its format needs more registers).
template <int T, int XT, int YT>
static hipError_t launch_gemm_tm(void *y, const uint8_t *w, const uint16_t *x, int M, int N,
                                 int K, hipStream_t st, const Scratch &sc) {
    int tm = tuning().gemm_tm;
    int big = -1;  // whole areas per XCD for the mixed kernel
    if (tm != 128 && tm != 256) {
        const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
        const int c = std::max(1, cus / 8);  // CUs per XCD
        const int64_t rows = (M + kRowsPerWg - 1) / kRowsPerWg;
        const int64_t t128 = rows * ((N + 127) / 128), t256 = rows * ((N + 255) / 256);
        tm = 128;
        if (T != 14 && t128 >= cus) {
            const int64_t a = (t256 + 7) / 8, u128 = (t128 + 7) / 8;  // per XCD
            int64_t best = ((u128 + c - 1) / c) * kHalfTileCost;
            for (int64_t r = 1; r <= (a + c - 1) / c; ++r) {
                const int64_t halves = 2 * std::max<int64_t>(0, a - r * c);
                const int64_t cost = r * kBigTileCost + (halves + c - 1) / c * kHalfTileCost;
                if (cost < best) {
                    best = cost;
                    tm = 256;
                    big = halves ? (int)(r * c) : -1;
                }
            }
        }
    }
    if (tuning().gemm_mixed > 0 && T != 14) big = tuning().gemm_mixed;
    if constexpr (T == 14) {
        // Q6_K (128-token tiles only): the same four-wave rule as below
        // ([2048 x 11008] at m = 512: 49.1 -> 45.5 us on one box)
        int nw = tuning().gemm_nw;
        if (nw != 4 && nw != 8) {
            const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
            const int64_t tiles8 = (int64_t)((M + kRowsPerWg - 1) / kRowsPerWg) * ((N + 127) / 128);
            const int64_t splits8 = std::min<int64_t>(cus / std::max<int64_t>(1, tiles8), (K / 256) / 2);
            nw = splits8 >= 8 ? 4 : 8;
        }
        if (nw == 4) return launch_gemm_t<T, XT, YT, 128, 4>(y, w, x, M, N, K, st, sc);
    }
    if constexpr (T != 14) {
        // Four-wave workgroups (128-row tiles, one wave per SIMD) for shapes
        // that the eight-wave plan splits 8 ways or more: twice the tiles
        // halve the split count and the fp32 partials ([2048 x 11008] and
        // [2048 x 8192] at m = 512: 32 MiB -> 16 MiB, 42.8 -> 40.0 and
        // 31.5 -> 29.1 us on one box; shapes split 4 ways or less measured
        // slower with them).
        int nw = tuning().gemm_nw;
        if (nw != 4 && nw != 8 && tm == 128 && big <= 0) {
            const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
            const int64_t tiles8 = (int64_t)((M + kRowsPerWg - 1) / kRowsPerWg) * ((N + 127) / 128);
            const int64_t splits8 = std::min<int64_t>(cus / std::max<int64_t>(1, tiles8), (K / 256) / 2);
            nw = splits8 >= 8 ? 4 : 8;
        }
        if (nw == 4) {
            if (tm == 256) return launch_gemm_t<T, XT, YT, 256, 4>(y, w, x, M, N, K, st, sc);
            return launch_gemm_t<T, XT, YT, 128, 4>(y, w, x, M, N, K, st, sc);
        }
        if (big > 0) return launch_gemm_mixed<T, XT, YT>(y, w, x, M, N, K, big, st);
        if (tm == 256) return launch_gemm_t<T, XT, YT, 256>(y, w, x, M, N, K, st, sc);
    }
    return launch_gemm_t<T, XT, YT, 128>(y, w, x, M, N, K, st, sc);
}

template <int T>
static hipError_t launch_gemm_xy(void *y, int y_dtype, const uint8_t *w, const void *x,
                                 int x_dtype, int M, int N, int K, hipStream_t st,
                                 const Scratch &sc) {
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            return launch_gemm_tm<T, RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16>(y, w, xx, M, N, K, st, sc);
        return launch_gemm_tm<T, RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st, sc);
    }
    if (y_dtype == RXQ4_DTYPE_F16)
        return launch_gemm_tm<T, RXQ4_DTYPE_F16, RXQ4_DTYPE_F16>(y, w, xx, M, N, K, st, sc);
    return launch_gemm_tm<T, RXQ4_DTYPE_F16, RXQ4_DTYPE_F32>(y, w, xx, M, N, K, st, sc);
}

hipError_t launch_gemm(int ggml_type, void *y, int y_dtype, const uint8_t *w, const void *x,
                       int x_dtype, int M, int N, int K, hipStream_t st, const Scratch &sc) {
    if (ggml_type == 14) return launch_gemm_xy<14>(y, y_dtype, w, x, x_dtype, M, N, K, st, sc);
    if (ggml_type == 13) return launch_gemm_xy<13>(y, y_dtype, w, x, x_dtype, M, N, K, st, sc);
    return launch_gemm_xy<12>(y, y_dtype, w, x, x_dtype, M, N, K, st, sc);
}

template <int XT, int YT>
static hipError_t launch_tokens_t(void *y, const uint8_t *w, const uint16_t *x, int M, int n_tok,
                                  int K, hipStream_t st, const Scratch &sc) {
    // Four waves split K.  Two row tiles per wave halve the x traffic per
    // weight byte and pay off once there are enough of them to give about
    // four waves per CU (1024 waves); a measured sweep of 1/2/4 row tiles and
    // 1/2/4/8 waves on gate+up [22016 x 2048], down [2048 x 11008] and QKV
    // [2560 x 2048] at 2..16 tokens put these two shapes first.  Long rows
    // with few row tiles (down) also split K over workgroups: 32-row tiles x
    // up to CUs / tiles splits of at least 8 super-blocks, fp32 partials
    // summed in split order by tokens_reduce_kernel (down m = 8: 12.4 us
    // unsplit on 128 workgroups).
    // Up to 8 tokens the wide weight loads win (the x lanes of tokens >= N
    // read nothing); with 9..16 tokens the x fragments' 64-byte runs per
    // token matter more (measured on 36 distinct layers).
    constexpr int kWaves = 4;
    const int nb = K / 256;
    const int t2 = (M + 31) / 32;
    const bool wide = n_tok <= 8;
    const int cus = device_info().cu_count > 0 ? device_info().cu_count : 256;
    if ((M + 63) / 64 >= cus) {
        // Workgroups of W = 4, 6 or 8 waves (16 rows each), one per CU when
        // they fit: W minimises the rows of the busiest CU, 16 W times the
        // rounds of workgroups (ties to the larger W).  [22016 x 2048]: 230
        // workgroups of 96 rows (4 waves: 344 put two on 88 CUs; 8 waves:
        // 172 leave 84 CUs idle); m = 16: 13.5 / 11.8 / 11.1 us with 4 / 8 /
        // 6 waves.
        const int g64 = (M + 63) / 64;
        int nw = tuning().tokens_waves;
        if (nw != 4 && nw != 6 && nw != 8) {
            int best = 0;
            for (const int c : {8, 6, 4}) {
                const int groups = (M + 16 * c - 1) / (16 * c);
                const int busiest = 16 * c * ((groups + cus - 1) / cus);  // rows of the busiest CU
                if (best == 0 || busiest < best) best = busiest, nw = c;
            }
        }
        if (nw == 8)
            gemv_tokens_lds_kernel<XT, YT, 1, 8>
                <<<(M + 127) / 128, 512, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
        else if (nw == 6)
            gemv_tokens_lds_kernel<XT, YT, 1, 6>
                <<<(M + 95) / 96, 384, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
        else
            gemv_tokens_lds_kernel<XT, YT, 1, 4><<<g64, 256, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
        return hipGetLastError();
    }
    if (nb >= 16) {
        // Long rows: 64-row workgroups with x staged in LDS and K split over
        // workgroups (about one per CU, at least 4 super-blocks a split).
        const int g64 = (M + 63) / 64;
        int splits = tuning().tokens_lds_split ? std::min(tuning().tokens_lds_split, nb)
                                               : std::max(1, std::min(cus / g64, nb / 4));
        splits = (int)std::min<size_t>(
            splits, std::max<size_t>(1, sc.capacity() / ((size_t)n_tok * M * sizeof(float))));
        const int sbps = (nb + splits - 1) / splits;
        splits = (nb + sbps - 1) / sbps;
        float *ws = nullptr;
        if (splits > 1) {
            hipError_t e = sc.get(st, (size_t)splits * n_tok * M * sizeof(float), &ws);
            if (e != hipSuccess) return e;
        }
        gemv_tokens_lds_kernel<XT, YT, 1, 4>
            <<<dim3(g64, splits), 256, 0, st>>>(y, w, x, M, n_tok, K, ws, sbps);
        if (splits > 1) {
            const int64_t n = (int64_t)n_tok * M;
            tokens_reduce_kernel<YT><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(y, ws, n, splits);
        }
        return hipGetLastError();
    }
    // Short rows (nb < 16): the register kernel, never split over K (every
    // row is at most 15 super-blocks, dealt to the waves of one workgroup).
    if (t2 * kWaves >= 1024) {
        const dim3 grid(t2, 1);
        if (wide)
            gemv_tokens_kernel<XT, YT, 2, kWaves, true>
                <<<grid, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
        else
            gemv_tokens_kernel<XT, YT, 2, kWaves, false>
                <<<grid, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
    } else {
        const int t1 = (M + 15) / 16;
        if (wide)
            gemv_tokens_kernel<XT, YT, 1, kWaves, true>
                <<<t1, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
        else
            gemv_tokens_kernel<XT, YT, 1, kWaves, false>
                <<<t1, kWaves * 64, 0, st>>>(y, w, x, M, n_tok, K, nullptr, nb);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_tokens(void *y, int y_dtype, const uint8_t *w, const void *x,
                              int x_dtype, int M, int n_tok, int K, hipStream_t st,
                              const Scratch &sc) {
    const uint16_t *xx = static_cast<const uint16_t *>(x);
    if (x_dtype == RXQ4_DTYPE_BF16) {
        if (y_dtype == RXQ4_DTYPE_BF16)
            return launch_tokens_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_BF16>(y, w, xx, M, n_tok, K, st, sc);
        return launch_tokens_t<RXQ4_DTYPE_BF16, RXQ4_DTYPE_F32>(y, w, xx, M, n_tok, K, st, sc);
    }
    if (y_dtype == RXQ4_DTYPE_F16)
        return launch_tokens_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F16>(y, w, xx, M, n_tok, K, st, sc);
    return launch_tokens_t<RXQ4_DTYPE_F16, RXQ4_DTYPE_F32>(y, w, xx, M, n_tok, K, st, sc);
}

}  // namespace rxq4
