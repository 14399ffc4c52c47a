// embed_q4k.hip -- Q4_K embedding-row dequantisation for gfx950.
//
// Replaces dequant_embedding_q4k_kernel (reference q4_gemm.cu:545-572) and
// adds the batched gather the reference API cannot express.  A thread makes
// G groups of 8 consecutive outputs of one row: per group one 16-byte block
// header load, one 8-byte quant load (the group's low or high nibbles),
// w = (d*sc)*q - dmin*m in fp32 (one rounding, as the reference) and one
// 16-byte store of 8 fp16 (RNE).  With K a multiple of 512*G the groups of a
// thread are 512 outputs apart and lane j of a wave writes outputs 8j..8j+7
// of each 512-output run, so every store instruction writes 1 KB contiguous
// (16 outputs per thread in one piece, stores 32 bytes apart across the
// wave, measured 7.06 us against 6.55 us for 4096 fp16 rows of 2048).  The
// stores are nontemporal (6.56 -> 5.65 us; a plain 16 MiB write of zeros
// takes 4.62-4.70 us on the same box).  All of a thread's loads are issued
// before its arithmetic.  Only the addressed
// rows are read.  Bytes per launch: unique_rows*K/256*144 (header reads are
// L2 hits after the first) + n_ids*K*2 written + n_ids*4 ids.
#include "launch.h"
#include "q4k_device.h"

namespace rxq4 {

// Thread c of row i: output groups e_k = 512*G*(c/64) + 8*(c%64) + 512*k
// (kContig) or 8*G*c + 8*k, k < G.
template <bool kBatched, int G, bool kContig>
__global__ __launch_bounds__(256) void embed_kernel(uint16_t *__restrict__ dst,
                                                    const uint8_t *__restrict__ w,
                                                    const int32_t *__restrict__ ids,
                                                    int token_id, int64_t n_vocab,
                                                    int n_ids, int K) {
    const int per_row = K / (8 * G);
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // kContig: per_row is a multiple of 64, so a wave's threads share a row
    // and the row index, the id and the row address are scalars (the id a
    // scalar load: 4096 Zipf ids into fp16 rows of 2048 4.98-5.14 ->
    // 4.90-4.92 us)
    int64_t i;
    if (kContig) {
        const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4u + (threadIdx.x >> 6)));
        i = (int64_t)(wave / (uint32_t)(per_row >> 6));
    } else {
        i = t / per_row;
    }
    const int c = (int)(t - i * per_row);
    if (i >= n_ids) return;
    // output element groups (8 each) of this thread
    int e[G];
#pragma unroll
    for (int k = 0; k < G; ++k)
        e[k] = kContig ? (c >> 6) * (512 * G) + 8 * (c & 63) + 512 * k : c * 8 * G + 8 * k;
    int64_t id = token_id;
    if (kBatched) {
        id = ids[i];
        if (id < 0 || id >= n_vocab) {
#pragma unroll
            for (int k = 0; k < G; ++k)
                store16_nt(dst + i * K + e[k], u32x4{0, 0, 0, 0});
            return;
        }
    }
    const int nb = K >> 8;
    const uint8_t *rowp = w + id * (int64_t)(nb * kBlockBytes);
    u32x4 hd[G];
    u32x2 qv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int b = e[k] >> 8, pos = e[k] & 255;
        const uint32_t boff = (uint32_t)(b * kBlockBytes);  // 32-bit offsets from the row
        hd[k] = load16(rowp + boff);
        qv[k] = *reinterpret_cast<const u32x2 *>(rowp + (boff + (uint32_t)(16 + 32 * (pos >> 6) + (pos & 31))));
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int pos = e[k] & 255;
        const int il = pos >> 6, hi = (pos >> 5) & 1;
        const u32x4 h = hd[k];
        const float d = f16_bits_to_f32(h.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(h.x >> 16);
        uint32_t sc, mn;
        scale_one(h.y, h.z, h.w, 2 * il + hi, &sc, &mn);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t qw[2] = {qv[k].x, qv[k].y};
        uint32_t packed[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t word = qw[j >> 1];
            const int sh = (j & 1) * 16;
            uint32_t b0 = (word >> sh) & 0xFFu, b1 = (word >> (sh + 8)) & 0xFFu;
            b0 = hi ? (b0 >> 4) : (b0 & 0xFu);
            b1 = hi ? (b1 >> 4) : (b1 & 0xFu);
            const float v0 = ds * (float)b0 - dm;
            const float v1 = ds * (float)b1 - dm;
            packed[j] = (uint32_t)f32_to_f16_bits(v0) | ((uint32_t)f32_to_f16_bits(v1) << 16);
        }
        store16_nt(dst + i * K + e[k], u32x4{packed[0], packed[1], packed[2], packed[3]});
    }
}

template <int G, bool C>
static void launch_embed_v(uint16_t *dst, const uint8_t *w, const int32_t *ids, int token_id,
                           int64_t n_vocab, int n_ids, int K, hipStream_t st) {
    const int64_t grid = ((int64_t)n_ids * (K / (8 * G)) + 255) / 256;
    if (ids)
        embed_kernel<true, G, C><<<(unsigned)grid, 256, 0, st>>>(dst, w, ids, 0, n_vocab, n_ids, K);
    else
        embed_kernel<false, G, C><<<(unsigned)grid, 256, 0, st>>>(dst, w, nullptr, token_id, 0, 1, K);
}

hipError_t launch_embed(uint16_t *dst, const uint8_t *w, const int32_t *ids, int token_id,
                        int64_t n_vocab, int n_ids, int K, hipStream_t st) {
    const int64_t threads = (int64_t)n_ids * (K >> 4);
    const int64_t grid = (threads + 255) / 256;
    if (grid <= 0) return hipSuccess;
    // the contiguous-store kernels form the wave index blockIdx.x * 4 + w in
    // 32 bits (2^30 workgroups: 16 TB of output, far past any device)
    if (grid > (int64_t)1 << 30) return hipErrorInvalidValue;
    // 8-output groups per thread: 4 (stores contiguous across the wave in
    // 512-output runs) when K allows, else 2, or 2 adjacent ones
    if (K % 2048 == 0)
        launch_embed_v<4, true>(dst, w, ids, token_id, n_vocab, n_ids, K, st);
    else if (K % 1024 == 0)
        launch_embed_v<2, true>(dst, w, ids, token_id, n_vocab, n_ids, K, st);
    else
        launch_embed_v<2, false>(dst, w, ids, token_id, n_vocab, n_ids, K, st);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Quantiser (the reference ships none): one wave per 256-value block, four
// values per lane, eight lanes per 32-value sub-block.  Same arithmetic, in the
// same order, as the oracle's quantize_block; only min/max, +, *, correctly
// rounded / and rint are used, so the bytes are identical.
#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void quantize_kernel(uint8_t *__restrict__ dst,
                                                       const float *__restrict__ src,
                                                       int64_t n_blocks) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= n_blocks) return;
    const float *v = src + blk * kQK + lane * 4;
    const float x0 = v[0], x1 = v[1], x2 = v[2], x3 = v[3];
    float lo = x0, hi = x0;
    lo = x1 < lo ? x1 : lo; hi = x1 > hi ? x1 : hi;
    lo = x2 < lo ? x2 : lo; hi = x2 > hi ? x2 : hi;
    lo = x3 < lo ? x3 : lo; hi = x3 > hi ? x3 : hi;
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        const float ol = __shfl_xor(lo, off, 64), oh = __shfl_xor(hi, off, 64);
        lo = ol < lo ? ol : lo;
        hi = oh > hi ? oh : hi;
    }
    const float mo = lo < 0.0f ? -lo : 0.0f;
    const float top = hi > 0.0f ? hi : 0.0f;
    const float span = (top + mo) / 15.0f;
    float max_span = span, max_off = mo;
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        const float os = __shfl_xor(max_span, off, 64), oo = __shfl_xor(max_off, off, 64);
        max_span = os > max_span ? os : max_span;
        max_off = oo > max_off ? oo : max_off;
    }
    const uint16_t d_raw = f32_to_f16_bits(max_span / 63.0f);
    const uint16_t dmin_raw = f32_to_f16_bits(max_off / 63.0f);
    const float d = f16_bits_to_f32(d_raw);
    const float dmin = f16_bits_to_f32(dmin_raw);
    float scf = 0.0f, mnf = 0.0f;
    if (d > 0.0f) scf = fminf(fmaxf(rintf(span / d), 0.0f), 63.0f);
    if (dmin > 0.0f) mnf = fminf(fmaxf(rintf(mo / dmin), 0.0f), 63.0f);
    const float step = d * scf;
    const float bias = dmin * mnf;
    const float xs[4] = {x0, x1, x2, x3};
    uint32_t qpack = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float qv = 0.0f;
        if (step > 0.0f) qv = fminf(fmaxf(rintf((xs[i] + bias) / step), 0.0f), 15.0f);
        qpack |= ((uint32_t)qv) << (8 * i);
    }
    uint8_t *out = dst + blk * kBlockBytes;
    // Element e = 4*lane + i sits in sub-block j = lane / 8.  Byte
    // qs[32*il + l] = q[64*il + l] | q[64*il + 32 + l] << 4: lanes of even
    // sub-blocks combine with the lane 8 above.
    const uint32_t upper = __shfl(qpack, (lane + 8) & 63, 64);
    const int j = lane >> 3;
    if ((j & 1) == 0) {
        const int il = j >> 1;
        *reinterpret_cast<uint32_t *>(out + 16 + 32 * il + (4 * lane - 64 * il)) =
            qpack | (upper << 4);
    }
    // Header: gather the eight (sc, m) pairs and pack them (GGML layout).
    const uint32_t scu = (uint32_t)scf, mnu = (uint32_t)mnf;
    uint32_t sc[8], mn[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        sc[s] = __shfl(scu, 8 * s, 64);
        mn[s] = __shfl(mnu, 8 * s, 64);
    }
    if (lane == 0) {
        uint32_t words[3] = {0, 0, 0};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t b0 = (sc[s] & 63u) | ((sc[s + 4] >> 4) << 6);
            const uint32_t b4 = (mn[s] & 63u) | ((mn[s + 4] >> 4) << 6);
            const uint32_t b8 = (sc[s + 4] & 0xFu) | ((mn[s + 4] & 0xFu) << 4);
            words[0] |= b0 << (8 * s);
            words[1] |= b4 << (8 * s);
            words[2] |= b8 << (8 * s);
        }
        *reinterpret_cast<u32x4 *>(out) =
            u32x4{(uint32_t)d_raw | ((uint32_t)dmin_raw << 16), words[0], words[1], words[2]};
    }
}

hipError_t launch_quantize(uint8_t *dst, const float *src, int64_t n_blocks, hipStream_t st) {
    const int64_t grid = (n_blocks + 3) / 4;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
    quantize_kernel<<<(unsigned)grid, 256, 0, st>>>(dst, src, n_blocks);
    return hipGetLastError();
}

}  // namespace rxq4
