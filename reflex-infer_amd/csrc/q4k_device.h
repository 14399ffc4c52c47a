// q4k_device.h -- Q4_K block format and device helpers shared by the gfx950
// kernels.
//
// GGUF Q4_K super-block (reference q4_gemm.cu:147-154): 256 weights in 144
// bytes = 9 aligned 16-byte chunks.
//   bytes  0..1   d     fp16 super-block scale
//   bytes  2..3   dmin  fp16 super-block min
//   bytes  4..15  scales[12]: eight 6-bit (sc, m) pairs, GGML packing
//                 (unpacked by get_scale_min_k4, q4_gemm.cu:192-202)
//   bytes 16..143 qs[128]: byte 32*il + l holds element 64*il + l in its low
//                 nibble and element 64*il + 32 + l in its high nibble
// Element value: w = d*sc[s]*q - dmin*m[s], s = sub-block (32 elements).
// d*sc and (d*sc)*q and dmin*m are exact in fp32, so w has exactly one
// rounding whatever the evaluation order or FMA contraction.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rxq4 {

constexpr int kQK = 256;
constexpr int kBlockBytes = 144;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32, RNE
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __builtin_bit_cast(float, bits16 << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);  // RNE
}

__device__ __forceinline__ half2_t as_half2(uint32_t v) {
    return __builtin_bit_cast(half2_t, v);
}

// 16-byte global load through the vector memory path.
__device__ __forceinline__ u32x4 load16(const void *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}

// 16-byte store marked nontemporal, for outputs no later access in the
// kernel reads (the embedding gathers: 4096 fp16 rows of 2048 in 5.65 us
// against 6.56 us with ordinary stores).
__device__ __forceinline__ void store16_nt(void *p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p));
}

// The (sc, m) pairs of sub-blocks 2*il and 2*il+1 from the three scale dwords
// s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].  Returns
// sc_lo | sc_hi << 8 in *sc and m_lo | m_hi << 8 in *mn.  Same values as
// get_scale_min_k4(2*il) / get_scale_min_k4(2*il+1).
__device__ __forceinline__ void scale_pair(uint32_t s0, uint32_t s1, uint32_t s2, int il,
                                           uint32_t *sc, uint32_t *mn) {
    const int sh = (il & 1) << 4;
    const uint32_t a = s0 >> sh, b = s1 >> sh, c = s2 >> sh;
    if (il < 2) {
        *sc = a & 0x3F3Fu;
        *mn = b & 0x3F3Fu;
    } else {
        *sc = (c & 0x0F0Fu) | ((a >> 2) & 0x3030u);
        *mn = ((c >> 4) & 0x0F0Fu) | ((b >> 2) & 0x3030u);
    }
}

// The (sc, m) pair of one sub-block j in [0, 8).
__device__ __forceinline__ void scale_one(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                          uint32_t *sc, uint32_t *mn) {
    uint32_t p, q;
    scale_pair(s0, s1, s2, j >> 1, &p, &q);
    const int sh = (j & 1) << 3;
    *sc = (p >> sh) & 0xFFu;
    *mn = (q >> sh) & 0xFFu;
}

// v_alignbyte: bytes r.. (r < 4) of the 8-byte value hi:lo.
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, int r) {
    return __builtin_amdgcn_alignbyte(hi, lo, (uint32_t)r);
}

// Sum over the lanes of aligned groups of `width` lanes (power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Combine each lane's x with x of lane ^ 16 (ROW = 16) or lane ^ 32 (ROW =
// 32) on the VALU: v_permlane{16,32}_swap on two copies of x leaves, in
// every lane, its own value in one result and its partner's in the other
// (which one depends on the lane), so max / sum of the two results equal
// fmaxf / + of x and the partner's x (both commutative) with no LDS
// instruction (__shfl_xor is a ds_bpermute, queued behind LDS traffic).
template <int ROW>
__device__ __forceinline__ void swap_rows(float x, float &a, float &b) {
    static_assert(ROW == 16 || ROW == 32, "row swaps of 16 or 32 lanes");
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    uint32_t r0, r1;
    if constexpr (ROW == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        r0 = r[0];
        r1 = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        r0 = r[0];
        r1 = r[1];
    }
    a = __builtin_bit_cast(float, r0);
    b = __builtin_bit_cast(float, r1);
}

template <int ROW>
__device__ __forceinline__ float max_xor_rows(float x) {
    float a, b;
    swap_rows<ROW>(x, a, b);
    return fmaxf(a, b);
}

template <int ROW>
__device__ __forceinline__ float sum_xor_rows(float x) {
    float a, b;
    swap_rows<ROW>(x, a, b);
    return a + b;
}

// v + v[lane ^ q] for q = W/2, W/4, ..., 1 (the __shfl_xor butterfly over
// aligned groups of W = 32 or 64 lanes; every lane ends with its group's
// sum), on the VALU: the xor-32 / xor-16 steps by row swaps, then DPP
// rotations within 16-lane rows.  After the steps above q, lanes whose
// indices differ only in bits above q's hold equal values, and row_ror:q
// reaches lane (l + q) mod 16, which differs from l ^ q only in those
// bits, so every step adds the same two values, in the same order, as the
// shuffle butterfly: the results are bit-identical.
template <int CTRL>
__device__ __forceinline__ float dpp_row_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
    return v + __builtin_bit_cast(float, moved);
}

template <int W>
__device__ __forceinline__ float butterfly_sum(float v) {
    static_assert(W == 32 || W == 64, "groups of 32 or 64 lanes");
    if constexpr (W == 64) v = sum_xor_rows<32>(v);
    v = sum_xor_rows<16>(v);
    v = dpp_row_add<0x128>(v);  // row_ror:8
    v = dpp_row_add<0x124>(v);  // row_ror:4
    v = dpp_row_add<0x122>(v);  // row_ror:2
    v = dpp_row_add<0x121>(v);  // row_ror:1
    return v;
}

// The maximum over aligned groups of W = 32 or 64 lanes (exact in any
// order), every lane getting it: row swaps, then DPP rotations.
template <int CTRL>
__device__ __forceinline__ float dpp_row_max(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
    return fmaxf(v, __builtin_bit_cast(float, moved));
}

template <int W>
__device__ __forceinline__ float butterfly_max(float v) {
    static_assert(W == 32 || W == 64, "groups of 32 or 64 lanes");
    if constexpr (W == 64) v = max_xor_rows<32>(v);
    v = max_xor_rows<16>(v);
    v = dpp_row_max<0x128>(v);
    v = dpp_row_max<0x124>(v);
    v = dpp_row_max<0x122>(v);
    v = dpp_row_max<0x121>(v);
    return v;
}

// Workgroup barrier without the fence of __syncthreads (which waits for all
// outstanding vector memory operations); callers wait for what they need.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Buffer resource over `bytes` bytes at `base` (raw buffer, no swizzle);
// loads past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes,
                                             0x00020000);
}

// 16 bytes per lane from rsrc + voffset into registers (zeros past the end).
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int voffset) {
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, 0, 0);
}

// 4 and 8 bytes per lane from rsrc + voffset (dword-aligned voffset).
__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t rsrc, int voffset) {
    return __builtin_amdgcn_raw_buffer_load_b32(rsrc, voffset, 0, 0);
}

__device__ __forceinline__ u32x2 buffer_load8(__amdgpu_buffer_rsrc_t rsrc, int voffset) {
    return __builtin_amdgcn_raw_buffer_load_b64(rsrc, voffset, 0, 0);
}

// 16 bytes per lane, global (rsrc + voffset + soffset) -> LDS at
// lds + 16 * lane; soffset is wave-uniform.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds,
                                                int voffset, int soffset = 0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (void __attribute__((address_space(3))) *)lds, 16, voffset, soffset, 0, 0);
}

// buffer_to_lds16 marked nontemporal (cache policy 2 = nt), for data read
// once: a stream whose every load instruction covers whole 128-byte lines.
__device__ __forceinline__ void buffer_to_lds16_nt(__amdgpu_buffer_rsrc_t rsrc, void *lds,
                                                   int voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (void __attribute__((address_space(3))) *)lds, 16, voffset, 0, 0, 2);
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt untouched).
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

// s_waitcnt vmcnt(N) (lgkmcnt and expcnt untouched).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace rxq4
