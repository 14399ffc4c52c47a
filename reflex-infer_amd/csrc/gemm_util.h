// gemm_util.h -- Q4_K dequantisation into MFMA operands and the 32x32x16
// MFMA / output helpers shared by the gfx950 GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

}  // namespace rxq4
