// mfma_util.h -- operand packing, 16x16x32 MFMA and typed stores shared by
// the gfx950 matrix-core kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q4k_device.h"
#include "rxq4.h"

namespace rxq4 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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

}  // namespace rxq4
