// gfx950 MFMA wrappers (bf16 / fp16 inputs, fp32 accumulation).
//
// Operand layouts used throughout (wave64, lane l):
//   16x16x32: A lane l holds row (l % 16), k = 8*(l/16) .. +7
//             B lane l holds col (l % 16), k = 8*(l/16) .. +7
//             D lane l holds rows 4*(l/16) + i (i = 0..3), col (l % 16)
//   32x32x16: A lane l holds row (l % 32), k = 8*(l/32) .. +7
//             B lane l holds col (l % 32), k = 8*(l/32) .. +7
//             D lane l holds rows 8*(i/4) + 4*(l/32) + (i%4) (i = 0..15), col (l % 32)
// A and B place the same k at the same (lane group, element) position, so the
// product is the plain dot product over k whatever order the unit sums in.
#pragma once

#include "tm_common.h"

#include <type_traits>

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void tm_static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    tm_static_for<N, I + 1>(f);
  }
}

typedef __bf16 tm_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 tm_f16x8 __attribute__((ext_vector_type(8)));
typedef float tm_f32x4 __attribute__((ext_vector_type(4)));
typedef float tm_f32x16 __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ tm_f32x4 tm_mfma16x16x32(uint4 a, uint4 b, tm_f32x4 c) {
  if constexpr (DT == TM_DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(tm_bf16x8, a),
                                                   __builtin_bit_cast(tm_bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tm_f16x8, a),
                                                  __builtin_bit_cast(tm_f16x8, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ tm_f32x16 tm_mfma32x32x16(uint4 a, uint4 b, tm_f32x16 c) {
  if constexpr (DT == TM_DT_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(tm_bf16x8, a),
                                                   __builtin_bit_cast(tm_bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(tm_f16x8, a),
                                                  __builtin_bit_cast(tm_f16x8, b), c, 0, 0, 0);
  }
}
