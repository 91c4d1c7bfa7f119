// 16-bit operand helpers of the GEMM kernels.  A call's 16-bit type is bf16
// or fp16 (F16): it is the type of the activations and weights of the 16-bit
// recipe (MFMA operands), the type mxfp4 weights are dequantised to, and the
// type of the biases, of the rounded intermediates and of the output.
#pragma once

#include "common.h"

namespace mi355 {

typedef float m16_f32x4 __attribute__((ext_vector_type(4)));
typedef float m16_f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 m16_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 m16_f16x8 __attribute__((ext_vector_type(8)));

template <bool F16>
__device__ __forceinline__ float ld16(uint16_t v) {
  if constexpr (F16) return f16_to_f32(v);
  else return bf16_to_f32(v);
}
template <bool F16>
__device__ __forceinline__ uint16_t st16(float v) {
  if constexpr (F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}
template <bool F16>
__device__ __forceinline__ float rnd16(float v) {
  return ld16<F16>(st16<F16>(v));
}

// D += A * B over 8 16-bit values per lane (16x16x32) ...
template <bool F16>
__device__ __forceinline__ m16_f32x4 mfma16_16x16x32(uint4 a, uint4 b, m16_f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(m16_f16x8, a),
                                                  __builtin_bit_cast(m16_f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(m16_bf16x8, a),
                                                   __builtin_bit_cast(m16_bf16x8, b), c, 0, 0, 0);
}
// ... and 32x32x16
template <bool F16>
__device__ __forceinline__ m16_f32x16 mfma16_32x32x16(uint4 a, uint4 b, m16_f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(m16_f16x8, a),
                                                  __builtin_bit_cast(m16_f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(m16_bf16x8, a),
                                                   __builtin_bit_cast(m16_bf16x8, b), c, 0, 0, 0);
}

// 8 e2m1 codes (one 32-bit word, value t in bits 4t..4t+3) -> 8 16-bit
// values scaled by the fp32 scale (v_cvt_scalef32_pk_{bf16,f16}_fp4).
template <bool F16>
__device__ __forceinline__ uint4 fp4x8_to16(uint32_t w, float sc) {
  uint4 r;
  if constexpr (F16) {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 0));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 1));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 2));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 3));
  } else {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
  }
  return r;
}

// GLU activations of the w13 epilogue: SiLU-and-mul rounds silu(g) to the
// 16-bit type before the multiply; swigluoai clamps, then (u + 1) g
// sigmoid(alpha g) in fp32.
template <bool F16>
__device__ __forceinline__ float glu16(float g, float u, int act, float alpha, float limit) {
  if (act == MI355MOE_ACT_SILU) return rnd16<F16>(g / (1.f + expf(-g))) * u;
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  return (u + 1.f) * (g * (1.f / (1.f + expf(-g * alpha))));
}

}  // namespace mi355
