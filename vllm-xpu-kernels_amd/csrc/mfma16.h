// 16-bit operand helpers of the GEMM kernels.  A call's 16-bit type is bf16
// or fp16 (F16): it is the type of the activations and weights of the 16-bit
// recipe (MFMA operands), the type mxfp4 weights are dequantised to, and the
// type of the biases, of the rounded intermediates and of the output.
#pragma once

#include "common.h"
#include "moe_gemm.h"

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

// 8 fp8 codes (byte t = value t; e4m3, or e5m2 with E5M2) -> 8 16-bit
// values, exactly: every e4m3 and e5m2 value is a bf16 and an fp16 value,
// and the scale is 1 (v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8}, one 16-bit
// half of the source word per instruction).
template <bool E5M2, bool F16, bool HI>
__device__ __forceinline__ uint32_t fp8x2_to16(uint32_t v) {
  if constexpr (E5M2 && F16)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(v, 1.0f, HI));
  else if constexpr (E5M2)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(v, 1.0f, HI));
  else if constexpr (F16)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 1.0f, HI));
  else
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, HI));
}
template <bool E5M2, bool F16>
__device__ __forceinline__ uint4 fp8x8_to16(uint2 w) {
  return make_uint4(fp8x2_to16<E5M2, F16, false>(w.x), fp8x2_to16<E5M2, F16, true>(w.x),
                    fp8x2_to16<E5M2, F16, false>(w.y), fp8x2_to16<E5M2, F16, true>(w.y));
}

// 8 signed int4 values (two's-complement nibbles, value t in bits 4t..4t+3)
// -> 8 16-bit values T(v * scale), the reference's dequantisation
// (gemm_xe2.hpp:455-470: the 16-bit weight times its 16-bit group scale).
template <bool F16>
__device__ __forceinline__ uint4 int4x8_to16(uint32_t w, float sc) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = static_cast<float>(static_cast<int32_t>(w << (28 - 8 * i)) >> 28) * sc;
    const float hi = static_cast<float>(static_cast<int32_t>(w << (24 - 8 * i)) >> 28) * sc;
    o[i] = st16<F16>(lo) | (static_cast<uint32_t>(st16<F16>(hi)) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 4-bit weights (recipes MXFP4 and INT4), one 32-value K block (16 bytes) of
// weight row `wrow` of expert e at a time.  Its scale code: the e8m0 byte
// (mxfp4, [E, ldb_rows, K/32] or K-blocked) or the bits of the 16-bit group
// scale (int4, [E, ldb_rows, K/w_group] in the call's 16-bit type).
template <int RECIPE>
__device__ __forceinline__ uint32_t w4_scale_code(const GemmArgs& a, int e, int64_t wrow,
                                                  int64_t blk32, const WStride& sst) {
  if constexpr (RECIPE == MI355MOE_RECIPE_INT4) {
    // row-major [E, ldb_rows, K/group], or K-blocked [E, K/group, ldb_rows]
    const int64_t groups = a.K / a.w_group, g = (blk32 * 32) / a.w_group;
    const uint16_t* s = static_cast<const uint16_t*>(a.b_scale);
    return a.w_kblock ? s[(static_cast<int64_t>(e) * groups + g) * a.ldb_rows + wrow]
                      : s[(static_cast<int64_t>(e) * a.ldb_rows + wrow) * groups + g];
  } else {
    return static_cast<const uint8_t*>(a.b_scale)
        [static_cast<int64_t>(e) * a.ldb_rows * (a.K / 32) + wrow * sst.row + blk32 * sst.kblk];
  }
}
// 8 values of a block word under its scale code (mxfp4: code 0 -> 0, as the
// reference's kernel maps e8m0 0, gemm_xe2.hpp:411-418).
template <int RECIPE, bool F16>
__device__ __forceinline__ uint4 w4_decode8(uint32_t w, uint32_t code) {
  if constexpr (RECIPE == MI355MOE_RECIPE_INT4) {
    return int4x8_to16<F16>(w, ld16<F16>(static_cast<uint16_t>(code)));
  } else {
    return fp4x8_to16<F16>(code ? w : 0u, __uint_as_float(code << 23));
  }
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
