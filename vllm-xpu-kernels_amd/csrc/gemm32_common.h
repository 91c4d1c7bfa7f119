// Helpers shared by the 32x32-MFMA grouped-GEMM kernels (128-slot x
// 256-weight-row tiles, 4 waves as 2 (slots) x 2 (weight rows)).
#pragma once

#include "moe_gemm.h"

namespace mi355 {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma32_bf16(uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// e4m3 x e4m3, 32x32x64, unit e8m0 scales.
__device__ __forceinline__ f32x16 mfma32_fp8(uint4 a0, uint4 a1, uint4 b0,
                                             uint4 b1, f32x16 c) {
  i32x8_t a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
               (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  i32x8_t b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
               (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127,
                                                         0, 127);
}

__device__ __forceinline__ uint4 fp4x8_bf16(uint32_t w, float sc) {
  uint4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
  return r;
}

__device__ __forceinline__ float bround(float v, bool f16) {
  return f16 ? f16_to_f32(f32_to_f16(v)) : bf16_to_f32(f32_to_bf16(v));
}

__device__ __forceinline__ float glu_act(float g, float u, const GemmArgs& a) {
  if (a.act == MI355MOE_ACT_SILU) {
    float s = bf16_to_f32(f32_to_bf16(g / (1.f + expf(-g))));
    return s * u;
  }
  g = g > a.limit ? a.limit : g;
  u = u > a.limit ? a.limit : (u < -a.limit ? -a.limit : u);
  return (u + 1.f) * (g * (1.f / (1.f + expf(-g * a.alpha))));
}

// Epilogue of a 128x256 tile.  acc[i][j][r] holds slot m = 64wm + 32j + l32
// and tile weight row wtile_row[i] + 8*(r/4) + 4*h + r%4 (GLU: tiles 0,1 are
// gate rows, 2,3 the matching up rows).  n0: first output column of the
// tile; s_drow: destination rows; s_amax: [2][128] scratch (QOUT);
// ngroup: index of the tile's 128-column scale group (QOUT).
template <bool kGlu, bool QOUT>
__device__ __forceinline__ void epilogue_32x32(const GemmArgs& a, void* qs,
                                               f32x16 (&acc)[4][2], int e,
                                               int64_t n0, int wm, int wn,
                                               int l32, int h,
                                               const int* s_drow,
                                               float (*s_amax)[128],
                                               int ngroup) {
  const int64_t N = a.N;
  const bool f16 = a.out_f16 != 0;
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  constexpr int NO = kGlu ? 2 : 4;  // output n-tiles per wave
  // output column of (tile i, reg r)
  auto out_col = [&](int i, int r) -> int64_t {
    const int tr = (kGlu ? 64 * wn + 32 * i : 128 * wn + 32 * i) + 8 * (r >> 2) + 4 * h + (r & 3);
    return n0 + tr;
  };
  float ov[NO][2][16];
#pragma unroll
  for (int i = 0; i < NO; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = out_col(i, r);
        const bool nok = n < N;
        float v = acc[i][j][r];
        if (a.bias && nok) v += bf16_to_f32(a.bias[bias_base + n]);
        v = bround(v, f16);
        if constexpr (kGlu) {
          float u = acc[i + 2][j][r];
          if (a.bias && nok) u += bf16_to_f32(a.bias[bias_base + a.up_off + n]);
          u = bround(u, f16);
          if (a.clamp_limit > 0.f) {
            v = fminf(v, a.clamp_limit);
            u = fminf(fmaxf(u, -a.clamp_limit), a.clamp_limit);
          }
          v = bround(glu_act(v, u, a), f16);
        }
        ov[i][j][r] = nok ? v : 0.f;
      }
    }
  }

  if constexpr (QOUT) {
    // e4m3 activation with one fp32 scale per (slot, 128 columns): the two
    // waves with the same wm cover the block's 128 columns.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float m = 1e-10f;
#pragma unroll
      for (int i = 0; i < NO; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(ov[i][j][r]));
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      if (h == 0) s_amax[wn][64 * wm + 32 * j + l32] = m;
    }
    __syncthreads();
    uint8_t* dq = static_cast<uint8_t*>(a.D);
    float* ds = static_cast<float*>(qs);
    const int64_t ngroups = N / 128;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 64 * wm + 32 * j + l32;
      const int drow = s_drow[row];
      if (drow < 0) continue;
      const float am = fmaxf(s_amax[0][row], s_amax[1][row]);
      const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
      const float inv = 1.0f / sc;
      if (wn == 0 && h == 0) ds[static_cast<int64_t>(drow) * ngroups + ngroup] = sc;
#pragma unroll
      for (int i = 0; i < NO; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t w = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = fminf(fmaxf(ov[i][j][4 * g + r] * inv, -448.f), 448.f);
            w |= f32_to_e4m3(x) << (8 * r);
          }
          *reinterpret_cast<uint32_t*>(dq + static_cast<int64_t>(drow) * N + out_col(i, 4 * g)) = w;
        }
      }
    }
  } else {
    uint16_t* d = static_cast<uint16_t*>(a.D);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int drow = s_drow[64 * wm + 32 * j + l32];
      if (drow < 0) continue;
#pragma unroll
      for (int i = 0; i < NO; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t n = out_col(i, 4 * g);
          uint16_t hv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            hv[r] = f16 ? f32_to_f16(ov[i][j][4 * g + r]) : f32_to_bf16(ov[i][j][4 * g + r]);
          uint16_t* dst = d + static_cast<int64_t>(drow) * N + n;
          if (n + 3 < N && (N & 3) == 0) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(
                hv[0] | (uint32_t(hv[1]) << 16), hv[2] | (uint32_t(hv[3]) << 16));
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) dst[r] = hv[r];
          }
        }
      }
    }
  }
}

}  // namespace mi355
