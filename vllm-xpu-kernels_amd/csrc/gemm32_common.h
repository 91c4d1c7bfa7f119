// Helpers shared by the 32x32-MFMA grouped-GEMM kernels (128-slot x
// 256-weight-row tiles, 4 waves as 2 (slots) x 2 (weight rows)).
#pragma once

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));


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


// Round to the 16-bit output type and back.
template <bool F16>
__device__ __forceinline__ float round16(float v) {
  if constexpr (F16) return f16_to_f32(f32_to_f16(v));
  else return bf16_to_f32(f32_to_bf16(v));
}
template <bool F16>
__device__ __forceinline__ uint16_t to16(float v) {
  if constexpr (F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}

// x * sigmoid(k x) with the hardware exp2 and reciprocal (about 1 ulp each,
// far below the 16-bit rounding that follows).  Saturates cleanly: k x ->
// -inf gives x * rcp(inf) = -0, k x -> +inf gives x.
__device__ __forceinline__ float x_sigmoid(float x, float k) {
  const float e = __builtin_amdgcn_exp2f(-k * x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

// silu(g) rounded to the activation type, times u (silu_and_mul); swigluoai:
// clamp, then (u + 1) * g * sigmoid(alpha g).
template <bool F16>
__device__ __forceinline__ float glu_act(float g, float u, const GemmArgs& a) {
  if (a.act == MI355MOE_ACT_SILU) return round16<F16>(x_sigmoid(g, 1.f)) * u;
  g = g > a.limit ? a.limit : g;
  u = u > a.limit ? a.limit : (u < -a.limit ? -a.limit : u);
  return (u + 1.f) * x_sigmoid(g, a.alpha);
}

// Epilogue of a 128x256 tile.  acc[i][j][r] holds slot m = 64wm + 32j + l32
// and tile weight row wtile_row[i] + 8*(r/4) + 4*h + r%4 (GLU: tiles 0,1 are
// gate rows, 2,3 the matching up rows).  n0: first output column of the
// tile; s_drow: destination rows; s_amax: [2][128] scratch (QOUT);
// ngroup: index of the tile's 128-column scale group (QOUT); stage: LDS of at
// least 128 x (2 x 256 + 16) bytes that no wave reads any more once all waves
// arrive here (the K loop's buffers).  The output tile is transposed through
// `stage` so that every global store writes 16 contiguous bytes of one row.
template <bool kGlu, bool QOUT, bool F16>
__device__ __forceinline__ void epilogue_32x32(const GemmArgs& a, void* qs,
                                               f32x16 (&acc)[4][2], int e,
                                               int64_t n0, int wm, int wn,
                                               int l32, int h,
                                               const int* s_drow,
                                               float (*s_amax)[128],
                                               int ngroup, uint8_t* stage) {
  const int64_t N = a.N;
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  const float es = a.expert_scale ? a.expert_scale[e] : 1.f;  // recipe BF16 only
  constexpr int NO = kGlu ? 2 : 4;       // output n-tiles per wave
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns of the tile
  // tile column of (tile i, reg r)
  auto tile_col = [&](int i, int r) -> int {
    return (kGlu ? 64 * wn + 32 * i : 128 * wn + 32 * i) + 8 * (r >> 2) + 4 * h + (r & 3);
  };
  float ov[NO][2][16];
#pragma unroll
  for (int i = 0; i < NO; ++i) {
    float bg[16], bu[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bg[r] = 0.f;
      bu[r] = 0.f;
    }
    if (a.bias) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + tile_col(i, r);
        if (n < N) {
          bg[r] = ld16<F16>(a.bias[bias_base + n]);
          if constexpr (kGlu) bu[r] = ld16<F16>(a.bias[bias_base + a.up_off + n]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = round16<F16>(acc[i][j][r] * es + bg[r]);
        if constexpr (kGlu) {
          float u = round16<F16>(acc[i + 2][j][r] * es + bu[r]);
          glu_clamp(a, n0 + tile_col(i, r), v, u);
          v = round16<F16>(glu_act<F16>(v, u, a));
        }
        ov[i][j][r] = v;
      }
    }
  }

  if constexpr (QOUT) {
    // e4m3 activation with one fp32 scale per (slot, 128 columns): the two
    // waves with the same wm cover the block's 128 columns.  Columns past N
    // do not exist here (N % 128 == 0).
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
    __syncthreads();  // s_amax published; the K loop's LDS is free
    constexpr int PITCH = NOUT + 16;
    float* ds = static_cast<float*>(qs);
    const int64_t ngroups = N / 128;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 64 * wm + 32 * j + l32;
      const float am = fmaxf(s_amax[0][row], s_amax[1][row]);
      const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
      const float inv = 1.0f / sc;
      const int drow = s_drow[row];
      if (wn == 0 && h == 0 && drow >= 0) ds[static_cast<int64_t>(drow) * ngroups + ngroup] = sc;
#pragma unroll
      for (int i = 0; i < NO; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t w = e4m3x4_sat(ov[i][j][4 * g] * inv, ov[i][j][4 * g + 1] * inv,
                                        ov[i][j][4 * g + 2] * inv, ov[i][j][4 * g + 3] * inv);
          *reinterpret_cast<uint32_t*>(stage + row * PITCH + tile_col(i, 4 * g)) = w;
        }
      }
    }
    __syncthreads();
    uint8_t* dq = static_cast<uint8_t*>(a.D);
    constexpr int CPR = NOUT / 16;
    for (int idx = threadIdx.x; idx < 128 * CPR; idx += 256) {
      const int row = idx / CPR, ch = idx % CPR;
      const int drow = s_drow[row];
      if (drow < 0) continue;
      *reinterpret_cast<uint4*>(dq + static_cast<int64_t>(drow) * N + n0 + ch * 16) =
          *reinterpret_cast<const uint4*>(stage + row * PITCH + ch * 16);
    }
  } else {
    constexpr int PITCH = 2 * NOUT + 16;
    __syncthreads();  // the K loop's LDS is free
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 64 * wm + 32 * j + l32;
#pragma unroll
      for (int i = 0; i < NO; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t lo = to16<F16>(ov[i][j][4 * g]) | (uint32_t(to16<F16>(ov[i][j][4 * g + 1])) << 16);
          const uint32_t hi = to16<F16>(ov[i][j][4 * g + 2]) | (uint32_t(to16<F16>(ov[i][j][4 * g + 3])) << 16);
          *reinterpret_cast<uint2*>(stage + row * PITCH + 2 * tile_col(i, 4 * g)) = make_uint2(lo, hi);
        }
      }
    }
    __syncthreads();
    uint16_t* d = static_cast<uint16_t*>(a.D);
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(a.D) & 15) == 0;
    constexpr int CPR = 2 * NOUT / 16;
    for (int idx = threadIdx.x; idx < 128 * CPR; idx += 256) {
      const int row = idx / CPR, ch = idx % CPR;
      const int drow = s_drow[row];
      const int64_t col = n0 + ch * 8;
      if (drow < 0 || col >= N) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + row * PITCH + ch * 16);
      uint16_t* dst = d + static_cast<int64_t>(drow) * N + col;
      if (vec) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (col + k < N) dst[k] = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
      }
    }
  }
}

}  // namespace mi355
