// Bandwidth-bound helpers of the MoE path: activations (silu_and_mul,
// swigluoai_and_mul), per-token-group fp8 / mxfp4 activation quantisers and
// the top-k reductions (moe_sum, moe_gather).  Every kernel moves 16 bytes
// per lane per access where the row length allows it.
#include "common.h"

namespace mi355 {
namespace {

// ----------------------------------------------------------------- helpers
template <typename E>
struct Vec8 {  // 8 elements of a 16-bit type in one uint4
  static __device__ __forceinline__ void load(const uint16_t* p, float* f) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = E::ld(static_cast<uint16_t>(w[i] & 0xFFFFu));
      f[2 * i + 1] = E::ld(static_cast<uint16_t>(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(E::st(f[2 * i])) |
             (static_cast<uint32_t>(E::st(f[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};

// 8 consecutive elements from index i (a multiple of 8): 16-byte loads when
// VEC (the base pointer is 16-byte aligned), element loads otherwise.
template <typename E, bool VEC>
__device__ __forceinline__ void load8(const void* p, int64_t i, float* f) {
  if constexpr (VEC && sizeof(typename E::T) == 2) {
    Vec8<E>::load(static_cast<const uint16_t*>(p) + i, f);
  } else if constexpr (VEC) {
    const uint4* q = reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i);
    const uint4 a = q[0], b = q[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = __uint_as_float(w[k]);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = E::ld(static_cast<const typename E::T*>(p)[i + k]);
  }
}

// Quantised outputs are written once and read by a later kernel:
// non-temporal stores.
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_nt(uint8_t* p, uint32_t lo, uint32_t hi) {
  nt_u32x2 v = {lo, hi};
  __builtin_nontemporal_store(v, reinterpret_cast<nt_u32x2*>(p));
}
__device__ __forceinline__ void store_nt(uint8_t* p, uint32_t w) {
  __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(p));
}

template <typename E>
__device__ __forceinline__ float ldx(const void* p, int64_t i) {
  return E::ld(static_cast<const typename E::T*>(p)[i]);
}
template <typename E>
__device__ __forceinline__ void stx(void* p, int64_t i, float v) {
  static_cast<typename E::T*>(p)[i] = E::st(v);
}

// ------------------------------------------------------------- activations
template <typename E>
__device__ __forceinline__ float silu_mul(float g, float u) {
  // reference rounds silu(g) to the element type before the multiply
  float s = E::ld(E::st(g / (1.f + expf(-g))));
  return s * u;
}
__device__ __forceinline__ float swigluoai(float g, float u, float alpha,
                                           float limit) {
  g = g > limit ? limit : g;
  u = u > limit ? limit : (u < -limit ? -limit : u);
  float glu = g * (1.f / (1.f + expf(-g * alpha)));
  return (u + 1.f) * glu;
}

template <typename E>
__global__ __launch_bounds__(256) void silu_and_mul_kernel(
    void* __restrict__ out, const void* __restrict__ in, int64_t rows,
    int64_t d) {
  const int64_t r = blockIdx.y;
  const typename E::T* x = static_cast<const typename E::T*>(in) + r * 2 * d;
  typename E::T* y = static_cast<typename E::T*>(out) + r * d;
  if constexpr (sizeof(typename E::T) == 2) {
    if ((d & 7) == 0) {
      for (int64_t c = (blockIdx.x * 256 + threadIdx.x) * 8; c < d;
           c += static_cast<int64_t>(gridDim.x) * 256 * 8) {
        float g[8], u[8], o[8];
        Vec8<E>::load(x + c, g);
        Vec8<E>::load(x + d + c, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = silu_mul<E>(g[i], u[i]);
        Vec8<E>::store(y + c, o);
      }
      return;
    }
  }
  for (int64_t c = blockIdx.x * 256 + threadIdx.x; c < d;
       c += static_cast<int64_t>(gridDim.x) * 256)
    y[c] = E::st(silu_mul<E>(E::ld(x[c]), E::ld(x[d + c])));
}

template <typename E>
__global__ __launch_bounds__(256) void swigluoai_kernel(
    void* __restrict__ out, const void* __restrict__ in, int64_t rows,
    int64_t d, float alpha, float limit) {
  const int64_t r = blockIdx.y;
  const typename E::T* x = static_cast<const typename E::T*>(in) + r * 2 * d;
  typename E::T* y = static_cast<typename E::T*>(out) + r * d;
  for (int64_t c = blockIdx.x * 256 + threadIdx.x; c < d;
       c += static_cast<int64_t>(gridDim.x) * 256)
    y[c] = E::st(swigluoai(E::ld(x[2 * c]), E::ld(x[2 * c + 1]), alpha, limit));
}

// Gated activations other than SiLU (gelu_erf, gelu_tanh: common.h).
enum GluAct { GLU_GELU = 0, GLU_GELU_TANH = 1, GLU_SWIGLUSTEP = 2 };
// gate g, up u -> output before the final rounding to E: gelu forms round
// act(g) to E first (the activation returns the element type), swiglustep
// stays in fp32.
template <typename E, int ACT>
__device__ __forceinline__ float glu_op(float g, float u, float limit) {
  if constexpr (ACT == GLU_GELU) {
    return E::ld(E::st(gelu_erf(g))) * u;
  } else if constexpr (ACT == GLU_GELU_TANH) {
    return E::ld(E::st(gelu_tanh(g))) * u;
  } else {
    const float sg = fminf(g / (1.f + expf(-g)), limit);
    return sg * fminf(fmaxf(u, -limit), limit);
  }
}

template <typename E, int ACT>
__global__ __launch_bounds__(256) void glu_act_kernel(
    void* __restrict__ out, const void* __restrict__ in, int64_t rows, int64_t d,
    float limit) {
  const int64_t r = blockIdx.y;
  const typename E::T* x = static_cast<const typename E::T*>(in) + r * 2 * d;
  typename E::T* y = static_cast<typename E::T*>(out) + r * d;
  if constexpr (sizeof(typename E::T) == 2) {
    if ((d & 7) == 0) {
      for (int64_t c = (blockIdx.x * 256 + threadIdx.x) * 8; c < d;
           c += static_cast<int64_t>(gridDim.x) * 256 * 8) {
        float g[8], u[8], o[8];
        Vec8<E>::load(x + c, g);
        Vec8<E>::load(x + d + c, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = glu_op<E, ACT>(g[i], u[i], limit);
        Vec8<E>::store(y + c, o);
      }
      return;
    }
  }
  for (int64_t c = blockIdx.x * 256 + threadIdx.x; c < d;
       c += static_cast<int64_t>(gridDim.x) * 256)
    y[c] = E::st(glu_op<E, ACT>(E::ld(x[c]), E::ld(x[d + c]), limit));
}

template <typename E>
__global__ __launch_bounds__(256) void relu2_kernel(void* __restrict__ out,
                                                    const void* __restrict__ in,
                                                    int64_t n) {
  const typename E::T* x = static_cast<const typename E::T*>(in);
  typename E::T* y = static_cast<typename E::T*>(out);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const float r = fmaxf(E::ld(x[i]), 0.f);
    y[i] = E::st(r * r);
  }
}

// ----------------------------------------------------------- quantisation
// One group of G elements is owned by G/8 consecutive lanes (8 elements per
// lane); requires G % 8 == 0 and G/8 a power of two <= 64.
template <typename E, bool VEC>
__global__ __launch_bounds__(256) void group_fp8_quant_kernel(
    const void* __restrict__ in, uint8_t* __restrict__ q,
    float* __restrict__ s, int64_t rows, int64_t cols, int group, float eps,
    float fp8_max, int ue8m0) {
  const int lpg = group >> 3;
  const int64_t ngroups = rows * (cols / group);
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t g = gtid / lpg;
  const int sub = static_cast<int>(gtid % lpg);
  const bool active = g < ngroups;
  const int64_t base = (active ? g : 0) * group + sub * 8;
  float v[8];
  load8<E, VEC>(in, base, v);
  float amax = eps;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  if (lpg == 16) {  // a group of 128 is one DPP row of 16 lanes
    amax = row16_max(amax);
  } else {
    for (int o = lpg >> 1; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  }
  float ys = fmaxf(amax / fp8_max, 1.0f / (fp8_max * 512.0f));
  if (ue8m0) ys = pow2i(ceil_log2(fmaxf(fabsf(ys), 1e-10f)));
  if (!active) return;
  if (sub == 0) s[g] = ys;
  const float inv = 1.0f / ys;
  uint32_t lo = 0, hi = 0;
  if (fp8_max == 448.0f) {  // the e4m3 range: two values per hardware convert
    lo = e4m3x4_sat(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    hi = e4m3x4_sat(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = fminf(fmaxf(v[i] * inv, -fp8_max), fp8_max);
      uint32_t b = f32_to_e4m3(x);
      if (i < 4) lo |= b << (8 * i); else hi |= b << (8 * (i - 4));
    }
  }
  store_nt(q + base, lo, hi);
}

// mxfp4: groups of 32 owned by 4 lanes x 8 elements.
template <typename E, bool VEC>
__global__ __launch_bounds__(256) void group_mxfp4_quant_kernel(
    const void* __restrict__ in, uint8_t* __restrict__ q,
    float* __restrict__ s, int64_t rows, int64_t cols, float eps) {
  const int64_t ngroups = rows * (cols / 32);
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t g = gtid >> 2;
  const int sub = static_cast<int>(gtid & 3);
  const bool active = g < ngroups;
  const int64_t base = (active ? g : 0) * 32 + sub * 8;
  float v[8];
  load8<E, VEC>(in, base, v);
  float amax = eps;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float ys = pow2i(ceil_log2(fmaxf(fabsf(amax / 6.0f), eps)));
  if (!active) return;
  if (sub == 0) s[g] = ys;
  const float inv = 1.0f / ys;
  uint32_t packed = 0;
  if constexpr (sizeof(typename E::T) == 2) {  // 16-bit values: hardware conversion
    const float sn = fp4_prescale(inv);
    packed = fp4x2_code16<0>(packed, v[0], v[1], sn);
    packed = fp4x2_code16<1>(packed, v[2], v[3], sn);
    packed = fp4x2_code16<2>(packed, v[4], v[5], sn);
    packed = fp4x2_code16<3>(packed, v[6], v[7], sn);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = fminf(fmaxf(v[i] * inv, -6.0f), 6.0f);
      packed |= fp4_code(x) << (4 * i);
    }
  }
  store_nt(q + base / 2, packed);
}

// mxfp8 activations (the reference's _quant_mxfp8_act_xpu,
// vllm_xpu_kernels/moe_utils.py:90-104: per_token_group_fp8_quant with group
// 32, eps 1e-10, +-448 and ue8m0 scales): groups of 32 owned by 4 lanes x 8
// elements; codes e4m3 [rows, cols], each scale stored as its e8m0 byte
// (exponent + 127) at s[row * s_ld + group].
template <typename E, bool VEC>
__global__ __launch_bounds__(256) void group_mx8_quant_kernel(
    const void* __restrict__ in, uint8_t* __restrict__ q, uint8_t* __restrict__ s,
    int64_t s_ld, int64_t rows, int64_t cols) {
  const int64_t gpr = cols / 32;
  const int64_t ngroups = rows * gpr;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t g = gtid >> 2;
  const int sub = static_cast<int>(gtid & 3);
  const bool active = g < ngroups;
  const int64_t base = (active ? g : 0) * 32 + sub * 8;
  float v[8];
  load8<E, VEC>(in, base, v);
  float amax = 1e-10f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float ys0 = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
  const int ex = ceil_log2(fmaxf(fabsf(ys0), 1e-10f));
  const float ys = pow2i(ex);
  if (!active) return;
  if (sub == 0) s[(g / gpr) * s_ld + g % gpr] = static_cast<uint8_t>(ex + 127);
  const float inv = 1.0f / ys;
  const uint32_t lo = e4m3x4_sat(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
  const uint32_t hi = e4m3x4_sat(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
  store_nt(q + base, lo, hi);
}

// --------------------------------------------- fused SiLU-and-mul + quant
// f32 -> OCP e5m2 (float8_e5m2: bias 15, 2 mantissa bits), round to nearest
// even; callers clamp to +-57344 first.
__device__ __forceinline__ uint32_t f32_to_e5m2(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;   // NaN
  uint32_t r;
  if (a < 0x38800000u) {                       // |x| < 2^-14: subnormal range
    const float f = __uint_as_float(a) * 65536.0f;  // exact: units of 2^-16
    r = static_cast<uint32_t>(__builtin_rintf(f));  // 0..4 (4 = 2^-14, normal)
  } else {
    const uint32_t lsb = (a >> 21) & 1u;
    const uint32_t rounded = a + 0xFFFFFu + lsb;
    r = (((rounded >> 23) - 112u) << 2) | ((rounded >> 21) & 3u);
    if (r > 0x7Bu) r = 0x7Bu;                  // saturate at 57344
  }
  return sign | r;
}

enum QOut { Q_E4M3 = 0, Q_E5M2 = 1, Q_I8 = 2 };

// silu(g) * u in fp32 with no intermediate rounding, as both fused
// quantisers compute it.
// silu(g) * u in fp32 with the hardware exp2 and reciprocal (about 1 ulp
// each; the division of the quantisers below stays exact).  Saturates
// cleanly: g -> -inf gives g * rcp(inf) = -0.
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.f + e) * u;
}

// One lane: 8 consecutive output columns c0..c0+7 of row r (16 bytes of gate
// and of up); a group of G columns is owned by G/8 consecutive lanes, which
// exchange their maxima with xor shuffles (hidden % G == 0, so groups never
// straddle rows and the lanes of a group are aligned).
template <typename E, int QO>
__global__ __launch_bounds__(256) void silu_mul_block_quant_kernel(
    const void* __restrict__ in, uint8_t* __restrict__ q, float* __restrict__ s,
    int64_t rows, int64_t hidden, int group, int64_t sst, int64_t ssg,
    const float* __restrict__ scale_ub, int ue8m0) {
  const int lpg = group >> 3;
  const int64_t cpr = hidden >> 3;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const bool active = gtid < rows * cpr;
  const int64_t r = active ? gtid / cpr : 0;
  const int64_t c0 = (active ? gtid % cpr : 0) * 8;
  const uint16_t* x = static_cast<const uint16_t*>(in) + r * 2 * hidden;
  float g[8], u[8], v[8];
  Vec8<E>::load(x + c0, g);
  Vec8<E>::load(x + hidden + c0, u);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = silu_mul_f32(g[i], u[i]);
    amax = fmaxf(amax, fabsf(v[i]));
  }
  for (int o = 1; o < lpg; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  float ys;
  if constexpr (QO == Q_I8) {
    ys = fmaxf(amax / 127.0f, 1.1920928955078125e-7f);  // FLT_EPSILON
  } else {
    constexpr float qmax = QO == Q_E4M3 ? 448.0f : 57344.0f;
    constexpr float min_sf = 1.0f / (qmax * 512.0f);
    ys = fmaxf(amax / qmax, min_sf);
    if (scale_ub) ys = fmaxf(fminf(ys, *scale_ub), min_sf);
    if (ue8m0) ys = pow2i(ceil_log2(fmaxf(fabsf(ys), 1e-10f)));
  }
  if (!active) return;
  if ((gtid & (lpg - 1)) == 0) s[r * sst + (c0 / group) * ssg] = ys;
  uint32_t lo = 0, hi = 0;
  if constexpr (QO == Q_E4M3) {
    lo = e4m3x4_sat(v[0] / ys, v[1] / ys, v[2] / ys, v[3] / ys);
    hi = e4m3x4_sat(v[4] / ys, v[5] / ys, v[6] / ys, v[7] / ys);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t b;
      if constexpr (QO == Q_I8) {
        const float t = fminf(fmaxf(__builtin_rintf(v[i] / ys), -128.0f), 127.0f);
        b = static_cast<uint32_t>(static_cast<int32_t>(t)) & 0xFFu;
      } else {
        b = f32_to_e5m2(fminf(fmaxf(v[i] / ys, -57344.0f), 57344.0f));
      }
      if (i < 4) lo |= b << (8 * i); else hi |= b << (8 * (i - 4));
    }
  }
  store_nt(q + r * hidden + c0, lo, hi);
}

// mxfp4: groups of 32 columns, 4 lanes each.
template <typename E>
__global__ __launch_bounds__(256) void silu_mul_mxfp4_quant_kernel(
    const void* __restrict__ in, uint8_t* __restrict__ q, float* __restrict__ s,
    int64_t rows, int64_t hidden, int64_t sst, int64_t ssg, float eps) {
  const int64_t cpr = hidden >> 3;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const bool active = gtid < rows * cpr;
  const int64_t r = active ? gtid / cpr : 0;
  const int64_t c0 = (active ? gtid % cpr : 0) * 8;
  const uint16_t* x = static_cast<const uint16_t*>(in) + r * 2 * hidden;
  float g[8], u[8], v[8];
  Vec8<E>::load(x + c0, g);
  Vec8<E>::load(x + hidden + c0, u);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = silu_mul_f32(g[i], u[i]);
    amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float ys = pow2i(ceil_log2(fmaxf(fabsf(amax / 6.0f), eps)));
  if (!active) return;
  if ((gtid & 3) == 0) s[r * sst + (c0 >> 5) * ssg] = ys;
  const float inv = 1.0f / ys;
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    packed |= fp4_code(fminf(fmaxf(v[i] * inv, -6.0f), 6.0f)) << (4 * i);
  store_nt(q + (r * hidden + c0) / 2, packed);
}

// -------------------------------------------------------------- reductions
template <typename E, typename Id>
__global__ __launch_bounds__(256) void moe_sum_kernel(
    const void* __restrict__ in, void* __restrict__ out, int64_t T, int topk,
    int64_t H, const Id* __restrict__ ids, const int32_t* __restrict__ map,
    int64_t map_len) {
  const int64_t t = blockIdx.y;
  const int64_t h = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.f;
  for (int j = 0; j < topk; ++j) {
    if (ids) {
      int64_t e = static_cast<int64_t>(ids[t * topk + j]);
      if (e < 0) continue;
      if (map && (e >= map_len || map[e] < 0)) continue;
    }
    acc += ldx<E>(in, (t * topk + j) * H + h);
  }
  stx<E>(out, t * H + h, acc);
}

template <typename E>
__global__ __launch_bounds__(256) void moe_gather_kernel(
    void* __restrict__ out, const void* __restrict__ in,
    const float* __restrict__ w, const int32_t* __restrict__ perm, int64_t T,
    int topk, int64_t H) {
  const int64_t t = blockIdx.y;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (h0 >= H) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const bool vec = sizeof(typename E::T) == 2 && (H & 7) == 0;
  for (int j = 0; j < topk; ++j) {
    const int p = perm[t * topk + j];
    if (p < 0) continue;
    const float wj = w[t * topk + j];
    const int64_t row = static_cast<int64_t>(p) * H;
    if constexpr (sizeof(typename E::T) == 2) {
      if (vec) {
        float f[8];
        Vec8<E>::load(static_cast<const uint16_t*>(in) + row + h0, f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += wj * f[i];
        continue;
      }
    }
    for (int i = 0; i < 8 && h0 + i < H; ++i) acc[i] += wj * ldx<E>(in, row + h0 + i);
  }
  if constexpr (sizeof(typename E::T) == 2) {
    if (vec) {
      Vec8<E>::store(static_cast<uint16_t*>(out) + t * H + h0, acc);
      return;
    }
  }
  for (int i = 0; i < 8 && h0 + i < H; ++i) stx<E>(out, t * H + h0 + i, acc[i]);
}

}  // namespace

// mxfp8 quantisation of 16-bit x [rows, cols] (cols % 32 == 0): codes q
// [rows, cols] e4m3, scale bytes s [rows, s_ld] (group_mx8_quant_kernel).
int mx8_quant_rows(const void* x, bool f16, uint8_t* q, uint8_t* s, int64_t s_ld,
                   int64_t rows, int64_t cols, hipStream_t st) {
  MI_ARG(cols % 32 == 0 && s_ld >= cols / 32, "mxfp8 quantisation needs cols % 32 == 0");
  if (rows == 0) return MI355MOE_OK;
  const int64_t threads = rows * (cols / 32) * 4;
  dim3 grid(static_cast<unsigned>(cdiv(threads, 256)));
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  if (f16) {
    if (vec) group_mx8_quant_kernel<F16, true><<<grid, dim3(256), 0, st>>>(x, q, s, s_ld, rows, cols);
    else group_mx8_quant_kernel<F16, false><<<grid, dim3(256), 0, st>>>(x, q, s, s_ld, rows, cols);
  } else {
    if (vec) group_mx8_quant_kernel<BF16, true><<<grid, dim3(256), 0, st>>>(x, q, s, s_ld, rows, cols);
    else group_mx8_quant_kernel<BF16, false><<<grid, dim3(256), 0, st>>>(x, q, s, s_ld, rows, cols);
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace mi355

using namespace mi355;

#define MI_DISPATCH_FLOAT(dt, KERNEL_CALL, what)                                \
  switch (dt) {                                                                 \
    case MI355MOE_F32: { using E = F32; KERNEL_CALL; break; }                   \
    case MI355MOE_BF16: { using E = BF16; KERNEL_CALL; break; }                 \
    case MI355MOE_F16: { using E = F16; KERNEL_CALL; break; }                   \
    default: return set_error(MI355MOE_ERR_INVALID, what);                      \
  }

extern "C" int mi355moe_silu_and_mul(void* out, const void* in, int dt,
                                     int64_t rows, int64_t d, void* stream) {
  MI_ARG(rows >= 0 && d >= 0, "invalid shape");
  if (rows == 0 || d == 0) return MI355MOE_OK;
  MI_ARG(rows <= 0x7fffffff, "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per = (d & 7) == 0 ? d / 8 : d;
  dim3 grid(static_cast<unsigned>(std::min<int64_t>(cdiv(per, 256), 64)),
            static_cast<unsigned>(rows));
  MI_DISPATCH_FLOAT(dt, (silu_and_mul_kernel<E><<<grid, dim3(256), 0, st>>>(out, in, rows, d)),
                    "silu_and_mul: unsupported dtype")
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_swigluoai_and_mul(void* out, const void* in, int dt,
                                          int64_t rows, int64_t d, float alpha,
                                          float limit, void* stream) {
  MI_ARG(rows >= 0 && d >= 0, "invalid shape");
  if (rows == 0 || d == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(std::min<int64_t>(cdiv(d, 256), 64)),
            static_cast<unsigned>(rows));
  MI_DISPATCH_FLOAT(dt, (swigluoai_kernel<E><<<grid, dim3(256), 0, st>>>(out, in, rows, d, alpha, limit)),
                    "swigluoai_and_mul: unsupported dtype")
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

namespace {
int launch_glu(int act, void* out, const void* in, int dt, int64_t rows, int64_t d,
               float limit, void* stream, const char* what) {
  MI_ARG(rows >= 0 && d >= 0, "invalid shape");
  if (rows == 0 || d == 0) return MI355MOE_OK;
  MI_ARG(rows <= 0x7fffffff, "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per = (d & 7) == 0 ? d / 8 : d;
  dim3 grid(static_cast<unsigned>(std::min<int64_t>(cdiv(per, 256), 64)),
            static_cast<unsigned>(rows));
  switch (act) {
    case GLU_GELU:
      MI_DISPATCH_FLOAT(dt, (glu_act_kernel<E, GLU_GELU><<<grid, dim3(256), 0, st>>>(out, in, rows, d, limit)), what)
      break;
    case GLU_GELU_TANH:
      MI_DISPATCH_FLOAT(dt, (glu_act_kernel<E, GLU_GELU_TANH><<<grid, dim3(256), 0, st>>>(out, in, rows, d, limit)), what)
      break;
    default:
      MI_DISPATCH_FLOAT(dt, (glu_act_kernel<E, GLU_SWIGLUSTEP><<<grid, dim3(256), 0, st>>>(out, in, rows, d, limit)), what)
      break;
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
}  // namespace

extern "C" int mi355moe_gelu_and_mul(void* out, const void* in, int dt, int64_t rows,
                                     int64_t d, void* stream) {
  return launch_glu(GLU_GELU, out, in, dt, rows, d, 0.f, stream,
                    "gelu_and_mul: unsupported dtype");
}

extern "C" int mi355moe_gelu_tanh_and_mul(void* out, const void* in, int dt, int64_t rows,
                                          int64_t d, void* stream) {
  return launch_glu(GLU_GELU_TANH, out, in, dt, rows, d, 0.f, stream,
                    "gelu_tanh_and_mul: unsupported dtype");
}

extern "C" int mi355moe_swiglustep_and_mul(void* out, const void* in, int dt, int64_t rows,
                                           int64_t d, float limit, void* stream) {
  return launch_glu(GLU_SWIGLUSTEP, out, in, dt, rows, d, limit, stream,
                    "swiglustep_and_mul: unsupported dtype");
}

extern "C" int mi355moe_relu2_no_mul(void* out, const void* in, int dt, int64_t rows,
                                     int64_t d, void* stream) {
  MI_ARG(rows >= 0 && d >= 0, "invalid shape");
  const int64_t n = rows * d;
  if (n == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(std::min<int64_t>(cdiv(n, 256), 8192)));
  MI_DISPATCH_FLOAT(dt, (relu2_kernel<E><<<grid, dim3(256), 0, st>>>(out, in, n)),
                    "relu2_no_mul: unsupported dtype")
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_per_token_group_fp8_quant(
    const void* in, int dt, void* q, float* s, int64_t rows, int64_t cols,
    int64_t group, float eps, float /*fp8_min*/, float fp8_max, int ue8m0,
    void* stream) {
  MI_ARG(group > 0 && cols % group == 0,
         "the last dimension must be divisible by group_size");
  MI_ARG(group % 8 == 0 && group <= 512 && ((group / 8) & (group / 8 - 1)) == 0,
         "group_size must be 8 x a power of two, at most 512");
  if (rows == 0 || cols == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t threads = rows * cols / 8;
  dim3 grid(static_cast<unsigned>(cdiv(threads, 256)));
  if ((reinterpret_cast<uintptr_t>(in) & 15) == 0) {
    MI_DISPATCH_FLOAT(dt, (group_fp8_quant_kernel<E, true><<<grid, dim3(256), 0, st>>>(in, static_cast<uint8_t*>(q), s, rows, cols, (int)group, eps, fp8_max, ue8m0)),
                      "per_token_group_fp8_quant: unsupported dtype")
  } else {
    MI_DISPATCH_FLOAT(dt, (group_fp8_quant_kernel<E, false><<<grid, dim3(256), 0, st>>>(in, static_cast<uint8_t*>(q), s, rows, cols, (int)group, eps, fp8_max, ue8m0)),
                      "per_token_group_fp8_quant: unsupported dtype")
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_per_token_group_quant_mxfp4(
    const void* in, int dt, uint8_t* q, float* s, int64_t rows, int64_t cols,
    int64_t group, float eps, void* stream) {
  MI_ARG(group == 32, "group_size must be 32 for MXFP4");
  MI_ARG(cols % 32 == 0, "the last dimension must be divisible by 32");
  if (rows == 0 || cols == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t threads = rows * cols / 8;
  dim3 grid(static_cast<unsigned>(cdiv(threads, 256)));
  if ((reinterpret_cast<uintptr_t>(in) & 15) == 0) {
    MI_DISPATCH_FLOAT(dt, (group_mxfp4_quant_kernel<E, true><<<grid, dim3(256), 0, st>>>(in, q, s, rows, cols, eps)),
                      "per_token_group_quant_mxfp4: unsupported dtype")
  } else {
    MI_DISPATCH_FLOAT(dt, (group_mxfp4_quant_kernel<E, false><<<grid, dim3(256), 0, st>>>(in, q, s, rows, cols, eps)),
                      "per_token_group_quant_mxfp4: unsupported dtype")
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

#define MI_DISPATCH_HALF(dt, KERNEL_CALL, what)                                 \
  switch (dt) {                                                                 \
    case MI355MOE_BF16: { using E = BF16; KERNEL_CALL; break; }                 \
    case MI355MOE_F16: { using E = F16; KERNEL_CALL; break; }                   \
    default: return set_error(MI355MOE_ERR_INVALID, what);                      \
  }

extern "C" int mi355moe_silu_and_mul_per_block_quant(
    void* out, int out_dtype, const void* in, int in_dtype, float* scales,
    int64_t sst, int64_t ssg, int64_t rows, int64_t hidden, int64_t group,
    const float* scale_ub, int ue8m0, void* stream) {
  MI_ARG(out_dtype == MI355MOE_FP8E4M3 || out_dtype == MI355MOE_FP8E5M2 ||
             out_dtype == MI355MOE_I8,
         "out must be float8_e4m3fn, float8_e5m2, or int8");
  MI_ARG(in_dtype == MI355MOE_F16 || in_dtype == MI355MOE_BF16,
         "input must be float16 or bfloat16");
  MI_ARG(group == 32 || group == 64 || group == 128, "group_size must be 32, 64, or 128");
  MI_ARG(!scale_ub || out_dtype != MI355MOE_I8, "scale_ub is only supported for FP8 output");
  MI_ARG(rows >= 0 && hidden >= 0, "invalid shape");
  MI_ARG(hidden % group == 0, "hidden_size must be divisible by group_size");
  if (rows == 0 || hidden == 0) return MI355MOE_OK;
  MI_ARG(out && in && scales, "null pointer");
  MI_ARG((reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
         "input must be 16-byte and out 8-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(cdiv(rows * (hidden / 8), 256)));
  uint8_t* q = static_cast<uint8_t*>(out);
#define MI_BQ(QO) \
  MI_DISPATCH_HALF(in_dtype, (silu_mul_block_quant_kernel<E, QO><<<grid, dim3(256), 0, st>>>( \
      in, q, scales, rows, hidden, static_cast<int>(group), sst, ssg, scale_ub, ue8m0)), \
      "input must be float16 or bfloat16")
  if (out_dtype == MI355MOE_FP8E4M3) { MI_BQ(Q_E4M3) }
  else if (out_dtype == MI355MOE_FP8E5M2) { MI_BQ(Q_E5M2) }
  else { MI_BQ(Q_I8) }
#undef MI_BQ
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_silu_and_mul_mxfp4_quant(uint8_t* out, const void* in, int in_dtype,
                                                 float* scales, int64_t sst, int64_t ssg,
                                                 int64_t rows, int64_t hidden, int64_t group,
                                                 float eps, void* stream) {
  MI_ARG(in_dtype == MI355MOE_F16 || in_dtype == MI355MOE_BF16,
         "input must be float16 or bfloat16");
  MI_ARG(group == 32, "MXFP4 requires group_size == 32");
  MI_ARG(rows >= 0 && hidden >= 0, "invalid shape");
  MI_ARG(hidden % group == 0, "hidden_size must be divisible by group_size");
  MI_ARG(eps >= 1.17549435e-38f && eps <= 3.40282347e+38f,
         "eps must be a normal float (at least 2^-126)");
  if (rows == 0 || hidden == 0) return MI355MOE_OK;
  MI_ARG(out && in && scales, "null pointer");
  MI_ARG((reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 3) == 0,
         "input must be 16-byte and out 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(cdiv(rows * (hidden / 8), 256)));
  MI_DISPATCH_HALF(in_dtype, (silu_mul_mxfp4_quant_kernel<E><<<grid, dim3(256), 0, st>>>(
                                  in, out, scales, rows, hidden, sst, ssg, eps)),
                   "input must be float16 or bfloat16")
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_moe_sum(const void* in, void* out, int dt, int64_t T,
                                int64_t topk, int64_t H, const void* ids,
                                int ids_dtype, const int32_t* map,
                                int64_t map_len, void* stream) {
  MI_ARG(!(map && !ids), "expert_map requires topk_ids");
  MI_ARG(topk > 0, "topk must be positive");
  if (T == 0 || H == 0) return MI355MOE_OK;
  MI_ARG(T <= 0x7fffffff, "too many tokens");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(cdiv(H, 256)), static_cast<unsigned>(T));
  if (!ids || ids_dtype == MI355MOE_I32) {
    MI_DISPATCH_FLOAT(dt, (moe_sum_kernel<E, int32_t><<<grid, dim3(256), 0, st>>>(in, out, T, (int)topk, H, static_cast<const int32_t*>(ids), map, map_len)),
                      "moe_sum: unsupported dtype")
  } else if (ids_dtype == MI355MOE_I64) {
    MI_DISPATCH_FLOAT(dt, (moe_sum_kernel<E, int64_t><<<grid, dim3(256), 0, st>>>(in, out, T, (int)topk, H, static_cast<const int64_t*>(ids), map, map_len)),
                      "moe_sum: unsupported dtype")
  } else {
    return set_error(MI355MOE_ERR_INVALID, "topk_ids must be int32 or int64");
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" int mi355moe_moe_gather(void* out, const void* in, int dt,
                                   const float* w, const int32_t* perm,
                                   int64_t T, int64_t topk, int64_t H,
                                   void* stream) {
  MI_ARG(topk > 0, "topk must be positive");
  if (T == 0 || H == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(cdiv(cdiv(H, 8), 256)), static_cast<unsigned>(T));
  MI_DISPATCH_FLOAT(dt, (moe_gather_kernel<E><<<grid, dim3(256), 0, st>>>(out, in, w, perm, T, (int)topk, H)),
                    "moe_gather: unsupported dtype")
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
