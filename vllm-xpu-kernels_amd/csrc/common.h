// Shared device/host helpers for the MI355X (gfx950) fused-MoE library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/mi355moe.h"

namespace mi355 {

// ---------------------------------------------------------------------------
// Error plumbing: every C-ABI entry point returns 0 or a negative code and
// leaves a message in a thread-local buffer (mi355moe_last_error()).
// ---------------------------------------------------------------------------
int set_error(int code, const std::string& msg);

#define MI_CHECK(cond, code, msg)                                  \
  do {                                                             \
    if (!(cond)) return ::mi355::set_error((code), (msg));         \
  } while (0)

#define MI_ARG(cond, msg) MI_CHECK(cond, MI355MOE_ERR_INVALID, msg)

#define MI_HIP(expr)                                                         \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess)                                                    \
      return ::mi355::set_error(MI355MOE_ERR_HIP,                            \
                                std::string("HIP error: ") +                 \
                                    hipGetErrorString(_e) + " at " #expr);   \
  } while (0)

#define MI_LAUNCH_CHECK()                                                    \
  do {                                                                       \
    hipError_t _e = hipGetLastError();                                       \
    if (_e != hipSuccess)                                                    \
      return ::mi355::set_error(MI355MOE_ERR_HIP,                            \
                                std::string("kernel launch failed: ") +      \
                                    hipGetErrorString(_e));                  \
  } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16/fp16 are carried as raw 16-bit words; fp32->bf16
// uses the hardware RNE convert (v_cvt_pk_bf16_f32 on gfx950).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, v);
}

// Element-type traits used by templated kernels: load as float, store from
// float with one rounding.
struct F32 {
  using T = float;
  static __device__ __forceinline__ float ld(float v) { return v; }
  static __device__ __forceinline__ float st(float v) { return v; }
};
struct BF16 {
  using T = uint16_t;
  static __device__ __forceinline__ float ld(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t st(float v) { return f32_to_bf16(v); }
};
struct F16 {
  using T = uint16_t;
  static __device__ __forceinline__ float ld(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t st(float v) { return f32_to_f16(v); }
};

// GELU in fp32, textbook forms: exact (erf) and the tanh approximation
// sqrt(2/pi) (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_erf(float f) {
  return f * 0.5f * (1.0f + erff(f * 0.70710678118654752f));
}
__device__ __forceinline__ float gelu_tanh(float f) {
  const float inner = 0.7978845608028654f * (f + 0.044715f * (f * f * f));
  return 0.5f * f * (1.0f + tanhf(inner));
}

// OCP e4m3fn decode (bias 7, no infinities, 0x7f/0xff NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xFu;
  uint32_t m = b & 0x7u;
  float v;
  if (e == 0) {
    v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  if ((b & 0x7Fu) == 0x7Fu) v = __uint_as_float(0x7FC00000u);
  return __uint_as_float(__float_as_uint(v) | s);
}

// fp32 -> OCP e4m3fn, round to nearest even, for |x| <= 448 (callers clamp
// first, as the reference quantisers do).  Subnormals (|x| < 2^-6) are on the
// 2^-9 grid.
__device__ __forceinline__ uint32_t f32_to_e4m3_sw(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;  // NaN
  uint32_t r;
  if (a < 0x3C800000u) {                      // |x| < 2^-6: subnormal range
    float f = __uint_as_float(a) * 512.0f;    // exact scaling to units of 2^-9
    // round half to even on the integer grid 0..8
    float fl = __builtin_floorf(f);
    float d = f - fl;
    uint32_t q = static_cast<uint32_t>(fl);
    if (d > 0.5f || (d == 0.5f && (q & 1u))) q += 1u;
    r = q;                                     // q == 8 -> 0x08 = 2^-6 (normal)
  } else {
    // normal: keep 3 mantissa bits, RNE on the dropped 20 bits
    uint32_t lsb = (a >> 20) & 1u;
    uint32_t rounded = a + 0x7FFFFu + lsb;
    uint32_t e = (rounded >> 23) - 120u;
    uint32_t m = (rounded >> 20) & 0x7u;
    r = (e << 3) | m;
    if (r > 0x7Eu) r = 0x7Eu;                  // saturate at 448
  }
  return sign | r;
}

// f32 -> e4m3 code.  |x| <= 448 (every caller clamps to that range first):
// the hardware convert (v_cvt_pk_fp8_f32, round to nearest even), which gives
// the same code as the rules above for every float in that range, checked
// exhaustively on gfx950; NaN and larger magnitudes follow the rules above.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  if (!(__builtin_fabsf(x) <= 448.0f)) return f32_to_e4m3_sw(x);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false)) & 0xFFu;
}

// e4m3 bytes 0..3 of v0..v3, each clamped to [-448, 448] first (fmaxf /
// fminf also take NaN into that range), two values per hardware convert:
// byte for byte the codes f32_to_e4m3 gives for the clamped values, without
// its out-of-range branch.
__device__ __forceinline__ uint32_t e4m3x4_sat(float v0, float v1, float v2, float v3) {
  auto c = [](float x) { return fminf(fmaxf(x, -448.f), 448.f); };
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(c(v0), c(v1), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c(v2), c(v3), w, true);
  return static_cast<uint32_t>(w);
}

// ceil(log2(x)) of a positive finite float, exactly from its bits (a
// mantissa above the power of two rounds the exponent up), and 2^e.
__device__ __forceinline__ int ceil_log2(float x) {
  uint32_t u = __float_as_uint(x);
  int e = static_cast<int>((u >> 23) & 0xFF) - 127;
  return (u & 0x7FFFFFu) ? e + 1 : e;
}
__device__ __forceinline__ float pow2i(int e) {
  return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}
// e2m1 code (sign in bit 3) of x in [-6, 6], magnitude by strict midpoints
// (ties round down in magnitude), the rounding of the reference's mxfp4
// quantiser (csrc/quantization/fp4/mxfp4_quant.h:17-25).
__device__ __forceinline__ uint32_t fp4_code(float x) {
  float a = fabsf(x);
  uint32_t c = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) +
               (a > 2.5f) + (a > 3.5f) + (a > 5.0f);
  return c | (x < 0.f ? 0x8u : 0u);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// a and b rounded to the 16-bit type (nearest even, one conversion for
// both) and packed, a in the low half
template <bool F16>
__device__ __forceinline__ uint32_t pack16x2(float a, float b) {
  if constexpr (F16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// the two 16-bit values of a packed pair as floats (a the low half)
template <bool F16>
__device__ __forceinline__ void unpack16x2(uint32_t p, float& a, float& b) {
  if constexpr (F16) {
    a = f16_to_f32(static_cast<uint16_t>(p));
    b = f16_to_f32(static_cast<uint16_t>(p >> 16));
  } else {
    a = __uint_as_float(p << 16);
    b = __uint_as_float(p & 0xffff0000u);
  }
}
// each of v[0..N-1] rounded to the 16-bit type (N even), two values per
// conversion
template <bool F16, int N>
__device__ __forceinline__ void round16xn(float (&v)[N]) {
  static_assert(N % 2 == 0, "pairs");
#pragma unroll
  for (int i = 0; i < N; i += 2) unpack16x2<F16>(pack16x2<F16>(v[i], v[i + 1]), v[i], v[i + 1]);
}
// fp4_code's rounding from the hardware conversion (round to nearest even),
// for values that are 16-bit floats (at most 11 significant bits) times a
// power of two s: the operands are multiplied by sn = s (1 - 2^-12) (exact:
// 11 + 12 bits), which moves a value that lies on one of fp4_code's
// midpoints just below it (the tie then rounds down in magnitude, as
// fp4_code's strict comparisons do) and keeps every other value on its side
// of every midpoint (its distance to one is more than 2^-11 of itself);
// adding +0 gives -0 code 0, as in fp4_code, and the clamp to [-6, 6] is
// fp4_code's.  fp4x4_code16: the codes of x0 .. x3 in bits 0-15, x0 in the
// low nibble.
__device__ __forceinline__ float fp4_prescale(float s) { return s * (1.0f - 1.0f / 4096.0f); }
__device__ __forceinline__ float fp4_pre(float x, float sn) {
  return fminf(fmaxf(__builtin_fmaf(x, sn, 0.0f), -6.0f), 6.0f);
}
template <int BYTE>
__device__ __forceinline__ uint32_t fp4x2_code16(uint32_t old, float x0, float x1, float sn) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, fp4_pre(x0, sn), fp4_pre(x1, sn), 1.0f,
                                                  BYTE);
}
__device__ __forceinline__ uint32_t fp4x4_code16(float x0, float x1, float x2, float x3,
                                                 float sn) {
  return fp4x2_code16<1>(fp4x2_code16<0>(0u, x0, x1, sn), x2, x3, sn) & 0xffffu;
}

// Maximum of a non-negative float over lanes l, l ^ 16, l ^ 32, l ^ 48, in every
// one of them: the row-pair and half-wave swaps of gfx950 (VALU, no LDS
// round trip), each called with both operands the same register so either
// result holds the partner rows; non-negative floats order as their bits.
__device__ __forceinline__ float max_over_rows(float m) {
  uint32_t u = __float_as_uint(m);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  u = r16[0] > r16[1] ? r16[0] : r16[1];
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  u = r32[0] > r32[1] ? r32[0] : r32[1];
  return __uint_as_float(u);
}
// Maximum over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15), in every
// lane of the row: quad lane swaps (xor 1, xor 2), then the half-row and row
// mirrors, each pairing a lane with one that holds the other half's
// maximum.  All lanes of the row must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
}

// e4m3 quantisation with one fp32 scale per 1 x 128 block, chunk c of 8
// values (16 lanes per block, consecutive and aligned): amax from 1e-10,
// scale = max(amax / 448, 1 / (448 * 512)), code = e4m3(clamp(v / scale))
// with the division done as v * (1 / scale) -- the arithmetic of
// per_token_group_fp8_quant (group 128, eps 1e-10, fp8_max 448, no ue8m0).
// Chunks >= `chunks` are inactive but take part in the block's shuffles;
// all 64 lanes must be active.
// fp8_quant_regs takes the chunk's 8 values already loaded (u).
template <bool F16>
__device__ __forceinline__ void fp8_quant_regs(const uint4 u, uint8_t* __restrict__ q,
                                               float* __restrict__ s, int64_t c,
                                               int64_t chunks) {
  const bool active = c < chunks;
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = static_cast<uint16_t>(w[i] & 0xFFFFu), hi = static_cast<uint16_t>(w[i] >> 16);
    v[2 * i] = F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
    v[2 * i + 1] = F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
  }
  float amax = 1e-10f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = row16_max(amax);
  const float ys = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
  if (!active) return;
  if ((c & 15) == 0) s[c >> 4] = ys;
  const float inv = 1.0f / ys;
  const uint32_t lo = e4m3x4_sat(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
  const uint32_t hi = e4m3x4_sat(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
  *reinterpret_cast<uint2*>(q + c * 8) = make_uint2(lo, hi);
}
template <bool F16>
__device__ __forceinline__ void fp8_quant_block8(const uint16_t* __restrict__ x,
                                                 uint8_t* __restrict__ q,
                                                 float* __restrict__ s, int64_t c,
                                                 int64_t chunks) {
  const uint4 u = *reinterpret_cast<const uint4*>(x + (c < chunks ? c : 0) * 8);
  fp8_quant_regs<F16>(u, q, s, c, chunks);
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) reductions via cross-lane shuffles.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace mi355
