// C-ABI entry points of the grouped GEMM and of the whole fused-MoE layer.
//
// Fused layer (one call, no host synchronisation, 4-5 launches):
//   1. stable counting sort of topk_ids into block-aligned sorted slots
//   2. (fp8block) 1x128 e4m3 quantisation of hidden_states, once per token
//      (skipped when the caller hands them over quantised: hidden_scale)
//   3. w13 grouped GEMM gathering activation rows through the sorted slots,
//      GLU epilogue (SiLU-mul / swigluoai), activation written in slot order
//      (fp8block: re-quantised to e4m3 + 1x128 scales in the same epilogue)
//   4. w2 grouped GEMM reading the activation rows contiguously, writing each
//      slot's row to its flat (token, j) position
//   5. weighted top-k reduction y[t] = sum_j w[t,j] * G2[t*k + j] in fixed j
//      order (no floating-point atomics).
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

struct Carver {
  uint8_t* base;
  size_t off = 0;
  template <typename T>
  T* take(int64_t n) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += static_cast<size_t>(n) * sizeof(T);
    return p;
  }
};

// Buffer sizes of the block-aligned slot layout (the reference's
// max_num_tokens_padded rule, tests/ops/moe_align_block_size_ops.py:71-86).
void padded_sizes(int64_t slots, int64_t experts, int64_t bm,
                  int64_t& max_padded, int64_t& max_blocks) {
  max_padded = slots + experts * (bm - 1);
  if (slots < experts) max_padded = std::min(max_padded, slots * bm);
  max_blocks = cdiv(max_padded, bm);
}

// Blocks that can hold at least one valid slot: every active expert adds at
// most one partial block, so ceil(slots/bm) + min(E, slots) bounds them.
int64_t launch_blocks(int64_t slots, int64_t experts, int64_t bm,
                      int64_t max_blocks) {
  int64_t b = cdiv(slots, bm) + std::min(experts, slots);
  return std::min(b, max_blocks);
}

template <typename Id, bool F16>
__global__ __launch_bounds__(256) void weighted_topk_sum_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ g2,
    const float* __restrict__ w, const Id* __restrict__ ids,
    const int32_t* __restrict__ map, int64_t map_len, int64_t num_experts,
    int64_t T, int topk, int64_t H) {
  const int64_t t = blockIdx.y;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (h0 >= H) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto routed = [&](int j) {  // the slot's expert is on this rank
    int64_t id = static_cast<int64_t>(ids[t * topk + j]);
    if (map) {
      if (id < 0 || id >= map_len) return false;
      id = map[id];
    }
    return id >= 0 && id < num_experts;
  };
  if ((H & 7) == 0) {
    // eight slots' rows in flight at a time (read once: non-temporal),
    // summed in slot order
    for (int j0 = 0; j0 < topk; j0 += 8) {
      bool ok[8];
      uint4 u[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int j = j0 + q;
        ok[q] = j < topk && routed(j);
        const int64_t slot = t * topk + (ok[q] ? j : 0);
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g2 + slot * H + h0));
        u[q] = make_uint4(v[0], v[1], v[2], v[3]);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (!ok[q]) continue;
        const float wj = w[t * topk + j0 + q];
        const uint32_t wd[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += wj * ld16<F16>(static_cast<uint16_t>(wd[i] & 0xFFFF));
          acc[2 * i + 1] += wj * ld16<F16>(static_cast<uint16_t>(wd[i] >> 16));
        }
      }
    }
  } else {
    for (int j = 0; j < topk; ++j) {
      if (!routed(j)) continue;
      const float wj = w[t * topk + j];
      const uint16_t* row = g2 + (t * topk + j) * H + h0;
      for (int i = 0; i < 8 && h0 + i < H; ++i) acc[i] += wj * ld16<F16>(row[i]);
    }
  }
  uint16_t* o = out + t * H + h0;
  if ((H & 7) == 0) {
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      wd[i] = st16<F16>(acc[2 * i]) | (uint32_t(st16<F16>(acc[2 * i + 1])) << 16);
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4{wd[0], wd[1], wd[2], wd[3]}, reinterpret_cast<u32x4*>(o));
  } else {
    for (int i = 0; i < 8 && h0 + i < H; ++i) o[i] = st16<F16>(acc[i]);
  }
}

// Decode: the split-K w2 partials summed and reduced over each token's top-k
// slots in one launch.  Workgroup (tile, t) makes columns [256 tile, +256)
// of token t:
//   y[t, h] = T(sum_j w[t,j] * T(sum_z part(slot, h, z) + bias[e, h]))
// (T the call's 16-bit type)
// with the slot's partial tile found through its sorted position
// (inv_pos[t k + j], -1 for slots the sort dropped): four groups of 64
// threads finish the slots j = g, g + 4, ... (4 columns per thread) into
// LDS, then one group sums them in j order -- the same operations in the
// same order as the STREAM finalize launch followed by
// weighted_topk_sum_kernel.  Partial layout of a 256-column STREAM tile:
// column c of slot m is float (2 (64 (c / 32) + 16 ((c % 16) / 4) + m) +
// (c % 32) / 16) 4 + c % 4.
constexpr int kFuseMaxTopk = 32;
template <bool F16>
__global__ __launch_bounds__(256) void finalize_topk_sum_kernel(
    uint16_t* __restrict__ out, const float* __restrict__ part, int ks, int n_tiles,
    const int32_t* __restrict__ inv_pos, const int32_t* __restrict__ block_expert,
    const uint16_t* __restrict__ bias, const float* __restrict__ escale,
    const float* __restrict__ w, int topk, int64_t H) {
  __shared__ float4 s_g[kFuseMaxTopk][64];
  const int64_t t = blockIdx.y;
  const int nt = blockIdx.x;
  const int cg = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int c = 4 * cg;
  const int64_t h = static_cast<int64_t>(nt) * 256 + c;  // H % 4 == 0: h < H covers h..h+3
  const int wv = c / 32, tt = (c % 32) / 16, q = (c % 16) / 4;
  for (int j = grp; j < topk; j += 4) {
    const int pos = inv_pos[t * topk + j];
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
    if (pos >= 0 && h < H) {
      const int blk = pos / 16, m = pos % 16;
      const float* tp = part + (static_cast<int64_t>(blk) * n_tiles + nt) * ks * 4096 +
                        (2 * (64 * wv + 16 * q + m) + tt) * 4;
      float v0 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f;
      for (int z = 0; z < ks; ++z) {
        const float4 a = *reinterpret_cast<const float4*>(tp + z * 4096);
        v0 += a.x; v1 += a.y; v2 += a.z; v3 += a.w;
      }
      if (escale) {  // per-expert factor before the bias (recipe BF16)
        const float es = escale[block_expert[blk]];
        v0 *= es; v1 *= es; v2 *= es; v3 *= es;
      }
      if (bias) {
        const uint16_t* b = bias + static_cast<int64_t>(block_expert[blk]) * H + h;
        v0 += ld16<F16>(b[0]); v1 += ld16<F16>(b[1]);
        v2 += ld16<F16>(b[2]); v3 += ld16<F16>(b[3]);
      }
      g = make_float4(rnd16<F16>((v0)), rnd16<F16>((v1)),
                      rnd16<F16>((v2)), rnd16<F16>((v3)));
    }
    s_g[j][cg] = g;
  }
  __syncthreads();
  if (grp != 0 || h >= H) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int j = 0; j < topk; ++j) {
    if (inv_pos[t * topk + j] < 0) continue;
    const float wj = w[t * topk + j];
    const float4 g = s_g[j][cg];
    a0 += wj * g.x; a1 += wj * g.y; a2 += wj * g.z; a3 += wj * g.w;
  }
  *reinterpret_cast<uint2*>(out + t * H + h) =
      make_uint2(st16<F16>(a0) | (uint32_t(st16<F16>(a1)) << 16),
                 st16<F16>(a2) | (uint32_t(st16<F16>(a3)) << 16));
}

struct FusedActArgs {
  const uint16_t* g1;
  void* act;
  float* acts;
  const int32_t* ntp;
  int64_t rows, inter;
  float clamp, limit;
};

// e8m0 code rows [rows, w] -> [rows, ld] (ld > w), the padding set to 127
// (scale 1.0): a kernel that moves codes four at a time past the last 32-K
// block of a row then reads finite scales (with zero data there).
__global__ __launch_bounds__(256) void repack_codes_kernel(const uint8_t* __restrict__ src,
                                                           uint8_t* __restrict__ dst, int64_t w,
                                                           int64_t ld, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = i / ld, c = i % ld;
  dst[i] = c < w ? src[r * w + c] : static_cast<uint8_t>(127);
}

// Activation scales by sorted position: st[g * ldp + p] = the scale of
// group g of the row that position p holds (its token for w13), 0 for
// padding positions.  Grid (positions / 256, groups / 8): a thread moves
// eight groups of one position (16-byte loads of one row, stores coalesced
// across the wave's positions).  Positions past the padded slot count
// (*ntp, from the sort) are not written: no GEMM tile reads them.
__global__ __launch_bounds__(256) void scales_by_position_kernel(
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ ntp,
    const float* __restrict__ s, float* __restrict__ st, int64_t groups, int64_t ldp,
    int64_t max_padded, int32_t num_valid, int32_t a_div) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= max_padded || p >= *ntp) return;
  const int64_t g0 = static_cast<int64_t>(blockIdx.y) * 8;
  const int64_t ge = groups < g0 + 8 ? groups : g0 + 8;
  const int32_t rid = sorted[p];
  const bool ok = rid >= 0 && rid < num_valid;
  const float* row = s + static_cast<int64_t>(ok ? rid / a_div : 0) * groups;
  int64_t g = g0;
  if ((groups & 3) == 0 && (reinterpret_cast<uintptr_t>(s) & 15) == 0) {
    for (; g < ge; g += 4) {
      const float4 v = ok ? *reinterpret_cast<const float4*>(row + g) : make_float4(0.f, 0.f, 0.f, 0.f);
      st[g * ldp + p] = v.x;
      st[(g + 1) * ldp + p] = v.y;
      st[(g + 2) * ldp + p] = v.z;
      st[(g + 3) * ldp + p] = v.w;
    }
  }
  for (; g < ge; ++g) st[g * ldp + p] = ok ? row[g] : 0.f;
}

// e8m0 code words by sorted position: st[wd * ldp + p] = codes 4 wd .. 4 wd
// + 3 of the row that position p holds (its token for w13; codes past the
// row's w codes read 127, scale 1.0), 0x7f7f7f7f for padding positions.
// Grid (positions / 256, words / 4): a thread moves four words of one
// position (one 16-byte load where the row allows it).  Positions past the
// padded slot count (*ntp) are not written: no GEMM tile reads them.
__global__ __launch_bounds__(256) void codes_by_position_kernel(
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ ntp,
    const uint8_t* __restrict__ c, uint32_t* __restrict__ st, int64_t w, int64_t ld,
    int64_t nwords, int64_t ldp, int64_t max_padded, int32_t num_valid, int32_t a_div) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= max_padded || p >= *ntp) return;
  const int64_t w0 = static_cast<int64_t>(blockIdx.y) * 4;
  const int32_t rid = sorted[p];
  uint32_t v[4] = {0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu};
  if (rid >= 0 && rid < num_valid) {
    const uint8_t* row = c + static_cast<int64_t>(rid / a_div) * ld;
    if (4 * (w0 + 4) <= w && (reinterpret_cast<uintptr_t>(row + 4 * w0) & 15) == 0) {
      const uint4 u = *reinterpret_cast<const uint4*>(row + 4 * w0);
      v[0] = u.x;
      v[1] = u.y;
      v[2] = u.z;
      v[3] = u.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int64_t j = 4 * (w0 + i) + b;
          v[i] |= static_cast<uint32_t>(j < w ? row[j] : 127u) << (8 * b);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (w0 + i < nwords) st[(w0 + i) * ldp + p] = v[i];
}

// Rows of w units [rows, w] -> [rows, ld] (ld > w), the padding zeroed: the
// caller's e2m1 hidden states copied to 128-byte-aligned rows (a zero e2m1
// code meets only the zeroed weights past K).
template <typename U>
__global__ __launch_bounds__(256) void repack_rows_kernel(const U* __restrict__ src,
                                                          U* __restrict__ dst, int64_t w,
                                                          int64_t ld, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = i / ld, c = i % ld;
  dst[i] = c < w ? src[r * w + c] : U{};
}

// Activations without a GEMM-epilogue form (gelu, gelu_tanh, swiglustep,
// relu2_no_mul): the w13 output G1 (16-bit [rows, 2I] by sorted position,
// gate | up) -> activation [rows, K2], K2 = I (gated) or 2I (relu2_no_mul),
// with the reference's rounding points (G1 and, for gelu, act(gate) rounded
// to the 16-bit type; swiglustep in fp32; gemm1_clamp_limit on the 16-bit
// halves first;
// fused_moe_interface.py:383-396).  Each lane makes 8 output columns; Q8:
// e4m3 with 1x128 scales of the 16-bit activation (16 lanes per group), as the
// fp8 GLU epilogues quantise it.  Rows from *ntp on (padding past the last
// block) are not touched; K2 % 128 == 0 when Q8, so a group's lanes share a
// row and leave together.
template <int ACT, bool Q8, bool F16>
__global__ __launch_bounds__(256) void fused_act_kernel(
    const uint16_t* __restrict__ g1, void* __restrict__ act, float* __restrict__ acts,
    const int32_t* __restrict__ ntp, int64_t inter, float clamp, float limit) {
  const int64_t k2 = ACT == MI355MOE_ACT_RELU2 ? 2 * inter : inter;
  const int64_t cpr = k2 >> 3;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t r = gtid / cpr;
  const int64_t c0 = (gtid % cpr) * 8;
  if (r >= *ntp) return;
  const uint16_t* x = g1 + r * 2 * inter;
  const uint4 xa = *reinterpret_cast<const uint4*>(x + c0);
  const uint32_t wa[4] = {xa.x, xa.y, xa.z, xa.w};
  float y[8];
  if constexpr (ACT == MI355MOE_ACT_RELU2) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = ld16<F16>(static_cast<uint16_t>(wa[i >> 1] >> (16 * (i & 1))));
      if (clamp > 0.f)
        v = rnd16<F16>(c0 + i < inter ? fminf(v, clamp) : fminf(fmaxf(v, -clamp), clamp));
      const float p = fmaxf(v, 0.f);
      y[i] = rnd16<F16>(p * p);
    }
  } else {
    const uint4 xb = *reinterpret_cast<const uint4*>(x + inter + c0);
    const uint32_t wb[4] = {xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float g = ld16<F16>(static_cast<uint16_t>(wa[i >> 1] >> (16 * (i & 1))));
      float u = ld16<F16>(static_cast<uint16_t>(wb[i >> 1] >> (16 * (i & 1))));
      if (clamp > 0.f) {
        g = rnd16<F16>(fminf(g, clamp));
        u = rnd16<F16>(fminf(fmaxf(u, -clamp), clamp));
      }
      float v;
      if constexpr (ACT == MI355MOE_ACT_GELU) {
        v = rnd16<F16>(gelu_erf(g)) * u;
      } else if constexpr (ACT == MI355MOE_ACT_GELU_TANH) {
        v = rnd16<F16>(gelu_tanh(g)) * u;
      } else {
        v = fminf(g / (1.f + expf(-g)), limit) * fminf(fmaxf(u, -limit), limit);
      }
      y[i] = rnd16<F16>(v);
    }
  }
  if constexpr (Q8) {
    float amax = 1e-10f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(y[i]));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float sc = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
    if ((gtid & 15) == 0) acts[r * (k2 / 128) + c0 / 128] = sc;
    const float inv = 1.0f / sc;
    const uint32_t lo = e4m3x4_sat(y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv);
    const uint32_t hi = e4m3x4_sat(y[4] * inv, y[5] * inv, y[6] * inv, y[7] * inv);
    *reinterpret_cast<uint2*>(static_cast<uint8_t*>(act) + r * k2 + c0) = make_uint2(lo, hi);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = st16<F16>(y[2 * i]) | (static_cast<uint32_t>(st16<F16>(y[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(act) + r * k2 + c0) =
        make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <bool Q8, bool F16>
void launch_fused_act(int act, const FusedActArgs& f, hipStream_t st) {
  const int64_t k2 = act == MI355MOE_ACT_RELU2 ? 2 * f.inter : f.inter;
  dim3 grid(static_cast<unsigned>(cdiv(f.rows * (k2 / 8), 256)));
  switch (act) {
    case MI355MOE_ACT_GELU:
      fused_act_kernel<MI355MOE_ACT_GELU, Q8, F16><<<grid, dim3(256), 0, st>>>(
          f.g1, f.act, f.acts, f.ntp, f.inter, f.clamp, f.limit);
      break;
    case MI355MOE_ACT_GELU_TANH:
      fused_act_kernel<MI355MOE_ACT_GELU_TANH, Q8, F16><<<grid, dim3(256), 0, st>>>(
          f.g1, f.act, f.acts, f.ntp, f.inter, f.clamp, f.limit);
      break;
    case MI355MOE_ACT_SWIGLUSTEP:
      fused_act_kernel<MI355MOE_ACT_SWIGLUSTEP, Q8, F16><<<grid, dim3(256), 0, st>>>(
          f.g1, f.act, f.acts, f.ntp, f.inter, f.clamp, f.limit);
      break;
    default:
      fused_act_kernel<MI355MOE_ACT_RELU2, Q8, F16><<<grid, dim3(256), 0, st>>>(
          f.g1, f.act, f.acts, f.ntp, f.inter, f.clamp, f.limit);
      break;
  }
}

int group_quant_fp8(const void* x, int dt, uint8_t* q, float* s, int64_t rows,
                    int64_t cols, hipStream_t st) {
  return mi355moe_per_token_group_fp8_quant(x, dt, q, s, rows, cols, 128, 1e-10f,
                                            -448.f, 448.f, 0, st);
}

struct FusedLayout {
  int bm;
  GemmTile tile;
  int64_t slots, max_padded, max_blocks, grid_blocks;
  int32_t *sorted, *eids, *ntp;
  int32_t* cum;     // [E+1] padded slot start of every expert
  int ks1, ks2;     // STREAM split-K of w13 / w2 (1: none)
  float *part1, *part2;    // split-K partial tiles
  int32_t* inv;     // [slots] sorted position of every flat slot (-1: dropped)
  int32_t* sortws;  // multi-workgroup sort scratch (sortws_bytes, may be 0)
  size_t sortws_bytes;
  uint8_t* xq;    // fp8 hidden [T, H]
  float* xs;      // [T, H/128]
  void* act;      // bf16 [max_padded, K2] or e4m3 [max_padded, K2] (mxfp4 w4a4:
                  // packed e2m1 [max_padded, K2/2])
  float* acts;    // [max_padded, K2/128] (ldp: [K2/128, ldp], by sorted position)
  // fp8 block-scaled prefill on the 320-slot kernel: both GEMMs read their
  // activation scales by sorted position, [K/128, ldp] (ldp: max_padded
  // rounded up to 64; 0 otherwise); xst holds the hidden states' scales so
  float* xst;
  int64_t ldp;
  // MX on the 320-slot kernel: the hidden states' e8m0 code words by sorted
  // position, [ld1 / 4, ldp] (and the activation's, acts8, [ld2 / 4, ldp])
  uint32_t* xs8t;
  uint8_t* xs8;   // MX: e8m0 scales of the quantised hidden [T, ld1]
  uint8_t* acts8; // MX: e8m0 scales of the activation [max_padded, ld2]
  int64_t ld1, ld2;
  // w4a4 on the 320-slot kernel: row pitches (bytes, multiples of 128) of
  // the e2m1 hidden copy xp [T, p1] (null when H / 2 is already one) and of
  // the activation act [max_padded, p2]; 0 when unused
  uint8_t* xp;
  int64_t p1, p2;
  uint16_t* g1;   // generic activations: w13 output bf16 [max_padded, 2I]
  uint16_t* g2;   // bf16 [slots, H]
  bool token_w2;  // STREAM w2 token-major: it writes the layer output
  bool khalves;   // fp8 decode: w13 in K halves (no split launch) writes the
                  // 16-bit activation act16, which the token-major w2 quantises
  uint16_t* act16;  // [max_padded, K2]
  size_t bytes;
};

// Activations the w13 GEMM epilogue applies itself; the others run as a
// separate kernel over the stored w13 output.
bool epilogue_act(int act) {
  return act == MI355MOE_ACT_SILU || act == MI355MOE_ACT_SWIGLUOAI;
}
// Width of the activation (and K of the w2 GEMM): relu2_no_mul keeps all 2I.
// x rounded to nearest even in the call's 16-bit type (host side).
float round_to_16(float x, bool f16) {
  if (f16) return static_cast<float>(static_cast<_Float16>(x));
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7F800000u) != 0x7F800000u) u += 0x7FFFu + ((u >> 16) & 1u);
  u &= 0xFFFF0000u;
  std::memcpy(&x, &u, 4);
  return x;
}

int64_t act_width(const mi355moe_fused_moe_args* a) {
  return a->activation == MI355MOE_ACT_RELU2 ? 2 * a->inter : a->inter;
}

// MX recipes (scales of both operands in the MFMA): mxfp8, and mxfp4 with
// pre-quantised (e2m1) hidden states; the GEMMs then run recipe
// gemm_recipe().
bool mx_layer(const mi355moe_fused_moe_args* a) {
  return a->recipe == MI355MOE_RECIPE_MXFP8 ||
         (a->recipe == MI355MOE_RECIPE_MXFP4 && a->hidden_scale != nullptr);
}
int gemm_recipe(const mi355moe_fused_moe_args* a) {
  return a->recipe == MI355MOE_RECIPE_MXFP4 && a->hidden_scale ? RECIPE_MX4A4 : a->recipe;
}

// At most 16 slots on the STREAM kernels: the w13 launch sorts the slots
// itself (and quantises fp8 activations into LDS) instead of a sort
// launch before it.  MI355MOE_STREAM_SELF_SORT=0 keeps the sort launch (the
// same outputs).  Read per call.
bool stream_self_sort_enabled() {
  const char* v = getenv("MI355MOE_STREAM_SELF_SORT");
  return !(v && v[0] == '0');
}
// At most 16 slots, top-k dividing 8 and enough output columns to fill the
// GPU: the w2 launch runs token-major and writes the layer output (no top-k
// reduction launch).  MI355MOE_STREAM_TOKEN_W2=0 keeps the reduction launch
// (the same arithmetic).  Read per call.
bool stream_token_w2_enabled() {
  const char* v = getenv("MI355MOE_STREAM_TOKEN_W2");
  return !(v && v[0] == '0');
}
// Split-K w13 with a 16-bit activation: the w2 launch rebuilds its
// activation rows from the w13 partial tiles (no w13 finalize launch).
// MI355MOE_STREAM_W2_FINISHES_W13=0 keeps the finalize launch (the same
// arithmetic).  Read per call.
bool stream_w2_finishes_w13_enabled() {
  const char* v = getenv("MI355MOE_STREAM_W2_FINISHES_W13");
  return !(v && v[0] == '0');
}
// fp8block decode whose w13 would split K (too few 128-column tiles to fill
// the GPU) and whose w2 runs token-major: w13 runs 64-column workgroups over
// both K halves (GemmArgs::khalves) and stores the 16-bit activation, which
// each token-major w2 wave quantises for its own slot (GemmArgs::tok_xq) --
// no partial-sum launch.  MI355MOE_STREAM_KHALVES=0 keeps the split launch
// and its finalize (the same arithmetic).  Read per call.
// fp8 block-scaled prefill on the 320-slot kernel: activation scales stored
// by sorted position ([K/128, positions]), gathered once per layer, instead
// of read row by row inside the GEMM (one cache line per slot row and K
// stage).  MI355MOE_SCALES_BY_POSITION=0 keeps the row-major scales (the
// same arithmetic).  Read per call.
bool scales_by_position_enabled() {
  const char* v = getenv("MI355MOE_SCALES_BY_POSITION");
  return !(v && v[0] == '0');
}
bool stream_khalves_enabled() {
  const char* v = getenv("MI355MOE_STREAM_KHALVES");
  return !(v && v[0] == '0');
}

FusedLayout plan(const mi355moe_fused_moe_args* a, uint8_t* base) {
  FusedLayout L{};
  const int64_t E = a->num_experts;
  L.slots = a->num_tokens * a->topk;
  const int64_t H = a->hidden, I = a->inter, K2 = act_width(a);
  const bool glu = epilogue_act(a->activation);
  const bool kblock = a->w_layout == MI355MOE_WLAYOUT_KBLOCK;
  const bool wide_ok = wide_ok_for(gemm_recipe(a), a->num_tokens, 2 * I, H, kblock) &&
                       wide_ok_for(gemm_recipe(a), L.slots + E * kWideBM, H, K2, kblock);
  L.tile = pick_tile(gemm_recipe(a), wide_ok, L.slots, E, &L.bm);
  // K-blocked weights: the families that read them (STREAM, SMALL, WIDE, and
  // BIG for fp8, whose 8-wave kernel takes K <= 8192, and for mxfp4)
  if (kblock && a->recipe != MI355MOE_RECIPE_MXFP4 &&
      L.tile != TILE_STREAM && L.tile != TILE_SMALL && L.tile != TILE_WIDE &&
      !(L.tile == TILE_BIG && a->recipe == MI355MOE_RECIPE_FP8BLOCK)) {
    L.tile = TILE_SMALL;
    L.bm = 64;
  }
  padded_sizes(L.slots, E, L.bm, L.max_padded, L.max_blocks);
  L.grid_blocks = launch_blocks(L.slots, E, L.bm, L.max_blocks);
  Carver c{base};
  L.sorted = c.take<int32_t>(std::max<int64_t>(L.max_padded, 1));
  L.eids = c.take<int32_t>(std::max<int64_t>(L.max_blocks, 1));
  L.ntp = c.take<int32_t>(1);
  L.cum = c.take<int32_t>(E + 1);
  L.ks1 = L.ks2 = 1;
  L.part1 = L.part2 = nullptr;
  if (L.tile == TILE_STREAM) {
    const int64_t act_blocks = std::min<int64_t>(L.slots, E);
    // GLU tiles cover 128 activation columns, STORE tiles 256 of G1
    const int64_t nt1 = glu ? cdiv(I, 128) : cdiv(2 * I, 256), nt2 = cdiv(H, 256);
    L.ks1 = stream_ksplit(nt1, act_blocks, H);
    L.ks2 = stream_ksplit(nt2, act_blocks, K2);
    const int64_t T = a->num_tokens, k = a->topk;
    L.token_w2 = L.ks2 <= 1 && L.slots <= 16 && k <= 8 && 8 % k == 0 &&
                 cdiv(H, 32 * (8 / k)) * T >= 192 && stream_token_w2_enabled();
    // (the w13 tile then quantises the whole K of every token: the LDS
    // tile must hold it where the layer quantises its own activation)
    L.khalves = L.token_w2 && L.ks1 > 1 && glu && a->recipe == MI355MOE_RECIPE_FP8BLOCK &&
                K2 % 128 == 0 && K2 <= kStreamTokXBytes &&
                (a->hidden_scale || T * H <= kStreamSelfXBytes) && stream_khalves_enabled();
    if (L.khalves) L.ks1 = 1;
    const int64_t tile_f = 512 * 8;
    if (L.ks1 > 1) L.part1 = c.take<float>(L.max_blocks * nt1 * L.ks1 * tile_f);
    if (L.ks2 > 1) L.part2 = c.take<float>(L.max_blocks * nt2 * L.ks2 * tile_f);
  }
  L.inv = c.take<int32_t>(std::max<int64_t>(L.slots, 1));
  L.sortws_bytes = counting_sort_ws_bytes(L.slots, E);
  L.sortws = c.take<int32_t>(static_cast<int64_t>(L.sortws_bytes / sizeof(int32_t)));
  const bool fp8 = a->recipe == MI355MOE_RECIPE_FP8BLOCK;
  if (mx_layer(a)) {
    // e8m0 scale rows padded to a multiple of 4 bytes
    L.ld1 = (a->hidden / 32 + 3) / 4 * 4;
    L.ld2 = (K2 / 32 + 3) / 4 * 4;
    if (!a->hidden_scale) L.xq = c.take<uint8_t>(a->num_tokens * a->hidden);
    // the layer's own codes, or the caller's repacked to 4-byte rows
    if (!a->hidden_scale || L.ld1 != a->hidden / 32)
      L.xs8 = c.take<uint8_t>(a->num_tokens * L.ld1);
    if (gemm_recipe(a) == RECIPE_MX4A4 && L.tile == TILE_WIDE) {
      L.p1 = (a->hidden / 2 + 127) / 128 * 128;
      L.p2 = (K2 / 2 + 127) / 128 * 128;
      if (L.p1 != a->hidden / 2) L.xp = c.take<uint8_t>(a->num_tokens * L.p1);
    }
    L.act = c.take<uint8_t>(L.max_padded * (gemm_recipe(a) == RECIPE_MX4A4
                                                ? (L.p2 ? L.p2 : K2 / 2) : K2));
    if (L.tile == TILE_WIDE && scales_by_position_enabled()) {
      L.ldp = (L.max_padded + 63) / 64 * 64;
      L.xs8t = c.take<uint32_t>((L.ld1 / 4) * L.ldp);
      L.acts8 = c.take<uint8_t>(L.ld2 * L.ldp);
    } else {
      L.acts8 = c.take<uint8_t>(L.max_padded * L.ld2);
    }
  } else if (fp8) {
    L.xq = c.take<uint8_t>(a->num_tokens * a->hidden);
    L.xs = c.take<float>(a->num_tokens * (a->hidden / 128));
    L.act = c.take<uint8_t>(L.max_padded * K2);
    // (the 320-slot and 128-slot fp8 kernels, which take K <= 8192)
    if ((L.tile == TILE_WIDE || L.tile == TILE_BIG) && glu && K2 % 128 == 0 &&
        a->hidden <= 8192 && K2 <= 8192 && scales_by_position_enabled()) {
      L.ldp = (L.max_padded + 63) / 64 * 64;
      L.xst = c.take<float>((a->hidden / 128) * L.ldp);
      L.acts = c.take<float>((K2 / 128) * L.ldp);
    } else {
      L.acts = c.take<float>(L.max_padded * (K2 / 128));
    }
  } else {
    L.act = c.take<uint16_t>(L.max_padded * K2);
  }
  L.g1 = glu ? nullptr : c.take<uint16_t>(L.max_padded * 2 * I);
  L.g2 = c.take<uint16_t>(L.slots * a->hidden);
  L.act16 = L.khalves ? c.take<uint16_t>(L.max_padded * K2) : nullptr;
  L.bytes = c.off + 256;
  return L;
}

}  // namespace
}  // namespace mi355

using namespace mi355;

extern "C" size_t mi355moe_fused_moe_workspace_size(const mi355moe_fused_moe_args* a) {
  if (!a) return 0;
  return plan(a, nullptr).bytes;
}

namespace mi355 {
namespace {
int validate(const mi355moe_fused_moe_args* a);
int fused_moe_impl(const mi355moe_fused_moe_args* a, void* ws, size_t ws_bytes,
                   void* stream, hipEvent_t* ev);
}
}  // namespace mi355

struct mi355moe_timer_s {
  int max_steps;
  std::vector<hipEvent_t> ev;  // (kFusedStages + 1) per step
};

extern "C" int mi355moe_fused_moe(const mi355moe_fused_moe_args* a, void* ws,
                                  size_t ws_bytes, void* stream) {
  return fused_moe_impl(a, ws, ws_bytes, stream, nullptr);
}

// ----------------------------------------------- allocation-free variant
// Scratch of mi355moe_fused_moe_noalloc: a file-scope device array, one copy
// per GPU the library runs on, held until the process ends.  Host code never
// uses its name as an address: the address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept per device.  Every
// call on a GPU reuses that GPU's array (the kernels initialise what they
// read), so calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t scratch[MI355MOE_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // by device ordinal

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream).
int scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  MI_HIP(hipGetDevice(&dev));
  int sdev = dev;
  if (stream) MI_HIP(hipStreamGetDevice(stream, &sdev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (static_cast<size_t>(sdev) >= g_scratch_ptr.size())
    g_scratch_ptr.resize(static_cast<size_t>(sdev) + 1, nullptr);
  if (!g_scratch_ptr[sdev]) {
    if (sdev != dev) MI_HIP(hipSetDevice(sdev));
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (sdev != dev) MI_HIP(hipSetDevice(dev));
    if (rc != hipSuccess || p == nullptr)
      return set_error(MI355MOE_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") +
                                             hipGetErrorString(rc));
    g_scratch_ptr[sdev] = p;
  }
  *out = g_scratch_ptr[sdev];
  return MI355MOE_OK;
}
}  // namespace

extern "C" int mi355moe_fused_moe_noalloc(const mi355moe_fused_moe_args* a, void* stream) {
  if (int rc = validate(a)) return rc;   // before the arguments size anything
  const size_t need = mi355moe_fused_moe_workspace_size(a);
  MI_CHECK(need <= MI355MOE_NOALLOC_SCRATCH_BYTES, MI355MOE_ERR_WORKSPACE,
           "fused_moe_noalloc: this call needs " + std::to_string(need) +
               " bytes of scratch, more than the static " +
               std::to_string(MI355MOE_NOALLOC_SCRATCH_BYTES) +
               " (use mi355moe_fused_moe with a caller workspace)");
  void* ptr = nullptr;
  if (int rc = scratch_address(static_cast<hipStream_t>(stream), &ptr)) return rc;
  return fused_moe_impl(a, ptr, MI355MOE_NOALLOC_SCRATCH_BYTES, stream, nullptr);
}

extern "C" int mi355moe_timer_create(int max_steps, mi355moe_timer* out) {
  MI_ARG(max_steps > 0 && out != nullptr, "invalid timer arguments");
  auto* t = new mi355moe_timer_s{max_steps, {}};
  t->ev.resize(static_cast<size_t>(max_steps) * (MI355MOE_FUSED_STAGES + 1));
  for (auto& e : t->ev) {
    hipError_t rc = hipEventCreate(&e);
    if (rc != hipSuccess) {
      for (auto& f : t->ev) if (f) (void)hipEventDestroy(f);
      delete t;
      return set_error(MI355MOE_ERR_HIP, std::string("hipEventCreate: ") + hipGetErrorString(rc));
    }
  }
  *out = t;
  return MI355MOE_OK;
}

extern "C" int mi355moe_timer_destroy(mi355moe_timer t) {
  if (!t) return MI355MOE_OK;
  for (auto& e : t->ev) if (e) (void)hipEventDestroy(e);
  delete t;
  return MI355MOE_OK;
}

extern "C" int mi355moe_fused_moe_timed(const mi355moe_fused_moe_args* a, void* ws,
                                        size_t ws_bytes, void* stream,
                                        mi355moe_timer t, int step) {
  MI_ARG(t && step >= 0 && step < t->max_steps, "timer step out of range");
  return fused_moe_impl(a, ws, ws_bytes, stream,
                        &t->ev[static_cast<size_t>(step) * (MI355MOE_FUSED_STAGES + 1)]);
}

extern "C" int mi355moe_timer_stage_ms(mi355moe_timer t, int step, float* ms) {
  MI_ARG(t && ms && step >= 0 && step < t->max_steps, "timer step out of range");
  hipEvent_t* e = &t->ev[static_cast<size_t>(step) * (MI355MOE_FUSED_STAGES + 1)];
  MI_HIP(hipEventSynchronize(e[MI355MOE_FUSED_STAGES]));
  for (int i = 0; i < MI355MOE_FUSED_STAGES; ++i) MI_HIP(hipEventElapsedTime(&ms[i], e[i], e[i + 1]));
  return MI355MOE_OK;
}

namespace mi355 {
namespace {
// Argument checks of the fused layer, before any sizing or launch (both
// entry points): MI355MOE_OK or the error code, with the message set.
int validate(const mi355moe_fused_moe_args* a) {
  MI_ARG(a != nullptr, "null arguments");
  const int64_t T = a->num_tokens, H = a->hidden, I = a->inter,
                E = a->num_experts, k = a->topk;
  MI_ARG(T >= 0 && H > 0 && I > 0 && E > 0 && k > 0, "invalid layer shape");
  MI_ARG(E <= 1024, "num_experts must be at most 1024");
  MI_ARG(a->act_dtype == MI355MOE_BF16 || a->act_dtype == MI355MOE_F16,
         "hidden_states must be bfloat16 or float16");
  MI_ARG(!a->hidden_scale || a->recipe == MI355MOE_RECIPE_FP8BLOCK ||
             a->recipe == MI355MOE_RECIPE_MXFP8 || a->recipe == MI355MOE_RECIPE_MXFP4,
         "pre-quantised hidden_states (hidden_scale) need the fp8block, mxfp8 or "
         "mxfp4 recipe");
  MI_ARG(a->ids_dtype == MI355MOE_I32 || a->ids_dtype == MI355MOE_I64,
         "topk_ids must be int32 or int64");
  MI_ARG(a->activation >= MI355MOE_ACT_SILU && a->activation <= MI355MOE_ACT_RELU2,
         "unsupported activation");
  const int recipe = a->recipe;
  if (recipe == MI355MOE_RECIPE_FP8BLOCK) {
    MI_ARG(H % 128 == 0 && I % 128 == 0,
           "fp8 block-scaled weights need hidden and intermediate sizes % 128 == 0");
    MI_ARG(a->w13_scale && a->w2_scale, "fp8 block-scaled weights need scales");
    MI_ARG(a->w13_scale_rows == 0 || a->w13_scale_rows == 128 || a->w13_scale_rows == 64,
           "w13_scale_rows must be 128 or 64");
  } else if (recipe == MI355MOE_RECIPE_INT4) {
    const int64_t g = a->w_group;
    MI_ARG(g == 32 || g == 64 || g == 128 || g == 256,
           "int4 group size must be 32, 64, 128 or 256");
    MI_ARG(H % g == 0 && act_width(a) % g == 0,
           "int4 weights need hidden and intermediate sizes % group_size == 0");
    MI_ARG(a->w13_scale && a->w2_scale, "int4 weights need group scales");
  } else if (recipe == MI355MOE_RECIPE_MXFP4) {
    MI_ARG(H % 32 == 0 && I % 32 == 0, "mxfp4 weights need K % 32 == 0");
    MI_ARG(a->w13_scale && a->w2_scale, "mxfp4 weights need e8m0 scales");
  } else if (recipe == MI355MOE_RECIPE_MXFP8) {
    MI_ARG(H % 32 == 0 && I % 32 == 0, "mxfp8 weights need hidden and intermediate sizes % 32 == 0");
    MI_ARG(a->w13_scale && a->w2_scale, "mxfp8 weights need e8m0 scales");
  } else if (is_w8a16_recipe(recipe)) {
    MI_CHECK(H % 32 == 0 && act_width(a) % 32 == 0, MI355MOE_ERR_UNSUPPORTED,
             "per-expert fp8 weights need hidden and intermediate sizes % 32 == 0 (others "
             "run on 16-bit copies, recipe BF16)");
    MI_ARG(a->w13_scale && a->w2_scale, "per-expert fp8 weights need f32 scales [E]");
  } else {
    MI_ARG(recipe == MI355MOE_RECIPE_BF16, "unknown recipe");
    MI_ARG(H % 8 == 0 && I % 8 == 0, "bf16 weights need K % 8 == 0");
  }
  MI_ARG(a->w_layout == MI355MOE_WLAYOUT_NK || a->w_layout == MI355MOE_WLAYOUT_KBLOCK,
         "unknown weight layout");
  const bool kblock = a->w_layout == MI355MOE_WLAYOUT_KBLOCK;
  MI_ARG(!kblock || (recipe == MI355MOE_RECIPE_BF16 && H % 32 == 0 && I % 32 == 0) ||
             (recipe == MI355MOE_RECIPE_FP8BLOCK && H <= 8192 && act_width(a) <= 8192) ||
             (recipe == MI355MOE_RECIPE_MXFP8 && H % 128 == 0 && act_width(a) % 128 == 0) ||
             is_w8a16_recipe(recipe) || recipe == MI355MOE_RECIPE_INT4 ||
             recipe == MI355MOE_RECIPE_MXFP4,
         "K-blocked weights need the bf16 recipe (hidden and intermediate sizes "
         "% 32 == 0), the fp8block recipe (sizes at most 8192), mxfp8 (sizes % 128 "
         "== 0), per-expert fp8, int4 or mxfp4");
  MI_ARG(!mx_layer(a) || epilogue_act(a->activation),
         "mxfp8 and pre-quantised mxfp4 layers support the silu and swigluoai activations");
  return MI355MOE_OK;
}

int fused_moe_impl(const mi355moe_fused_moe_args* a, void* ws, size_t ws_bytes,
                   void* stream, hipEvent_t* ev) {
  if (int rc = validate(a)) return rc;
  const int64_t T = a->num_tokens, H = a->hidden, I = a->inter, E = a->num_experts,
                k = a->topk;
  const int recipe = a->recipe;
  const bool kblock = a->w_layout == MI355MOE_WLAYOUT_KBLOCK;
  if (T == 0) return MI355MOE_OK;
  FusedLayout L = plan(a, static_cast<uint8_t*>(ws));
  MI_CHECK(ws && ws_bytes >= L.bytes, MI355MOE_ERR_WORKSPACE,
           "workspace too small for fused_moe");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t id_bound = a->expert_map ? a->expert_map_len : E;
  auto mark = [&](int i) -> int {
    if (ev) MI_HIP(hipEventRecord(ev[i], st));
    return MI355MOE_OK;
  };

  const bool fp8 = recipe == MI355MOE_RECIPE_FP8BLOCK;
  const bool mx = mx_layer(a);
  const int grecipe = gemm_recipe(a);
  const bool f16 = a->act_dtype == MI355MOE_F16;  // the call's 16-bit type
  // caller-quantised hidden states (e4m3 + 1x128 scales) go to w13 as given
  const bool preq = fp8 && a->hidden_scale;

  if (int m = mark(0)) return m;
  const bool glu = epilogue_act(a->activation);
  // at most 16 slots on the STREAM kernels: the w13 launch routes them
  // itself (and quantises fp8 activations into LDS)
  // (fp8: every token row's K range of a split fits the kernel's LDS tile)
  const int64_t self_per = cdiv(cdiv(H, 128), L.ks1);
  const bool self_quant_ok =
      H % 128 == 0 && T * self_per * 128 <= kStreamSelfXBytes &&
      (reinterpret_cast<uintptr_t>(a->hidden_states) & 15) == 0;
  const bool self_sort = L.tile == TILE_STREAM && L.slots <= 16 && !mx && glu &&
                         (!fp8 || preq || self_quant_ok) && stream_self_sort_enabled();
  // up to 4096 slots: the sort and the e4m3 activation quantisation share
  // one launch (the quantisation stage is then empty)
  int rc = 1;
  if (self_sort) {
    rc = 0;
  } else if (fp8 && !preq) {
    rc = run_sort_quant_fp8(a->topk_ids, a->ids_dtype, L.slots, id_bound, a->expert_map, E,
                            L.bm, L.sorted, L.max_padded, L.eids, L.max_blocks, L.ntp, L.inv,
                            static_cast<int32_t>(L.slots), L.cum, a->hidden_states, f16, L.xq,
                            L.xs, T, H, st);
    if (rc < 0) return rc;
  }
  const bool quantised = rc == 0;
  if (!quantised && !self_sort) {
    rc = run_counting_sort(a->topk_ids, a->ids_dtype, L.slots, id_bound,
                           a->expert_map, E, L.bm, L.sorted, L.max_padded,
                           L.eids, L.max_blocks, L.ntp, L.inv, nullptr,
                           static_cast<int32_t>(L.slots), L.sortws, L.sortws_bytes, st,
                           L.cum);
    if (rc) return rc;
  }

  if (int m = mark(1)) return m;
  if (fp8 && !preq && !quantised && !self_sort) {
    rc = group_quant_fp8(a->hidden_states, a->act_dtype, L.xq, L.xs, T, H, st);
    if (rc) return rc;
  }
  if (mx && !a->hidden_scale) {
    rc = mx8_quant_rows(a->hidden_states, f16, L.xq, L.xs8, L.ld1, T, H, st);
    if (rc) return rc;
  }
  // caller's codes [T, H/32] with rows not a multiple of 4 bytes: copied into
  // 4-byte rows, which the 320-slot kernels move four codes at a time (unless
  // the codes are gathered by position below, which pads the rows itself)
  const bool repack = mx && a->hidden_scale && L.ld1 != H / 32 && !L.xs8t;
  if (repack) {
    const int64_t n = T * L.ld1;
    repack_codes_kernel<<<static_cast<unsigned>(cdiv(n, 256)), dim3(256), 0, st>>>(
        static_cast<const uint8_t*>(a->hidden_scale), L.xs8, H / 32, L.ld1, n);
    MI_LAUNCH_CHECK();
  }
  if (L.xp) {
    const int64_t rb = H / 2;  // packed e2m1 row bytes (H % 32 == 0)
    if ((reinterpret_cast<uintptr_t>(a->hidden_states) & 15) == 0) {
      const int64_t n = T * (L.p1 / 16);
      repack_rows_kernel<uint4><<<static_cast<unsigned>(cdiv(n, 256)), dim3(256), 0, st>>>(
          static_cast<const uint4*>(a->hidden_states), reinterpret_cast<uint4*>(L.xp), rb / 16,
          L.p1 / 16, n);
    } else {
      const int64_t n = T * L.p1;
      repack_rows_kernel<uint8_t><<<static_cast<unsigned>(cdiv(n, 256)), dim3(256), 0, st>>>(
          static_cast<const uint8_t*>(a->hidden_states), L.xp, rb, L.p1, n);
    }
    MI_LAUNCH_CHECK();
  }
  if (L.xs8t) {  // the hidden states' e8m0 codes by sorted position
    const bool own = !a->hidden_scale;  // the layer's own codes, L.xs8: [T, ld1]
    const int64_t nwords = L.ld1 / 4;
    const dim3 sg(static_cast<unsigned>(cdiv(L.max_padded, 256)),
                  static_cast<unsigned>(cdiv(nwords, 4)));
    codes_by_position_kernel<<<sg, dim3(256), 0, st>>>(
        L.sorted, L.ntp, own ? L.xs8 : static_cast<const uint8_t*>(a->hidden_scale), L.xs8t,
        own ? L.ld1 : H / 32, own ? L.ld1 : H / 32, nwords, L.ldp, L.max_padded,
        static_cast<int32_t>(L.slots), static_cast<int32_t>(k));
    MI_LAUNCH_CHECK();
  }
  if (L.xst) {  // the hidden states' scales by sorted position
    const dim3 grid(static_cast<unsigned>(cdiv(L.max_padded, 256)),
                    static_cast<unsigned>(cdiv(H / 128, 8)));
    scales_by_position_kernel<<<grid, dim3(256), 0, st>>>(
        L.sorted, L.ntp, preq ? static_cast<const float*>(a->hidden_scale) : L.xs, L.xst, H / 128,
        L.ldp, L.max_padded, static_cast<int32_t>(L.slots), static_cast<int32_t>(k));
    MI_LAUNCH_CHECK();
  }
  if (int m = mark(2)) return m;

  // gelu / gelu_tanh / swiglustep / relu2_no_mul: w13 stores G1, a separate
  // kernel applies the activation (and the fp8 re-quantisation)
  const int64_t K2 = act_width(a);
  GemmArgs g1{};
  g1.A = (fp8 && !preq) || (mx && !a->hidden_scale) ? static_cast<const void*>(L.xq)
         : L.xp ? static_cast<const void*>(L.xp) : a->hidden_states;
  g1.lda = L.xp ? L.p1 : 0;
  g1.ldd = L.p2;
  g1.a_scale = L.xst ? L.xst
               : preq ? static_cast<const float*>(a->hidden_scale) : (fp8 ? L.xs : nullptr);
  g1.a_scale_tld = L.xst ? L.ldp : 0;
  g1.q_scale_tld = L.xst ? L.ldp : 0;  // the w13 epilogue writes w2's scales by position
  if (mx) {
    g1.a_mxs = L.xs8t ? reinterpret_cast<const uint8_t*>(L.xs8t)
               : a->hidden_scale && !repack ? static_cast<const uint8_t*>(a->hidden_scale) : L.xs8;
    g1.a_mxs_ld = a->hidden_scale && !repack && !L.xs8t ? H / 32 : L.ld1;
    g1.q_mxs_ld = L.ld2;
    g1.a_scale_tld = L.xs8t ? L.ldp : 0;
    g1.q_scale_tld = L.xs8t ? L.ldp : 0;
  }
  g1.B = a->w13;
  g1.b_scale = a->w13_scale;
  g1.bias = static_cast<const uint16_t*>(a->w13_bias);
  g1.D = glu ? L.act : static_cast<void*>(L.g1);
  g1.row_ids = L.sorted;
  g1.block_expert = L.eids;
  g1.ntp = L.ntp;
  g1.expert_cum = L.cum;
  g1.num_valid = static_cast<int32_t>(L.slots);
  g1.a_div = static_cast<int32_t>(k);
  g1.a_by_pos = 0;
  g1.d_by_pos = 1;
  g1.N = glu ? I : 2 * I;
  g1.K = H;
  g1.ldb_rows = 2 * I;
  g1.up_off = glu ? I : 0;
  // the reference clamps the 16-bit G1 in place: with the limit itself in
  // that type, clamping 16-bit values needs no rounding afterwards
  const float clamp16 = a->gemm1_clamp_limit > 0.f ? round_to_16(a->gemm1_clamp_limit, f16) : 0.f;
  g1.clamp_limit = clamp16;
  g1.alpha = a->swiglu_alpha;
  g1.limit = a->swiglu_limit;
  g1.act = a->activation;
  g1.ksplit = L.ks1;
  g1.part = L.part1;
  g1.w_kblock = kblock;
  g1.out_f16 = f16;
  g1.w_group = static_cast<int32_t>(a->w_group);
  g1.ws_rows64 = recipe == MI355MOE_RECIPE_FP8BLOCK && a->w13_scale_rows == 64;
  g1.expert_scale = recipe == MI355MOE_RECIPE_BF16 || is_w8a16_recipe(recipe)
                        ? static_cast<const float*>(a->w13_scale)
                        : nullptr;
  if (self_sort) {
    g1.sr_ids = a->topk_ids;
    g1.sr_ids_dtype = a->ids_dtype;
    g1.sr_map = a->expert_map;
    g1.sr_id_bound = id_bound;
    g1.sr_keys = static_cast<int32_t>(E);
    g1.sr_max_padded = L.max_padded;
    g1.sr_max_blocks = L.max_blocks;
    g1.sr_sorted = L.sorted;
    g1.sr_eids = L.eids;
    g1.sr_ntp = L.ntp;
    g1.sr_cum = L.cum;
    g1.sr_inv = L.inv;
    if (fp8 && !preq) g1.sr_x = static_cast<const uint16_t*>(a->hidden_states);
  }
  // decode: w2 writes the output token-major (C3 shapes), or rebuilds its
  // activation rows from the split-K w13 partials (16-bit activations)
  const bool token_w2 = L.token_w2;
  const int64_t per2 = cdiv(cdiv(K2, 128), L.ks2 > 1 ? L.ks2 : 1);
  const bool w2_finishes_w13 = L.tile == TILE_STREAM && L.ks1 > 1 && glu && !fp8 && !mx &&
                               !token_w2 && 16 * per2 * 128 * 2 <= kStreamG1FinBytes &&
                               stream_w2_finishes_w13_enabled();
  g1.partials_only = w2_finishes_w13;
  if (L.khalves) {
    g1.khalves = 1;
    g1.D = L.act16;
  }
  if (glu) {
    rc = launch_tile_gemm(L.tile, L.bm, grecipe, EPI_GLU, (fp8 && !L.khalves) || mx, g1, L.grid_blocks,
                          mx ? static_cast<void*>(L.acts8) : static_cast<void*>(L.acts), st);
    if (rc) return rc;
  } else {
    rc = launch_tile_gemm(L.tile, L.bm, grecipe, EPI_STORE, false, g1, L.grid_blocks, nullptr,
                          st);
    if (rc) return rc;
    const FusedActArgs f{L.g1, L.act, L.acts, L.ntp, L.max_padded, I,
                         clamp16, a->swiglu_limit};
    if (fp8) {
      if (f16) launch_fused_act<true, true>(a->activation, f, st);
      else launch_fused_act<true, false>(a->activation, f, st);
    } else {
      if (f16) launch_fused_act<false, true>(a->activation, f, st);
      else launch_fused_act<false, false>(a->activation, f, st);
    }
    MI_LAUNCH_CHECK();
  }
  if (int m = mark(3)) return m;

  GemmArgs g2{};
  g2.A = L.act;
  g2.lda = L.p2;
  g2.a_scale = fp8 ? L.acts : nullptr;
  g2.a_scale_tld = L.xst ? L.ldp : 0;
  if (mx) {
    g2.a_mxs = L.acts8;
    g2.a_mxs_ld = L.ld2;
    g2.a_scale_tld = L.xs8t ? L.ldp : 0;
  }
  g2.B = a->w2;
  g2.b_scale = a->w2_scale;
  g2.bias = static_cast<const uint16_t*>(a->w2_bias);
  g2.D = L.g2;
  g2.row_ids = L.sorted;
  g2.block_expert = L.eids;
  g2.ntp = L.ntp;
  g2.expert_cum = L.cum;
  g2.num_valid = static_cast<int32_t>(L.slots);
  g2.a_div = 1;
  g2.a_by_pos = 1;
  g2.d_by_pos = 0;
  g2.N = H;
  g2.K = K2;
  g2.ldb_rows = H;
  g2.up_off = 0;
  g2.ksplit = L.ks2;
  g2.part = L.part2;
  g2.w_kblock = kblock;
  g2.out_f16 = f16;
  g2.w_group = static_cast<int32_t>(a->w_group);
  g2.expert_scale = recipe == MI355MOE_RECIPE_BF16 || is_w8a16_recipe(recipe)
                        ? static_cast<const float*>(a->w2_scale)
                        : nullptr;
  if (w2_finishes_w13) {
    g2.g1f.part = L.part1;
    g2.g1f.ks = L.ks1;
    g2.g1f.n_tiles = static_cast<int32_t>(cdiv(I, 128));
    g2.g1f.N = g1.N;
    g2.g1f.up_off = g1.up_off;
    g2.g1f.ldb_rows = g1.ldb_rows;
    g2.g1f.bias = g1.bias;
    g2.g1f.expert_scale = g1.expert_scale;
    g2.g1f.clamp_limit = g1.clamp_limit;
    g2.g1f.alpha = g1.alpha;
    g2.g1f.limit = g1.limit;
    g2.g1f.act = g1.act;
  }
  if (token_w2) {
    if (L.khalves) {  // each wave quantises its slot's 16-bit row
      g2.A = L.act16;
      g2.a_scale = nullptr;
      g2.tok_xq = 1;
    }
    // column-group width: the fewest columns per CU over the rounds of
    // workgroups (256 CUs), the widest group on ties
    {
      const int64_t groups = 8 / k;
      int best = 32;
      int64_t best_cost = cdiv(cdiv(H, 32 * groups) * T, 256) * 32;
      for (int cw = 28; cw >= 16; cw -= 4) {
        const int64_t cost = cdiv(cdiv(H, cw * groups) * T, 256) * cw;
        if (cost < best_cost) {
          best = cw;
          best_cost = cost;
        }
      }
      g2.tok_cw = best;
    }
    g2.tok_inv = L.inv;
    g2.tok_w = a->topk_weights;
    g2.topk = static_cast<int32_t>(k);
    g2.tok_out = a->output;
    rc = launch_tile_gemm(L.tile, L.bm, grecipe, EPI_STORE, false, g2, L.grid_blocks, nullptr,
                          st);
    if (rc) return rc;
    if (int m = mark(4)) return m;
    return mark(5);
  }
  // split-K decode: the partial sums are finished by the top-k reduction
  const bool fuse_reduce = L.tile == TILE_STREAM && L.ks2 > 1 && k <= kFuseMaxTopk;
  g2.partials_only = fuse_reduce;
  rc = launch_tile_gemm(L.tile, L.bm, grecipe, EPI_STORE, false, g2, L.grid_blocks, nullptr, st);
  if (rc) return rc;
  if (int m = mark(4)) return m;
  if (fuse_reduce) {
    dim3 grid(static_cast<unsigned>(cdiv(H, 256)), static_cast<unsigned>(T));
    auto fin = f16 ? finalize_topk_sum_kernel<true> : finalize_topk_sum_kernel<false>;
    fin<<<grid, dim3(256), 0, st>>>(
        static_cast<uint16_t*>(a->output), L.part2, L.ks2, static_cast<int>(cdiv(H, 256)),
        L.inv, L.eids, static_cast<const uint16_t*>(a->w2_bias), g2.expert_scale,
        a->topk_weights, static_cast<int>(k), H);
    MI_LAUNCH_CHECK();
    return mark(5);
  }

  // Slots dropped by the sort (invalid or non-local experts) were never
  // written by the w2 GEMM; the reduction skips them by the same rule.
  dim3 grid(static_cast<unsigned>(cdiv(cdiv(H, 8), 256)), static_cast<unsigned>(T));
  if (a->ids_dtype == MI355MOE_I32) {
    auto red = f16 ? weighted_topk_sum_kernel<int32_t, true>
                   : weighted_topk_sum_kernel<int32_t, false>;
    red<<<grid, dim3(256), 0, st>>>(static_cast<uint16_t*>(a->output), L.g2, a->topk_weights,
                                    static_cast<const int32_t*>(a->topk_ids), a->expert_map,
                                    a->expert_map_len, E, T, (int)k, H);
  } else {
    auto red = f16 ? weighted_topk_sum_kernel<int64_t, true>
                   : weighted_topk_sum_kernel<int64_t, false>;
    red<<<grid, dim3(256), 0, st>>>(static_cast<uint16_t*>(a->output), L.g2, a->topk_weights,
                                    static_cast<const int64_t*>(a->topk_ids), a->expert_map,
                                    a->expert_map_len, E, T, (int)k, H);
  }
  MI_LAUNCH_CHECK();
  return mark(5);
}
}  // namespace
}  // namespace mi355

// ------------------------------------------------------------ grouped GEMM
namespace {
struct GGLayout {
  int bm;
  GemmTile tile;
  int64_t max_padded, max_blocks, grid_blocks;
  int32_t *rows, *eids, *ntp;
  int32_t* cum;     // [E+1] padded row start of every expert
  uint8_t* aq;
  float* as;
  size_t bytes;
};
GGLayout gg_plan(int recipe, bool need_quant, int64_t M, int64_t K, int64_t E,
                 uint8_t* base) {
  GGLayout L{};
  L.tile = pick_tile(recipe, wide_ok_for(recipe, M, 0, K), M, E, &L.bm);
  padded_sizes(M, E, L.bm, L.max_padded, L.max_blocks);
  L.grid_blocks = launch_blocks(M, E, L.bm, L.max_blocks);
  Carver c{base};
  L.rows = c.take<int32_t>(std::max<int64_t>(L.max_padded, 1));
  L.eids = c.take<int32_t>(std::max<int64_t>(L.max_blocks, 1));
  L.ntp = c.take<int32_t>(1);
  L.cum = c.take<int32_t>(E + 1);
  if (need_quant) {
    L.aq = c.take<uint8_t>(M * K);
    L.as = c.take<float>(M * (K / 128));
  }
  L.bytes = c.off + 256;
  (void)recipe;
  return L;
}
}  // namespace

extern "C" size_t mi355moe_grouped_gemm_workspace_size(int64_t total_rows,
                                                       int64_t num_experts) {
  // worst case: the fp8 recipe quantising a 16-bit A; K is not known here, so
  // callers that pass a 16-bit A to the fp8 recipe must use
  // mi355moe_grouped_gemm_workspace_size_k.
  return gg_plan(0, false, total_rows, 0, num_experts, nullptr).bytes;
}

extern "C" size_t mi355moe_grouped_gemm_workspace_size_k(int recipe, int a_dtype,
                                                         int64_t total_rows,
                                                         int64_t K,
                                                         int64_t num_experts) {
  const bool q = recipe == MI355MOE_RECIPE_FP8BLOCK && a_dtype != MI355MOE_FP8E4M3;
  return gg_plan(recipe, q, total_rows, K, num_experts, nullptr).bytes;
}

namespace {
int grouped_gemm_impl(int recipe, const void* A, int a_dtype, const float* a_scale,
                      const void* B, const void* b_scale, int64_t w_group, const void* bias,
                      void* D, int out_dtype, const int32_t* rows_per_expert, int64_t M,
                      int64_t N, int64_t K, int64_t E, void* ws, size_t ws_bytes,
                      void* stream) {
  MI_ARG(M >= 0 && N > 0 && K > 0 && E > 0 && E <= 1024, "invalid GEMM shape");
  MI_ARG(N % 8 == 0, "N must be a multiple of 8");
  MI_ARG(out_dtype == MI355MOE_BF16 || out_dtype == MI355MOE_F16, "output must be 16-bit");
  bool need_quant = false;
  if (recipe == MI355MOE_RECIPE_FP8BLOCK) {
    MI_ARG(N % 128 == 0 && K % 128 == 0, "fp8 block scaling needs N and K % 128 == 0");
    MI_ARG(b_scale != nullptr, "fp8 block scaling needs ptr_B_scale");
    if (a_dtype == MI355MOE_FP8E4M3) {
      MI_ARG(a_scale != nullptr, "e4m3 activations need ptr_A_scale [M, K/128]");
    } else {
      MI_ARG(a_dtype == MI355MOE_BF16 || a_dtype == MI355MOE_F16,
             "activations must be bfloat16, float16 or e4m3");
      need_quant = true;
    }
  } else if (recipe == MI355MOE_RECIPE_INT4) {
    MI_ARG(w_group == 32 || w_group == 64 || w_group == 128 || w_group == 256,
           "int4 group size must be 32, 64, 128 or 256");
    MI_ARG(K % w_group == 0, "int4 needs K % group_size == 0");
    MI_ARG(a_dtype == MI355MOE_BF16 || a_dtype == MI355MOE_F16,
           "int4 activations must be bfloat16 or float16");
    MI_ARG(out_dtype == a_dtype, "int4: the output must have the activation dtype");
    MI_ARG(b_scale != nullptr, "int4 needs group scales");
  } else if (recipe == MI355MOE_RECIPE_MXFP4) {
    MI_ARG(K % 32 == 0, "mxfp4 needs K % 32 == 0");
    MI_ARG(a_dtype == MI355MOE_BF16 || a_dtype == MI355MOE_F16,
           "mxfp4 activations must be bfloat16 or float16");
    MI_ARG(out_dtype == a_dtype, "mxfp4: the output must have the activation dtype");
    MI_ARG(b_scale != nullptr, "mxfp4 needs e8m0 scales");
  } else if (is_w8a16_recipe(recipe)) {
    // row-major [E, N, K] e4m3 / e5m2 weights, f32 scales [E]; the STREAM
    // kernels at any M
    MI_ARG(a_dtype == MI355MOE_BF16 || a_dtype == MI355MOE_F16,
           "per-expert fp8 weights need bfloat16 or float16 activations");
    MI_ARG(out_dtype == a_dtype, "per-expert fp8: the output must have the activation dtype");
    MI_CHECK(K % 32 == 0, MI355MOE_ERR_UNSUPPORTED, "per-expert fp8 weights need K % 32 == 0");
    MI_ARG(b_scale != nullptr, "per-expert fp8 weights need f32 scales [E]");
  } else {
    MI_ARG(recipe == MI355MOE_RECIPE_BF16, "unknown recipe");
    MI_ARG(a_dtype == MI355MOE_BF16 || a_dtype == MI355MOE_F16,
           "16-bit recipe needs bfloat16 or float16 activations (and weights)");
    MI_ARG(out_dtype == a_dtype, "16-bit recipe: the output must have the activation dtype");
    MI_ARG(K % 8 == 0, "K must be a multiple of 8");
  }
  if (M == 0) return MI355MOE_OK;
  GGLayout L = gg_plan(recipe, need_quant, M, K, E, static_cast<uint8_t*>(ws));
  MI_CHECK(ws && ws_bytes >= L.bytes, MI355MOE_ERR_WORKSPACE,
           "workspace too small for grouped_gemm");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = run_segments_to_blocks(rows_per_expert, E, L.bm, L.rows, L.max_padded,
                                  L.eids, L.max_blocks, L.ntp,
                                  static_cast<int32_t>(M), st, L.cum);
  if (rc) return rc;
  const void* Aq = A;
  const float* As = a_scale;
  if (need_quant) {
    rc = mi355moe_per_token_group_fp8_quant(A, a_dtype, L.aq, L.as, M, K, 128,
                                            1e-10f, -448.f, 448.f, 0, st);
    if (rc) return rc;
    Aq = L.aq;
    As = L.as;
  }
  GemmArgs g{};
  g.A = Aq;
  g.a_scale = As;
  g.B = B;
  g.b_scale = b_scale;
  g.bias = static_cast<const uint16_t*>(bias);
  g.D = D;
  g.row_ids = L.rows;
  g.block_expert = L.eids;
  g.ntp = L.ntp;
  g.expert_cum = L.cum;
  g.num_valid = static_cast<int32_t>(M);
  g.a_div = 1;
  g.N = N;
  g.K = K;
  g.ldb_rows = N;
  g.out_f16 = out_dtype == MI355MOE_F16;
  g.expert_scale = recipe == MI355MOE_RECIPE_BF16 || is_w8a16_recipe(recipe)
                       ? static_cast<const float*>(b_scale)
                       : nullptr;
  g.w_group = static_cast<int32_t>(w_group);
  return launch_tile_gemm(L.tile, L.bm, recipe, EPI_STORE, false, g, L.grid_blocks, nullptr, st);
}
}  // namespace

extern "C" int mi355moe_grouped_gemm(int recipe, const void* A, int a_dtype,
                                     const float* a_scale, const void* B,
                                     const void* b_scale, const void* bias,
                                     void* D, int out_dtype,
                                     const int32_t* rows_per_expert,
                                     int64_t M, int64_t N, int64_t K, int64_t E,
                                     void* ws, size_t ws_bytes, void* stream) {
  MI_ARG(recipe != MI355MOE_RECIPE_INT4, "int4 weights: use mi355moe_grouped_gemm_int4");
  return grouped_gemm_impl(recipe, A, a_dtype, a_scale, B, b_scale, 0, bias, D, out_dtype,
                           rows_per_expert, M, N, K, E, ws, ws_bytes, stream);
}

extern "C" int mi355moe_grouped_gemm_int4(const void* A, int a_dtype, const void* B,
                                          const void* b_scale, int64_t group_size,
                                          const void* bias, void* D,
                                          const int32_t* rows_per_expert, int64_t M,
                                          int64_t N, int64_t K, int64_t E, void* ws,
                                          size_t ws_bytes, void* stream) {
  return grouped_gemm_impl(MI355MOE_RECIPE_INT4, A, a_dtype, nullptr, B, b_scale, group_size,
                           bias, D, a_dtype, rows_per_expert, M, N, K, E, ws, ws_bytes,
                           stream);
}

// ------------------------------------------------- K-blocked weight packing
namespace {
// dst[e][kb][n][B bytes] = src[e][n][B kb .. B kb + B); one thread moves one
// 16-byte chunk (cpb chunks per block row), destination-ordered so the
// writes are contiguous.
__global__ __launch_bounds__(256) void pack_kblock_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst,
                                                          int64_t N, int64_t row_chunks,
                                                          int cpb, int64_t chunks) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int c = static_cast<int>(i % cpb);
  const int64_t row = i / cpb;  // (e, kb, n)
  const int64_t n = row % N;
  const int64_t ekb = row / N;
  const int64_t nkb = row_chunks / cpb;
  const int64_t e = ekb / nkb, kb = ekb % nkb;
  dst[i] = src[(e * N + n) * row_chunks + kb * cpb + c];
}
}  // namespace

extern "C" int mi355moe_pack_weights_kblock(const void* src, void* dst, int dtype,
                                            int64_t num_experts, int64_t N, int64_t K,
                                            void* stream) {
  using namespace mi355;
  MI_ARG(dtype == MI355MOE_BF16 || dtype == MI355MOE_F16 || dtype == MI355MOE_FP8E4M3 ||
             dtype == MI355MOE_U8,
         "weights must be 16-bit, e4m3 or packed e2m1 pairs (u8)");
  // bytes per K block: 32 16-bit values, 128 e4m3 values, 32 e2m1 values;
  // K counts values
  const int64_t blk_bytes = dtype == MI355MOE_FP8E4M3 ? 128 : (dtype == MI355MOE_U8 ? 16 : 64);
  const int64_t kblk = dtype == MI355MOE_FP8E4M3 ? 128 : 32;
  MI_ARG(num_experts > 0 && N > 0 && K > 0 && K % kblk == 0,
         "K-blocked packing needs positive sizes and K % 32 == 0 (16-bit, e2m1) or "
         "K % 128 == 0 (e4m3)");
  const int64_t row_bytes = K / kblk * blk_bytes;
  MI_ARG(src && dst && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
             (reinterpret_cast<uintptr_t>(dst) & 15) == 0,
         "weights must be 16-byte aligned");
  const int64_t bytes = num_experts * N * row_bytes;
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  MI_ARG(s0 + bytes <= d0 || d0 + bytes <= s0, "src and dst overlap");
  const int64_t chunks = bytes / 16;
  const int64_t blocks = cdiv(chunks, 256);
  MI_ARG(blocks < (int64_t(1) << 31), "weights too large");
  pack_kblock_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), N, row_bytes / 16,
      static_cast<int>(blk_bytes / 16), chunks);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

namespace {
// dst[e][kb][n] = src[e][n][kb] (bytes), one thread per destination byte.
__global__ __launch_bounds__(256) void pack_scales_kernel(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ dst,
                                                          int64_t N, int64_t KB,
                                                          int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t n = i % N;
  const int64_t ekb = i / N;
  const int64_t e = ekb / KB, kb = ekb % KB;
  dst[i] = src[(e * N + n) * KB + kb];
}
}  // namespace

extern "C" int mi355moe_pack_scales_kblock(const void* src, void* dst, int64_t num_experts,
                                           int64_t N, int64_t kblocks, void* stream) {
  using namespace mi355;
  MI_ARG(num_experts > 0 && N > 0 && kblocks > 0, "scale packing needs positive sizes");
  MI_ARG(src && dst, "null scales");
  const int64_t total = num_experts * N * kblocks;
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  MI_ARG(s0 + total <= d0 || d0 + total <= s0, "src and dst overlap");
  const int64_t blocks = cdiv(total, 256);
  MI_ARG(blocks < (int64_t(1) << 31), "scales too large");
  pack_scales_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), N, kblocks, total);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
