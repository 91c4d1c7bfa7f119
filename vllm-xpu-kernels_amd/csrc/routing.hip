// Routing: softmax / sigmoid top-k and grouped top-k, one 64-lane wavefront
// per token.  Ties always go to the lower expert index (reference:
// csrc/moe/topk.cpp:536-545, csrc/moe/grouped_topk.cpp:36-45).
#include "common.h"

namespace mi355 {
namespace {

constexpr int kWavesPerBlock = 4;

template <typename In>
__device__ __forceinline__ float load_in(const void* p, int64_t i);
template <>
__device__ __forceinline__ float load_in<F32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float load_in<BF16>(const void* p, int64_t i) {
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_in<F16>(const void* p, int64_t i) {
  return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ void store_idx(void* p, int dt, int64_t i, int v) {
  if (dt == MI355MOE_I64)
    static_cast<int64_t*>(p)[i] = v;
  else
    static_cast<int32_t*>(p)[i] = v;  // I32 and U32 share the bit pattern
}

// (value desc, index asc) "is a better than b"
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// One in-row argmax step over (value, aux, index): every lane compares with
// the lane that the DPP control CTRL names inside its row of 16.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& v, float& aux, int& idx) {
  const float ov = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
  const float oa = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(aux), CTRL, 0xF, 0xF, false));
  const int oi = __builtin_amdgcn_update_dpp(0, idx, CTRL, 0xF, 0xF, false);
  if (better(ov, oi, v, idx)) {
    v = ov;
    aux = oa;
    idx = oi;
  }
}

// (value desc, index asc) as one unsigned key, larger = better: the value's
// bits in an order-preserving map (-0 counted as +0, NaN below -inf) above
// the complement of the index.  Distinct entries have distinct keys, so the
// maximum does not depend on the reduction order, and it is the entry that
// `better` prefers to every other.  Key 0 is below every entry.
__device__ __forceinline__ uint64_t desc_key(float v, int idx) {
  uint32_t u = __float_as_uint(v + 0.0f);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (v != v) u = 0u;
  return (static_cast<uint64_t>(u) << 32) | static_cast<uint32_t>(~idx);
}
__device__ __forceinline__ int key_index(uint64_t k) {
  return static_cast<int>(~static_cast<uint32_t>(k));
}
__device__ __forceinline__ float key_value(uint64_t k) {  // non-NaN keys
  const uint32_t u = static_cast<uint32_t>(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
// One DPP step of a 64-bit maximum: lanes of the rows in ROWMASK compare
// with the lane CTRL names (the others keep their own key).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t k) {
  const uint32_t lo = static_cast<uint32_t>(k), hi = static_cast<uint32_t>(k >> 32);
  const uint32_t olo = __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWMASK, 0xF, false);
  const uint32_t ohi = __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWMASK, 0xF, false);
  const uint64_t o = (static_cast<uint64_t>(ohi) << 32) | olo;
  return o > k ? o : k;
}
// Wave-wide maximum key, returned wave-uniform: within each row of 16 lanes
// the quad swaps and the half-row and row mirrors, then lane 15 of rows 0
// and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3
// (row_bcast:31), so lane 63 holds the maximum.  All 64 lanes active.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  k = dpp_max_u64<0xB1, 0xF>(k);   // quad_perm [1,0,3,2]
  k = dpp_max_u64<0x4E, 0xF>(k);   // quad_perm [2,3,0,1]
  k = dpp_max_u64<0x141, 0xF>(k);  // row_half_mirror
  k = dpp_max_u64<0x140, 0xF>(k);  // row_mirror
  k = dpp_max_u64<0x142, 0xA>(k);  // row_bcast:15
  k = dpp_max_u64<0x143, 0xC>(k);  // row_bcast:31
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(k), 63);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(k >> 32), 63);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Wave-wide fmaxf, wave-uniform (the same steps as wave_max_key; fmaxf is
// exact and ignores NaN, so the order does not change the result).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = row16_max(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                           0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                           0x143, 0xC, 0xF, false)));
  return readlane_f32(v, 63);
}

enum GateMode { GATE_SOFTMAX = 0, GATE_SIGMOID = 1, GATE_SOFTPLUS_SQRT = 2 };

// sqrt(softplus(x)) in fp32, softplus(x) = x above 20, else log(1 + e^x)
// (reference csrc/moe/topk_softplus_sqrt_kernels.cpp:233-262, 300-310)
__device__ __forceinline__ float softplus_sqrt(float x) {
  return sqrtf(x > 20.f ? x : logf(1.f + expf(x)));
}

__device__ __forceinline__ int64_t load_id(const void* p, int dt, int64_t i) {
  if (dt == MI355MOE_I64) return static_cast<const int64_t*>(p)[i];
  if (dt == MI355MOE_U32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const int32_t*>(p)[i];
}

// Lane l holds experts e = i*64 + l, i < VPT (coalesced loads).
template <typename In, int VPT, int MODE>
__global__ __launch_bounds__(256) void topk_gating_kernel(
    const void* __restrict__ gating, float* __restrict__ out_w,
    void* __restrict__ out_idx, int idx_dtype, int32_t* __restrict__ out_src,
    const float* __restrict__ bias, int num_tokens, int num_experts, int k,
    int renormalize, float rsf, const void* __restrict__ input_ids,
    const void* __restrict__ tid2eid) {
  constexpr bool SIGMOID = MODE == GATE_SIGMOID;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= num_tokens) return;
  const int64_t base = static_cast<int64_t>(row) * num_experts;
  if constexpr (MODE == GATE_SOFTPLUS_SQRT) {
    if (tid2eid) {
      // hash routing: the experts of the token id are fixed by the table;
      // weights sqrt(softplus) of those logits, non-finite ones 0
      // (topk_softplus_sqrt_kernels.cpp:238-296)
      float wv = 0.f;
      int64_t ex = 0;
      if (lane < k) {
        const int64_t tok = load_id(input_ids, idx_dtype, row);
        ex = load_id(tid2eid, idx_dtype, tok * k + lane);
        if (ex >= 0 && ex < num_experts) {
          wv = softplus_sqrt(load_in<In>(gating, base + ex));
          if (!isfinite(wv)) wv = 0.f;
        }
      }
      const float wsum = wave_sum(lane < k ? wv : 0.f);
      if (lane < k) {
        float scale = rsf;
        if (renormalize) scale /= (wsum > 0.f ? wsum : 1.f);
        const int64_t o = static_cast<int64_t>(row) * k + lane;
        out_w[o] = wv * scale;
        store_idx(out_idx, idx_dtype, o,
                  ex >= 0 && ex < num_experts ? static_cast<int>(ex) : num_experts);
        out_src[o] = lane * num_tokens + row;
      }
      return;
    }
  }

  float p[VPT], sel[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    int e = i * 64 + lane;
    p[i] = e < num_experts ? load_in<In>(gating, base + e) : -INFINITY;
  }
  if constexpr (MODE == GATE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) m = fmaxf(m, p[i]);
    m = wave_max_dpp(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      int e = i * 64 + lane;
      p[i] = e < num_experts ? expf(p[i] - m) : 0.f;
      s += p[i];
    }
    s = wave_sum(s);
    const float r = 1.f / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i) p[i] *= r;
  } else if constexpr (MODE == GATE_SOFTPLUS_SQRT) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) p[i] = softplus_sqrt(p[i]);
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      float sg = 1.f / (1.f + expf(-p[i]));
      // round to the input dtype (csrc/moe/topk.cpp:19-23)
      if constexpr (std::is_same<In, BF16>::value) sg = bf16_to_f32(f32_to_bf16(sg));
      if constexpr (std::is_same<In, F16>::value) sg = f16_to_f32(f32_to_f16(sg));
      p[i] = sg;
    }
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    int e = i * 64 + lane;
    if (e < num_experts)
      sel[i] = bias ? p[i] + bias[e] : p[i];
    else
      sel[i] = -INFINITY;
  }

  // selection keys (experts past E: key 0, never chosen over an expert)
  uint64_t key[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = i * 64 + lane;
    key[i] = e < num_experts ? desc_key(sel[i], e) : 0ull;
  }
  float wsum = 0.f;
  float myw = 0.f;  // lane j < k keeps the j-th weight
  int myid = 0;
  for (int j = 0; j < k; ++j) {
    uint64_t bk = key[0];
    float bp = p[0];
#pragma unroll
    for (int i = 1; i < VPT; ++i)
      if (key[i] > bk) {
        bk = key[i];
        bp = p[i];
      }
    const uint64_t wk = wave_max_key(bk);  // the round's winner, wave-uniform
    const int bi = key_index(wk);
    const int wl = bi & 63;
    bp = readlane_f32(bp, wl);  // the winning lane's best is the winner
    // softplus_sqrt reports the biased value minus the bias, (s + b) - b
    if constexpr (MODE == GATE_SOFTPLUS_SQRT) {
      const float bv = key_value(wk);
      bp = bias ? bv - bias[bi] : bv;
    }
    wsum += bp;
    if (lane == j) {
      myw = bp;
      myid = bi;
    }
    // retire the winner (-inf, so that ties with other -inf entries still go
    // by index; softplus_sqrt: -10000, as its reference kernel, :393-401)
    if (lane == wl) {
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        if (i == (bi >> 6)) key[i] = desc_key(MODE == GATE_SOFTPLUS_SQRT ? -10000.f : -INFINITY, bi);
    }
  }
  if (lane < k) {
    float scale = rsf;
    if (renormalize) scale /= (wsum > 0.f ? wsum : 1.f);
    const int64_t o = static_cast<int64_t>(row) * k + lane;
    out_w[o] = myw * scale;
    store_idx(out_idx, idx_dtype, o, myid);
    out_src[o] = lane * num_tokens + row;
  }
}

template <typename In, int MODE>
int launch_topk(float* w, void* idx, int idt, int32_t* src, const void* g,
                int64_t T, int64_t E, int64_t k, int renorm, const float* bias,
                float rsf, hipStream_t st, const void* input_ids = nullptr,
                const void* tid2eid = nullptr) {
  dim3 grid(static_cast<unsigned>(cdiv(T, kWavesPerBlock))), block(256);
  if (T == 0) return MI355MOE_OK;
#define MI_TOPK_CASE(V)                                                       \
  if (E <= 64 * V) {                                                          \
    hipLaunchKernelGGL((topk_gating_kernel<In, V, MODE>), grid, block, 0,     \
                       st, g, w, idx, idt, src, bias, (int)T, (int)E, (int)k, \
                       renorm, rsf, input_ids, tid2eid);                      \
    MI_LAUNCH_CHECK();                                                        \
    return MI355MOE_OK;                                                       \
  }
  MI_TOPK_CASE(1)
  MI_TOPK_CASE(2)
  MI_TOPK_CASE(4)
  MI_TOPK_CASE(8)
  MI_TOPK_CASE(16)
#undef MI_TOPK_CASE
  return set_error(MI355MOE_ERR_UNSUPPORTED, "num_experts > 1024 is not supported");
}

template <int MODE>
int topk_dispatch(float* w, void* idx, int idt, int32_t* src, const void* g,
                  int gdt, int64_t T, int64_t E, int64_t k, int renorm,
                  const float* bias, float rsf, void* stream,
                  const void* input_ids = nullptr, const void* tid2eid = nullptr) {
  MI_ARG(T >= 0 && E > 0, "invalid num_tokens / num_experts");
  MI_ARG(k > 0 && k <= E && k <= 64, "topk must be in [1, min(num_experts, 64)]");
  MI_ARG(idt == MI355MOE_I32 || idt == MI355MOE_I64 || idt == MI355MOE_U32,
         "topk_indices must be int32, int64 or uint32");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (gdt) {
    case MI355MOE_F32: return launch_topk<F32, MODE>(w, idx, idt, src, g, T, E, k, renorm, bias, rsf, st, input_ids, tid2eid);
    case MI355MOE_BF16: return launch_topk<BF16, MODE>(w, idx, idt, src, g, T, E, k, renorm, bias, rsf, st, input_ids, tid2eid);
    case MI355MOE_F16: return launch_topk<F16, MODE>(w, idx, idt, src, g, T, E, k, renorm, bias, rsf, st, input_ids, tid2eid);
    default: return set_error(MI355MOE_ERR_INVALID, "gating_output must be float32, bfloat16 or float16");
  }
}

// ----------------------------------------------------------------------------
// grouped top-k (DeepSeek-V3 noaux_tc routing).  One wave per token; the
// token's scores and scores_with_bias rows are staged in LDS (no global
// load inside the selection rounds).
//   group score = top1 + top2 of scores_with_bias in the group (fp32 sum,
//                 stored in the input dtype)
//   keep topk_group groups by (score desc, group asc)
//   ids = top-k of scores_with_bias over kept groups (value desc, id asc)
//   w   = scores[id] / (1e-20 + sum) * rsf   (or scores[id] * rsf)
// FUSED: the kernel reads the gating logits and forms the two rows itself,
// as the reference's fused_grouped_topk does with torch ops
// (tests/ops/grouped_topk_op.py:67-92, scoring "sigmoid"):
//   scores = T(sigmoid(x)),  scores_with_bias = T(float(scores) + bias[e])
// with T the input dtype and the sigmoid 1 / (1 + exp(-x)) in fp32.
// ----------------------------------------------------------------------------
constexpr int kMaxGroupedExperts = 1024;

template <typename In>
__device__ __forceinline__ float round_in(float v) {
  if constexpr (std::is_same<In, BF16>::value) return bf16_to_f32(f32_to_bf16(v));
  else if constexpr (std::is_same<In, F16>::value) return f16_to_f32(f32_to_f16(v));
  else return v;
}

// top-2 (t1 >= t2) of two top-2 pairs
__device__ __forceinline__ void merge_top2(float& t1, float& t2, float o1, float o2) {
  if (o1 > t1) {
    t2 = fmaxf(t1, o2);
    t1 = o1;
  } else {
    t2 = fmaxf(t2, o1);
  }
}

// Lane l holds experts e = i * 64 + l, i < VPT, of both rows in registers
// (all loads issued up front); the group scan reads the biased row back
// from LDS once; the k selection rounds run on the registers.
template <typename In, bool FUSED, int VPT>
__global__ __launch_bounds__(256) void grouped_topk_kernel(
    const void* __restrict__ scores, const void* __restrict__ scores_b,
    const float* __restrict__ bias, void* __restrict__ out_v, int32_t* __restrict__ out_i,
    int num_tokens, int num_experts, int n_group, int topk_group, int k, int renormalize,
    float rsf) {
  __shared__ float s_sb[kWavesPerBlock][VPT * 64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWavesPerBlock + wave;
  if (row >= num_tokens) return;  // whole wave exits together
  const int64_t base = static_cast<int64_t>(row) * num_experts;
  float* sb = s_sb[wave];
  float sc[VPT], sv[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = i * 64 + lane;
    const bool in = e < num_experts;
    if constexpr (FUSED) {
      sc[i] = in ? load_in<In>(scores, base + e) : 0.f;
      sv[i] = in && bias ? bias[e] : 0.f;
    } else {
      sc[i] = in ? load_in<In>(scores, base + e) : 0.f;
      sv[i] = in ? load_in<In>(scores_b, base + e) : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = i * 64 + lane;
    if constexpr (FUSED) {
      sc[i] = round_in<In>(1.0f / (1.0f + expf(-sc[i])));
      sv[i] = round_in<In>(sc[i] + sv[i]);
    }
    if (e >= num_experts) sv[i] = -INFINITY;
    sb[e] = sv[i];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const int epg = num_experts / n_group;

  // --- group scores.  When n_group divides 64, lpg = 64 / n_group lanes
  //     share a group (lane l: group l / lpg, members l % lpg + lpg i) and
  //     merge their top-2 pairs with xor shuffles; else lane g < n_group
  //     scans its group alone.
  float gscore = -INFINITY;
  {
    float t1 = -INFINITY, t2 = -INFINITY;
    int lpg = 1;
    if ((64 % n_group) == 0) {
      lpg = 64 / n_group;
      const int gi = lane / lpg, sub = lane % lpg;
      for (int i = sub; i < epg; i += lpg) {
        const float v = sb[gi * epg + i];
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
      for (int m = 1; m < lpg; m <<= 1) {
        const float o1 = __shfl_xor(t1, m, 64), o2 = __shfl_xor(t2, m, 64);
        merge_top2(t1, t2, o1, o2);
      }
    } else if (lane < n_group) {
      for (int i = 0; i < epg; ++i) {
        const float v = sb[lane * epg + i];
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
    }
    // group g's pair now sits in lane g * lpg: move it to lane g
    const int src = lane < n_group ? lane * lpg : 0;
    t1 = __shfl(t1, src, 64);
    t2 = __shfl(t2, src, 64);
    if (lane < n_group) {
      const float sum = round_in<In>((epg >= 2) ? t1 + t2 : t1 + t1);
      gscore = __builtin_isfinite(sum) ? sum : -INFINITY;
    }
  }
  // --- pick topk_group groups: group g (lane g) is kept when fewer than
  //     topk_group groups beat it (score desc, group asc -- the order in
  //     which rounds of argmax would pick them); thr is the score of the
  //     last kept group
  unsigned long long kept = 0ull;
  float thr = -INFINITY;
  {
    int rank = 0;
    for (int j = 0; j < n_group; ++j) {  // uniform
      const float sj = readlane_f32(gscore, j);
      rank += better(sj, j, gscore, lane) ? 1 : 0;
    }
    const bool in = lane < n_group;
    kept = __ballot(in && rank < topk_group);
    const unsigned long long last = __ballot(in && rank == topk_group - 1);
    thr = readlane_f32(gscore, static_cast<int>(__builtin_ctzll(last)));
  }
  const bool proceed = thr != -INFINITY;
  float myv = 0.f;
  int myid = 0;
  if (proceed) {
    float wsum = 1e-20f;
    // candidates: experts of dropped groups and non-finite values become
    // -inf; each round retires its winner (to -inf, as the candidates
    // dropped above)
    uint64_t key[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = i * 64 + lane;
      if (e >= num_experts || !((kept >> (e / epg)) & 1ull) || !__builtin_isfinite(sv[i]))
        sv[i] = -INFINITY;
      key[i] = desc_key(sv[i], e);
    }
    for (int j = 0; j < k; ++j) {
      uint64_t bk = key[0];
      float aux = sc[0];
#pragma unroll
      for (int i = 1; i < VPT; ++i)
        if (key[i] > bk) {
          bk = key[i];
          aux = sc[i];
        }
      const int bi = key_index(wave_max_key(bk));
      aux = readlane_f32(aux, bi & 63);  // the winning lane's best is the winner
      wsum += aux;
      if (lane == j) {
        myv = aux;
        myid = bi;
      }
      if (lane == (bi & 63)) {
#pragma unroll
        for (int i = 0; i < VPT; ++i)
          if (i == (bi >> 6)) key[i] = desc_key(-INFINITY, bi);
      }
    }
    if (lane < k) myv = renormalize ? myv / wsum * rsf : myv * rsf;
  } else if (lane < k) {
    myv = 1.f / k;
    myid = lane;
  }
  if (lane < k) {
    const int64_t o = static_cast<int64_t>(row) * k + lane;
    out_i[o] = myid;
    if constexpr (std::is_same<In, F32>::value)
      static_cast<float*>(out_v)[o] = myv;
    else if constexpr (std::is_same<In, BF16>::value)
      static_cast<uint16_t*>(out_v)[o] = f32_to_bf16(myv);
    else
      static_cast<uint16_t*>(out_v)[o] = f32_to_f16(myv);
  }
}

// Four tokens per wave, one per row of 16 lanes (E = 16 VPT experts, lane
// `sub` of a row holding experts sub * VPT .. sub * VPT + VPT - 1, groups of
// E / n_group experts spanning whole lane chunks, n_group dividing 16, k up
// to 16): every argmax is row-local (four DPP steps over (value, aux,
// index), no cross-row reads), and the four rows run side by side.  Same selection,
// ties and roundings as grouped_topk_kernel.
__device__ __forceinline__ void row_argmax(float& v, float& aux, int& idx) {
  argmax_dpp_step<0xB1>(v, aux, idx);   // quad_perm [1,0,3,2]
  argmax_dpp_step<0x4E>(v, aux, idx);   // quad_perm [2,3,0,1]
  argmax_dpp_step<0x141>(v, aux, idx);  // row_half_mirror
  argmax_dpp_step<0x140>(v, aux, idx);  // row_mirror
}

template <typename In, bool FUSED, int VPT>
__global__ __launch_bounds__(256) void grouped_topk_row16_kernel(
    const void* __restrict__ scores, const void* __restrict__ scores_b,
    const float* __restrict__ bias, void* __restrict__ out_v, int32_t* __restrict__ out_i,
    int num_tokens, int n_group, int topk_group, int k, int renormalize, float rsf) {
  constexpr int E = 16 * VPT;
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int row = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  if ((row & ~3) >= num_tokens) return;  // whole wave exits together
  const bool valid = row < num_tokens;
  const int64_t base = static_cast<int64_t>(valid ? row : 0) * E + sub * VPT;
  float sc[VPT], sv[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    sc[i] = load_in<In>(scores, base + i);
    sv[i] = FUSED ? (bias ? bias[sub * VPT + i] : 0.f) : load_in<In>(scores_b, base + i);
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    if constexpr (FUSED) {
      sc[i] = round_in<In>(1.0f / (1.0f + expf(-sc[i])));
      sv[i] = round_in<In>(sc[i] + sv[i]);
    }
  }
  // --- group scores: lpg = 16 / n_group lanes per group
  const int lpg = 16 / n_group;
  const int grp = sub / lpg;
  float gscore;
  {
    float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const float v = sv[i];
      if (v > t1) {
        t2 = t1;
        t1 = v;
      } else if (v > t2) {
        t2 = v;
      }
    }
    for (int m = 1; m < lpg; m <<= 1) {
      const float o1 = __shfl_xor(t1, m, 64), o2 = __shfl_xor(t2, m, 64);
      merge_top2(t1, t2, o1, o2);
    }
    const float sum = round_in<In>((E / n_group >= 2) ? t1 + t2 : t1 + t1);
    gscore = __builtin_isfinite(sum) ? sum : -INFINITY;
  }
  // --- pick topk_group groups (lanes of one group carry the same pair)
  unsigned kept = 0u;
  float thr = -INFINITY;
  {
    float gv = gscore;
    for (int j = 0; j < topk_group; ++j) {
      float v = gv, aux = 0.f;
      int gi = grp;
      row_argmax(v, aux, gi);
      thr = v;
      kept |= 1u << gi;
      if (grp == gi) gv = -INFINITY;
    }
  }
  const bool proceed = thr != -INFINITY;
  float myv = 0.f;
  int myid = 0;
  if (proceed) {
    float wsum = 1e-20f;
    const bool mine_kept = (kept >> grp) & 1u;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (!mine_kept || !__builtin_isfinite(sv[i])) sv[i] = -INFINITY;
    for (int j = 0; j < k; ++j) {
      float bv = sv[0], aux = sc[0];
      int bi = sub * VPT;
#pragma unroll
      for (int i = 1; i < VPT; ++i)
        if (sv[i] > bv) {   // ids grow with i: ties keep the lower one
          bv = sv[i];
          aux = sc[i];
          bi = sub * VPT + i;
        }
      row_argmax(bv, aux, bi);
      wsum += aux;
      if (sub == j) {
        myv = aux;
        myid = bi;
      }
      if (sub == bi / VPT) {
#pragma unroll
        for (int i = 0; i < VPT; ++i)
          if (i == bi % VPT) sv[i] = -INFINITY;
      }
    }
    if (sub < k) myv = renormalize ? myv / wsum * rsf : myv * rsf;
  } else if (sub < k) {
    myv = 1.f / k;
    myid = sub;
  }
  if (valid && sub < k) {
    const int64_t o = static_cast<int64_t>(row) * k + sub;
    out_i[o] = myid;
    if constexpr (std::is_same<In, F32>::value)
      static_cast<float*>(out_v)[o] = myv;
    else if constexpr (std::is_same<In, BF16>::value)
      static_cast<uint16_t*>(out_v)[o] = f32_to_bf16(myv);
    else
      static_cast<uint16_t*>(out_v)[o] = f32_to_f16(myv);
  }
}

int grouped_topk_launch(bool fused, void* vals, int32_t* ids, const void* scores,
                        const void* scores_b, const float* bias, int dt, int64_t T, int64_t E,
                        int64_t n_group, int64_t topk_group, int64_t k, int renorm, float rsf,
                        void* stream) {
  MI_ARG(E > 0 && E <= kMaxGroupedExperts, "num_experts must be in [1, 1024]");
  MI_ARG(n_group > 0 && n_group <= 32, "n_group must be in [1, 32]");
  MI_ARG(E % n_group == 0, "num_experts must be divisible by n_group");
  MI_ARG(topk_group > 0 && topk_group <= n_group, "topk_group must be in [1, n_group]");
  MI_ARG(k > 0 && k <= 32, "topk must be in [1, 32]");
  MI_ARG(k <= topk_group * (E / n_group), "topk exceeds the experts of the kept groups");
  if (T == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // four tokens per wave where the groups tile the 16 lane chunks, from
  // 2048 tokens on (DeepSeek-V3 shape, fused sigmoid: 9.7 / 13.9 us at 4096 /
  // 8192 tokens against 12.5 / 20.2 one token per wave; below 2048 one token
  // per wave is as fast or faster, 8.6-8.8 against 9.1-9.4 us at 64-1024)
  if (T >= 2048 && E % 16 == 0 && (E == 128 || E == 256 || E == 512) && 16 % n_group == 0 &&
      k <= 16) {
    dim3 grid(static_cast<unsigned>(cdiv(T, 4 * kWavesPerBlock))), block(256);
#define MI_GR2(In, V)                                                                         \
  if (fused)                                                                                  \
    hipLaunchKernelGGL((grouped_topk_row16_kernel<In, true, V>), grid, block, 0, st, scores,  \
                       nullptr, bias, vals, ids, (int)T, (int)n_group, (int)topk_group,       \
                       (int)k, renorm, rsf);                                                  \
  else                                                                                        \
    hipLaunchKernelGGL((grouped_topk_row16_kernel<In, false, V>), grid, block, 0, st, scores, \
                       scores_b, nullptr, vals, ids, (int)T, (int)n_group, (int)topk_group,   \
                       (int)k, renorm, rsf);
#define MI_GR(In)                        \
  if (E == 128) { MI_GR2(In, 8) }        \
  else if (E == 256) { MI_GR2(In, 16) }  \
  else { MI_GR2(In, 32) }
    switch (dt) {
      case MI355MOE_F32: MI_GR(F32) break;
      case MI355MOE_BF16: MI_GR(BF16) break;
      case MI355MOE_F16: MI_GR(F16) break;
      default:
        return set_error(MI355MOE_ERR_INVALID, fused ? "gating_output must be float32, bfloat16 or float16"
                                                     : "scores must be float32, bfloat16 or float16");
    }
#undef MI_GR
#undef MI_GR2
    MI_LAUNCH_CHECK();
    return MI355MOE_OK;
  }
  dim3 grid(static_cast<unsigned>(cdiv(T, kWavesPerBlock))), block(256);
#define MI_GT2(In, V)                                                                      \
  if (fused)                                                                                 \
    hipLaunchKernelGGL((grouped_topk_kernel<In, true, V>), grid, block, 0, st, scores,       \
                       nullptr, bias, vals, ids, (int)T, (int)E, (int)n_group,               \
                       (int)topk_group, (int)k, renorm, rsf);                                \
  else                                                                                       \
    hipLaunchKernelGGL((grouped_topk_kernel<In, false, V>), grid, block, 0, st, scores,      \
                       scores_b, nullptr, vals, ids, (int)T, (int)E, (int)n_group,           \
                       (int)topk_group, (int)k, renorm, rsf);
#define MI_GT(In)                  \
  if (E <= 64) { MI_GT2(In, 1) }   \
  else if (E <= 128) { MI_GT2(In, 2) } \
  else if (E <= 256) { MI_GT2(In, 4) } \
  else if (E <= 512) { MI_GT2(In, 8) } \
  else { MI_GT2(In, 16) }
  switch (dt) {
    case MI355MOE_F32: MI_GT(F32) break;
    case MI355MOE_BF16: MI_GT(BF16) break;
    case MI355MOE_F16: MI_GT(F16) break;
    default:
      return set_error(MI355MOE_ERR_INVALID, fused ? "gating_output must be float32, bfloat16 or float16"
                                                   : "scores must be float32, bfloat16 or float16");
  }
#undef MI_GT
#undef MI_GT2
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace
}  // namespace mi355

using namespace mi355;

extern "C" int mi355moe_topk_softmax(float* w, void* idx, int idt, int32_t* src,
                                     const void* g, int gdt, int64_t T,
                                     int64_t E, int64_t k, int renorm,
                                     const float* bias, void* stream) {
  return topk_dispatch<GATE_SOFTMAX>(w, idx, idt, src, g, gdt, T, E, k, renorm, bias, 1.f, stream);
}

extern "C" int mi355moe_topk_sigmoid(float* w, void* idx, int idt, int32_t* src,
                                     const void* g, int gdt, int64_t T,
                                     int64_t E, int64_t k, int renorm,
                                     const float* bias, float rsf,
                                     void* stream) {
  return topk_dispatch<GATE_SIGMOID>(w, idx, idt, src, g, gdt, T, E, k, renorm, bias, rsf, stream);
}

extern "C" int mi355moe_topk_softplus_sqrt(float* w, void* idx, int idt, int32_t* src,
                                          const void* g, int gdt, int64_t T, int64_t E,
                                          int64_t k, int renorm, float rsf,
                                          const float* correction_bias,
                                          const void* input_ids, const void* tid2eid,
                                          void* stream) {
  // the reference kernel's expert counts (topk_softplus_sqrt_kernels.cpp:538-591)
  MI_ARG(E == 1 || E == 2 || E == 4 || E == 8 || E == 16 || E == 32 || E == 64 || E == 128 ||
             E == 256 || E == 512 || E == 192 || E == 320 || E == 384 || E == 448 || E == 576,
         "Unsupported expert number");
  MI_ARG(!tid2eid || input_ids, "input_ids is required for hash MoE");
  return topk_dispatch<GATE_SOFTPLUS_SQRT>(w, idx, idt, src, g, gdt, T, E, k, renorm,
                                           correction_bias, rsf, stream, input_ids, tid2eid);
}

extern "C" int mi355moe_grouped_topk(void* vals, int32_t* ids, const void* scores,
                                     const void* scores_b, int dt, int64_t T,
                                     int64_t E, int64_t n_group,
                                     int64_t topk_group, int64_t k, int renorm,
                                     float rsf, void* stream) {
  return grouped_topk_launch(false, vals, ids, scores, scores_b, nullptr, dt, T, E, n_group,
                             topk_group, k, renorm, rsf, stream);
}

extern "C" int mi355moe_fused_grouped_topk(void* vals, int32_t* ids, const void* gating_output,
                                           const float* bias, int dt, int64_t T, int64_t E,
                                           int64_t n_group, int64_t topk_group, int64_t k,
                                           int renorm, float rsf, void* stream) {
  return grouped_topk_launch(true, vals, ids, gating_output, nullptr, bias, dt, T, E, n_group,
                             topk_group, k, renorm, rsf, stream);
}
