// Decode grouped GEMM: weight streaming with independent wavefronts.
//
// At decode an expert sees a handful of slots, so the GEMM is a stream over
// the active experts' weights.  A workgroup = 8 wavefronts = 16 sorted slots of
// one expert; every wave owns two 16-row weight sub-tiles (GLU: the gate rows
// and the matching up rows of 16 activation columns; STORE: 32 output columns)
// and walks the whole K range on its own: no LDS and no barrier inside the K
// loop.  Weight fragments are prefetched PD K-stages ahead in VGPRs; the few
// activation rows are read through L1/L2 (every workgroup of the expert reads
// the same rows).  The MFMA A operand is the weight (16 rows n), the B operand
// the activation (16 slots m): lane l holds rows n = 4*(l/16) + r of slot
// m = l%16.  The only barrier is in the fp8 epilogue, which finds the amax of
// each slot's 128 activation columns across the 8 waves.
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int KS = 128;   // K elements per stage
constexpr int WAVES = 8;

__device__ __forceinline__ f32x4 mma_fp8(uint4 a0, uint4 a1, uint4 b0, uint4 b1) {
  i32x8 a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
             (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  i32x8 b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
             (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}
// Per-stage register fragments of one lane.
template <int RECIPE>
struct Frag;
template <>
struct Frag<MI355MOE_RECIPE_FP8BLOCK> {  // 32 e4m3 of the weight row / act row
  uint4 w[2][2];
  uint4 x[2];
  float xs;     // activation scale of the 128-K block
  float ws[2];  // weight-block scales, loaded with the stage (a load issued in
                // the compute step would wait for every prefetched stage)
};
template <>
struct Frag<MI355MOE_RECIPE_BF16> {      // 4 MFMA steps x 8 bf16
  uint4 w[2][4];
  uint4 x[4];
};
template <>
struct Frag<MI355MOE_RECIPE_FP8> {       // 32 fp8 of the weight row (K 32q..32q+31
  uint4 w[2][2];                         // of the stage), 4 MFMA steps x 8 16-bit
  uint4 x[4];                            // activations of the same K
};
template <>
struct Frag<MI355MOE_RECIPE_FP8E5M2> : Frag<MI355MOE_RECIPE_FP8> {};
template <>
struct Frag<MI355MOE_RECIPE_MXFP4> {     // 32 e2m1 + e8m0 of the weight row
  uint4 w[2];
  uint32_t sc[2];                        // scale codes (w4_scale_code)
  uint4 x[4];
};
template <>
struct Frag<MI355MOE_RECIPE_INT4> : Frag<MI355MOE_RECIPE_MXFP4> {};  // 32 int4 + scale
template <>
struct Frag<MI355MOE_RECIPE_MXFP8> {     // 32 e4m3 of the weight / act row + e8m0 codes
  uint4 w[2][2];
  uint32_t ws[2];
  uint4 x[2];
  uint32_t xs;
};
template <>
struct Frag<RECIPE_MX4A4> {              // 32 e2m1 (16 bytes) of each + e8m0 codes
  uint4 w[2];
  uint32_t ws[2];
  uint4 x;
  uint32_t xs;
};

// MX recipes: one 16x16x128 MFMA per stage with the e8m0 codes of both
// operands in the instruction (format 0 e4m3, 4 e2m1), accumulating in c.
// Lane l holds row l % 16, and its code scales K block l / 16 of that row.
// e2m1 operand: K 32q..32q+31 (q = l / 16) in the low four dwords; e4m3
// operand: K 16q..16q+15 in dwords 0-3 and 64+16q..64+16q+15 in dwords 4-7
// (measured with a one-wave probe; the unit-scale fp8 kernels do not care,
// both operands sharing any K order).
template <int FMT>
__device__ __forceinline__ f32x4 mma_mx(uint4 a0, uint4 a1, uint32_t as, uint4 b0, uint4 b1,
                                        uint32_t bs, f32x4 c) {
  i32x8 a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
             (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  i32x8 b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
             (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT, FMT, 0, as, 0, bs);
}

// Routing of at most 16 slots (GemmArgs::sr_ids), run by wave 0 of every
// workgroup: slot i's key is the counting sort's (ids outside [0,
// sr_id_bound) and unmapped ids dropped); rank = number of distinct routed
// experts below its expert, within = earlier slots of the same expert, so
// its sorted position is 16 rank + within (one 16-slot block per expert).
// Fills this block's rows, every slot's position, the experts by rank and
// their count.
__device__ __forceinline__ void route_slots(const GemmArgs& a, int blk, int lane, int* s_arow,
                                            int* s_drow, int* s_pos, int* s_dkey, int* s_nd) {
  constexpr int kNone = 0x7fffffff;
  int key = kNone;
  if (lane < a.num_valid) {
    int64_t v;
    if (a.sr_ids_dtype == MI355MOE_I64) v = static_cast<const int64_t*>(a.sr_ids)[lane];
    else if (a.sr_ids_dtype == MI355MOE_U32) v = static_cast<const uint32_t*>(a.sr_ids)[lane];
    else v = static_cast<const int32_t*>(a.sr_ids)[lane];
    if (v >= 0 && v < a.sr_id_bound) {
      if (a.sr_map) v = a.sr_map[v];
      if (v >= 0 && v < a.sr_keys) key = static_cast<int>(v);
    }
  }
  const bool routed = key != kNone;
  int within = 0;
  bool first = routed;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int kj = __shfl(key, j, 64);
    if (j < lane && kj == key) {
      ++within;
      first = false;
    }
  }
  const uint64_t fm = __ballot(first);
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int kj = __shfl(key, j, 64);
    if (((fm >> j) & 1ull) && kj < key) ++rank;
  }
  if (lane < 16) {
    s_arow[lane] = -1;
    s_drow[lane] = -1;
    s_pos[lane] = routed ? 16 * rank + within : -1;
  }
  if (routed && rank == blk) {
    s_arow[within] = a.a_by_pos ? blk * 16 + within : lane / a.a_div;
    s_drow[within] = a.d_by_pos ? blk * 16 + within : lane;
  }
  if (first) s_dkey[rank] = key;
  if (lane == 0) *s_nd = __popcll(fm);
}

// The counting sort's outputs for the routing above (workgroup (0, 0, 0)):
// sorted ids padded with num_valid, block experts (0 past the routed ones),
// padded expert starts, the padded slot count and every slot's position.
__device__ __forceinline__ void write_routing(const GemmArgs& a, int tid, int nthreads,
                                              const int* s_pos, const int* s_dkey, int nd) {
  for (int64_t p = tid; p < a.sr_max_padded; p += nthreads) a.sr_sorted[p] = a.num_valid;
  for (int64_t b = tid; b < a.sr_max_blocks; b += nthreads)
    a.sr_eids[b] = b < nd ? s_dkey[b] : 0;
  for (int x = tid; x <= a.sr_keys; x += nthreads) {
    int below = 0;
    for (int d = 0; d < nd; ++d) below += s_dkey[d] < x ? 1 : 0;
    a.sr_cum[x] = 16 * below;
  }
  if (tid == 0) *a.sr_ntp = 16 * nd;
  if (tid < a.num_valid) a.sr_inv[tid] = s_pos[tid];
  __syncthreads();  // the padding above is written before the slots below
  if (tid < a.num_valid && s_pos[tid] >= 0 && s_pos[tid] < a.sr_max_padded)
    a.sr_sorted[s_pos[tid]] = tid;
}

template <int RECIPE, int EPI, bool QOUT, int PD, bool F16, bool SELF8 = false,
          bool TOKM = false, bool XL = false, bool KH = false, bool XQ = false>
__global__ __launch_bounds__(512) void moe_gemm_stream_kernel(const GemmArgs a,
                                                              void* __restrict__ qs) {
  constexpr bool kFp8 = RECIPE == MI355MOE_RECIPE_FP8BLOCK;
  constexpr bool kFp4 = RECIPE == MI355MOE_RECIPE_MXFP4 || RECIPE == MI355MOE_RECIPE_INT4;
  constexpr bool kMx8 = RECIPE == MI355MOE_RECIPE_MXFP8;
  constexpr bool kMx4 = RECIPE == RECIPE_MX4A4;
  constexpr bool kMx = kMx8 || kMx4;
  constexpr bool kW8 = is_w8a16_recipe(RECIPE);  // fp8 weights, 16-bit activations
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int XB = (kFp8 || kMx8) ? 1 : 2;  // bytes per activation element (mx4: packed)

  static_assert(!SELF8 || (kFp8 && kGlu), "in-kernel quantisation: fp8block w13");
  static_assert(!TOKM || (!kGlu && !QOUT), "token-major form: STORE w2");
  static_assert(!XL || (!kGlu && !QOUT && !kFp8 && !kMx && !TOKM),
                "activation rows from the w13 partials: 16-bit activation, STORE w2");
  static_assert(!KH || (kGlu && !QOUT && !TOKM && !XL), "K halves: 16-bit GLU w13");
  static_assert(!XQ || (TOKM && kFp8), "per-wave quantisation: token-major fp8block w2");
  using FragT = Frag<RECIPE>;

  __shared__ int s_arow[16];
  __shared__ int s_drow[16];
  __shared__ float s_amax[WAVES][16];
  __shared__ int s_pos[16], s_dkey[16], s_nd;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, q = lane >> 4;
  const int blk = blockIdx.y;
  const int64_t K = a.K, N = a.N;
  int e;
  int tpos = -1;  // token-major: this wave's slot's sorted position (-1: dropped)
  if constexpr (TOKM) {
    tpos = a.tok_inv[static_cast<int64_t>(blockIdx.y) * a.topk + wave % a.topk];
    e = a.block_expert[tpos >= 0 ? tpos / 16 : 0];
  } else if (a.sr_ids && !a.finalize) {  // uniform: this launch sorts the slots itself
    if (wave == 0) route_slots(a, blk, lane, s_arow, s_drow, s_pos, s_dkey, &s_nd);
    __syncthreads();
    const int nd = s_nd;
    if (blockIdx.x == 0 && blk == 0 && blockIdx.z == 0)
      write_routing(a, tid, WAVES * 64, s_pos, s_dkey, nd);
    if (blk >= nd) return;  // uniform
    e = s_dkey[blk];
  } else {
    if (blk * 16 >= *a.ntp) return;  // uniform
    e = a.block_expert[blk];
    if (tid < 16) {
      const int rid = a.row_ids[static_cast<int64_t>(blk) * 16 + tid];
      const bool ok = rid >= 0 && rid < a.num_valid;
      s_arow[tid] = ok ? (a.a_by_pos ? blk * 16 + tid : rid / a.a_div) : -1;
      s_drow[tid] = ok ? (a.d_by_pos ? blk * 16 + tid : rid) : -1;
    }
    __syncthreads();
  }

  // output columns of this wave: GLU 16 activation columns, STORE 32 columns
  // (token-major: the 32 columns of its group, shared by the group's slots;
  // K halves: column group wave % 4 of the workgroup's 64)
  const int tcw = TOKM && a.tok_cw > 0 ? a.tok_cw : 32;  // token-major group width
  const int64_t col0 =
      TOKM ? (static_cast<int64_t>(blockIdx.x) * (WAVES / a.topk) + wave / a.topk) * tcw
      : KH ? static_cast<int64_t>(blockIdx.x) * 64 + (wave & 3) * 16
           : static_cast<int64_t>(blockIdx.x) * (kGlu ? 128 : 256) + wave * (kGlu ? 16 : 32);
  const int64_t wrow_bytes = (kFp4 || kMx4) ? K / 2 : (kW8 ? K : K * XB);
  const uint8_t* wexp = static_cast<const uint8_t*>(a.B) +
                        static_cast<int64_t>(e) * a.ldb_rows * wrow_bytes;
  int64_t wrow[2];
  bool wok[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t n = kGlu ? col0 + l16 : col0 + 16 * t + l16;
    if (TOKM && 16 * t + l16 >= tcw) n = col0 + tcw - 1;
    wok[t] = n < N;
    wrow[t] = (kGlu && t == 1 ? a.up_off : 0) + (wok[t] ? n : 0);
  }
  // weights (and mxfp4 scales) may be K-blocked
  const WStride wst = (kFp4 || kMx4) ? w_stride4(a)
                                     : (kW8 ? w_stride8w(a)
                                            : ((kFp8 || kMx8) ? w_stride8(a) : w_stride16(a)));
  const WStride sst = s_stride4(a);
  const uint8_t* wp0 = wexp + wrow[0] * wst.row;
  const uint8_t* wp1 = wexp + wrow[1] * wst.row;
  const int arow = TOKM ? (l16 == 0 ? tpos : -1) : s_arow[l16];
  const bool xok = arow >= 0;
  const uint8_t* xp = static_cast<const uint8_t*>(a.A) +
                      static_cast<int64_t>(xok ? arow : 0) * (kMx4 ? K / 2 : K * XB);
  const uint8_t* xsp8 = kMx ? a.a_mxs + static_cast<int64_t>(xok ? arow : 0) * a.a_mxs_ld
                            : nullptr;

  // fp8 weight-block scale rows, applied to the MFMA result: the block of
  // the lane's output rows 4 q .. 4 q + 3 of each sub-tile, which share one
  // block (sub-tiles start at multiples of 4 rows; a token-major group of
  // 28 columns puts the block boundary inside a sub-tile)
  const int wsh = 7 - a.ws_rows64;
  const int64_t wsrows = a.ldb_rows >> wsh;
  int64_t wsr[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t n = kGlu ? col0 + 4 * q : col0 + 16 * t + 4 * q;
    wsr[t] = ((kGlu && t == 1 ? a.up_off : 0) + (n < N ? n : 0)) >> wsh;
  }

  const float* bsc = static_cast<const float*>(a.b_scale);
  const int64_t xsrow = static_cast<int64_t>(xok ? arow : 0) * (K / 128);
  // Loads are unconditional and in bounds: rows past N and padding slots read
  // row 0 (their outputs are never stored), the K tail re-reads the last
  // chunk and compute() zeroes it.  A load under a condition would make the
  // compiler wait for every prefetched stage where the branches join.
  // ---- this split's (K halves: this wave's half's) K stages [s0, s0 + nk)
  const int ks = a.ksplit > 1 ? a.ksplit : 1;
  const int nparts = KH ? 2 : ks;
  const int nk_all = static_cast<int>((K + KS - 1) / KS);
  const int per = (nk_all + nparts - 1) / nparts;
  const int s0 = (KH ? (wave >> 2) : static_cast<int>(blockIdx.z)) * per;
  const int nk = a.finalize || (TOKM && tpos < 0) ? 0  // a dropped slot streams nothing
                                                    : ((nk_all - s0) < per ? (nk_all - s0) : per);
  // SELF8: every token row's K range of the split (K halves: the whole K),
  // e4m3, and its 1 x 128 scales in LDS (row pitch xrs bytes)
  __shared__ __attribute__((aligned(16))) uint8_t s_xq[SELF8 ? kStreamSelfXBytes : 16];
  __shared__ float s_xsc[SELF8 ? kStreamSelfXBytes / 128 : 1];
  const int64_t kx0 = KH ? 0 : static_cast<int64_t>(s0) * KS;
  const int xrs = (KH ? nk_all : per) * KS;
  // XQ: each wave's slot row, e4m3, and its 1 x 128 scales
  __shared__ __attribute__((aligned(16))) uint8_t s_tq[XQ ? WAVES * kStreamTokXBytes : 16];
  __shared__ float s_tqs[XQ ? WAVES * (kStreamTokXBytes / 128) : 1];
  // XL: this workgroup's 16 activation rows over the split's K range (16-bit,
  // row pitch xrs elements), rebuilt from the w13 partials below
  __shared__ __attribute__((aligned(16))) uint16_t s_xa[XL ? kStreamG1FinBytes / 2 : 8];
  auto load = [&](FragT& f, int64_t k0) {
    if constexpr (kMx) {  // K % 32 == 0; addresses clamped into range
      // the lane's e8m0 codes: block q of the stage (row l16)
      const int64_t k = k0 + 32 * q;
      const int64_t kb = (k < K ? k : K - 32) / 32;
#pragma unroll
      for (int t = 0; t < 2; ++t)
        f.ws[t] = w4_scale_code<MI355MOE_RECIPE_MXFP4>(a, e, wrow[t], kb, sst);
      f.xs = xsp8[kb];
      if constexpr (kMx8) {
        // e4m3 operand bytes 0-15 hold K 16q..16q+15 of the stage, bytes
        // 16-31 K 64+16q..64+16q+15 (lane groups 0-1 fill scale block 0
        // and 2, groups 2-3 blocks 1 and 3)
        const int64_t h0 = k0 + 16 * q, h1 = k0 + 64 + 16 * q;
        const int64_t c0 = h0 < K ? h0 : K - 16, c1 = h1 < K ? h1 : K - 16;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint8_t* wp = t ? wp1 : wp0;
          f.w[t][0] = *reinterpret_cast<const uint4*>(wp + (c0 >> 7) * wst.kblk + (c0 & 127));
          f.w[t][1] = *reinterpret_cast<const uint4*>(wp + (c1 >> 7) * wst.kblk + (c1 & 127));
        }
        f.x[0] = *reinterpret_cast<const uint4*>(xp + c0);
        f.x[1] = *reinterpret_cast<const uint4*>(xp + c1);
      } else {
        // e2m1: the lane's 32 values are K 32q..32q+31 of the stage
#pragma unroll
        for (int t = 0; t < 2; ++t)
          f.w[t] = *reinterpret_cast<const uint4*>((t ? wp1 : wp0) + kb * wst.kblk);
        f.x = *reinterpret_cast<const uint4*>(xp + kb * 16);
      }
    } else if constexpr (kFp8) {  // K % 128 == 0: no tail
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint8_t* p = (t ? wp1 : wp0) + (k0 >> 7) * wst.kblk + 32 * q;
        f.w[t][0] = *reinterpret_cast<const uint4*>(p);
        f.w[t][1] = *reinterpret_cast<const uint4*>(p + 16);
        f.ws[t] = bsc[(static_cast<int64_t>(e) * wsrows + wsr[t]) * (K / 128) + k0 / 128];
      }
      if constexpr (SELF8 || XQ) {
        // the activation in LDS, read by compute(): the first stages'
        // weights are requested before it is quantised
      } else {
        const uint8_t* px = xp + k0 + 32 * q;
        f.x[0] = *reinterpret_cast<const uint4*>(px);
        f.x[1] = *reinterpret_cast<const uint4*>(px + 16);
        f.xs = a.a_scale[xsrow + k0 / 128];
      }
    } else if constexpr (kW8) {  // K % 32 == 0: a lane's 32 K values lie in or past K
      const int64_t k = k0 + 32 * q;
      const int64_t kc = k < K ? k : K - 32;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint8_t* p = (t ? wp1 : wp0) + (kc >> 5) * wst.kblk;  // one 32-byte K block
        f.w[t][0] = *reinterpret_cast<const uint4*>(p);
        f.w[t][1] = *reinterpret_cast<const uint4*>(p + 16);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
        f.x[s] = XL ? *reinterpret_cast<const uint4*>(s_xa + l16 * xrs + (kc - kx0) + 8 * s)
                    : *reinterpret_cast<const uint4*>(xp + (kc + 8 * s) * 2);
    } else if constexpr (kFp4) {  // K % 32 == 0
      const int64_t k = k0 + 32 * q;
      const int64_t kc = k < K ? k : K - 32;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f.w[t] = *reinterpret_cast<const uint4*>((t ? wp1 : wp0) + (kc / 32) * wst.kblk);
        f.sc[t] = w4_scale_code<RECIPE>(a, e, wrow[t], kc / 32, sst);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
        f.x[s] = XL ? *reinterpret_cast<const uint4*>(s_xa + l16 * xrs + (kc - kx0) + 8 * s)
                    : *reinterpret_cast<const uint4*>(xp + (kc + 8 * s) * 2);
    } else {  // K % 8 == 0
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int64_t k = k0 + 32 * s + 8 * q;
        const int64_t kc = k + 8 <= K ? k : K - 8;
#pragma unroll
        for (int t = 0; t < 2; ++t)
          f.w[t][s] = *reinterpret_cast<const uint4*>((t ? wp1 : wp0) + w_koff16(wst, kc));
        f.x[s] = XL ? *reinterpret_cast<const uint4*>(s_xa + l16 * xrs + (kc - kx0))
                    : *reinterpret_cast<const uint4*>(xp + kc * 2);
      }
    }
  };

  f32x4 acc[2];
  acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
  acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const FragT& fin, int64_t k0) {
    FragT f = fin;
    if (!kMx && k0 + KS > K) {  // the last stage of a K that is not a multiple of 128
      const uint4 z4 = make_uint4(0, 0, 0, 0);
      if constexpr (kFp4) {
        if (k0 + 32 * q >= K) {
          f.w[0] = f.w[1] = z4;
          f.sc[0] = f.sc[1] = 0u;
        }
      } else if constexpr (kW8) {
        if (k0 + 32 * q >= K) f.w[0][0] = f.w[0][1] = f.w[1][0] = f.w[1][1] = z4;
      } else if constexpr (!kFp8 && !kMx) {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
          if (k0 + 32 * s2 + 8 * q + 8 > K) f.w[0][s2] = f.w[1][s2] = z4;
      }
    }
    if constexpr (kMx) {
      // past K (last stage of a K % 128 != 0): zero weights, unit scales
      const uint4 z4 = make_uint4(0, 0, 0, 0);
      const bool slive = k0 + 32 * q < K;  // this lane's scale block
      const uint32_t xs = slive ? f.xs : 127u;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t ws = slive ? f.ws[t] : 127u;
        if constexpr (kMx8) {
          const bool live0 = k0 + 32 * (q >> 1) < K, live1 = k0 + 64 + 32 * (q >> 1) < K;
          acc[t] = mma_mx<0>(live0 ? f.w[t][0] : z4, live1 ? f.w[t][1] : z4, ws, f.x[0], f.x[1],
                             xs, acc[t]);
        } else {
          acc[t] = mma_mx<4>(slive ? f.w[t] : z4, z4, ws, f.x, z4, xs, acc[t]);
        }
      }
    } else if constexpr (kFp8) {
      if constexpr (SELF8) {
        const int64_t kk = k0 - kx0;
        const uint8_t* px = s_xq + (xok ? arow : 0) * xrs + kk + 32 * q;
        f.x[0] = *reinterpret_cast<const uint4*>(px);
        f.x[1] = *reinterpret_cast<const uint4*>(px + 16);
        f.xs = s_xsc[(xok ? arow : 0) * (xrs / 128) + kk / 128];
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4 p = mma_fp8(f.w[t][0], f.w[t][1], f.x[0], f.x[1]);
        acc[t] += p * (f.xs * f.ws[t]);
      }
    } else if constexpr (kFp4) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 w = f.w[t];
        const uint32_t c = f.sc[t];
        acc[t] = mfma16_16x16x32<F16>(w4_decode8<RECIPE, F16>(w.x, c), f.x[0], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(w4_decode8<RECIPE, F16>(w.y, c), f.x[1], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(w4_decode8<RECIPE, F16>(w.z, c), f.x[2], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(w4_decode8<RECIPE, F16>(w.w, c), f.x[3], acc[t]);
      }
    } else if constexpr (kW8) {
      constexpr bool k52 = RECIPE == MI355MOE_RECIPE_FP8E5M2;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 a0 = f.w[t][0], a1 = f.w[t][1];
        acc[t] = mfma16_16x16x32<F16>(fp8x8_to16<k52, F16>(make_uint2(a0.x, a0.y)), f.x[0], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(fp8x8_to16<k52, F16>(make_uint2(a0.z, a0.w)), f.x[1], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(fp8x8_to16<k52, F16>(make_uint2(a1.x, a1.y)), f.x[2], acc[t]);
        acc[t] = mfma16_16x16x32<F16>(fp8x8_to16<k52, F16>(make_uint2(a1.z, a1.w)), f.x[3], acc[t]);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t] = mfma16_16x16x32<F16>(f.w[t][s], f.x[s], acc[t]);
    }
  };

  // ---- K loop, PD stages in flight
  FragT buf[PD];
  // XQ: the stage's activation operand from the wave's quantised row in LDS,
  // read as the stage is prefetched (PD stages ahead of its MFMAs)
  auto ldsx = [&](FragT& f, int64_t k0) {
    if constexpr (XQ) {
      const uint8_t* px = s_tq + wave * kStreamTokXBytes + k0 + 32 * q;
      f.x[0] = *reinterpret_cast<const uint4*>(px);
      f.x[1] = *reinterpret_cast<const uint4*>(px + 16);
      f.xs = s_tqs[wave * (kStreamTokXBytes / 128) + k0 / 128];
    }
  };
  auto prefetch = [&]() {
    if (nk > 0) {
#pragma unroll
      for (int d = 0; d < PD; ++d)
        load(buf[d], static_cast<int64_t>(s0 + (d < nk ? d : nk - 1)) * KS);
    }
  };
  if constexpr (SELF8) {
    prefetch();  // the weights of the first stages, in flight while the tile is quantised
    // quantise the tile with the group quantiser itself: 16 lanes (8 values
    // each) per 128-value block; the trip count is uniform, lanes past the
    // end take part in the shuffles and store nothing
    const int T = a.num_valid / a.a_div;
    const int cpr = (KH ? nk_all : nk) * 16;  // 8-value chunks of a row in this split
    const int nch = T * cpr;
    for (int base = 0; base < nch; base += WAVES * 64) {
      const int i = base + tid;
      const bool act = i < nch;
      const int r = act ? i / cpr : 0;
      fp8_quant_block8<F16>(a.sr_x + static_cast<int64_t>(r) * K + kx0, s_xq + r * xrs,
                            s_xsc + r * (xrs / KS), act ? i % cpr : cpr, cpr);
    }
    __syncthreads();
  }
  if constexpr (XQ) {
    prefetch();  // the weights of the first stages, in flight while the row is quantised
    if (nk > 0) {  // wave-uniform: a kept slot
      // the group quantiser over the wave's 16-bit row: 16 lanes (8 values
      // each) per 128-value block, all 64 lanes in every round
      // (every round's load in flight before the first is used)
      constexpr int R = kStreamTokXBytes / 512;  // rounds of 64 chunks
      const uint16_t* xr = static_cast<const uint16_t*>(a.A) + static_cast<int64_t>(tpos) * K;
      const int cpr = static_cast<int>(K / 8);
      uint4 u[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = 64 * r + lane;
        u[r] = *reinterpret_cast<const uint4*>(xr + 8 * (c < cpr ? c : 0));
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = 64 * r + lane;
        if (64 * r < cpr)  // uniform
          fp8_quant_regs<F16>(u[r], s_tq + wave * kStreamTokXBytes,
                              s_tqs + wave * (kStreamTokXBytes / 128), c < cpr ? c : cpr, cpr);
      }
      // the row is read back by other lanes of the same wave
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
      for (int d = 0; d < PD; ++d) ldsx(buf[d], static_cast<int64_t>(s0 + (d < nk ? d : nk - 1)) * KS);
    }
  }
  if constexpr (XL) {
    // the w13 finalize of this block's valid slots on the split's columns:
    // its partial tiles summed in split order, then its GLU epilogue (the
    // finalize launch's operations; 4 columns per item)
    const G1Fin& g = a.g1f;
    const int n4 = nk * KS / 4;
    const float es1 = g.expert_scale ? g.expert_scale[e] : 1.f;
    const int64_t bb = static_cast<int64_t>(e) * g.ldb_rows;
    for (int it = tid; it < 16 * n4; it += WAVES * 64) {
      const int m = it / n4, c4 = it - m * n4;
      if (s_arow[m] < 0) continue;  // padding slot: its outputs are never stored
      const int64_t c = kx0 + 4 * c4;
      const int tid13 = static_cast<int>((c % 128) / 16) * 64 + static_cast<int>((c % 16) / 4) * 16 + m;
      const float* tp = g.part + (static_cast<int64_t>(blk) * g.n_tiles + c / 128) * g.ks * 4096 +
                        8 * tid13;
      float gv[4] = {0.f, 0.f, 0.f, 0.f}, uv[4] = {0.f, 0.f, 0.f, 0.f};
      for (int z = 0; z < g.ks; ++z) {
        const float4 g4 = *reinterpret_cast<const float4*>(tp + z * 4096);
        const float4 u4 = *reinterpret_cast<const float4*>(tp + z * 4096 + 4);
        gv[0] += g4.x; gv[1] += g4.y; gv[2] += g4.z; gv[3] += g4.w;
        uv[0] += u4.x; uv[1] += u4.y; uv[2] += u4.z; uv[3] += u4.w;
      }
      uint32_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = c + r;
        const bool nok = n < g.N;
        float v = gv[r] * es1;
        if (g.bias && nok) v += ld16<F16>(g.bias[bb + n]);
        v = rnd16<F16>(v);
        float u = uv[r] * es1;
        if (g.bias && nok) u += ld16<F16>(g.bias[bb + g.up_off + n]);
        u = rnd16<F16>(u);
        glu_clamp_with(g.clamp_limit, g.act, g.N, n, v, u);
        v = rnd16<F16>(glu16<F16>(v, u, g.act, g.alpha, g.limit));
        o[r] = st16<F16>(nok ? v : 0.f);
      }
      *reinterpret_cast<uint2*>(s_xa + m * xrs + 4 * c4) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    }
    __syncthreads();
  }
  if constexpr (!SELF8 && !XQ) prefetch();
  int kt = 0;
  // main part: every prefetch is in range, so no load sits in a branch
  for (; kt + 2 * PD <= nk; kt += PD) {
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      compute(buf[d], static_cast<int64_t>(s0 + kt + d) * KS);
      load(buf[d], static_cast<int64_t>(s0 + kt + d + PD) * KS);
      ldsx(buf[d], static_cast<int64_t>(s0 + kt + d + PD) * KS);
    }
  }
  // remainder: fewer than 2 PD stages
  for (; kt < nk; kt += PD) {
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      const int k = kt + d;
      if (k < nk) {
        compute(buf[d], static_cast<int64_t>(s0 + k) * KS);
        if (k + PD < nk) {
          load(buf[d], static_cast<int64_t>(s0 + k + PD) * KS);
          ldsx(buf[d], static_cast<int64_t>(s0 + k + PD) * KS);
        }
      }
    }
  }

  // ---- K halves: the upper half's sums join the lower half's (the split-K
  //      finalize's order: half 0, then half 1); the lower waves go on
  if constexpr (KH) {
    __shared__ f32x4 s_kh[4][2][64];
    if (wave >= 4) {
      s_kh[wave - 4][0][lane] = acc[0];
      s_kh[wave - 4][1][lane] = acc[1];
    }
    __syncthreads();
    if (wave >= 4) return;
    acc[0] += s_kh[wave][0][lane];
    acc[1] += s_kh[wave][1][lane];
  }
  // ---- split-K: the split launch leaves its partial tile; the finalize
  //      launch sums the partials in split order (bit-reproducible)
  if (ks > 1) {
    const int64_t tile_id = static_cast<int64_t>(blk) * gridDim.x + blockIdx.x;
    if (!a.finalize) {
      float4* mine = reinterpret_cast<float4*>(a.part + (tile_id * ks + blockIdx.z) * (512 * 8)) + 2 * tid;
      mine[0] = make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
      mine[1] = make_float4(acc[1][0], acc[1][1], acc[1][2], acc[1][3]);
      return;
    }
    for (int z = 0; z < ks; ++z) {
      const float4* p = reinterpret_cast<const float4*>(a.part + (tile_id * ks + z) * (512 * 8)) + 2 * tid;
      const float4 v0 = p[0], v1 = p[1];
      acc[0] += f32x4{v0.x, v0.y, v0.z, v0.w};
      acc[1] += f32x4{v1.x, v1.y, v1.z, v1.w};
    }
  }

  // ---- epilogue: lane holds slot m = l16, columns col0 + 4q + r
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  const float es = a.expert_scale ? a.expert_scale[e] : 1.f;
  const int drow = s_drow[l16];
  constexpr int NO = kGlu ? 1 : 2;
  float ov[NO][4];
#pragma unroll
  for (int t = 0; t < NO; ++t) {
    const int64_t n = col0 + 16 * t + 4 * q;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool nok = n + r < N;
      float v = acc[t][r] * es;
      if (a.bias && nok) v += ld16<F16>(a.bias[bias_base + n + r]);
      v = rnd16<F16>(v);
      if constexpr (kGlu) {
        float u = acc[1][r] * es;
        if (a.bias && nok) u += ld16<F16>(a.bias[bias_base + a.up_off + n + r]);
        u = rnd16<F16>(u);
        glu_clamp(a, n + r, v, u);
        v = rnd16<F16>(glu16<F16>(v, u, a.act, a.alpha, a.limit));
      }
      ov[t][r] = nok ? v : 0.f;
    }
  }
  if constexpr (TOKM) {
    // the group's slots summed in j order: the top-k reduction's arithmetic
    // on the rounded slot values (lane l16 = 0 holds this wave's slot)
    __shared__ float s_tok[WAVES][32];
    if (l16 == 0) {
#pragma unroll
      for (int t = 0; t < NO; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_tok[wave][16 * t + 4 * q + r] = ov[t][r];
    }
    __syncthreads();
    if (wave % a.topk != 0 || lane >= tcw || col0 + lane >= N) return;
    const int64_t t = blockIdx.y;
    float acc1 = 0.f;
    for (int j = 0; j < a.topk; ++j) {
      const int64_t slot = t * a.topk + j;
      if (a.tok_inv[slot] < 0) continue;
      const float wj = a.tok_w[slot];
      acc1 += wj * s_tok[wave + j][lane];
    }
    static_cast<uint16_t*>(a.tok_out)[t * N + col0 + lane] = st16<F16>(acc1);
  } else if constexpr (QOUT && kMx) {
    // MX activation for the w2 GEMM, one e8m0 scale per 32 columns (the
    // output columns of waves 2p and 2p + 1): mxfp8 as per_token_group_fp8_quant
    // with ue8m0 scales, mxfp4 as per_token_group_quant_mxfp4 (eps 1e-10)
    float m = 1e-10f;
#pragma unroll
    for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(ov[0][r]));
    m = max_over_rows(m);
    if (q == 0) s_amax[wave][l16] = m;
    __syncthreads();
    if (drow < 0) return;
    const float am = fmaxf(s_amax[wave & ~1][l16], s_amax[wave | 1][l16]);
    int ex;
    if constexpr (kMx8) ex = ceil_log2(fmaxf(fabsf(fmaxf(am / 448.f, 1.0f / (448.f * 512.f))), 1e-10f));
    else ex = ceil_log2(fmaxf(fabsf(am / 6.0f), 1e-10f));
    const float inv = 1.0f / pow2i(ex);
    // N % 32 == 0: a lane's 4 columns, and a wave pair's 32, lie wholly
    // inside or wholly past N (the last column tile of an N % 128 != 0)
    if (col0 + 4 * q >= N) return;
    if ((wave & 1) == 0 && q == 0)
      static_cast<uint8_t*>(qs)[static_cast<int64_t>(drow) * a.q_mxs_ld + col0 / 32] =
          static_cast<uint8_t>(ex + 127);
    if constexpr (kMx8) {
      const uint32_t w =
          e4m3x4_sat(ov[0][0] * inv, ov[0][1] * inv, ov[0][2] * inv, ov[0][3] * inv);
      *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.D) + static_cast<int64_t>(drow) * N +
                                   col0 + 4 * q) = w;
    } else {
      // (ov holds 16-bit values, inv is a power of two)
      const uint32_t w = fp4x4_code16(ov[0][0], ov[0][1], ov[0][2], ov[0][3], fp4_prescale(inv));
      *reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(a.D) + static_cast<int64_t>(drow) * (N / 2) +
                                   (col0 + 4 * q) / 2) = static_cast<uint16_t>(w);
    }
  } else if constexpr (QOUT) {
    float m = 1e-10f;
#pragma unroll
    for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(ov[0][r]));
    m = max_over_rows(m);
    if (q == 0) s_amax[wave][l16] = m;
    __syncthreads();
    if (drow < 0) return;
    float am = s_amax[0][l16];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) am = fmaxf(am, s_amax[w][l16]);
    const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
    const float inv = 1.0f / sc;
    if (wave == 0 && q == 0)
      static_cast<float*>(qs)[static_cast<int64_t>(drow) * (N / 128) + blockIdx.x] = sc;
    const uint32_t w =
        e4m3x4_sat(ov[0][0] * inv, ov[0][1] * inv, ov[0][2] * inv, ov[0][3] * inv);
    *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.D) + static_cast<int64_t>(drow) * N +
                                 col0 + 4 * q) = w;
  } else {
    if (drow < 0) return;
    uint16_t* d = static_cast<uint16_t*>(a.D);
#pragma unroll
    for (int t = 0; t < NO; ++t) {
      const int64_t n = col0 + 16 * t + 4 * q;
      uint16_t h[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) h[r] = st16<F16>(ov[t][r]);
      uint16_t* dst = d + static_cast<int64_t>(drow) * N + n;
      if (n + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<uint2*>(dst) =
            make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) dst[r] = h[r];
      }
    }
  }
}

template <int RECIPE, int EPI, bool QOUT, bool F16>
int launch_stream_t(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  constexpr int PD = 2;  // stages in flight per wave (deeper costs occupancy, measured no faster)
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  dim3 grid(static_cast<unsigned>(cdiv(a.N, cols)), static_cast<unsigned>(max_blocks),
            static_cast<unsigned>(a.ksplit > 1 ? a.ksplit : 1));
  GemmArgs g = a;
  g.finalize = 0;
  if constexpr (EPI == EPI_STORE && !QOUT && RECIPE != MI355MOE_RECIPE_FP8BLOCK &&
                !is_mx_recipe(RECIPE)) {
    if (a.g1f.part) {  // activation rows rebuilt from the w13 partials
      moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, false, false, true>
          <<<grid, dim3(512), 0, st>>>(g, qs);
      MI_LAUNCH_CHECK();
      if (a.ksplit > 1 && !a.partials_only) {
        grid.z = 1;
        g.finalize = 1;
        g.g1f.part = nullptr;
        moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16><<<grid, dim3(512), 0, st>>>(g, qs);
        MI_LAUNCH_CHECK();
      }
      return MI355MOE_OK;
    }
  }
  if constexpr (EPI == EPI_STORE && !QOUT) {
    if (a.tok_out) {  // token-major w2: the output itself, no split
      const int groups = WAVES / a.topk;
      const int cw = a.tok_cw > 0 ? a.tok_cw : 32;
      const dim3 tg(static_cast<unsigned>(cdiv(a.N, static_cast<int64_t>(cw) * groups)),
                    static_cast<unsigned>(a.num_valid / a.topk), 1);
      if constexpr (RECIPE == MI355MOE_RECIPE_FP8BLOCK) {
        if (a.tok_xq) {  // each wave quantises its 16-bit activation row
          moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, false, true, false, false, true>
              <<<tg, dim3(512), 0, st>>>(g, qs);
          MI_LAUNCH_CHECK();
          return MI355MOE_OK;
        }
      }
      moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, false, true><<<tg, dim3(512), 0, st>>>(g, qs);
      MI_LAUNCH_CHECK();
      return MI355MOE_OK;
    }
  }
  if constexpr (RECIPE == MI355MOE_RECIPE_FP8BLOCK && EPI == EPI_GLU && !QOUT) {
    if (a.khalves) {  // 64 activation columns x both K halves per workgroup, no split
      const dim3 kg(static_cast<unsigned>(cdiv(a.N, 64)), static_cast<unsigned>(max_blocks), 1);
      if (a.sr_x)
        moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, true, false, false, true>
            <<<kg, dim3(512), 0, st>>>(g, qs);
      else
        moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, false, false, false, true>
            <<<kg, dim3(512), 0, st>>>(g, qs);
      MI_LAUNCH_CHECK();
      return MI355MOE_OK;
    }
  }
  if constexpr (RECIPE == MI355MOE_RECIPE_FP8BLOCK && EPI == EPI_GLU) {
    if (a.sr_x)
      moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16, true><<<grid, dim3(512), 0, st>>>(g, qs);
    else
      moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16><<<grid, dim3(512), 0, st>>>(g, qs);
  } else {
    moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16><<<grid, dim3(512), 0, st>>>(g, qs);
  }
  MI_LAUNCH_CHECK();
  if (a.ksplit > 1 && !a.partials_only) {  // sum the partial tiles and run the epilogue
    // (the routing is read back from what the split launch wrote)
    grid.z = 1;
    g.finalize = 1;
    moe_gemm_stream_kernel<RECIPE, EPI, QOUT, PD, F16><<<grid, dim3(512), 0, st>>>(g, qs);
    MI_LAUNCH_CHECK();
  }
  return MI355MOE_OK;
}
template <int RECIPE, int EPI, bool QOUT>
int launch_stream(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  return a.out_f16 ? launch_stream_t<RECIPE, EPI, QOUT, true>(a, max_blocks, qs, st)
                   : launch_stream_t<RECIPE, EPI, QOUT, false>(a, max_blocks, qs, st);
}

}  // namespace

int stream_ksplit(int64_t n_tiles, int64_t blocks, int64_t K) {
  // split only grids that leave most CUs idle (the partial-sum launch costs a
  // few microseconds); then aim for about 256 workgroups (one per CU; 512
  // and more measured 2-6% slower at decode: C2 / C5 T=1 46.3 / 44.7 us at
  // 512, 43.9 / 42.0 at 256, C3 T=1 equal), at most 8 splits and at least
  // two K stages per split
  const int64_t wgs = n_tiles * (blocks > 0 ? blocks : 1);
  if (wgs >= 192) return 1;
  int64_t s = 256 / (wgs > 0 ? wgs : 1);
  const int64_t nk = cdiv(K, KS);
  if (s > 8) s = 8;
  if (s > nk / 2) s = nk / 2;
  if (s < 2) return 1;
  const int64_t per = cdiv(nk, s);
  return static_cast<int>(cdiv(nk, per));  // no empty split
}

// 16-slot blocks (the caller aligns expert segments to 16).
int launch_moe_gemm_stream(int recipe, int epi, bool qout, const GemmArgs& a,
                           int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  if (qout) {
    MI_ARG(epi == EPI_GLU, "quantised activation output needs the GLU epilogue");
    if (recipe == MI355MOE_RECIPE_MXFP8) {
      MI_ARG(a.N % 32 == 0, "mxfp8 activation output needs I % 32 == 0");
      return launch_stream<MI355MOE_RECIPE_MXFP8, EPI_GLU, true>(a, max_blocks, qs, st);
    }
    if (recipe == RECIPE_MX4A4) {
      MI_ARG(a.N % 32 == 0, "mxfp4 activation output needs I % 32 == 0");
      return launch_stream<RECIPE_MX4A4, EPI_GLU, true>(a, max_blocks, qs, st);
    }
    MI_ARG(recipe == MI355MOE_RECIPE_FP8BLOCK && a.N % 128 == 0,
           "fp8 activation output needs the fp8block recipe and I % 128 == 0");
    return launch_stream<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, true>(a, max_blocks, qs, st);
  }
  switch (recipe) {
    case MI355MOE_RECIPE_BF16:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_BF16, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_BF16, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_FP8BLOCK:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_FP8BLOCK, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_MXFP4:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_MXFP4, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_MXFP4, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_INT4:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_INT4, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_INT4, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_MXFP8:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_MXFP8, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_MXFP8, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_FP8:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_FP8, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_FP8, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_FP8E5M2:
      return epi == EPI_GLU ? launch_stream<MI355MOE_RECIPE_FP8E5M2, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<MI355MOE_RECIPE_FP8E5M2, EPI_STORE, false>(a, max_blocks, qs, st);
    case RECIPE_MX4A4:
      return epi == EPI_GLU ? launch_stream<RECIPE_MX4A4, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_stream<RECIPE_MX4A4, EPI_STORE, false>(a, max_blocks, qs, st);
    default:
      return set_error(MI355MOE_ERR_INVALID, "unknown recipe");
  }
}

}  // namespace mi355
