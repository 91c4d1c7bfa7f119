// Grouped GEMM over block-aligned expert segments on gfx950 MFMA.
//
// Layout of one workgroup (256 threads = 4 wavefronts): BM sorted slots of a
// single expert x BN output columns; wave w owns columns [w*BN/4, (w+1)*BN/4)
// for all BM rows.  The MFMA's A operand is the expert weight fragment (16
// output columns, loaded straight from HBM into VGPRs: weights are streamed
// exactly once per workgroup) and its B operand is the activation fragment
// (16 slots, staged in LDS and shared by the 4 waves), so every lane ends up
// holding 4 consecutive output columns of one slot row.
//
//   bf16     v_mfma_f32_16x16x32_bf16 (fp16 calls: _f16), K stage 128 (4
//            MFMA steps)
//   fp8block v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 x e4m3, unit scales), one
//            MFMA per 128-wide K block; the fp32 block scales of the weight
//            (128x128) and activation (1x128) multiply its partial sum.
//   mxfp4    e2m1 weights converted in registers to the call's 16-bit type
//            with their e8m0 scale (v_cvt_scalef32_pk_{bf16,f16}_fp4), then
//            the 16-bit MFMA.
//
// Epilogues: STORE (bias, round) and GLU (gate/up halves of w13 -> SiLU-mul or
// swigluoai), optionally re-quantising the activation to e4m3 with 1x128
// scales for the w2 GEMM.
#include <cstdlib>
#include <cstring>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int KB = 128;  // K elements per LDS stage


// e4m3 x e4m3, 16x16x128, scale exponents 127 (= 1.0) on both operands.
__device__ __forceinline__ f32x4 mfma_fp8(uint4 a0, uint4 a1, uint4 b0,
                                          uint4 b1) {
  i32x8 a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
             (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  i32x8 b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
             (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127,
                                                          0, 127);
}

// Waves per SIMD the register allocation must allow: the 16-slot 4-bit
// kernels are latency-bound and keep six (80 registers); the others take
// what they need.
template <int RECIPE, int BM>
constexpr int small_min_waves() {
  constexpr bool k4 = RECIPE == MI355MOE_RECIPE_MXFP4 || RECIPE == MI355MOE_RECIPE_INT4;
  return k4 && BM == 16 ? 6 : 1;
}

template <int RECIPE, int BM, int BN, int EPI, bool QOUT, bool F16>
__global__ __launch_bounds__(256, (small_min_waves<RECIPE, BM>())) void moe_gemm_kernel(
    const GemmArgs a, void* __restrict__ qs) {
  constexpr bool kFp8 = RECIPE == MI355MOE_RECIPE_FP8BLOCK;
  constexpr bool kFp4 = RECIPE == MI355MOE_RECIPE_MXFP4 || RECIPE == MI355MOE_RECIPE_INT4;
  constexpr bool kW8 = is_w8a16_recipe(RECIPE);  // fp8 weights, 16-bit activations
  constexpr int XB = kFp8 ? 1 : 2;      // bytes per activation element
  constexpr int ROWB = KB * XB + 16;    // padded LDS row pitch (bytes)
  constexpr int CPR = KB * XB / 16;     // 16-byte chunks per staged row
  constexpr int MT = BM / 16;
  constexpr int WN = BN / 4;
  constexpr int NT = WN / 16;
  constexpr int NB = EPI == EPI_GLU ? 2 * NT : NT;
  constexpr int KS = kFp8 ? 1 : 4;      // MFMA k-steps per stage

  __shared__ __attribute__((aligned(16))) uint8_t sX[BM * ROWB];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ float s_xs[BM];
  __shared__ float s_amax[4][BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, q = lane >> 4;
  int blk = blockIdx.y, ntile = blockIdx.x;
  const int nblk = (*a.ntp + BM - 1) / BM;  // blocks holding valid slots
  // Where the blocks hold enough 16-bit rows, XCD x (workgroups are
  // dispatched round-robin over the 8 XCDs) takes the contiguous range
  // [x*per, (x+1)*per) of the valid (block, N-tile) pairs in block-major
  // order, so that one L2 serves a block's activation rows to all its
  // N-tiles (C5 T=128 w2: 170 -> 144 MB fetched per launch, C2 T=256 -2 %);
  // with e4m3 activations (C3 T=256 +1 %) or nearly empty blocks (C5 T=32
  // w2 +5 %) the N-tiles stay spread over the XCDs
  const bool xcd = a.xcd_order > 0 ||
                   (a.xcd_order == 0 && XB == 2 && a.num_valid >= 8 * nblk);
  if (xcd) {
    const int n_tiles = static_cast<int>(gridDim.x);
    const int valid = nblk * n_tiles;
    const int lin = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
    const int per = (valid + 7) / 8;
    const int tile = (lin & 7) * per + (lin >> 3);
    if ((lin >> 3) >= per || tile >= valid) return;  // uniform
    blk = tile / n_tiles;
    ntile = tile - blk * n_tiles;
  } else if (blk >= nblk) {
    return;  // uniform for the workgroup
  }
  const int e = a.block_expert[blk];
  const int64_t K = a.K;
  const int64_t wrow_bytes = kFp4 ? K / 2 : (kW8 ? K : K * XB);

  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    const bool ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }

  const int64_t nbase = static_cast<int64_t>(ntile) * BN + wave * WN;
  const uint8_t* wbase = static_cast<const uint8_t*>(a.B) +
                         static_cast<int64_t>(e) * a.ldb_rows * wrow_bytes;
  // weights (and mxfp4 scales) may be K-blocked
  const WStride wst = kFp4 ? w_stride4(a)
                           : (kW8 ? w_stride8w(a) : (kFp8 ? w_stride8(a) : w_stride16(a)));
  const WStride sst = s_stride4(a);
  const uint8_t* wptr[NB];
  bool wok[NB];
  int64_t wrow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int64_t n = nbase + (j % NT) * 16 + l16;
    wok[j] = n < a.N;
    wrow[j] = (j >= NT ? a.up_off : 0) + (wok[j] ? n : 0);
    wptr[j] = wbase + wrow[j] * wst.row;
  }

  f32x4 acc[MT][NB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();

  if constexpr (kFp4) {
    // 4-bit weights, software-pipelined one stage ahead: the raw words and
    // scale codes of stage k0 + KB and its activation chunks are in flight
    // while stage k0 computes.  Every load is unconditional, from an address
    // clamped into range (rows past N read row 0, chunks past K the last
    // chunk; K % 32 == 0), and out-of-range data is zeroed where it is used:
    // a load under a branch makes the compiler wait for every load in flight
    // where the branches join.  The raw weight registers are decoded before
    // they are reloaded, so no copy waits for the next stage's loads.
    static_assert(BM * CPR % 256 == 0, "whole activation chunks per thread");
    constexpr int ACH = BM * CPR / 256;  // activation chunks per thread
    uint4 rw[NB];
    uint32_t rc[NB];
    auto load_w4 = [&](int64_t k) {
      const int64_t kk = k + 32 * q;
      const int64_t blk32 = (kk < K ? kk : K - 32) / 32;  // the lane's 32-value block
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        rw[j] = *reinterpret_cast<const uint4*>(wptr[j] + blk32 * wst.kblk);
        rc[j] = w4_scale_code<RECIPE>(a, e, wrow[j], blk32, sst);
      }
    };
    // chunk i of this thread: activation row xar[i] (-1: padding slot), K
    // offset xc inside the stage (the same for every i: 256 % CPR == 0);
    // addresses are recomputed per stage to keep registers for occupancy
    static_assert(256 % CPR == 0, "one chunk column per thread");
    const int xc = (tid % CPR) * 8;
    int xar[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) xar[i] = s_arow[(tid + 256 * i) / CPR];
    uint4 av[ACH];
    auto load_x = [&](int64_t k0) {
      const int64_t kk = k0 + xc;
      const int64_t off = (kk < K ? kk : K - 8) * XB;
#pragma unroll
      for (int i = 0; i < ACH; ++i)
        av[i] = *reinterpret_cast<const uint4*>(
            static_cast<const uint8_t*>(a.A) +
            static_cast<int64_t>(xar[i] >= 0 ? xar[i] : 0) * K * XB + off);
    };
    // the same issue order as in the loop (weights, then activation), so
    // that the waits at the loop top count the activation loads as newer
    load_w4(0);
    __builtin_amdgcn_sched_barrier(0);
    load_x(0);
    for (int64_t k0 = 0; k0 < K; k0 += KB) {
      uint4 wf[KS][NB];
      const bool klive = k0 + 32 * q < K;  // this lane's 32-value block of the stage
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        // masks rather than selects: a select becomes a branch around copies
        const uint32_t m = klive && wok[j] ? ~0u : 0u;
        const uint32_t c = rc[j] & m;
        wf[0][j] = w4_decode8<RECIPE, F16>(rw[j].x & m, c);
        wf[1][j] = w4_decode8<RECIPE, F16>(rw[j].y & m, c);
        wf[2][j] = w4_decode8<RECIPE, F16>(rw[j].z & m, c);
        wf[3][j] = w4_decode8<RECIPE, F16>(rw[j].w & m, c);
      }
      load_w4(k0 + KB);  // past K on the last stage: clamped, unused
      // issued before anything below waits for this stage's activation
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();   // the previous stage's fragment reads are done
#pragma unroll
      for (int i = 0; i < ACH; ++i) {
        const int idx = tid + 256 * i;
        const uint32_t m = xar[i] >= 0 && k0 + xc < K ? ~0u : 0u;
        *reinterpret_cast<uint4*>(sX + (idx / CPR) * ROWB + (idx % CPR) * 16) =
            make_uint4(av[i].x & m, av[i].y & m, av[i].z & m, av[i].w & m);
      }
      load_x(k0 + KB);
      __syncthreads();
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint8_t* xr = sX + (mt * 16 + l16) * ROWB;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint4 x = *reinterpret_cast<const uint4*>(xr + (32 * q + 8 * s) * 2);
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[mt][j] = mfma16_16x16x32<F16>(wf[s][j], x, acc[mt][j]);
        }
      }
    }
  } else {
    // 16-bit and fp8 weights.  Per stage: the weight fragments HBM -> VGPR,
    // then the activation chunks of the stage -> LDS.  STORE kernels load
    // unconditionally from addresses clamped into range (rows past N read
    // row 0, K past the end the last chunk), zero the out-of-range data
    // where it is used, and keep all of a thread's activation chunks in
    // flight together (one wait per stage; a load under a branch makes the
    // compiler wait for every load in flight).  GLU kernels, which hold
    // twice the weight fragments, move the activation one chunk at a time
    // under conditions: in flight together the chunks cost them a wave per
    // SIMD and measured slower (C2 T=256 w13 +2 %; STORE -3 to -20 %).
    constexpr bool kBatchX = EPI != EPI_GLU;
    constexpr int NCH = BM * CPR;           // activation chunks per stage
    constexpr int ACH = (NCH + 255) / 256;  // per thread
    static_assert(256 % CPR == 0, "one chunk column per thread");
    constexpr int KE = 16 / XB;             // K elements per chunk
    const int xc = (tid % CPR) * KE;
    int xar[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int idx = tid + 256 * i;
      xar[i] = idx < NCH ? s_arow[idx / CPR] : -1;
    }
    const int xsr = kFp8 && tid < BM ? s_arow[tid] : -1;  // fp8: this thread's scale row
    for (int64_t k0 = 0; k0 < K; k0 += KB) {
      const int kb = static_cast<int>(K - k0 < KB ? K - k0 : KB);
      // ---- weight fragments: HBM -> VGPR
      // (fp8 weights: the lane's 32 K values 32q..32q+31 of the stage)
      uint4 wf[kW8 ? 1 : KS][NB][kFp8 || kW8 ? 2 : 1];
      float wsc[NB];
  #pragma unroll
      for (int j = 0; j < NB; ++j) {
        if constexpr (kFp8) {  // K % 128 == 0: no tail
          const uint4* p = reinterpret_cast<const uint4*>(wptr[j] + (k0 >> 7) * wst.kblk + 32 * q);
          wf[0][j][0] = kBatchX || wok[j] ? p[0] : make_uint4(0, 0, 0, 0);
          wf[0][j][1] = kBatchX || wok[j] ? p[1] : make_uint4(0, 0, 0, 0);
          const float* bs = static_cast<const float*>(a.b_scale);
          const int wsh = 7 - a.ws_rows64;  // weight rows per scale row: 128 or 64
          wsc[j] = bs[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + (wrow[j] >> wsh)) *
                          (K / 128) + k0 / 128];
        } else if constexpr (kW8) {  // K % 32 == 0: a chunk lies wholly in or past K
          const int64_t kc = k0 + 32 * q < K ? k0 + 32 * q : K - 32;
          const uint4* p = reinterpret_cast<const uint4*>(wptr[j] + (kc >> 5) * wst.kblk);
          wf[0][j][0] = kBatchX || wok[j] ? p[0] : make_uint4(0, 0, 0, 0);
          wf[0][j][1] = kBatchX || wok[j] ? p[1] : make_uint4(0, 0, 0, 0);
        } else {
  #pragma unroll
          for (int s = 0; s < KS; ++s) {
            const int64_t kk = k0 + 32 * s + 8 * q;
            if constexpr (kBatchX)
              wf[s][j][0] = *reinterpret_cast<const uint4*>(
                  wptr[j] + w_koff16(wst, kk + 8 <= K ? kk : K - 8));
            else
              wf[s][j][0] = wok[j] && 32 * s + 8 * q + 8 <= kb
                                ? *reinterpret_cast<const uint4*>(wptr[j] + w_koff16(wst, kk))
                                : make_uint4(0, 0, 0, 0);
          }
        }
      }
      // ---- activation tile -> LDS
      const int64_t xoff = (k0 + xc < K ? k0 + xc : K - KE) * XB;
      auto xload = [&](int i) {
        return *reinterpret_cast<const uint4*>(
            static_cast<const uint8_t*>(a.A) +
            static_cast<int64_t>(xar[i] >= 0 ? xar[i] : 0) * K * XB + xoff);
      };
      auto xstore = [&](int i, const uint4& v) {
        const int idx = tid + 256 * i;
        const uint32_t m = xar[i] >= 0 && xc < kb ? ~0u : 0u;
        if (idx < NCH)
          *reinterpret_cast<uint4*>(sX + (idx / CPR) * ROWB + (idx % CPR) * 16) =
              make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
      };
      if constexpr (kBatchX) {
        uint4 av[ACH];
  #pragma unroll
        for (int i = 0; i < ACH; ++i) av[i] = xload(i);
        float xsv = 0.f;
        if constexpr (kFp8)
          xsv = a.a_scale[static_cast<int64_t>(xsr >= 0 ? xsr : 0) * (K / 128) + k0 / 128];
        __syncthreads();  // the previous stage's fragment reads are done
  #pragma unroll
        for (int i = 0; i < ACH; ++i) xstore(i, av[i]);
        if constexpr (kFp8) {
          if (tid < BM) s_xs[tid] = xsr >= 0 ? xsv : 0.f;
        }
      } else {
        __syncthreads();  // the previous stage's fragment reads are done
        for (int idx = tid; idx < NCH; idx += 256) {
          const int r = idx / CPR, c = idx % CPR;
          const int ar = s_arow[r];
          uint4 v = make_uint4(0, 0, 0, 0);
          if (ar >= 0 && c * 16 < kb * XB)
            v = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.A) +
                                                (static_cast<int64_t>(ar) * K + k0) * XB +
                                                c * 16);
          *reinterpret_cast<uint4*>(sX + r * ROWB + c * 16) = v;
        }
        if constexpr (kFp8) {
          if (tid < BM) {
            const int ar = s_arow[tid];
            s_xs[tid] = ar >= 0 ? a.a_scale[static_cast<int64_t>(ar) * (K / 128) + k0 / 128] : 0.f;
          }
        }
      }
      __syncthreads();
      // ---- MFMA
  #pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint8_t* xr = sX + (mt * 16 + l16) * ROWB;
        if constexpr (kFp8) {
          const uint4 x0 = *reinterpret_cast<const uint4*>(xr + 32 * q);
          const uint4 x1 = *reinterpret_cast<const uint4*>(xr + 32 * q + 16);
          const float xs = s_xs[mt * 16 + l16];
  #pragma unroll
          for (int j = 0; j < NB; ++j) {
            f32x4 p = mfma_fp8(wf[0][j][0], wf[0][j][1], x0, x1);
            const float sc = xs * wsc[j];
            acc[mt][j] += p * sc;
          }
        } else if constexpr (kW8) {
          // the activation in the weights' K order: step s takes K 32q + 8s
          // .. + 7; a chunk past K (the last stage of a K % 128 != 0) reads
          // back in-range data and is zeroed
          const uint32_t m = 32 * q < kb ? ~0u : 0u;
          constexpr bool k52 = RECIPE == MI355MOE_RECIPE_FP8E5M2;
  #pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint4 x = *reinterpret_cast<const uint4*>(xr + (32 * q + 8 * s) * 2);
  #pragma unroll
            for (int j = 0; j < NB; ++j) {
              const uint4 w = wf[0][j][s >> 1];
              const uint2 h = (s & 1) ? make_uint2(w.z & m, w.w & m) : make_uint2(w.x & m, w.y & m);
              acc[mt][j] = mfma16_16x16x32<F16>(fp8x8_to16<k52, F16>(h), x, acc[mt][j]);
            }
          }
        } else {
  #pragma unroll
          for (int s = 0; s < KS; ++s) {
            const int koff = 32 * s + 8 * q;
            const uint4 x = *reinterpret_cast<const uint4*>(xr + koff * 2);
            // weights past K (the last stage of a K % 128 != 0) read back in-range data
            const uint32_t m = koff + 8 <= kb ? ~0u : 0u;
  #pragma unroll
            for (int j = 0; j < NB; ++j) {
              const uint4 w = wf[s][j][0];
              acc[mt][j] = mfma16_16x16x32<F16>(make_uint4(w.x & m, w.y & m, w.z & m, w.w & m),
                                                x, acc[mt][j]);
            }
          }
        }
      }
    }
  }

  // ---- epilogue: lane holds D[row = mt*16 + l16][n = nbase + j*16 + 4q + r]
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  const float es = a.expert_scale ? a.expert_scale[e] : 1.f;
  float outv[MT][NT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t n = nbase + j * 16 + 4 * q;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool nok = n + r < a.N;
        float v = acc[mt][j][r] * es;
        if (a.bias && nok) v += ld16<F16>(a.bias[bias_base + n + r]);
        v = rnd16<F16>(v);
        if constexpr (EPI == EPI_GLU) {
          float u = acc[mt][j + NT][r] * es;
          if (a.bias && nok) u += ld16<F16>(a.bias[bias_base + a.up_off + n + r]);
          u = rnd16<F16>(u);
          glu_clamp(a, n + r, v, u);
          v = rnd16<F16>(glu16<F16>(v, u, a.act, a.alpha, a.limit));
        }
        outv[mt][j][r] = nok ? v : 0.f;
      }
    }
  }

  if constexpr (QOUT) {
    // e4m3 output with one fp32 scale per (row, 128 columns): BN == 128 and
    // the 4 waves cover the 128 columns of the group.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float m = 1e-10f;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(outv[mt][j][r]));
      m = max_over_rows(m);
      if (q == 0) s_amax[wave][mt * 16 + l16] = m;
    }
    __syncthreads();
    uint8_t* dq = static_cast<uint8_t*>(a.D);
    float* ds = static_cast<float*>(qs);
    const int64_t ngroups = a.N / 128;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = mt * 16 + l16;
      const int drow = s_drow[row];
      if (drow < 0) continue;
      const float am = fmaxf(fmaxf(s_amax[0][row], s_amax[1][row]),
                             fmaxf(s_amax[2][row], s_amax[3][row]));
      const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
      const float inv = 1.0f / sc;
      if (wave == 0 && q == 0) ds[static_cast<int64_t>(drow) * ngroups + ntile] = sc;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t n = nbase + j * 16 + 4 * q;
        const uint32_t w = e4m3x4_sat(outv[mt][j][0] * inv, outv[mt][j][1] * inv,
                                      outv[mt][j][2] * inv, outv[mt][j][3] * inv);
        *reinterpret_cast<uint32_t*>(dq + static_cast<int64_t>(drow) * a.N + n) = w;
      }
    }
  } else {
    uint16_t* d = static_cast<uint16_t*>(a.D);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int drow = s_drow[mt * 16 + l16];
      if (drow < 0) continue;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t n = nbase + j * 16 + 4 * q;
        uint16_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          h[r] = st16<F16>(outv[mt][j][r]);
        uint16_t* dst = d + static_cast<int64_t>(drow) * a.N + n;
        if (n + 3 < a.N && (a.N & 3) == 0) {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < a.N) dst[r] = h[r];
        }
      }
    }
  }
}

template <int RECIPE, int BM, int EPI, bool QOUT>
void launch_tile(const GemmArgs& a, int64_t max_blocks, void* qs,
                 hipStream_t st) {
  constexpr int BN = (BM == 16 && !QOUT) ? 64 : 128;
  GemmArgs b = a;
  // MI355MOE_SMALL_XCD=1 / 0 forces the XCD order on / off (measurements);
  // read per call
  const char* xv = getenv("MI355MOE_SMALL_XCD");
  b.xcd_order = !xv ? 0 : (xv[0] == '1' ? 1 : -1);
  const int64_t nx = cdiv(a.N, BN);
  // in the XCD order workgroup w takes tile (w % 8) * per + w / 8, per = the
  // valid tiles / 8 rounded up: the launch covers a multiple of 8
  // workgroups (those past max_blocks exit at once in the other order)
  const int64_t ny = cdiv(cdiv(nx * max_blocks, 8) * 8, nx);
  dim3 grid(static_cast<unsigned>(nx), static_cast<unsigned>(ny));
  if (b.out_f16)
    moe_gemm_kernel<RECIPE, BM, BN, EPI, QOUT, true><<<grid, dim3(256), 0, st>>>(b, qs);
  else
    moe_gemm_kernel<RECIPE, BM, BN, EPI, QOUT, false><<<grid, dim3(256), 0, st>>>(b, qs);
}

template <int RECIPE, int EPI, bool QOUT>
int launch_bm(int bm, const GemmArgs& a, int64_t max_blocks, void* qs,
              hipStream_t st) {
  switch (bm) {
    case 16: launch_tile<RECIPE, 16, EPI, QOUT>(a, max_blocks, qs, st); break;
    case 32: launch_tile<RECIPE, 32, EPI, QOUT>(a, max_blocks, qs, st); break;
    case 64: launch_tile<RECIPE, 64, EPI, QOUT>(a, max_blocks, qs, st); break;
    case 128: launch_tile<RECIPE, 128, EPI, QOUT>(a, max_blocks, qs, st); break;
    default: return set_error(MI355MOE_ERR_INVALID, "block_m must be 16, 32, 64 or 128");
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace

int pick_block_m(int64_t slots, int64_t num_experts) {
  const int64_t active = slots < num_experts ? slots : num_experts;
  const int64_t avg = active > 0 ? slots / active : 0;
  if (avg <= 24) return 16;
  if (avg <= 48) return 32;
  if (avg <= 96) return 64;
  return 128;
}

bool wide_ok_for(int recipe, int64_t a_rows, int64_t ldb_rows, int64_t K, bool w_kblock) {
  if (recipe == MI355MOE_RECIPE_BF16) return K % 32 == 0 && wide_offsets_fit(a_rows, ldb_rows, K);
  if (recipe == MI355MOE_RECIPE_FP8BLOCK) return wide8_shape_ok(a_rows, ldb_rows, K);
  if (recipe == MI355MOE_RECIPE_MXFP8)
    return w_kblock && ldb_rows % 4 == 0 && wide8_shape_ok(a_rows, ldb_rows, K);
  if (recipe == RECIPE_MX4A4)
    return w_kblock && ldb_rows % 4 == 0 && wide8_shape_ok_mx4(a_rows, ldb_rows, K);
  if (recipe == MI355MOE_RECIPE_MXFP4 || recipe == MI355MOE_RECIPE_INT4 ||
      is_w8a16_recipe(recipe))
    return w_kblock && wide4_shape_ok(a_rows, ldb_rows, ldb_rows, K);
  return false;
}

GemmTile pick_tile(int recipe, bool wide_ok, int64_t slots, int64_t num_experts, int* bm) {
  // MI355MOE_GEMM_TILE forces a family (tests, measurements); read per call
  const int force = [] {
    const char* v = getenv("MI355MOE_GEMM_TILE");
    if (!v) return -1;
    if (!strcmp(v, "stream")) return static_cast<int>(TILE_STREAM);
    if (!strcmp(v, "small")) return static_cast<int>(TILE_SMALL);
    if (!strcmp(v, "big")) return static_cast<int>(TILE_BIG);
    if (!strcmp(v, "bigreg")) return static_cast<int>(TILE_BIGREG);
    if (!strcmp(v, "wide")) return static_cast<int>(TILE_WIDE);
    return -1;
  }();
  const int64_t active = slots < num_experts ? slots : num_experts;
  const int64_t avg = active > 0 ? slots / active : 0;
  GemmTile t;
  int b;
  if ((recipe == MI355MOE_RECIPE_MXFP8 || recipe == RECIPE_MX4A4) && wide_ok && avg > 16) {
    // the 320-slot kernel with the e8m0 codes in the MFMA from 17 slots per
    // expert on (16-slot STREAM blocks would stream an expert's weights once
    // per block)
    t = TILE_WIDE, b = kWideBM;
  } else if (is_mx_recipe(recipe)) {
    t = TILE_STREAM, b = 16;
  } else if (is_w8a16_recipe(recipe)) {
    // the 16-bit rule; prefill on the 320-slot kernel of the 4-bit weights
    // (WIDE4 reads fp8 fragments too), which needs K-blocked weights
    if (avg <= kStreamMaxAvg16) t = TILE_STREAM, b = 16;
    else if (avg <= kSmallMaxAvg16 || !wide_ok) t = TILE_SMALL, b = 64;
    else t = TILE_WIDE, b = kWideBM;
  } else if (recipe == MI355MOE_RECIPE_FP8BLOCK) {
    // a 320-slot fp8 stage is 73 KB, so the WIDE kernel keeps one stage of
    // DMA in flight against the 128-slot kernel's two: it wins where experts
    // average well above 128 slots (fewer weight passes), not at about 128
    if (avg <= 4) t = TILE_STREAM, b = 16;
    else if (avg <= 12) t = TILE_SMALL, b = 16;
    else if (avg > 160 && wide_ok) t = TILE_WIDE, b = kWideBM;
    else t = TILE_BIG, b = 128;
  } else if (recipe == MI355MOE_RECIPE_MXFP4 || recipe == MI355MOE_RECIPE_INT4) {
    if (avg <= 2) t = TILE_STREAM, b = 16;
    // 32-slot blocks from 12 slots per expert on: one block holds most
    // experts, so each expert's weights stream once (C5 T=128, 16 slots per
    // expert: 157 -> 127 us per layer against 16-slot blocks)
    else if (avg <= 12) t = TILE_SMALL, b = 16;
    else if (avg <= 40 || (!wide_ok && avg <= 48)) t = TILE_SMALL, b = 32;
    else if (wide_ok) t = TILE_WIDE, b = kWideBM;
    else t = TILE_BIG, b = 128;
  } else {
    if (avg <= kStreamMaxAvg16) t = TILE_STREAM, b = 16;
    else if (avg <= kSmallMaxAvg16 || (!wide_ok && avg <= 96)) t = TILE_SMALL, b = 64;
    else if (wide_ok) t = TILE_WIDE, b = kWideBM;
    else t = TILE_BIG, b = 128;
  }
  if (force >= 0 && !is_mx_recipe(recipe) && !is_w8a16_recipe(recipe)) {
    t = static_cast<GemmTile>(force);
    if (t == TILE_WIDE && !wide_ok) t = TILE_BIG;
    b = t == TILE_STREAM ? 16
        : t == TILE_WIDE ? kWideBM
        : (t == TILE_BIG || t == TILE_BIGREG) ? 128
                                              : pick_block_m(slots, num_experts);
  }
  *bm = b;
  return t;
}

int launch_tile_gemm(GemmTile tile, int bm, int recipe, int epi, bool qout,
                     const GemmArgs& a, int64_t max_blocks, void* qs,
                     hipStream_t st) {
  MI_ARG(!a.w_kblock ||
             (recipe == MI355MOE_RECIPE_BF16 && a.K % 32 == 0 &&
              (tile == TILE_STREAM || tile == TILE_SMALL || tile == TILE_WIDE)) ||
             (recipe == MI355MOE_RECIPE_FP8BLOCK &&
              (tile == TILE_STREAM || tile == TILE_SMALL || tile == TILE_WIDE ||
               (tile == TILE_BIG && big8_supported(recipe, a)))) ||
             recipe == MI355MOE_RECIPE_MXFP4 || recipe == MI355MOE_RECIPE_INT4 ||
             is_mx_recipe(recipe) || (is_w8a16_recipe(recipe) && a.K % 32 == 0),
         "K-blocked weights need the bf16 (K % 32 == 0), fp8block, mxfp4, mxfp8 or "
         "per-expert fp8 (K % 32 == 0) recipe and a kernel family that reads them");
  MI_ARG(!is_mx_recipe(recipe) || tile == TILE_STREAM || tile == TILE_WIDE,
         "MX recipes run the STREAM and WIDE kernels");
  MI_CHECK(!is_w8a16_recipe(recipe) || tile == TILE_STREAM || tile == TILE_SMALL ||
               tile == TILE_WIDE,
           MI355MOE_ERR_UNSUPPORTED,
           "per-expert fp8 weights run the STREAM, SMALL and WIDE kernels");
  switch (tile) {
    case TILE_STREAM: return launch_moe_gemm_stream(recipe, epi, qout, a, max_blocks, qs, st);
    case TILE_BIG:
      if (big8_supported(recipe, a))
        return launch_moe_gemm_big8(recipe, epi, qout, a, max_blocks, qs, st);
      if (pipe_supported(recipe, a))
        return launch_moe_gemm_pipe(recipe, epi, qout, a, max_blocks, qs, st);
      return launch_moe_gemm_big(recipe, epi, qout, a, max_blocks, qs, st);
    case TILE_BIGREG: return launch_moe_gemm_big(recipe, epi, qout, a, max_blocks, qs, st);
    case TILE_WIDE:
      if (recipe == MI355MOE_RECIPE_FP8BLOCK || is_mx_recipe(recipe))
        return launch_moe_gemm_wide8(recipe, epi, qout, a, max_blocks, qs, st);
      MI_ARG(!qout, "wide GEMM: no fp8 activation output");
      if (recipe == MI355MOE_RECIPE_MXFP4 || recipe == MI355MOE_RECIPE_INT4 ||
          is_w8a16_recipe(recipe))
        return launch_moe_gemm_wide4(recipe, epi, a, max_blocks, st);
      return launch_moe_gemm_wide(recipe, epi, a, max_blocks, st);
    default: return launch_moe_gemm_q(recipe, epi, qout, bm, a, max_blocks, qs, st);
  }
}

int launch_moe_gemm_q(int recipe, int epi, bool qout, int bm, const GemmArgs& a,
                      int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  if (qout) {
    MI_ARG(recipe == MI355MOE_RECIPE_FP8BLOCK && epi == EPI_GLU && a.N % 128 == 0,
           "fp8 activation output needs the fp8block recipe and I % 128 == 0");
    return launch_bm<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, true>(bm, a, max_blocks, qs, st);
  }
#define MI_EPI(R)                                                            \
  return epi == EPI_GLU ? launch_bm<R, EPI_GLU, false>(bm, a, max_blocks, qs, st) \
                        : launch_bm<R, EPI_STORE, false>(bm, a, max_blocks, qs, st);
  switch (recipe) {
    case MI355MOE_RECIPE_BF16: MI_EPI(MI355MOE_RECIPE_BF16)
    case MI355MOE_RECIPE_FP8BLOCK: MI_EPI(MI355MOE_RECIPE_FP8BLOCK)
    case MI355MOE_RECIPE_MXFP4: MI_EPI(MI355MOE_RECIPE_MXFP4)
    case MI355MOE_RECIPE_INT4: MI_EPI(MI355MOE_RECIPE_INT4)
    default: break;
  }
#undef MI_EPI
  if (is_w8a16_recipe(recipe)) {  // 64-slot blocks only (the tile choice's)
    MI_ARG(bm == 64, "per-expert fp8 weights: 64-slot blocks");
    if (recipe == MI355MOE_RECIPE_FP8) {
      if (epi == EPI_GLU) launch_tile<MI355MOE_RECIPE_FP8, 64, EPI_GLU, false>(a, max_blocks, qs, st);
      else launch_tile<MI355MOE_RECIPE_FP8, 64, EPI_STORE, false>(a, max_blocks, qs, st);
    } else {
      if (epi == EPI_GLU) launch_tile<MI355MOE_RECIPE_FP8E5M2, 64, EPI_GLU, false>(a, max_blocks, qs, st);
      else launch_tile<MI355MOE_RECIPE_FP8E5M2, 64, EPI_STORE, false>(a, max_blocks, qs, st);
    }
    MI_LAUNCH_CHECK();
    return MI355MOE_OK;
  }
  return set_error(MI355MOE_ERR_INVALID, "unknown recipe");
}

int launch_moe_gemm(int recipe, int epi, int bm, const GemmArgs& a,
                    int64_t max_blocks, hipStream_t st) {
  return launch_moe_gemm_q(recipe, epi, false, bm, a, max_blocks, nullptr, st);
}

}  // namespace mi355
