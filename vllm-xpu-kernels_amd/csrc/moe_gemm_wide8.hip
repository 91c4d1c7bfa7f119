// Prefill grouped GEMM for fp8 e4m3 weights with 128x128 block scales and
// e4m3 activations with 1x128 scales: 320-slot x 256-weight-row tiles, 8
// waves, 2-slot LDS ring fed by direct global->LDS DMA.
//
// Why 320 slots.  A tile streams its 256 weight rows over the whole K, so the
// weight bytes a layer moves are (tiles per expert) x (expert weights);
// routing spreads n +- sqrt(n) slots over an expert and 320 slots hold the
// usual prefill n = 256 with four standard deviations to spare, where
// 128-slot blocks stream every expert's weights three times.  Compute and
// activation DMA scale with the valid slots only.
//
// Waves.  Eight waves, two per SIMD (waves w and w + 4 share SIMD w % 4), each
// owning 160 slots x 64 weight rows: 4 x 10 tiles of the 16x16x128 e4m3 MFMA
// with the weight as the A operand (160 accumulator registers).  One MFMA
// covers one whole 128-K scale block, so its result is scaled and added at
// once (acc += p * xs * ws).  The four weight fragments of a stage stay in
// registers; the ten activation fragments stream from LDS one tile ahead.
//
// Stages.  A stage holds 128 K elements (128 bytes) of the 320 activation
// rows and 256 weight rows plus the 320 activation scales of the 128-K block:
// 73.25 KB, so two fit.  Waves 0-3 move 10 activation blocks of 8 rows each,
// waves 4-7 8 weight blocks and the scales (global_load_lds_dwordx4 /
// _dword).  16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7), so
// sixteen rows read at one logical chunk hit sixteen distinct bank groups.
// DMA addresses are a scalar base plus 32-bit lane offsets recomputed each
// stage from small LDS tables (no registers held across the K loop).
//
// Pipeline.  Iteration kt waits for its own DMA of stage kt, meets the others
// at a barrier (stage kt is complete and visible, and every wave has finished
// reading stage kt-1), then issues stage kt+1 into stage kt-1's slot and
// computes stage kt while that DMA is in flight.
//
// Tiles, GLU pairing and the fp8 activation output are those of the other
// prefill kernels: a GLU tile's 256 weight rows are 128 gate rows and the
// matching 128 up rows, so its 128 output columns are one whole 1x128
// quantisation group of the next GEMM's input.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int BM = 320, BN = 256, ROWB = 128, KE = 128;
static_assert(BM == kWideBM, "block size of the WIDE family");
constexpr int A_BYTES = BM * ROWB;                 // 40 KB
constexpr int W_BYTES = BN * ROWB;                 // 32 KB
constexpr int S_OFF = A_BYTES + W_BYTES;           // activation scales
constexpr int STAGE = S_OFF + BM * 4;              // 73.25 KB
constexpr int NSTAGE = 2;
constexpr int RING = NSTAGE * STAGE;
constexpr int A_BLK = BM / 8 / 4;                  // activation blocks per wave (waves 0-3)
constexpr int W_BLK = BN / 8 / 4;                  // weight blocks per wave (waves 4-7)
constexpr int MAX_KBLK = 64;                       // K <= 8192
constexpr int TJ = BM / 2 / 16;                    // activation tiles per wave
static_assert(BM * (2 * 128 + 16) <= RING, "GLU output tile staged in one pass");
static_assert(BM / 2 * (2 * 256 + 16) <= RING, "STORE output tile staged in two passes");
static_assert(BM * (128 + 16) + 4 * BM * 4 <= RING, "fp8 output tile and row maxima");

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)p));
}
// 16 (dma16) or 4 (dma4) bytes per lane from sbase + voff (scalar base,
// 32-bit lane offset) into LDS at lds_base + 16 lane (4 lane).
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(reinterpret_cast<uint64_t>(sbase)), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(reinterpret_cast<uint64_t>(sbase)), "s"(lds_base) : "memory", "m0");
}
// readfirstlane returns int: each half goes through uint32_t so that the low
// half is zero-extended.
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return reinterpret_cast<const uint8_t*>((hi << 32) | lo);
}
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// e4m3 x e4m3, 16x16x128, unit e8m0 scales, C = 0.
__device__ __forceinline__ f32x4_t mfma16(const i32x8_t& a, const i32x8_t& b) {
  const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}
// 32 bytes of one row as one MFMA operand: chunks at byte offsets o0, o1
__device__ __forceinline__ i32x8_t ld32(const uint8_t* S, int o0, int o1) {
  const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(S + o0);
  const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(S + o1);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <bool F16>
__device__ __forceinline__ float round16(float v) {
  if constexpr (F16) return f16_to_f32(f32_to_f16(v));
  else return bf16_to_f32(f32_to_bf16(v));
}
template <bool F16>
__device__ __forceinline__ uint32_t to16(float v) {
  if constexpr (F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}
__device__ __forceinline__ float x_sigmoid(float x, float k) {
  const float e = __builtin_amdgcn_exp2f(-k * x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

// Weight fragments of one wave (4 tiles of 16 rows).  Tile rows start at
// multiples of 16, where the row swizzle (r >> 1) & 7 depends on r % 16 only:
// one base offset per chunk, tiles at constant distances.
template <bool kGlu>
__device__ __forceinline__ void read_w(i32x8_t (&w)[4], const uint8_t* S, int wo0, int wo1) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = kGlu ? (i < 2 ? 0 : 128) + 16 * (i & 1) : 16 * i;  // tile row - wave row
    w[i] = ld32(S + t * ROWB, wo0, wo1);
  }
}

template <int EPI, bool QOUT, bool F16>
__global__ __launch_bounds__(512) void moe_gemm_wide8_kernel(const GemmArgs a, void* __restrict__ qs) {
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns per tile

  __shared__ __attribute__((aligned(1024))) uint8_t lds[RING];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ uint32_t s_woff[BN];       // byte offset of tile weight row r in the expert
  __shared__ float s_wsc[4][MAX_KBLK];  // weight-block scales of the tile's four 64-row quarters

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
  const int wm = wave >> 2, wn = wave & 3;
  const int l16 = lane & 15, g = lane >> 4;

  // XCD-aware order (as in the other prefill kernels): XCD x takes the
  // contiguous range [x*per, (x+1)*per) of the tiles ordered by tile_coords.
  const int n_tiles = static_cast<int>((a.N + NOUT - 1) / NOUT);
  const int valid = (*a.ntp / BM) * n_tiles;
  const int bid = static_cast<int>(blockIdx.x);
  const int per = (valid + 7) / 8;
  const int tile = (bid & 7) * per + (bid >> 3);
  if ((bid >> 3) >= per || tile >= valid) return;  // uniform
  int blk, ntile;
  tile_coords(a, tile, n_tiles, BM, blk, ntile);
  const int e = a.block_expert[blk];
  const int64_t K = a.K, N = a.N;
  const int64_t n0 = static_cast<int64_t>(ntile) * NOUT;
  const int nkb = static_cast<int>(K / 128);

  int ok = 0;
  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }
  // weight row staged at tile row r (rows past N read row 0: finite data
  // whose outputs are never stored); GLU: [0,128) gate, [128,256) up
  auto wrow_of = [&](int r) -> int64_t {
    if constexpr (kGlu) {
      const int64_t c = n0 + (r & 127);
      return (r >= 128 ? a.up_off : 0) + (c < N ? c : 0);
    } else {
      const int64_t c = n0 + r;
      return c < N ? c : 0;
    }
  };
  // weights may be K-blocked: row stride and bytes between two K stages
  const WStride wst = w_stride8(a);
  if (tid < BN) s_woff[tid] = static_cast<uint32_t>(wrow_of(tid) * wst.row);
  {
    const float* bsc = static_cast<const float*>(a.b_scale);
    const int wsh = 7 - a.ws_rows64;  // weight rows per scale row: 128 or 64
    for (int i = tid; i < 4 * nkb; i += 512) {
      const int t = i / nkb, kb = i % nkb;
      const int64_t wr = wrow_of(64 * t) >> wsh;
      s_wsc[t][kb] = bsc[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + wr) * nkb + kb];
    }
  }
  // valid slots form a prefix of the block
  const int v = __syncthreads_count(ok);

  // DMA of stage kt into slot kt % 2.  Waves 0-3: activation blocks
  // A_BLK wave + q (8 rows each; blocks of padding only are skipped); waves
  // 4-7: weight blocks W_BLK (wave - 4) + q and the activation scales of the
  // 128-K block, 64 slots per dword DMA (wave 4: groups 0, 1; waves 5-7:
  // groups 2-4).  Offsets come from s_arow / s_woff at every issue.
  const bool a_wave = wave < 4;
  const uint8_t* abase = uniform_ptr(a.A);
  const uint8_t* wbase = uniform_ptr(static_cast<const uint8_t*>(a.B) +
                                     static_cast<int64_t>(e) * a.ldb_rows * K);
  const uint8_t* sbase = uniform_ptr(a.a_scale);
  // Lane l of a block b moves row 8 b + l / 8, 16-byte slot l % 8; that row's
  // swizzle is (4 b + l / 16) & 7 = (l / 16) ^ 4 (b & 1), so the lane's
  // source chunk is c0 ^ 64 (b & 1) bytes.  Table entries are read at
  // immediate offsets from one lane address.
  // Per-wave lane addresses into the tables, so that block q's entry sits at
  // an immediate offset; A_BLK and W_BLK are even, so a block's parity is q's.
  static_assert(A_BLK % 2 == 0 && W_BLK % 2 == 0, "block parity is q's");
  const uint32_t ring0 = lds_off(lds);
  const int w4 = wave - 4;
  const int b0 = a_wave ? A_BLK * wave : W_BLK * w4;  // first block of the wave
  const int* arow_w = s_arow + b0 * 8 + (lane >> 3);
  const uint32_t* woff_w = s_woff + b0 * 8 + (lane >> 3);
  const int d0 = w4 <= 0 ? 0 : w4 + 1;               // scale groups of waves 4-7
  const int dn = w4 == 0 ? 2 : 1;
  const int* arow_s = s_arow + d0 * 64 + lane;
  const uint32_t c0 = static_cast<uint32_t>((lane & 7) ^ (lane >> 4)) << 4;
  const uint32_t Ku = static_cast<uint32_t>(K), nkbu = static_cast<uint32_t>(nkb);
  const uint32_t wkstep = static_cast<uint32_t>(wst.kblk);
  auto issue = [&](int kt) {
    const uint32_t base = ring0 + (kt & 1) * STAGE;
    const uint32_t kofs = static_cast<uint32_t>(kt) * ROWB;
    const uint32_t wkofs = static_cast<uint32_t>(kt) * wkstep;
    if (a_wave) {
      const uint32_t dst = base + b0 * 1024;
#pragma unroll
      for (int q = 0; q < A_BLK; ++q) {
        if ((b0 + q) * 8 < v) {
          const int ar = arow_w[q * 8];
          const uint32_t off = static_cast<uint32_t>(ar >= 0 ? ar : 0) * Ku + kofs +
                               (c0 ^ ((q & 1) << 6));
          dma16(off, abase, __builtin_amdgcn_readfirstlane(dst + q * 1024));
        }
      }
    } else {
      const uint32_t dst = base + A_BYTES + b0 * 1024;
#pragma unroll
      for (int q = 0; q < W_BLK; ++q) {
        const uint32_t off = woff_w[q * 8] + wkofs + (c0 ^ ((q & 1) << 6));
        dma16(off, wbase, __builtin_amdgcn_readfirstlane(dst + q * 1024));
      }
      const uint32_t sdst = base + S_OFF + d0 * 256;
#pragma unroll
      for (int dd = 0; dd < 2; ++dd) {
        if (dd < dn && (d0 + dd) * 64 < v) {
          const int ar = arow_s[dd * 64];
          const uint32_t off = (static_cast<uint32_t>(ar >= 0 ? ar : 0) * nkbu +
                                static_cast<uint32_t>(kt)) * 4u;
          dma4(off, sbase, __builtin_amdgcn_readfirstlane(sdst + dd * 256));
        }
      }
    }
  };

  // fragment offsets: chunks 2g and 2g + 1 of the wave's first activation /
  // weight row + l%16
  const int mx = (BM / 2) * wm + l16;
  const int rw = (kGlu ? 32 * wn : 64 * wn) + l16;
  const int xo0 = mx * ROWB + (((2 * g) ^ swz(mx)) << 4);
  const int xo1 = mx * ROWB + (((2 * g + 1) ^ swz(mx)) << 4);
  const int wo0 = A_BYTES + rw * ROWB + (((2 * g) ^ swz(rw)) << 4);
  const int wo1 = A_BYTES + rw * ROWB + (((2 * g + 1) ^ swz(rw)) << 4);
  // s_wsc quarter of weight tile i: GLU tile rows 128 (i / 2) + 32 wn + 16 (i % 2),
  // STORE 64 wn + 16 i
  int wblk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wblk[i] = kGlu ? 2 * (i >> 1) + (wn >> 1) : wn;
  // activation tiles of this wave holding valid slots
  const int vw = v - (BM / 2) * wm;
  const int nj = vw <= 0 ? 0 : (vw >= BM / 2 ? TJ : (vw + 15) / 16);

  f32x4_t acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = static_cast<int>(K / KE);
  issue(0);
  auto kloop = [&](auto nj_c) {
    constexpr int NJ = decltype(nj_c)::value;
    for (int kt = 0; kt < nk; ++kt) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's DMA of stage kt
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); // its reads of stage kt-1
      __builtin_amdgcn_s_barrier();
      if (kt + 1 < nk) issue(kt + 1);
      const uint8_t* S = lds + (kt & 1) * STAGE;
      i32x8_t w[4];
      read_w<kGlu>(w, S, wo0, wo1);
      float ws[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ws[i] = s_wsc[wblk[i]][kt];
      if constexpr (NJ > 0) {
        const float* xsp = reinterpret_cast<const float*>(S + S_OFF) + (BM / 2) * wm + l16;
        i32x8_t x = ld32(S, xo0, xo1);
        float xs = xsp[0];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          i32x8_t xn = x;
          float xsn = xs;
          if (j + 1 < NJ) {  // next tile's fragment, one tile ahead
            xn = ld32(S + (j + 1) * 16 * ROWB, xo0, xo1);
            xsn = xsp[16 * (j + 1)];
          }
          f32x4_t pr[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) pr[i] = mfma16(w[i], x);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float sc = xs * ws[i];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += pr[i][r] * sc;
          }
          x = xn;
          xs = xsn;
        }
      }
    }
  };
  switch (nj) {
    case 10: kloop(std::integral_constant<int, 10>{}); break;
    case 9: kloop(std::integral_constant<int, 9>{}); break;
    case 8: kloop(std::integral_constant<int, 8>{}); break;
    case 7: kloop(std::integral_constant<int, 7>{}); break;
    case 6: kloop(std::integral_constant<int, 6>{}); break;
    case 5: kloop(std::integral_constant<int, 5>{}); break;
    case 4: kloop(std::integral_constant<int, 4>{}); break;
    case 3: kloop(std::integral_constant<int, 3>{}); break;
    case 2: kloop(std::integral_constant<int, 2>{}); break;
    case 1: kloop(std::integral_constant<int, 1>{}); break;
    default: kloop(std::integral_constant<int, 0>{}); break;
  }
  static_assert(TJ == 10, "kloop variants cover 0..TJ activation tiles");

  // ---- epilogue
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  __syncthreads();  // the ring is free
  // output column of (tile i, reg r): GLU tiles 0,1 are gate rows whose up
  // rows are tiles 2,3 in the same lanes
  auto tcol = [&](int i, int r) -> int {
    return (kGlu ? 32 * wn + 16 * i : 64 * wn + 16 * i) + 4 * g + r;
  };
  constexpr int NI = kGlu ? 2 : 4;
  // bias, rounding and activation of (tile i, activation tile j)
  auto outv = [&](int i, int j, float (&o)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float bg = 0.f, bu = 0.f;
      if (a.bias) {
        const int64_t n = n0 + tcol(i, r);
        if (n < N) {
          bg = ld16<F16>(a.bias[bias_base + n]);
          if constexpr (kGlu) bu = ld16<F16>(a.bias[bias_base + a.up_off + n]);
        }
      }
      float gv = round16<F16>(acc[i][j][r] + bg);
      if constexpr (kGlu) {
        float u = round16<F16>(acc[i + 2][j][r] + bu);
        glu_clamp(a, n0 + tcol(i, r), gv, u);
        float y;
        if (a.act == MI355MOE_ACT_SILU) {
          y = round16<F16>(x_sigmoid(gv, 1.f)) * u;
        } else {
          gv = gv > a.limit ? a.limit : gv;
          u = u > a.limit ? a.limit : (u < -a.limit ? -a.limit : u);
          y = (u + 1.f) * x_sigmoid(gv, a.alpha);
        }
        gv = round16<F16>(y);
      }
      o[r] = gv;
    }
  };

  if constexpr (QOUT) {
    // e4m3 activation with one fp32 scale per (slot, 128 columns): the four
    // waves with the same wm cover the tile's 128 columns (N % 128 == 0).
    // Lane l holds slots 160 wm + 16 j + l%16; lanes l, l+16, l+32, l+48 hold
    // the same slot.  Row maxima go to LDS after the staged tile.
    constexpr int PITCH = NOUT + 16;
    float (*s_amax)[BM] = reinterpret_cast<float (*)[BM]>(lds + BM * PITCH);
    float ov[NI][TJ][4];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      float m = 1e-10f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        outv(i, j, ov[i][j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(ov[i][j][r]));
      }
      m = max_over_rows(m);
      if (g == 0) s_amax[wn][(BM / 2) * wm + 16 * j + l16] = m;
    }
    __syncthreads();
    float* ds = static_cast<float*>(qs);
    const int64_t ngroups = N / 128;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int row = (BM / 2) * wm + 16 * j + l16;
      const float am = fmaxf(fmaxf(s_amax[0][row], s_amax[1][row]),
                             fmaxf(s_amax[2][row], s_amax[3][row]));
      const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
      const float inv = 1.0f / sc;
      const int drow = s_drow[row];
      if (wn == 0 && g == 0 && drow >= 0) ds[static_cast<int64_t>(drow) * ngroups + ntile] = sc;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint32_t w = e4m3x4_sat(ov[i][j][0] * inv, ov[i][j][1] * inv, ov[i][j][2] * inv,
                                      ov[i][j][3] * inv);
        *reinterpret_cast<uint32_t*>(lds + row * PITCH + tcol(i, 0)) = w;
      }
    }
    __syncthreads();
    uint8_t* dq = static_cast<uint8_t*>(a.D);
    constexpr int CPR = NOUT / 16;
    for (int idx = tid; idx < BM * CPR; idx += 512) {
      const int row = idx / CPR, ch = idx % CPR;
      const int drow = s_drow[row];
      if (drow < 0) continue;
      *reinterpret_cast<uint4*>(dq + static_cast<int64_t>(drow) * N + n0 + ch * 16) =
          *reinterpret_cast<const uint4*>(lds + row * PITCH + ch * 16);
    }
  } else {
    // 16-bit output staged in LDS (STORE tiles in two passes of 160 rows,
    // one per wave half) and written with 16-byte row-contiguous stores
    constexpr int PITCH = 2 * NOUT + 16;
    constexpr int PASSES = BM * PITCH <= RING ? 1 : 2;
    constexpr int PROWS = BM / PASSES;
    uint16_t* d = static_cast<uint16_t*>(a.D);
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(a.D) & 15) == 0;
    constexpr int CPR = 2 * NOUT / 16;
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
      if (PASSES == 1 || wm == pass) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            float o[4];
            outv(i, j, o);
            const int srow = (BM / 2) * wm + 16 * j + l16 - pass * PROWS;
            const uint32_t lo = to16<F16>(o[0]) | (to16<F16>(o[1]) << 16);
            const uint32_t hi = to16<F16>(o[2]) | (to16<F16>(o[3]) << 16);
            *reinterpret_cast<uint2*>(lds + srow * PITCH + 2 * tcol(i, 0)) = make_uint2(lo, hi);
          }
      }
      __syncthreads();
      for (int idx = tid; idx < PROWS * CPR; idx += 512) {
        const int srow = idx / CPR, ch = idx % CPR;
        const int drow = s_drow[pass * PROWS + srow];
        const int64_t col = n0 + ch * 8;
        if (drow < 0 || col >= N) continue;
        const uint4 val = *reinterpret_cast<const uint4*>(lds + srow * PITCH + ch * 16);
        uint16_t* dst = d + static_cast<int64_t>(drow) * N + col;
        if (vec) {
          *reinterpret_cast<uint4*>(dst) = val;
        } else {
          const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (col + k < N) dst[k] = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
        }
      }
      if (pass + 1 < PASSES) __syncthreads();  // the staging area is rewritten
    }
  }
}

template <int EPI, bool QOUT, bool F16>
int launch_w8(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_wide8_kernel<EPI, QOUT, F16><<<grid, dim3(512), 0, st>>>(a, qs);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace

bool wide8_supported(int recipe, const GemmArgs& a) {
  // MX weight codes move 4 tile rows per lane: row counts and the up-row
  // offset in whole 4-byte words
  const bool codes4 = a.ldb_rows % 4 == 0 && a.up_off % 4 == 0 && a.N % 4 == 0;
  if (recipe == RECIPE_MX4A4)
    return a.w_kblock && codes4 && a.a_mxs_ld % 4 == 0 && a.K % 32 == 0 && a.K > 0;
  return (recipe == MI355MOE_RECIPE_FP8BLOCK ||
          (recipe == MI355MOE_RECIPE_MXFP8 && a.w_kblock && codes4 && a.a_mxs_ld % 4 == 0)) &&
         a.K % 128 == 0 && a.K > 0 && a.K / 128 <= MAX_KBLK;
}

bool wide8_shape_ok(int64_t a_rows, int64_t ldb_rows, int64_t K) {
  const int64_t lim = int64_t(1) << 32;
  return K % 128 == 0 && K > 0 && K / 128 <= MAX_KBLK && a_rows * K < lim && ldb_rows * K < lim;
}

bool wide8_shape_ok_mx4(int64_t a_rows, int64_t ldb_rows, int64_t K) {
  const int64_t lim = int64_t(1) << 32;
  return K % 32 == 0 && K > 0 && a_rows * (K / 2) < lim && ldb_rows * (K / 2) < lim;
}

// kWideBM-slot blocks; fp8 block-scaled (or mxfp8, K-blocked) weights,
// K % 128 == 0, K <= 8192.
int launch_moe_gemm_wide8(int recipe, int epi, bool qout, const GemmArgs& a,
                          int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  MI_ARG(wide8_supported(recipe, a), "fp8 prefill GEMM: needs K % 128 == 0 and K <= 8192");
  // activation rows: tokens (gathered) or padded slots (by position)
  const int64_t a_rows = a.a_by_pos ? max_blocks * BM : a.num_valid;
  MI_ARG(recipe == RECIPE_MX4A4 ? wide8_shape_ok_mx4(a_rows, a.ldb_rows, a.K)
                                 : wide8_shape_ok(a_rows, a.ldb_rows, a.K),
         "fp8 prefill GEMM: activation and per-expert weight bytes must stay below 4 GiB");
  static const bool v1 = [] {
    const char* e = getenv("MI355MOE_WIDE8");
    return e && !strcmp(e, "v1");
  }();
  if (qout)
    MI_ARG(epi == EPI_GLU && a.N % (recipe == RECIPE_MX4A4 ? 32 : 128) == 0,
           "fp8 activation output needs the GLU epilogue and I % 128 == 0 (mxfp4: % 32)");
  if (!v1 || recipe == MI355MOE_RECIPE_MXFP8 || recipe == RECIPE_MX4A4)
    return launch_moe_gemm_wide8p(recipe, epi, qout, a, max_blocks, qs, st);
  if (qout) {
    return a.out_f16 ? launch_w8<EPI_GLU, true, true>(a, max_blocks, qs, st)
                     : launch_w8<EPI_GLU, true, false>(a, max_blocks, qs, st);
  }
  if (epi == EPI_GLU)
    return a.out_f16 ? launch_w8<EPI_GLU, false, true>(a, max_blocks, qs, st)
                     : launch_w8<EPI_GLU, false, false>(a, max_blocks, qs, st);
  return a.out_f16 ? launch_w8<EPI_STORE, false, true>(a, max_blocks, qs, st)
                   : launch_w8<EPI_STORE, false, false>(a, max_blocks, qs, st);
}

}  // namespace mi355
