// Prefill grouped GEMM for fp8 e4m3 weights with 128x128 block scales and
// e4m3 activations with 1x128 scales: 128-slot x 256-weight-row tiles, 8
// waves, 3-slot LDS ring fed by direct global->LDS DMA.  The 128-slot
// member of the fp8 prefill family (about 100-160 slots per expert, or
// skewed routing): a 48.5 KB stage keeps two stages of DMA in flight.
//
// Waves.  Eight waves, two per SIMD (waves w and w + 4 share SIMD w % 4), each
// owning 64 slots x 64 weight rows: 4 x 4 tiles of the 16x16x128 e4m3 MFMA
// with the weight as the A operand.  One MFMA covers one whole 128-K scale
// block, so its result is scaled and added at once (acc += p * xs * ws, one
// FMA per output element per block) and the partial products never outlive
// the instruction that made them; the FMAs of one tile run while the MFMAs
// of the next do.
//
// Stages.  A stage holds 128 K elements (128 bytes) of the 128 activation
// rows and 256 weight rows plus the block's 128 activation scales: 48.5 KB,
// written by 48 global_load_lds_dwordx4 (8 rows x 128 B each) and two
// global_load_lds_dword.  16-byte chunk c of row r sits at slot
// c ^ ((r >> 1) & 7), so sixteen rows read at one logical chunk hit sixteen
// distinct bank groups.
//
// Pipeline.  A wave computes stage kt from registers and reads stage kt+1's
// fragments into the same registers as the MFMAs release them; the barrier
// before stage kt's MFMAs certifies that every wave's reads of stage kt are
// complete, so the DMA of stage kt+3 goes into that slot while stage kt
// computes (two stages of lookahead in three slots).
//
// Tiles, GLU pairing and the fp8 activation output are those of the 128x256
// kernels: a GLU tile's 256 weight rows are 128 gate rows and the matching
// 128 up rows, so its 128 output columns are one whole 1x128 quantisation
// group of the next GEMM's input.
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int BM = 128, BN = 256, ROWB = 128, KE = 128;
constexpr int A_BYTES = BM * ROWB;                 // 16 KB
constexpr int W_BYTES = BN * ROWB;                 // 32 KB
constexpr int S_OFF = A_BYTES + W_BYTES;           // activation scales
constexpr int STAGE = S_OFF + BM * 4;              // 48.5 KB
constexpr int NSTAGE = 3;
constexpr int DMA_PER_WAVE = (A_BYTES + W_BYTES) / 1024 / 8;  // 6
constexpr int MAX_KBLK = 64;                       // K <= 8192
constexpr int EPI_BYTES = BM * (2 * 256 + 16);     // largest staged output tile

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)p));
}
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(lds_base) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// wave-uniform number of DMA instructions allowed to stay outstanding
__device__ __forceinline__ void wait_vm_dyn(int n) {
  switch (n) {
    case 6: wait_vm<6>(); break;
    case 8: wait_vm<8>(); break;
    case 12: wait_vm<12>(); break;
    case 16: wait_vm<16>(); break;
    default: wait_vm<0>(); break;  // 0, and never less strict than needed
  }
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

// Fragments of one wave: [j] activation tiles (slots 64 wm + 16 j + l%16),
// [i] weight tiles; two 16-byte chunks each (K [32g, 32g + 32) of the stage,
// g = l / 16).
typedef i32x8_t XFrag[4];
typedef i32x8_t WFrag[4];

// Tile rows start at multiples of 16, where the slot swizzle (r >> 1) & 7
// depends on r % 16 only: one base offset per chunk, tiles at constant
// distances (16 rows = 2 KB).
__device__ __forceinline__ void read_x(XFrag& x, const uint8_t* S, const int (&xo)[2]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = ld32(S + j * 16 * ROWB, xo[0], xo[1]);
}
template <bool kGlu>
__device__ __forceinline__ void read_w(WFrag& w, int i0, const uint8_t* S, const int (&wo)[2]) {
#pragma unroll
  for (int i = i0; i < i0 + 2; ++i) {
    const int t = kGlu ? (i < 2 ? 0 : 128) + 16 * (i & 1) : 16 * i;  // tile row - wave row
    w[i] = ld32(S + t * ROWB, wo[0], wo[1]);
  }
}

template <int EPI, bool QOUT, bool F16>
__global__ __launch_bounds__(512) void moe_gemm_big8_kernel(const GemmArgs a, void* __restrict__ qs) {
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns per tile

  __shared__ __attribute__((aligned(1024))) uint8_t lds[NSTAGE * STAGE > EPI_BYTES ? NSTAGE * STAGE : EPI_BYTES];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ float s_wsc[4][MAX_KBLK];  // weight-block scales of the tile's four 64-row quarters
  __shared__ float s_amax[4][BM];       // QOUT: per-wave-column row maxima

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

  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    const bool ok = rid >= 0 && rid < a.num_valid;
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
  {
    const float* bsc = static_cast<const float*>(a.b_scale);
    const int wsh = 7 - a.ws_rows64;  // weight rows per scale row: 128 or 64
    for (int i = tid; i < 4 * nkb; i += 512) {
      const int t = i / nkb, kb = i % nkb;
      const int64_t wr = wrow_of(64 * t) >> wsh;
      s_wsc[t][kb] = bsc[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + wr) * nkb + kb];
    }
  }
  __syncthreads();

  // DMA sources: blocks b = 6 wave + q of a stage, activation rows for b < 16
  // (8 rows each), weight rows after; wave 0 also moves the activation
  // scales of the stage's 128-K block (128 floats, two 256-byte DMAs).
  // weights may be K-blocked: bytes between two K stages of a weight row
  const WStride wst = w_stride8(a);
  auto kstep = [&](int q) -> int64_t {  // uniform: activation or weight source
    return DMA_PER_WAVE * wave + q < 16 ? static_cast<int64_t>(ROWB) : wst.kblk;
  };
  const uint8_t* src[DMA_PER_WAVE];
  {
    const uint8_t* abase = static_cast<const uint8_t*>(a.A);
    const uint8_t* wexp = static_cast<const uint8_t*>(a.B) +
                          static_cast<int64_t>(e) * a.ldb_rows * K;
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q) {
      const int b = DMA_PER_WAVE * wave + q;
      const int r = (b < 16 ? b : b - 16) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz(r);
      if (b < 16) {
        const int ar = s_arow[r];
        src[q] = abase + static_cast<int64_t>(ar >= 0 ? ar : 0) * K + c * 16;
      } else {
        src[q] = wexp + wrow_of(r) * wst.row + c * 16;
      }
    }
  }
  const int nd = DMA_PER_WAVE + (wave == 0 ? 2 : 0);
  const float* ssrc0 = a.a_scale;
  const float* ssrc1 = a.a_scale;
  // scale step from one K stage to the next: 1 (row-major) or the by-position
  // pitch, whose 128 scales of a stage are four cache lines
  const int64_t sstep = a.a_scale_tld ? a.a_scale_tld : 1;
  if (wave == 0) {
    if (a.a_scale_tld) {
      ssrc0 += static_cast<int64_t>(blk) * BM + lane;
      ssrc1 += static_cast<int64_t>(blk) * BM + 64 + lane;
    } else {
      const int r0 = s_arow[lane], r1 = s_arow[64 + lane];
      ssrc0 += static_cast<int64_t>(r0 >= 0 ? r0 : 0) * nkb;
      ssrc1 += static_cast<int64_t>(r1 >= 0 ? r1 : 0) * nkb;
    }
  }
  const uint32_t ring0 = lds_off(lds);
  const uint32_t dst0 = DMA_PER_WAVE * wave * 1024;
  auto issue = [&](int kt) {
    const uint32_t base = ring0 + (kt % NSTAGE) * STAGE;
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q)
      dma16(src[q] + kt * kstep(q), __builtin_amdgcn_readfirstlane(base + dst0 + q * 1024));
    if (wave == 0) {
      dma4(ssrc0 + kt * sstep, __builtin_amdgcn_readfirstlane(base + S_OFF));
      dma4(ssrc1 + kt * sstep, __builtin_amdgcn_readfirstlane(base + S_OFF + 256));
    }
  };

  // fragment offsets: chunks 2g and 2g + 1 of the wave's first activation /
  // weight row + l%16
  int xo[2], wo[2];
  {
    const int mx = 64 * wm + l16;
    const int rw = (kGlu ? 32 * wn : 64 * wn) + l16;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int ch = 2 * g + c;
      xo[c] = mx * ROWB + ((ch ^ swz(mx)) << 4);
      wo[c] = A_BYTES + rw * ROWB + ((ch ^ swz(rw)) << 4);
    }
  }
  // s_wsc quarter of weight tile i: GLU tile rows 128 (i / 2) + 32 wn + 16 (i % 2),
  // STORE 64 wn + 16 i
  int wblk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wblk[i] = kGlu ? 2 * (i >> 1) + (wn >> 1) : wn;

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = static_cast<int>(K / KE);
  for (int s = 0; s < NSTAGE && s < nk; ++s) issue(s);
  XFrag xf;
  WFrag wf;
  wait_vm_dyn(nd * ((nk - 1) < NSTAGE - 1 ? (nk - 1) : NSTAGE - 1));
  __builtin_amdgcn_s_barrier();
  read_x(xf, lds, xo);
  read_w<kGlu>(wf, 0, lds, wo);
  read_w<kGlu>(wf, 2, lds, wo);

  // Stage kt.  Its fragments are in registers; the barrier publishes stage
  // kt+1 and certifies that every wave's reads of stage kt are complete
  // (lgkmcnt(0) before it), so the DMA of stage kt+3 goes into that slot
  // between the MFMAs.  Stage kt+1's fragments replace those of stage kt,
  // each group right after the MFMAs that last read it.
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    const uint8_t* cur = lds + (kt % NSTAGE) * STAGE;
    const uint8_t* nxt = lds + ((kt + 1) % NSTAGE) * STAGE;
    float xs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xs[j] = reinterpret_cast<const float*>(cur + S_OFF)[64 * wm + 16 * j + l16];
    float ws[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ws[i] = s_wsc[wblk[i]][kt];
    if (more) {
      // stage kt+1 landed (stage kt+2 may pend)
      const int issued = (kt + NSTAGE - 1 < nk ? kt + NSTAGE - 1 : nk - 1);
      wait_vm_dyn(nd * (issued - (kt + 1)));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const bool dma = kt + NSTAGE < nk;
    const uint32_t dbase = ring0 + (kt % NSTAGE) * STAGE;
    const int kn = kt + NSTAGE;  // stage whose DMA goes out in this iteration
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // four MFMAs in flight, then their scale FMAs
      f32x4_t pr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) pr[j] = mfma16(wf[i], xf[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float sc = xs[j] * ws[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] += pr[j][r] * sc;
      }
      __builtin_amdgcn_sched_barrier(0);
      if (dma) {
        // DMA instructions 2i, 2i + 1 of stage kt+3 (and wave 0's scales)
#pragma unroll
        for (int q = 2 * i; q < 2 * i + 2; ++q)
          if (q < DMA_PER_WAVE)
            dma16(src[q] + kn * kstep(q), __builtin_amdgcn_readfirstlane(dbase + dst0 + q * 1024));
        if (i == 3 && wave == 0) {
          dma4(ssrc0 + (kt + NSTAGE) * sstep, __builtin_amdgcn_readfirstlane(dbase + S_OFF));
          dma4(ssrc1 + (kt + NSTAGE) * sstep, __builtin_amdgcn_readfirstlane(dbase + S_OFF + 256));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage kt+1's fragments (after the last stage: a stale slot, unused;
    // unconditional so the loads land in the loop-carried registers)
    read_w<kGlu>(wf, 0, nxt, wo);
    read_w<kGlu>(wf, 2, nxt, wo);
    read_x(xf, nxt, xo);
  }

  // ---- epilogue
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  __syncthreads();  // the ring is free
  // output column of (tile i, reg r): GLU tiles 0,1 are gate rows whose up
  // rows are tiles 2,3 in the same lanes
  auto tcol = [&](int i, int r) -> int {
    return (kGlu ? 32 * wn + 16 * i : 64 * wn + 16 * i) + 4 * g + r;
  };
  constexpr int NI = kGlu ? 2 : 4;
  float ov[NI][4][4];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float bg[4], bu[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bg[r] = 0.f;
      bu[r] = 0.f;
      if (a.bias) {
        const int64_t n = n0 + tcol(i, r);
        if (n < N) {
          bg[r] = ld16<F16>(a.bias[bias_base + n]);
          if constexpr (kGlu) bu[r] = ld16<F16>(a.bias[bias_base + a.up_off + n]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float gv = round16<F16>(acc[i][j][r] + bg[r]);
        if constexpr (kGlu) {
          float u = round16<F16>(acc[i + 2][j][r] + bu[r]);
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
        ov[i][j][r] = gv;
      }
    }
  }

  if constexpr (QOUT) {
    // e4m3 activation with one fp32 scale per (slot, 128 columns): the four
    // waves with the same wm cover the tile's 128 columns (N % 128 == 0).
    // Lane l holds slots 64 wm + 16 j + l%16; lanes l, l+16, l+32, l+48 hold
    // the same slot.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float m = 1e-10f;
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(ov[i][j][r]));
      m = max_over_rows(m);
      if (g == 0) s_amax[wn][64 * wm + 16 * j + l16] = m;
    }
    __syncthreads();
    constexpr int PITCH = NOUT + 16;
    float* ds = static_cast<float*>(qs);
    const int64_t ngroups = N / 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 64 * wm + 16 * j + l16;
      const float am = fmaxf(fmaxf(s_amax[0][row], s_amax[1][row]),
                             fmaxf(s_amax[2][row], s_amax[3][row]));
      const float sc = fmaxf(am / 448.f, 1.0f / (448.f * 512.f));
      const float inv = 1.0f / sc;
      const int drow = s_drow[row];
      if (wn == 0 && g == 0 && drow >= 0) {
        if (a.q_scale_tld) ds[static_cast<int64_t>(ntile) * a.q_scale_tld + drow] = sc;
        else ds[static_cast<int64_t>(drow) * ngroups + ntile] = sc;
      }
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
    constexpr int PITCH = 2 * NOUT + 16;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 64 * wm + 16 * j + l16;
        const uint32_t lo = to16<F16>(ov[i][j][0]) | (to16<F16>(ov[i][j][1]) << 16);
        const uint32_t hi = to16<F16>(ov[i][j][2]) | (to16<F16>(ov[i][j][3]) << 16);
        *reinterpret_cast<uint2*>(lds + row * PITCH + 2 * tcol(i, 0)) = make_uint2(lo, hi);
      }
    __syncthreads();
    uint16_t* d = static_cast<uint16_t*>(a.D);
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(a.D) & 15) == 0;
    constexpr int CPR = 2 * NOUT / 16;
    for (int idx = tid; idx < BM * CPR; idx += 512) {
      const int row = idx / CPR, ch = idx % CPR;
      const int drow = s_drow[row];
      const int64_t col = n0 + ch * 8;
      if (drow < 0 || col >= N) continue;
      const uint4 val = *reinterpret_cast<const uint4*>(lds + row * PITCH + ch * 16);
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
  }
}

template <int EPI, bool QOUT, bool F16>
int launch_b8(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_big8_kernel<EPI, QOUT, F16><<<grid, dim3(512), 0, st>>>(a, qs);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace

bool big8_supported(int recipe, const GemmArgs& a) {
  return recipe == MI355MOE_RECIPE_FP8BLOCK && a.K % 128 == 0 && a.K > 0 &&
         a.K / 128 <= MAX_KBLK;
}

// 128-slot blocks; fp8 block-scaled weights, K % 128 == 0, K <= 8192.
int launch_moe_gemm_big8(int recipe, int epi, bool qout, const GemmArgs& a,
                          int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  MI_ARG(big8_supported(recipe, a), "fp8 prefill GEMM: needs K % 128 == 0 and K <= 8192");
  if (qout) {
    MI_ARG(epi == EPI_GLU && a.N % 128 == 0,
           "fp8 activation output needs the GLU epilogue and I % 128 == 0");
    return a.out_f16 ? launch_b8<EPI_GLU, true, true>(a, max_blocks, qs, st)
                     : launch_b8<EPI_GLU, true, false>(a, max_blocks, qs, st);
  }
  if (epi == EPI_GLU)
    return a.out_f16 ? launch_b8<EPI_GLU, false, true>(a, max_blocks, qs, st)
                     : launch_b8<EPI_GLU, false, false>(a, max_blocks, qs, st);
  return a.out_f16 ? launch_b8<EPI_STORE, false, true>(a, max_blocks, qs, st)
                   : launch_b8<EPI_STORE, false, false>(a, max_blocks, qs, st);
}

}  // namespace mi355
