// Prefill grouped GEMM with a 3-stage LDS ring fed by direct global->LDS DMA.
//
// Tile and wave layout are those of the 128x256 kernel (gemm32_common.h):
// 128 sorted slots x 256 weight rows, 4 waves as 2 x 2, 32x32 MFMA with the
// weight as the A operand.  Every K stage moves 128 bytes of each of the 128
// activation rows and 256 weight rows (64 bf16 or 128 e4m3 elements) with
// global_load_lds_dwordx4: lane l of one instruction writes LDS bytes
// [16l, 16l+16) of a 1 KB block holding 8 rows, so rows are stored
// unpadded and the 16-byte chunk c of row r is placed at slot c ^ ((r>>1)&7)
// (the source address is permuted, the LDS side is linear) to keep the
// fragment reads free of bank conflicts.
//
// Pipeline: stages k and k+1 are in flight while stage k-1 is computed; each
// wave waits for its own DMAs with an explicit vmcnt, then one s_barrier
// publishes the stage.  The DMAs are issued from inline assembly so that the
// compiler's wait-count pass, which cannot tell the ring's buffers apart,
// does not drain the whole pipeline before every LDS read; for the same
// reason the K loop issues no other global loads (fp8 weight-block scales are
// staged in LDS up front, activation scales travel with the stage's DMA).
#include "gemm32_common.h"

namespace mi355 {
namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int BM = 128, BN = 256, ROWB = 128;
constexpr int A_BYTES = BM * ROWB;            // 16 KB
constexpr int W_BYTES = BN * ROWB;            // 32 KB
constexpr int S_BYTES = BM * 4;               // fp8 activation scales
constexpr int STAGE = A_BYTES + W_BYTES + S_BYTES;
constexpr int NSTAGE = 3;
constexpr int DMA_PER_WAVE = (A_BYTES + W_BYTES) / 1024 / 4;  // 12
constexpr int MAX_KBLK = 64;                  // fp8: K/128 staged scales per row block

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

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

template <int RECIPE, int EPI, bool QOUT, bool F16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void moe_gemm_pipe_kernel(const GemmArgs a,
                                                               void* __restrict__ qs) {
  constexpr bool kFp8 = RECIPE == MI355MOE_RECIPE_FP8BLOCK;
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int KE = kFp8 ? 128 : 64;  // K elements per stage
  constexpr int XB = kFp8 ? 1 : 2;

  __shared__ __attribute__((aligned(1024))) uint8_t ring[NSTAGE * STAGE];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ float s_amax[2][128];
  __shared__ float s_wsc[4][MAX_KBLK];  // fp8: weight-block scales of the tile's four 64-row quarters

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;
  // XCD-aware tile order.  Workgroups are dealt round-robin to the 8 XCDs;
  // give XCD x the contiguous range [x*per, (x+1)*per) of the valid tiles
  // (ordered by tile_coords), so the tiles that share an expert's weight rows
  // or a block's activation rows meet in the same L2.
  // The 1-D grid is a multiple of 8 and >= the tile upper bound, so every
  // XCD receives at least `per` workgroups.
  const int n_tiles = static_cast<int>((a.N + (kGlu ? 127 : BN - 1)) / (kGlu ? 128 : BN));
  const int valid = (*a.ntp / BM) * n_tiles;
  const int bid = static_cast<int>(blockIdx.x);
  const int per = (valid + 7) / 8;
  const int tile = (bid & 7) * per + (bid >> 3);
  if ((bid >> 3) >= per || tile >= valid) return;  // uniform
  int blk, ntile;
  tile_coords(a, tile, n_tiles, BM, blk, ntile);
  const int e = a.block_expert[blk];
  const int64_t K = a.K;
  const int64_t N = a.N;
  const int64_t n0 = static_cast<int64_t>(ntile) * (kGlu ? 128 : BN);
  const int64_t wrow_bytes = K * XB;

  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    const bool ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }
  // weight row staged at tile row r (rows past N read row 0: finite data whose
  // outputs are never stored)
  auto wrow_of = [&](int r) -> int64_t {
    if constexpr (kGlu) {
      const int64_t c = n0 + (r & 127);
      return (r >= 128 ? a.up_off : 0) + (c < N ? c : 0);
    } else {
      const int64_t c = n0 + r;
      return c < N ? c : 0;
    }
  };
  if constexpr (kFp8) {
    // the scale rows of tile rows 64 t .. 64 t + 63 (t < 4): non-GLU weight
    // rows n0 + 64 t; GLU gate rows n0 + 64 t (t < 2), up rows up_off + n0 +
    // 64 (t - 2); one scale row per 128 weight rows, or per 64 (ws_rows64)
    const int nkb = static_cast<int>(K / 128);
    const float* bsc = static_cast<const float*>(a.b_scale);
    const int wsh = 7 - a.ws_rows64;
    for (int i = tid; i < 4 * nkb; i += 256) {
      const int t = i / nkb, kb = i % nkb;
      const int64_t wr = wrow_of(64 * t) >> wsh;
      s_wsc[t][kb] = bsc[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + wr) * nkb + kb];
    }
  }
  __syncthreads();

  // ---- DMA sources of this wave's 12 instructions per stage (+2 for wave 0
  //      under fp8: the 128 activation scales)
  const uint8_t* src[DMA_PER_WAVE];
  uint32_t dst[DMA_PER_WAVE];
  const uint8_t* abase = static_cast<const uint8_t*>(a.A);
  const uint8_t* wexp = static_cast<const uint8_t*>(a.B) +
                        static_cast<int64_t>(e) * a.ldb_rows * wrow_bytes;
  const uint32_t ring0 = lds_off(ring);
#pragma unroll
  for (int i = 0; i < DMA_PER_WAVE; ++i) {
    const int blk1k = wave * DMA_PER_WAVE + i;          // 1 KB block of the stage
    const int r = (blk1k & 15) * 8 + (lane >> 3);       // row within its region
    const int c = (lane & 7) ^ swz(r);                  // source chunk for this slot
    if (blk1k < 16) {                                    // activation rows
      const int ar = s_arow[r];
      src[i] = abase + static_cast<int64_t>(ar >= 0 ? ar : 0) * K * XB + c * 16;
    } else {                                             // weight rows
      const int wr = (blk1k - 16) * 8 + (lane >> 3);
      src[i] = wexp + wrow_of(wr) * wrow_bytes + c * 16;
    }
    dst[i] = blk1k * 1024;
  }
  const float* ssrc = nullptr;
  if constexpr (kFp8) {
    if (wave == 0) {
      const int ar0 = s_arow[lane], ar1 = s_arow[64 + lane];
      (void)ar1;
      ssrc = a.a_scale + static_cast<int64_t>(ar0 >= 0 ? ar0 : 0) * (K / 128);
    }
  }
  const float* ssrc1 = nullptr;
  if constexpr (kFp8) {
    if (wave == 0) {
      const int ar1 = s_arow[64 + lane];
      ssrc1 = a.a_scale + static_cast<int64_t>(ar1 >= 0 ? ar1 : 0) * (K / 128);
    }
  }

  auto issue = [&](int kt, int buf) {
    const uint32_t base = ring0 + buf * STAGE;
    const int64_t koff = static_cast<int64_t>(kt) * ROWB;
#pragma unroll
    for (int i = 0; i < DMA_PER_WAVE; ++i)
      dma16(src[i] + koff, __builtin_amdgcn_readfirstlane(base + dst[i]));
    if constexpr (kFp8) {
      if (wave == 0) {
        dma4(ssrc + kt, __builtin_amdgcn_readfirstlane(base + A_BYTES + W_BYTES));
        dma4(ssrc1 + kt, __builtin_amdgcn_readfirstlane(base + A_BYTES + W_BYTES + 256));
      }
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  int wtile_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kGlu)
      wtile_row[i] = (i < 2 ? 0 : 128) + 64 * wn + 32 * (i & 1);
    else
      wtile_row[i] = 128 * wn + 32 * i;
  }

  const int nk = static_cast<int>(K / KE);
  issue(0, 0);
  if (nk > 1) issue(1, 1);
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt % NSTAGE;
    if (kt + 1 < nk) {
      if (kFp8 && wave == 0) wait_vm<DMA_PER_WAVE + 2>();
      else wait_vm<DMA_PER_WAVE>();
    } else {
      wait_vm<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (kt + 2 < nk) issue(kt + 2, (kt + 2) % NSTAGE);

    const uint8_t* As = ring + cur * STAGE;
    const uint8_t* Ws = As + A_BYTES;
    if constexpr (kFp8) {
      const float* xsc = reinterpret_cast<const float*>(Ws + W_BYTES);
      float ws[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ws[i] = s_wsc[wtile_row[i] >> 6][kt];  // 32-row tiles: one quarter
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = 64 * wm + 32 * j + l32;
        const uint8_t* xr = As + m * ROWB;
        const int sw = swz(m);
        const uint4 x0 = *reinterpret_cast<const uint4*>(xr + (((2 * h) ^ sw) << 4));
        const uint4 x1 = *reinterpret_cast<const uint4*>(xr + (((2 * h + 1) ^ sw) << 4));
        const uint4 x2 = *reinterpret_cast<const uint4*>(xr + (((4 + 2 * h) ^ sw) << 4));
        const uint4 x3 = *reinterpret_cast<const uint4*>(xr + (((5 + 2 * h) ^ sw) << 4));
        const float xs = xsc[m];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int wr = wtile_row[i] + l32;
          const uint8_t* wp = Ws + wr * ROWB;
          const int swr = swz(wr);
          f32x16 p;
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = 0.f;
          p = mfma32_fp8(*reinterpret_cast<const uint4*>(wp + (((2 * h) ^ swr) << 4)),
                         *reinterpret_cast<const uint4*>(wp + (((2 * h + 1) ^ swr) << 4)),
                         x0, x1, p);
          p = mfma32_fp8(*reinterpret_cast<const uint4*>(wp + (((4 + 2 * h) ^ swr) << 4)),
                         *reinterpret_cast<const uint4*>(wp + (((5 + 2 * h) ^ swr) << 4)),
                         x2, x3, p);
          const float s = xs * ws[i];
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += p[r] * s;
        }
      }
    } else {
      // read every fragment of the stage into its own registers first, so
      // the MFMAs of step ks overlap the LDS latency of steps ks+1..3
      uint4 xf[4][2], wf[4][4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = 2 * ks + h;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = 64 * wm + 32 * j + l32;
          xf[ks][j] = *reinterpret_cast<const uint4*>(As + m * ROWB + ((c ^ swz(m)) << 4));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int wr = wtile_row[i] + l32;
          wf[ks][i] = *reinterpret_cast<const uint4*>(Ws + wr * ROWB + ((c ^ swz(wr)) << 4));
        }
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma16_32x32x16<F16>(wf[ks][i], xf[ks][j], acc[i][j]);
      // keep the 24 LDS reads ahead of the 32 MFMAs (the default schedule
      // re-interleaves them one pair at a time and exposes LDS latency)
      __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
    }
  }

  static_assert(sizeof(ring) >= 128 * (2 * 256 + 16), "epilogue staging");
  epilogue_32x32<kGlu, QOUT, F16>(a, qs, acc, e, n0, wm, wn, l32, h, s_drow, s_amax, ntile, ring);
}

template <int RECIPE, int EPI, bool QOUT, bool F16>
int launch_pipe_t(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : BN;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_pipe_kernel<RECIPE, EPI, QOUT, F16><<<grid, dim3(256), 0, st>>>(a, qs);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
template <int RECIPE, int EPI, bool QOUT>
int launch_pipe(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  return a.out_f16 ? launch_pipe_t<RECIPE, EPI, QOUT, true>(a, max_blocks, qs, st)
                   : launch_pipe_t<RECIPE, EPI, QOUT, false>(a, max_blocks, qs, st);
}

}  // namespace

bool pipe_supported(int recipe, const GemmArgs& a) {
  if (recipe == MI355MOE_RECIPE_FP8BLOCK) return a.K % 128 == 0 && a.K / 128 <= MAX_KBLK;
  if (recipe == MI355MOE_RECIPE_BF16) return a.K % 64 == 0;
  return false;
}

// 128-slot blocks; K % 64 (bf16) or K % 128 (fp8) == 0.
int launch_moe_gemm_pipe(int recipe, int epi, bool qout, const GemmArgs& a,
                         int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  MI_ARG(pipe_supported(recipe, a), "pipelined GEMM: unsupported recipe or K");
  if (qout) {
    MI_ARG(recipe == MI355MOE_RECIPE_FP8BLOCK && epi == EPI_GLU && a.N % 128 == 0,
           "fp8 activation output needs the fp8block recipe and I % 128 == 0");
    return launch_pipe<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, true>(a, max_blocks, qs, st);
  }
  if (recipe == MI355MOE_RECIPE_FP8BLOCK)
    return epi == EPI_GLU ? launch_pipe<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, false>(a, max_blocks, qs, st)
                          : launch_pipe<MI355MOE_RECIPE_FP8BLOCK, EPI_STORE, false>(a, max_blocks, qs, st);
  return epi == EPI_GLU ? launch_pipe<MI355MOE_RECIPE_BF16, EPI_GLU, false>(a, max_blocks, qs, st)
                        : launch_pipe<MI355MOE_RECIPE_BF16, EPI_STORE, false>(a, max_blocks, qs, st);
}

}  // namespace mi355
