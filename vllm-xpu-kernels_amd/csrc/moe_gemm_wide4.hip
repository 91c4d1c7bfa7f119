// Prefill grouped GEMM for mxfp4 weights (e2m1 values, e8m0 scale per 32 along
// K) and bf16 activations: 320-slot x 256-weight-row tiles, 8 waves, 6-slot
// LDS ring fed by direct global->LDS DMA, weights dequantised to bf16 as
// their MFMA fragments are read.
//
// Why this shape.  The tile, waves and epilogue are those of the bf16 WIDE
// kernel (moe_gemm_wide.hip: 320 slots hold an expert's n +- 4 sigma routed
// rows, 2 waves per SIMD of 160 x 64 each, 32x32x16 bf16 MFMAs).  The weight
// operand of a 32-element K stage is 16 bytes of e2m1 per row instead of 64
// of bf16, so a stage is 20 KB of activations + 4 KB of weights + 256 bytes
// of scales and six fit in LDS: five stages of DMA in flight.
//
// Layout.  The weights and scales are K-blocked (MI355MOE_WLAYOUT_KBLOCK:
// [E, K/32, N, 16 B] and [E, K/32, N]), so a stage's 256 weight rows are one
// 4 KB run and their scales one 256-byte run (two 128-byte runs for a GLU
// tile's gate and up halves).  Activation rows as in the bf16 kernel (16-byte
// chunk c of row r at slot c ^ ((r >> 2) & 3)); weight row r at 16 r, its
// scale at byte r.  Waves 0-3 move 5 activation blocks each, waves 4-7 one
// 64-row weight block each, wave 4 also the scales (one dword DMA: lane l
// moves the scale bytes of rows 4l..4l+3).
//
// Dequantisation.  A lane's MFMA fragment of weight row r for K step ks is
// the 8 values [16 ks + 8 h, +8): 4 bytes of e2m1, converted with
// v_cvt_scalef32_pk_{bf16,f16}_fp4 (the call's 16-bit type) under the row's scale (2^(code - 127); code 0
// gives 0, as the other mxfp4 kernels).
//
// Per-expert fp8 weights (recipes FP8 / FP8E5M2, K-blocked [E, K/32, N, 32
// bytes]) run the same kernel: a stage's weights are 256 rows x 32 bytes
// (8 KB, five stages in the ring, no scales), waves 4-7 move 64 rows each
// with two transfers, a fragment is 8 fp8 bytes converted exactly by
// v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8} at scale 1, and the epilogue
// multiplies the accumulators by the expert's scale.
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int MG = 5;                          // 32-row groups per wave
constexpr int BM = 2 * 32 * MG, BN = 256, ROWB = 64, KE = 32;
static_assert(BM == kWideBM, "block size of the WIDE family");
constexpr int A_BYTES = BM * ROWB;             // 20 KB of bf16 activations
constexpr int W_OFF = A_BYTES;                 // 256 weight rows
constexpr int A_DMA = BM / 16 / 4;             // activation blocks per wave (waves 0-3)
constexpr int DMA_MAX = A_DMA;                 // DMA instructions per wave and stage
// Stage geometry of the weight format: e2m1 (16 bytes a row + 256 e8m0 scale
// bytes, 24.25 KB, six stages), int4 (16 bytes a row + 256 16-bit group
// scales, 24.5 KB, six stages) or fp8 (32 bytes a row, 28 KB, five stages).
template <int WREC>
struct Geom {
  static constexpr bool W8 = is_w8a16_recipe(WREC);
  static constexpr int WROW = W8 ? 32 : 16;    // weight bytes per row and stage
  static constexpr int SROW = W8 ? 0 : (WREC == MI355MOE_RECIPE_INT4 ? 2 : 1);  // scale bytes
  static constexpr int S_OFF = W_OFF + BN * WROW;
  static constexpr int STAGE = S_OFF + BN * SROW;
  static constexpr int NSTAGE = W8 ? 5 : 6;
  static constexpr int RING = NSTAGE * STAGE;
  static_assert(RING <= 150 * 1024, "LDS budget");
  static_assert(BM * (2 * 128 + 16) <= RING, "GLU output tile staged in one pass");
  static_assert(BM / 2 * (2 * 256 + 16) <= RING, "STORE output tile staged in two passes");
  static_assert(A_DMA >= 2, "two weight transfers per wave fit the offset array");
};

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
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// wave-uniform count of DMA instructions allowed to stay outstanding (a
// count above 20 waits for 20: never less strict than asked)
__device__ __forceinline__ void wait_vm_dyn(int n) {
  switch (n) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    case 15: wait_vm<15>(); break;
    case 16: wait_vm<16>(); break;
    case 17: wait_vm<17>(); break;
    case 18: wait_vm<18>(); break;
    case 19: wait_vm<19>(); break;
    default: wait_vm<20>(); break;
  }
}
__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }


template <bool F16>
__device__ __forceinline__ float round16(float v) {
  if constexpr (F16) return f16_to_f32(f32_to_f16(v));
  else return bf16_to_f32(f32_to_bf16(v));
}
// x * sigmoid(k x) with the hardware exp2 and reciprocal (about 1 ulp each,
// far below the 16-bit rounding that follows)
__device__ __forceinline__ float x_sigmoid(float x, float k) {
  const float e = __builtin_amdgcn_exp2f(-k * x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

// Fragments of one 16-element K step: MG activation tiles (rows 160 wm + 32 j
// + l32) and 2 dequantised weight tiles.
struct Frag {
  uint4 x[MG];
  uint4 w[2];
};

// Activation tile j sits 32 x 64 bytes past tile 0 (rows 32 apart share the
// swizzle).  Weight tile i: row woff_r + i * wstep_r; e2m1: its 4 bytes at
// W_OFF + 16 row + wb, its scale at S_OFF + row; fp8: its 8 bytes at W_OFF +
// 32 row + wb.
template <int NJ, bool F16, int WREC>
__device__ __forceinline__ void read_frag(Frag& f, const uint8_t* S, int xoff, int wrow0,
                                          int wstep_r, int wb) {
  constexpr bool W8 = is_w8a16_recipe(WREC);
#pragma unroll
  for (int j = 0; j < NJ; ++j) f.x[j] = *reinterpret_cast<const uint4*>(S + xoff + j * 32 * ROWB);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = wrow0 + i * wstep_r;
    if constexpr (W8) {
      const uint2 w = *reinterpret_cast<const uint2*>(S + W_OFF + 32 * r + wb);
      f.w[i] = fp8x8_to16<WREC == MI355MOE_RECIPE_FP8E5M2, F16>(w);
    } else if constexpr (WREC == MI355MOE_RECIPE_INT4) {  // T(v * scale)
      const uint32_t w = *reinterpret_cast<const uint32_t*>(S + W_OFF + 16 * r + wb);
      const uint16_t sc = *reinterpret_cast<const uint16_t*>(S + Geom<WREC>::S_OFF + 2 * r);
      f.w[i] = int4x8_to16<F16>(w, ld16<F16>(sc));
    } else {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(S + W_OFF + 16 * r + wb);
      const uint32_t code = S[Geom<WREC>::S_OFF + r];
      f.w[i] = fp4x8_to16<F16>(w, __uint_as_float(code << 23));
    }
  }
}

template <int NJ, bool F16>
__device__ __forceinline__ void mfma_step(f32x16 (&acc)[2][MG], const Frag& f) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16_32x32x16<F16>(f.w[i], f.x[j], acc[i][j]);
}

template <int EPI, bool F16, int WREC>
__global__ __launch_bounds__(512) void moe_gemm_wide4_kernel(const GemmArgs a) {
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns per tile
  constexpr bool W8 = is_w8a16_recipe(WREC);
  constexpr bool I4 = WREC == MI355MOE_RECIPE_INT4;
  using G = Geom<WREC>;
  constexpr int STAGE = G::STAGE, NSTAGE = G::NSTAGE, RING_BYTES = G::RING;

  __shared__ __attribute__((aligned(1024))) uint8_t lds[RING_BYTES];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, h = lane >> 5;

  // XCD-aware tile order (as in the other prefill kernels)
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

  int ok = 0;
  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }
  // valid slots form a prefix of the block
  const int v = __syncthreads_count(ok);

  // weight row staged at tile row r; rows past N read row 0 (finite data
  // whose outputs are never stored; N % 4 == 0 keeps each 4-row scale group
  // on one side of N).  GLU: rows [0,128) gate, [128,256) up.
  auto wrow_of = [&](int r) -> int64_t {
    if constexpr (kGlu) {
      const int64_t c = n0 + (r & 127);
      return (r >= 128 ? a.up_off : 0) + (c < N ? c : 0);
    } else {
      const int64_t c = n0 + r;
      return c < N ? c : 0;
    }
  };

  // DMA of this wave: waves 0-3 activation blocks A_DMA wave + q (16 rows x
  // 64 bytes each; blocks of padding only are skipped, so the used ones are a
  // prefix of q); waves 4-7 weight rows 64 (wave - 4) + lane (16 bytes each)
  // and, wave 4, the scale bytes of rows 4 lane..4 lane+3.  Sources are a
  // scalar base plus 32-bit lane offsets (launch_moe_gemm_wide4 checks the
  // sizes).
  const bool a_wave = wave < 4;
  const int64_t ebytes = a.ldb_rows * (W8 ? K : K / 2);  // one expert's weight bytes
  const uint8_t* abase = uniform_ptr(a.A);
  const uint8_t* wexp = uniform_ptr(static_cast<const uint8_t*>(a.B) + static_cast<int64_t>(e) * ebytes);
  // scales: e8m0 [E, K/32, N] bytes, or int4's 16-bit [E, K/group, N]
  const int64_t sgroups = I4 ? K / a.w_group : K / 32;
  const uint8_t* sexp = uniform_ptr(static_cast<const uint8_t*>(a.b_scale) +
                                    static_cast<int64_t>(e) * a.ldb_rows * sgroups * G::SROW);
  const int64_t wkstep = a.ldb_rows * G::WROW;  // K-blocked: bytes between two K stages
  const int64_t skstep = a.ldb_rows * G::SROW;  // bytes between two scale groups
  uint32_t voff[DMA_MAX];
  int nd = 0;
  if (a_wave) {
#pragma unroll
    for (int q = 0; q < A_DMA; ++q) {
      const int b = A_DMA * wave + q;
      const int r = b * 16 + (lane >> 2);
      const int ar = s_arow[r];
      voff[q] = static_cast<uint32_t>(static_cast<int64_t>(ar >= 0 ? ar : 0) * K * 2 +
                                      (((lane & 3) ^ swz(r)) << 4));
      nd += b * 16 < v ? 1 : 0;
    }
  } else if constexpr (W8) {
    // transfer i: rows 64 (wave - 4) + 32 i + lane / 2, 16-byte half lane % 2
#pragma unroll
    for (int i = 0; i < 2; ++i)
      voff[i] = static_cast<uint32_t>(wrow_of(64 * (wave - 4) + 32 * i + (lane >> 1)) * 32 +
                                      16 * (lane & 1));
#pragma unroll
    for (int q = 2; q < DMA_MAX; ++q) voff[q] = 0;
    nd = 2;
  } else if constexpr (I4) {
    // wave 4 also moves the 256 rows' 16-bit scales: lane l rows 2 l, 2 l + 1
    // (and 128 + 2 l, + 1); N and up_off % 4 == 0 keep each pair of rows on
    // one side of N
    voff[0] = static_cast<uint32_t>(wrow_of(64 * (wave - 4) + lane) * 16);
    voff[1] = static_cast<uint32_t>(wrow_of(2 * lane) * 2);
    voff[2] = static_cast<uint32_t>(wrow_of(128 + 2 * lane) * 2);
#pragma unroll
    for (int q = 3; q < DMA_MAX; ++q) voff[q] = 0;
    nd = wave == 4 ? 3 : 1;
  } else {
    voff[0] = static_cast<uint32_t>(wrow_of(64 * (wave - 4) + lane) * 16);
    voff[1] = static_cast<uint32_t>(wrow_of(4 * lane));
#pragma unroll
    for (int q = 2; q < DMA_MAX; ++q) voff[q] = 0;
    nd = wave == 4 ? 2 : 1;
  }
  const uint32_t ring0 = lds_off(lds);
  const int nk = static_cast<int>(K / KE);
  auto issue = [&](int kt) {  // this wave's DMA of stage kt
    const uint32_t base = ring0 + (kt % NSTAGE) * STAGE;
    if (a_wave) {
      const uint8_t* sb = abase + static_cast<int64_t>(kt) * ROWB;
#pragma unroll
      for (int q = 0; q < A_DMA; ++q)
        if (q < nd)
          dma16(voff[q], sb, __builtin_amdgcn_readfirstlane(base + (A_DMA * wave + q) * 1024));
    } else if constexpr (W8) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        dma16(voff[i], wexp + static_cast<int64_t>(kt) * wkstep,
              __builtin_amdgcn_readfirstlane(base + W_OFF + 2048 * (wave - 4) + 1024 * i));
    } else if constexpr (I4) {
      dma16(voff[0], wexp + static_cast<int64_t>(kt) * wkstep,
            __builtin_amdgcn_readfirstlane(base + W_OFF + 1024 * (wave - 4)));
      if (wave == 4) {  // the group of this 32-value stage
        const uint8_t* sb = sexp + static_cast<int64_t>(kt) * 32 / a.w_group * skstep;
        dma4(voff[1], sb, __builtin_amdgcn_readfirstlane(base + G::S_OFF));
        dma4(voff[2], sb, __builtin_amdgcn_readfirstlane(base + G::S_OFF + 256));
      }
    } else {
      dma16(voff[0], wexp + static_cast<int64_t>(kt) * wkstep,
            __builtin_amdgcn_readfirstlane(base + W_OFF + 1024 * (wave - 4)));
      if (wave == 4)
        dma4(voff[1], sexp + static_cast<int64_t>(kt) * skstep,
             __builtin_amdgcn_readfirstlane(base + G::S_OFF));
    }
  };
  // this wave's DMA instructions still allowed in flight once stage s has
  // landed, when it has issued stages up to `last`
  auto pending_after = [&](int s, int last) -> int {
    const int l = last < nk - 1 ? last : nk - 1;
    return l > s ? nd * (l - s) : 0;
  };
  for (int s = 0; s < NSTAGE - 1 && s < nk; ++s) issue(s);

  // per-wave MFMA rows: 160 wm + [0, 32 nj)
  const int vw = v - 32 * MG * wm;
  const int nj = vw <= 0 ? 0 : (vw >= 32 * MG ? MG : (vw + 31) / 32);

  // fragment offsets: activation chunk c = 2 ks + h (every row this lane
  // reads has the swizzle of l32); weight row of tile 0 and tile distance
  int xoff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c = (2 * ks + h) ^ swz(l32);
    xoff[ks] = (32 * MG * wm + l32) * ROWB + (c << 4);
  }
  const int wrow0 = (kGlu ? 32 * wn : 64 * wn) + l32;
  constexpr int WSTEP_R = kGlu ? 128 : 32;
  // byte offset of the lane's fragment in its weight row: K steps 0 and 1
  const int wb0 = W8 ? 8 * h : 4 * h, wb1 = W8 ? 16 + 8 * h : 8 + 4 * h;

  f32x16 acc[2][MG];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < MG; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // K loop.  Stage kt's fragments are in registers when iteration kt starts;
  // its first K step runs, then the barrier publishes stage kt+1 and its
  // fragment reads go out while the second K step's MFMAs run.  Stage kt-1
  // was consumed by every wave before that barrier, so the DMA of stage
  // kt + NSTAGE - 1 into its slot is issued after it.  The next stage's
  // fragment reads are unconditional (after the last stage they read a stale
  // slot, unused).
  auto kloop = [&](auto nj_c) {
    constexpr int NJ = decltype(nj_c)::value;
    Frag f0, f1;
    wait_vm_dyn(pending_after(0, NSTAGE - 2));
    __builtin_amdgcn_s_barrier();
    read_frag<NJ, F16, WREC>(f0, lds, xoff[0], wrow0, WSTEP_R, wb0);
    read_frag<NJ, F16, WREC>(f1, lds, xoff[1], wrow0, WSTEP_R, wb1);
    for (int kt = 0; kt < nk; ++kt) {
      mfma_step<NJ, F16>(acc, f0);
      // stage kt+1 landed; later stages this wave issued may pend
      wait_vm_dyn(pending_after(kt + 1, kt + NSTAGE - 2));
      __builtin_amdgcn_s_barrier();
      const uint8_t* S1 = lds + ((kt + 1) % NSTAGE) * STAGE;
      read_frag<NJ, F16, WREC>(f0, S1, xoff[0], wrow0, WSTEP_R, wb0);
      if (kt + NSTAGE - 1 < nk) issue(kt + NSTAGE - 1);
      mfma_step<NJ, F16>(acc, f1);
      read_frag<NJ, F16, WREC>(f1, S1, xoff[1], wrow0, WSTEP_R, wb1);
    }
  };
  switch (nj) {
    case 5: kloop(std::integral_constant<int, 5>{}); break;
    case 4: kloop(std::integral_constant<int, 4>{}); break;
    case 3: kloop(std::integral_constant<int, 3>{}); break;
    case 2: kloop(std::integral_constant<int, 2>{}); break;
    case 1: kloop(std::integral_constant<int, 1>{}); break;
    default: kloop(std::integral_constant<int, 0>{}); break;
  }
  static_assert(MG == 5, "kloop variants cover 0..MG row groups");

  // ---- epilogue: bias, rounding, activation; output tile staged in LDS and
  //      written with 16-byte row-contiguous stores (STORE tiles in two
  //      passes of 160 rows, one per wave half)
  constexpr int PITCH = 2 * NOUT + 16;
  constexpr int PASSES = BM * PITCH <= RING_BYTES ? 1 : 2;
  constexpr int PROWS = BM / PASSES;
  const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
  const float es = W8 && a.expert_scale ? a.expert_scale[e] : 1.f;  // per-expert fp8
  auto tcol = [&](int i, int r) -> int {  // tile output column of (i, r)
    return (kGlu ? 32 * wn : 64 * wn + 32 * i) + 8 * (r >> 2) + 4 * h + (r & 3);
  };
  constexpr int NI = kGlu ? 1 : 2;
  uint16_t* d = static_cast<uint16_t*>(a.D);
  const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(a.D) & 15) == 0;
  constexpr int CPR = 2 * NOUT / 16;  // 16-byte chunks per row
  __syncthreads();  // every wave is done with the ring
  // the tile's 16-bit outputs into the LDS staging rows of pass `pass`,
  // specialised on the activation, gemm1_clamp_limit and the bias (uniform
  // per launch) so that no value branches on them; gate and up rounded two
  // values per conversion
  auto stage_out = [&](int pass, auto silu_c, auto clamp_c, auto bias_c) {
    constexpr bool SILU = decltype(silu_c)::value;
    constexpr bool CLAMP = decltype(clamp_c)::value;
    constexpr bool HASB = decltype(bias_c)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float bg[16], bu[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + tcol(i, r);
        const bool has = HASB && n < N;
        bg[r] = has ? ld16<F16>(a.bias[bias_base + n]) : 0.f;
        bu[r] = has && kGlu ? ld16<F16>(a.bias[bias_base + a.up_off + n]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < MG; ++j) {
        const int srow = 32 * MG * wm + 32 * j + l32 - pass * PROWS;
        float ov[16];  // rounded to the 16-bit type once, in the packing below
#pragma unroll
        for (int r = 0; r < 16; ++r) ov[r] = HASB ? (W8 ? acc[i][j][r] * es : acc[i][j][r]) + bg[r] : (W8 ? acc[i][j][r] * es : acc[i][j][r]);
        if constexpr (kGlu) {
          float u[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) u[r] = HASB ? (W8 ? acc[1][j][r] * es : acc[1][j][r]) + bu[r] : (W8 ? acc[1][j][r] * es : acc[1][j][r]);
          round16xn<F16>(ov);
          round16xn<F16>(u);
          if constexpr (CLAMP)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              glu_clamp_with(a.clamp_limit, SILU ? MI355MOE_ACT_SILU : MI355MOE_ACT_SWIGLUOAI, N,
                             n0 + tcol(i, r), ov[r], u[r]);
          if constexpr (SILU) {
            float sg[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) sg[r] = x_sigmoid(ov[r], 1.f);
            round16xn<F16>(sg);
#pragma unroll
            for (int r = 0; r < 16; ++r) ov[r] = sg[r] * u[r];
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float gc = ov[r] > a.limit ? a.limit : ov[r];
              const float uc = u[r] > a.limit ? a.limit : (u[r] < -a.limit ? -a.limit : u[r]);
              ov[r] = (uc + 1.f) * x_sigmoid(gc, a.alpha);
            }
          }
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const uint32_t lo = pack16x2<F16>(ov[4 * g4], ov[4 * g4 + 1]);
          const uint32_t hi = pack16x2<F16>(ov[4 * g4 + 2], ov[4 * g4 + 3]);
          *reinterpret_cast<uint2*>(lds + srow * PITCH + 2 * tcol(i, 4 * g4)) = make_uint2(lo, hi);
        }
      }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto stage_pass = [&](int pass) {
    auto with_bias = [&](auto silu_c, auto clamp_c) {
      if (a.bias) stage_out(pass, silu_c, clamp_c, T_{});
      else stage_out(pass, silu_c, clamp_c, F_{});
    };
    if constexpr (!kGlu) {
      with_bias(T_{}, F_{});
    } else {
      const bool clamp = a.clamp_limit > 0.f;
      if (a.act == MI355MOE_ACT_SILU) {
        if (clamp) with_bias(T_{}, T_{});
        else with_bias(T_{}, F_{});
      } else {
        if (clamp) with_bias(F_{}, T_{});
        else with_bias(F_{}, F_{});
      }
    }
  };
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    if (PASSES == 1 || wm == pass) stage_pass(pass);
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

template <int EPI, bool F16, int WREC>
int launch_wide4(const GemmArgs& a, int64_t max_blocks, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_wide4_kernel<EPI, F16, WREC><<<grid, dim3(512), 0, st>>>(a);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace

bool wide4_shape_ok(int64_t a_rows, int64_t ldb_rows, int64_t N, int64_t K) {
  const int64_t lim = int64_t(1) << 32;
  return K % 32 == 0 && K > 0 && ldb_rows % 4 == 0 && N % 4 == 0 && a_rows * K * 2 < lim &&
         ldb_rows * K < lim;
}

template <int WREC>
int launch_wide4_rec(int epi, const GemmArgs& a, int64_t max_blocks, hipStream_t st) {
  if (epi == EPI_GLU)
    return a.out_f16 ? launch_wide4<EPI_GLU, true, WREC>(a, max_blocks, st)
                     : launch_wide4<EPI_GLU, false, WREC>(a, max_blocks, st);
  return a.out_f16 ? launch_wide4<EPI_STORE, true, WREC>(a, max_blocks, st)
                   : launch_wide4<EPI_STORE, false, WREC>(a, max_blocks, st);
}

// kWideBM-slot blocks; K-blocked mxfp4 weights and scales, or K-blocked
// per-expert fp8 weights ([E, K/32, N, 32 bytes]); K % 32 == 0.
int launch_moe_gemm_wide4(int recipe, int epi, const GemmArgs& a, int64_t max_blocks,
                          hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  MI_ARG((recipe == MI355MOE_RECIPE_MXFP4 || recipe == MI355MOE_RECIPE_INT4 ||
          is_w8a16_recipe(recipe)) &&
             a.w_kblock,
         "4-bit / fp8-weight prefill GEMM: needs K-blocked mxfp4, int4 or per-expert fp8 "
         "weights");
  const int64_t a_rows = a.a_by_pos ? max_blocks * BM : a.num_valid;
  MI_ARG(wide4_shape_ok(a_rows, a.ldb_rows, a.N, a.K) && (a.up_off & 3) == 0,
         "4-bit / fp8-weight prefill GEMM: needs K % 32 == 0, N and weight rows % 4 == 0 "
         "and activation / per-expert weight bytes below 4 GiB");
  if (recipe == MI355MOE_RECIPE_FP8) return launch_wide4_rec<MI355MOE_RECIPE_FP8>(epi, a, max_blocks, st);
  if (recipe == MI355MOE_RECIPE_FP8E5M2)
    return launch_wide4_rec<MI355MOE_RECIPE_FP8E5M2>(epi, a, max_blocks, st);
  if (recipe == MI355MOE_RECIPE_INT4) {
    MI_ARG(a.w_group >= 32 && a.K % a.w_group == 0, "int4 prefill GEMM: group size >= 32");
    return launch_wide4_rec<MI355MOE_RECIPE_INT4>(epi, a, max_blocks, st);
  }
  return launch_wide4_rec<MI355MOE_RECIPE_MXFP4>(epi, a, max_blocks, st);
}

}  // namespace mi355
