// Prefill grouped GEMM for bf16 weights: 320-slot x 256-weight-row tiles,
// 8 waves, 4-slot LDS ring fed by direct global->LDS DMA.
//
// Why this shape.  A tile streams its expert's 256 weight rows over the whole
// K once, so the weight bytes a layer moves into LDS are (tiles per expert) x
// (weight bytes).  Routing spreads about n +- sqrt(n) slots over an expert, and
// a 256-slot block at n = 256 leaves half the experts with a second, nearly
// empty block that streams the weights a second time; 320 slots hold n + 4
// sigma.  Compute and activation DMA scale with the valid rows only (empty
// 32-row groups skip their MFMAs, empty 16-row groups their DMA).  Each K
// element moves (320 + 256) x 2 bytes into LDS for 2 x 320 x 256 flops.  Two
// waves per SIMD (waves w and w + 4 share SIMD w % 4) let one wave's MFMAs
// cover the other's LDS latency; each wave keeps its 160 x 64 accumulator
// block (10 32x32 tiles, 160 registers) resident.
//
// Layout.  A K stage holds 32 bf16 (64 bytes) of each of the 320 activation
// rows and 256 weight rows: 36 KB, written by 36 global_load_lds_dwordx4 (16
// rows x 64 B each; lane l writes LDS bytes [16l, 16l + 16) of its 1 KB
// block): waves 0-3 stage 5 activation blocks each, waves 4-7 4 weight blocks
// each.  16-byte chunk c of row r sits at slot c ^ ((r >> 2) & 3): sixteen
// consecutive rows read at one logical chunk then hit sixteen distinct 16-byte
// bank groups.  A and W use the same K permutation, so the MFMA sums are
// unchanged.
//
// Pipeline.  Up to three stages are in flight ahead of the one computed; the
// barrier that publishes stage kt+1 sits between the two K steps of stage kt,
// so stage kt+1's fragment reads overlap stage kt's second MFMA group (all
// waves meet the barrier together, and without this every stage would start
// with the matrix cores idle behind the LDS reads).  The DMA instructions of
// stage kt+3 are issued between MFMAs so the vector-memory queue drains while
// the matrix cores run.
//
// Padding.  The slots of a block are its expert's rows followed by padding;
// with v valid slots, DMA of 16-row groups at or past v is skipped, and a wave
// runs the MFMAs of its 32-row groups that hold valid slots only.
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int MG = 5;                          // 32-row groups per wave
constexpr int BM = 2 * 32 * MG, BN = 256, ROWB = 64, KE = 32;
static_assert(BM == kWideBM, "block size of the WIDE family");
constexpr int A_BYTES = BM * ROWB;             // 20 KB
constexpr int STAGE = (BM + BN) * ROWB;        // 36 KB
constexpr int NSTAGE = 4;
constexpr int A_DMA = BM / 16 / 4;             // activation blocks per wave (waves 0-3)
constexpr int W_DMA = BN / 16 / 4;             // weight blocks per wave (waves 4-7)
constexpr int DMA_PER_WAVE = A_DMA > W_DMA ? A_DMA : W_DMA;
constexpr int RING_BYTES = NSTAGE * STAGE;
constexpr int LDS_BYTES = RING_BYTES;
static_assert(BM * (2 * 128 + 16) <= RING_BYTES, "GLU output tile staged in one pass");
static_assert(BM / 2 * (2 * 256 + 16) <= RING_BYTES, "STORE output tile staged in two passes");

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t*)p));
}
// 16 bytes per lane from sbase + voff (scalar base, 32-bit lane offset) into
// LDS at lds_base + 16 lane.
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(reinterpret_cast<uint64_t>(sbase)), "s"(lds_base) : "memory", "m0");
}
// readfirstlane returns int: each half goes through uint32_t so that the low
// half is zero-extended (a sign-extended low half with bit 31 set would fill
// the high half with ones).
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return reinterpret_cast<const uint8_t*>((hi << 32) | lo);
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// wave-uniform count of DMA instructions allowed to stay outstanding
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
    default: wait_vm<10>(); break;
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
// + l32) and 2 weight tiles.
struct Frag {
  uint4 x[MG];
  uint4 w[2];
};

// The swizzle of rows r + 32 j equals that of r, so fragment j sits a
// constant 32 x 64 bytes past fragment 0 (immediate offsets of one address).
// Weight tile 1 sits `wstep` bytes past weight tile 0.
template <int NJ>
__device__ __forceinline__ void read_frag(Frag& f, const uint8_t* S, int xoff, int woff,
                                          int wstep) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) f.x[j] = *reinterpret_cast<const uint4*>(S + xoff + j * 32 * ROWB);
#pragma unroll
  for (int i = 0; i < 2; ++i) f.w[i] = *reinterpret_cast<const uint4*>(S + woff + i * wstep);
}

// 2 x NJ MFMAs of one K step; with `dma`, the step's DMA instructions q0 and
// q0 + 1 go out between its two MFMA groups and after them.
template <int NJ, bool F16>
__device__ __forceinline__ void mfma_step(f32x16 (&acc)[2][MG], const Frag& f, bool dma,
                                          const uint32_t (&voff)[DMA_PER_WAVE],
                                          const uint8_t* sbase, uint32_t dst_base, int nd,
                                          int q0) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16_32x32x16<F16>(f.w[i], f.x[j], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
    const int q = q0 + i;
    if (dma && q < nd) dma16(voff[q], sbase, __builtin_amdgcn_readfirstlane(dst_base + q * 1024));
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int EPI, bool F16>
__global__ __launch_bounds__(512) void moe_gemm_wide_kernel(const GemmArgs a) {
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns per tile

  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, h = lane >> 5;

  // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs;
  // XCD x takes the contiguous range [x*per, (x+1)*per) of the valid tiles
  // (ordered by tile_coords), so the tiles sharing an expert's weight rows or
  // a block's activation rows meet in one L2.
  // The grid is a multiple of 8 and at least the tile upper bound.
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
  const int64_t wrow_bytes = K * 2;

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
  // whose outputs are never stored).  GLU: rows [0,128) gate, [128,256) up.
  auto wrow_of = [&](int r) -> int64_t {
    if constexpr (kGlu) {
      const int64_t c = n0 + (r & 127);
      return (r >= 128 ? a.up_off : 0) + (c < N ? c : 0);
    } else {
      const int64_t c = n0 + r;
      return c < N ? c : 0;
    }
  };

  // DMA instructions of this wave: waves 0-3 stage activation blocks
  // A_DMA wave + q, waves 4-7 weight blocks W_DMA (wave - 4) + q (a block is
  // 16 rows of a stage).  Activation blocks of padding only are skipped; the
  // used instructions are a prefix of q.  The bytes between two K stages of a
  // wave's sources are uniform per wave.
  // Sources are a scalar base (the activation matrix or the expert's weights)
  // plus 32-bit lane offsets (launch_moe_gemm_wide checks that both fit).
  const bool a_wave = wave < 4;
  const WStride wst = w_stride16(a);
  const int64_t kstep = a_wave ? ROWB : wst.kblk;
  const uint8_t* sbase0 = uniform_ptr(
      a_wave ? static_cast<const uint8_t*>(a.A)
             : static_cast<const uint8_t*>(a.B) + static_cast<int64_t>(e) * a.ldb_rows * wrow_bytes);
  uint32_t voff[DMA_PER_WAVE];
  int nd = 0;
#pragma unroll
  for (int q = 0; q < DMA_PER_WAVE; ++q) {
    int64_t o;
    bool use;
    if (a_wave) {
      const int b = A_DMA * wave + (q < A_DMA ? q : 0);
      const int r = b * 16 + (lane >> 2);
      const int ar = s_arow[r];
      o = static_cast<int64_t>(ar >= 0 ? ar : 0) * wrow_bytes + (((lane & 3) ^ swz(r)) << 4);
      use = q < A_DMA && b * 16 < v;
    } else {
      const int b = W_DMA * (wave - 4) + (q < W_DMA ? q : 0);
      const int r = b * 16 + (lane >> 2);
      o = wrow_of(r) * wst.row + (((lane & 3) ^ swz(r)) << 4);
      use = q < W_DMA;
    }
    voff[q] = static_cast<uint32_t>(o);
    nd += use ? 1 : 0;
  }
  // LDS block of src[0]
  const uint32_t dst0 = a_wave ? A_DMA * wave * 1024 : A_BYTES + W_DMA * (wave - 4) * 1024;

  // per-wave MFMA rows: 160 wm + [0, 32 nj)
  const int vw = v - 32 * MG * wm;
  const int nj = vw <= 0 ? 0 : (vw >= 32 * MG ? MG : (vw + 31) / 32);

  // fragment offsets within a stage: chunk c = 2 ks + h; every row this lane
  // reads (l32 plus a multiple of 32) has the swizzle of l32
  int xoff[2], woff[2];
  constexpr int WSTEP = (kGlu ? 128 : 32) * ROWB;  // weight tile 1 - tile 0
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c = (2 * ks + h) ^ swz(l32);
    xoff[ks] = (32 * MG * wm + l32) * ROWB + (c << 4);
    woff[ks] = A_BYTES + ((kGlu ? 32 * wn : 64 * wn) + l32) * ROWB + (c << 4);
  }

  f32x16 acc[2][MG];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < MG; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const uint32_t ring0 = lds_off(lds);
  const int nk = static_cast<int>(K / KE);
  auto issue_all = [&](int kt) {
    const uint32_t base = ring0 + (kt % NSTAGE) * STAGE + dst0;
    const uint8_t* sb = sbase0 + static_cast<int64_t>(kt) * kstep;
#pragma unroll
    for (int q = 0; q < DMA_PER_WAVE; ++q)
      if (q < nd) dma16(voff[q], sb, __builtin_amdgcn_readfirstlane(base + q * 1024));
  };
  for (int s = 0; s < 3 && s < nk; ++s) issue_all(s);

  // K loop.  Stage kt's fragments are in registers when iteration kt starts;
  // its first K step runs, then the barrier publishes stage kt+1 and its
  // fragment reads go out while the second K step's MFMAs run.  Stage kt-1
  // was consumed by every wave before that barrier, so the DMA of stage kt+3
  // into its slot is issued after it.
  auto kloop = [&](auto nj_c) {
    constexpr int NJ = decltype(nj_c)::value;
    Frag f0, f1;
    {
      wait_vm_dyn(nd * ((nk - 1) < 2 ? (nk - 1) : 2));
      __builtin_amdgcn_s_barrier();
      read_frag<NJ>(f0, lds, xoff[0], woff[0], WSTEP);
      read_frag<NJ>(f1, lds, xoff[1], woff[1], WSTEP);
    }
    // The next stage's fragment reads are unconditional (after the last
    // stage they read a stale slot, unused): reads under a condition make
    // the compiler copy every loop-carried fragment register where the
    // branches join.
    for (int kt = 0; kt < nk; ++kt) {
      mfma_step<NJ, F16>(acc, f0, false, voff, sbase0, 0, 0, 0);
      // stage kt+1 landed; stage kt+2 (if issued) may pend
      wait_vm_dyn(kt + 2 < nk ? nd : 0);
      __builtin_amdgcn_s_barrier();
      read_frag<NJ>(f0, lds + ((kt + 1) % NSTAGE) * STAGE, xoff[0], woff[0], WSTEP);
      const bool dma = kt + 3 < nk;
      const uint8_t* sb = sbase0 + static_cast<int64_t>(kt + 3) * kstep;
      const uint32_t dbase = ring0 + ((kt + 3) % NSTAGE) * STAGE + dst0;
      mfma_step<NJ, F16>(acc, f1, dma, voff, sb, dbase, nd, 0);
      if (dma && nd > 2) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 2; q < DMA_PER_WAVE; ++q)
          if (q < nd) dma16(voff[q], sb, __builtin_amdgcn_readfirstlane(dbase + q * 1024));
        __builtin_amdgcn_sched_barrier(0);
      }
      read_frag<NJ>(f1, lds + ((kt + 1) % NSTAGE) * STAGE, xoff[1], woff[1], WSTEP);
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
  const float es = a.expert_scale ? a.expert_scale[e] : 1.f;  // recipe BF16 only
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
        for (int r = 0; r < 16; ++r) ov[r] = HASB ? acc[i][j][r] * es + bg[r] : acc[i][j][r] * es;
        if constexpr (kGlu) {
          float u[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) u[r] = HASB ? acc[1][j][r] * es + bu[r] : acc[1][j][r] * es;
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

template <int EPI, bool F16>
int launch_wide(const GemmArgs& a, int64_t max_blocks, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_wide_kernel<EPI, F16><<<grid, dim3(512), 0, st>>>(a);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace

bool wide_supported(int recipe, const GemmArgs& a) {
  return recipe == MI355MOE_RECIPE_BF16 && a.K % KE == 0 && a.K > 0;
}

bool wide_offsets_fit(int64_t a_rows, int64_t ldb_rows, int64_t K) {
  const int64_t lim = int64_t(1) << 32;
  return a_rows * K * 2 < lim && ldb_rows * K * 2 < lim;
}

// 320-slot blocks; bf16 weights, K % 32 == 0.
int launch_moe_gemm_wide(int recipe, int epi, const GemmArgs& a,
                         int64_t max_blocks, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  MI_ARG(wide_supported(recipe, a), "wide GEMM: needs bf16 weights and K % 32 == 0");
  // activation rows: tokens (gathered) or padded slots (by position)
  const int64_t a_rows = a.a_by_pos ? max_blocks * BM : a.num_valid;
  MI_ARG(wide_offsets_fit(a_rows, a.ldb_rows, a.K),
         "wide GEMM: activation and per-expert weight bytes must stay below 4 GiB");
  if (epi == EPI_GLU)
    return a.out_f16 ? launch_wide<EPI_GLU, true>(a, max_blocks, st)
                     : launch_wide<EPI_GLU, false>(a, max_blocks, st);
  return a.out_f16 ? launch_wide<EPI_STORE, true>(a, max_blocks, st)
                   : launch_wide<EPI_STORE, false>(a, max_blocks, st);
}

}  // namespace mi355
