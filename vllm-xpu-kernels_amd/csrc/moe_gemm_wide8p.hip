// Prefill grouped GEMM for fp8 e4m3 weights with 128x128 block scales and
// e4m3 activations with 1x128 scales: 320-slot x 256-weight-row tiles, 8
// waves, each wave owning 32 weight rows x all 320 slots.
//
// Data movement: both operands go global->LDS (global_load_lds), so no VGPR
// holds data in flight.
//   * activations: the 320 rows x 128 bytes of the stage plus their 320
//     scales go into a 2-slot ring, 40 rows and 40 scales per wave; one
//     barrier per stage makes a slot visible and frees the other.  They are
//     mostly L2 hits (every N-tile of an expert reads the same rows).  The
//     transfer of stage kt + 1 is issued during stage kt, spread over the
//     slot tiles.
//   * weights (the HBM stream of the kernel): every wave moves its own two
//     16-row fragments of a stage (4 KB) into its own region of a 2-slot
//     weight ring, in lane order, two stages ahead: the transfer of stage
//     kt + 2 goes out during stage kt after the activation parts, and the
//     top of stage kt + 1 waits for all but those four newest transfers.  At
//     the top of a stage each wave reads its fragments (four conflict-free
//     16-byte LDS reads) into the operand registers, which frees the slot
//     for the transfer two stages ahead.  Only the wave that wrote a weight
//     region reads it, so the weights need no barrier.
// Measured against loading the weights one stage ahead into VGPRs (C3,
// T=8192): w2 1626 -> 1558 us, w13 2906 -> 2886 us per launch.
//
// Compute: per stage and wave 2 x 20 v_mfma_scale_f32_16x16x128_f8f6f4 (one
// MFMA covers a whole 128-K scale block, unit e8m0 scales), each result
// scaled and added with one FMA per element: acc += p * (xs * ws), the same
// operations in the same order as the other fp8 kernels.  The 20 activation
// fragments stream from LDS one tile ahead; slot tiles made only of padding
// are skipped in pairs (the K loop is specialised on their number).
//
// LDS layout of an activation slot: rows of 128 bytes whose 16-byte chunk c
// holds source chunk c ^ ((r >> 1) & 7), then the 320 scales in slot order
// (with scales by sorted position each wave's transfer reads 256 contiguous
// bytes; lane l16 reads the scale of slot 16 j + l16 at float 16 j + l16).  Within each group of 16 rows, row t holds slot
// (t >> 1) + 8 (t & 1): lane l16 reads row 2 (l16 & 7) + (l16 >> 3), so
// lanes 0-7 read even rows and lanes 8-15 odd rows, and with the chunk
// swizzle each 8-lane group covers one half of the banks.  A 16-byte read of
// rows 0..15 at one logical chunk in plain order (every lane group spread
// over both halves) moves 74 TB/s over the chip, this order 120 TB/s, the
// same as lane-linear reads.
#include <type_traits>

#include "mfma16.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
// global-address-space view of a byte pointer: loads through it are
// global_load (scalar base + 32-bit lane offset), not FLAT loads, which
// would also count in lgkmcnt and so be waited for with every LDS read
typedef __attribute__((address_space(1))) const uint8_t gbyte_t;
typedef __attribute__((address_space(1))) const i32x4_t gi32x4_t;

constexpr int BM = 320, BN = 256, KE = 128;
static_assert(BM == kWideBM, "block size of the WIDE family");
constexpr int WAVES = 8;
constexpr int TJ = BM / 16;                 // slot tiles per wave
constexpr int AROWS = BM / WAVES;           // activation rows moved per wave
constexpr int A_BYTES = BM * KE;            // 40 KB of activations per stage
constexpr int A_SLOT = A_BYTES + 2 * BM * 4;  // + scales (e2m1: two words of codes)
constexpr int DUMMY = 2 * A_SLOT;           // scale DMA target of waves 5-7
constexpr int W_OFF = DUMMY + 256;          // weight ring: 2 slots x 8 waves x 4 KB
constexpr int WSLOT = WAVES * 4096;
constexpr int RING = W_OFF + 2 * WSLOT;
// MX: e8m0 codes of the tile's weight rows, 2 slots x 8 32-K blocks; block b
// at byte CPITCH b of a slot (the 16 padding bytes put the four blocks a
// wave reads at once in different LDS banks)
constexpr int C_OFF = RING;
constexpr int CPITCH = 256 + 16;
constexpr int CSLOT = 8 * CPITCH;
constexpr int RING_MX = C_OFF + 2 * CSLOT;
constexpr int MAX_KBLK = 64;                // K <= 8192
static_assert(RING <= 150 * 1024, "LDS budget");
static_assert(BM * (128 + 16) + WAVES * BM * 4 + 4 * BM * 4 <= RING, "e4m3 output tile, amax, scales");

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
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return reinterpret_cast<const uint8_t*>((hi << 32) | lo);
}
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
// LDS row (within its group of 16) that lane l16 reads, and the slot that
// LDS row t holds: inverse permutations of 0..15
__device__ __forceinline__ int lds_row_of_lane(int l16) { return 2 * (l16 & 7) + (l16 >> 3); }
__device__ __forceinline__ int slot_of_lds_row(int t) { return (t >> 1) + 8 * (t & 1); }

__device__ __forceinline__ f32x4_t mfma8(const i32x8_t& a, const i32x8_t& b) {
  const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ i32x8_t ld32(const uint8_t* S, int o0, int o1) {
  const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(S + o0);
  const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(S + o1);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ float x_sigmoid(float x, float k) {
  const float e = __builtin_amdgcn_exp2f(-k * x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

// MXK: 0 fp8 block-scaled, 1 mxfp8, 2 mxfp4 x mxfp4 (e2m1 weights and
// activations, a stage of 256 K values = 128 bytes per row, two MFMA K-steps).
template <int EPI, bool QOUT, bool F16, int MXK>
__global__ __launch_bounds__(512) void moe_gemm_wide8p_kernel(const GemmArgs a,
                                                              void* __restrict__ qs) {
  constexpr bool MX = MXK != 0;   // e8m0 codes of both operands in the MFMA
  constexpr bool MX4 = MXK == 2;
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int NOUT = kGlu ? 128 : 256;  // output columns per tile

  __shared__ __attribute__((aligned(1024))) uint8_t lds[MX ? RING_MX : RING];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ float s_wsc[4][MAX_KBLK];    // block scales of the tile's four 64-row quarters

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;

  // XCD-aware order: XCD x takes the contiguous range [x*per, (x+1)*per) of
  // the tiles ordered by tile_coords (all N-tiles of an expert's block run
  // side by side in one L2).
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
  const int nkb = static_cast<int>(MX4 ? (K + 255) / 256 : K / KE);  // K stages
  const int nblk = static_cast<int>(K / 32);                           // 32-K blocks

  int ok = 0;
  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }
  // weight row of tile row r (rows past N read row 0: finite data whose
  // outputs are never stored); GLU: [0,128) gate, [128,256) up
  auto wrow_of = [&](int r) -> int64_t {
    if constexpr (kGlu) {
      const int64_t c = n0 + (r & 127);
      return (r >= 128 ? a.up_off : 0) + (c < N ? c : 0);
    } else {
      const int64_t c = n0 + r;
      return c < N ? c : 0;
    }
  };
  if constexpr (!MX) {
    const float* bsc = static_cast<const float*>(a.b_scale);
    const int wsh = 7 - a.ws_rows64;  // weight rows per scale row: 128 or 64
    for (int i = tid; i < 4 * nkb; i += 512) {
      const int t = i / nkb, kb = i % nkb;
      const int64_t wr = wrow_of(64 * t) >> wsh;
      s_wsc[t][kb] = bsc[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + wr) * nkb + kb];
    }
  }
  const int v = __syncthreads_count(ok);  // valid slots form a prefix of the block

  // ---- DMA addressing (per-lane 32-bit offsets, held across the K loop)
  const uint32_t ring0 = lds_off(lds);
  const WStride wst = MX4 ? w_stride4(a) : w_stride8(a);
  const uint8_t* abase = uniform_ptr(a.A);
  const uint8_t* sbase = MX ? uniform_ptr(a.a_mxs) : uniform_ptr(a.a_scale);
  const uint8_t* wbase = uniform_ptr(static_cast<const uint8_t*>(a.B) +
                                     static_cast<int64_t>(e) * a.ldb_rows * (MX4 ? K / 2 : K));
  const uint32_t Ku = static_cast<uint32_t>(MX4 ? K / 2 : K);  // activation row bytes
  const uint32_t Kp = MX4 && a.lda ? static_cast<uint32_t>(a.lda) : Ku;  // row pitch
  // activation rows 40 wave + 8 q + lane / 8, 16-byte chunk lane % 8 of the
  // LDS row, read from source chunk (lane % 8) ^ swz(row)
  uint32_t aoff[AROWS / 8];
#pragma unroll
  for (int q = 0; q < AROWS / 8; ++q) {
    const int r = AROWS * wave + 8 * q + (lane >> 3);
    const int ar = s_arow[(r & ~15) | slot_of_lds_row(r & 15)];
    aoff[q] = static_cast<uint32_t>(ar >= 0 ? ar : 0) * Kp +
              (MX4 ? 0u : static_cast<uint32_t>((lane & 7) ^ swz(r)) << 4);
  }
  // e2m1: the lane's source chunk of part q, added per stage (chunks past
  // the row end in the last stage of a K % 256 != 0 re-read chunk 0)
  auto achunk = [&](int q) -> uint32_t {
    const int r = AROWS * wave + 8 * q + (lane >> 3);
    return static_cast<uint32_t>((lane & 7) ^ swz(r)) << 4;
  };
  // scales: waves 0-4 move them, LDS position p = 64 wave + lane holding the
  // scale of slot p (mxfp8: the four e8m0 codes of the stage's 32-K blocks);
  // waves 5-7 issue the same DMA as wave 0 (so that no branch splits the K
  // loop) into a dummy area
  const bool s_wave = wave < BM / 64;
  uint32_t soff = 0;
  {
    const int p = s_wave ? 64 * wave + lane : lane;
    const int ar = s_arow[p];
    if (a.a_scale_tld)  // by sorted position: padding slots read their own (unused) entry
      soff = static_cast<uint32_t>(blk * BM + p) * 4u;
    else
      soff = static_cast<uint32_t>(ar >= 0 ? ar : 0) *
             (MX ? static_cast<uint32_t>(a.a_mxs_ld) : static_cast<uint32_t>(nkb) * 4u);
  }
  // byte step of the scale transfer from one K stage to the next
  // (MX by position: code word w of position P at (w * a_scale_tld + P) * 4)
  const uint32_t sstep = a.a_scale_tld ? static_cast<uint32_t>(a.a_scale_tld) * 4u : 4u;
  // the wave's weight fragments f = 0, 1: GLU gate rows 16 wave + l16 and the
  // matching up rows; STORE rows 32 wave + 16 f + l16.  Lane (l16, g) loads
  // the 32 bytes at K byte 32 g of its row of the stage (mxfp8: the 16 bytes
  // at 16 g and at 64 + 16 g, the scaled MFMA's e4m3 operand order).
  // fp8 / mxfp8: a fragment's 16 rows x 128 bytes are staged like the
  // activation rows (LDS row t holds fragment row slot_of_lds_row(t), its
  // 16-byte chunk c source chunk c ^ swz(t)): transfer (f, h) moves LDS rows
  // 8 h .. 8 h + 7 of fragment f, eight whole 128-byte rows of the stage
  // (contiguous in the K-blocked layout), so every cache line it touches is
  // read whole, and the fragments are read with the activation offsets.
  uint32_t woff[2][2];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = 8 * h + (lane >> 3);
      const int fr = slot_of_lds_row(t);
      const int r = kGlu ? (f ? 128 : 0) + 16 * wave + fr : 32 * wave + 16 * f + fr;
      woff[f][h] = static_cast<uint32_t>(wrow_of(r) * wst.row) +
                   (static_cast<uint32_t>((lane & 7) ^ swz(t)) << 4);
    }
  // e2m1 (K-blocked [E, K/32, ldb_rows, 16 bytes]): lane (l16, g) of half h
  // moves the 16 bytes of 32-K block 8 kt + 4 h + g of its row (eight whole
  // lines per transfer already), into the wave's region in lane order
  if constexpr (MX4) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int r = kGlu ? (f ? 128 : 0) + 16 * wave + l16 : 32 * wave + 16 * f + l16;
      woff[f][0] = static_cast<uint32_t>(wrow_of(r) * wst.row);
    }
  }
  // MX weight codes (K-blocked [E, K/32, ldb_rows]): the workgroup stages the
  // codes of its 256 tile rows for the stage's 32-K blocks, the code of
  // (block b, tile row r) at byte CPITCH b + r of the code slot.  Wave w
  // moves block w, lane l the 4 bytes of tile rows 4 l .. 4 l + 3 (two whole
  // 128-byte lines per wave); mxfp8 has four blocks per stage, and waves 4-7
  // repeat wave 0's transfer into the dummy area.
  uint32_t coff = 0;
  const uint8_t* cbase = nullptr;
  const uint32_t ldb = static_cast<uint32_t>(a.ldb_rows);
  const bool c_wave = MX4 || wave < 4;
  if constexpr (MX) {
    coff = static_cast<uint32_t>(wrow_of(4 * lane));
    cbase = uniform_ptr(static_cast<const uint8_t*>(a.b_scale) +
                        static_cast<int64_t>(e) * (K / 32) * a.ldb_rows);
  }
  const uint32_t wkstep = static_cast<uint32_t>(wst.kblk);

  // part q of the activation DMA of stage kt into ring slot `parity` & 1:
  // q < 5 eight of the wave's 40 rows, q = 5 the scales
  constexpr int ACT_PARTS = AROWS / 8 + 1;
  auto issue_act_part = [&](int q, int kt, int parity) {
    const uint32_t slot = ring0 + (parity & 1) * A_SLOT;
    const uint32_t k0 = static_cast<uint32_t>(kt) * KE;  // stage start in row bytes
    if (q < AROWS / 8) {
      uint32_t off = aoff[q] + k0;
      if constexpr (MX4) {
        const uint32_t ch = achunk(q);
        off += k0 + ch < Ku ? ch : 0u;
      }
      dma16(off, abase, slot + (AROWS * wave + 8 * q) * KE);
    } else if constexpr (MX4) {
      // eight e8m0 codes per slot: blocks 8 kt .. 8 kt + 3 and + 4 .. + 7
      // (the second word re-reads the first past the code row)
      const uint32_t c0 = 8u * static_cast<uint32_t>(kt);
      const uint32_t c1 = c0 + 4u < static_cast<uint32_t>(a.a_mxs_ld) ? c0 + 4u : c0;
      const uint32_t o0 = a.a_scale_tld ? (c0 >> 2) * sstep : c0;
      const uint32_t o1 = a.a_scale_tld ? (c1 >> 2) * sstep : c1;
      dma4(soff + o0, sbase, s_wave ? slot + A_BYTES + 256 * wave : ring0 + DUMMY);
      dma4(soff + o1, sbase, s_wave ? slot + A_BYTES + BM * 4 + 256 * wave : ring0 + DUMMY);
    } else {
      dma4(soff + sstep * kt, sbase, s_wave ? slot + A_BYTES + 256 * wave : ring0 + DUMMY);
    }
  };
  // weight fragments of stage kt: the wave's 4 KB region of weight slot
  // `slot`, 1 KB per (fragment f, half h) in lane order
  const uint32_t wring = ring0 + W_OFF + static_cast<uint32_t>(wave) * 4096u;
  auto issue_w = [&](int kt, int slot) {
    const uint32_t kofs = static_cast<uint32_t>(kt) * wkstep;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t off;
        if constexpr (MX4) {  // blocks past K re-read the last block
          const int b = 8 * kt + 4 * h + g;
          off = woff[f][0] + static_cast<uint32_t>(b < nblk ? b : nblk - 1) * wkstep;
        } else {
          off = woff[f][h] + kofs;
        }
        dma16(off, wbase, wring + slot * WSLOT + (2 * f + h) * 1024);
      }
  };
  // the weight codes of stage kt into code slot `slot` (e2m1: blocks past K
  // re-read the last block)
  auto issue_c = [&](int kt, int slot) {
    const int b = (MX4 ? 8 : 4) * kt + (c_wave ? wave : 0);
    const int bc = MX4 && b >= nblk ? nblk - 1 : b;
    dma4(coff + static_cast<uint32_t>(bc) * ldb, cbase,
         c_wave ? ring0 + C_OFF + slot * CSLOT + CPITCH * wave : ring0 + DUMMY);
  };
  // the wave's weight fragments of ring slot `slot` (o0, o1: the activation
  // fragment offsets of the lane)
  auto read_w = [&](int slot, i32x8_t (&w)[2], int o0, int o1) {
    if constexpr (MX4) {
      const uint8_t* W = lds + W_OFF + slot * WSLOT + wave * 4096 + 16 * lane;
#pragma unroll
      for (int f = 0; f < 2; ++f) w[f] = ld32(W, 2 * f * 1024, (2 * f + 1) * 1024);
    } else {
      const uint8_t* W = lds + W_OFF + slot * WSLOT + wave * 4096;
#pragma unroll
      for (int f = 0; f < 2; ++f) w[f] = ld32(W + f * 2048, o0, o1);
    }
  };
  // tile rows of the lane's weight row l16 in fragments 0 and 1
  const int rf0 = kGlu ? 16 * wave + l16 : 32 * wave + l16;
  const int rf1 = kGlu ? 128 + 16 * wave + l16 : 32 * wave + 16 + l16;
  // mxfp8: e8m0 codes of the lane's weight rows for its 32-K block g
  auto read_wc = [&](int slot, uint32_t (&c)[2]) {
    const uint8_t* C = lds + C_OFF + slot * CSLOT + CPITCH * g;
    c[0] = C[rf0];
    c[1] = C[rf1];
  };
  // e2m1: the same for blocks g (step 0) and 4 + g (step 1)
  auto read_wc4 = [&](int slot, uint32_t (&c)[2][2]) {
    const uint8_t* C = lds + C_OFF + slot * CSLOT + CPITCH * g;
    c[0][0] = C[rf0];
    c[0][1] = C[4 * CPITCH + rf0];
    c[1][0] = C[rf1];
    c[1][1] = C[4 * CPITCH + rf1];
  };

  // fragment offsets within an activation slot: chunks 2g and 2g + 1 of the
  // LDS row holding slot l16 (+ 16 j rows for tile j; the swizzle depends on
  // the row % 16 only)
  const int xr = lds_row_of_lane(l16);
  const int xc0 = MX ? g : 2 * g, xc1 = MX ? g + 4 : 2 * g + 1;  // logical chunks
  const int xo0 = xr * KE + ((xc0 ^ swz(xr)) << 4);
  const int xo1 = xr * KE + ((xc1 ^ swz(xr)) << 4);
  // s_wsc quarter of fragment f: GLU tile rows 16 wave (gate) and 128 +
  // 16 wave (up); STORE rows 32 wave .. 32 wave + 31
  const int wsel0 = kGlu ? (wave >> 2) : (wave >> 1), wsel1 = kGlu ? 2 + (wave >> 2) : (wave >> 1);
  // slot tiles holding valid slots, rounded up to pairs
  const int njv = (v + 15) / 16;
  const int nj = njv <= 0 ? 0 : (njv >= TJ ? TJ : ((njv + 1) & ~1));

  f32x4_t acc[2][TJ];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = nkb;
  // Stage kt: the six parts of the activation DMA of stage kt + 1 go out one
  // every second slot tile (a wave that issues them back to back stalls
  // until the DMA path takes them, and computes nothing meanwhile), then the
  // weight DMA of stage kt + 2; MX weight codes of stage kt + 1 go out first,
  // right after the barrier.  Transfers complete in issue order, so the wait
  // at the top of stage kt + 1 for all but the four newest covers the codes
  // and activations of kt + 1 and the weights of kt + 1 (issued during kt - 1).
  // Stages past the end move the last stage's (in-bounds, unused) data
  // instead of branching around the transfers.
  auto kloop = [&](auto nj_c) {
    constexpr int NJ = decltype(nj_c)::value;
    // slot tile after which part q of the activation DMA is issued (parts
    // past the last tile follow the loop)
    auto part_at = [](int q) { return 2 * q; };
    constexpr int W_AT = 11;   // tile after which the weight DMA of stage kt + 2 goes out
    i32x8_t wc[2];
    if constexpr (MX) issue_c(0, 0);
#pragma unroll
    for (int q = 0; q < ACT_PARTS; ++q) issue_act_part(q, 0, 0);
    issue_w(0, 0);
    issue_w(nk > 1 ? 1 : 0, 1);
    for (int kt = 0; kt < nk; ++kt) {
      // everything but the newest transfers (the four of the weights of
      // stage kt + 1, issued during kt - 1)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      __builtin_amdgcn_s_barrier();   // act(kt) visible; act slot (kt+1)&1 free
      asm volatile("" ::: "memory");  // no LDS read moves above the barrier
      const int kn = kt + 1 < nk ? kt + 1 : kt;
      const int kq = kt + 2 < nk ? kt + 2 : nk - 1;
      // the codes of stage kt + 1, into the slot every wave finished reading
      // in stage kt - 1 (all are past the barrier); they land before the
      // weights issued later in this stage, so the wait above covers them
      if constexpr (MX) issue_c(kn, (kt + 1) & 1);
      if constexpr (MX4) {
        // last stage of a K % 256 != 0: zero this lane's weight chunks of
        // blocks past K (the DMA re-read the last block there; with a zero
        // weight operand the product is zero, e2m1 holding no Inf or NaN,
        // whatever the activation data and the finite codes)
        if (8 * kt + 8 > nblk) {
          uint8_t* W = lds + W_OFF + (kt & 1) * WSLOT + wave * 4096 + 16 * lane;
#pragma unroll
          for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              if (8 * kt + 4 * h + g >= nblk)
                *reinterpret_cast<uint4*>(W + (2 * f + h) * 1024) = make_uint4(0, 0, 0, 0);
        }
      }
      read_w(kt & 1, wc, xo0, xo1);
      if constexpr (MX4 && NJ > 0) {
        uint32_t wcode[2][2];
        read_wc4(kt & 1, wcode);
        const uint8_t* S = lds + (kt & 1) * A_SLOT;
        const uint32_t* xsp = reinterpret_cast<const uint32_t*>(S + A_BYTES) + l16;
        i32x8_t x = ld32(S, xo0, xo1);
        // an e2m1 operand is four VGPRs: the low half of a fragment feeds
        // K-step 0, the high half K-step 1.  Step 1 of tile j - 1 goes out
        // with step 0 of tile j, so the two MFMAs into one accumulator are
        // four apart, not two.
        i32x8_t xp = x;
        uint32_t xc1p = 0;
        auto step1 = [&](int jj, const i32x8_t& xv, uint32_t xc) {
#pragma unroll
          for (int f = 0; f < 2; ++f)
            acc[f][jj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                __builtin_shufflevector(wc[f], wc[f], 4, 5, 6, 7, 0, 1, 2, 3),
                __builtin_shufflevector(xv, xv, 4, 5, 6, 7, 0, 1, 2, 3), acc[f][jj], 4, 4, 0,
                wcode[f][1], 0, xc);
        };
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          i32x8_t xn = x;
          if (j + 1 < NJ) xn = ld32(S + (j + 1) * 16 * KE, xo0, xo1);
          const uint32_t xc0 = (xsp[16 * j] >> (8 * g)) & 0xffu;       // block g
          const uint32_t xc1 = (xsp[BM + 16 * j] >> (8 * g)) & 0xffu;  // block 4 + g
          if (j > 0) step1(j - 1, xp, xc1p);
#pragma unroll
          for (int f = 0; f < 2; ++f)
            acc[f][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wc[f], x, acc[f][j], 4, 4, 0, wcode[f][0], 0, xc0);
#pragma unroll
          for (int q = 0; q < ACT_PARTS; ++q)
            if (part_at(q) == j) issue_act_part(q, kn, kt + 1);
          if (j == W_AT) issue_w(kq, kt & 1);
          xp = x;
          xc1p = xc1;
          x = xn;
        }
        step1(NJ - 1, xp, xc1p);
      } else if constexpr (MX && NJ > 0) {
        uint32_t wcode[2];
        read_wc(kt & 1, wcode);
        const uint8_t* S = lds + (kt & 1) * A_SLOT;
        const uint32_t* xsp = reinterpret_cast<const uint32_t*>(S + A_BYTES) + l16;
        i32x8_t x = ld32(S, xo0, xo1);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          i32x8_t xn = x;
          if (j + 1 < NJ) xn = ld32(S + (j + 1) * 16 * KE, xo0, xo1);
          const uint32_t xcode = (xsp[16 * j] >> (8 * g)) & 0xffu;  // slot's 32-K block g
          acc[0][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              wc[0], x, acc[0][j], 0, 0, 0, wcode[0], 0, xcode);
          acc[1][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              wc[1], x, acc[1][j], 0, 0, 0, wcode[1], 0, xcode);
#pragma unroll
          for (int q = 0; q < ACT_PARTS; ++q)
            if (part_at(q) == j) issue_act_part(q, kn, kt + 1);
          if (j == W_AT) issue_w(kq, kt & 1);
          x = xn;
        }
      } else if constexpr (NJ > 0) {
        const float ws0 = s_wsc[wsel0][kt], ws1 = s_wsc[wsel1][kt];
        const uint8_t* S = lds + (kt & 1) * A_SLOT;
        const float* xsp = reinterpret_cast<const float*>(S + A_BYTES) + l16;
        // software pipeline: the scaling FMAs of slot tile j-1 follow the
        // MFMAs of tile j, so no wave waits for its own MFMA results
        i32x8_t x = ld32(S, xo0, xo1);
        f32x4_t q0 = {0.f, 0.f, 0.f, 0.f}, q1 = q0;
        float qs = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          i32x8_t xn = x;
          if (j + 1 < NJ) xn = ld32(S + (j + 1) * 16 * KE, xo0, xo1);
          const float xs = xsp[16 * j];
          const f32x4_t p0 = mfma8(wc[0], x);
          const f32x4_t p1 = mfma8(wc[1], x);
#pragma unroll
          for (int q = 0; q < ACT_PARTS; ++q)
            if (part_at(q) == j) issue_act_part(q, kn, kt + 1);
          if (j == W_AT) issue_w(kq, kt & 1);
          if (j > 0) {
            const float s0 = qs * ws0, s1 = qs * ws1;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc[0][j - 1][r] += q0[r] * s0;
              acc[1][j - 1][r] += q1[r] * s1;
            }
          }
          q0 = p0;
          q1 = p1;
          qs = xs;
          x = xn;
        }
        {
          const float s0 = qs * ws0, s1 = qs * ws1;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[0][NJ - 1][r] += q0[r] * s0;
            acc[1][NJ - 1][r] += q1[r] * s1;
          }
        }
      }
#pragma unroll
      for (int q = 0; q < ACT_PARTS; ++q)
        if (part_at(q) >= NJ) issue_act_part(q, kn, kt + 1);
      if (NJ <= W_AT) issue_w(kq, kt & 1);
    }
  };
  switch (nj) {
    case 20: kloop(std::integral_constant<int, 20>{}); break;
    case 18: kloop(std::integral_constant<int, 18>{}); break;
    case 16: kloop(std::integral_constant<int, 16>{}); break;
    case 14: kloop(std::integral_constant<int, 14>{}); break;
    case 12: kloop(std::integral_constant<int, 12>{}); break;
    case 10: kloop(std::integral_constant<int, 10>{}); break;
    case 8: kloop(std::integral_constant<int, 8>{}); break;
    case 6: kloop(std::integral_constant<int, 6>{}); break;
    case 4: kloop(std::integral_constant<int, 4>{}); break;
    case 2: kloop(std::integral_constant<int, 2>{}); break;
    default: kloop(std::integral_constant<int, 0>{}); break;
  }
  static_assert(TJ == 20, "kloop variants cover the even tile counts up to TJ");

  // The epilogue, specialised on the activation, on gemm1_clamp_limit and on
  // the presence of a bias (uniform per launch), so that no value of the
  // tile branches on them.
  auto epilogue = [&](auto silu_c, auto clamp_c, auto bias_c) {
    constexpr bool SILU = decltype(silu_c)::value;
    constexpr bool CLAMP = decltype(clamp_c)::value;
    constexpr bool HASB = decltype(bias_c)::value;
    // ---- epilogue: lane holds slot 16 j + l16, rows 4 g + r of fragment f
    const int64_t bias_base = static_cast<int64_t>(e) * a.ldb_rows;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // the ring is free
    // output column (within the tile) of (fragment f, reg r)
    auto tcol = [&](int f, int r) -> int {
      return (kGlu ? 16 * wave : 32 * wave + 16 * f) + 4 * g + r;
    };
    constexpr int NF = kGlu ? 1 : 2;
    // the biases of the lane's output columns, the same for all its slots
    float bgs[NF][4], bus[4];
  #pragma unroll
    for (int f = 0; f < NF; ++f)
  #pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = n0 + tcol(f, r);
        const bool has = HASB && n < N;
        bgs[f][r] = has ? ld16<F16>(a.bias[bias_base + n]) : 0.f;
        if (f == 0) bus[r] = has && kGlu ? ld16<F16>(a.bias[bias_base + a.up_off + n]) : 0.f;
      }
    // the lane's four outputs of (fragment f, slot tile j) before their final
    // rounding to the 16-bit type: GLU act(round16(gate), round16(up)),
    // STORE acc + bias (the accumulators are never -0, so no bias adds 0)
    auto outv = [&](int f, int j, float (&o)[4]) {
      float gv[4];
  #pragma unroll
      for (int r = 0; r < 4; ++r) gv[r] = HASB ? acc[f][j][r] + bgs[f][r] : acc[f][j][r];
      if constexpr (kGlu) {
        float u[4];
  #pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = HASB ? acc[1][j][r] + bus[r] : acc[1][j][r];
        round16xn<F16>(gv);
        round16xn<F16>(u);
        if constexpr (CLAMP)
  #pragma unroll
          for (int r = 0; r < 4; ++r)
            glu_clamp_with(a.clamp_limit, SILU ? MI355MOE_ACT_SILU : MI355MOE_ACT_SWIGLUOAI, N,
                           n0 + tcol(f, r), gv[r], u[r]);
        if constexpr (SILU) {
          float sg[4];
  #pragma unroll
          for (int r = 0; r < 4; ++r) sg[r] = x_sigmoid(gv[r], 1.f);
          round16xn<F16>(sg);
  #pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = sg[r] * u[r];
        } else {
  #pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float gc = gv[r] > a.limit ? a.limit : gv[r];
            const float uc = u[r] > a.limit ? a.limit : (u[r] < -a.limit ? -a.limit : u[r]);
            o[r] = (uc + 1.f) * x_sigmoid(gc, a.alpha);
          }
        }
      } else {
  #pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = gv[r];
      }
    };

    if constexpr (QOUT && !MX) {
      // e4m3 activation with one fp32 scale per (slot, 128 columns), the
      // tile's 128 columns (N % 128 == 0): the GLU outputs staged in LDS as
      // 16-bit values (their rounding), one barrier, then 16 lanes per slot
      // row take its amax (one DPP reduction), quantise its 8-column chunks
      // and store the row's 128 bytes
      constexpr int P16 = 2 * NOUT + 16;  // staging row pitch (bytes)
  #pragma unroll
      for (int j = 0; j < TJ; ++j) {
        float o[4];
        outv(0, j, o);
        *reinterpret_cast<uint2*>(lds + (16 * j + l16) * P16 + 2 * tcol(0, 0)) =
            make_uint2(pack16x2<F16>(o[0], o[1]), pack16x2<F16>(o[2], o[3]));
      }
      __syncthreads();
      float* ds = static_cast<float*>(qs);
      uint8_t* dq = static_cast<uint8_t*>(a.D);
      const int64_t ngroups = N / 128;
      const int c = tid & 15;  // the lane's 8-column chunk of the row
      for (int row = tid >> 4; row < BM; row += 512 / 16) {  // every lane, every pass
        const uint4 u = *reinterpret_cast<const uint4*>(lds + row * P16 + 16 * c);
        float x[8];
        unpack16x2<F16>(u.x, x[0], x[1]);
        unpack16x2<F16>(u.y, x[2], x[3]);
        unpack16x2<F16>(u.z, x[4], x[5]);
        unpack16x2<F16>(u.w, x[6], x[7]);
        float m = 1e-10f;
  #pragma unroll
        for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(x[k]));
        m = row16_max(m);
        const float sc = fmaxf(m / 448.f, 1.0f / (448.f * 512.f));
        const float inv = 1.0f / sc;
        const int drow = s_drow[row];
        if (drow >= 0) {
          const uint32_t lo = e4m3x4_sat(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv);
          const uint32_t hi = e4m3x4_sat(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv);
          *reinterpret_cast<uint2*>(dq + static_cast<int64_t>(drow) * N + n0 + 8 * c) =
              make_uint2(lo, hi);
          if (c == 0) {
            if (a.q_scale_tld) ds[static_cast<int64_t>(ntile) * a.q_scale_tld + drow] = sc;
            else ds[static_cast<int64_t>(drow) * ngroups + ntile] = sc;
          }
        }
      }
    } else if constexpr (QOUT) {
      // MX activation for the w2 GEMM, one e8m0 code per 32 columns: mxfp8 as
      // per_token_group_fp8_quant with ue8m0 scales, e2m1 as
      // per_token_group_quant_mxfp4 (eps 1e-10).  Staged like the e4m3 path;
      // 16 lanes per slot row, so a 32-column group is a DPP quad.  N % 32 ==
      // 0: groups past N (the last tile of an N % 128 != 0) get code 127
      // (scale 1.0) where the padded code row holds them -- the w2 GEMM reads
      // them, four codes at a time, against zero data -- and no data.
      constexpr int P16 = 2 * NOUT + 16;  // staging row pitch (bytes)
  #pragma unroll
      for (int j = 0; j < TJ; ++j) {
        float o[4];
        outv(0, j, o);
        *reinterpret_cast<uint2*>(lds + (16 * j + l16) * P16 + 2 * tcol(0, 0)) =
            make_uint2(pack16x2<F16>(o[0], o[1]), pack16x2<F16>(o[2], o[3]));
      }
      __syncthreads();
      uint8_t* dq = static_cast<uint8_t*>(a.D);
      uint8_t* qc = static_cast<uint8_t*>(qs);
      const int64_t orow = MX4 ? (a.ldd ? a.ldd : N / 2) : N;  // output row pitch (bytes)
      const int c = tid & 15;  // the lane's 8-column chunk of the row
      const int p = c >> 2;    // its 32-column group
      for (int row = tid >> 4; row < BM; row += 512 / 16) {  // every lane, every pass
        const uint4 u = *reinterpret_cast<const uint4*>(lds + row * P16 + 16 * c);
        float x[8];
        unpack16x2<F16>(u.x, x[0], x[1]);
        unpack16x2<F16>(u.y, x[2], x[3]);
        unpack16x2<F16>(u.z, x[4], x[5]);
        unpack16x2<F16>(u.w, x[6], x[7]);
        float m = 1e-10f;
  #pragma unroll
        for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(x[k]));
        m = fmaxf(m, dpp_f32<0xB1>(m));  // quad_perm [1,0,3,2]
        m = fmaxf(m, dpp_f32<0x4E>(m));  // quad_perm [2,3,0,1]
        int ex;
        if constexpr (MX4) ex = ceil_log2(fmaxf(fabsf(m / 6.0f), 1e-10f));
        else ex = ceil_log2(fmaxf(fabsf(fmaxf(m / 448.f, 1.0f / (448.f * 512.f))), 1e-10f));
        const float inv = 1.0f / pow2i(ex);
        const int drow = s_drow[row];
        if (drow < 0) continue;
        if ((c & 3) == 0 && n0 / 32 + p < a.q_mxs_ld) {
          const uint8_t code = static_cast<uint8_t>(n0 + 32 * p < N ? ex + 127 : 127);
          // by position: the tile's four codes are byte p of word n0 / 128
          if (a.q_scale_tld) qc[((n0 >> 7) * a.q_scale_tld + drow) * 4 + p] = code;
          else qc[static_cast<int64_t>(drow) * a.q_mxs_ld + n0 / 32 + p] = code;
        }
        if (n0 + 8 * c >= N) continue;
        if constexpr (MX4) {
          // e2m1 pairs, the even column in the low nibble (x holds 16-bit
          // values, inv is a power of two)
          const float sn = fp4_prescale(inv);
          const uint32_t w = fp4x4_code16(x[0], x[1], x[2], x[3], sn) |
                             (fp4x4_code16(x[4], x[5], x[6], x[7], sn) << 16);
          *reinterpret_cast<uint32_t*>(dq + static_cast<int64_t>(drow) * orow + (n0 + 8 * c) / 2) =
              w;
        } else {
          const uint32_t lo = e4m3x4_sat(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv);
          const uint32_t hi = e4m3x4_sat(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv);
          *reinterpret_cast<uint2*>(dq + static_cast<int64_t>(drow) * orow + n0 + 8 * c) =
              make_uint2(lo, hi);
        }
      }
    } else {
      // 16-bit output staged in LDS (STORE tiles in two passes of 160 slots)
      // and written with 16-byte row-contiguous stores
      constexpr int PITCH = 2 * NOUT + 16;
      // passes of a whole number of slot tiles each, as few as the ring holds
      constexpr int PASSES = BM * PITCH <= RING ? 1 : BM / 2 * PITCH <= RING ? 2
                           : BM / 4 * PITCH <= RING ? 4 : 5;
      static_assert(BM / PASSES * PITCH <= RING && TJ % PASSES == 0, "staging passes");
      constexpr int PROWS = BM / PASSES;
      constexpr int PJ = TJ / PASSES;
      uint16_t* d = static_cast<uint16_t*>(a.D);
      const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(a.D) & 15) == 0;
      constexpr int CPR = 2 * NOUT / 16;
  #pragma unroll
      for (int pass = 0; pass < PASSES; ++pass) {
  #pragma unroll
        for (int f = 0; f < NF; ++f)
  #pragma unroll
          for (int jj = 0; jj < PJ; ++jj) {
            const int j = pass * PJ + jj;
            float o[4];
            outv(f, j, o);
            const int srow = 16 * jj + l16;
            const uint32_t lo = pack16x2<F16>(o[0], o[1]);
            const uint32_t hi = pack16x2<F16>(o[2], o[3]);
            *reinterpret_cast<uint2*>(lds + srow * PITCH + 2 * tcol(f, 0)) = make_uint2(lo, hi);
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
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  const bool hasb = a.bias != nullptr;
  auto run = [&](auto silu_c, auto clamp_c) {
    if (hasb) epilogue(silu_c, clamp_c, T_{});
    else epilogue(silu_c, clamp_c, F_{});
  };
  if constexpr (!kGlu) {
    run(T_{}, F_{});
  } else {
    const bool clamp = a.clamp_limit > 0.f;
    if (a.act == MI355MOE_ACT_SILU) {
      if (clamp) run(T_{}, T_{});
      else run(T_{}, F_{});
    } else {
      if (clamp) run(F_{}, T_{});
      else run(F_{}, F_{});
    }
  }
}

template <int EPI, bool QOUT, bool F16, int MXK>
int launch_w8p(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : 256;
  const int64_t total = cdiv(a.N, cols) * max_blocks;
  dim3 grid(static_cast<unsigned>(cdiv(total, 8) * 8));
  moe_gemm_wide8p_kernel<EPI, QOUT, F16, MXK><<<grid, dim3(512), 0, st>>>(a, qs);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

template <int MXK>
int launch_w8p_recipe(int epi, bool qout, const GemmArgs& a, int64_t max_blocks, void* qs,
                      hipStream_t st) {
  if (qout)
    return a.out_f16 ? launch_w8p<EPI_GLU, true, true, MXK>(a, max_blocks, qs, st)
                     : launch_w8p<EPI_GLU, true, false, MXK>(a, max_blocks, qs, st);
  if (epi == EPI_GLU)
    return a.out_f16 ? launch_w8p<EPI_GLU, false, true, MXK>(a, max_blocks, qs, st)
                     : launch_w8p<EPI_GLU, false, false, MXK>(a, max_blocks, qs, st);
  return a.out_f16 ? launch_w8p<EPI_STORE, false, true, MXK>(a, max_blocks, qs, st)
                   : launch_w8p<EPI_STORE, false, false, MXK>(a, max_blocks, qs, st);
}

}  // namespace

// kWideBM-slot blocks; fp8 block-scaled weights (K % 128 == 0, K <= 8192),
// or mxfp8 weights with K-blocked e8m0 scales ([E, K/32, ldb_rows]) and e8m0
// activation codes (a_mxs; K % 128 == 0), or e2m1 x e2m1 (RECIPE_MX4A4,
// K-blocked mxfp4 weights and scales; K % 32 == 0); the caller checks
// wide8_supported / wide8_shape_ok.
int launch_moe_gemm_wide8p(int recipe, int epi, bool qout, const GemmArgs& a,
                           int64_t max_blocks, void* qs, hipStream_t st) {
  if (recipe == MI355MOE_RECIPE_MXFP8)
    return launch_w8p_recipe<1>(epi, qout, a, max_blocks, qs, st);
  if (recipe == RECIPE_MX4A4)
    return launch_w8p_recipe<2>(epi, qout, a, max_blocks, qs, st);
  return launch_w8p_recipe<0>(epi, qout, a, max_blocks, qs, st);
}

}  // namespace mi355
