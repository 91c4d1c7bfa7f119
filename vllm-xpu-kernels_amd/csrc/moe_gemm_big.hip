// Prefill grouped GEMM: 128-slot x 256-weight-row tiles, both operands staged
// through double-buffered LDS, 32x32 MFMA.
//
// Workgroup = 4 wavefronts in a 2 (slots) x 2 (weight rows) grid; wave (wm,wn)
// owns slots [64wm, 64wm+64) and weight rows [128wn, 128wn+128) of the tile
// (GLU: gate rows [64wn, 64wn+64) of the tile's gate half and the matching up
// rows), i.e. 4 x 2 MFMA tiles of 32x32.  The MFMA A operand is the weight
// (rows n), the B operand the activation (columns m), so lane l owns slot
// m = l%32 and weight rows n = 8*(r/4) + 4*(l/32) + r%4 of accumulator r:
// one fp8 scale product per tile and 8-byte output stores.
//
// K stage: 128 bytes of every staged row (64 bf16 / 128 e4m3 / 128 e2m1 that
// are expanded to bf16 on their way into LDS).  Global loads of stage k+1 are
// issued into registers before the MFMAs of stage k and written to the other
// LDS buffer after them, one barrier per stage.
#include "gemm32_common.h"

namespace mi355 {
namespace {

constexpr int BM = 128;       // slots per tile
constexpr int BN = 256;       // weight rows per tile
constexpr int ROWB = 128;     // staged bytes per row per K stage
constexpr int PITCH = ROWB + 16;
constexpr int A_CH = BM * ROWB / 16;   // 16-byte chunks of the activation tile
constexpr int W_CH = BN * ROWB / 16;   // of the weight tile (bf16 / e4m3)

// Weight row (within the expert) staged at tile row r.
__device__ __forceinline__ int64_t tile_wrow(int r, int64_t n0, bool glu,
                                             int64_t up_off, int64_t N,
                                             bool& ok) {
  int64_t n;
  if (glu) {
    // tile rows [0,128) = gate rows n0 + [0,128), [128,256) = up rows
    const int64_t c = n0 + (r & 127);
    ok = c < N;
    n = (r >= 128 ? up_off : 0) + (ok ? c : 0);
  } else {
    const int64_t c = n0 + r;
    ok = c < N;
    n = ok ? c : 0;
  }
  return n;
}

template <int RECIPE, int EPI, bool QOUT, bool F16>
__global__ __launch_bounds__(256, 1) void moe_gemm_big_kernel(const GemmArgs a,
                                                              void* __restrict__ qs) {
  constexpr bool kFp8 = RECIPE == MI355MOE_RECIPE_FP8BLOCK;
  constexpr bool kFp4 = RECIPE == MI355MOE_RECIPE_MXFP4 || RECIPE == MI355MOE_RECIPE_INT4;
  constexpr bool kGlu = EPI == EPI_GLU;
  constexpr int KE = kFp8 ? 128 : 64;        // K elements per stage
  // per-thread staging: activations, then weights
  constexpr int NA = A_CH / 256;             // 4
  constexpr int NW = kFp4 ? (BN * 32 / 16) / 256 : W_CH / 256;  // 2 or 8

  __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) uint8_t sW[2][BN * PITCH];
  __shared__ int s_arow[BM];
  __shared__ int s_drow[BM];
  __shared__ float s_xs[2][BM];
  __shared__ float s_amax[2][128];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;
  const int blk = blockIdx.y;
  if (blk * BM >= *a.ntp) return;  // uniform
  const int e = a.block_expert[blk];
  const int64_t K = a.K;
  const int64_t N = a.N;
  // GLU tiles cover 128 output (activation) columns, others 256
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (kGlu ? 128 : BN);
  const int64_t wrow_bytes = kFp4 ? K / 2 : (kFp8 ? K : 2 * K);

  if (tid < BM) {
    const int rid = a.row_ids[static_cast<int64_t>(blk) * BM + tid];
    const bool ok = rid >= 0 && rid < a.num_valid;
    s_arow[tid] = ok ? (a.a_by_pos ? blk * BM + tid : rid / a.a_div) : -1;
    s_drow[tid] = ok ? (a.d_by_pos ? blk * BM + tid : rid) : -1;
  }
  __syncthreads();

  // ---- per-thread global source addresses (fixed across K stages)
  const uint8_t* abase = static_cast<const uint8_t*>(a.A);
  const int64_t arow_bytes = (kFp8 ? 1 : 2) * K;
  const uint8_t* asrc[NA];
  bool aok[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int idx = i * 256 + tid;
    const int r = idx / (ROWB / 16), c = idx % (ROWB / 16);
    const int ar = s_arow[r];
    aok[i] = ar >= 0;
    asrc[i] = abase + static_cast<int64_t>(aok[i] ? ar : 0) * arow_bytes + c * 16;
  }
  const uint8_t* wexp = static_cast<const uint8_t*>(a.B) +
                        static_cast<int64_t>(e) * a.ldb_rows * wrow_bytes;
  // mxfp4 weights and scales may be K-blocked (16-bit and fp8 weights here
  // are row-major)
  const WStride wst = kFp4 ? w_stride4(a) : WStride{wrow_bytes, 0};
  const WStride sst = s_stride4(a);
  const uint8_t* wsrc[NW];
  bool wokv[NW];
  int64_t wrowv[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int idx = i * 256 + tid;
    const int per_row = kFp4 ? 2 : ROWB / 16;
    const int r = idx / per_row, c = idx % per_row;
    bool ok;
    const int64_t n = tile_wrow(r, n0, kGlu, a.up_off, N, ok);
    wokv[i] = ok;
    wrowv[i] = n;
    wsrc[i] = kFp4 ? wexp + n * wst.row + c * wst.kblk : wexp + n * wrow_bytes + c * 16;
  }

  uint4 ra[NA], rw[NW];
  uint32_t rsc[kFp4 ? NW : 1];
  auto gload = [&](int64_t k0) {
    const int64_t kb = K - k0;  // elements left
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = i * 256 + tid;
      const int c = idx % (ROWB / 16);
      const bool ok = aok[i] && (c * 16) < kb * (kFp8 ? 1 : 2);
      ra[i] = ok ? *reinterpret_cast<const uint4*>(asrc[i] + k0 * (kFp8 ? 1 : 2))
                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int idx = i * 256 + tid;
      if constexpr (kFp4) {
        const int c = idx % 2;  // 16 bytes = 32 e2m1 values = one scale group
        const bool ok = wokv[i] && 32 * c < kb;
        rw[i] = ok ? *reinterpret_cast<const uint4*>(wsrc[i] + (k0 / 32) * wst.kblk)
                   : make_uint4(0, 0, 0, 0);
        rsc[i] = ok ? w4_scale_code<RECIPE>(a, e, wrowv[i], k0 / 32 + c, sst) : 0u;
      } else {
        const int c = idx % (ROWB / 16);
        const bool ok = wokv[i] && (c * 16) < kb * (kFp8 ? 1 : 2);
        rw[i] = ok ? *reinterpret_cast<const uint4*>(wsrc[i] + k0 * (kFp8 ? 1 : 2))
                   : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto lstore = [&](int buf, int64_t k0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = i * 256 + tid;
      const int r = idx / (ROWB / 16), c = idx % (ROWB / 16);
      *reinterpret_cast<uint4*>(&sA[buf][r * PITCH + c * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int idx = i * 256 + tid;
      if constexpr (kFp4) {
        const int r = idx / 2, c = idx % 2;
        const uint4 v = rw[i];
        uint8_t* d = &sW[buf][r * PITCH + c * 64];
        *reinterpret_cast<uint4*>(d) = w4_decode8<RECIPE, F16>(v.x, rsc[i]);
        *reinterpret_cast<uint4*>(d + 16) = w4_decode8<RECIPE, F16>(v.y, rsc[i]);
        *reinterpret_cast<uint4*>(d + 32) = w4_decode8<RECIPE, F16>(v.z, rsc[i]);
        *reinterpret_cast<uint4*>(d + 48) = w4_decode8<RECIPE, F16>(v.w, rsc[i]);
      } else {
        const int r = idx / (ROWB / 16), c = idx % (ROWB / 16);
        *reinterpret_cast<uint4*>(&sW[buf][r * PITCH + c * 16]) = rw[i];
      }
    }
    if constexpr (kFp8) {
      if (tid < BM) {
        const int ar = s_arow[tid];
        s_xs[buf][tid] = ar >= 0 ? a.a_scale[static_cast<int64_t>(ar) * (K / 128) + k0 / 128]
                                 : 0.f;
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

  // weight tile rows of this wave's 4 n-tiles
  int wtile_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kGlu)  // 2 gate tiles then the 2 matching up tiles
      wtile_row[i] = (i < 2 ? 0 : 128) + 64 * wn + 32 * (i & 1);
    else
      wtile_row[i] = 128 * wn + 32 * i;
  }
  // fp8 weight-block scale rows of the 4 n-tiles
  const float* bsc = static_cast<const float*>(a.b_scale);
  const int wsh = 7 - a.ws_rows64;  // 32-row sub-tiles sit inside one 128- or 64-row block
  int64_t wsc_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bool ok;
    wsc_row[i] = tile_wrow(wtile_row[i], n0, kGlu, a.up_off, N, ok) >> wsh;
  }

  const int nk = static_cast<int>((K + KE - 1) / KE);
  gload(0);
  lstore(0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const int64_t k0 = static_cast<int64_t>(kt) * KE;
    if (kt + 1 < nk) gload(k0 + KE);
    const uint8_t* As = sA[cur];
    const uint8_t* Ws = sW[cur];
    if constexpr (kFp8) {
      float ws[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ws[i] = bsc[(static_cast<int64_t>(e) * (a.ldb_rows >> wsh) + wsc_row[i]) * (K / 128) +
                    k0 / 128];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = 64 * wm + 32 * j + l32;
        const uint8_t* xr = As + m * PITCH + 32 * h;
        const uint4 x0 = *reinterpret_cast<const uint4*>(xr);
        const uint4 x1 = *reinterpret_cast<const uint4*>(xr + 16);
        const uint4 x2 = *reinterpret_cast<const uint4*>(xr + 64);
        const uint4 x3 = *reinterpret_cast<const uint4*>(xr + 80);
        const float xs = s_xs[cur][m];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint8_t* wr = Ws + (wtile_row[i] + l32) * PITCH + 32 * h;
          f32x16 p;
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = 0.f;
          p = mfma32_fp8(*reinterpret_cast<const uint4*>(wr),
                         *reinterpret_cast<const uint4*>(wr + 16), x0, x1, p);
          p = mfma32_fp8(*reinterpret_cast<const uint4*>(wr + 64),
                         *reinterpret_cast<const uint4*>(wr + 80), x2, x3, p);
          const float s = xs * ws[i];
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += p[r] * s;
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int koff = (16 * ks + 8 * h) * 2;
        uint4 xf[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          xf[j] = *reinterpret_cast<const uint4*>(As + (64 * wm + 32 * j + l32) * PITCH + koff);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 wf =
              *reinterpret_cast<const uint4*>(Ws + (wtile_row[i] + l32) * PITCH + koff);
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma16_32x32x16<F16>(wf, xf[j], acc[i][j]);
        }
      }
    }
    if (kt + 1 < nk) lstore(cur ^ 1, k0 + KE);
    __syncthreads();
  }

  static_assert(sizeof(sW) >= 128 * (2 * 256 + 16), "epilogue staging");
  epilogue_32x32<kGlu, QOUT, F16>(a, qs, acc, e, n0, wm, wn, l32, h, s_drow, s_amax,
                                static_cast<int>(blockIdx.x), &sW[0][0]);
}

template <int RECIPE, int EPI, bool QOUT, bool F16>
int launch_big_t(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  const int64_t cols = EPI == EPI_GLU ? 128 : BN;
  dim3 grid(static_cast<unsigned>(cdiv(a.N, cols)), static_cast<unsigned>(max_blocks));
  moe_gemm_big_kernel<RECIPE, EPI, QOUT, F16><<<grid, dim3(256), 0, st>>>(a, qs);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
template <int RECIPE, int EPI, bool QOUT>
int launch_big(const GemmArgs& a, int64_t max_blocks, void* qs, hipStream_t st) {
  return a.out_f16 ? launch_big_t<RECIPE, EPI, QOUT, true>(a, max_blocks, qs, st)
                   : launch_big_t<RECIPE, EPI, QOUT, false>(a, max_blocks, qs, st);
}

}  // namespace

// 128-slot blocks only (the caller aligns expert segments to 128).
int launch_moe_gemm_big(int recipe, int epi, bool qout, const GemmArgs& a,
                        int64_t max_blocks, void* qs, hipStream_t st) {
  if (max_blocks <= 0 || a.N <= 0) return MI355MOE_OK;
  if (qout) {
    MI_ARG(recipe == MI355MOE_RECIPE_FP8BLOCK && epi == EPI_GLU && a.N % 128 == 0,
           "fp8 activation output needs the fp8block recipe and I % 128 == 0");
    return launch_big<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, true>(a, max_blocks, qs, st);
  }
  switch (recipe) {
    case MI355MOE_RECIPE_BF16:
      return epi == EPI_GLU ? launch_big<MI355MOE_RECIPE_BF16, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_big<MI355MOE_RECIPE_BF16, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_FP8BLOCK:
      return epi == EPI_GLU ? launch_big<MI355MOE_RECIPE_FP8BLOCK, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_big<MI355MOE_RECIPE_FP8BLOCK, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_MXFP4:
      return epi == EPI_GLU ? launch_big<MI355MOE_RECIPE_MXFP4, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_big<MI355MOE_RECIPE_MXFP4, EPI_STORE, false>(a, max_blocks, qs, st);
    case MI355MOE_RECIPE_INT4:
      return epi == EPI_GLU ? launch_big<MI355MOE_RECIPE_INT4, EPI_GLU, false>(a, max_blocks, qs, st)
                            : launch_big<MI355MOE_RECIPE_INT4, EPI_STORE, false>(a, max_blocks, qs, st);
    default:
      return set_error(MI355MOE_ERR_INVALID, "unknown recipe");
  }
}

}  // namespace mi355
