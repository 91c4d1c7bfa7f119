// Grouped-GEMM launcher shared by the grouped_gemm and fused_moe entry points.
#pragma once

#include "common.h"

namespace mi355 {

// One launch computes, for every block b of BM sorted slots (all of one
// expert e = block_expert[b]):
//   rows  r_i = row_ids[b*BM + i]   (r_i >= num_valid: padding slot)
//   A row = a_by_pos ? b*BM+i : r_i / a_div
//   D row = d_by_pos ? b*BM+i : r_i
//   STORE: D[row, n] = T(sum_k A[row,k] W_e[n,k] + bias_e[n])
//   GLU:   g = T(acc(n) + b(n)), u = T(acc(I+n) + b(I+n)),
//          D[row, n] = act(g, u)          (n < N = I; W_e has 2I rows)
// Recipe codes of the grouped-GEMM kernels beyond the C ABI's: e2m1
// activations with e8m0 scales against mxfp4 weights (both scales in the
// MFMA), which the fused layer runs for mxfp4 with pre-quantised inputs.
constexpr int RECIPE_MX4A4 = 16;
__host__ __device__ constexpr bool is_mx_recipe(int r) {
  return r == MI355MOE_RECIPE_MXFP8 || r == RECIPE_MX4A4;
}
// Per-expert fp8 weights (e4m3 or e5m2) against 16-bit activations: the
// STREAM kernels convert them to the activations' type as they load them.
__host__ __device__ constexpr bool is_w8a16_recipe(int r) {
  return r == MI355MOE_RECIPE_FP8 || r == MI355MOE_RECIPE_FP8E5M2;
}
// 16-bit (and w8a16) weights: layers averaging at most this many slots per
// active expert run the STREAM kernels, up to kSmallMaxAvg16 the 64-slot
// SMALL kernels
constexpr int64_t kStreamMaxAvg16 = 10;
constexpr int64_t kSmallMaxAvg16 = 48;

// The split-K w13 GEMM of the fused layer left its partial tiles (no
// finalize launch); the STREAM w2 launch rebuilds each workgroup's 16-bit
// activation rows from them (part != null): the w13 tile's partials summed
// in split order, then its GLU epilogue (expert scale, bias, rounding,
// clamp, activation).  The w13 GEMM's own parameters.
struct G1Fin {
  const float* part;     // [blocks, n_tiles, ks, 512 x 8]
  int32_t ks, n_tiles;
  int64_t N, up_off, ldb_rows;
  const uint16_t* bias;
  const float* expert_scale;
  float clamp_limit, alpha, limit;
  int32_t act;
};
// LDS bytes for those rows: 16 slots x the split's K range, 16-bit.
constexpr int64_t kStreamG1FinBytes = 32768;

struct GemmArgs {
  const void* A;
  const float* a_scale;  // fp8: [rowsA, K/128]
  const void* B;         // [E, ldb_rows, K] (mxfp4: K/2 bytes per row)
  const void* b_scale;   // fp8: f32 [E, ldb_rows/128, K/128] (or /64, ws_rows64);
                         // mxfp4: u8 [E, ldb_rows, K/32]
  const uint16_t* bias;  // [E, ldb_rows] bf16 or null
  void* D;
  const int32_t* row_ids;
  const int32_t* block_expert;
  const int32_t* ntp;    // [1] number of valid padded slots
  const int32_t* expert_cum;  // [E+1] padded slot start per expert, or null
  int32_t num_valid;
  int32_t a_div;
  int32_t a_by_pos;
  int32_t d_by_pos;
  int64_t N;
  int64_t K;
  int64_t ldb_rows;
  int64_t up_off;        // GLU: row offset of the up half (= I)
  float clamp_limit;     // GLU: <= 0 off
  float alpha;           // swigluoai alpha
  float limit;           // swigluoai limit
  int32_t act;           // mi355moe_activation
  int32_t out_f16;       // store fp16 instead of bf16 (recipe BF16 only)
  // Weight layout: 0 row-major [E, ldb_rows, K]; 1 K-blocked [E, K/B,
  // ldb_rows, B] (recipe BF16: B = 32, FP8BLOCK: B = 128, MXFP4: B = 32
  // elements, with the e8m0 scales K-blocked too, [E, K/32, ldb_rows]),
  // in which the K-slices of consecutive weight rows are contiguous, so a
  // 16-row fragment of one K block is a single 1-2 KiB run of HBM instead of
  // 16 runs of 64-128 bytes.
  int32_t w_kblock;
  // STREAM family split-K: ksplit workgroups share one output tile, each
  // summing 1/ksplit of the K stages into an fp32 partial tile in `part`; a
  // second launch adds the partials in split order and runs the epilogue.
  // (No workgroup waits for another: the per-XCD L2s are not coherent, so a
  // device-scope fence would write back and invalidate a whole L2.)
  int32_t ksplit;        // 0 or 1: no split
  float* part;           // [blocks, n_tiles, ksplit, 512 x 8]
  int32_t finalize;      // set by the launcher for the second launch
  int32_t partials_only; // split launch only: the caller consumes `part`
  // Recipe BF16 only, optional: fp32 [E] factor on each expert's accumulators
  // before the bias (per-expert-scaled fp8 weights, converted exactly to the
  // 16-bit type: D = T(s_e * sum_k A W_e + bias_e)).
  const float* expert_scale;
  int32_t w_group;       // recipe INT4: K values per 16-bit scale (32..256)
  // recipe FP8BLOCK: 1 = b_scale [E, ldb_rows/64, K/128], one scale row per
  // 64 weight rows (the split gate / up halves of an interleaved swigluoai
  // w13, whose 128-row blocks each held 64 gates and their 64 ups); 0 = 128
  int32_t ws_rows64;
  // SMALL kernels, order of the (M-block, N-tile) pairs over the XCDs (set
  // by the launcher): 1 = all N-tiles of an M-block on one XCD, -1 = spread
  // round-robin, 0 = the first for 16-bit activations averaging 8 or more
  // valid rows per block, else the second
  int32_t xcd_order;
  // MX recipes: e8m0 activation scales u8, row r's 32-K group g at
  // a_mxs[r * a_mxs_ld + g] (a_mxs_ld >= K/32; a multiple of 4 where a kernel
  // moves them four at a time); the w13 epilogue of the fused layer writes
  // its quantised output's scales to qs with row stride q_mxs_ld.
  const uint8_t* a_mxs;
  int64_t a_mxs_ld;
  int64_t q_mxs_ld;
  // STREAM w13 of the fused layer with at most 16 slots (num_valid): every
  // workgroup of the split launch sorts the top-k ids itself, with the
  // counting sort's key rule and ordering (block b = the b-th smallest
  // routed expert, its rows the expert's slots in flat order), and
  // workgroup (0, 0, 0) writes the sort's outputs (sr_sorted padded with
  // num_valid, sr_eids, sr_ntp, sr_cum, sr_inv) for the launches that
  // follow, so no sort launch runs.  With sr_x (fp8block recipe) the
  // activation is the 16-bit hidden states [T, K], quantised per 1 x 128
  // block by the group quantiser into LDS before the K loop.
  const void* sr_ids;    // null: the sort launch ran
  int32_t sr_ids_dtype;
  const int32_t* sr_map;
  int64_t sr_id_bound;
  int32_t sr_keys;       // experts (sort keys)
  int64_t sr_max_padded, sr_max_blocks;
  int32_t *sr_sorted, *sr_eids, *sr_ntp, *sr_cum, *sr_inv;
  const uint16_t* sr_x;
  // STREAM w2 of the fused layer in token-major form (tok_out set; STORE,
  // no split, 8 % topk == 0): workgroup (x, t) covers token t and 8 / topk
  // groups of 32 output columns; wave w takes slot j = w % topk of the token
  // (its sorted position tok_inv[t topk + j], its expert block_expert[pos /
  // 16], activation row pos) over the group's 32 weight rows, and the
  // group's slots are summed through LDS into
  //   tok_out[t, n] = T(sum_j tok_w[t topk + j] * T(acc_j(n) + bias_j(n)))
  // over the slots the sort kept, in j order -- the arithmetic of the
  // separate top-k reduction launch, which is then not needed.
  const int32_t* tok_inv;
  const float* tok_w;
  int32_t topk;
  void* tok_out;
  // columns per group (a multiple of 4 up to 32; 0: 32): a narrower group
  // gives more workgroups (7168 columns in 28-column groups: 256, one per
  // CU, against 224); the rows of a wave's 32-row tile past the group read
  // the group's last row again (the same cache lines) and are not stored
  int32_t tok_cw;
  // Token-major w2, fp8block recipe: A is the 16-bit activation [rows, K]
  // (no a_scale); each wave quantises its slot's row per 1 x 128 block with
  // the group quantiser into LDS before its K loop (K <= kStreamTokXBytes).
  int32_t tok_xq;
  // STREAM w13 GLU without a split launch: the workgroup's 8 waves are 4
  // groups of 16 activation columns (64 per workgroup) x 2 halves of the K
  // stages; the upper half's sums are added to the lower half's through LDS
  // (the split-K finalize's order), then the GLU epilogue stores the 16-bit
  // activation.  Decode grids with too few 128-column tiles to fill the GPU.
  int32_t khalves;
  // STREAM w2 of the fused layer (16-bit activation): its activation rows
  // rebuilt from the w13 partials (G1Fin) instead of read from A.
  G1Fin g1f;
  // 320-slot fp8 / MX kernel: activation scales by sorted position instead
  // of by row (a_scale[kb * a_scale_tld + position], 0: the row-major
  // [rows, K/128]; MX: the 4-code words of a_mxs, word w of a position at
  // (w * a_scale_tld + position) * 4 bytes), and the w13 epilogue's output
  // scales / codes the same way (q_scale_tld).  A stage's 320 scales are then
  // about ten cache lines instead of one line per slot row.
  int64_t a_scale_tld, q_scale_tld;
  // 320-slot e2m1 x e2m1 kernel: row pitch in bytes of A and of its e2m1
  // output D (0: the packed K / 2 and N / 2).  A pitch that is a multiple of
  // 128 keeps every 128-byte stage of a row inside one cache line.
  int64_t lda, ldd;
};
// LDS bytes a STREAM workgroup gives the in-kernel-quantised activation
// (GemmArgs::sr_x): tokens x the split's K range, e4m3 (and 1 x 128 scales).
constexpr int64_t kStreamSelfXBytes = 32768;
// LDS bytes per wave for the token-major w2's quantised row (tok_xq).
constexpr int64_t kStreamTokXBytes = 4096;

// gemm1_clamp_limit on the (gate, up) pair of GLU output column n, both
// already in the 16-bit type (the host rounds the limit to that type, so the
// result needs no further rounding).  The reference clamps G1's columns
// [0, I) from above and [I, 2I) on both sides (fused_moe_interface.py:
// 384-389).  swigluoai's G1 interleaves gate and up (column n's pair at 2n,
// 2n + 1): both are clamped from above, and from below where 2n >= I; for
// the other activations gate = [0, I) and up = [I, 2I).
// (limit L, activation act, N = I of the GEMM)
__device__ __forceinline__ void glu_clamp_with(float L, int act, int64_t N, int64_t n, float& g,
                                               float& u) {
  if (!(L > 0.f)) return;
  const bool swig = act == MI355MOE_ACT_SWIGLUOAI;
  const bool upper_half = 2 * n >= N;
  g = fminf(g, L);
  if (swig && upper_half) g = fmaxf(g, -L);
  u = fminf(u, L);
  if (!swig || upper_half) u = fmaxf(u, -L);
}
__device__ __forceinline__ void glu_clamp(const GemmArgs& a, int64_t n, float& g, float& u) {
  glu_clamp_with(a.clamp_limit, a.act, a.N, n, g, u);
}

enum GemmEpi { EPI_STORE = 0, EPI_GLU = 1 };

// Byte strides of 16-bit weights: element (row r, k) of one expert sits at
// r * row + (k / 32) * kblk + (k % 32) * 2 (row-major: row = 2K, kblk = 64;
// K-blocked: row = 64, kblk = 64 ldb_rows).  An expert spans 2 K ldb_rows
// bytes in both layouts.
struct WStride {
  int64_t row, kblk;
};
__device__ __forceinline__ WStride w_stride16(const GemmArgs& a) {
  return a.w_kblock ? WStride{64, a.ldb_rows * 64} : WStride{a.K * 2, 64};
}
__device__ __forceinline__ int64_t w_koff16(const WStride& s, int64_t k) {
  return (k >> 5) * s.kblk + (k & 31) * 2;
}
// e4m3 weights (K blocks of 128 bytes): element (row r, k) at r * row +
// (k / 128) * kblk + k % 128.
__device__ __forceinline__ WStride w_stride8(const GemmArgs& a) {
  return a.w_kblock ? WStride{128, a.ldb_rows * 128} : WStride{a.K, 128};
}
// per-expert fp8 weights (K blocks of 32 bytes): element (row r, k) at r *
// row + (k / 32) * kblk + k % 32.
__device__ __forceinline__ WStride w_stride8w(const GemmArgs& a) {
  return a.w_kblock ? WStride{32, a.ldb_rows * 32} : WStride{a.K, 32};
}
// mxfp4 e2m1 pairs (K blocks of 32 values = 16 bytes): block kb of row r at
// r * row + kb * kblk; its e8m0 scale byte at r * row + kb * kblk of
// s_stride4 (row-major scales [E, N, K/32], K-blocked [E, K/32, N]).
__device__ __forceinline__ WStride w_stride4(const GemmArgs& a) {
  return a.w_kblock ? WStride{16, a.ldb_rows * 16} : WStride{a.K / 2, 16};
}
__device__ __forceinline__ WStride s_stride4(const GemmArgs& a) {
  return a.w_kblock ? WStride{1, a.ldb_rows} : WStride{a.K / 32, 1};
}

// Tile t of the (block, N-tile) grid.  With expert_cum the order is (expert,
// N-tile, block): the blocks of one expert take the same weight rows back
// to back, so they share them in L2 instead of each streaming them from
// HBM; without it, row-major (block, N-tile).
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int t, int n_tiles, int bm,
                                            int& blk, int& nt) {
  if (a.expert_cum) {
    const int b0 = t / n_tiles;
    const int e = a.block_expert[b0];
    const int fb = a.expert_cum[e] / bm;
    const int nb = a.expert_cum[e + 1] / bm - fb;
    const int local = t - fb * n_tiles;
    nt = local / nb;
    blk = fb + local % nb;
  } else {
    blk = t / n_tiles;
    nt = t % n_tiles;
  }
}

// Launch over max_blocks M-blocks of bm rows.  bm in {16, 32, 64, 128}.
int launch_moe_gemm(int recipe, int epi, int bm, const GemmArgs& a,
                    int64_t max_blocks, hipStream_t st);

// Block size by the expected rows per active expert (16 up to 24, 32 up to
// 48, 64 up to 96, else 128): the SMALL family's block when forced.
int pick_block_m(int64_t slots, int64_t num_experts);

// Kernel family and block size by recipe and the expected slots per active
// expert (avg), break points measured over the benchmark configurations
// (bf16 Qwen3-30B-A3B, fp8 DeepSeek-V3 and Qwen3-235B, mxfp4 gpt-oss-20b,
// 1..8192 tokens, every family forced in turn):
//   bf16   avg <= 10 STREAM;  <= 48 SMALL bm 64;                     else WIDE
//   fp8    avg <= 4  STREAM;  <= 12 SMALL bm 16;   <= 160 BIG;        else WIDE
//   mxfp4  avg <= 2  STREAM;  <= 24 SMALL bm 16;   <= 40 SMALL bm 32; else WIDE
// STREAM: independent-wave weight streaming, 16-slot blocks; SMALL: LDS-shared
// activation tile; BIG: 128x256 LDS-staged tiles, 128-slot blocks; WIDE:
// 320x256 tiles, 320-slot blocks (kWideBM), where the shape fits (wide_ok,
// see wide_ok_for; otherwise bf16 SMALL bm 64 up to avg 96, mxfp4 SMALL bm 32
// up to 48, then BIG).
// MI355MOE_GEMM_TILE=stream|small|big|bigreg|wide overrides (A/B
// measurements; wide falls back to big where it does not apply, small takes
// pick_block_m's block size).
// (TILE_BIG runs the 8-wave fp8 kernel where big8_supported(), else the
// LDS-DMA pipelined kernel where pipe_supported(), else the register-staged
// one, which TILE_BIGREG forces.)
enum GemmTile { TILE_STREAM = 0, TILE_SMALL = 1, TILE_BIG = 2, TILE_BIGREG = 3, TILE_WIDE = 4 };
constexpr int kWideBM = 320;  // slots per block of the WIDE family
GemmTile pick_tile(int recipe, bool wide_ok, int64_t slots, int64_t num_experts, int* bm);
// Whether a GEMM with a_rows activation rows, ldb_rows weight rows per
// expert (0: not known yet), reduction length K and the given weight layout
// fits the WIDE kernels (mxfp4: K-blocked weights only).
bool wide_ok_for(int recipe, int64_t a_rows, int64_t ldb_rows, int64_t K, bool w_kblock = false);

// Launch the chosen family over max_blocks blocks of bm slots.
int launch_tile_gemm(GemmTile tile, int bm, int recipe, int epi, bool qout,
                     const GemmArgs& a, int64_t max_blocks, void* qs,
                     hipStream_t st);

int launch_moe_gemm_q(int recipe, int epi, bool qout, int bm, const GemmArgs& a,
                      int64_t max_blocks, void* qs, hipStream_t st);
// 128-slot blocks; GLU tiles cover 128 output columns, STORE tiles 256.
int launch_moe_gemm_big(int recipe, int epi, bool qout, const GemmArgs& a,
                        int64_t max_blocks, void* qs, hipStream_t st);
// 128-slot blocks, 3-stage global->LDS DMA ring (moe_gemm_pipe.hip).
bool pipe_supported(int recipe, const GemmArgs& a);
int launch_moe_gemm_pipe(int recipe, int epi, bool qout, const GemmArgs& a,
                         int64_t max_blocks, void* qs, hipStream_t st);
// 128-slot blocks, fp8 block-scaled weights, K % 128 == 0, K <= 8192
// (moe_gemm_big8.hip).
bool big8_supported(int recipe, const GemmArgs& a);
int launch_moe_gemm_big8(int recipe, int epi, bool qout, const GemmArgs& a,
                         int64_t max_blocks, void* qs, hipStream_t st);
// kWideBM-slot blocks, fp8 block-scaled weights, K % 128 == 0, K <= 8192
// (moe_gemm_wide8.hip); mxfp8 (K-blocked weights and e8m0 scales) runs the
// 8-wave kernel only.
bool wide8_supported(int recipe, const GemmArgs& a);
bool wide8_shape_ok(int64_t a_rows, int64_t ldb_rows, int64_t K);
// e2m1 x e2m1 (RECIPE_MX4A4) on the same tiles: K % 32 == 0, 32-bit byte offsets
bool wide8_shape_ok_mx4(int64_t a_rows, int64_t ldb_rows, int64_t K);
int launch_moe_gemm_wide8(int recipe, int epi, bool qout, const GemmArgs& a,
                          int64_t max_blocks, void* qs, hipStream_t st);
// The same tiles with each wave's weight fragments in a private LDS ring
// (moe_gemm_wide8p.hip); launch_moe_gemm_wide8 dispatches to it.
int launch_moe_gemm_wide8p(int recipe, int epi, bool qout, const GemmArgs& a,
                           int64_t max_blocks, void* qs, hipStream_t st);
// kWideBM-slot blocks, bf16 weights, K % 32 == 0 (moe_gemm_wide.hip).
bool wide_supported(int recipe, const GemmArgs& a);
// The WIDE family addresses activations and one expert's weights with 32-bit
// byte offsets: a_rows x K and ldb_rows x K 16-bit elements must fit.
bool wide_offsets_fit(int64_t a_rows, int64_t ldb_rows, int64_t K);
int launch_moe_gemm_wide(int recipe, int epi, const GemmArgs& a,
                         int64_t max_blocks, hipStream_t st);
// kWideBM-slot blocks, K-blocked mxfp4 weights and scales, K % 32 == 0, N and
// ldb_rows % 4 == 0 (moe_gemm_wide4.hip).
bool wide4_shape_ok(int64_t a_rows, int64_t ldb_rows, int64_t N, int64_t K);
int launch_moe_gemm_wide4(int recipe, int epi, const GemmArgs& a,
                          int64_t max_blocks, hipStream_t st);
// 16-slot blocks; GLU blocks cover 128 output columns, STORE blocks 256.
int launch_moe_gemm_stream(int recipe, int epi, bool qout, const GemmArgs& a,
                           int64_t max_blocks, void* qs, hipStream_t st);

size_t counting_sort_ws_bytes(int64_t numel, int64_t num_keys);
// Stable counting sort of ids into expert order (align.hip).  id_start and
// dedupe_k > 0 select the fused_moe_prologue form: keys are id - id_start,
// only the first occurrence of an expert among a token's dedupe_k ids is
// kept, sorted entries past the last sorted slot are left as they were, and
// with inv_rows > 0 the position of slot t * dedupe_k + j goes to
// inv[j * inv_rows + t].
int run_counting_sort(const void* ids, int ids_dtype, int64_t numel,
                      int64_t id_bound, const int32_t* map, int64_t num_keys,
                      int64_t bs, int32_t* sorted, int64_t max_padded,
                      int32_t* eids, int64_t max_blocks, int32_t* ntp,
                      int32_t* inv, int32_t* counts, int32_t pad,
                      void* ws, size_t ws_bytes, hipStream_t st,
                      int32_t* cum_out = nullptr, int64_t id_start = 0,
                      int dedupe_k = 0, int64_t inv_rows = 0);
// The one-workgroup sort and the e4m3 1 x 128 quantisation of x [rows, cols]
// (16-bit, f16 or bf16) in one launch (align.hip).  Returns 1 without
// launching when the sort needs more than one workgroup or x does not fit
// (16-byte alignment, cols % 128 == 0, i32 / i64 ids).
int run_sort_quant_fp8(const void* ids, int ids_dtype, int64_t numel, int64_t id_bound,
                       const int32_t* map, int64_t num_keys, int64_t bs, int32_t* sorted,
                       int64_t max_padded, int32_t* eids, int64_t max_blocks, int32_t* ntp,
                       int32_t* inv, int32_t pad, int32_t* cum_out, const void* x, bool f16,
                       uint8_t* xq, float* xs, int64_t rows, int64_t cols, hipStream_t st);
// mxfp8 quantisation (per 32, ue8m0 scales stored as e8m0 bytes) of a
// 16-bit x [rows, cols] (elementwise.hip).
int mx8_quant_rows(const void* x, bool f16, uint8_t* q, uint8_t* s, int64_t s_ld,
                   int64_t rows, int64_t cols, hipStream_t st);
// K stages per split of the STREAM family for a GEMM of n_tiles output tiles
// over about `blocks` expert blocks (1: no split)
int stream_ksplit(int64_t n_tiles, int64_t blocks, int64_t K);
int run_segments_to_blocks(const int32_t* rows, int64_t num_keys, int64_t bs,
                           int32_t* row_ids, int64_t max_padded,
                           int32_t* eids, int64_t max_blocks, int32_t* ntp,
                           int32_t pad, hipStream_t st, int32_t* cum_out = nullptr);

}  // namespace mi355
