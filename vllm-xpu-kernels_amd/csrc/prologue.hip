// fused_moe_prologue: the TRT-LLM-style permutation into one byte workspace
// (reference csrc/moe/fused_moe_prologue.cpp:5-151, fused_moe_prologue.hpp).
//
// The workspace holds ten sections, each padded to 256 bytes, in the
// reference's order (fused_moe_prologue.cpp:91-100); the layout is the wire
// format a consumer reads, so it is reproduced exactly.  The permutation is
// the reference's: expanded (unpermuted) row r = j * num_rows + t for top-k
// position j of token t; permuted rows in expert order and, inside an expert,
// in token order; a token that lists one expert twice is routed to it once
// (its first position); experts outside this rank's range are dropped.
//
// Two launches instead of the reference's four: the library's stable
// counting sort (align.hip) writes the permuted row of every expanded row
// (unpermuted_row_to_permuted_row, -1 where a slot is not routed to this
// rank) and the per-expert offsets; then an expand kernel, one wave per
// (token, column chunk), reads the token's activation row once and stores it
// to each of its permuted rows (the reference gathers: one read per permuted row) and fills
// the other index maps, the token scales and the scale rows.  The sort's
// counters live in the blocked_* sections, which the reference also uses as
// its own scratch; their contents afterwards are unspecified.
#include "common.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

enum Section {
  kPermToUnperm = 0,     // permuted_row_to_unpermuted_row   i32 [N]
  kPermExperts,          // permuted_token_selected_experts  i32 [N]
  kUnpermToPerm,         // unpermuted_row_to_permuted_row   i32 [N]
  kBlockedCounts,        // blocked_expert_counts            i32 [E * nblk]
  kBlockedCumsum,        // blocked_expert_counts_cumsum     i32 [E * nblk]
  kBlockedRows,          // blocked_row_to_unpermuted_row    i32 [E * T]
  kFirstTokenOffset,     // expert_first_token_offset        i64 [E + 1]
  kTokenScales,          // permuted_token_final_scales      f32 [N]
  kPermutedData,         // overlapped_gemm1_gemm2_inputs    [N, hidden]
  kPermutedScales,       // permuted_act_scales              [N * hidden / block_k]
  kSections
};
static_assert(kSections == MI355MOE_PROLOGUE_SECTIONS, "section count");

// Tokens per block of the reference's blocked prefix sum
// (fused_moe_prologue.hpp:35-46); it only sizes the blocked_* sections.
int64_t tokens_per_block(int64_t T, int64_t E) {
  for (int64_t tpb = 32; tpb <= 1024; tpb *= 2)
    if (cdiv(T, tpb) * E <= tpb) return tpb;
  return 1024;
}

struct Layout {
  size_t off[kSections];
  size_t size[kSections];
  size_t total;
};

Layout layout(int64_t T, int64_t k, int64_t hidden, int64_t elem_bytes, int64_t block_k,
              int64_t scale_bytes, int64_t E) {
  const int64_t N = T * k;
  const int64_t nblk = T > 0 ? cdiv(T, tokens_per_block(T, E)) : 0;
  const int64_t raw[kSections] = {
      N * 4, N * 4, N * 4, E * nblk * 4, E * nblk * 4, E * T * 4, (E + 1) * 8, N * 4,
      N * hidden * elem_bytes,
      scale_bytes > 0 ? (N * hidden / block_k) * scale_bytes : 0};
  Layout L{};
  size_t at = 0;
  for (int s = 0; s < kSections; ++s) {
    L.size[s] = (static_cast<size_t>(raw[s]) + 255) & ~size_t(255);
    L.off[s] = at;
    at += L.size[s];
  }
  L.total = at;
  return L;
}

// Copy `bytes` from s to d with one wave in 4- or 1-byte steps (rows whose
// ends are not 16-byte aligned, and the short scale rows).
__device__ __forceinline__ void copy_small(const uint8_t* __restrict__ s,
                                           uint8_t* __restrict__ d, int64_t bytes, int lane) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(d) |
                       static_cast<uintptr_t>(bytes);
  if ((al & 3) == 0) {
    const uint32_t* s1 = reinterpret_cast<const uint32_t*>(s);
    uint32_t* d1 = reinterpret_cast<uint32_t*>(d);
    for (int64_t c = lane; c < (bytes >> 2); c += 64) d1[c] = s1[c];
  } else {
    for (int64_t c = lane; c < bytes; c += 64) d[c] = s[c];
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Work unit of a wave: (token t, column chunk c) of NV * 64 16-byte pieces
// of the row (vector path) or the whole row (4- / 1-byte path).
// unperm_to_perm holds the sort's permuted row of every expanded row
// j * T + t (-1: not routed here).  The wave reads its piece of the token's
// row once and stores it to each of the token's permuted rows; the chunk-0
// unit also writes the per-row index and scale entries and the scale rows.
template <typename Id, int NV>
__global__ __launch_bounds__(256) void prologue_expand_kernel(
    const uint8_t* __restrict__ in, int64_t row_bytes, const uint8_t* __restrict__ in_scales,
    int64_t srow_bytes, const Id* __restrict__ ids, const float* __restrict__ token_scales,
    int64_t T, int k, int64_t start, const int32_t* __restrict__ cum, int E,
    const int32_t* __restrict__ unperm_to_perm, int32_t* __restrict__ perm_to_unperm,
    int32_t* __restrict__ perm_experts, int64_t* __restrict__ first_token_offset,
    float* __restrict__ perm_token_scales, uint8_t* __restrict__ out,
    uint8_t* __restrict__ out_scales, int64_t chunks_per_row) {
  if (blockIdx.x == 0)
    for (int e = threadIdx.x; e <= E; e += 256) first_token_offset[e] = cum[e];
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
  const bool vec = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out) |
                     static_cast<uintptr_t>(row_bytes)) & 15) == 0;
  const int64_t units = T * chunks_per_row;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); w < units;
       w += nwaves) {
    const int64_t t = w / chunks_per_row, chunk = w % chunks_per_row;
    const uint8_t* src = in + t * row_bytes;
    if (vec) {
      const uint4* s4 = reinterpret_cast<const uint4*>(src);
      const int64_t n = row_bytes >> 4;
      const int64_t c0 = chunk * NV * 64 + lane;
      // loads clamped into the row (a repeated last piece is not stored) so
      // that they are unconditional and the buffer stays in registers
      uint4 v[NV];
#pragma unroll
      for (int u = 0; u < NV; ++u) v[u] = s4[c0 + u * 64 < n ? c0 + u * 64 : n - 1];
      for (int j = 0; j < k; ++j) {
        const int32_t p = unperm_to_perm[static_cast<int64_t>(j) * T + t];
        if (p < 0) continue;
        // the permuted rows are written once and read by a later kernel:
        // non-temporal stores
        u32x4* d4 = reinterpret_cast<u32x4*>(out + static_cast<int64_t>(p) * row_bytes);
#pragma unroll
        for (int u = 0; u < NV; ++u)
          if (c0 + u * 64 < n)
            __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v[u]), d4 + c0 + u * 64);
      }
    }
    if (chunk != 0) continue;
    // 4-byte scale rows: each 64-word piece read once, stored k times
    const bool svec = srow_bytes > 0 && ((reinterpret_cast<uintptr_t>(in_scales) |
                                          reinterpret_cast<uintptr_t>(out_scales) |
                                          static_cast<uintptr_t>(srow_bytes)) & 3) == 0;
    if (svec) {
      const int64_t nd = srow_bytes >> 2;
      const uint32_t* ss = reinterpret_cast<const uint32_t*>(in_scales) + t * nd;
      for (int64_t c = lane; c - lane < nd; c += 64) {
        const uint32_t v = c < nd ? ss[c] : 0u;
        for (int j = 0; j < k; ++j) {
          const int32_t p = unperm_to_perm[static_cast<int64_t>(j) * T + t];
          if (p >= 0 && c < nd)
            reinterpret_cast<uint32_t*>(out_scales)[static_cast<int64_t>(p) * nd + c] = v;
        }
      }
    }
    for (int j = 0; j < k; ++j) {
      if (vec && (svec || srow_bytes == 0)) break;
      const int32_t p = unperm_to_perm[static_cast<int64_t>(j) * T + t];
      if (p < 0) continue;
      if (!vec) copy_small(src, out + static_cast<int64_t>(p) * row_bytes, row_bytes, lane);
      if (srow_bytes > 0 && !svec)
        copy_small(in_scales + t * srow_bytes, out_scales + static_cast<int64_t>(p) * srow_bytes,
                   srow_bytes, lane);
    }
    for (int j = lane; j < k; j += 64) {
      const int64_t r = static_cast<int64_t>(j) * T + t;
      const int32_t p = unperm_to_perm[r];
      if (p >= 0) {
        perm_to_unperm[p] = static_cast<int32_t>(r);
        perm_experts[p] = static_cast<int32_t>(static_cast<int64_t>(ids[t * k + j]) - start);
        perm_token_scales[p] = token_scales ? token_scales[t * k + j] : 1.0f;
      }
    }
  }
}

}  // namespace
}  // namespace mi355

using namespace mi355;

extern "C" size_t mi355moe_fused_moe_prologue_workspace_layout(
    int64_t num_rows, int64_t experts_per_token, int64_t hidden_size, int64_t elem_bytes,
    int64_t block_k, int64_t scale_bytes, int64_t num_experts_on_rank, size_t* offsets,
    size_t* sizes) {
  if (num_rows < 0 || experts_per_token <= 0 || hidden_size <= 0 || elem_bytes <= 0 ||
      num_experts_on_rank <= 0 || (scale_bytes > 0 && block_k <= 0))
    return 0;
  const Layout L = layout(num_rows, experts_per_token, hidden_size, elem_bytes, block_k,
                          scale_bytes, num_experts_on_rank);
  for (int s = 0; s < kSections; ++s) {
    if (offsets) offsets[s] = L.off[s];
    if (sizes) sizes[s] = L.size[s];
  }
  return L.total;
}

extern "C" int mi355moe_fused_moe_prologue(
    const void* input, int64_t elem_bytes, const void* input_scales, int64_t scale_bytes,
    const void* token_selected_experts, int ids_dtype, const float* token_final_scales,
    void* workspace, size_t workspace_bytes, int64_t num_rows, int64_t hidden_size,
    int64_t inter_size, int64_t block_k, int64_t experts_per_token, int64_t ep_rank,
    int64_t ep_size, int64_t num_experts_on_rank, void* stream) {
  (void)inter_size;  // sizes no section (as in the reference)
  MI_ARG(ep_rank >= 0 && ep_rank < ep_size, "ep_rank must be in [0, ep_size)");
  MI_ARG(num_experts_on_rank > 0 && num_experts_on_rank <= 1024,
         "num_experts_on_rank must be in [1, 1024]");
  MI_ARG(experts_per_token > 0 && num_rows >= 0, "invalid token_selected_experts shape");
  MI_ARG(num_rows * experts_per_token < (int64_t(1) << 31), "too many expanded rows");
  MI_ARG(hidden_size > 0 && (elem_bytes == 1 || elem_bytes == 2),
         "input must hold 1- or 2-byte elements");
  MI_ARG(ids_dtype == MI355MOE_I64 || ids_dtype == MI355MOE_I32,
         "token_selected_experts must be int64 or int32");
  MI_ARG(scale_bytes == 0 || scale_bytes == 1 || scale_bytes == 4,
         "input_scales must be float32 or e8m0");
  MI_ARG(scale_bytes == 0 || (input_scales && block_k > 0 && hidden_size % block_k == 0),
         "input_scales need block_k dividing hidden_size");
  const Layout L = layout(num_rows, experts_per_token, hidden_size, elem_bytes, block_k,
                          scale_bytes, num_experts_on_rank);
  MI_ARG(workspace && workspace_bytes >= L.total,
         "workspace is smaller than the prologue layout");
  MI_ARG((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
         "workspace must be 16-byte aligned");
  const int64_t N = num_rows * experts_per_token;
  if (N == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  auto sec = [&](int s) { return ws + L.off[s]; };
  const int64_t E = num_experts_on_rank;
  const int64_t start = num_experts_on_rank * ep_rank;
  int32_t* u2p = reinterpret_cast<int32_t*>(sec(kUnpermToPerm));

  // sort scratch: per-expert starts [E + 1], then the multi-workgroup sort's
  // counters when the blocked_* sections (contiguous) hold them.  The sort
  // writes the permuted row of every expanded row j * T + t (-1: not routed)
  // straight into unpermuted_row_to_permuted_row.
  int32_t* cum = reinterpret_cast<int32_t*>(sec(kBlockedCounts));
  const size_t scratch_lo = (L.off[kBlockedCounts] + (E + 1) * 4 + 255) & ~size_t(255);
  const size_t scratch_hi = L.off[kFirstTokenOffset];
  const size_t need = counting_sort_ws_bytes(N, E);
  void* sort_ws = (need > 0 && scratch_lo + need <= scratch_hi) ? ws + scratch_lo : nullptr;
  int rc = run_counting_sort(token_selected_experts, ids_dtype, N, E, nullptr, E, 1, nullptr, 0,
                             nullptr, 0, nullptr, u2p, nullptr, 0, sort_ws, sort_ws ? need : 0,
                             st, cum, start, static_cast<int>(experts_per_token), num_rows);
  if (rc) return rc;

  const int64_t row_bytes = hidden_size * elem_bytes;
  const int64_t srow_bytes = scale_bytes > 0 ? (hidden_size / block_k) * scale_bytes : 0;
  // one (token, 4 KiB column chunk) unit per wave, four waves a workgroup
  constexpr int kNV = 4;
  const bool vec = ((reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(
                         sec(kPermutedData)) | static_cast<uintptr_t>(row_bytes)) & 15) == 0;
  const int64_t chunks_per_row = vec ? cdiv(row_bytes >> 4, kNV * 64) : 1;
  const int64_t wgs = cdiv(num_rows * chunks_per_row, 4);
  const unsigned grid = static_cast<unsigned>(wgs < (1 << 20) ? wgs : (1 << 20));
  auto by_nv = [&](auto id_tag) {
    using Id = decltype(id_tag);
    prologue_expand_kernel<Id, kNV><<<grid, 256, 0, st>>>(
        static_cast<const uint8_t*>(input), row_bytes,
        static_cast<const uint8_t*>(input_scales), srow_bytes,
        static_cast<const Id*>(token_selected_experts), token_final_scales, num_rows,
        static_cast<int>(experts_per_token), start, cum, static_cast<int>(E), u2p,
        reinterpret_cast<int32_t*>(sec(kPermToUnperm)),
        reinterpret_cast<int32_t*>(sec(kPermExperts)),
        reinterpret_cast<int64_t*>(sec(kFirstTokenOffset)),
        reinterpret_cast<float*>(sec(kTokenScales)), sec(kPermutedData),
        srow_bytes > 0 ? sec(kPermutedScales) : nullptr, chunks_per_row);
  };
  if (ids_dtype == MI355MOE_I64) by_nv(int64_t{});
  else by_nv(int32_t{});
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
