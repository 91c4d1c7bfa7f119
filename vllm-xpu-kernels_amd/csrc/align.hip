// Token -> expert alignment: a deterministic, stable counting sort of the
// flattened top-k expert ids.  Up to kOneBlockMax ids it runs in one
// 1024-thread workgroup (one launch, the decode case); larger inputs use
// three launches over 1024-id chunks (count, scan, scatter) with the same
// ordering rule, so that the scattered stores of the sorted ids spread over
// the whole GPU instead of one CU.
//
// The 16 wavefronts each own a contiguous chunk of the flat ids, so
// "chunk order, then rank inside the chunk" is flat order.  Per-chunk expert
// counts live in LDS (16 x E ints); a block-wide scan turns them into each
// chunk's first output slot per expert; the scatter pass ranks the lanes of
// every 64-element step that carry the same expert with 11 ballots (one per
// key bit), so no atomics decide the order.  Replaces the reference's
// count + device-atomic scatter (csrc/moe/moe_align_sum_kernels.cpp:135-455),
// whose within-expert order is not deterministic.
#include <type_traits>

#include "common.h"
#include "moe_gemm.h"

namespace mi355 {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kMaxKeys = 1024;
constexpr uint32_t kInvalidKey = 2047u;  // 11 bits, never a valid key

// Options of the fused_moe_prologue sort: ids are shifted by `start` (the
// rank's first expert); with dedupe_k > 1 a slot whose token chose the same
// expert at an earlier top-k position is dropped (only the first occurrence
// of an expert per token is routed); keep_tail leaves sorted_ids past the
// last sorted slot as it was; inv_rows > 0 stores the position of flat slot
// i = t * k + j (k = dedupe_k) at inv_pos[j * inv_rows + t].
struct KeyXform {
  int64_t start;
  int dedupe_k;
  bool keep_tail;
  int64_t inv_rows;
};

__device__ __forceinline__ int64_t inv_index(int64_t i, const KeyXform& xf) {
  return xf.inv_rows > 0 ? (i % xf.dedupe_k) * xf.inv_rows + i / xf.dedupe_k : i;
}

template <typename Id>
__device__ __forceinline__ uint32_t load_key(const Id* ids, int64_t i,
                                             int64_t id_bound,
                                             const int32_t* map,
                                             int num_keys, KeyXform xf = {}) {
  const Id raw = ids[i];
  int64_t v = static_cast<int64_t>(raw) - xf.start;
  if (v < 0 || v >= id_bound) return kInvalidKey;
  if (xf.dedupe_k > 1) {
    for (int64_t q = i - i % xf.dedupe_k; q < i; ++q)
      if (ids[q] == raw) return kInvalidKey;
  }
  if (map) v = map[v];
  if (v < 0 || v >= num_keys) return kInvalidKey;
  return static_cast<uint32_t>(v);
}

// Block-wide exclusive scan of one int per thread (1024 threads).
__device__ int block_exclusive_scan(int v, int* s_wave_tot, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_wave_tot[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int t = lane < kSortWaves ? s_wave_tot[lane] : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int y = __shfl_up(t, o, 64);
      if (lane >= o) t += y;
    }
    if (lane < kSortWaves) s_wave_tot[lane] = t;  // inclusive wave totals
  }
  __syncthreads();
  int before = wave > 0 ? s_wave_tot[wave - 1] : 0;
  total = s_wave_tot[kSortWaves - 1];
  __syncthreads();
  return before + x - v;
}

// Multi-LoRA alignment (moe_lora_align_block_size): workgroup w sorts, for
// the adapter lora_ids[w], only the slots of tokens mapped to it, into its own
// slices of the outputs; invalid (-1, >= max_loras) or disabled adapters
// write nothing; unused blocks get expert id -1.
struct LoraSel {
  const int32_t* tok_lora;  // [tokens] adapter of every token
  int topk;
  const int32_t* lora_ids;
  const int32_t* enabled;   // [> max_loras] adapter_enabled
  int max_loras;
};

template <typename Id, bool LORA = false>
__device__ __forceinline__ void counting_sort_body(
    const Id* __restrict__ ids, int64_t numel, int64_t id_bound,
    const int32_t* __restrict__ map, int num_keys, int block_size,
    int32_t* __restrict__ sorted_ids, int64_t max_padded,
    int32_t* __restrict__ expert_ids, int64_t max_blocks,
    int32_t* __restrict__ ntp, int32_t* __restrict__ inv_pos,
    int32_t* __restrict__ counts_out, int32_t* __restrict__ cum_out,
    int32_t pad_value, LoraSel lora, KeyXform xf) {
  __shared__ int s_cnt[kSortWaves][kMaxKeys];
  __shared__ int s_cum[kMaxKeys + 1];
  __shared__ int s_wave_tot[kSortWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int lora_id = 0;
  if constexpr (LORA) {
    lora_id = lora.lora_ids[blockIdx.x];  // uniform
    if (lora_id < 0 || lora_id >= lora.max_loras || lora.enabled[lora_id] == 0) return;
    sorted_ids += static_cast<int64_t>(lora_id) * max_padded;
    expert_ids += static_cast<int64_t>(lora_id) * max_blocks;
    ntp += lora_id;
  }
  // the slot's key, or kInvalidKey (bad or unmapped id, another adapter)
  auto key_of = [&](int64_t i) -> uint32_t {
    const uint32_t key = load_key(ids, i, id_bound, map, num_keys, xf);
    if constexpr (LORA) {
      if (lora.tok_lora[i / lora.topk] != lora_id) return kInvalidKey;
    }
    return key;
  };

  for (int i = tid; i < kSortWaves * kMaxKeys; i += kSortThreads)
    (&s_cnt[0][0])[i] = 0;
  __syncthreads();

  const int64_t chunk = ((numel + kSortWaves - 1) / kSortWaves + 63) / 64 * 64;
  const int64_t lo = wave * chunk;
  const int64_t hi = lo + chunk < numel ? lo + chunk : numel;
  const int steps = static_cast<int>(chunk / 64);

  // phase 1: per-chunk counts
  for (int s = 0; s < steps; ++s) {
    int64_t i = lo + static_cast<int64_t>(s) * 64 + lane;
    if (i < hi) {
      uint32_t key = key_of(i);
      if (key != kInvalidKey) atomicAdd(&s_cnt[wave][key], 1);
    }
  }
  __syncthreads();

  // phase 2: per-expert totals, chunk-exclusive offsets, padded scan
  int total_e = 0;
  if (tid < num_keys) {
    for (int w = 0; w < kSortWaves; ++w) {
      int c = s_cnt[w][tid];
      s_cnt[w][tid] = total_e;
      total_e += c;
    }
  }
  const int padded = (total_e + block_size - 1) / block_size * block_size;
  int total_padded = 0;
  const int start = block_exclusive_scan(tid < num_keys ? padded : 0,
                                         s_wave_tot, total_padded);
  if (tid < num_keys) {
    s_cum[tid] = start;
    for (int w = 0; w < kSortWaves; ++w) s_cnt[w][tid] += start;
    if (counts_out) counts_out[tid] = total_e;
    if (cum_out) cum_out[tid] = start;
  }
  if (tid == 0) {
    s_cum[num_keys] = total_padded;
    if (ntp) ntp[0] = total_padded;
    if (cum_out) cum_out[num_keys] = total_padded;
  }
  __syncthreads();

  // padding slots inside each expert's range and the tail
  if (sorted_ids) {
    if (tid < num_keys) {
      for (int p = start + total_e; p < start + padded && p < max_padded; ++p)
        sorted_ids[p] = pad_value;
    }
    if (!xf.keep_tail)
      for (int64_t p = total_padded + tid; p < max_padded; p += kSortThreads)
        sorted_ids[p] = pad_value;
  }
  // expert id of every block (binary search over the padded prefix)
  if (expert_ids) {
    const int nblk = total_padded / block_size;
    for (int64_t b = tid; b < max_blocks; b += kSortThreads) {
      int e = 0;
      if (b < nblk) {
        int lo_e = 0, hi_e = num_keys - 1;
        const int p = static_cast<int>(b) * block_size;
        while (lo_e < hi_e) {  // last e with s_cum[e] <= p
          int mid = (lo_e + hi_e + 1) >> 1;
          if (s_cum[mid] <= p) lo_e = mid; else hi_e = mid - 1;
        }
        e = lo_e;
      }
      expert_ids[b] = b < nblk ? e : (LORA ? -1 : 0);
    }
  }

  // phase 3: stable scatter
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int s = 0; s < steps; ++s) {
    int64_t i = lo + static_cast<int64_t>(s) * 64 + lane;
    uint32_t key = kInvalidKey;
    if (i < hi) key = key_of(i);
    unsigned long long same = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      unsigned long long bb = __ballot((key >> b) & 1u);
      same &= ((key >> b) & 1u) ? bb : ~bb;
    }
    const int rank = __popcll(same & below);
    const int cnt = __popcll(same);
    int pos = -1;
    if (key != kInvalidKey) {
      pos = s_cnt[wave][key] + rank;
      if (sorted_ids && pos < max_padded) sorted_ids[pos] = static_cast<int32_t>(i);
    }
    if (inv_pos && i < hi) inv_pos[inv_index(i, xf)] = pos;
    __syncthreads();
    if (key != kInvalidKey && rank == 0) s_cnt[wave][key] += cnt;
    __syncthreads();
  }
}

template <typename Id, bool LORA = false>
__global__ __launch_bounds__(kSortThreads) void counting_sort_kernel(
    const Id* __restrict__ ids, int64_t numel, int64_t id_bound,
    const int32_t* __restrict__ map, int num_keys, int block_size,
    int32_t* __restrict__ sorted_ids, int64_t max_padded,
    int32_t* __restrict__ expert_ids, int64_t max_blocks,
    int32_t* __restrict__ ntp, int32_t* __restrict__ inv_pos,
    int32_t* __restrict__ counts_out, int32_t* __restrict__ cum_out,
    int32_t pad_value, LoraSel lora = {}, KeyXform xf = {}) {
  counting_sort_body<Id, LORA>(ids, numel, id_bound, map, num_keys, block_size, sorted_ids,
                               max_padded, expert_ids, max_blocks, ntp, inv_pos, counts_out,
                               cum_out, pad_value, lora, xf);
}

// The fused layer's first launch at small token counts: workgroup 0 runs the
// one-workgroup sort, workgroups 1.. quantise the activations to e4m3 with one
// fp32 scale per 1 x 128 block (fp8_quant_block8 in common.h, the arithmetic
// of per_token_group_fp8_quant), the two jobs being independent.
template <typename Id, bool F16>
__global__ __launch_bounds__(kSortThreads) void sort_quant_kernel(
    const Id* __restrict__ ids, int64_t numel, int64_t id_bound,
    const int32_t* __restrict__ map, int num_keys, int block_size,
    int32_t* __restrict__ sorted_ids, int64_t max_padded,
    int32_t* __restrict__ expert_ids, int64_t max_blocks,
    int32_t* __restrict__ ntp, int32_t* __restrict__ inv_pos,
    int32_t* __restrict__ cum_out, int32_t pad_value, const uint16_t* __restrict__ x,
    uint8_t* __restrict__ xq, float* __restrict__ xs, int64_t chunks) {
  if (blockIdx.x == 0) {
    counting_sort_body<Id, false>(ids, numel, id_bound, map, num_keys, block_size, sorted_ids,
                                  max_padded, expert_ids, max_blocks, ntp, inv_pos, nullptr,
                                  cum_out, pad_value, LoraSel{}, KeyXform{});
    return;
  }
  fp8_quant_block8<F16>(x, xq, xs, (static_cast<int64_t>(blockIdx.x) - 1) * kSortThreads +
                                       threadIdx.x, chunks);
}

// ---------------------------------------------------------------------------
// Multi-workgroup sort.  Chunk c holds ids [c*chunk, (c+1)*chunk); chunk is a
// multiple of 256 so each of a chunk's 4 waves owns a contiguous multiple of
// 64 ids.  "chunk order, wave order, rank inside the 64-id step" is flat
// order, as in the one-workgroup kernel.
constexpr int kOneBlockMax = 4096;
constexpr int kChunkIds = 1024;
constexpr int kMaxChunks = 1024;

inline int64_t sort_chunk(int64_t numel) {
  int64_t c = cdiv(numel, kChunkIds);
  if (c > kMaxChunks) c = kMaxChunks;
  return cdiv(cdiv(numel, c), 256) * 256;
}

// per-chunk expert counts: cnt[c][e]
template <typename Id>
__global__ __launch_bounds__(256) void chunk_count_kernel(
    const Id* __restrict__ ids, int64_t numel, int64_t id_bound,
    const int32_t* __restrict__ map, int num_keys, int64_t chunk,
    int32_t* __restrict__ cnt, KeyXform xf) {
  __shared__ int s[kMaxKeys];
  for (int e = threadIdx.x; e < num_keys; e += 256) s[e] = 0;
  __syncthreads();
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t hi = lo + chunk < numel ? lo + chunk : numel;
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
    const uint32_t key = load_key(ids, i, id_bound, map, num_keys, xf);
    if (key != kInvalidKey) atomicAdd(&s[key], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_keys; e += 256)
    cnt[static_cast<int64_t>(blockIdx.x) * num_keys + e] = s[e];
}

// cnt[c][e] -> ids of expert e in chunks before c; cum[e] = padded start of
// expert e (cum[num_keys] = total padded), tot[e] = its id count.  The
// chunk counts are read 8 at a time so the loads overlap.
__global__ __launch_bounds__(kSortThreads) void chunk_scan_kernel(
    int32_t* __restrict__ cnt, int nchunks, int num_keys, int block_size,
    int32_t* __restrict__ cum, int32_t* __restrict__ tot,
    int32_t* __restrict__ ntp, int32_t* __restrict__ counts_out,
    int32_t* __restrict__ cum_out) {
  __shared__ int s_wave_tot[kSortWaves];
  const int tid = threadIdx.x;
  int total_e = 0;
  if (tid < num_keys) {
    for (int c0 = 0; c0 < nchunks; c0 += 8) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = c0 + u < nchunks ? cnt[static_cast<int64_t>(c0 + u) * num_keys + tid] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (c0 + u < nchunks) cnt[static_cast<int64_t>(c0 + u) * num_keys + tid] = total_e;
        total_e += v[u];
      }
    }
  }
  const int padded = (total_e + block_size - 1) / block_size * block_size;
  int total_padded = 0;
  const int start = block_exclusive_scan(tid < num_keys ? padded : 0, s_wave_tot,
                                         total_padded);
  if (tid < num_keys) {
    cum[tid] = start;
    tot[tid] = total_e;
    if (counts_out) counts_out[tid] = total_e;
    if (cum_out) cum_out[tid] = start;
  }
  if (tid == 0) {
    cum[num_keys] = total_padded;
    if (ntp) ntp[0] = total_padded;
    if (cum_out) cum_out[num_keys] = total_padded;
  }
}

// Stable scatter of chunk blockIdx.x, then (grid-strided) the padding slots,
// the tail past the padded total and the expert id of every block.
template <typename Id>
__global__ __launch_bounds__(256) void chunk_scatter_kernel(
    const Id* __restrict__ ids, int64_t numel, int64_t id_bound,
    const int32_t* __restrict__ map, int num_keys, int64_t chunk,
    const int32_t* __restrict__ off, const int32_t* __restrict__ cum,
    const int32_t* __restrict__ tot, int block_size,
    int32_t* __restrict__ sorted_ids, int64_t max_padded,
    int32_t* __restrict__ expert_ids, int64_t max_blocks,
    int32_t* __restrict__ inv_pos, int32_t pad_value, KeyXform xf) {
  __shared__ int s_cnt[4][kMaxKeys];
  __shared__ int s_cum[kMaxKeys + 1];
  __shared__ int s_tot[kMaxKeys];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 4 * kMaxKeys; i += 256) (&s_cnt[0][0])[i] = 0;
  for (int e = tid; e <= num_keys; e += 256) {
    s_cum[e] = cum[e];
    if (e < num_keys) s_tot[e] = tot[e];
  }
  __syncthreads();

  const int64_t sub = chunk / 4;
  const int64_t clo = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t lo = clo + wave * sub;
  const int64_t hi0 = lo + sub < numel ? lo + sub : numel;
  const int64_t hi = hi0 > lo ? hi0 : lo;
  const int steps = static_cast<int>(sub / 64);
  for (int s = 0; s < steps; ++s) {
    const int64_t i = lo + static_cast<int64_t>(s) * 64 + lane;
    if (i < hi) {
      const uint32_t key = load_key(ids, i, id_bound, map, num_keys, xf);
      if (key != kInvalidKey) atomicAdd(&s_cnt[wave][key], 1);
    }
  }
  __syncthreads();
  // wave w's first slot for expert e: expert start + ids in earlier chunks
  // + ids of waves < w
  for (int e = tid; e < num_keys; e += 256) {
    int run = s_cum[e] + off[static_cast<int64_t>(blockIdx.x) * num_keys + e];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int c = s_cnt[w][e];
      s_cnt[w][e] = run;
      run += c;
    }
  }
  __syncthreads();
  // each wave ranks its own 64-id steps; its counters are its own, and the
  // LDS accesses of one wave execute in program order
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int s = 0; s < steps; ++s) {
    const int64_t i = lo + static_cast<int64_t>(s) * 64 + lane;
    uint32_t key = kInvalidKey;
    if (i < hi) key = load_key(ids, i, id_bound, map, num_keys, xf);
    unsigned long long same = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      const unsigned long long bb = __ballot((key >> b) & 1u);
      same &= ((key >> b) & 1u) ? bb : ~bb;
    }
    const int rank = __popcll(same & below);
    const int cnt = __popcll(same);
    int pos = -1;
    if (key != kInvalidKey) {
      pos = s_cnt[wave][key] + rank;
      if (sorted_ids && pos < max_padded) sorted_ids[pos] = static_cast<int32_t>(i);
    }
    if (inv_pos && i < hi) inv_pos[inv_index(i, xf)] = pos;
    if (key != kInvalidKey && rank == 0) s_cnt[wave][key] += cnt;
  }

  // padding slots of every expert and the tail, expert id of every block
  const int total_padded = s_cum[num_keys];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  auto expert_at = [&](int p) -> int {  // last e with s_cum[e] <= p
    int lo_e = 0, hi_e = num_keys - 1;
    while (lo_e < hi_e) {
      const int mid = (lo_e + hi_e + 1) >> 1;
      if (s_cum[mid] <= p) lo_e = mid; else hi_e = mid - 1;
    }
    return lo_e;
  };
  if (sorted_ids) {
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + tid; p < max_padded; p += stride) {
      if (p >= total_padded) {
        if (!xf.keep_tail) sorted_ids[p] = pad_value;
      } else {
        const int e = expert_at(static_cast<int>(p));
        if (p - s_cum[e] >= s_tot[e]) sorted_ids[p] = pad_value;
      }
    }
  }
  if (expert_ids) {
    const int nblk = total_padded / block_size;
    for (int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + tid; b < max_blocks; b += stride)
      expert_ids[b] = b < nblk ? expert_at(static_cast<int>(b) * block_size) : 0;
  }
}

// rows_per_expert (contiguous segments) -> block-padded row list:
// row_ids[p] = first_row(e) + r for r < rows(e), else pad_value.
__global__ __launch_bounds__(kSortThreads) void segments_to_blocks_kernel(
    const int32_t* __restrict__ rows, int num_keys, int block_size,
    int32_t* __restrict__ row_ids, int64_t max_padded,
    int32_t* __restrict__ expert_ids, int64_t max_blocks,
    int32_t* __restrict__ ntp, int32_t* __restrict__ cum_out, int32_t pad_value) {
  __shared__ int s_cum[kMaxKeys + 1];
  __shared__ int s_off[kMaxKeys + 1];
  __shared__ int s_wave_tot[kSortWaves];
  const int tid = threadIdx.x;
  const int c = tid < num_keys ? rows[tid] : 0;
  const int padded = (c + block_size - 1) / block_size * block_size;
  int tp = 0, tr = 0;
  int start = block_exclusive_scan(padded, s_wave_tot, tp);
  int roff = block_exclusive_scan(c, s_wave_tot, tr);
  if (tid < num_keys) {
    s_cum[tid] = start;
    s_off[tid] = roff;
    if (cum_out) cum_out[tid] = start;
  }
  if (tid == 0) {
    s_cum[num_keys] = tp;
    s_off[num_keys] = tr;
    if (ntp) ntp[0] = tp;
    if (cum_out) cum_out[num_keys] = tp;
  }
  __syncthreads();
  for (int64_t p = tid; p < max_padded; p += kSortThreads) {
    int v = pad_value;
    if (p < tp) {
      int lo_e = 0, hi_e = num_keys - 1;
      while (lo_e < hi_e) {
        int mid = (lo_e + hi_e + 1) >> 1;
        if (s_cum[mid] <= p) lo_e = mid; else hi_e = mid - 1;
      }
      int r = static_cast<int>(p) - s_cum[lo_e];
      if (r < s_off[lo_e + 1] - s_off[lo_e]) v = s_off[lo_e] + r;
    }
    row_ids[p] = v;
  }
  const int nblk = tp / block_size;
  for (int64_t b = tid; b < max_blocks; b += kSortThreads) {
    int e = 0;
    if (b < nblk) {
      const int p = static_cast<int>(b) * block_size;
      int lo_e = 0, hi_e = num_keys - 1;
      while (lo_e < hi_e) {
        int mid = (lo_e + hi_e + 1) >> 1;
        if (s_cum[mid] <= p) lo_e = mid; else hi_e = mid - 1;
      }
      e = lo_e;
    }
    expert_ids[b] = e;
  }
}

// Row copies of remap_hidden_states: remapped[perm[i]] = hidden[i / topk].
__global__ __launch_bounds__(256) void remap_copy_kernel(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
    int64_t row_bytes, const int32_t* __restrict__ perm, int topk,
    int64_t slots) {
  const int64_t i = blockIdx.x;
  if (i >= slots) return;
  const int p = perm[i];
  if (p < 0) return;
  const uint8_t* s = src + (i / topk) * row_bytes;
  uint8_t* d = dst + static_cast<int64_t>(p) * row_bytes;
  if ((row_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(src) |
                                 reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
    const int64_t n = row_bytes >> 4;
    for (int64_t j = threadIdx.x; j < n; j += 256)
      reinterpret_cast<uint4*>(d)[j] = reinterpret_cast<const uint4*>(s)[j];
  } else {
    for (int64_t j = threadIdx.x; j < row_bytes; j += 256) d[j] = s[j];
  }
}

__global__ void init_expert_map_kernel(int32_t* map, int num_experts,
                                       int ep_rank, int ep_size) {
  int g = blockIdx.x * blockDim.x + threadIdx.x;
  int total = num_experts * ep_size;
  if (g >= total) return;
  int lo = ep_rank * num_experts;
  map[g] = (g >= lo && g < lo + num_experts) ? g - lo : -1;
}

template <typename Id>
void launch_sort(const void* ids, int64_t numel, int64_t id_bound,
                 const int32_t* map, int num_keys, int bs, int32_t* sorted,
                 int64_t max_padded, int32_t* eids, int64_t max_blocks,
                 int32_t* ntp, int32_t* inv, int32_t* counts, int32_t* cum_out,
                 int32_t pad, int32_t* ws, hipStream_t st, KeyXform xf) {
  const Id* id = static_cast<const Id*>(ids);
  if (!ws) {
    counting_sort_kernel<Id><<<1, kSortThreads, 0, st>>>(
        id, numel, id_bound, map, num_keys, bs, sorted, max_padded, eids,
        max_blocks, ntp, inv, counts, cum_out, pad, LoraSel{}, xf);
    return;
  }
  const int64_t chunk = sort_chunk(numel);
  const int nchunks = static_cast<int>(cdiv(numel, chunk));
  int32_t* cnt = ws;
  int32_t* cum = cnt + static_cast<int64_t>(nchunks) * num_keys;
  int32_t* tot = cum + num_keys + 1;
  chunk_count_kernel<Id><<<nchunks, 256, 0, st>>>(id, numel, id_bound, map,
                                                   num_keys, chunk, cnt, xf);
  chunk_scan_kernel<<<1, kSortThreads, 0, st>>>(cnt, nchunks, num_keys, bs, cum,
                                                tot, ntp, counts, cum_out);
  chunk_scatter_kernel<Id><<<nchunks, 256, 0, st>>>(
      id, numel, id_bound, map, num_keys, chunk, cnt, cum, tot, bs, sorted,
      max_padded, eids, max_blocks, inv, pad, xf);
}

}  // namespace

// Workspace of the multi-workgroup sort (0: the one-workgroup kernel runs).
size_t counting_sort_ws_bytes(int64_t numel, int64_t num_keys) {
  if (numel <= kOneBlockMax || num_keys <= 0) return 0;
  const int64_t nchunks = cdiv(numel, sort_chunk(numel));
  return static_cast<size_t>(nchunks * num_keys + 2 * num_keys + 1) * sizeof(int32_t);
}

// Shared by the fused layer and the alignment entry points.  ws: at least
// counting_sort_ws_bytes(numel, num_keys) bytes, or null (one workgroup).
int run_counting_sort(const void* ids, int ids_dtype, int64_t numel,
                      int64_t id_bound, const int32_t* map, int64_t num_keys,
                      int64_t bs, int32_t* sorted, int64_t max_padded,
                      int32_t* eids, int64_t max_blocks, int32_t* ntp,
                      int32_t* inv, int32_t* counts, int32_t pad,
                      void* ws, size_t ws_bytes, hipStream_t st, int32_t* cum_out,
                      int64_t id_start, int dedupe_k, int64_t inv_rows) {
  // the prologue's sort (dedupe_k > 0) writes only the sorted slots
  const KeyXform xf{id_start, dedupe_k, dedupe_k > 0, dedupe_k > 0 ? inv_rows : 0};
  MI_ARG(num_keys > 0 && num_keys <= kMaxKeys,
         "padded_num_experts must be less than 1024");
  MI_ARG(bs > 0, "block_size must be positive");
  MI_ARG(numel >= 0 && numel < (int64_t(1) << 31), "too many topk_ids");
  const size_t need = counting_sort_ws_bytes(numel, num_keys);
  int32_t* w = (need > 0 && ws && ws_bytes >= need) ? static_cast<int32_t*>(ws) : nullptr;
  switch (ids_dtype) {
    case MI355MOE_I32:
      launch_sort<int32_t>(ids, numel, id_bound, map, (int)num_keys, (int)bs, sorted, max_padded, eids, max_blocks, ntp, inv, counts, cum_out, pad, w, st, xf);
      break;
    case MI355MOE_I64:
      launch_sort<int64_t>(ids, numel, id_bound, map, (int)num_keys, (int)bs, sorted, max_padded, eids, max_blocks, ntp, inv, counts, cum_out, pad, w, st, xf);
      break;
    case MI355MOE_U32:
      launch_sort<uint32_t>(ids, numel, id_bound, map, (int)num_keys, (int)bs, sorted, max_padded, eids, max_blocks, ntp, inv, counts, cum_out, pad, w, st, xf);
      break;
    default:
      return set_error(MI355MOE_ERR_INVALID, "topk_ids must be int32, int64 or uint32");
  }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

// run_counting_sort's one-workgroup form plus the e4m3 1 x 128 quantisation
// of x [rows, cols] (16-bit, 16-byte aligned, cols % 128 == 0) in the same
// launch.  Returns 1 (nothing launched) when the sort needs more than one
// workgroup; the caller then runs the two steps separately.
int run_sort_quant_fp8(const void* ids, int ids_dtype, int64_t numel, int64_t id_bound,
                       const int32_t* map, int64_t num_keys, int64_t bs, int32_t* sorted,
                       int64_t max_padded, int32_t* eids, int64_t max_blocks, int32_t* ntp,
                       int32_t* inv, int32_t pad, int32_t* cum_out, const void* x, bool f16,
                       uint8_t* xq, float* xs, int64_t rows, int64_t cols, hipStream_t st) {
  if (numel > kOneBlockMax || num_keys <= 0 || num_keys > kMaxKeys || bs <= 0 ||
      cols % 128 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) != 0 ||
      (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64))
    return 1;
  const int64_t chunks = rows * cols / 8;
  const dim3 grid(static_cast<unsigned>(1 + cdiv(chunks, kSortThreads)));
  auto go = [&](auto id_tag, auto f16_tag) {
    using Id = decltype(id_tag);
    sort_quant_kernel<Id, decltype(f16_tag)::value><<<grid, kSortThreads, 0, st>>>(
        static_cast<const Id*>(ids), numel, id_bound, map, static_cast<int>(num_keys),
        static_cast<int>(bs), sorted, max_padded, eids, max_blocks, ntp, inv, cum_out, pad,
        static_cast<const uint16_t*>(x), xq, xs, chunks);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (ids_dtype == MI355MOE_I32) { if (f16) go(int32_t{}, T_{}); else go(int32_t{}, F_{}); }
  else { if (f16) go(int64_t{}, T_{}); else go(int64_t{}, F_{}); }
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

int run_segments_to_blocks(const int32_t* rows, int64_t num_keys, int64_t bs,
                           int32_t* row_ids, int64_t max_padded,
                           int32_t* eids, int64_t max_blocks, int32_t* ntp,
                           int32_t pad, hipStream_t st, int32_t* cum_out) {
  MI_ARG(num_keys > 0 && num_keys <= kMaxKeys, "num_experts must be in [1, 1024]");
  hipLaunchKernelGGL(segments_to_blocks_kernel, dim3(1), dim3(kSortThreads), 0,
                     st, rows, (int)num_keys, (int)bs, row_ids, max_padded,
                     eids, max_blocks, ntp, cum_out, pad);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

}  // namespace mi355

using namespace mi355;

extern "C" size_t mi355moe_moe_align_block_size_workspace_size(int64_t numel,
                                                               int64_t num_experts) {
  return counting_sort_ws_bytes(numel, num_experts);
}

extern "C" int mi355moe_moe_align_block_size(
    const void* topk_ids, int ids_dtype, int64_t numel, int64_t num_experts,
    int64_t block_size, int32_t* sorted_token_ids, int64_t max_num_tokens_padded,
    int32_t* expert_ids, int64_t max_num_m_blocks, int32_t* ntp,
    const int32_t* expert_map, void* workspace, size_t workspace_bytes,
    void* stream) {
  MI_ARG(num_experts > 0, "num_experts must be positive");
  MI_ARG((num_experts + 31) / 32 * 32 < 1024,
         "padded_num_experts must be less than 1024");
  return run_counting_sort(topk_ids, ids_dtype, numel, num_experts, expert_map,
                           num_experts, block_size, sorted_token_ids,
                           max_num_tokens_padded, expert_ids, max_num_m_blocks,
                           ntp, nullptr, nullptr, static_cast<int32_t>(numel),
                           workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                           nullptr);
}

extern "C" int mi355moe_moe_lora_align_block_size(
    const void* topk_ids, int ids_dtype, int64_t num_tokens, int64_t topk,
    const int32_t* token_lora_mapping, int64_t num_experts, int64_t block_size,
    int64_t max_loras, int64_t max_num_tokens_padded, int64_t max_num_m_blocks,
    int32_t* sorted_token_ids, int32_t* expert_ids, int32_t* num_tokens_post_pad,
    const int32_t* adapter_enabled, const int32_t* lora_ids, int64_t num_lora_slots,
    const int32_t* expert_map, void* stream) {
  MI_ARG(block_size > 0, "block_size should be greater than 0. ");
  MI_ARG((num_experts + 31) / 32 * 32 < 1024, "padded_num_experts must be less than 1024");
  MI_ARG(num_tokens >= 0 && topk > 0 && max_loras >= 0 && num_lora_slots >= 0,
         "invalid LoRA alignment sizes");
  MI_ARG(ids_dtype == MI355MOE_I32 || ids_dtype == MI355MOE_I64,
         "topk_ids must be int32 or int64");
  if (num_lora_slots == 0 || max_loras == 0) return MI355MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const LoraSel sel{token_lora_mapping, static_cast<int>(topk), lora_ids, adapter_enabled,
                    static_cast<int>(max_loras)};
  const int64_t numel = num_tokens * topk;
  dim3 grid(static_cast<unsigned>(num_lora_slots));
  if (ids_dtype == MI355MOE_I32)
    counting_sort_kernel<int32_t, true><<<grid, dim3(kSortThreads), 0, st>>>(
        static_cast<const int32_t*>(topk_ids), numel, num_experts, expert_map,
        static_cast<int>(num_experts), static_cast<int>(block_size), sorted_token_ids,
        max_num_tokens_padded, expert_ids, max_num_m_blocks, num_tokens_post_pad, nullptr,
        nullptr, nullptr, static_cast<int32_t>(numel), sel);
  else
    counting_sort_kernel<int64_t, true><<<grid, dim3(kSortThreads), 0, st>>>(
        static_cast<const int64_t*>(topk_ids), numel, num_experts, expert_map,
        static_cast<int>(num_experts), static_cast<int>(block_size), sorted_token_ids,
        max_num_tokens_padded, expert_ids, max_num_m_blocks, num_tokens_post_pad, nullptr,
        nullptr, nullptr, static_cast<int32_t>(numel), sel);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}

extern "C" size_t mi355moe_remap_hidden_states_workspace_size(int64_t num_tokens,
                                                              int64_t topk,
                                                              int64_t local_experts) {
  return counting_sort_ws_bytes(num_tokens * topk, local_experts);
}

extern "C" int mi355moe_remap_hidden_states(
    const void* hidden, int64_t elem_bytes, const void* hscales,
    int64_t scale_cols, int64_t scale_bytes, void* remapped,
    void* remapped_scales, const int32_t* expert_map, int32_t* rows_per_expert,
    int32_t* perm, const void* topk_ids, int ids_dtype, int64_t T, int64_t H,
    int64_t k, int64_t total_experts, int64_t local_experts, void* workspace,
    size_t workspace_bytes, void* stream) {
  MI_ARG(local_experts > 0 && local_experts <= 1024,
         "local experts number must be in [1, 1024]");
  MI_ARG(k > 0, "Unsupported TopK value");
  MI_ARG(elem_bytes > 0 && H > 0, "invalid hidden_states");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t slots = T * k;
  if (slots == 0) return MI355MOE_OK;
  int rc = run_counting_sort(topk_ids, ids_dtype, slots, total_experts,
                             expert_map, local_experts, 1, nullptr, 0, nullptr,
                             0, nullptr, perm, rows_per_expert, 0, workspace,
                             workspace_bytes, st, nullptr);
  if (rc) return rc;
  hipLaunchKernelGGL(remap_copy_kernel, dim3(static_cast<unsigned>(slots)),
                     dim3(256), 0, st, static_cast<const uint8_t*>(hidden),
                     static_cast<uint8_t*>(remapped), H * elem_bytes, perm,
                     (int)k, slots);
  MI_LAUNCH_CHECK();
  if (hscales && remapped_scales) {
    hipLaunchKernelGGL(remap_copy_kernel, dim3(static_cast<unsigned>(slots)),
                       dim3(256), 0, st, static_cast<const uint8_t*>(hscales),
                       static_cast<uint8_t*>(remapped_scales),
                       scale_cols * scale_bytes, perm, (int)k, slots);
    MI_LAUNCH_CHECK();
  }
  return MI355MOE_OK;
}

extern "C" int mi355moe_init_expert_map(int32_t* map, int64_t num_experts,
                                        int64_t ep_rank, int64_t ep_size,
                                        void* stream) {
  MI_ARG(num_experts > 0 && ep_size > 0 && ep_rank >= 0 && ep_rank < ep_size,
         "invalid expert-parallel configuration");
  int64_t total = num_experts * ep_size;
  hipLaunchKernelGGL(init_expert_map_kernel,
                     dim3(static_cast<unsigned>(cdiv(total, 256))), dim3(256),
                     0, static_cast<hipStream_t>(stream), map, (int)num_experts,
                     (int)ep_rank, (int)ep_size);
  MI_LAUNCH_CHECK();
  return MI355MOE_OK;
}
