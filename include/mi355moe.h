/*
 * mi355moe.h — C ABI of the MI355X (gfx950) fused Mixture-of-Experts library.
 *
 * Plain pointers, sizes and enums only; no torch types.  Every function is
 * asynchronous on the given HIP stream (`stream` is a hipStream_t, NULL = the
 * null stream), never synchronises the host, and returns MI355MOE_OK (0) or a
 * negative mi355moe_status; mi355moe_last_error() then returns a
 * thread-local message whose substrings mirror the reference's TORCH_CHECK
 * messages.  Device pointers are caller-allocated.  Functions that need
 * scratch memory take a caller-provided workspace sized by the matching
 * *_workspace_size query.
 *
 * Each entry point cites the reference interface it replaces (paths relative
 * to the vllm-xpu-kernels repository root).
 */
#ifndef MI355MOE_H_
#define MI355MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MI355MOE_OK = 0,
  MI355MOE_ERR_INVALID = -1,     /* bad argument (shape, dtype, size)       */
  MI355MOE_ERR_UNSUPPORTED = -2, /* valid but not implemented combination   */
  MI355MOE_ERR_HIP = -3,         /* HIP runtime / launch failure            */
  MI355MOE_ERR_WORKSPACE = -4    /* workspace too small                     */
} mi355moe_status;

typedef enum {
  MI355MOE_F32 = 0,
  MI355MOE_BF16 = 1,
  MI355MOE_F16 = 2,
  MI355MOE_I32 = 3,
  MI355MOE_I64 = 4,
  MI355MOE_U32 = 5,
  MI355MOE_FP8E4M3 = 6, /* OCP float8_e4m3fn                              */
  MI355MOE_U8 = 7,      /* raw bytes: packed e2m1 pairs or e8m0 scales    */
  MI355MOE_I16 = 8,
  MI355MOE_FP8E5M2 = 9, /* OCP float8_e5m2                                */
  MI355MOE_I8 = 10
} mi355moe_dtype;

/* Weight recipes of the grouped GEMM / fused layer
 * (vllm_xpu_kernels/fused_moe_interface.py:33-45). */
typedef enum {
  MI355MOE_RECIPE_BF16 = 0,     /* 16-bit weights and activations of one
                                   type, bf16 or fp16                     */
  MI355MOE_RECIPE_FP8BLOCK = 1, /* e4m3 weights, fp32 128x128 block scales;
                                   activations quantised 1x128 e4m3       */
  MI355MOE_RECIPE_MXFP4 = 2,    /* e2m1 weights packed along K, e8m0 scale
                                   per 32 along K; bf16 or fp16
                                   activations (weights dequantised to
                                   their type)                            */
  MI355MOE_RECIPE_INT4 = 3,     /* signed int4 weights (two's complement,
                                   the even K value in the low nibble)
                                   packed along K [E, N, K/2], scales
                                   [E, N, K/group] in the activations'
                                   16-bit type, group 32/64/128/256:
                                   w = T(v * scale) (w4a16); K-blocked:
                                   weights [E, K/32, N, 16 bytes], scales
                                   [E, K/group, N]                        */
  MI355MOE_RECIPE_MXFP8 = 4,    /* e4m3 weights [E, N, K] with an e8m0 scale
                                   (u8) per 32 along K, [E, N, K/32];
                                   activations quantised per 32 to e4m3
                                   with ue8m0 scales (the reference's
                                   _quant_mxfp8_act_xpu), both scales in
                                   the scaled MFMA (vllm_xpu_kernels/
                                   moe_utils.py:76-104)                   */
  MI355MOE_RECIPE_FP8 = 5,      /* per-expert fp8 (the reference's recipe
                                   "fp8", vllm_xpu_kernels/
                                   fused_moe_interface.py:42-59, w8a16):
                                   e4m3 weights [E, N, K] (K-blocked
                                   [E, K/32, N, 32]) with an f32 scale per
                                   expert ([E] in w13_scale / w2_scale) and
                                   16-bit activations; each weight is
                                   converted exactly to the activations'
                                   type as it is loaded and the expert's
                                   scale multiplies the accumulators (every
                                   layer size; the prefill kernel needs the
                                   K-blocked layout).  Hidden or
                                   intermediate sizes not % 32 return
                                   MI355MOE_ERR_UNSUPPORTED (run them as
                                   RECIPE_BF16 on exact 16-bit copies)    */
  MI355MOE_RECIPE_FP8E5M2 = 6   /* as RECIPE_FP8 with e5m2 weights        */
} mi355moe_recipe;

typedef enum {
  MI355MOE_ACT_SILU = 0,       /* silu(x[:, :I]) * x[:, I:]                */
  MI355MOE_ACT_SWIGLUOAI = 1,  /* interleaved gate/up, alpha 1.702, lim 7  */
  MI355MOE_ACT_GELU = 2,       /* gelu(x[:, :I]) * x[:, I:] (erf form)     */
  MI355MOE_ACT_GELU_TANH = 3,  /* gelu_tanh(x[:, :I]) * x[:, I:]           */
  MI355MOE_ACT_SWIGLUSTEP = 4, /* min(silu(g), lim) * clamp(u, +-lim)      */
  MI355MOE_ACT_RELU2 = 5       /* relu(x)^2 over all 2I columns, no gate:
                                  w2 then has K = 2I (relu2_no_mul)        */
} mi355moe_activation;

/* Layout of the fused layer's weights.  NK is the canonical [E, N, K] (K
 * contiguous).  KBLOCK is the same data K-blocked, [E, K/B, N, B] with
 * B = 32 values (64 bytes) for 16-bit, B = 128 (128 bytes) for e4m3 and
 * B = 32 (16 bytes) for e2m1 weights, whose e8m0 scales are then [E, K/32, N]:
 * the K-slices of consecutive weight rows are contiguous, so a kernel that
 * streams a 16-row weight fragment of one K stage reads one run of 0.25-2 KiB
 * instead of 16 short runs.  KBLOCK needs hidden and intermediate sizes
 * % B == 0 and, for fp8block, of at most 8192; mi355moe_pack_weights_kblock
 * and mi355moe_pack_scales_kblock make it. */
typedef enum {
  MI355MOE_WLAYOUT_NK = 0,
  MI355MOE_WLAYOUT_KBLOCK = 1
} mi355moe_weight_layout;

const char* mi355moe_last_error(void);
int mi355moe_version(void);

/* ---------------------------------------------------------------- routing */

/* Replaces torch.ops._moe_C.topk_softmax (csrc/moe/torch_bindings.cpp:59-63,
 * csrc/moe/topk.cpp:848-898).  gating [T,E] (f32/bf16/f16) -> weights f32
 * [T,k], ids [T,k] (i32/i64/u32), token_expert_indices i32 [T,k].
 * bias: optional f32 [E] added for selection only. */
int mi355moe_topk_softmax(float* topk_weights, void* topk_indices,
                          int indices_dtype, int32_t* token_expert_indices,
                          const void* gating_output, int gating_dtype,
                          int64_t num_tokens, int64_t num_experts,
                          int64_t topk, int renormalize, const float* bias,
                          void* stream);

/* Replaces torch.ops._moe_C.topk_sigmoid (csrc/moe/torch_bindings.cpp:65-69,
 * csrc/moe/topk.cpp:900-952). */
int mi355moe_topk_sigmoid(float* topk_weights, void* topk_indices,
                          int indices_dtype, int32_t* token_expert_indices,
                          const void* gating_output, int gating_dtype,
                          int64_t num_tokens, int64_t num_experts,
                          int64_t topk, int renormalize, const float* bias,
                          float routed_scaling_factor, void* stream);

/* Replaces torch.ops._moe_C.topk_softplus_sqrt (csrc/moe/torch_bindings.cpp:
 * 70-76, csrc/moe/topk_softplus_sqrt_kernels.cpp:225-416, 596-772).  Scores
 * sqrt(softplus(x)) in fp32 (softplus(x) = x above 20, else log(1 + e^x));
 * top-k of score + correction_bias (ties to the lower id), each weight the
 * chosen (score + bias) - bias; weights times routed_scaling_factor, divided
 * by their sum when renormalize.  With tid2eid (and input_ids, both of the
 * indices' dtype) the experts are tid2eid[input_ids[t] * topk + j] and the
 * weights their scores (non-finite -> 0).  num_experts one of 1..512 (powers
 * of two), 192, 320, 384, 448, 576. */
int mi355moe_topk_softplus_sqrt(float* topk_weights, void* topk_indices, int indices_dtype,
                                int32_t* token_expert_indices, const void* gating_output,
                                int gating_dtype, int64_t num_tokens, int64_t num_experts,
                                int64_t topk, int renormalize, float routed_scaling_factor,
                                const float* correction_bias, const void* input_ids,
                                const void* tid2eid, void* stream);

/* Replaces torch.ops._moe_C.grouped_topk (csrc/moe/torch_bindings.cpp:53-57,
 * csrc/moe/grouped_topk.cpp:782-876).  scores / scores_with_bias [T,E] in
 * `dtype` (f32/bf16/f16) -> values [T,k] (same dtype), ids i32 [T,k]. */
int mi355moe_grouped_topk(void* topk_values, int32_t* topk_indices,
                          const void* scores, const void* scores_with_bias,
                          int dtype, int64_t num_tokens, int64_t num_experts,
                          int64_t n_group, int64_t topk_group, int64_t topk,
                          int renormalize, float routed_scaling_factor,
                          void* stream);

/* Replaces the reference's fused_grouped_topk with scoring "sigmoid"
 * (tests/ops/grouped_topk_op.py:67-92: torch sigmoid, + the correction
 * bias, then torch.ops._moe_C.grouped_topk) in one launch: gating_output
 * [T,E] in `dtype` (f32/bf16/f16), bias f32 [E] or null; the kernel forms
 * scores = T(sigmoid(x)) and scores_with_bias = T(scores + bias) per element
 * (T: the input dtype) and selects as mi355moe_grouped_topk. */
int mi355moe_fused_grouped_topk(void* topk_values, int32_t* topk_indices,
                                const void* gating_output, const float* bias, int dtype,
                                int64_t num_tokens, int64_t num_experts, int64_t n_group,
                                int64_t topk_group, int64_t topk, int renormalize,
                                float routed_scaling_factor, void* stream);

/* ----------------------------------------------------- alignment / permute */

/* Replaces torch.ops._moe_C.moe_lora_align_block_size
 * (csrc/moe/torch_bindings.cpp:37-50, csrc/moe/moe_align_sum_kernels.cpp:
 * 725-1031, 1374-1520).  One stable counting sort per entry of lora_ids
 * (num_lora_slots of them, max_loras + 1 at most): adapter id = lora_ids[w];
 * -1, ids >= max_loras and adapters with adapter_enabled[id] == 0 write
 * nothing.  Otherwise only the slots of tokens with token_lora_mapping[t] ==
 * id are sorted, into sorted_token_ids[id * max_num_tokens_padded ...] (pad
 * value num_tokens * topk), expert_ids[id * max_num_m_blocks ...] (unused
 * blocks -1) and num_tokens_post_pad[id].  topk_ids [num_tokens, topk] i32 or
 * i64; the other index arrays i32; expert_map optional i32 [num_experts]. */
int mi355moe_moe_lora_align_block_size(
    const void* topk_ids, int ids_dtype, int64_t num_tokens, int64_t topk,
    const int32_t* token_lora_mapping, int64_t num_experts, int64_t block_size,
    int64_t max_loras, int64_t max_num_tokens_padded, int64_t max_num_m_blocks,
    int32_t* sorted_token_ids, int32_t* expert_ids, int32_t* num_tokens_post_pad,
    const int32_t* adapter_enabled, const int32_t* lora_ids, int64_t num_lora_slots,
    const int32_t* expert_map, void* stream);

/* Replaces torch.ops._moe_C.moe_align_block_size
 * (csrc/moe/torch_bindings.cpp:14-20, csrc/moe/moe_align_sum_kernels.cpp:
 * 1034-1181).  Deterministic: a stable counting sort (tokens of one expert
 * keep their flat order).  expert_map: optional i32 [num_experts]. */
size_t mi355moe_moe_align_block_size_workspace_size(int64_t numel,
                                                    int64_t num_experts);
int mi355moe_moe_align_block_size(const void* topk_ids, int ids_dtype,
                                  int64_t numel, int64_t num_experts,
                                  int64_t block_size,
                                  int32_t* sorted_token_ids,
                                  int64_t max_num_tokens_padded,
                                  int32_t* expert_ids,
                                  int64_t max_num_m_blocks,
                                  int32_t* num_tokens_post_pad,
                                  const int32_t* expert_map,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* fused_moe_prologue workspace: ten sections, each padded to 256 bytes, in
 * this order (the reference's, csrc/moe/fused_moe_prologue.cpp:40-102):
 *   0 permuted_row_to_unpermuted_row  i32 [N]      expanded row j*T + t
 *   1 permuted_token_selected_experts i32 [N]      expert - rank's first
 *   2 unpermuted_row_to_permuted_row  i32 [N]      -1: not routed here
 *   3 blocked_expert_counts           i32 [E*nblk] scratch
 *   4 blocked_expert_counts_cumsum    i32 [E*nblk] scratch
 *   5 blocked_row_to_unpermuted_row   i32 [E*T]    scratch
 *   6 expert_first_token_offset       i64 [E+1]
 *   7 permuted_token_final_scales     f32 [N]
 *   8 overlapped_gemm1_gemm2_inputs   [N, hidden] input elements
 *   9 permuted_act_scales             [N*hidden/block_k] scale elements
 * with N = T * k, E = num_experts_on_rank and nblk = ceil(T / b), b the
 * smallest of 32, 64, ..., 1024 with ceil(T / b) * E <= b (else 1024).
 * Rows past expert_first_token_offset[E] are not written.  Section 2 holds
 * -1 for expanded rows not routed to this rank, where the reference leaves
 * the bytes as they were. */
#define MI355MOE_PROLOGUE_SECTIONS 10

/* Byte layout of the fused_moe_prologue workspace: returns the total size
 * and, when non-null, the offset and padded size of each section
 * (offsets[10], sizes[10]); 0 for invalid sizes.  scale_bytes 0: no
 * activation scales (section 9 empty). */
size_t mi355moe_fused_moe_prologue_workspace_layout(
    int64_t num_rows, int64_t experts_per_token, int64_t hidden_size, int64_t elem_bytes,
    int64_t block_k, int64_t scale_bytes, int64_t num_experts_on_rank, size_t* offsets,
    size_t* sizes);

/* Replaces torch.ops._moe_C.fused_moe_prologue (csrc/moe/torch_bindings.cpp:
 * 83-92, csrc/moe/fused_moe_prologue.cpp:5-151, fused_moe_prologue.hpp:
 * 154-709).  input [num_rows, hidden_size] of elem_bytes (2: bf16 / fp16,
 * 1: e4m3 or packed e2m1 pairs); input_scales [num_rows, hidden_size /
 * block_k] of scale_bytes (4: f32, 1: e8m0; 0: none); token_selected_experts
 * [num_rows, experts_per_token] i64 (or i32); token_final_scales f32 of the
 * same shape (null: 1.0).  This rank owns experts [ep_rank * E, (ep_rank +
 * 1) * E) with E = num_experts_on_rank <= 1024.  Permuted rows are in expert
 * order and token order inside an expert; a token listing an expert twice
 * is routed to it once.  inter_size is accepted and unused, as in the
 * reference.  The workspace must hold the layout above. */
int mi355moe_fused_moe_prologue(
    const void* input, int64_t elem_bytes, const void* input_scales, int64_t scale_bytes,
    const void* token_selected_experts, int ids_dtype, const float* token_final_scales,
    void* workspace, size_t workspace_bytes, int64_t num_rows, int64_t hidden_size,
    int64_t inter_size, int64_t block_k, int64_t experts_per_token, int64_t ep_rank,
    int64_t ep_size, int64_t num_experts_on_rank, void* stream);

/* Replaces torch.ops._moe_C.remap_hidden_states
 * (csrc/moe/torch_bindings.cpp:99-108, csrc/moe/remap_hidden_states.cpp:
 * 418-568).  Stable order within an expert.  hidden [T,H] (elem_bytes per
 * element), optional scales [T,S] (scale_bytes per element). */
size_t mi355moe_remap_hidden_states_workspace_size(int64_t num_tokens,
                                                   int64_t topk,
                                                   int64_t local_experts);
int mi355moe_remap_hidden_states(const void* hidden_states, int64_t elem_bytes,
                                 const void* hidden_scales, int64_t scale_cols,
                                 int64_t scale_bytes, void* remapped,
                                 void* remapped_scales,
                                 const int32_t* expert_map,
                                 int32_t* rows_per_expert,
                                 int32_t* unpermuted_row_to_permuted_row,
                                 const void* topk_ids, int ids_dtype,
                                 int64_t num_tokens, int64_t hidden_cols,
                                 int64_t topk, int64_t total_experts,
                                 int64_t local_experts, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Replaces torch.ops._moe_C.init_expert_map (csrc/moe/torch_bindings.cpp:
 * 93-98, csrc/moe/init_expert_map.cpp:9-95). */
int mi355moe_init_expert_map(int32_t* expert_map, int64_t num_experts,
                             int64_t ep_rank, int64_t ep_size, void* stream);

/* -------------------------------------------------------------- reductions */

/* Replaces torch.ops._moe_C.moe_sum (csrc/moe/torch_bindings.cpp:7-10,
 * csrc/moe/moe_align_sum_kernels.cpp:1224-1372).  input [T,k,H] -> out
 * [T,H]; optional topk_ids [T,k] / expert_map skip padded or non-local
 * slots. */
int mi355moe_moe_sum(const void* input, void* output, int dtype,
                     int64_t num_tokens, int64_t topk, int64_t hidden,
                     const void* topk_ids, int ids_dtype,
                     const int32_t* expert_map, int64_t expert_map_len,
                     void* stream);

/* Replaces torch.ops._moe_C.moe_gather (csrc/moe/torch_bindings.cpp:78-82,
 * csrc/moe/moe_gather.cpp:161-204).  out[t] = sum_j w[t,j]*in[perm[t,j]]. */
int mi355moe_moe_gather(void* output, const void* moe_output, int dtype,
                        const float* topk_weights, const int32_t* perm,
                        int64_t num_tokens, int64_t topk, int64_t hidden,
                        void* stream);

/* ------------------------------------------------------------ activations */

/* Replaces torch.ops._C.silu_and_mul (csrc/torch_bindings.cpp:80-81,
 * csrc/activation.cpp:492-499).  in [rows, 2d] -> out [rows, d]. */
int mi355moe_silu_and_mul(void* out, const void* input, int dtype,
                          int64_t rows, int64_t d, void* stream);

/* Replaces torch.ops._C.swigluoai_and_mul (csrc/torch_bindings.cpp:187-191,
 * csrc/activation.cpp:626-689). */
int mi355moe_swigluoai_and_mul(void* out, const void* input, int dtype,
                               int64_t rows, int64_t d, float alpha,
                               float limit, void* stream);

/* Replace torch.ops._C.gelu_and_mul / gelu_tanh_and_mul (csrc/
 * torch_bindings.cpp:112-116, csrc/activation.cpp:52-73, 577-593):
 * in [rows, 2d] -> out[r, c] = T(T(act(x[r, c])) * x[r, d + c]), act the
 * exact (erf) or tanh-approximated GELU in fp32; dtype F32, F16 or BF16. */
int mi355moe_gelu_and_mul(void* out, const void* input, int dtype, int64_t rows,
                          int64_t d, void* stream);
int mi355moe_gelu_tanh_and_mul(void* out, const void* input, int dtype, int64_t rows,
                               int64_t d, void* stream);

/* Replaces torch.ops._C.swiglustep_and_mul (csrc/torch_bindings.cpp:197-201,
 * csrc/activation.cpp:297-311, 711-716): out = T(min(silu(g), limit) *
 * clamp(u, -limit, limit)) in fp32, g = x[:, :d], u = x[:, d:]. */
int mi355moe_swiglustep_and_mul(void* out, const void* input, int dtype, int64_t rows,
                                int64_t d, float limit, void* stream);

/* Replaces torch.ops._C.relu2_no_mul (csrc/torch_bindings.cpp:193-195,
 * csrc/activation.cpp:44-50, 674-681): out[r, c] = T(max(x, 0)^2),
 * in and out [rows, d]. */
int mi355moe_relu2_no_mul(void* out, const void* input, int dtype, int64_t rows,
                          int64_t d, void* stream);

/* ----------------------------------------------------------- quantisation */

/* Replaces torch.ops._C.per_token_group_fp8_quant (csrc/torch_bindings.cpp:
 * 170-177, csrc/quantization/fp8/fp8_quant.cpp:724-881).  Row-major scales
 * [rows, cols/group]. */
int mi355moe_per_token_group_fp8_quant(const void* input, int dtype,
                                       void* output_q, float* output_s,
                                       int64_t rows, int64_t cols,
                                       int64_t group_size, float eps,
                                       float fp8_min, float fp8_max,
                                       int scale_ue8m0, void* stream);

/* Replaces torch.ops._C.per_token_group_quant_mxfp4 (csrc/torch_bindings.cpp:
 * 180-184, csrc/quantization/fp4/mxfp4_quant.cpp:24-126). */
int mi355moe_per_token_group_quant_mxfp4(const void* input, int dtype,
                                         uint8_t* output_q, float* output_s,
                                         int64_t rows, int64_t cols,
                                         int64_t group_size, float eps,
                                         void* stream);

/* Replaces torch.ops._C.silu_and_mul_per_block_quant (csrc/torch_bindings.cpp:
 * 88-101, csrc/quantization/fused_kernels/fused_silu_mul_block_quant.cpp:
 * 14-137 kernel, 141-239 checks).  input [rows, 2*hidden] bf16/f16 (gate ||
 * up); r = silu(gate) * up in fp32; per group of group_size (32, 64, 128)
 * columns: s = max(amax / qmax, 1 / (qmax * 512)) for fp8 (then clamped to
 * *scale_ub if given, and rounded up to a power of two if scale_ue8m0),
 * s = max(amax / 127, FLT_EPSILON) for int8; out [rows, hidden] of out_dtype
 * (FP8E4M3, FP8E5M2, I8) = saturate(r / s).  Scale (t, g) is stored at
 * scales[t * scale_stride_token + g * scale_stride_group]. */
int mi355moe_silu_and_mul_per_block_quant(void* out, int out_dtype, const void* input,
                                          int in_dtype, float* scales,
                                          int64_t scale_stride_token,
                                          int64_t scale_stride_group, int64_t rows,
                                          int64_t hidden, int64_t group_size,
                                          const float* scale_ub, int scale_ue8m0,
                                          void* stream);

/* Replaces torch.ops._C.silu_and_mul_mxfp4_quant (csrc/torch_bindings.cpp:
 * 103-107, csrc/quantization/fused_kernels/fused_silu_mul_mxfp4_quant.cpp:
 * 18-130 kernel, 134-209 checks).  r as above; per 32 columns s =
 * 2^ceil(log2(max(amax / 6, eps))) (fp32, stored like the block quantiser's
 * scales); out [rows, hidden/2] e2m1 codes of clamp(r / s, +-6), two per
 * byte, the even column in the low nibble.  eps must be a normal float. */
int mi355moe_silu_and_mul_mxfp4_quant(uint8_t* out, const void* input, int in_dtype,
                                      float* scales, int64_t scale_stride_token,
                                      int64_t scale_stride_group, int64_t rows,
                                      int64_t hidden, int64_t group_size, float eps,
                                      void* stream);

/* ------------------------------------------------------------ grouped GEMM */

/* Replaces torch.ops._xpu_C.cutlass_grouped_gemm_interface
 * (csrc/xpu/torch_bindings.cpp:46-53, csrc/xpu/grouped_gemm/
 * grouped_gemm_interface.cpp:12-60).  Rows of expert e are contiguous in A
 * and D (prefix sums of rows_per_expert, read on device).
 *   recipe BF16:     A bf16 or f16 [M,K]; B of the same type [E,N,K];
 *                    b_scale optional f32 [E]: each expert's accumulators
 *                    times b_scale[e] before the bias (per-expert-scaled
 *                    fp8 weights converted exactly to the 16-bit type; the
 *                    reference's acc * s_e, gemm_xe2.hpp:192-198)
 *   recipe FP8BLOCK: A e4m3 [M,K] + a_scale f32 [M,K/128] (1x128 groups),
 *                    or A bf16/f16 (quantised 1x128 in the workspace);
 *                    B e4m3 [E,N,K] + b_scale f32 [E,N/128,K/128]
 *   recipe MXFP4:    A bf16 or f16 [M,K]; B u8 [E,N,K/2] + b_scale e8m0
 *                    [E,N,K/32]
 *   recipe FP8 / FP8E5M2: A bf16 or f16 [M,K]; B e4m3 / e5m2 [E,N,K]
 *                    (K % 32 == 0) + b_scale f32 [E]: the weights read as
 *                    fp8 and converted exactly to a_dtype, the STREAM or
 *                    SMALL kernels at any M
 * bias: optional [E,N] in out_dtype; D [M,N] bf16 or f16 (out_dtype; equal
 * to a_dtype for recipes BF16, MXFP4, FP8 and FP8E5M2). */
size_t mi355moe_grouped_gemm_workspace_size(int64_t total_rows,
                                            int64_t num_experts);
/* Workspace including the on-the-fly 1x128 quantisation a 16-bit A needs
 * under the fp8 recipe. */
size_t mi355moe_grouped_gemm_workspace_size_k(int recipe, int a_dtype,
                                              int64_t total_rows, int64_t K,
                                              int64_t num_experts);
int mi355moe_grouped_gemm(int recipe, const void* A, int a_dtype,
                          const float* a_scale, const void* B,
                          const void* b_scale, const void* bias, void* D,
                          int out_dtype, const int32_t* rows_per_expert,
                          int64_t total_rows, int64_t N, int64_t K,
                          int64_t num_experts, void* workspace,
                          size_t workspace_bytes, void* stream);

/* The int4 (w4a16) path of torch.ops._xpu_C.cutlass_grouped_gemm_interface
 * (csrc/xpu/grouped_gemm/xe_2/grouped_gemm_xe2_interface.hpp:178, 267-290,
 * gemm_xe2.hpp:391-471): B [E, N, K/2] two's-complement int4 (the even K value
 * in the low nibble), b_scale [E, N, K/group_size] in a_dtype (bf16 or
 * f16), group_size 32/64/128/256; D [M, N] in a_dtype. */
int mi355moe_grouped_gemm_int4(const void* A, int a_dtype, const void* B,
                               const void* b_scale, int64_t group_size, const void* bias,
                               void* D, const int32_t* rows_per_expert, int64_t total_rows,
                               int64_t N, int64_t K, int64_t num_experts, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- fused MoE layer */

/* The whole XpuFusedMoe.apply path (vllm_xpu_kernels/fused_moe_interface.py:
 * 273-419) in one call: align -> [act quant] -> w13 grouped GEMM with the
 * activation (and fp8 re-quantisation) fused in its epilogue -> w2 grouped
 * GEMM -> weighted top-k reduction.  Weights use the canonical layout:
 * w13 [E, 2I, H] (gate rows 0..I-1, up rows I..2I-1; swigluoai weights are
 * de-interleaved by the caller), w2 [E, H, I], K contiguous. */
typedef struct {
  int recipe;            /* mi355moe_recipe                                  */
  int activation;        /* mi355moe_activation                              */
  int act_dtype;         /* MI355MOE_BF16 or MI355MOE_F16: hidden_states,
                            output, biases, 16-bit weights and intermediates */
  int ids_dtype;         /* dtype of topk_ids: I32 or I64                    */
  int64_t num_tokens;    /* T                                                */
  int64_t hidden;        /* H                                                */
  int64_t inter;         /* I                                                */
  int64_t num_experts;   /* E (local experts)                                */
  int64_t topk;          /* k                                                */
  const void* hidden_states;  /* [T, H]                                      */
  const float* topk_weights;  /* [T, k] f32                                  */
  const void* topk_ids;       /* [T, k]                                      */
  const int32_t* expert_map;  /* optional [expert_map_len]: global -> local  */
  int64_t expert_map_len;
  const void* w13;            /* per recipe                                  */
  const void* w13_scale;      /* per recipe; BF16: optional f32 [E] factor
                                 on the accumulators (per-expert fp8 on
                                 16-bit copies); FP8 / FP8E5M2: f32 [E]   */
  const void* w13_bias;       /* optional [E, 2I] bf16 (same row order)      */
  const void* w2;
  const void* w2_scale;       /* as w13_scale                               */
  const void* w2_bias;        /* optional [E, H] bf16                        */
  float gemm1_clamp_limit;    /* <= 0: off                                   */
  float swiglu_alpha;         /* swigluoai alpha (1.702)                     */
  float swiglu_limit;         /* swigluoai limit (7.0)                       */
  void* output;               /* [T, H]                                      */
  int w_layout;               /* mi355moe_weight_layout of w13 and w2 (bf16) */
  /* Optional (the reference's a1q_scale, vllm_xpu_kernels/
   * fused_moe_interface.py:326-360, moe_utils.py:189-199): when non-null,
   * hidden_states are already quantised and the layer uses them with these
   * scales as they are; act_dtype still names the output's type.
   *   FP8BLOCK  e4m3 [T, H] + f32 [T, H/128] (1x128 groups)
   *   MXFP8     e4m3 [T, H] + e8m0 u8 [T, H/32]
   *   MXFP4     packed e2m1 [T, H/2] + e8m0 u8 [T, H/32]: both GEMMs then
   *             run e2m1 x e2m1 (the w13 epilogue re-quantises the
   *             activation to mxfp4 for w2, as the reference's qdq_act). */
  const void* hidden_scale;
  /* recipe INT4: K values per group scale (32, 64, 128 or 256) */
  int64_t w_group;
  /* recipe FP8BLOCK: w13 rows per w13_scale row, 128 (0 also means 128) or
   * 64.  64 is the layout of an interleaved swigluoai w13 (gate row 2j, up
   * row 2j + 1, 128 x 128 scale blocks, as the reference's) split into a
   * gate half and an up half: row n of either half keeps the scale of
   * interleaved block n / 64 of its half, so w13_scale is [E, 2I/64, H/128]
   * with its two halves equal to the reference's [E, 2I/128, H/128]. */
  int64_t w13_scale_rows;
} mi355moe_fused_moe_args;

/* One-time weight preparation, the counterpart of the repacking the
 * reference's XpuFusedMoe.__init__ does on its weights
 * (vllm_xpu_kernels/fused_moe_interface.py:194-206): src [E, N, K] -> dst
 * [E, K/B, N, B] (MI355MOE_WLAYOUT_KBLOCK): dtype BF16 or F16 (B = 32),
 * FP8E4M3 (B = 128) or U8 = packed e2m1 pairs (B = 32 values = 16 bytes; K
 * counts values); K % B == 0; src and dst must not overlap. */
int mi355moe_pack_weights_kblock(const void* src, void* dst, int dtype,
                                 int64_t num_experts, int64_t N, int64_t K,
                                 void* stream);
/* mxfp4 e8m0 scales for MI355MOE_WLAYOUT_KBLOCK: u8 [E, N, kblocks] ->
 * [E, kblocks, N] (kblocks = K/32); src and dst must not overlap. */
int mi355moe_pack_scales_kblock(const void* src, void* dst, int64_t num_experts,
                                int64_t N, int64_t kblocks, void* stream);

size_t mi355moe_fused_moe_workspace_size(const mi355moe_fused_moe_args* args);
int mi355moe_fused_moe(const mi355moe_fused_moe_args* args, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Allocation-free variant of mi355moe_fused_moe.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a static device array of MI355MOE_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends); the call allocates nothing and returns
 * MI355MOE_ERR_WORKSPACE when mi355moe_fused_moe_workspace_size(args) exceeds
 * it (64 MiB covers decode batches: DeepSeek-V3 shape up to 256 tokens,
 * Qwen3-30B-A3B up to 512).  Calls that overlap on one GPU share that array
 * and race. */
#define MI355MOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int mi355moe_fused_moe_noalloc(const mi355moe_fused_moe_args* args, void* stream);

/* Stage timing (no counterpart in the reference, whose benchmark brackets
 * each op with torch.xpu.Event, benchmark/src/fused_moe_interface_.py:144-226).
 * mi355moe_fused_moe_timed records HIP events on `stream` around its five
 * stages (align, activation quant, w13 GEMM, w2 GEMM, top-k reduction) into
 * slot `step` of the timer; mi355moe_timer_stage_ms waits for that step and
 * returns the five stage durations in milliseconds. */
#define MI355MOE_FUSED_STAGES 5
typedef struct mi355moe_timer_s* mi355moe_timer;
int mi355moe_timer_create(int max_steps, mi355moe_timer* out);
int mi355moe_timer_destroy(mi355moe_timer timer);
int mi355moe_fused_moe_timed(const mi355moe_fused_moe_args* args,
                             void* workspace, size_t workspace_bytes,
                             void* stream, mi355moe_timer timer, int step);
int mi355moe_timer_stage_ms(mi355moe_timer timer, int step, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* MI355MOE_H_ */
