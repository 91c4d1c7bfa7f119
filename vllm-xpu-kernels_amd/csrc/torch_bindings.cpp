// PyTorch-ROCm op registration over the mi355moe C ABI.
//
// Registers the reference's schemas verbatim in the same namespaces
// (_moe_C, _C, _xpu_C; reference csrc/moe/torch_bindings.cpp,
// csrc/torch_bindings.cpp, csrc/xpu/torch_bindings.cpp) for the CUDA dispatch
// key, which is how HIP devices appear in PyTorch-ROCm.  There is no CPU
// implementation: the ops exist only on the GPU.  Argument checks mirror the
// reference's TORCH_CHECK messages; the C ABI's own checks surface through
// mi355moe_last_error().
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "../../include/mi355moe.h"

namespace {

// PyTorch-ROCm exposes HIP devices as DeviceType::CUDA ("masquerading").
using DevGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

hipStream_t cur_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_rc(int rc, const char* op) {
  TORCH_CHECK(rc == MI355MOE_OK, op, ": ", mi355moe_last_error());
}

int dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return MI355MOE_F32;
    case at::kBFloat16: return MI355MOE_BF16;
    case at::kHalf: return MI355MOE_F16;
    case at::kInt: return MI355MOE_I32;
    case at::kLong: return MI355MOE_I64;
    case at::kUInt32: return MI355MOE_U32;
    case at::kFloat8_e4m3fn: return MI355MOE_FP8E4M3;
    case at::kByte: return MI355MOE_U8;
    case at::kFloat4_e2m1fn_x2: return MI355MOE_U8;
    case at::kFloat8_e8m0fnu: return MI355MOE_U8;
    case at::kShort: return MI355MOE_I16;
    case at::kFloat8_e5m2: return MI355MOE_FP8E5M2;
    case at::kChar: return MI355MOE_I8;
    default: return -1;
  }
}

void check_gpu(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be on a GPU device");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

const void* opt_ptr(const std::optional<at::Tensor>& t) {
  return t.has_value() ? t->data_ptr() : nullptr;
}

// ------------------------------------------------------------------ routing
void topk_softmax(at::Tensor& topk_weights, at::Tensor& topk_indices,
                  at::Tensor& token_expert_indices, at::Tensor& gating_output,
                  bool renormalize, const std::optional<at::Tensor>& bias) {
  check_gpu(gating_output, "gating_output");
  check_gpu(topk_weights, "topk_weights");
  check_gpu(topk_indices, "topk_indices");
  check_gpu(token_expert_indices, "token_expert_indices");
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  TORCH_CHECK(token_expert_indices.scalar_type() == at::kInt,
              "token_expert_indices must be int32");
  const int64_t E = gating_output.size(-1);
  const int64_t T = gating_output.numel() / E;
  const int64_t k = topk_weights.size(-1);
  if (bias) {
    check_gpu(*bias, "bias");
    TORCH_CHECK(bias->scalar_type() == at::kFloat, "bias must be float32");
    TORCH_CHECK(bias->numel() == E, "bias must have num_experts elements");
  }
  DevGuard g(gating_output.device());
  check_rc(mi355moe_topk_softmax(
               topk_weights.data_ptr<float>(), topk_indices.data_ptr(),
               dtype_code(topk_indices.scalar_type()),
               token_expert_indices.data_ptr<int32_t>(), gating_output.data_ptr(),
               dtype_code(gating_output.scalar_type()), T, E, k, renormalize,
               bias ? bias->data_ptr<float>() : nullptr, cur_stream(gating_output)),
           "topk_softmax");
}

void topk_sigmoid(at::Tensor& topk_weights, at::Tensor& topk_indices,
                  at::Tensor& token_expert_indices, at::Tensor& gating_output,
                  bool renormalize, const std::optional<at::Tensor>& bias,
                  double routed_scaling_factor) {
  check_gpu(gating_output, "gating_output");
  check_gpu(topk_weights, "topk_weights");
  check_gpu(topk_indices, "topk_indices");
  check_gpu(token_expert_indices, "token_expert_indices");
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  const int64_t E = gating_output.size(-1);
  const int64_t T = gating_output.numel() / E;
  const int64_t k = topk_weights.size(-1);
  if (bias) {
    check_gpu(*bias, "bias");
    TORCH_CHECK(bias->scalar_type() == at::kFloat, "bias must be float32");
  }
  DevGuard g(gating_output.device());
  check_rc(mi355moe_topk_sigmoid(
               topk_weights.data_ptr<float>(), topk_indices.data_ptr(),
               dtype_code(topk_indices.scalar_type()),
               token_expert_indices.data_ptr<int32_t>(), gating_output.data_ptr(),
               dtype_code(gating_output.scalar_type()), T, E, k, renormalize,
               bias ? bias->data_ptr<float>() : nullptr,
               static_cast<float>(routed_scaling_factor), cur_stream(gating_output)),
           "topk_sigmoid");
}

// reference csrc/moe/topk_softplus_sqrt_kernels.cpp:596-772
void topk_softplus_sqrt(at::Tensor& topk_weights, at::Tensor& topk_indices,
                        at::Tensor& token_expert_indices, at::Tensor& gating_output,
                        bool renormalize, double routed_scaling_factor,
                        const std::optional<at::Tensor>& correction_bias,
                        const std::optional<at::Tensor>& input_ids,
                        const std::optional<at::Tensor>& tid2eid) {
  check_gpu(gating_output, "gating_output");
  check_gpu(topk_weights, "topk_weights");
  check_gpu(topk_indices, "topk_indices");
  check_gpu(token_expert_indices, "token_expert_indices");
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  const int64_t E = gating_output.size(-1);
  const int64_t T = gating_output.numel() / E;
  const int64_t k = topk_weights.size(-1);
  if (correction_bias) {
    check_gpu(*correction_bias, "correction_bias");
    TORCH_CHECK(correction_bias->scalar_type() == at::kFloat, "correction_bias must be float32");
  }
  if (tid2eid) {
    TORCH_CHECK(input_ids.has_value(), "input_ids is required for hash MoE");
    check_gpu(*input_ids, "input_ids");
    check_gpu(*tid2eid, "tid2eid");
    TORCH_CHECK(input_ids->scalar_type() == topk_indices.scalar_type(),
                "input_ids dtype must match topk_indices dtype");
    TORCH_CHECK(tid2eid->scalar_type() == topk_indices.scalar_type(),
                "tid2eid dtype must match topk_indices dtype");
    TORCH_CHECK(input_ids->numel() >= T, "input_ids needs one id per token");
  }
  DevGuard g(gating_output.device());
  check_rc(mi355moe_topk_softplus_sqrt(
               topk_weights.data_ptr<float>(), topk_indices.data_ptr(),
               dtype_code(topk_indices.scalar_type()),
               token_expert_indices.data_ptr<int32_t>(), gating_output.data_ptr(),
               dtype_code(gating_output.scalar_type()), T, E, k, renormalize,
               static_cast<float>(routed_scaling_factor),
               correction_bias ? correction_bias->data_ptr<float>() : nullptr,
               tid2eid ? input_ids->data_ptr() : nullptr,
               tid2eid ? tid2eid->data_ptr() : nullptr, cur_stream(gating_output)),
           "topk_softplus_sqrt");
}

std::tuple<at::Tensor, at::Tensor> grouped_topk(at::Tensor& scores,
                                                at::Tensor& scores_with_bias,
                                                int64_t n_group,
                                                int64_t topk_group, int64_t topk,
                                                bool renormalize,
                                                double routed_scaling_factor) {
  check_gpu(scores, "scores");
  check_gpu(scores_with_bias, "scores_with_bias");
  TORCH_CHECK(scores.scalar_type() == scores_with_bias.scalar_type(),
              "scores and scores_with_bias must have the same dtype");
  TORCH_CHECK(n_group <= 32,
              "n_group should be smaller than or equal to 32 for now");
  TORCH_CHECK(topk <= 32, "topk should be smaller than or equal to 32 for now");
  const int64_t T = scores.size(0), E = scores.size(1);
  auto vals = at::empty({T, topk}, scores.options());
  auto ids = at::empty({T, topk}, scores.options().dtype(at::kInt));
  DevGuard g(scores.device());
  check_rc(mi355moe_grouped_topk(vals.data_ptr(), ids.data_ptr<int32_t>(),
                                 scores.data_ptr(), scores_with_bias.data_ptr(),
                                 dtype_code(scores.scalar_type()), T, E, n_group,
                                 topk_group, topk, renormalize,
                                 static_cast<float>(routed_scaling_factor),
                                 cur_stream(scores)),
           "grouped_topk");
  return {vals, ids};
}

// sigmoid scoring + correction bias + grouped top-k in one launch
std::tuple<at::Tensor, at::Tensor> mi355_fused_grouped_topk(
    const at::Tensor& gating_output, const std::optional<at::Tensor>& bias, int64_t n_group,
    int64_t topk_group, int64_t topk, bool renormalize, double routed_scaling_factor) {
  check_gpu(gating_output, "gating_output");
  TORCH_CHECK(gating_output.dim() == 2 && gating_output.is_contiguous(),
              "gating_output must be a contiguous [num_tokens, num_experts] tensor");
  const int64_t T = gating_output.size(0), E = gating_output.size(1);
  if (bias) {
    check_gpu(*bias, "e_score_correction_bias");
    TORCH_CHECK(bias->scalar_type() == at::kFloat && bias->numel() == E && bias->is_contiguous(),
                "e_score_correction_bias must be a contiguous float32 [num_experts] tensor");
  }
  auto vals = at::empty({T, topk}, gating_output.options());
  auto ids = at::empty({T, topk}, gating_output.options().dtype(at::kInt));
  DevGuard g(gating_output.device());
  check_rc(mi355moe_fused_grouped_topk(vals.data_ptr(), ids.data_ptr<int32_t>(),
                                       gating_output.data_ptr(),
                                       bias ? bias->data_ptr<float>() : nullptr,
                                       dtype_code(gating_output.scalar_type()), T, E, n_group,
                                       topk_group, topk, renormalize,
                                       static_cast<float>(routed_scaling_factor),
                                       cur_stream(gating_output)),
           "fused_grouped_topk");
  return {vals, ids};
}

// ------------------------------------------------------------ meta kernels
// Shape functions for FakeTensor tracing (torch.compile, opcheck): the ops
// that only write into the caller's outputs change no metadata, so their
// meta kernel consumes the arguments and returns nothing; the ops that return
// tensors give them their shapes (symbolic sizes allowed).
void meta_noop(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const size_t n = op.schema().arguments().size();
  stack->erase(stack->end() - static_cast<std::ptrdiff_t>(n), stack->end());
}

std::tuple<at::Tensor, at::Tensor> grouped_topk_meta(
    at::Tensor& scores, at::Tensor&, int64_t, int64_t, int64_t topk, bool,
    double) {
  auto vals = at::empty_symint({scores.sym_size(0), c10::SymInt(topk)}, scores.options());
  auto ids = at::empty_symint({scores.sym_size(0), c10::SymInt(topk)},
                              scores.options().dtype(at::kInt));
  return {vals, ids};
}

std::tuple<at::Tensor, at::Tensor> fused_grouped_topk_meta(
    const at::Tensor& gating_output, const std::optional<at::Tensor>&, int64_t, int64_t,
    int64_t topk, bool, double) {
  auto vals = at::empty_symint({gating_output.sym_size(0), c10::SymInt(topk)},
                               gating_output.options());
  auto ids = at::empty_symint({gating_output.sym_size(0), c10::SymInt(topk)},
                              gating_output.options().dtype(at::kInt));
  return {vals, ids};
}

// ---------------------------------------------------------------- alignment
void moe_align_block_size(at::Tensor topk_ids, int64_t num_experts,
                          int64_t block_size, at::Tensor sorted_token_ids,
                          at::Tensor experts_ids, at::Tensor num_tokens_post_pad,
                          const std::optional<at::Tensor>& maybe_expert_map) {
  check_gpu(topk_ids, "topk_ids");
  check_gpu(sorted_token_ids, "sorted_token_ids");
  check_gpu(experts_ids, "experts_ids");
  check_gpu(num_tokens_post_pad, "num_tokens_post_pad");
  TORCH_CHECK(sorted_token_ids.scalar_type() == at::kInt &&
                  experts_ids.scalar_type() == at::kInt &&
                  num_tokens_post_pad.scalar_type() == at::kInt,
              "sorted_token_ids, experts_ids and num_tokens_post_pad must be int32");
  if (maybe_expert_map) {
    check_gpu(*maybe_expert_map, "expert_map");
    TORCH_CHECK(maybe_expert_map->scalar_type() == at::kInt, "expert_map must be int32");
  }
  DevGuard g(topk_ids.device());
  const size_t ws_bytes =
      mi355moe_moe_align_block_size_workspace_size(topk_ids.numel(), num_experts);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({static_cast<int64_t>(ws_bytes)}, topk_ids.options().dtype(at::kByte));
  check_rc(mi355moe_moe_align_block_size(
               topk_ids.data_ptr(), dtype_code(topk_ids.scalar_type()),
               topk_ids.numel(), num_experts, block_size,
               sorted_token_ids.data_ptr<int32_t>(), sorted_token_ids.numel(),
               experts_ids.data_ptr<int32_t>(), experts_ids.numel(),
               num_tokens_post_pad.data_ptr<int32_t>(),
               maybe_expert_map ? maybe_expert_map->data_ptr<int32_t>() : nullptr,
               ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, cur_stream(topk_ids)),
           "moe_align_block_size");
}

void moe_lora_align_block_size(at::Tensor topk_ids, at::Tensor token_lora_mapping,
                               int64_t num_experts, int64_t block_size, int64_t max_loras,
                               int64_t max_num_tokens_padded, int64_t max_num_m_blocks,
                               at::Tensor sorted_token_ids, at::Tensor experts_ids,
                               at::Tensor num_tokens_post_pad, at::Tensor adapter_enabled,
                               at::Tensor lora_ids,
                               const std::optional<at::Tensor>& maybe_expert_map) {
  TORCH_CHECK(block_size > 0, "block_size should be greater than 0. ");
  TORCH_CHECK((num_experts + 31) / 32 * 32 < 1024, "padded_num_experts must be less than 1024");
  check_gpu(topk_ids, "topk_ids");
  TORCH_CHECK(topk_ids.dim() == 2, "topk_ids must be [num_tokens, topk]");
  for (auto* t : {&token_lora_mapping, &sorted_token_ids, &experts_ids, &num_tokens_post_pad,
                  &adapter_enabled, &lora_ids}) {
    check_gpu(*t, "LoRA alignment tensor");
    TORCH_CHECK(t->scalar_type() == at::kInt,
                "token_lora_mapping, sorted_token_ids, experts_ids, num_tokens_post_pad, "
                "adapter_enabled and lora_ids must be int32");
  }
  TORCH_CHECK(max_loras >= 0 && max_num_tokens_padded >= 0 && max_num_m_blocks >= 0,
              "max_loras, max_num_tokens_padded and max_num_m_blocks must be >= 0");
  TORCH_CHECK(token_lora_mapping.numel() >= topk_ids.size(0),
              "token_lora_mapping needs one entry per token");
  TORCH_CHECK(sorted_token_ids.numel() >= max_loras * max_num_tokens_padded &&
                  experts_ids.numel() >= max_loras * max_num_m_blocks &&
                  num_tokens_post_pad.numel() >= max_loras &&
                  adapter_enabled.numel() >= max_loras,
              "LoRA alignment outputs are smaller than max_loras slices");
  if (maybe_expert_map) {
    check_gpu(*maybe_expert_map, "expert_map");
    TORCH_CHECK(maybe_expert_map->scalar_type() == at::kInt &&
                    maybe_expert_map->numel() >= num_experts,
                "expert_map must be int32 [num_experts]");
  }
  DevGuard g(topk_ids.device());
  // one workgroup per entry of lora_ids, at most max_loras + 1 of them (the
  // real adapters and a possible -1)
  const int64_t slots = std::min<int64_t>(lora_ids.numel(), max_loras + 1);
  check_rc(mi355moe_moe_lora_align_block_size(
               topk_ids.data_ptr(), dtype_code(topk_ids.scalar_type()), topk_ids.size(0),
               topk_ids.size(1), token_lora_mapping.data_ptr<int32_t>(), num_experts,
               block_size, max_loras, max_num_tokens_padded, max_num_m_blocks,
               sorted_token_ids.data_ptr<int32_t>(), experts_ids.data_ptr<int32_t>(),
               num_tokens_post_pad.data_ptr<int32_t>(), adapter_enabled.data_ptr<int32_t>(),
               lora_ids.data_ptr<int32_t>(), slots,
               maybe_expert_map ? maybe_expert_map->data_ptr<int32_t>() : nullptr,
               cur_stream(topk_ids)),
           "moe_lora_align_block_size");
}

// Input / scale pairs as the reference dispatches them
// (fused_moe_prologue.cpp:186-215): bf16 and fp16 without scales (given
// scales are ignored), e4m3 with f32 or e8m0 scales, packed e2m1 with e8m0.
void fused_moe_prologue(at::Tensor input, const std::optional<at::Tensor>& input_scales,
                        at::Tensor token_selected_experts, at::Tensor token_final_scales,
                        at::Tensor workspace, int64_t hidden_size, int64_t inter_size,
                        int64_t block_k, int64_t ep_rank, int64_t ep_size,
                        int64_t num_experts_on_rank) {
  check_gpu(input, "input");
  check_gpu(token_selected_experts, "token_selected_experts");
  check_gpu(token_final_scales, "token_final_scales");
  check_gpu(workspace, "workspace");
  TORCH_CHECK(input.dim() == 2 && input.size(1) == hidden_size,
              "input must be [num_rows, hidden_size]");
  TORCH_CHECK(token_selected_experts.dim() == 2 &&
                  token_selected_experts.size(0) == input.size(0),
              "token_selected_experts must be [num_rows, experts_per_token]");
  TORCH_CHECK(token_selected_experts.scalar_type() == at::kLong ||
                  token_selected_experts.scalar_type() == at::kInt,
              "token_selected_experts must be int64");
  TORCH_CHECK(token_final_scales.scalar_type() == at::kFloat &&
                  token_final_scales.sizes() == token_selected_experts.sizes(),
              "token_final_scales must be float32 [num_rows, experts_per_token]");
  TORCH_CHECK(workspace.scalar_type() == at::kByte && workspace.is_contiguous(),
              "workspace must be a contiguous uint8 tensor");
  const auto dt = input.scalar_type();
  int64_t elem_bytes = 0, scale_bytes = 0;
  const void* scales = nullptr;
  if (dt == at::kBFloat16 || dt == at::kHalf) {
    elem_bytes = 2;
  } else if (dt == at::kFloat8_e4m3fn || dt == at::kFloat4_e2m1fn_x2) {
    elem_bytes = 1;
    TORCH_CHECK(input_scales.has_value(), "fp8 and fp4 inputs need input_scales");
    const auto sdt = input_scales->scalar_type();
    TORCH_CHECK(sdt == at::kFloat8_e8m0fnu || (dt == at::kFloat8_e4m3fn && sdt == at::kFloat),
                "input_scales must be e8m0 (or float32 with e4m3 input)");
    check_gpu(*input_scales, "input_scales");
    TORCH_CHECK(block_k > 0 && hidden_size % block_k == 0 &&
                    input_scales->numel() == input.size(0) * (hidden_size / block_k),
                "input_scales must be [num_rows, hidden_size / block_k]");
    scale_bytes = sdt == at::kFloat ? 4 : 1;
    scales = input_scales->data_ptr();
  } else {
    TORCH_CHECK(false, "fused_moe_prologue: unsupported input dtype ", dt);
  }
  DevGuard g(input.device());
  check_rc(mi355moe_fused_moe_prologue(
               input.data_ptr(), elem_bytes, scales, scale_bytes,
               token_selected_experts.data_ptr(), dtype_code(token_selected_experts.scalar_type()),
               token_final_scales.data_ptr<float>(), workspace.data_ptr(),
               static_cast<size_t>(workspace.numel()), input.size(0), hidden_size, inter_size,
               block_k, token_selected_experts.size(1), ep_rank, ep_size, num_experts_on_rank,
               cur_stream(input)),
           "fused_moe_prologue");
}

void remap_hidden_states(at::Tensor& hidden_states,
                         const std::optional<at::Tensor>& hidden_states_scales,
                         at::Tensor& remapped_hidden_states,
                         const std::optional<at::Tensor>& remapped_hidden_states_scales,
                         const std::optional<at::Tensor>& expert_map,
                         at::Tensor& rows_per_expert,
                         at::Tensor& unpermuted_row_to_permuted_row,
                         at::Tensor& topk_ids, int64_t total_experts_num,
                         int64_t local_experts_num) {
  check_gpu(hidden_states, "hidden_states");
  check_gpu(remapped_hidden_states, "remapped_hidden_states");
  check_gpu(rows_per_expert, "rows_per_expert");
  check_gpu(unpermuted_row_to_permuted_row, "unpermuted_row_to_permuted_row");
  check_gpu(topk_ids, "topk_ids");
  TORCH_CHECK(local_experts_num <= 1024,
              "local experts number should be less than or equal to 1024");
  const int64_t T = hidden_states.size(0);
  const int64_t k = topk_ids.size(1);
  int64_t scale_cols = 0, scale_bytes = 0;
  if (hidden_states_scales && remapped_hidden_states_scales) {
    scale_cols = hidden_states_scales->numel() / std::max<int64_t>(T, 1);
    scale_bytes = hidden_states_scales->element_size();
  }
  DevGuard g(hidden_states.device());
  const size_t ws_bytes =
      mi355moe_remap_hidden_states_workspace_size(T, k, local_experts_num);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({static_cast<int64_t>(ws_bytes)}, topk_ids.options().dtype(at::kByte));
  check_rc(mi355moe_remap_hidden_states(
               hidden_states.data_ptr(), hidden_states.element_size(),
               opt_ptr(hidden_states_scales), scale_cols, scale_bytes,
               remapped_hidden_states.data_ptr(),
               remapped_hidden_states_scales ? remapped_hidden_states_scales->data_ptr()
                                             : nullptr,
               expert_map ? expert_map->data_ptr<int32_t>() : nullptr,
               rows_per_expert.data_ptr<int32_t>(),
               unpermuted_row_to_permuted_row.data_ptr<int32_t>(),
               topk_ids.data_ptr(), dtype_code(topk_ids.scalar_type()), T,
               hidden_states.numel() / std::max<int64_t>(T, 1), k,
               total_experts_num, local_experts_num, ws_bytes ? ws.data_ptr() : nullptr,
               ws_bytes, cur_stream(hidden_states)),
           "remap_hidden_states");
}

void init_expert_map(at::Tensor expert_map, int64_t num_experts,
                     int64_t ep_rank, int64_t ep_size) {
  check_gpu(expert_map, "expert_map");
  TORCH_CHECK(expert_map.scalar_type() == at::kInt, "expert_map must be int32");
  TORCH_CHECK(expert_map.numel() >= num_experts * ep_size,
              "expert_map must hold num_experts * ep_size entries");
  DevGuard g(expert_map.device());
  check_rc(mi355moe_init_expert_map(expert_map.data_ptr<int32_t>(), num_experts,
                                    ep_rank, ep_size, cur_stream(expert_map)),
           "init_expert_map");
}

// --------------------------------------------------------------- reductions
void moe_sum(at::Tensor& input, at::Tensor& output,
             const std::optional<at::Tensor>& topk_ids,
             const std::optional<at::Tensor>& expert_map) {
  const int64_t H = input.size(-1);
  const int64_t T = output.numel() / H;
  const int64_t topk = input.size(1);
  TORCH_CHECK(input.scalar_type() == output.scalar_type(),
              "moe_sum: input and output must have the same dtype");
  TORCH_CHECK(input.device() == output.device(),
              "moe_sum: input and output must be on the same device");
  TORCH_CHECK(input.is_contiguous() && output.is_contiguous(),
              "moe_sum expects contiguous input and output");
  TORCH_CHECK(input.numel() == output.numel() * topk,
              "moe_sum: input shape must be [num_tokens, topk, hidden] matching "
              "output [num_tokens, hidden]");
  TORCH_CHECK(!(expert_map.has_value() && !topk_ids.has_value()),
              "moe_sum: expert_map requires topk_ids to be provided");
  if (topk_ids) {
    const auto& tk = *topk_ids;
    TORCH_CHECK(tk.is_contiguous(), "moe_sum: topk_ids must be contiguous");
    TORCH_CHECK(tk.device() == input.device(),
                "moe_sum: topk_ids must be on the same device as input");
    TORCH_CHECK(tk.dim() == 2 && tk.size(0) == T && tk.size(1) == topk,
                "moe_sum: topk_ids must have shape [num_tokens, topk]");
    if (expert_map) {
      const auto& em = *expert_map;
      TORCH_CHECK(em.scalar_type() == at::kInt, "moe_sum: expert_map must be int32");
      TORCH_CHECK(em.is_contiguous(), "moe_sum: expert_map must be contiguous");
      TORCH_CHECK(em.device() == input.device(),
                  "moe_sum: expert_map must be on the same device as input");
    }
  }
  TORCH_CHECK(input.is_cuda(), "moe_sum: input must be on a GPU device");
  DevGuard g(input.device());
  check_rc(mi355moe_moe_sum(input.data_ptr(), output.data_ptr(),
                            dtype_code(input.scalar_type()), T, topk, H,
                            topk_ids ? topk_ids->data_ptr() : nullptr,
                            topk_ids ? dtype_code(topk_ids->scalar_type()) : MI355MOE_I32,
                            expert_map ? expert_map->data_ptr<int32_t>() : nullptr,
                            expert_map ? expert_map->numel() : 0, cur_stream(input)),
           "moe_sum");
}

void moe_gather(at::Tensor& output, at::Tensor& moe_output,
                at::Tensor& topk_weights, at::Tensor& perm, int64_t num_experts) {
  check_gpu(output, "output");
  check_gpu(moe_output, "moe_output");
  check_gpu(topk_weights, "topk_weights");
  check_gpu(perm, "unpermuted_row_to_permuted_row");
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  TORCH_CHECK(perm.scalar_type() == at::kInt, "unpermuted_row_to_permuted_row must be int32");
  TORCH_CHECK(output.scalar_type() == moe_output.scalar_type(),
              "output and moe_output must have the same dtype");
  const int64_t T = output.size(0), H = output.size(1), k = perm.size(1);
  (void)num_experts;
  DevGuard g(output.device());
  check_rc(mi355moe_moe_gather(output.data_ptr(), moe_output.data_ptr(),
                               dtype_code(output.scalar_type()),
                               topk_weights.data_ptr<float>(),
                               perm.data_ptr<int32_t>(), T, k, H, cur_stream(output)),
           "moe_gather");
}

// ------------------------------------------------------------- activations
// in [..., 2d] -> out [..., d] of the same dtype; returns (rows, d)
std::pair<int64_t, int64_t> gated_shape(const at::Tensor& out, const at::Tensor& input) {
  check_gpu(out, "out");
  check_gpu(input, "input");
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), "out and input must have the same dtype");
  const int64_t d = input.size(-1) / 2;
  const int64_t rows = input.numel() / std::max<int64_t>(2 * d, 1);
  TORCH_CHECK(input.size(-1) == 2 * d && out.size(-1) == d && out.numel() == rows * d,
              "out must be [..., d] for input [..., 2 * d]");
  return {rows, d};
}

void silu_and_mul(at::Tensor& out, at::Tensor& input) {
  const auto [rows, d] = gated_shape(out, input);
  DevGuard g(input.device());
  check_rc(mi355moe_silu_and_mul(out.data_ptr(), input.data_ptr(),
                                 dtype_code(input.scalar_type()), rows, d,
                                 cur_stream(input)),
           "silu_and_mul");
}

void swigluoai_and_mul(at::Tensor& out, at::Tensor& input, double alpha, double limit) {
  const auto [rows, d] = gated_shape(out, input);
  DevGuard g(input.device());
  check_rc(mi355moe_swigluoai_and_mul(out.data_ptr(), input.data_ptr(),
                                      dtype_code(input.scalar_type()), rows, d,
                                      static_cast<float>(alpha),
                                      static_cast<float>(limit), cur_stream(input)),
           "swigluoai_and_mul");
}

// reference csrc/activation.cpp:577-593
void gelu_and_mul(at::Tensor& out, const at::Tensor& input) {
  const auto [rows, d] = gated_shape(out, input);
  DevGuard g(input.device());
  check_rc(mi355moe_gelu_and_mul(out.data_ptr(), input.data_ptr(),
                                 dtype_code(input.scalar_type()), rows, d, cur_stream(input)),
           "gelu_and_mul");
}

void gelu_tanh_and_mul(at::Tensor& out, const at::Tensor& input) {
  const auto [rows, d] = gated_shape(out, input);
  DevGuard g(input.device());
  check_rc(mi355moe_gelu_tanh_and_mul(out.data_ptr(), input.data_ptr(),
                                      dtype_code(input.scalar_type()), rows, d,
                                      cur_stream(input)),
           "gelu_tanh_and_mul");
}

// reference csrc/activation.cpp:711-716
void swiglustep_and_mul(at::Tensor& out, const at::Tensor& input, double limit) {
  const auto [rows, d] = gated_shape(out, input);
  DevGuard g(input.device());
  check_rc(mi355moe_swiglustep_and_mul(out.data_ptr(), input.data_ptr(),
                                       dtype_code(input.scalar_type()), rows, d,
                                       static_cast<float>(limit), cur_stream(input)),
           "swiglustep_and_mul");
}

// reference csrc/activation.cpp:674-681 (input and out [..., d])
void relu2_no_mul(at::Tensor& out, at::Tensor& input) {
  check_gpu(out, "out");
  check_gpu(input, "input");
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), "out and input must have the same dtype");
  TORCH_CHECK(out.numel() == input.numel(), "out must have the shape of input");
  const int64_t d = input.dim() > 0 ? input.size(-1) : 1;
  const int64_t rows = d > 0 ? input.numel() / d : 0;
  DevGuard g(input.device());
  check_rc(mi355moe_relu2_no_mul(out.data_ptr(), input.data_ptr(),
                                 dtype_code(input.scalar_type()), rows, d, cur_stream(input)),
           "relu2_no_mul");
}

// ------------------------------------------------------------ quantisation
void per_token_group_fp8_quant(const at::Tensor& input, at::Tensor& output_q,
                               at::Tensor& output_s, int64_t group_size,
                               double eps, double fp8_min, double fp8_max,
                               bool scale_ue8m0, bool, bool) {
  check_gpu(input, "input");
  check_gpu(output_q, "output_q");
  check_gpu(output_s, "output_s");
  TORCH_CHECK(output_q.scalar_type() == at::kFloat8_e4m3fn, "output_q must be float8_e4m3fn");
  TORCH_CHECK(output_s.scalar_type() == at::kFloat, "output_s must be float32");
  TORCH_CHECK(input.numel() % group_size == 0,
              "the last dimension of input must be divisible by group_size");
  const int64_t cols = input.size(-1);
  const int64_t rows = input.numel() / std::max<int64_t>(cols, 1);
  DevGuard g(input.device());
  check_rc(mi355moe_per_token_group_fp8_quant(
               input.data_ptr(), dtype_code(input.scalar_type()), output_q.data_ptr(),
               output_s.data_ptr<float>(), rows, cols, group_size,
               static_cast<float>(eps), static_cast<float>(fp8_min),
               static_cast<float>(fp8_max), scale_ue8m0, cur_stream(input)),
           "per_token_group_fp8_quant");
}

void per_token_group_quant_mxfp4(const at::Tensor& input, at::Tensor& output_q,
                                 at::Tensor& output_s, int64_t group_size,
                                 double eps) {
  check_gpu(input, "input");
  check_gpu(output_q, "output_q");
  check_gpu(output_s, "output_s");
  TORCH_CHECK(output_s.scalar_type() == at::kFloat, "output_s must be float32");
  const int64_t cols = input.size(-1);
  const int64_t rows = input.numel() / std::max<int64_t>(cols, 1);
  DevGuard g(input.device());
  check_rc(mi355moe_per_token_group_quant_mxfp4(
               input.data_ptr(), dtype_code(input.scalar_type()),
               static_cast<uint8_t*>(output_q.data_ptr()), output_s.data_ptr<float>(),
               rows, cols, group_size, static_cast<float>(eps), cur_stream(input)),
           "per_token_group_quant_mxfp4");
}

// Scales of the fused quantisers are written at t * sst + g * ssg: the tensor
// must have exactly that layout (row-major [T, G] or a transposed [G, T]).
void check_scale_strides(const at::Tensor& s, int64_t sst, int64_t ssg) {
  TORCH_CHECK((s.size(0) <= 1 || s.stride(0) == sst) && (s.size(1) <= 1 || s.stride(1) == ssg),
              "scales must be row-major [num_tokens, num_groups] or the transpose of a "
              "row-major [num_groups, num_tokens] tensor");
}

// reference csrc/quantization/fused_kernels/fused_silu_mul_block_quant.cpp:141-239
void silu_and_mul_per_block_quant(at::Tensor& out, const at::Tensor& input, at::Tensor& scales,
                                  int64_t group_size, const std::optional<at::Tensor>& scale_ub,
                                  bool is_scale_transposed, bool scale_ue8m0) {
  TORCH_CHECK(out.scalar_type() == at::kFloat8_e4m3fn || out.scalar_type() == at::kFloat8_e5m2 ||
                  out.scalar_type() == at::kChar,
              "out must be float8_e4m3fn, float8_e5m2, or int8");
  TORCH_CHECK(input.scalar_type() == at::kHalf || input.scalar_type() == at::kBFloat16,
              "input must be float16 or bfloat16");
  TORCH_CHECK(out.is_contiguous(), "out must be contiguous");
  TORCH_CHECK(input.is_contiguous(), "input must be contiguous");
  TORCH_CHECK(scales.scalar_type() == at::kFloat, "scales must be float32");
  TORCH_CHECK(group_size == 32 || group_size == 64 || group_size == 128,
              "group_size must be 32, 64, or 128, got ", group_size);
  if (scale_ub.has_value())
    TORCH_CHECK(out.scalar_type() != at::kChar, "scale_ub is only supported for FP8 output");
  TORCH_CHECK(input.dim() == 2, "input must be 2-dimensional");
  TORCH_CHECK(out.dim() == 2, "out must be 2-dimensional");
  const int64_t T = input.size(0);
  const int64_t hidden = out.size(-1);
  const int64_t groups = hidden / group_size;
  TORCH_CHECK(input.size(-1) == hidden * 2, "input last dim must be 2 * hidden_size");
  TORCH_CHECK(hidden % group_size == 0, "hidden_size must be divisible by group_size");
  TORCH_CHECK(out.size(0) == T, "out.size(0) must equal num_tokens (input.size(0))");
  TORCH_CHECK(scales.size(0) == T && scales.size(1) == groups,
              "scales must have logical shape [num_tokens, num_groups]");
  if (T == 0) return;
  check_gpu(input, "input");
  check_gpu(out, "out");
  TORCH_CHECK(scales.is_cuda(), "scales must be on a GPU device");
  const float* ub = nullptr;
  if (scale_ub.has_value()) {
    check_gpu(*scale_ub, "scale_ub");
    TORCH_CHECK(scale_ub->scalar_type() == at::kFloat && scale_ub->numel() >= 1,
                "scale_ub must be a float32 tensor");
    ub = scale_ub->data_ptr<float>();
  }
  const int64_t sst = is_scale_transposed ? 1 : groups;
  const int64_t ssg = is_scale_transposed ? T : 1;
  check_scale_strides(scales, sst, ssg);
  DevGuard g(input.device());
  check_rc(mi355moe_silu_and_mul_per_block_quant(
               out.data_ptr(), dtype_code(out.scalar_type()), input.data_ptr(),
               dtype_code(input.scalar_type()), scales.data_ptr<float>(), sst, ssg, T, hidden,
               group_size, ub, scale_ue8m0, cur_stream(input)),
           "silu_and_mul_per_block_quant");
}

// reference csrc/quantization/fused_kernels/fused_silu_mul_mxfp4_quant.cpp:134-209
void silu_and_mul_mxfp4_quant(at::Tensor& out, const at::Tensor& input, at::Tensor& scales,
                              int64_t group_size, double eps) {
  TORCH_CHECK(input.scalar_type() == at::kHalf || input.scalar_type() == at::kBFloat16,
              "input must be float16 or bfloat16");
  TORCH_CHECK(out.scalar_type() == at::kByte, "out must be uint8 (packed FP4)");
  TORCH_CHECK(out.is_contiguous(), "out must be contiguous");
  TORCH_CHECK(input.is_contiguous(), "input must be contiguous");
  TORCH_CHECK(scales.scalar_type() == at::kFloat, "scales must be float32");
  TORCH_CHECK(group_size == 32, "MXFP4 requires group_size == 32, got ", group_size);
  TORCH_CHECK(input.dim() == 2, "input must be 2-dimensional");
  TORCH_CHECK(out.dim() == 2, "out must be 2-dimensional");
  TORCH_CHECK(scales.dim() == 2, "scales must be 2-dimensional");
  const int64_t T = input.size(0);
  const int64_t hidden = input.size(-1) / 2;
  const int64_t groups = hidden / group_size;
  TORCH_CHECK(input.size(-1) == hidden * 2, "input last dim must be 2 * hidden_size");
  TORCH_CHECK(hidden % group_size == 0, "hidden_size must be divisible by group_size");
  TORCH_CHECK(out.size(0) == T && out.size(1) == hidden / 2,
              "out must have shape [num_tokens, hidden_size / 2]");
  TORCH_CHECK(scales.size(0) == T && scales.size(1) == groups,
              "scales must have logical shape [num_tokens, num_groups]");
  if (T == 0) return;
  check_gpu(input, "input");
  check_gpu(out, "out");
  TORCH_CHECK(scales.is_cuda(), "scales must be on a GPU device");
  const bool transposed = scales.stride(0) < scales.stride(1);
  const int64_t sst = transposed ? 1 : groups;
  const int64_t ssg = transposed ? T : 1;
  check_scale_strides(scales, sst, ssg);
  DevGuard g(input.device());
  check_rc(mi355moe_silu_and_mul_mxfp4_quant(
               static_cast<uint8_t*>(out.data_ptr()), input.data_ptr(),
               dtype_code(input.scalar_type()), scales.data_ptr<float>(), sst, ssg, T, hidden,
               group_size, static_cast<float>(eps), cur_stream(input)),
           "silu_and_mul_mxfp4_quant");
}

// ------------------------------------------------------------- grouped GEMM
at::Tensor grouped_gemm_meta(at::Tensor&, const std::optional<at::Tensor>&, at::Tensor&,
                             const std::optional<at::Tensor>&,
                             const std::optional<at::Tensor>&, at::Tensor& ptr_D, at::Tensor&,
                             int64_t, int64_t, int64_t) {
  return ptr_D;  // written in place and returned
}

at::Tensor cutlass_grouped_gemm_interface(at::Tensor& ptr_A,
                                          const std::optional<at::Tensor>& ptr_A_scale,
                                          at::Tensor& ptr_B,
                                          const std::optional<at::Tensor>& ptr_B_scale,
                                          const std::optional<at::Tensor>& ptr_bias,
                                          at::Tensor& ptr_D, at::Tensor& rows_per_expert,
                                          int64_t N, int64_t K, int64_t num_experts) {
  TORCH_CHECK(N % 8 == 0, "N must be divisible by 8");
  TORCH_CHECK(ptr_A.dim() == 2, "ptr_A must be 2D [Total_M, K]");
  TORCH_CHECK(ptr_B.dim() == 3, "ptr_B must be 3D");
  TORCH_CHECK(ptr_D.dim() == 2, "ptr_D must be 2D [Total_M, N]");
  TORCH_CHECK(ptr_A.is_contiguous(), "ptr_A must be contiguous");
  TORCH_CHECK(ptr_B.is_contiguous(), "ptr_B must be contiguous");
  TORCH_CHECK(ptr_D.is_contiguous(), "ptr_D must be contiguous");
  check_gpu(rows_per_expert, "rows_per_expert");
  TORCH_CHECK(ptr_B.size(0) == num_experts, "ptr_B.size(0) must match num_experts");
  TORCH_CHECK(ptr_A.size(0) == ptr_D.size(0), "ptr_A.size(0) must match ptr_D.size(0)");
  if (ptr_bias) {
    TORCH_CHECK(ptr_bias->dim() == 2, "ptr_bias must be 2D [num_experts, N]");
    TORCH_CHECK(ptr_bias->is_contiguous(), "ptr_bias must be contiguous");
    TORCH_CHECK(ptr_bias->size(0) == num_experts, "ptr_bias.size(0) must match num_experts");
    TORCH_CHECK(ptr_bias->size(1) == N, "ptr_bias.size(1) must match N");
  }
  const auto bdt = ptr_B.scalar_type();
  // fp8 weights with one scale per expert (not the 3-D block scales): the
  // reference's w8a16 per-expert path, acc * s_e (gemm_xe2.hpp:192-198)
  const bool is_fp8_expert = (bdt == at::kFloat8_e4m3fn || bdt == at::kFloat8_e5m2) &&
                             ptr_B_scale.has_value() && ptr_B_scale->dim() != 3;
  const bool is_fp8 = bdt == at::kFloat8_e4m3fn && !is_fp8_expert;
  const bool is_mxfp4 = bdt == at::kFloat4_e2m1fn_x2 ||
                        (bdt == at::kByte && ptr_B_scale.has_value() &&
                         ptr_B_scale->scalar_type() != at::kFloat);
  int recipe = MI355MOE_RECIPE_BF16;
  at::Tensor B = ptr_B;
  at::Tensor expert_scale;
  // int4 (reference grouped_gemm_xe2_interface.hpp:178, 267-290): int8 B
  // [E, N, K/2] of two's-complement nibbles, 16-bit scales [E, N, K/group]
  if (bdt == at::kChar && ptr_B_scale.has_value()) {
    TORCH_CHECK(ptr_B_scale->dim() == 3, "ptr_scales of int4 must be 3D [num_experts, N, group_num]");
    TORCH_CHECK(ptr_B_scale->size(0) == num_experts, "ptr_scales.size(0) of int4 must match num_experts");
    TORCH_CHECK(ptr_B_scale->size(1) == N, "ptr_scales.size(1) of int4 must match N");
    TORCH_CHECK(K % ptr_B_scale->size(2) == 0, "ptr_scales.size(2) of int4 must divide K");
    TORCH_CHECK(ptr_B_scale->scalar_type() == ptr_A.scalar_type(),
                "int4 scales must have the activation dtype");
    TORCH_CHECK(ptr_B.size(1) == N && ptr_B.size(2) * 2 == K,
                "ptr_B logical N dimension must match ptr_D N dimension and N");
    TORCH_CHECK(ptr_A.size(1) == K, "ptr_A K dimension must match ptr_B logical K dimension and K");
    TORCH_CHECK(ptr_D.scalar_type() == ptr_A.scalar_type(), "ptr_D must have the activation dtype");
    const int64_t M = ptr_A.size(0);
    const int adt = dtype_code(ptr_A.scalar_type());
    const size_t ws_bytes = mi355moe_grouped_gemm_workspace_size_k(MI355MOE_RECIPE_INT4, adt, M, K,
                                                                   num_experts);
    auto ws = at::empty({static_cast<int64_t>(ws_bytes)}, ptr_A.options().dtype(at::kByte));
    const auto scales = ptr_B_scale->contiguous();
    DevGuard g(ptr_A.device());
    check_rc(mi355moe_grouped_gemm_int4(ptr_A.data_ptr(), adt, ptr_B.data_ptr(), scales.data_ptr(),
                                        K / ptr_B_scale->size(2), opt_ptr(ptr_bias),
                                        ptr_D.data_ptr(), rows_per_expert.data_ptr<int32_t>(), M,
                                        N, K, num_experts, ws.data_ptr(), ws_bytes,
                                        cur_stream(ptr_A)),
             "cutlass_grouped_gemm_interface");
    return ptr_D;
  }
  if (is_fp8_expert) {
    TORCH_CHECK(ptr_A.scalar_type() == at::kBFloat16 || ptr_A.scalar_type() == at::kHalf,
                "per-expert fp8 weights need bfloat16 or float16 activations");
    TORCH_CHECK(ptr_B_scale->numel() == num_experts,
                "per-expert fp8 scales must have num_experts elements");
    TORCH_CHECK(ptr_B.size(1) == K && ptr_B.size(2) == N,
                "ptr_A K dimension must match ptr_B logical K dimension and K");
    // every e4m3 / e5m2 value is exact in bf16 and fp16
    B = ptr_B.to(ptr_A.scalar_type()).transpose(1, 2).contiguous();
    expert_scale = ptr_B_scale->to(at::kFloat).reshape({num_experts}).contiguous();
  } else if (is_mxfp4) {
    recipe = MI355MOE_RECIPE_MXFP4;
    TORCH_CHECK(ptr_B_scale.has_value(), "mxfp4 weights need ptr_B_scale");
    TORCH_CHECK(ptr_B.size(1) == N && ptr_B.size(2) * 2 == K,
                "ptr_B logical N dimension must match ptr_D N dimension and N");
  } else if (is_fp8) {
    TORCH_CHECK(ptr_B_scale.has_value() && ptr_B_scale->dim() == 3,
                "block scales must be 3D [num_experts, N / 128, K / 128]");
    TORCH_CHECK(N % 128 == 0 && K % 128 == 0,
                "block-scaled grouped GEMM requires N and K divisible by 128");
    TORCH_CHECK(ptr_B_scale->size(0) == num_experts &&
                    ptr_B_scale->size(1) == N / 128 && ptr_B_scale->size(2) == K / 128,
                "block scales must have shape [num_experts, N / 128, K / 128]");
    const bool nk = ptr_B.size(1) == N && ptr_B.size(2) == K;
    const bool kn = N != K && ptr_B.size(1) == K && ptr_B.size(2) == N;
    TORCH_CHECK(nk || kn, "block FP8 ptr_B must be [num_experts, N, K] or "
                          "[num_experts, K, N] (N=", N, ", K=", K, "), got ",
                ptr_B.sizes());
    if (!nk) B = ptr_B.transpose(1, 2).contiguous();
    recipe = MI355MOE_RECIPE_FP8BLOCK;
  } else if (!is_fp8_expert) {
    TORCH_CHECK(bdt == ptr_A.scalar_type(),
                "bf16/fp16 weights must have the activation dtype");
    // reference layout is [E, K, N]
    TORCH_CHECK(ptr_B.size(1) == K && ptr_B.size(2) == N,
                "ptr_A K dimension must match ptr_B logical K dimension and K");
    B = ptr_B.transpose(1, 2).contiguous();
  }
  TORCH_CHECK(ptr_A.size(1) == K,
              "ptr_A K dimension must match ptr_B logical K dimension and K");
  TORCH_CHECK(ptr_D.size(1) == N,
              "ptr_B logical N dimension must match ptr_D N dimension and N");
  if (ptr_bias)
    TORCH_CHECK(ptr_bias->scalar_type() == ptr_D.scalar_type(),
                "ptr_bias must have the output dtype");
  const int64_t M = ptr_A.size(0);
  const int adt = dtype_code(ptr_A.scalar_type());
  const size_t ws_bytes =
      mi355moe_grouped_gemm_workspace_size_k(recipe, adt, M, K, num_experts);
  auto ws = at::empty({static_cast<int64_t>(ws_bytes)}, ptr_A.options().dtype(at::kByte));
  DevGuard g(ptr_A.device());
  check_rc(mi355moe_grouped_gemm(
               recipe, ptr_A.data_ptr(), adt,
               ptr_A_scale ? ptr_A_scale->data_ptr<float>() : nullptr, B.data_ptr(),
               is_fp8_expert ? expert_scale.data_ptr()
                             : (ptr_B_scale && recipe != MI355MOE_RECIPE_BF16
                                    ? ptr_B_scale->data_ptr() : nullptr),
               opt_ptr(ptr_bias),
               ptr_D.data_ptr(), dtype_code(ptr_D.scalar_type()),
               rows_per_expert.data_ptr<int32_t>(), M, N, K, num_experts,
               ws.data_ptr(), ws_bytes, cur_stream(ptr_A)),
           "cutlass_grouped_gemm_interface");
  return ptr_D;
}

// -------------------------------------------------------- fused MoE layer
// Not a reference op: the one-call layer used by XpuFusedMoe.apply.
void mi355_fused_moe(at::Tensor& output, const at::Tensor& hidden_states,
                     const at::Tensor& topk_weights, const at::Tensor& topk_ids,
                     const at::Tensor& w13, const std::optional<at::Tensor>& w13_scale,
                     const std::optional<at::Tensor>& w13_bias, const at::Tensor& w2,
                     const std::optional<at::Tensor>& w2_scale,
                     const std::optional<at::Tensor>& w2_bias, int64_t recipe,
                     int64_t activation, int64_t inter_size, double clamp_limit,
                     const std::optional<at::Tensor>& expert_map, int64_t w_layout,
                     const std::optional<at::Tensor>& hidden_scale, int64_t w_group,
                     int64_t w13_scale_rows) {
  check_gpu(output, "output");
  check_gpu(hidden_states, "hidden_states");
  // packed e2m1 hidden states (mxfp4 with a1q_scale) hold two values a byte
  const bool packed4 = hidden_scale && recipe == MI355MOE_RECIPE_MXFP4;
  const int64_t hidden = packed4 ? 2 * hidden_states.size(1) : hidden_states.size(1);
  if (hidden_scale) {
    check_gpu(*hidden_scale, "hidden_scale");
    TORCH_CHECK(hidden_scale->is_contiguous() && hidden_states.is_contiguous(),
                "a1q_scale and hidden_states must be contiguous");
    if (recipe == MI355MOE_RECIPE_FP8BLOCK) {
      TORCH_CHECK(hidden_states.scalar_type() == at::kFloat8_e4m3fn,
                  "pre-quantised hidden_states must be float8_e4m3fn");
      TORCH_CHECK(hidden_scale->scalar_type() == at::kFloat && hidden_scale->dim() == 2 &&
                      hidden_scale->size(0) == hidden_states.size(0) &&
                      hidden_scale->size(1) * 128 == hidden,
                  "a1q_scale must be float32 [num_tokens, hidden_size / 128]");
    } else {
      TORCH_CHECK(recipe == MI355MOE_RECIPE_MXFP8 || recipe == MI355MOE_RECIPE_MXFP4,
                  "pre-quantised hidden_states need the fp8block, mxfp8 or mxfp4 recipe");
      TORCH_CHECK(packed4 ? hidden_states.element_size() == 1 &&
                                hidden_states.scalar_type() != at::kFloat8_e4m3fn
                          : hidden_states.scalar_type() == at::kFloat8_e4m3fn,
                  "pre-quantised hidden_states must be float8_e4m3fn (mxfp8) or packed "
                  "e2m1 (mxfp4, uint8 / float4_e2m1fn_x2 [num_tokens, hidden_size / 2])");
      TORCH_CHECK(hidden_scale->element_size() == 1 && hidden_scale->dim() == 2 &&
                      hidden_scale->size(0) == hidden_states.size(0) &&
                      hidden_scale->size(1) * 32 == hidden,
                  "a1q_scale must be e8m0 (uint8 / float8_e8m0fnu) [num_tokens, hidden_size / 32]");
    }
  }
  check_gpu(topk_weights, "topk_weights");
  check_gpu(topk_ids, "topk_ids");
  check_gpu(w13, "w13");
  check_gpu(w2, "w2");
  if (recipe == MI355MOE_RECIPE_FP8 || recipe == MI355MOE_RECIPE_FP8E5M2) {
    const auto wt = recipe == MI355MOE_RECIPE_FP8 ? at::kFloat8_e4m3fn : at::kFloat8_e5m2;
    TORCH_CHECK(w13.scalar_type() == wt && w2.scalar_type() == wt,
                "per-expert fp8 weights must be float8_e4m3fn (recipe 5) or float8_e5m2 "
                "(recipe 6)");
    TORCH_CHECK(w13_scale && w2_scale && w13_scale->scalar_type() == at::kFloat &&
                    w2_scale->scalar_type() == at::kFloat &&
                    w13_scale->numel() == w13.size(0) && w2_scale->numel() == w2.size(0),
                "per-expert fp8 weights need float32 scales [num_experts]");
  }
  if (recipe == MI355MOE_RECIPE_FP8BLOCK) {
    const int64_t rows = w13_scale_rows ? w13_scale_rows : 128;
    TORCH_CHECK(rows == 128 || rows == 64, "w13_scale_rows must be 128 or 64");
    TORCH_CHECK(w13_scale && w2_scale && w13_scale->scalar_type() == at::kFloat &&
                    w2_scale->scalar_type() == at::kFloat && w13_scale->is_contiguous() &&
                    w2_scale->is_contiguous(),
                "fp8 block-scaled weights need contiguous float32 scales");
    TORCH_CHECK(w13_scale->numel() == w13.size(0) * (2 * inter_size / rows) * (hidden / 128),
                "w13_scale must be float32 [num_experts, 2 * inter_size / ", rows,
                ", hidden_size / 128]");
  }
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  TORCH_CHECK(topk_weights.sizes() == topk_ids.sizes(),
              "topk_weights must have the shape of topk_ids");
  TORCH_CHECK(output.dim() == 2 && output.size(0) == hidden_states.size(0) &&
                  output.size(1) == hidden,
              "output must match hidden_states");
  // The kernels write the output, and read the biases, in the call's 16-bit
  // type: hidden_states' type, or the output's when they come quantised.
  if (hidden_scale) {
    TORCH_CHECK(output.scalar_type() == at::kBFloat16 || output.scalar_type() == at::kHalf,
                "output must be bfloat16 or float16");
  } else {
    TORCH_CHECK(output.scalar_type() == hidden_states.scalar_type(),
                "output must have hidden_states' dtype");
  }
  mi355moe_fused_moe_args a{};
  a.recipe = static_cast<int>(recipe);
  a.activation = static_cast<int>(activation);
  a.act_dtype = dtype_code((hidden_scale ? output : hidden_states).scalar_type());
  a.ids_dtype = dtype_code(topk_ids.scalar_type());
  a.num_tokens = hidden_states.size(0);
  a.hidden = hidden;
  a.inter = inter_size;
  a.num_experts = w13.size(0);
  a.topk = topk_ids.size(1);
  a.hidden_states = hidden_states.data_ptr();
  a.topk_weights = topk_weights.data_ptr<float>();
  a.topk_ids = topk_ids.data_ptr();
  a.expert_map = expert_map ? expert_map->data_ptr<int32_t>() : nullptr;
  a.expert_map_len = expert_map ? expert_map->numel() : 0;
  a.w13 = w13.data_ptr();
  a.w13_scale = opt_ptr(w13_scale);
  a.w13_bias = opt_ptr(w13_bias);
  a.w2 = w2.data_ptr();
  a.w2_scale = opt_ptr(w2_scale);
  a.w2_bias = opt_ptr(w2_bias);
  a.gemm1_clamp_limit = static_cast<float>(clamp_limit);
  a.swiglu_alpha = 1.702f;
  a.swiglu_limit = 7.0f;
  a.output = output.data_ptr();
  a.w_layout = static_cast<int>(w_layout);
  a.hidden_scale = hidden_scale ? hidden_scale->data_ptr() : nullptr;
  a.w_group = w_group;
  a.w13_scale_rows = w13_scale_rows;
  for (const auto* b : {&w13_bias, &w2_bias})
    if (b->has_value())
      TORCH_CHECK((*b)->scalar_type() == output.scalar_type(),
                  "biases must have the output dtype");
  const size_t ws_bytes = mi355moe_fused_moe_workspace_size(&a);
  auto ws = at::empty({static_cast<int64_t>(ws_bytes)},
                      hidden_states.options().dtype(at::kByte));
  DevGuard g(hidden_states.device());
  check_rc(mi355moe_fused_moe(&a, ws.data_ptr(), ws_bytes, cur_stream(hidden_states)),
           "fused_moe");
}

// Not a reference op: one-time K-blocked repacking of [E, N, K] weights into
// dst [E, K/B, N, B] (B = 32 for 16-bit, 128 for e4m3; XpuFusedMoe.__init__).
void mi355_pack_weights_kblock(const at::Tensor& src, at::Tensor& dst) {
  check_gpu(src, "src");
  check_gpu(dst, "dst");
  TORCH_CHECK(src.dim() == 3 && src.is_contiguous() && dst.is_contiguous(),
              "src must be a contiguous [E, N, K] tensor");
  TORCH_CHECK(dst.scalar_type() == src.scalar_type() && dst.numel() == src.numel(),
              "dst must match src in dtype and size");
  DevGuard g(src.device());
  const int dt = dtype_code(src.scalar_type());
  // packed e2m1 pairs: K counts values, two per byte
  const int64_t K = dt == MI355MOE_U8 ? 2 * src.size(2) : src.size(2);
  check_rc(mi355moe_pack_weights_kblock(src.data_ptr(), dst.data_ptr(), dt, src.size(0),
                                        src.size(1), K, cur_stream(src)),
           "pack_weights_kblock");
}

// Not a reference op: mxfp4 e8m0 scales u8 [E, N, K/32] -> [E, K/32, N].
void mi355_pack_scales_kblock(const at::Tensor& src, at::Tensor& dst) {
  check_gpu(src, "src");
  check_gpu(dst, "dst");
  TORCH_CHECK(src.dim() == 3 && src.is_contiguous() && dst.is_contiguous() &&
                  src.element_size() == 1 && dst.element_size() == 1 &&
                  dst.numel() == src.numel(),
              "src must be a contiguous byte [E, N, K/32] tensor and dst match it");
  DevGuard g(src.device());
  check_rc(mi355moe_pack_scales_kblock(src.data_ptr(), dst.data_ptr(), src.size(0),
                                       src.size(1), src.size(2), cur_stream(src)),
           "pack_scales_kblock");
}

}  // namespace

TORCH_LIBRARY(_moe_C, m) {
  m.def("moe_sum(Tensor input, Tensor! output, Tensor? topk_ids, Tensor? expert_map) -> ()");
  m.def("moe_align_block_size(Tensor topk_ids, int num_experts, int block_size, "
        "Tensor! sorted_token_ids, Tensor! experts_ids, Tensor! num_tokens_post_pad, "
        "Tensor? maybe_expert_map) -> ()");
  m.def("moe_lora_align_block_size(Tensor topk_ids, Tensor token_lora_mapping, int "
        "num_experts, int block_size, int max_loras, int max_num_tokens_padded, int "
        "max_num_m_blocks, Tensor! sorted_token_ids, Tensor! experts_ids, Tensor! "
        "num_tokens_post_pad, Tensor! adapter_enabled, Tensor! lora_ids, Tensor? "
        "maybe_expert_map) -> ()");
  m.def("grouped_topk(Tensor scores, Tensor scores_with_bias, int n_group, int "
        "topk_group, int topk, bool renormalize, float routed_scaling_factor) -> "
        "(Tensor, Tensor)");
  m.def("topk_softmax(Tensor! topk_weights, Tensor! topk_indices, Tensor! "
        "token_expert_indices, Tensor gating_output, bool renormalize, Tensor? "
        "bias) -> ()");
  m.def("topk_sigmoid(Tensor! topk_weights, Tensor! topk_indices, Tensor! "
        "token_expert_indices, Tensor gating_output, bool renormalize, Tensor? "
        "bias, float routed_scaling_factor) -> ()");
  m.def("topk_softplus_sqrt(Tensor! topk_weights, Tensor! topk_indices, "
        "Tensor! token_expert_indices, Tensor gating_output, bool renormalize, "
        "float routed_scaling_factor, Tensor? correction_bias=None, Tensor? "
        "input_ids=None, Tensor? tid2eid=None) -> ()");
  m.def("moe_gather(Tensor! output, Tensor moe_output, Tensor topk_weights, "
        "Tensor unpermuted_row_to_permuted_row, int num_experts) -> ()");
  m.def("fused_moe_prologue(Tensor input, Tensor? input_scales, Tensor "
        "token_selected_experts, Tensor token_final_scales, Tensor! workspace, int "
        "hidden_size, int inter_size, int block_k, int ep_rank, int ep_size,int "
        "num_experts_on_rank) -> ()");
  m.def("init_expert_map(Tensor! expert_map, int num_experts, int ep_rank, int "
        "ep_size) -> ()");
  m.def("remap_hidden_states(Tensor hidden_states, Tensor? hidden_states_scales, "
        "Tensor! remapped_hidden_states, Tensor(b!)? remapped_hidden_states_scales, "
        "Tensor? expert_map, Tensor! rows_per_expert, Tensor! "
        "unpermuted_row_to_permuted_row, Tensor topk_ids, int total_experts_num, "
        "int local_experts_num) -> ()");
  m.def("mi355_fused_moe(Tensor! output, Tensor hidden_states, Tensor topk_weights, "
        "Tensor topk_ids, Tensor w13, Tensor? w13_scale, Tensor? w13_bias, Tensor w2, "
        "Tensor? w2_scale, Tensor? w2_bias, int recipe, int activation, int "
        "inter_size, float clamp_limit, Tensor? expert_map, int w_layout=0, "
        "Tensor? hidden_scale=None, int w_group=0, int w13_scale_rows=0) -> ()");
  m.def("mi355_pack_weights_kblock(Tensor src, Tensor! dst) -> ()");
  m.def("mi355_fused_grouped_topk(Tensor gating_output, Tensor? bias, int n_group, "
        "int topk_group, int topk, bool renormalize, float routed_scaling_factor) -> "
        "(Tensor, Tensor)");
  m.def("mi355_pack_scales_kblock(Tensor src, Tensor! dst) -> ()");
}

TORCH_LIBRARY_IMPL(_moe_C, CUDA, m) {
  m.impl("moe_sum", &moe_sum);
  m.impl("moe_align_block_size", &moe_align_block_size);
  m.impl("moe_lora_align_block_size", &moe_lora_align_block_size);
  m.impl("grouped_topk", &grouped_topk);
  m.impl("topk_softmax", &topk_softmax);
  m.impl("topk_sigmoid", &topk_sigmoid);
  m.impl("topk_softplus_sqrt", &topk_softplus_sqrt);
  m.impl("moe_gather", &moe_gather);
  m.impl("fused_moe_prologue", &fused_moe_prologue);
  m.impl("init_expert_map", &init_expert_map);
  m.impl("remap_hidden_states", &remap_hidden_states);
  m.impl("mi355_fused_moe", &mi355_fused_moe);
  m.impl("mi355_pack_weights_kblock", &mi355_pack_weights_kblock);
  m.impl("mi355_fused_grouped_topk", &mi355_fused_grouped_topk);
  m.impl("mi355_pack_scales_kblock", &mi355_pack_scales_kblock);
}

TORCH_LIBRARY_IMPL(_moe_C, Meta, m) {
  m.impl("grouped_topk", &grouped_topk_meta);
  m.impl("mi355_fused_grouped_topk", &fused_grouped_topk_meta);
  for (const char* op : {"moe_sum", "moe_align_block_size", "moe_lora_align_block_size",
                         "topk_softmax", "topk_sigmoid", "topk_softplus_sqrt", "moe_gather",
                         "fused_moe_prologue", "init_expert_map", "remap_hidden_states",
                         "mi355_fused_moe", "mi355_pack_weights_kblock",
                         "mi355_pack_scales_kblock"})
    m.impl(op, torch::CppFunction::makeFromBoxedFunction<&meta_noop>());
}

TORCH_LIBRARY(_C, m) {
  m.def("silu_and_mul(Tensor! result, Tensor input) -> ()");
  m.def("swigluoai_and_mul(Tensor! out, Tensor input, float alpha=1.702, float "
        "limit=7.0) -> ()");
  m.def("per_token_group_fp8_quant(Tensor input, Tensor! output_q, Tensor! "
        "output_s, int group_size, float eps, float fp8_min, float fp8_max, bool "
        "scale_ue8m0, bool dummy_is_scale_transposed, bool dummy_is_tma_aligned ) "
        "-> ()");
  m.def("per_token_group_quant_mxfp4(Tensor input, Tensor! output_q, Tensor! "
        "output_s, int group_size, float eps) -> ()");
  m.def("gelu_and_mul(Tensor! out, Tensor input) -> ()");
  m.def("gelu_tanh_and_mul(Tensor! out, Tensor input) -> ()");
  m.def("relu2_no_mul(Tensor! out, Tensor! input) -> ()");
  m.def("swiglustep_and_mul(Tensor! out, Tensor input, float limit=7.0) -> ()");
  m.def("silu_and_mul_per_block_quant(Tensor! out, Tensor input, Tensor! scales, "
        "int group_size, Tensor? scale_ub=None, bool is_scale_transposed=False, "
        "bool scale_ue8m0=False) -> ()");
  m.def("silu_and_mul_mxfp4_quant(Tensor! out, Tensor input, Tensor! scales, "
        "int group_size, float eps=1e-10) -> ()");
}

TORCH_LIBRARY_IMPL(_C, CUDA, m) {
  m.impl("silu_and_mul", &silu_and_mul);
  m.impl("swigluoai_and_mul", &swigluoai_and_mul);
  m.impl("per_token_group_fp8_quant", &per_token_group_fp8_quant);
  m.impl("silu_and_mul_per_block_quant", &silu_and_mul_per_block_quant);
  m.impl("gelu_and_mul", &gelu_and_mul);
  m.impl("gelu_tanh_and_mul", &gelu_tanh_and_mul);
  m.impl("relu2_no_mul", &relu2_no_mul);
  m.impl("swiglustep_and_mul", &swiglustep_and_mul);
  m.impl("silu_and_mul_mxfp4_quant", &silu_and_mul_mxfp4_quant);
  m.impl("per_token_group_quant_mxfp4", &per_token_group_quant_mxfp4);
}

TORCH_LIBRARY_IMPL(_C, Meta, m) {
  for (const char* op : {"silu_and_mul", "swigluoai_and_mul", "per_token_group_fp8_quant",
                         "silu_and_mul_per_block_quant", "gelu_and_mul", "gelu_tanh_and_mul",
                         "relu2_no_mul", "swiglustep_and_mul", "silu_and_mul_mxfp4_quant",
                         "per_token_group_quant_mxfp4"})
    m.impl(op, torch::CppFunction::makeFromBoxedFunction<&meta_noop>());
}

TORCH_LIBRARY(_xpu_C, m) {
  // the reference's schema (csrc/xpu/torch_bindings.cpp:46-49) with the write
  // to ptr_D, and the returned alias of it, annotated
  m.def("cutlass_grouped_gemm_interface(Tensor ptr_A, Tensor? ptr_A_scale, "
        "Tensor ptr_B, Tensor? ptr_B_scale, Tensor? ptr_bias, Tensor(a!) ptr_D, "
        "Tensor rows_per_expert, int N, int K, int num_experts) -> Tensor(a!)");
}

TORCH_LIBRARY_IMPL(_xpu_C, CUDA, m) {
  m.impl("cutlass_grouped_gemm_interface", &cutlass_grouped_gemm_interface);
}

TORCH_LIBRARY_IMPL(_xpu_C, Meta, m) {
  m.impl("cutlass_grouped_gemm_interface", &grouped_gemm_meta);
}
