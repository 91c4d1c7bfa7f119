"""Allocating Python wrappers over the registered ops.

They mirror the caller-side helpers vLLM and the reference tests use
(reference tests/ops/topk_op.py:62-147, tests/ops/grouped_topk_op.py:67-92,
tests/ops/moe_align_block_size_ops.py:14-100), so code written against the
reference can swap the import.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _ops  # noqa: F401

FP8_E4M3_MAX = 448.0


def topk_softmax(gating_output: torch.Tensor, topk: int, renormalize: bool,
                 bias: Optional[torch.Tensor] = None,
                 indices_type: Optional[torch.dtype] = None):
    T = gating_output.shape[0]
    dev = gating_output.device
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=indices_type or torch.int32, device=dev)
    tei = torch.empty(T, topk, dtype=torch.int32, device=dev)
    torch.ops._moe_C.topk_softmax(w, ids, tei, gating_output, renormalize, bias)
    return w, ids, tei


def topk_sigmoid(gating_output: torch.Tensor, topk: int, renormalize: bool,
                 bias: Optional[torch.Tensor] = None,
                 indices_type: Optional[torch.dtype] = None,
                 routed_scaling_factor: float = 1.0):
    T = gating_output.shape[0]
    dev = gating_output.device
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=indices_type or torch.int32, device=dev)
    tei = torch.empty(T, topk, dtype=torch.int32, device=dev)
    torch.ops._moe_C.topk_sigmoid(w, ids, tei, gating_output, renormalize, bias,
                                  routed_scaling_factor)
    return w, ids, tei


def topk_softplus_sqrt(gating_output: torch.Tensor, topk: int, renormalize: bool,
                       routed_scaling_factor: float = 1.0,
                       correction_bias: Optional[torch.Tensor] = None,
                       input_ids: Optional[torch.Tensor] = None,
                       tid2eid: Optional[torch.Tensor] = None):
    """sqrt(softplus) routing (reference csrc/moe/torch_bindings.cpp:70-76);
    returns (weights f32 [T, k], ids i32 [T, k])."""
    T = gating_output.shape[0]
    w = torch.empty(T, topk, dtype=torch.float32, device=gating_output.device)
    ids = torch.empty(T, topk, dtype=torch.int32, device=gating_output.device)
    src = torch.empty(T, topk, dtype=torch.int32, device=gating_output.device)
    torch.ops._moe_C.topk_softplus_sqrt(w, ids, src, gating_output, renormalize,
                                        routed_scaling_factor, correction_bias, input_ids,
                                        tid2eid)
    return w, ids


def grouped_topk(scores: torch.Tensor, scores_with_bias: torch.Tensor,
                 n_group: int, topk_group: int, topk: int, renormalize: bool,
                 routed_scaling_factor: float = 1.0):
    return torch.ops._moe_C.grouped_topk(scores, scores_with_bias, n_group,
                                         topk_group, topk, renormalize,
                                         routed_scaling_factor)


def fused_grouped_topk(gating_output: torch.Tensor, topk: int,
                       renormalize: bool,
                       e_score_correction_bias: torch.Tensor,
                       num_expert_group: int, topk_group: int,
                       scoring_func: str = "sigmoid",
                       routed_scaling_factor: float = 1.0):
    """Score function + correction bias + grouped top-k (reference
    tests/ops/grouped_topk_op.py:67-92).  "sigmoid" runs as one kernel that
    forms scores and scores_with_bias itself (the same per-element roundings
    as the torch ops); "softmax" keeps the caller-side torch.softmax.  Both
    take e_score_correction_bias=None as no correction (selection on the
    scores themselves); the reference requires a bias."""
    if scoring_func == "sigmoid":
        bias = e_score_correction_bias
        if bias is not None:
            bias = bias.to(torch.float32).contiguous()
        v, i = torch.ops._moe_C.mi355_fused_grouped_topk(
            gating_output.contiguous(), bias, num_expert_group, topk_group, topk,
            renormalize, routed_scaling_factor)
        return v.to(torch.float32), i
    if scoring_func == "softmax":
        scores = torch.softmax(gating_output, dim=-1)
    else:
        raise ValueError(f"Unsupported scoring function: {scoring_func}")
    swb = (scores if e_score_correction_bias is None
           else scores + e_score_correction_bias.unsqueeze(0))
    v, i = grouped_topk(scores, swb.to(scores.dtype), num_expert_group,
                        topk_group, topk, renormalize, routed_scaling_factor)
    return v.to(torch.float32), i


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def align_buffer_sizes(numel: int, num_experts: int, block_size: int,
                       pad_sorted_ids: bool = False):
    mx = numel + num_experts * (block_size - 1)
    if pad_sorted_ids:
        mx = _round_up(mx, block_size)
    if numel < num_experts:
        mx = min(numel * block_size, mx)
    return mx, (mx + block_size - 1) // block_size


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int,
                         num_experts: int,
                         expert_map: Optional[torch.Tensor] = None,
                         pad_sorted_ids: bool = False,
                         ignore_invalid_experts: bool = False):
    mx, nb = align_buffer_sizes(topk_ids.numel(), num_experts, block_size,
                                pad_sorted_ids)
    dev = topk_ids.device
    sorted_ids = torch.empty(mx, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(nb, dtype=torch.int32, device=dev)
    ntp = torch.empty(1, dtype=torch.int32, device=dev)
    torch.ops._moe_C.moe_align_block_size(
        topk_ids, num_experts, block_size, sorted_ids, expert_ids, ntp,
        expert_map if ignore_invalid_experts else None)
    if expert_map is not None and not ignore_invalid_experts:
        expert_ids = expert_map[expert_ids]
    return sorted_ids, expert_ids, ntp


def moe_lora_align_block_size(topk_ids: torch.Tensor,
                              token_lora_mapping: torch.Tensor,
                              num_experts: int, block_size: int, max_loras: int,
                              max_num_tokens_padded: int, max_num_m_blocks: int,
                              sorted_token_ids: torch.Tensor,
                              experts_ids: torch.Tensor,
                              num_tokens_post_pad: torch.Tensor,
                              adapter_enabled: torch.Tensor,
                              lora_ids: torch.Tensor,
                              expert_map: Optional[torch.Tensor] = None) -> None:
    torch.ops._moe_C.moe_lora_align_block_size(
        topk_ids, token_lora_mapping, num_experts, block_size, max_loras,
        max_num_tokens_padded, max_num_m_blocks, sorted_token_ids, experts_ids,
        num_tokens_post_pad, adapter_enabled, lora_ids, expert_map)


def fused_moe_prologue(input: torch.Tensor, input_scales: Optional[torch.Tensor],
                       token_selected_experts: torch.Tensor,
                       token_final_scales: torch.Tensor, workspace: torch.Tensor,
                       hidden_size: int, inter_size: int, block_k: int,
                       ep_rank: int, ep_size: int, num_experts_on_rank: int) -> None:
    torch.ops._moe_C.fused_moe_prologue(
        input, input_scales, token_selected_experts, token_final_scales, workspace,
        hidden_size, inter_size, block_k, ep_rank, ep_size, num_experts_on_rank)


def moe_sum(inp: torch.Tensor, out: torch.Tensor,
            topk_ids: Optional[torch.Tensor] = None,
            expert_map: Optional[torch.Tensor] = None) -> None:
    torch.ops._moe_C.moe_sum(inp, out, topk_ids, expert_map)


def moe_gather(out: torch.Tensor, moe_output: torch.Tensor,
               topk_weights: torch.Tensor, perm: torch.Tensor,
               num_experts: int) -> None:
    torch.ops._moe_C.moe_gather(out, moe_output, topk_weights, perm,
                                num_experts)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    d = x.shape[-1] // 2
    out = torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)
    torch.ops._C.silu_and_mul(out, x)
    return out


def swigluoai_and_mul(x: torch.Tensor, alpha: float = 1.702,
                      limit: float = 7.0) -> torch.Tensor:
    d = x.shape[-1] // 2
    out = torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)
    torch.ops._C.swigluoai_and_mul(out, x, alpha, limit)
    return out


def gelu_and_mul(x: torch.Tensor) -> torch.Tensor:
    out = torch.empty(x.shape[:-1] + (x.shape[-1] // 2,), dtype=x.dtype, device=x.device)
    torch.ops._C.gelu_and_mul(out, x)
    return out


def gelu_tanh_and_mul(x: torch.Tensor) -> torch.Tensor:
    out = torch.empty(x.shape[:-1] + (x.shape[-1] // 2,), dtype=x.dtype, device=x.device)
    torch.ops._C.gelu_tanh_and_mul(out, x)
    return out


def swiglustep_and_mul(x: torch.Tensor, limit: float = 7.0) -> torch.Tensor:
    out = torch.empty(x.shape[:-1] + (x.shape[-1] // 2,), dtype=x.dtype, device=x.device)
    torch.ops._C.swiglustep_and_mul(out, x, limit)
    return out


def relu2_no_mul(x: torch.Tensor) -> torch.Tensor:
    out = torch.empty_like(x)
    torch.ops._C.relu2_no_mul(out, x)
    return out


def per_token_group_fp8_quant(x: torch.Tensor, group_size: int = 128,
                              eps: float = 1e-10,
                              scale_ue8m0: bool = False):
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(x.shape[:-1] + (x.shape[-1] // group_size,),
                    dtype=torch.float32, device=x.device)
    torch.ops._C.per_token_group_fp8_quant(x, q, s, group_size, eps,
                                           -FP8_E4M3_MAX, FP8_E4M3_MAX,
                                           scale_ue8m0, False, False)
    return q, s


def per_token_group_quant_mxfp4(x: torch.Tensor, group_size: int = 32,
                                eps: float = 1e-10):
    M, N = x.shape
    q = torch.empty(M, N // 2, dtype=torch.uint8, device=x.device)
    s = torch.empty(M, N // group_size, dtype=torch.float32, device=x.device)
    torch.ops._C.per_token_group_quant_mxfp4(x, q, s, group_size, eps)
    return q.view(torch.float4_e2m1fn_x2), s


def silu_and_mul_per_block_quant(input: torch.Tensor, group_size: int,
                                 quant_dtype: torch.dtype,
                                 scale_ub: Optional[torch.Tensor] = None,
                                 is_scale_transposed: bool = False,
                                 scale_ue8m0: bool = False):
    """silu(gate) * up fused with per-group dynamic quantisation to
    float8_e4m3fn / float8_e5m2 / int8 (reference tests/register_ops.py:34-74
    allocation, csrc/torch_bindings.cpp:88-101 op).  Returns (out [T, H],
    scales [T, H/group_size]; a transposed view when is_scale_transposed)."""
    T, H = input.shape[0], input.shape[-1] // 2
    G = H // group_size
    out = torch.empty((T, H), dtype=quant_dtype, device=input.device)
    if is_scale_transposed:
        scales = torch.empty((G, T), dtype=torch.float32, device=input.device).t()
    else:
        scales = torch.empty((T, G), dtype=torch.float32, device=input.device)
    torch.ops._C.silu_and_mul_per_block_quant(out, input, scales, group_size,
                                              scale_ub, is_scale_transposed,
                                              scale_ue8m0)
    return out, scales


def silu_and_mul_mxfp4_quant(input: torch.Tensor, group_size: int = 32,
                             eps: float = 1e-10):
    """silu(gate) * up fused with mxfp4 quantisation (csrc/torch_bindings.cpp:
    103-107).  Returns (packed e2m1 uint8 [T, H/2], float32 power-of-two
    scales [T, H/32])."""
    T, H = input.shape[0], input.shape[-1] // 2
    out = torch.empty((T, H // 2), dtype=torch.uint8, device=input.device)
    scales = torch.empty((T, H // group_size), dtype=torch.float32, device=input.device)
    torch.ops._C.silu_and_mul_mxfp4_quant(out, input, scales, group_size, eps)
    return out, scales


def init_expert_map(num_experts: int, ep_rank: int, ep_size: int,
                    device) -> torch.Tensor:
    m = torch.empty(num_experts * ep_size, dtype=torch.int32, device=device)
    torch.ops._moe_C.init_expert_map(m, num_experts, ep_rank, ep_size)
    return m


def remap_hidden_states(hidden_states: torch.Tensor, topk_ids: torch.Tensor,
                        total_experts_num: int, local_experts_num: int,
                        expert_map: Optional[torch.Tensor] = None,
                        hidden_states_scales: Optional[torch.Tensor] = None):
    T, k = topk_ids.shape
    dev = hidden_states.device
    remapped = torch.empty((T * k,) + tuple(hidden_states.shape[1:]),
                           dtype=hidden_states.dtype, device=dev)
    rscales = None
    if hidden_states_scales is not None:
        rscales = torch.empty((T * k,) + tuple(hidden_states_scales.shape[1:]),
                              dtype=hidden_states_scales.dtype, device=dev)
    rows = torch.zeros(local_experts_num, dtype=torch.int32, device=dev)
    perm = torch.empty(T, k, dtype=torch.int32, device=dev)
    torch.ops._moe_C.remap_hidden_states(hidden_states, hidden_states_scales,
                                         remapped, rscales, expert_map, rows,
                                         perm, topk_ids, total_experts_num,
                                         local_experts_num)
    return remapped, rscales, rows, perm


def cutlass_grouped_gemm(ptr_A: torch.Tensor, ptr_B: torch.Tensor,
                         ptr_B_scale: Optional[torch.Tensor],
                         ptr_bias: Optional[torch.Tensor], ptr_D: torch.Tensor,
                         rows_per_expert: torch.Tensor, N: int, K: int,
                         num_experts: int,
                         ptr_A_scale: Optional[torch.Tensor] = None):
    return torch.ops._xpu_C.cutlass_grouped_gemm_interface(
        ptr_A, ptr_A_scale, ptr_B, ptr_B_scale, ptr_bias, ptr_D,
        rows_per_expert, N, K, num_experts)
