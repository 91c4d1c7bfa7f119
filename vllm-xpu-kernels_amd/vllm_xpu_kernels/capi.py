"""ctypes binding of the fused-layer C ABI (include/mi355moe.h).

This is the binding a non-torch host (or a maintainer wiring the library
into another runtime) would write; ``bench.py`` uses it for the stage-timed
entry point.  Pointers come from ``tensor.data_ptr()`` and the stream from
``torch.cuda.current_stream().cuda_stream``.
"""
from __future__ import annotations

import ctypes

import torch

from ._ops import lib

F32, BF16, F16, I32, I64 = 0, 1, 2, 3, 4
FUSED_STAGES = 5
STAGE_NAMES = ("align", "act_quant", "gemm_w13", "gemm_w2", "topk_reduce")


class FusedMoeArgs(ctypes.Structure):
    _fields_ = [("recipe", ctypes.c_int), ("activation", ctypes.c_int),
                ("act_dtype", ctypes.c_int), ("ids_dtype", ctypes.c_int),
                ("num_tokens", ctypes.c_int64), ("hidden", ctypes.c_int64),
                ("inter", ctypes.c_int64), ("num_experts", ctypes.c_int64),
                ("topk", ctypes.c_int64), ("hidden_states", ctypes.c_void_p),
                ("topk_weights", ctypes.c_void_p), ("topk_ids", ctypes.c_void_p),
                ("expert_map", ctypes.c_void_p), ("expert_map_len", ctypes.c_int64),
                ("w13", ctypes.c_void_p), ("w13_scale", ctypes.c_void_p),
                ("w13_bias", ctypes.c_void_p), ("w2", ctypes.c_void_p),
                ("w2_scale", ctypes.c_void_p), ("w2_bias", ctypes.c_void_p),
                ("gemm1_clamp_limit", ctypes.c_float),
                ("swiglu_alpha", ctypes.c_float),
                ("swiglu_limit", ctypes.c_float), ("output", ctypes.c_void_p),
                ("w_layout", ctypes.c_int),
                ("hidden_scale", ctypes.c_void_p),
                ("w_group", ctypes.c_int64),
                ("w13_scale_rows", ctypes.c_int64)]


lib.mi355moe_fused_moe_workspace_size.restype = ctypes.c_size_t
lib.mi355moe_fused_moe_workspace_size.argtypes = [ctypes.POINTER(FusedMoeArgs)]
lib.mi355moe_fused_moe.argtypes = [ctypes.POINTER(FusedMoeArgs), ctypes.c_void_p,
                                   ctypes.c_size_t, ctypes.c_void_p]
lib.mi355moe_fused_moe_timed.argtypes = [ctypes.POINTER(FusedMoeArgs),
                                         ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int]
lib.mi355moe_timer_create.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
lib.mi355moe_timer_destroy.argtypes = [ctypes.c_void_p]
lib.mi355moe_timer_stage_ms.argtypes = [ctypes.c_void_p, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float)]


lib.mi355moe_fused_moe_prologue_workspace_layout.restype = ctypes.c_size_t
lib.mi355moe_fused_moe_prologue_workspace_layout.argtypes = (
    [ctypes.c_int64] * 7 + [ctypes.POINTER(ctypes.c_size_t)] * 2)

PROLOGUE_SECTIONS = ("permuted_row_to_unpermuted_row", "permuted_token_selected_experts",
                     "unpermuted_row_to_permuted_row", "blocked_expert_counts",
                     "blocked_expert_counts_cumsum", "blocked_row_to_unpermuted_row",
                     "expert_first_token_offset", "permuted_token_final_scales",
                     "overlapped_gemm1_gemm2_inputs", "permuted_act_scales")


def prologue_layout(num_rows: int, experts_per_token: int, hidden_size: int,
                    elem_bytes: int, block_k: int, scale_bytes: int,
                    num_experts_on_rank: int) -> tuple[int, dict]:
    """Total bytes and {section: (padded size, offset)} of the
    fused_moe_prologue workspace (the reference's ``ws_map``)."""
    off = (ctypes.c_size_t * len(PROLOGUE_SECTIONS))()
    size = (ctypes.c_size_t * len(PROLOGUE_SECTIONS))()
    total = lib.mi355moe_fused_moe_prologue_workspace_layout(
        num_rows, experts_per_token, hidden_size, elem_bytes, block_k, scale_bytes,
        num_experts_on_rank, off, size)
    if total == 0:
        raise ValueError("invalid fused_moe_prologue sizes")
    return int(total), {n: (int(size[i]), int(off[i]))
                        for i, n in enumerate(PROLOGUE_SECTIONS)}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {lib.mi355moe_last_error().decode()}")


def fused_args(moe, output, hidden_states, topk_weights, topk_ids,
               expert_map=None, hidden_scale=None) -> FusedMoeArgs:
    """Arguments for an XpuFusedMoe's prepared weights (hidden_scale:
    hidden_states pre-quantised, its scales as XpuFusedMoe.apply takes them
    after conversion: f32 for fp8block, e8m0 bytes for mxfp8 / mxfp4, whose
    hidden_states are then packed e2m1 bytes [T, H/2])."""
    a = FusedMoeArgs()
    recipe, w13, w2, layout = moe._call_plan(hidden_states.dtype)
    a.recipe = recipe
    a.activation = moe._act
    a.act_dtype = F16 if output.dtype == torch.float16 else BF16
    b13, b2 = moe._biases(output.dtype)
    s13, s2 = moe._scales(hidden_states.dtype)
    a.ids_dtype = I64 if topk_ids.dtype == torch.int64 else I32
    a.num_tokens, a.hidden = hidden_states.shape
    if hidden_scale is not None:
        a.hidden_scale = hidden_scale.data_ptr()
        if moe.recipe.startswith("mxfp4"):
            a.hidden *= 2
    a.inter = moe.inter_size
    a.num_experts = moe.w13.shape[0]
    a.topk = topk_ids.shape[1]
    a.hidden_states = hidden_states.data_ptr()
    a.topk_weights = topk_weights.data_ptr()
    a.topk_ids = topk_ids.data_ptr()
    a.expert_map = expert_map.data_ptr() if expert_map is not None else None
    a.expert_map_len = expert_map.numel() if expert_map is not None else 0
    a.w13 = w13.data_ptr()
    a.w13_scale = s13.data_ptr() if s13 is not None else None
    a.w13_bias = b13.data_ptr() if b13 is not None else None
    a.w2 = w2.data_ptr()
    a.w2_scale = s2.data_ptr() if s2 is not None else None
    a.w2_bias = b2.data_ptr() if b2 is not None else None
    a.gemm1_clamp_limit = float(moe.gemm1_clamp_limit or 0.0)
    a.swiglu_alpha = 1.702
    a.swiglu_limit = 7.0
    a.output = output.data_ptr()
    a.w_layout = layout
    a.w_group = moe._w_group
    a.w13_scale_rows = moe._ws_rows
    return a


class StageTimer:
    """HIP-event timer of the five fused stages over `steps` calls."""

    def __init__(self, steps: int):
        self.steps = steps
        self.h = ctypes.c_void_p()
        _check(lib.mi355moe_timer_create(steps, ctypes.byref(self.h)), "timer_create")

    def run(self, args: FusedMoeArgs, ws: torch.Tensor, step: int) -> None:
        stream = torch.cuda.current_stream().cuda_stream
        _check(lib.mi355moe_fused_moe_timed(ctypes.byref(args), _p(ws), ws.numel(),
                                            ctypes.c_void_p(stream), self.h, step),
               "fused_moe_timed")

    def stage_ms(self, step: int) -> list[float]:
        buf = (ctypes.c_float * FUSED_STAGES)()
        _check(lib.mi355moe_timer_stage_ms(self.h, step, buf), "timer_stage_ms")
        return list(buf)

    def close(self) -> None:
        if self.h:
            lib.mi355moe_timer_destroy(self.h)
            self.h = ctypes.c_void_p()


def workspace_for(args: FusedMoeArgs, device) -> torch.Tensor:
    n = lib.mi355moe_fused_moe_workspace_size(ctypes.byref(args))
    return torch.empty(int(n), dtype=torch.uint8, device=device)
