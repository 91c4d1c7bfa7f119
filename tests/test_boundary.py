"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/mi355moe.h declares, rejects invalid arguments before any
device work, and the torch op schemas match the reference verbatim."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi355moe.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mi355moe_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from vllm_xpu_kernels import _ops
    return _ops.lib


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n


def test_version_and_error_plumbing(lib):
    assert lib.mi355moe_version() == 1
    rc = lib.mi355moe_moe_sum(None, None, 1, ctypes.c_int64(4), ctypes.c_int64(2),
                              ctypes.c_int64(8), None, 3, ctypes.c_void_p(16),
                              ctypes.c_int64(4), None)
    assert rc == -1
    assert b"expert_map requires topk_ids" in lib.mi355moe_last_error()


@pytest.mark.parametrize("call,msg", [
    (lambda L: L.mi355moe_topk_softmax(None, None, 3, None, None, 0,
                                       ctypes.c_int64(4), ctypes.c_int64(8),
                                       ctypes.c_int64(9), 1, None, None),
     b"topk must be in"),
    (lambda L: L.mi355moe_topk_softmax(None, None, 3, None, None, 0,
                                       ctypes.c_int64(4), ctypes.c_int64(2048),
                                       ctypes.c_int64(2), 1, None, None),
     b"num_experts > 1024"),
    (lambda L: L.mi355moe_grouped_topk(None, None, None, None, 0, ctypes.c_int64(4),
                                       ctypes.c_int64(256), ctypes.c_int64(33),
                                       ctypes.c_int64(4), ctypes.c_int64(8), 1,
                                       ctypes.c_float(1.0), None),
     b"n_group"),
    (lambda L: L.mi355moe_moe_align_block_size(None, 3, ctypes.c_int64(8),
                                               ctypes.c_int64(1024), ctypes.c_int64(16),
                                               None, ctypes.c_int64(0), None,
                                               ctypes.c_int64(0), None, None, None,
                                               ctypes.c_size_t(0), None),
     b"padded_num_experts must be less than 1024"),
    (lambda L: L.mi355moe_moe_lora_align_block_size(
        None, 3, ctypes.c_int64(8), ctypes.c_int64(2), None, ctypes.c_int64(64),
        ctypes.c_int64(0), ctypes.c_int64(2), ctypes.c_int64(0), ctypes.c_int64(0), None, None,
        None, None, None, ctypes.c_int64(3), None, None),
     b"block_size should be greater than 0"),
    (lambda L: L.mi355moe_per_token_group_fp8_quant(None, 1, None, None,
                                                    ctypes.c_int64(2), ctypes.c_int64(100),
                                                    ctypes.c_int64(128), ctypes.c_float(1e-10),
                                                    ctypes.c_float(-448), ctypes.c_float(448),
                                                    0, None),
     b"divisible by group_size"),
    (lambda L: L.mi355moe_grouped_gemm(1, None, 1, None, None, None, None, None, 1, None,
                                       ctypes.c_int64(4), ctypes.c_int64(204),
                                       ctypes.c_int64(256), ctypes.c_int64(2), None,
                                       ctypes.c_size_t(0), None),
     b"N must be a multiple of 8"),
    (lambda L: L.mi355moe_grouped_gemm(1, None, 1, None, None, None, None, None, 1, None,
                                       ctypes.c_int64(4), ctypes.c_int64(192),
                                       ctypes.c_int64(256), ctypes.c_int64(2), None,
                                       ctypes.c_size_t(0), None),
     b"% 128"),
    (lambda L: L.mi355moe_pack_weights_kblock(None, None, 1, ctypes.c_int64(2),
                                              ctypes.c_int64(64), ctypes.c_int64(48), None),
     b"K % 32 == 0"),
    (lambda L: L.mi355moe_pack_weights_kblock(None, None, 6, ctypes.c_int64(2),
                                              ctypes.c_int64(64), ctypes.c_int64(96), None),
     b"K % 128 == 0 (e4m3)"),
    (lambda L: L.mi355moe_pack_weights_kblock(None, None, 0, ctypes.c_int64(2),
                                              ctypes.c_int64(64), ctypes.c_int64(64), None),
     b"16-bit, e4m3 or packed e2m1"),
    (lambda L: L.mi355moe_pack_weights_kblock(None, None, 7, ctypes.c_int64(2),
                                              ctypes.c_int64(64), ctypes.c_int64(48), None),
     b"K % 32 == 0 (16-bit, e2m1)"),
    (lambda L: L.mi355moe_pack_scales_kblock(None, None, ctypes.c_int64(2),
                                             ctypes.c_int64(64), ctypes.c_int64(0), None),
     b"positive sizes"),
    (lambda L: L.mi355moe_silu_and_mul_per_block_quant(
        None, 6, None, 1, None, ctypes.c_int64(2), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(96), ctypes.c_int64(48), None, 0, None),
     b"group_size must be 32, 64, or 128"),
    (lambda L: L.mi355moe_silu_and_mul_per_block_quant(
        None, 1, None, 1, None, ctypes.c_int64(2), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(128), ctypes.c_int64(64), None, 0, None),
     b"out must be float8_e4m3fn, float8_e5m2, or int8"),
    (lambda L: L.mi355moe_silu_and_mul_per_block_quant(
        None, 10, None, 1, None, ctypes.c_int64(2), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(128), ctypes.c_int64(64), ctypes.c_void_p(256), 0, None),
     b"scale_ub is only supported for FP8 output"),
    (lambda L: L.mi355moe_silu_and_mul_per_block_quant(
        None, 9, None, 2, None, ctypes.c_int64(3), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(96), ctypes.c_int64(64), None, 0, None),
     b"hidden_size must be divisible by group_size"),
    (lambda L: L.mi355moe_silu_and_mul_per_block_quant(
        None, 6, None, 0, None, ctypes.c_int64(2), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(128), ctypes.c_int64(64), None, 0, None),
     b"input must be float16 or bfloat16"),
    (lambda L: L.mi355moe_silu_and_mul_mxfp4_quant(
        None, None, 1, None, ctypes.c_int64(2), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(128), ctypes.c_int64(64), ctypes.c_float(1e-10), None),
     b"MXFP4 requires group_size == 32"),
    (lambda L: L.mi355moe_topk_softplus_sqrt(None, None, 3, None, None, 0, ctypes.c_int64(4),
                                             ctypes.c_int64(100), ctypes.c_int64(8), 1,
                                             ctypes.c_float(1.0), None, None, None, None),
     b"Unsupported expert number"),
    (lambda L: L.mi355moe_topk_softplus_sqrt(None, None, 3, None, None, 0, ctypes.c_int64(4),
                                             ctypes.c_int64(256), ctypes.c_int64(8), 1,
                                             ctypes.c_float(1.0), None, None,
                                             ctypes.c_void_p(64), None),
     b"input_ids is required for hash MoE"),
    (lambda L: L.mi355moe_gelu_and_mul(None, None, 3, ctypes.c_int64(2), ctypes.c_int64(8), None),
     b"gelu_and_mul: unsupported dtype"),
    (lambda L: L.mi355moe_swiglustep_and_mul(None, None, 4, ctypes.c_int64(2), ctypes.c_int64(8),
                                             ctypes.c_float(7.0), None),
     b"swiglustep_and_mul: unsupported dtype"),
    (lambda L: L.mi355moe_relu2_no_mul(None, None, 7, ctypes.c_int64(2), ctypes.c_int64(8), None),
     b"relu2_no_mul: unsupported dtype"),
    (lambda L: L.mi355moe_silu_and_mul_mxfp4_quant(
        None, None, 1, None, ctypes.c_int64(4), ctypes.c_int64(1), ctypes.c_int64(4),
        ctypes.c_int64(128), ctypes.c_int64(32), ctypes.c_float(0.0), None),
     b"eps must be a normal float"),
])
def test_invalid_arguments_rejected_before_launch(lib, call, msg):
    rc = call(lib)
    assert rc < 0
    assert msg in lib.mi355moe_last_error()


@pytest.mark.parametrize("T,k,hidden,eb,bk,sb,E", [
    (1, 1, 128, 2, 1, 0, 2), (16, 2, 8192, 1, 128, 4, 16), (8192, 2, 8192, 1, 32, 1, 16),
    (3000, 8, 7168, 1, 128, 4, 256), (5, 3, 100, 2, 1, 0, 1000)])
def test_prologue_layout_matches_oracle(T, k, hidden, eb, bk, sb, E):
    """The C ABI's workspace layout (host-only) is the reference's byte layout."""
    from oracle import moe_oracle as O
    from vllm_xpu_kernels import capi
    total, ws = capi.prologue_layout(T, k, hidden, eb, bk, sb, E)
    assert (total, ws) == O.prologue_layout(T, k, hidden, eb, bk, sb, E)


def test_prologue_argument_validation(lib):
    lib.mi355moe_fused_moe_prologue.argtypes = (
        [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t] +
        [ctypes.c_int64] * 8 + [ctypes.c_void_p])

    def call(ws_bytes=1 << 20, E=16, rank=0, size=1, eb=2, sb=0, bk=1, hidden=256):
        return lib.mi355moe_fused_moe_prologue(16, eb, 16 if sb else None, sb, 16, 4, 16, 16,
                                               ws_bytes, 4, hidden, 512, bk, 2, rank, size, E,
                                               None)
    assert call(rank=2, size=2) == -1 and b"ep_rank" in lib.mi355moe_last_error()
    assert call(E=1025) == -1 and b"num_experts_on_rank" in lib.mi355moe_last_error()
    assert call(eb=4) == -1 and b"1- or 2-byte" in lib.mi355moe_last_error()
    assert call(eb=1, sb=4, bk=100) == -1 and b"block_k" in lib.mi355moe_last_error()
    assert call(ws_bytes=1024) == -1 and b"smaller than the prologue" in lib.mi355moe_last_error()


def test_fused_moe_workspace_query_and_validation(lib):
    from vllm_xpu_kernels import _ops  # noqa: F401

    class Args(ctypes.Structure):
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
                    ("gemm1_clamp_limit", ctypes.c_float), ("swiglu_alpha", ctypes.c_float),
                    ("swiglu_limit", ctypes.c_float), ("output", ctypes.c_void_p),
                    ("w_layout", ctypes.c_int),
                    ("hidden_scale", ctypes.c_void_p),
                    ("w_group", ctypes.c_int64), ("w13_scale_rows", ctypes.c_int64)]

    a = Args(recipe=1, activation=0, act_dtype=1, ids_dtype=3, num_tokens=64,
             hidden=7168, inter=2048, num_experts=256, topk=8)
    # this struct, not the ctypes binding's (which may have set argtypes;
    # restored at the end)
    saved = (lib.mi355moe_fused_moe_workspace_size.argtypes, lib.mi355moe_fused_moe.argtypes)
    lib.mi355moe_fused_moe_workspace_size.argtypes = None
    lib.mi355moe_fused_moe.argtypes = None
    try:
        _workspace_query_checks(lib, a)
    finally:
        lib.mi355moe_fused_moe_workspace_size.argtypes, lib.mi355moe_fused_moe.argtypes = saved


def _workspace_query_checks(lib, a):
    lib.mi355moe_fused_moe_workspace_size.restype = ctypes.c_size_t
    ws = lib.mi355moe_fused_moe_workspace_size(ctypes.byref(a))
    assert ws > 64 * 7168
    a.hidden = 7100
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"% 128" in lib.mi355moe_last_error()
    a.hidden = 7168
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"need scales" in lib.mi355moe_last_error()
    # fp8block w13 scale rows: 128 weight rows per scale row, or 64 (the split
    # swigluoai layout)
    a.w13_scale = a.w2_scale = 1
    a.w13_scale_rows = 96
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"w13_scale_rows" in lib.mi355moe_last_error()
    for rows in (0, 64, 128):
        a.w13_scale_rows = rows
        rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
        assert rc == -4 and b"workspace" in lib.mi355moe_last_error()
    a.w13_scale_rows = 0
    a.w13_scale = a.w2_scale = None
    # the K-blocked layout: bf16 with K % 32 == 0 or fp8block with K <= 8192
    a.w_layout = 1
    a.w13_scale = a.w2_scale = 1
    a.hidden = 8320
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"K-blocked weights need the bf16 recipe" in lib.mi355moe_last_error()
    a.recipe, a.hidden = 0, 7176
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"K-blocked weights need the bf16 recipe" in lib.mi355moe_last_error()
    a.w_layout = 7
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"unknown weight layout" in lib.mi355moe_last_error()
    a.w_layout, a.activation = 0, 6
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"unsupported activation" in lib.mi355moe_last_error()
    a.activation = 0
    # caller-quantised hidden states: fp8block and the MX recipes only
    a.w_layout, a.hidden_scale = 0, 64
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"need the fp8block, mxfp8 or mxfp4" in lib.mi355moe_last_error()
    a.hidden_scale = None
    # per-expert fp8 weights read as fp8 (recipes 5 / 6): sizes % 32 == 0
    # (else MI355MOE_ERR_UNSUPPORTED: the layer then runs on 16-bit copies),
    # any call size and either layout (these calls pass validation and stop
    # at the missing workspace)
    for recipe in (5, 6):
        a.recipe, a.hidden, a.num_tokens = recipe, 7168, 64
        a.w13_scale = a.w2_scale = None
        rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
        assert rc == -1 and b"f32 scales [E]" in lib.mi355moe_last_error()
        a.w13_scale = a.w2_scale = 1
        a.hidden = 7160
        rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
        assert rc == -2 and b"% 32 == 0" in lib.mi355moe_last_error()
        for T, layout in ((4096, 0), (64, 1), (4096, 1)):
            a.hidden, a.num_tokens, a.w_layout = 7200, T, layout
            rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
            assert rc == -4 and b"workspace" in lib.mi355moe_last_error()
        a.w_layout, a.hidden, a.num_tokens = 0, 7168, 64
    a.recipe = 7
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and b"unknown recipe" in lib.mi355moe_last_error()


# schema strings as written in the reference's registration files
# (csrc/moe/torch_bindings.cpp, csrc/torch_bindings.cpp, csrc/xpu/torch_bindings.cpp)
REFERENCE_SCHEMAS = {
    "_moe_C::moe_sum": "moe_sum(Tensor input, Tensor! output, Tensor? topk_ids, Tensor? expert_map) -> ()",
    "_moe_C::moe_align_block_size": "moe_align_block_size(Tensor topk_ids, int num_experts, int block_size, Tensor! sorted_token_ids, Tensor! experts_ids, Tensor! num_tokens_post_pad, Tensor? maybe_expert_map) -> ()",
    "_moe_C::moe_lora_align_block_size": "moe_lora_align_block_size(Tensor topk_ids, Tensor token_lora_mapping, int num_experts, int block_size, int max_loras, int max_num_tokens_padded, int max_num_m_blocks, Tensor! sorted_token_ids, Tensor! experts_ids, Tensor! num_tokens_post_pad, Tensor! adapter_enabled, Tensor! lora_ids, Tensor? maybe_expert_map) -> ()",
    "_moe_C::fused_moe_prologue": "fused_moe_prologue(Tensor input, Tensor? input_scales, Tensor token_selected_experts, Tensor token_final_scales, Tensor workspace, int hidden_size, int inter_size, int block_k, int ep_rank, int ep_size,int num_experts_on_rank) -> ()",
    "_moe_C::topk_softmax": "topk_softmax(Tensor! topk_weights, Tensor! topk_indices, Tensor! token_expert_indices, Tensor gating_output, bool renormalize, Tensor? bias) -> ()",
    "_moe_C::topk_sigmoid": "topk_sigmoid(Tensor! topk_weights, Tensor! topk_indices, Tensor! token_expert_indices, Tensor gating_output, bool renormalize, Tensor? bias, float routed_scaling_factor) -> ()",
    "_moe_C::topk_softplus_sqrt": "topk_softplus_sqrt(Tensor! topk_weights, Tensor! topk_indices, Tensor! token_expert_indices, Tensor gating_output, bool renormalize, float routed_scaling_factor, Tensor? correction_bias=None, Tensor? input_ids=None, Tensor? tid2eid=None) -> ()",
    "_moe_C::grouped_topk": "grouped_topk(Tensor scores, Tensor scores_with_bias, int n_group, int topk_group, int topk, bool renormalize, float routed_scaling_factor) -> (Tensor, Tensor)",
    "_moe_C::moe_gather": "moe_gather(Tensor! output, Tensor moe_output, Tensor topk_weights, Tensor unpermuted_row_to_permuted_row, int num_experts) -> ()",
    "_moe_C::init_expert_map": "init_expert_map(Tensor expert_map, int num_experts, int ep_rank, int ep_size) -> ()",
    "_moe_C::remap_hidden_states": "remap_hidden_states(Tensor hidden_states, Tensor? hidden_states_scales, Tensor remapped_hidden_states, Tensor? remapped_hidden_states_scales, Tensor? expert_map, Tensor rows_per_expert, Tensor unpermuted_row_to_permuted_row, Tensor topk_ids, int total_experts_num, int local_experts_num) -> ()",
    "_C::silu_and_mul": "silu_and_mul(Tensor! result, Tensor input) -> ()",
    "_C::swigluoai_and_mul": "swigluoai_and_mul(Tensor! out, Tensor input, float alpha=1.702, float limit=7.0) -> ()",
    "_C::per_token_group_fp8_quant": "per_token_group_fp8_quant(Tensor input, Tensor! output_q, Tensor! output_s, int group_size, float eps, float fp8_min, float fp8_max, bool scale_ue8m0, bool dummy_is_scale_transposed, bool dummy_is_tma_aligned ) -> ()",
    "_C::per_token_group_quant_mxfp4": "per_token_group_quant_mxfp4(Tensor input, Tensor! output_q, Tensor! output_s, int group_size, float eps) -> ()",
    "_C::gelu_and_mul": "gelu_and_mul(Tensor! out, Tensor input) -> ()",
    "_C::gelu_tanh_and_mul": "gelu_tanh_and_mul(Tensor! out, Tensor input) -> ()",
    "_C::relu2_no_mul": "relu2_no_mul(Tensor! out, Tensor! input) -> ()",
    "_C::swiglustep_and_mul": "swiglustep_and_mul(Tensor! out, Tensor input, float limit=7.0) -> ()",
    "_C::silu_and_mul_per_block_quant": "silu_and_mul_per_block_quant(Tensor! out, Tensor input, Tensor! scales, int group_size, Tensor? scale_ub=None, bool is_scale_transposed=False, bool scale_ue8m0=False) -> ()",
    "_C::silu_and_mul_mxfp4_quant": "silu_and_mul_mxfp4_quant(Tensor! out, Tensor input, Tensor! scales, int group_size, float eps=1e-10) -> ()",
    "_xpu_C::cutlass_grouped_gemm_interface": "cutlass_grouped_gemm_interface(Tensor ptr_A, Tensor? ptr_A_scale, Tensor ptr_B, Tensor? ptr_B_scale, Tensor? ptr_bias, Tensor ptr_D, Tensor rows_per_expert, int N, int K, int num_experts) -> Tensor",
}


# arguments the reference's kernels write without a mutation annotation in
# its schema: annotated here (Tensor(a!)), so that FakeTensor / functionalised
# tracing keeps the writes (opcheck's schema check fails without them)
WRITTEN_UNANNOTATED = {
    "_moe_C::fused_moe_prologue": {"workspace"},
    "_moe_C::init_expert_map": {"expert_map"},
    "_moe_C::remap_hidden_states": {"remapped_hidden_states", "remapped_hidden_states_scales",
                                    "rows_per_expert", "unpermuted_row_to_permuted_row"},
    "_xpu_C::cutlass_grouped_gemm_interface": {"ptr_D", "<return>"},
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_op_schemas_match_reference(name):
    """Names, argument names, types, order and defaults as the reference's
    registration; alias annotations too, except the writes it leaves
    unannotated (WRITTEN_UNANNOTATED), which are annotated here."""
    import vllm_xpu_kernels  # noqa: F401
    ns, op = name.split("::")
    ours = getattr(getattr(torch.ops, ns), op).default._schema
    ref = torch._C.parse_schema(ns + "::" + REFERENCE_SCHEMAS[name])
    added = WRITTEN_UNANNOTATED.get(name, set())
    if not added:
        assert str(ours) == str(ref)
        return
    assert ours.name == ref.name and len(ours.arguments) == len(ref.arguments)
    for a, b in zip(ours.arguments, ref.arguments):
        assert (a.name, str(a.type), a.default_value) == (b.name, str(b.type), b.default_value)
        if a.name in added:
            assert b.alias_info is None and a.alias_info is not None and a.alias_info.is_write
        else:
            assert str(a.alias_info) == str(b.alias_info)
    assert [str(r.type) for r in ours.returns] == [str(r.type) for r in ref.returns]
    if "<return>" in added:
        assert ours.returns[0].alias_info.is_write


def test_no_cpu_kernel_registered():
    """The ops exist only for GPU tensors: no silent CPU path."""
    import vllm_xpu_kernels  # noqa: F401
    x = torch.zeros(2, 8)
    out = torch.empty(2, 4)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops._C.silu_and_mul(out, x)


# Python entry points of the reference, parameter names, order and defaults as
# written in vllm_xpu_kernels/fused_moe_interface.py (XpuFusedMoe.__init__
# :166-180, XpuFusedMoe.apply :273-281, xpu_fused_moe :421-442).
_EMPTY = object()
REFERENCE_PY_SIGNATURES = {
    "XpuFusedMoe.__init__": [
        ("self", _EMPTY), ("w13", _EMPTY), ("w13_scales", _EMPTY), ("w13_bias", _EMPTY),
        ("w2", _EMPTY), ("w2_scales", _EMPTY), ("w2_bias", _EMPTY),
        ("n_experts_per_token", _EMPTY), ("activation", _EMPTY), ("num_experts", _EMPTY),
        ("ep_rank", 0), ("ep_size", 1), ("expert_map", None), ("gemm1_clamp_limit", None)],
    "XpuFusedMoe.apply": [
        ("self", _EMPTY), ("output", _EMPTY), ("hidden_states", _EMPTY),
        ("topk_weights", _EMPTY), ("topk_ids", _EMPTY), ("expert_map", None),
        ("a1q_scale", None)],
    "xpu_fused_moe": [
        ("hidden_states", _EMPTY), ("w13", _EMPTY), ("w13_scales", _EMPTY),
        ("w13_bias", _EMPTY), ("w2", _EMPTY), ("w2_scales", _EMPTY), ("w2_bias", _EMPTY),
        ("topk_weights", _EMPTY), ("topk_ids", _EMPTY), ("n_experts_per_token", _EMPTY),
        ("activation", _EMPTY), ("num_experts", _EMPTY), ("ep_rank", 0), ("ep_size", 1),
        ("expert_map", None), ("output", None), ("is_fp8", False), ("is_int4", False),
        ("is_mxfp4", False), ("is_mxfp8", False), ("is_block_fp8", False),
        ("gemm1_clamp_limit", None)],
}


@pytest.mark.parametrize("name", sorted(REFERENCE_PY_SIGNATURES))
def test_python_signatures_match_reference(name):
    import inspect

    from vllm_xpu_kernels import fused_moe_interface as F
    obj = F
    for part in name.split("."):
        obj = getattr(obj, part)
    params = list(inspect.signature(obj).parameters.values())
    got = [(p.name, _EMPTY if p.default is inspect.Parameter.empty else p.default)
           for p in params]
    assert got == REFERENCE_PY_SIGNATURES[name]
    assert all(p.kind == inspect.Parameter.POSITIONAL_OR_KEYWORD for p in params)


def _cpu_layer(monkeypatch, E=4, H=64, I=32, k=2):
    """A bf16 XpuFusedMoe on CPU tensors (row-major layout: the constructor
    then launches nothing)."""
    from vllm_xpu_kernels import fused_moe_interface as F
    monkeypatch.setenv(F.WEIGHT_LAYOUT_ENV, "nk")
    w13 = torch.zeros(E, H, 2 * I, dtype=torch.bfloat16)
    w2 = torch.zeros(E, I, H, dtype=torch.bfloat16)
    return F.XpuFusedMoe(w13, None, None, w2, None, None, k, "silu", E)


def test_apply_rejects_output_dtype_and_weight_shape(monkeypatch):
    moe = _cpu_layer(monkeypatch)
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    ids = torch.zeros(3, 2, dtype=torch.int32)
    w = torch.zeros(3, 2)
    with pytest.raises(ValueError, match="hidden_states' dtype"):
        moe.apply(torch.empty(3, 64, dtype=torch.float16), x, w, ids)
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        moe.apply(torch.empty(3, 64), x.float(), w, ids)
    with pytest.raises(ValueError, match="same shape"):
        moe.apply(torch.empty_like(x), x, torch.zeros(3, 3), ids)


def test_xpu_fused_moe_flags_checked_against_dtypes():
    from vllm_xpu_kernels import fused_moe_interface as F
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w13 = torch.zeros(4, 64, 64, dtype=torch.bfloat16)
    w2 = torch.zeros(4, 32, 64, dtype=torch.bfloat16)
    ids = torch.zeros(2, 2, dtype=torch.int32)
    tw = torch.zeros(2, 2)
    with pytest.raises(ValueError, match="is_block_fp8=True"):
        F.xpu_fused_moe(x, w13, None, None, w2, None, None, tw, ids, 2, "silu", 4,
                        is_block_fp8=True)
    with pytest.raises(ValueError, match="more than one recipe flag"):
        F.xpu_fused_moe(x, w13, None, None, w2, None, None, tw, ids, 2, "silu", 4,
                        is_fp8=True, is_int4=True)
    with pytest.raises(AssertionError, match="output shape"):
        F.xpu_fused_moe(x, w13, None, None, w2, None, None, tw, ids, 2, "silu", 4,
                        output=torch.empty(3, 64, dtype=torch.bfloat16))


def test_fused_moe_noalloc_rejects_calls_beyond_its_scratch(lib):
    """The allocation-free entry refuses, before any device work, a call
    whose workspace exceeds its static per-GPU scratch (C3 at 8192 tokens
    needs about 1.25 GB)."""
    from vllm_xpu_kernels import capi
    a = capi.FusedMoeArgs(recipe=1, activation=0, act_dtype=1, ids_dtype=3,
                          num_tokens=8192, hidden=7168, inter=2048, num_experts=256,
                          topk=8, w_layout=1, w13_scale=1, w2_scale=1)
    lib.mi355moe_fused_moe_noalloc.argtypes = [ctypes.POINTER(capi.FusedMoeArgs),
                                               ctypes.c_void_p]
    rc = lib.mi355moe_fused_moe_noalloc(ctypes.byref(a), None)
    assert rc == -4
    assert b"more than the static" in lib.mi355moe_last_error()


@pytest.mark.parametrize("field,value,message", [
    ("num_tokens", -1, b"invalid layer shape"), ("topk", 0, b"invalid layer shape"),
    ("num_experts", 2048, b"at most 1024"), ("hidden", 7100, b"% 128"),
    ("w13_scale", None, b"need scales"), ("w_layout", 7, b"unknown weight layout"),
    ("recipe", 9, b"unknown recipe"), ("ids_dtype", 1, b"int32 or int64")])
def test_fused_moe_noalloc_validates_before_sizing(lib, field, value, message):
    """The allocation-free entry checks its arguments before they size the
    scratch: invalid ones return MI355MOE_ERR_INVALID (-1) with the same
    message as the workspace entry, also when the shape would need more than
    the static scratch."""
    from vllm_xpu_kernels import capi
    kw = dict(recipe=1, activation=0, act_dtype=1, ids_dtype=3, num_tokens=8192, hidden=7168,
              inter=2048, num_experts=256, topk=8, w_layout=1, w13_scale=1, w2_scale=1)
    kw[field] = value
    a = capi.FusedMoeArgs(**kw)
    lib.mi355moe_fused_moe_noalloc.argtypes = [ctypes.POINTER(capi.FusedMoeArgs),
                                               ctypes.c_void_p]
    assert lib.mi355moe_fused_moe_noalloc(ctypes.byref(a), None) == -1
    assert message in lib.mi355moe_last_error()
    rc = lib.mi355moe_fused_moe(ctypes.byref(a), None, ctypes.c_size_t(0), None)
    assert rc == -1 and message in lib.mi355moe_last_error()


@pytest.mark.parametrize("weight_layout", ["nk", "kn"])
def test_block_fp8_inter_size_uses_scales(monkeypatch, weight_layout):
    """tests/fused_moe/test_fused_moe.py:37-60: fp8 weights [2, 512, 256] (or
    their transpose) with 128x128 block scales [2, 4, 2]: the intermediate
    size comes from the scales, 4 * 128 / 2 = 256, whatever the layout."""
    from vllm_xpu_kernels import fused_moe_interface as F
    monkeypatch.setenv(F.WEIGHT_LAYOUT_ENV, "nk")
    weight_nk = torch.zeros(2, 512, 256, dtype=torch.float8_e4m3fn)
    weight = weight_nk.transpose(-1, -2).contiguous() if weight_layout == "kn" else weight_nk
    w2 = torch.zeros(2, 256, 256, dtype=torch.float8_e4m3fn)
    moe = F.XpuFusedMoe(weight, torch.ones(2, 4, 2), None, w2, torch.ones(2, 2, 2), None,
                        1, "silu", 2)
    assert moe.inter_size == 256 and moe.recipe == "fp8block"


def test_prepare_in_place_host_logic(monkeypatch):
    """Weight preparation on host tensors (row-major layout, no device pass):
    by default the converted weights are written over the caller's tensors,
    which keep shape and dtype and hold exactly the bytes of
    MI355MOE_PREPARE_IN_PLACE=0's converted copy (that mode leaves them as
    they were); a second layer on them with the same arguments reuses the
    preparation, other arguments or a different partner tensor are refused.
    fp8 block-scaled swigluoai: the interleaved rows split into [gate; up]
    halves, the 128-row block scales repeated for both (one row per 64)."""
    from vllm_xpu_kernels import fused_moe_interface as F
    monkeypatch.setenv(F.WEIGHT_LAYOUT_ENV, "nk")
    E, H, I = 3, 64, 32
    g = torch.Generator().manual_seed(0)
    w13 = torch.randn(E, H, 2 * I, generator=g).to(torch.bfloat16)
    w2 = torch.randn(E, I, H, generator=g).to(torch.bfloat16)
    nk13, nk2 = w13.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
    split = torch.cat([nk13[:, 0::2], nk13[:, 1::2]], dim=1)
    for act, want13 in (("silu", nk13), ("swigluoai", split)):
        monkeypatch.setenv(F.PREPARE_IN_PLACE_ENV, "0")
        a13, a2 = w13.clone(), w2.clone()
        m0 = F.XpuFusedMoe(a13, None, None, a2, None, None, 1, act, E)
        assert torch.equal(a13, w13) and torch.equal(a2, w2)
        assert torch.equal(m0.w13, want13) and torch.equal(m0.w2, nk2)
        monkeypatch.delenv(F.PREPARE_IN_PLACE_ENV)
        m = F.XpuFusedMoe(a13, None, None, a2, None, None, 1, act, E)
        assert m.w13.data_ptr() == a13.data_ptr() and m.w2.data_ptr() == a2.data_ptr()
        assert a13.shape == w13.shape and a13.dtype == w13.dtype
        assert torch.equal(m.w13, want13) and torch.equal(m.w2, nk2)
        assert torch.equal(a13.flatten(), want13.flatten())
        m2 = F.XpuFusedMoe(a13, None, None, a2, None, None, 1, act, E)
        assert m2.w13.data_ptr() == a13.data_ptr() and torch.equal(m2.w13, want13)
        with pytest.raises(ValueError, match="other arguments"):
            F.XpuFusedMoe(a13, None, None, a2, None, None, 1, "gelu", E)
        with pytest.raises(ValueError, match="other arguments"):
            F.XpuFusedMoe(a13, None, None, w2.clone(), None, None, 1, act, E)
    # fp8 block scales: [E, 2I/128, H/128] -> [E, 2I/64, H/128], halves equal
    I8, H8 = 128, 256
    q13 = torch.randn(E, 2 * I8, H8, generator=g).to(torch.float8_e4m3fn)
    q2 = torch.randn(E, H8, I8, generator=g).to(torch.float8_e4m3fn)
    s13 = torch.rand(E, 2 * I8 // 128, H8 // 128, generator=g)
    s2 = torch.rand(E, H8 // 128, I8 // 128, generator=g)
    want = torch.cat([q13[:, 0::2], q13[:, 1::2]], dim=1).view(torch.uint8)
    q13b, q2b = q13.clone(), q2.clone()
    m = F.XpuFusedMoe(q13, s13, None, q2, s2, None, 1, "swigluoai", E)
    assert m.recipe == "fp8block" and m._ws_rows == 64
    assert torch.equal(m.w13.view(torch.uint8), want)
    assert torch.equal(m.gemm1_wei_scales, torch.cat([s13, s13], dim=1))
    assert torch.equal(m.gemm2_wei_scales, s2)
    assert F.XpuFusedMoe(q13b, s13, None, q2b, s2, None, 1, "silu", E)._ws_rows == 128


def test_mx_recipe_selection(monkeypatch):
    """Recipe detection of the reference (fused_moe_interface.py:33-61): e4m3
    weights with uint8 scales are mxfp8; e2m1 weights are mxfp4, or
    mxfp4_fp8 under VLLM_XPU_FUSED_MOE_USE_MXFP4_FP8, which then refuses
    pre-quantised input as the reference's quant_act_xpu does."""
    from vllm_xpu_kernels import fused_moe_interface as F
    monkeypatch.setenv(F.WEIGHT_LAYOUT_ENV, "nk")
    E, H, I = 2, 64, 32
    moe8 = F.XpuFusedMoe(torch.zeros(E, H, 2 * I, dtype=torch.float8_e4m3fn),
                         torch.zeros(E, H // 32, 2 * I, dtype=torch.uint8), None,
                         torch.zeros(E, I, H, dtype=torch.float8_e4m3fn),
                         torch.zeros(E, I // 32, H, dtype=torch.uint8), None, 1, "silu", E)
    assert moe8.recipe == "mxfp8" and moe8.inter_size == I
    assert tuple(moe8.w13.shape) == (E, 2 * I, H)
    assert tuple(moe8.gemm1_wei_scales.shape) == (E, 2 * I, H // 32)
    w13 = torch.zeros(E, 2 * I, H // 2, dtype=torch.uint8).view(torch.float4_e2m1fn_x2)
    w2 = torch.zeros(E, H, I // 2, dtype=torch.uint8).view(torch.float4_e2m1fn_x2)
    s13 = torch.zeros(E, 2 * I, H // 32, dtype=torch.uint8)
    s2 = torch.zeros(E, H, I // 32, dtype=torch.uint8)
    assert F.XpuFusedMoe(w13, s13, None, w2, s2, None, 1, "silu", E).recipe == "mxfp4"
    monkeypatch.setenv(F.USE_MXFP4_FP8_ENV, "1")
    moe = F.XpuFusedMoe(w13, s13, None, w2, s2, None, 1, "silu", E)
    assert moe.recipe == "mxfp4_fp8"
    with pytest.raises(NotImplementedError, match="mxfp4_fp8"):
        moe.apply(torch.empty(3, H, dtype=torch.bfloat16),
                  torch.zeros(3, H // 2, dtype=torch.uint8), torch.zeros(3, 1),
                  torch.zeros(3, 1, dtype=torch.int32),
                  a1q_scale=torch.zeros(3, H // 32, dtype=torch.uint8))


def test_every_op_has_a_meta_kernel():
    """Every op of the _moe_C, _C and _xpu_C namespaces has a Meta kernel
    (FakeTensor tracing, torch.compile): on meta tensors the in-place ops
    return nothing and the grouped GEMM returns its output argument, the
    routers [T, k] values and int32 ids."""
    from vllm_xpu_kernels import _ops  # noqa: F401
    names = sorted({n.split(".")[0] for n in torch._C._dispatch_get_all_op_names()
                    if n.partition("::")[0] in ("_moe_C", "_C", "_xpu_C")})
    assert len(names) >= 25
    missing = [n for n in names if not torch._C._dispatch_has_kernel_for_dispatch_key(n, "Meta")]
    assert not missing, missing
    m = torch.device("meta")
    d = torch.empty(16, 256, dtype=torch.bfloat16, device=m)
    out = torch.ops._xpu_C.cutlass_grouped_gemm_interface(
        torch.empty(16, 512, dtype=torch.bfloat16, device=m), None,
        torch.empty(3, 512, 256, dtype=torch.bfloat16, device=m), None, None, d,
        torch.empty(3, dtype=torch.int32, device=m), 256, 512, 3)
    assert out is d
    v, i = torch.ops._moe_C.mi355_fused_grouped_topk(
        torch.empty(33, 256, device=m), None, 8, 4, 8, True, 2.5)
    assert v.shape == i.shape == (33, 8) and i.dtype == torch.int32
    v, i = torch.ops._moe_C.grouped_topk(torch.empty(5, 64, device=m),
                                         torch.empty(5, 64, device=m), 1, 1, 6, True, 1.0)
    assert v.shape == (5, 6) and i.dtype == torch.int32
    assert torch.ops._C.silu_and_mul(torch.empty(4, 8, device=m),
                                     torch.empty(4, 16, device=m)) is None


@pytest.mark.parametrize("scoring", ["sigmoid", "softmax"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fused_grouped_topk_bias_optional_on_both_paths(scoring, with_bias):
    """Both scoring paths take e_score_correction_bias=None (no correction)
    and give float32 weights and int32 ids [T, k] (meta tensors: shapes only,
    through the ops' meta kernels)."""
    from vllm_xpu_kernels import ops
    m = torch.device("meta")
    bias = torch.empty(256, device=m) if with_bias else None
    v, i = ops.fused_grouped_topk(torch.empty(7, 256, device=m), 8, True, bias, 8, 4,
                                  scoring, 2.5)
    assert v.shape == i.shape == (7, 8)
    assert v.dtype == torch.float32 and i.dtype == torch.int32
