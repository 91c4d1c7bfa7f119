"""torch.library.opcheck over every registered op (the reference runs it on
its ops, tests/test_moe_align_block_size.py:427-476, tests/test_moe_sum.py,
tests/test_activation.py, with the checks of tests/utils.py:12-68): the
schema's mutation and alias annotations match what the kernel writes, the
meta kernel gives the real outputs' metadata (FakeTensor), and the op traces
through AOT dispatch with dynamic shapes.

Each case calls the package's own wrapper once on small inputs; a dispatch
mode records every call into the _moe_C / _C / _xpu_C namespaces with its
arguments as they were before the call, and opcheck replays each."""
import unittest.mock

import pytest
import torch
from torch.utils import _pytree as pytree
from torch.utils._python_dispatch import TorchDispatchMode

pytestmark = pytest.mark.gpu

NAMESPACES = ("_moe_C", "_C", "_xpu_C")
CHECKS = ("test_schema", "test_autograd_registration", "test_faketensor",
          "test_aot_dispatch_dynamic")
FP8 = (torch.float8_e4m3fn, torch.float8_e5m2, torch.float8_e8m0fnu, torch.float4_e2m1fn_x2)


def _allclose(a, b, rtol=1e-5, atol=1e-8, equal_nan=False):
    """torch.allclose, also for the 8-bit float types opcheck compares (as
    bytes: both sides come from the same deterministic kernel)."""
    if a.dtype in FP8 or b.dtype in FP8:
        return a.dtype == b.dtype and torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    return _REAL_ALLCLOSE(a, b, rtol=rtol, atol=atol, equal_nan=equal_nan)


_REAL_ALLCLOSE = torch.allclose


# The reference's grouped GEMM returns its output argument (schema
# "-> Tensor", csrc/xpu/torch_bindings.cpp:46-49): annotated here as the alias
# it is, Tensor(a!) -> Tensor(a!), which AOT dispatch refuses for any custom
# op ("output has alias annotations"); the other three checks apply.
ALIASING_RETURN = {"_xpu_C::cutlass_grouped_gemm_interface"}


def opcheck(op, args, kwargs=None):
    checks = CHECKS
    if op.name().split(".")[0] in ALIASING_RETURN:
        checks = tuple(c for c in CHECKS if c != "test_aot_dispatch_dynamic")
    with unittest.mock.patch("torch.allclose", new=_allclose):
        return torch.library.opcheck(op, args, kwargs, test_utils=checks,
                                     raise_exception=True)


class _Record(TorchDispatchMode):
    """Calls into this library's namespaces, with cloned arguments."""

    def __init__(self):
        super().__init__()
        self.calls = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func.namespace in NAMESPACES:
            snap = pytree.tree_map_only(torch.Tensor, lambda t: t.clone(), (args, kwargs))
            self.calls.append((func, snap))
        return func(*args, **kwargs)


def _ops():
    from vllm_xpu_kernels import ops
    return ops


def _randn(*shape, dtype=torch.float32, seed=0, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(dev)


def _ids(T, k, E, seed=0, dtype=torch.int32, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(dtype).to(dev)


def _case_routing():
    o = _ops()
    x = _randn(9, 64)
    o.topk_softmax(x, 4, True)
    o.topk_softmax(x, 4, False, _randn(64, seed=1))
    o.topk_sigmoid(x, 4, True, _randn(64, seed=1), routed_scaling_factor=2.5)
    o.topk_softplus_sqrt(_randn(9, 128), 8, True, 1.5, _randn(128, seed=2))
    s = _randn(9, 256).sigmoid()
    o.grouped_topk(s, s + _randn(256, seed=3) * 0.01, 8, 4, 8, True, 2.5)
    o.fused_grouped_topk(_randn(9, 256), 8, True, _randn(256, seed=3) * 0.01, 8, 4,
                         "sigmoid", 2.5)


def _case_align():
    o = _ops()
    ids = _ids(5, 4, 16)
    o.moe_align_block_size(ids, 4, 16)
    em = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    em[:8] = torch.arange(8, dtype=torch.int32, device="cuda")
    o.moe_align_block_size(ids, 4, 16, expert_map=em, ignore_invalid_experts=True)
    E, bs, max_loras = 16, 4, 2
    mx = (ids.numel() + E * (bs - 1) + bs - 1) // bs * bs
    nb = mx // bs
    dev = "cuda"
    o.moe_lora_align_block_size(
        ids, torch.tensor([0, 1, 1, 0, -1], dtype=torch.int32, device=dev), E, bs, max_loras,
        mx, nb, torch.empty(max_loras * mx, dtype=torch.int32, device=dev),
        torch.empty(max_loras * nb, dtype=torch.int32, device=dev),
        torch.empty(max_loras, dtype=torch.int32, device=dev),
        torch.ones(max_loras + 1, dtype=torch.int32, device=dev),
        torch.arange(max_loras + 2, dtype=torch.int32, device=dev))


def _case_combine():
    o = _ops()
    T, k, H = 6, 2, 64
    out = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
    o.moe_sum(_randn(T, k, H, dtype=torch.bfloat16), out)
    em = torch.tensor([0, -1, 1, -1], dtype=torch.int32, device="cuda")
    o.moe_sum(_randn(T, k, H, dtype=torch.bfloat16), out, _ids(T, k, 4), em)
    perm = torch.randperm(T * k, generator=torch.Generator().manual_seed(4)).reshape(T, k)
    o.moe_gather(out, _randn(T * k, H, dtype=torch.bfloat16), _randn(T, k).abs(),
                 perm.int().cuda(), 4)


def _case_expert_parallel():
    from vllm_xpu_kernels import capi
    o = _ops()
    o.init_expert_map(8, 1, 2, "cuda")
    x = _randn(5, 64, dtype=torch.bfloat16)
    em = o.init_expert_map(4, 1, 2, "cuda")
    o.remap_hidden_states(x, _ids(5, 2, 8), 8, 4, expert_map=em)
    T, k, H, E = 5, 2, 256, 8
    total, _ = capi.prologue_layout(T, k, H, 2, 1, 0, E)
    ws = torch.zeros(total, dtype=torch.uint8, device="cuda")
    o.fused_moe_prologue(_randn(T, H, dtype=torch.bfloat16), None, _ids(T, k, E, dtype=torch.int64),
                         _randn(T, k), ws, H, 512, 1, 0, 1, E)


def _case_activation():
    o = _ops()
    x = _randn(7, 256, dtype=torch.bfloat16)
    o.silu_and_mul(x)
    o.gelu_and_mul(x)
    o.gelu_tanh_and_mul(x)
    o.swigluoai_and_mul(x)
    o.swiglustep_and_mul(x)
    o.relu2_no_mul(x)


def _case_quant():
    o = _ops()
    x = _randn(7, 256, dtype=torch.bfloat16)
    o.per_token_group_fp8_quant(x, 128)
    o.per_token_group_quant_mxfp4(x, 32)
    o.silu_and_mul_per_block_quant(x, 64, torch.float8_e4m3fn)
    o.silu_and_mul_mxfp4_quant(x, 32)


def _case_grouped_gemm():
    from oracle import moe_oracle as O
    o = _ops()
    rows = [5, 0, 11]
    E, N, K = 3, 256, 256
    M = sum(rows)
    rpe = torch.tensor(rows, dtype=torch.int32, device="cuda")
    a = _randn(M, K, dtype=torch.bfloat16)
    w = _randn(E, K, N, dtype=torch.bfloat16, seed=1) * 0.05
    o.cutlass_grouped_gemm(a, w, None, None, torch.empty(M, N, dtype=torch.bfloat16,
                                                          device="cuda"), rpe, N, K, E)
    q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=torch.Generator()
                                                .manual_seed(2)) * 0.02)
    o.cutlass_grouped_gemm(a, q.cuda(), s.cuda(), None,
                           torch.empty(M, N, dtype=torch.bfloat16, device="cuda"), rpe, N, K, E)


def _case_layer():
    import dataclasses
    from vllm_xpu_kernels import workloads as W
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    for name in ("C1", "C5"):
        cfg = dataclasses.replace(W.config(name), hidden=256, inter=128, experts=8, topk=2)
        w = W.make_weights(cfg, "cuda")
        moe = XpuFusedMoe(*w.layer_args(), cfg.topk, cfg.activation, cfg.experts)
        x = W.make_activations(cfg, 5, "cuda")
        tw, ti = W.route(cfg, W.make_router_logits(cfg, 5, "cuda"))
        moe.apply(torch.empty_like(x), x, tw, ti)


CASES = {"routing": _case_routing, "align": _case_align, "combine": _case_combine,
         "expert_parallel": _case_expert_parallel, "activation": _case_activation,
         "quant": _case_quant, "grouped_gemm": _case_grouped_gemm, "layer": _case_layer}


def _registered_ops():
    names = set()
    for full in torch._C._dispatch_get_all_op_names():
        ns, _, name = full.partition("::")
        if ns in NAMESPACES:
            names.add(full.split(".")[0])
    return names


def _recorded(case):
    rec = _Record()
    with rec:
        CASES[case]()
    torch.cuda.synchronize()
    return rec.calls


@pytest.mark.parametrize("case", sorted(CASES))
def test_opcheck(dev, case):
    """Each distinct call signature of the case (op and argument kinds: the
    per-expert preparation calls repeat one signature) through opcheck."""
    calls = _recorded(case)
    assert calls
    done = set()
    for func, (args, kwargs) in calls:
        kinds = (func, tuple(type(a).__name__ if not isinstance(a, torch.Tensor) else a.dtype
                             for a in args))
        if kinds in done:
            continue
        done.add(kinds)
        print(f"opcheck {func}", flush=True)
        opcheck(func, args, kwargs)


def test_opcheck_covers_every_registered_op(dev):
    seen = set()
    for case in CASES:
        seen |= {f.name().split(".")[0] for f, _ in _recorded(case)}
    assert _registered_ops() <= seen, sorted(_registered_ops() - seen)


# the reference's own opcheck case (tests/test_moe_align_block_size.py:427-476)
@pytest.mark.parametrize("ep_size", [1, 2])
def test_moe_align_block_size_opcheck(dev, ep_size):
    num_experts, block_size = 4, 4
    expert_map = None
    if ep_size != 1:
        local = num_experts // ep_size
        chosen = torch.randperm(num_experts, device=dev)[:local].int()
        expert_map = torch.full((num_experts,), -1, device=dev, dtype=torch.int32)
        expert_map[chosen] = torch.arange(local, device=dev, dtype=torch.int32)
    topk_ids = torch.randint(0, num_experts, (3, 4), dtype=torch.int32, device=dev)
    max_padded = topk_ids.numel() + num_experts * (block_size - 1)
    sorted_ids = torch.full((max_padded,), topk_ids.numel(), dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max_padded // block_size, dtype=torch.int32, device=dev)
    ntp = torch.empty(1, dtype=torch.int32, device=dev)
    opcheck(torch.ops._moe_C.moe_align_block_size.default,
            (topk_ids, num_experts, block_size, sorted_ids, expert_ids, ntp, expert_map))
