"""GPU: the allocation-free entry point mi355moe_fused_moe_noalloc (static
per-GPU scratch) against mi355moe_fused_moe (caller workspace), through the C
ABI, on two calls in a row, the second with a smaller input: the two must be
bit-identical (same kernels, same order of operations)."""
import ctypes
import dataclasses

import pytest
import torch

pytestmark = pytest.mark.gpu


def _run_pair(cfg, T, dev, moe, w, seed, expert_map=None):
    from vllm_xpu_kernels import capi
    from vllm_xpu_kernels import workloads as W
    print(f"noalloc pair: {cfg.name} {cfg.recipe} E={cfg.experts} T={T} "
          f"expert_map={expert_map is not None}", flush=True)
    x = W.make_activations(cfg, T, dev, seed=seed)
    logits = W.make_router_logits(cfg, T, dev, seed=seed + 1)
    bias = W.make_correction_bias(cfg, dev) if cfg.routing == "grouped_sigmoid" else None
    tw, ti = W.route(cfg, logits, bias)
    ref = torch.empty_like(x)
    out = torch.full_like(x, float("nan"))
    a_ref = capi.fused_args(moe, ref, x, tw, ti, expert_map=expert_map)
    a_out = capi.fused_args(moe, out, x, tw, ti, expert_map=expert_map)
    ws = capi.workspace_for(a_ref, dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lib = capi.lib
    assert lib.mi355moe_fused_moe(ctypes.byref(a_ref), ctypes.c_void_p(ws.data_ptr()),
                                  ctypes.c_size_t(ws.numel()), stream) == 0
    lib.mi355moe_fused_moe_noalloc.argtypes = [ctypes.POINTER(capi.FusedMoeArgs),
                                               ctypes.c_void_p]
    rc = lib.mi355moe_fused_moe_noalloc(ctypes.byref(a_out), stream)
    assert rc == 0, lib.mi355moe_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"T={T}: {(out.float() - ref.float()).abs().max()}"


# after the first (larger) call the scratch holds its data: the decode
# calls that follow (T = 2, 1: at most 16 slots, the split-K and
# token-major kernels) must not depend on it
@pytest.mark.parametrize("name,E,sizes", [("C2", None, (64, 16, 2, 1)),
                                          ("C3", 32, (33, 4, 2, 1)),
                                          ("C3-fp8", 32, (33, 4, 2, 1)),
                                          ("C2-int4", None, (64, 16, 2, 1))])
def test_fused_moe_noalloc_matches_workspace_entry(dev, name, E, sizes):
    """C2 bf16, C3 fp8 block-scaled, C3 shapes with per-expert e4m3 weights
    (read as fp8) and C2 shapes with K-blocked int4 weights."""
    from vllm_xpu_kernels import workloads as W
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    cfg = W.config(name)
    if E is not None:
        cfg = dataclasses.replace(cfg, experts=E)
    w = W.make_weights(cfg, dev)
    moe = XpuFusedMoe(*w.layer_args(), cfg.topk, cfg.activation, cfg.experts)
    for i, T in enumerate(sizes):   # each call smaller than the one before
        _run_pair(cfg, T, dev, moe, w, seed=10 + 3 * i)


def test_fused_moe_noalloc_expert_map(dev):
    """Expert parallelism (rank 1 of 2: 16 local experts of C3's 32, the
    global -> local map of the layer): T = 33 then 2."""
    from vllm_xpu_kernels import workloads as W
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    cfg = dataclasses.replace(W.config("C3"), experts=32)
    local = dataclasses.replace(cfg, experts=16)
    w = W.make_weights(local, dev)
    moe = XpuFusedMoe(*w.layer_args(), cfg.topk, cfg.activation, 16, ep_rank=1, ep_size=2)
    assert moe.expert_map is not None and moe.expert_map.numel() == 32
    for i, T in enumerate((33, 2)):
        _run_pair(cfg, T, dev, moe, w, seed=40 + 3 * i, expert_map=moe.expert_map)
