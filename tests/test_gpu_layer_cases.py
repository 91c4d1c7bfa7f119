"""GPU parity: the reference's remaining layer test cases
(tests/fused_moe/test_fused_moe.py) against the CPU oracle.

* gemm1_clamp_limit (reference :912-994): G1 std about 8, so limits 5 and 10
  clamp a large share of gate/up values; SiLU as the reference, plus
  swigluoai (interleaved G1, where the reference's column-half clamp falls on
  both gate and up of the first I/2 pairs) and a limit that is not a bf16
  value.  Token counts cover the split-K STREAM, STREAM, SMALL and 128/320-slot
  kernels.
* expert parallelism (reference :534-909): E = 16 global experts, ep_size 4,
  the layer built on one rank's 4 experts with ep_rank / ep_size, for the
  16-bit, per-expert fp8, int4, mxfp4 and fp8block recipes.

Bars: the reference's (bf16 2e-2, fp16 1e-2, relative to the output scale
for the clamp cases); fp8block and MX re-quantise the activation and take
the fp8 bar of test_gpu_gemm_fused.py.
"""
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _layer_cls():
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    return XpuFusedMoe


def _W():
    from vllm_xpu_kernels import workloads
    return workloads


def _close_fp8(out, ref, rtol=2e-2, atol=2e-2, max_abs=8e-2):
    """fp8block bar: 99.9% of the elements within rtol/atol, all within
    max_abs (a one-ulp accumulation difference can flip one e4m3 code of
    the re-quantised activation)."""
    err = (out.float() - ref.float()).abs()
    bad = err > atol + rtol * ref.float().abs()
    assert bad.float().mean().item() <= 1e-3, f"{int(bad.sum())} elements off"
    assert err.max().item() <= max_abs, err.max().item()


# ---------------------------------------------------------- gemm1 clamp
@pytest.mark.parametrize("T", [1, 16, 64, 512, 2048])
@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
@pytest.mark.parametrize("limit", [5.0, 10.0, 7.3])
def test_fused_moe_clamp_limit(dev, T, activation, limit):
    g = torch.Generator().manual_seed(7)
    E, H, I, topk = 16, 1024, 1024, 1
    x = (torch.randn(T, H, generator=g) / 2).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * I, H, generator=g) / 2).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) / 16).to(torch.bfloat16)
    tw, ti = torch.topk(torch.randn(T, E, generator=g), k=topk, dim=-1, sorted=False)
    moe = _layer_cls()(w13.transpose(1, 2).contiguous().to(dev), None, None,
                       w2.transpose(1, 2).contiguous().to(dev), None, None, topk,
                       activation, E, gemm1_clamp_limit=limit)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, min(T, 48)).long()
    ref = O.fused_moe("bf16", x[toks], w13, None, None, w2, None, None, tw[toks], ti[toks],
                      activation=activation, gemm1_clamp_limit=limit)
    got = out.cpu()[toks]
    scale = ref.float().abs().max().item()
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=0.02 * scale)
    # the typical element far inside the bar, and the clamp took effect
    assert (got.float() - ref.float()).abs().mean() < 2e-3 * scale
    if activation == "silu" or limit < 7.0:   # swigluoai clamps at 7.0 itself
        free = O.fused_moe("bf16", x[toks], w13, None, None, w2, None, None, tw[toks],
                           ti[toks], activation=activation)
        assert (free.float() - ref.float()).abs().max() > 0.1 * scale


@pytest.mark.parametrize("tile", ["stream", "small", "big", "bigreg", "wide"])
@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
def test_fused_moe_clamp_limit_fp8_every_family(dev, monkeypatch, tile, activation):
    """gemm1_clamp_limit through each GEMM family's GLU epilogue, forced with
    MI355MOE_GEMM_TILE, on fp8 block-scaled weights (swigluoai: the same
    layer with bf16 weights, fp8 has no swigluoai layout)."""
    W = _W()
    monkeypatch.setenv("MI355MOE_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(17)
    E, H, I, topk, T = 8, 1024, 1024, 2, 600
    x = (torch.randn(T, H, generator=g) / 2).to(torch.bfloat16)
    w13 = torch.randn(E, 2 * I, H, generator=g) / 2
    w2 = torch.randn(E, H, I, generator=g) / 16
    tw, ti = torch.topk(torch.randn(T, E, generator=g).softmax(-1), k=topk, dim=-1)
    if activation == "silu":
        q13, s13 = W.fp8_block_quant(w13)
        q2, s2 = W.fp8_block_quant(w2)
        moe = _layer_cls()(q13.to(dev), s13.to(dev), None, q2.to(dev), s2.to(dev), None, topk,
                           activation, E, gemm1_clamp_limit=5.0)
        recipe, args = "fp8block", (q13, s13, None, q2, s2, None)
    else:
        b13, b2 = w13.to(torch.bfloat16), w2.to(torch.bfloat16)
        moe = _layer_cls()(b13.transpose(1, 2).contiguous().to(dev), None, None,
                           b2.transpose(1, 2).contiguous().to(dev), None, None, topk,
                           activation, E, gemm1_clamp_limit=5.0)
        recipe, args = "bf16", (b13, None, None, b2, None, None)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, 32).long()
    ref = O.fused_moe(recipe, x[toks], *args, tw[toks], ti[toks], activation=activation,
                      gemm1_clamp_limit=5.0)
    scale = ref.float().abs().max().item()
    got = out.cpu()[toks].float()
    err = (got - ref.float()).abs()
    # fp8: the re-quantised activation may flip a code on a one-ulp accumulation
    # difference; 99.9% within the reference's relative bar, all within 4x it
    assert (err > 0.02 * scale + 0.02 * ref.float().abs()).float().mean() <= 1e-3
    assert err.max() <= 0.08 * scale


@pytest.mark.parametrize("T", [1, 48, 1024])
def test_fused_moe_clamp_limit_mxfp4_swigluoai(dev, T):
    """gpt-oss's combination (mxfp4 weights, swigluoai, biases) with a clamp
    limit below the activation's own 7.0."""
    import dataclasses
    W = _W()
    cfg = dataclasses.replace(W.CONFIGS["C5"], hidden=512, inter=512, experts=8, topk=2)
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, T, dev) * 16
    tw, ti = W.route(cfg, W.make_router_logits(cfg, T, dev))
    moe = _layer_cls()(*w.layer_args(copy=True), cfg.topk, "swigluoai", cfg.experts,
                       gemm1_clamp_limit=3.0)
    out = torch.empty_like(x)
    moe.apply(out, x, tw, ti)
    toks = torch.linspace(0, T - 1, min(T, 48)).long().to(dev)
    ref = O.fused_moe("mxfp4", x[toks].cpu(), w.w13.view(torch.uint8).cpu(), w.w13_scale.cpu(),
                      w.w13_bias.cpu(), w.w2.view(torch.uint8).cpu(), w.w2_scale.cpu(),
                      w.w2_bias.cpu(), tw[toks].cpu(), ti[toks].cpu().long(),
                      activation="swigluoai", gemm1_clamp_limit=3.0)
    scale = ref.float().abs().max().item()
    torch.testing.assert_close(out[toks].cpu().float(), ref.float(), rtol=2e-2,
                               atol=0.02 * scale)


# ---------------------------------------------------- expert parallelism
EP_SIZE = 4
E_GLOBAL = 16


def _ep_weights(recipe, dt, g, H, I):
    """Global weights for E_GLOBAL experts: (reference-layout tensors for
    the layer, oracle-layout tensors), each (w13, s13, b13, w2, s2, b2)."""
    E = E_GLOBAL
    b13 = (torch.randn(E, 2 * I, generator=g) / 16).to(dt)
    b2 = (torch.randn(E, H, generator=g) / 16).to(dt)
    w13 = torch.randn(E, 2 * I, H, generator=g) / 16
    w2 = torch.randn(E, H, I, generator=g) / 16
    if recipe == "bf16":
        q13, q2 = w13.to(dt), w2.to(dt)
        lay = (q13.transpose(1, 2).contiguous(), None, b13, q2.transpose(1, 2).contiguous(),
               None, b2)
        return lay, (q13, None, b13, q2, None, b2)
    if recipe == "fp8":     # reference :576-606: e5m2 with a power-of-two scale per expert
        s13 = torch.pow(2.0, torch.randint(-3, 4, (E,), generator=g).float())
        s2 = torch.pow(2.0, torch.randint(-3, 4, (E,), generator=g).float())
        q13 = (w13 / s13.view(E, 1, 1)).to(torch.float8_e5m2)
        q2 = (w2 / s2.view(E, 1, 1)).to(torch.float8_e5m2)
        lay = (q13.transpose(1, 2).contiguous(), s13, b13, q2.transpose(1, 2).contiguous(),
               s2, b2)
        return lay, (q13, s13, b13, q2, s2, b2)
    if recipe == "int4":    # u4 with zero point 8, scales 2^-5 (reference :667-790)
        u13 = torch.randint(0, 0xff, (E, 2 * I, H // 2), generator=g).to(torch.uint8)
        u2 = torch.randint(0, 0xff, (E, H, I // 2), generator=g).to(torch.uint8)
        s13 = torch.full((E, 2 * I, H // 128), 2.0 ** -5).to(dt)
        s2 = torch.full((E, H, I // 128), 2.0 ** -5).to(dt)
        return (u13, s13, b13, u2, s2, b2), (u13 ^ 0x88, s13, b13, u2 ^ 0x88, s2, b2)
    W = _W()
    if recipe == "mxfp8":   # reference layout: e4m3 [E, K, N] + e8m0 [E, K/32, N]
        q13, s13 = W.mxfp8_quant(w13)
        q2, s2 = W.mxfp8_quant(w2)
        tr = lambda t: t.transpose(1, 2).contiguous()  # noqa: E731
        return (tr(q13), tr(s13), b13, tr(q2), tr(s2), b2), (q13, s13, b13, q2, s2, b2)
    if recipe == "mxfp4":
        q13, s13 = W.mxfp4_quant(w13)
        q2, s2 = W.mxfp4_quant(w2)
        lay = (q13.view(torch.float4_e2m1fn_x2), s13, b13, q2.view(torch.float4_e2m1fn_x2), s2,
               b2)
        return lay, (q13, s13, b13, q2, s2, b2)
    assert recipe == "fp8block"
    q13, s13 = W.fp8_block_quant(w13)
    q2, s2 = W.fp8_block_quant(w2)
    return (q13, s13, None, q2, s2, None), (q13, s13, None, q2, s2, None)


@pytest.mark.parametrize("recipe,dt", [("bf16", torch.float16), ("fp8", torch.float16),
                                       ("int4", torch.float16), ("mxfp4", torch.bfloat16),
                                       ("fp8block", torch.bfloat16), ("mxfp8", torch.bfloat16),
                                       ("mxfp8", torch.float16)])
@pytest.mark.parametrize("ep_rank", [0, 3])
@pytest.mark.parametrize("T", [1, 16, 512])
def test_fused_moe_ep(dev, recipe, dt, ep_rank, T):
    g = torch.Generator().manual_seed(7 + T + 100 * ep_rank)
    H, I, topk = 1024, 1024, 2
    lay, ora = _ep_weights(recipe, dt, g, H, I)
    x = (torch.randn(T, H, generator=g) / 16).to(dt)
    tw, ti = torch.topk(torch.randn(T, E_GLOBAL, generator=g), k=topk, dim=-1, sorted=False)
    e = E_GLOBAL // EP_SIZE
    lo, hi = e * ep_rank, e * (ep_rank + 1)
    loc = [None if t is None else t[lo:hi].contiguous().to(dev) for t in lay]
    moe = _layer_cls()(*loc, topk, "silu", e, ep_rank=ep_rank, ep_size=EP_SIZE)
    out = torch.empty(T, H, dtype=dt, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, min(T, 48)).long()
    ref = O.fused_moe(recipe, x[toks], *[None if t is None else t[lo:hi] for t in ora],
                      tw[toks], ti[toks], expert_map=O.init_expert_map(e, ep_rank, EP_SIZE))
    got = out.cpu()[toks]
    # tokens with no local expert give exact zeros
    local = ((ti[toks] >= lo) & (ti[toks] < hi)).any(-1)
    assert torch.all(got[~local] == 0)
    if recipe in ("fp8block", "mxfp8"):
        _close_fp8(got, ref)
    else:
        tol = 2e-2 if dt == torch.bfloat16 else 1e-2
        torch.testing.assert_close(got, ref, rtol=tol, atol=tol)
