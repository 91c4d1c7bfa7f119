"""GPU parity: grouped GEMM (cutlass_grouped_gemm_interface) and the fused
MoE layer (XpuFusedMoe.apply) against the CPU oracle.

Layer tolerance (bf16 outputs): rtol = atol = 2e-2, the bar of the reference's
own fused-MoE tests (tests/fused_moe/test_fused_moe.py:288-294).  Routing,
alignment and activation quantisation are bit-exact (other test files), so
the remaining difference is fp32 accumulation order and the resulting
one-ulp flips of intermediate bf16/e4m3 roundings.
"""
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

LAYER_RTOL = 2e-2
LAYER_ATOL = 2e-2
FP8_MAX_ABS = 8e-2


def _ops():
    from vllm_xpu_kernels import ops
    return ops


def _W():
    from vllm_xpu_kernels import workloads
    return workloads


def _close(out, ref, rtol=LAYER_RTOL, atol=LAYER_ATOL, fp8=False):
    """bf16 / mxfp4 layers: every element within rtol/atol.  fp8block layers
    re-quantise the intermediate activation to e4m3 (1/16 relative step):
    a one-ulp difference of an fp32 accumulation between GPU and oracle
    that flips one activation code (or a group's amax) moves an output by up
    to ~3e-2, so there 99.9% of the elements must meet rtol/atol and all of
    them FP8_MAX_ABS."""
    out = out.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(out).all()
    err = (out - ref).abs()
    if fp8:
        bad = err > atol + rtol * ref.abs()
        assert bad.float().mean().item() <= 1e-3, f"{int(bad.sum())} elements off"
        assert err.max().item() <= FP8_MAX_ABS, err.max().item()
    else:
        torch.testing.assert_close(out, ref, rtol=rtol, atol=atol)
    # and the typical error is far below the bar
    assert err.mean() <= 0.1 * atol + 0.01 * ref.abs().mean()


# ------------------------------------------------------------- grouped GEMM
ROWS = [130, 0, 67, 9]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_grouped_gemm_bf16_reference_layout(dev, dt):
    """16-bit weights [E, K, N] of the activations' type, bf16 or fp16 (the
    reference's tests/fused_moe/test_grouped_gemm.py:46 dtypes)."""
    g = torch.Generator().manual_seed(1)
    E, N, K = 4, 384, 256
    M = sum(ROWS)
    a = torch.randn(M, K, generator=g).to(dt)
    b_kn = (torch.randn(E, K, N, generator=g) * 0.05).to(dt)
    bias = (torch.randn(E, N, generator=g) * 0.1).to(dt)
    d = torch.empty(M, N, dtype=dt, device=dev)
    rows = torch.tensor(ROWS, dtype=torch.int32)
    out = _ops().cutlass_grouped_gemm(a.to(dev), b_kn.to(dev), None, bias.to(dev), d,
                                      rows.to(dev), N, K, E)
    ref = O.grouped_gemm("bf16", a, b_kn.transpose(1, 2).contiguous(), None, bias, ROWS,
                         out_dtype=dt)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_grouped_gemm_fp8_block(dev, layout):
    g = torch.Generator().manual_seed(2)
    E, N, K = 4, 512, 1024
    M = sum(ROWS)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=g) * 0.02)
    b = q if layout == "nk" else q.transpose(1, 2).contiguous()
    d = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), b.to(dev), s.to(dev), None, d,
                                torch.tensor(ROWS, dtype=torch.int32, device=dev), N, K, E)
    ref = O.grouped_gemm("fp8block", a, q, s, None, ROWS)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_grouped_gemm_fp8_block_all_finite_e4m3_kat(dev):
    """tests/fused_moe/test_grouped_gemm.py:275-307, bit-exact fp16 output."""
    n, k = 128, 256
    a = torch.eye(k, dtype=torch.float16)
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    b = codes.repeat((n * k + 253) // 254)[:n * k].reshape(1, n, k).view(torch.float8_e4m3fn)
    scales = torch.tensor([[[0.5, 2.0]]])
    out = torch.empty(k, n, dtype=torch.float16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), b.to(dev), scales.to(dev), None, out,
                                torch.tensor([k], dtype=torch.int32, device=dev), n, k, 1)
    ref = (b.float() * scales.repeat_interleave(128, 1).repeat_interleave(128, 2))[0].t()
    torch.testing.assert_close(out.cpu(), ref.half(), rtol=0, atol=0)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_grouped_gemm_mxfp4(dev, dt):
    g = torch.Generator().manual_seed(3)
    E, N, K = 4, 256, 512
    M = sum(ROWS)
    a = torch.randn(M, K, generator=g).to(dt)
    w = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    sc = torch.randint(118, 128, (E, N, K // 32), generator=g, dtype=torch.uint8)
    d = torch.empty(M, N, dtype=dt, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), w.to(dev).view(torch.float4_e2m1fn_x2), sc.to(dev),
                                None, d, torch.tensor(ROWS, dtype=torch.int32, device=dev),
                                N, K, E)
    ref = O.grouped_gemm("mxfp4", a, w, sc, None, ROWS, out_dtype=dt)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_grouped_gemm_mxfp4_zero_scale_code_is_zero(dev):
    """e8m0 code 0 dequantises to 0 (reference gemm_xe2.hpp:411-418)."""
    E, N, K = 1, 64, 64
    a = torch.ones(16, K, dtype=torch.bfloat16)
    w = torch.full((E, N, K // 2), 0x77, dtype=torch.uint8)   # 6.0, 6.0
    sc = torch.full((E, N, K // 32), 127, dtype=torch.uint8)
    sc[0, :, 0] = 0
    d = torch.empty(16, N, dtype=torch.bfloat16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), w.to(dev), sc.to(dev), None, d,
                                torch.tensor([16], dtype=torch.int32, device=dev), N, K, E)
    assert torch.equal(d.cpu().float(), torch.full((16, N), 6.0 * 32))


# -------------------------------------------------------------- fused layer
def _layer(cfg, T, dev, E=None, seed_shift=0):
    """Build weights/inputs of `cfg` (optionally with E experts), route on
    the GPU, run XpuFusedMoe; return everything the oracle needs."""
    W = _W()
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    if E is not None:
        import dataclasses
        cfg = dataclasses.replace(cfg, experts=E)
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, T, dev, seed=1 + seed_shift)
    logits = W.make_router_logits(cfg, T, dev, seed=2 + seed_shift)
    bias = W.make_correction_bias(cfg, dev) if cfg.routing == "grouped_sigmoid" else None
    tw, ti = W.route(cfg, logits, bias)
    # the layer prepares copies in place; w keeps the reference layouts
    moe = XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, cfg.activation, cfg.experts)
    out = torch.empty_like(x)
    moe.apply(out, x, tw, ti)
    return cfg, w, x, tw, ti, out, moe


def _oracle_layer(cfg, w, x, tw, ti, tokens=None, a1q_scale=None, compute_dtype=None):
    """Run the oracle on CPU copies of only the experts the (sampled) tokens
    route to (a1q_scale: x is pre-quantised with these scales; compute_dtype:
    the 16-bit type its GEMM outputs round to, bf16 if None)."""
    if tokens is not None:
        x, tw, ti = x[tokens], tw[tokens], ti[tokens]
        if a1q_scale is not None:
            a1q_scale = a1q_scale[tokens]
    ti_c = ti.cpu().long()
    used = torch.unique(ti_c)
    remap = torch.full((cfg.experts,), -1, dtype=torch.long)
    remap[used] = torch.arange(used.numel())
    ids = remap[ti_c]
    usedd = used.to(w.w13.device)
    if cfg.recipe == "bf16":
        w13 = w.w13.index_select(0, usedd).transpose(1, 2).contiguous().cpu()
        w2 = w.w2.index_select(0, usedd).transpose(1, 2).contiguous().cpu()
    elif cfg.recipe == "mxfp8":   # [E, K, N] + [E, K/32, N] -> [E, N, K] + [E, N, K/32]
        tr = lambda t: t.index_select(0, usedd).transpose(1, 2).contiguous().cpu()  # noqa: E731
        bias = lambda b: None if b is None else b.index_select(0, usedd).cpu()  # noqa: E731
        return O.fused_moe("mxfp8", x.cpu(), tr(w.w13), tr(w.w13_scale), bias(w.w13_bias),
                           tr(w.w2), tr(w.w2_scale), bias(w.w2_bias), tw.cpu(), ids,
                           activation=cfg.activation,
                           a1q_scale=None if a1q_scale is None else a1q_scale.cpu())
    else:
        w13 = w.w13.view(torch.uint8).index_select(0, usedd).cpu()
        w2 = w.w2.view(torch.uint8).index_select(0, usedd).cpu()
        if cfg.recipe == "fp8block":
            w13, w2 = w13.view(torch.float8_e4m3fn), w2.view(torch.float8_e4m3fn)
    s13 = w.w13_scale.index_select(0, usedd).cpu() if w.w13_scale is not None else None
    s2 = w.w2_scale.index_select(0, usedd).cpu() if w.w2_scale is not None else None
    b13 = w.w13_bias.index_select(0, usedd).cpu() if w.w13_bias is not None else None
    b2 = w.w2_bias.index_select(0, usedd).cpu() if w.w2_bias is not None else None
    return O.fused_moe(cfg.recipe, x.cpu(), w13, s13, b13, w2, s2, b2, tw.cpu(), ids,
                       activation=cfg.activation,
                       a1q_scale=None if a1q_scale is None else a1q_scale.cpu(),
                       compute_dtype=compute_dtype)


def test_fused_moe_c1_tiny(dev):
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C1"], 64, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


@pytest.mark.parametrize("T", [1, 16, 64, 256])
def test_fused_moe_c2_qwen3_30b_bf16(dev, T):
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C2"], T, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


@pytest.mark.parametrize("T", [1, 33])
def test_fused_moe_c3_deepseek_fp8_32_experts(dev, T):
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C3"], T, dev, E=32)
    _close(out, _oracle_layer(cfg, w, x, tw, ti), fp8=True)


def test_fused_moe_c3_full_size_every_token(dev):
    """Full DeepSeek-V3 shape (256 experts, T=64, the decode kernels): every
    token against the oracle run on the device, to the fp8 bar."""
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C3"], 64, dev)
    _close(out, _oracle_layer_on_device(cfg, w, x, tw, ti), fp8=True)


@pytest.mark.parametrize("T", [1, 256, 2048, 8192])
def test_fused_moe_fp8block_swigluoai_c3(dev, T):
    """fp8 block-scaled weights with an interleaved swigluoai w13 (gate row
    2j, up row 2j + 1, 128 x 128 scale blocks) at the DeepSeek-V3 shape (256
    experts, H=7168, I=2048): the layer splits the rows into gate and up
    halves read with one scale row per 64 weight rows, through the decode
    (T=1), small (T=256), 128-slot (T=2048) and 320-slot (T=8192) kernels;
    every token against the oracle run on the device (interleaved rows, the
    reference's block scales), to the fp8 bar."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C3"], activation="swigluoai")
    cfg, w, x, tw, ti, out, moe = _layer(cfg, T, dev)
    assert moe._ws_rows == 64 and moe.gemm1_wei_scales.shape[1] == 2 * cfg.inter // 64
    _close(out, _oracle_layer_on_device(cfg, w, x, tw, ti), fp8=True)


def test_fused_moe_c4_zipf_fp8(dev):
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C4"], 256, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti), fp8=True)


@pytest.mark.parametrize("T", [1, 32, 128])
def test_fused_moe_c5_gpt_oss_mxfp4_swigluoai(dev, T):
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS["C5"], T, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


@pytest.mark.parametrize("name,T", [("C2", 256), ("C2", 1), ("C3", 1)])
def test_fused_moe_deterministic(dev, name, T):
    """Bit-identical repeats; at T=1 the decode GEMMs split K over workgroups
    and a second launch sums the partial tiles in a fixed order."""
    cfg, w, x, tw, ti, out, moe = _layer(_W().CONFIGS[name], T, dev)
    for _ in range(3):
        again = torch.empty_like(out)
        moe.apply(again, x, tw, ti)
        assert torch.equal(out, again)


def test_fused_moe_expert_map(dev):
    """EP on one device: half of 16 experts local, others dropped
    (reference tests/fused_moe/test_fused_moe.py:539-657 method)."""
    import dataclasses
    W = _W()
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    cfg = dataclasses.replace(W.CONFIGS["C1"], experts=16)
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, 48, dev)
    tw, ti = W.route(cfg, W.make_router_logits(cfg, 48, dev))
    em = torch.full((16,), -1, dtype=torch.int32, device=dev)
    em[8:] = torch.arange(8, dtype=torch.int32, device=dev)
    # the rank's experts as new tensors (a slice would share w's storage,
    # which the layer's preparation rewrites)
    moe = XpuFusedMoe(w.w13[8:].clone(), None, None, w.w2[8:].clone(), None,
                      None, cfg.topk, "silu", 8, ep_rank=1, ep_size=2, expert_map=em)
    out = torch.empty_like(x)
    moe.apply(out, x, tw, ti, expert_map=em)
    # oracle: drop non-local slots
    tw_c = torch.where(ti >= 8, tw, torch.zeros_like(tw))
    ref = _oracle_layer(cfg, w, x, tw_c, ti)
    _close(out, ref)


# ------------------------------------------------- prefill (128x256) tiles
BIG_ROWS = [300, 260, 0, 129]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("recipe", ["bf16", "fp8block", "mxfp4"])
def test_grouped_gemm_big_tiles(dev, recipe, dt):
    """>96 rows per expert: bf16 and fp8 select the 320x256 kernels, mxfp4
    the LDS-staged 128x256 one; N=2880 is not a multiple of the tile (ragged
    last tile)."""
    g = torch.Generator().manual_seed(4)
    E, K = 4, 1024
    N = 640 if recipe == "fp8block" else 2880
    M = sum(BIG_ROWS)
    a = torch.randn(M, K, generator=g).to(dt)
    rows = torch.tensor(BIG_ROWS, dtype=torch.int32)
    d = torch.empty(M, N, dtype=dt, device=dev)
    if recipe == "bf16":
        b = (torch.randn(E, N, K, generator=g) * 0.03).to(dt)
        bias = (torch.randn(E, N, generator=g) * 0.1).to(dt)
        _ops().cutlass_grouped_gemm(a.to(dev), b.transpose(1, 2).contiguous().to(dev), None,
                                    bias.to(dev), d, rows.to(dev), N, K, E)
        ref = O.grouped_gemm("bf16", a, b, None, bias, BIG_ROWS, out_dtype=dt)
    elif recipe == "fp8block":
        q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=g) * 0.02)
        _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), s.to(dev), None, d, rows.to(dev),
                                    N, K, E)
        ref = O.grouped_gemm("fp8block", a, q, s, None, BIG_ROWS, out_dtype=dt)
    else:
        q, sc = O.to_mxfp4(torch.randn(E, N, K, generator=g) * 0.05)
        _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), sc.to(dev), None, d, rows.to(dev),
                                    N, K, E)
        ref = O.grouped_gemm("mxfp4", a, q, sc, None, BIG_ROWS, out_dtype=dt)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


# ------------------------------------------- bf16 prefill (320x256) tiles
WIDE_ROWS = [1, 31, 33, 64, 97, 159, 160, 161, 255, 319, 320, 321, 700]


@pytest.mark.parametrize("K", [32, 64, 96, 352])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_grouped_gemm_wide_tiles(dev, K, out_dtype):
    """bf16 weights with >96 rows per expert select the 320x256 kernel.
    Valid rows per 320-slot block 1..320 (every count of 32-row MFMA groups
    per wave half, 0..5, and of skipped 16-row DMA groups; experts of 1, 2
    and 3 blocks); K from one 32-element stage (shorter than the 3-deep
    prefetch) to 11; N=200 is one ragged tile; bias; bf16 or fp16 operands
    and output (one 16-bit type per call)."""
    g = torch.Generator().manual_seed(K)
    E, N = len(WIDE_ROWS), 200
    M = sum(WIDE_ROWS)
    a = torch.randn(M, K, generator=g).to(out_dtype)
    b = (torch.randn(E, N, K, generator=g) * 0.05).to(out_dtype)
    bias = (torch.randn(E, N, generator=g) * 0.1).to(out_dtype)
    rows = torch.tensor(WIDE_ROWS, dtype=torch.int32)
    d = torch.full((M, N), float("nan"), dtype=out_dtype, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), b.transpose(1, 2).contiguous().to(dev), None,
                                bias.to(dev), d, rows.to(dev), N, K, E)
    ref = O.grouped_gemm("bf16", a, b, None, bias, WIDE_ROWS, out_dtype=out_dtype)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
def test_fused_moe_wide_tiles_ragged(dev, activation):
    """Whole bf16 layer through the 320x256 kernels (256 slots per expert on
    average): I=224 leaves a ragged GLU tile and a 7-stage w2 K loop, H=352
    an 11-stage w13 loop; swigluoai adds biases and the clamps."""
    import dataclasses
    base = _W().CONFIGS["C5" if activation == "swigluoai" else "C2"]
    cfg = dataclasses.replace(base, recipe="bf16", hidden=352, inter=224, experts=8, topk=2)
    cfg, w, x, tw, ti, out, _ = _layer(cfg, 1024, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


# ------------------------------------------- fp8 prefill (320x256) tiles
W8_ROWS = [1, 15, 17, 64, 100, 159, 160, 161, 200, 319, 320, 321, 700, 1000, 1200]


@pytest.mark.parametrize("K", [128, 384, 1024])
def test_grouped_gemm_wide8_tiles(dev, K):
    """fp8 block-scaled weights with >160 rows per expert select the 320x256
    kernel.  Valid rows per 320-slot block 1..320 (every count of 16-slot
    MFMA tiles per wave half, 0..10, skipped 8-row DMA groups and 64-slot
    scale groups); experts of 1, 2 and 3 blocks; K from one 128-element
    stage (no DMA ahead) to 8; N=640 is two and a half 256-row tiles."""
    g = torch.Generator().manual_seed(K + 1)
    E, N = len(W8_ROWS), 640
    M = sum(W8_ROWS)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=g) * 0.02)
    rows = torch.tensor(W8_ROWS, dtype=torch.int32)
    d = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), s.to(dev), None, d, rows.to(dev),
                                N, K, E)
    ref = O.grouped_gemm("fp8block", a, q, s, None, W8_ROWS)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_grouped_gemm_big8_tiles(dev):
    """fp8 block-scaled weights with 97..160 rows per expert select the
    128x256 8-wave kernel (128-slot blocks; experts of 1 and 2 blocks, a
    partial last block)."""
    g = torch.Generator().manual_seed(13)
    rows_l = [129, 100, 150, 0, 201]
    E, N, K = len(rows_l), 384, 512
    M = sum(rows_l)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=g) * 0.02)
    d = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), s.to(dev), None, d,
                                torch.tensor(rows_l, dtype=torch.int32, device=dev), N, K, E)
    ref = O.grouped_gemm("fp8block", a, q, s, None, rows_l)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_grouped_gemm_fp8_k_beyond_wide8(dev):
    """K = 8320 exceeds the 320-slot kernel's scale table (64 blocks of 128):
    the 128x256 LDS pipeline kernel runs instead."""
    g = torch.Generator().manual_seed(11)
    rows_l = [150, 300]
    E, N, K = 2, 256, 8320
    M = sum(rows_l)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q, s = O.fp8_block_quant_weight(torch.randn(E, N, K, generator=g) * 0.01)
    d = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), s.to(dev), None, d,
                                torch.tensor(rows_l, dtype=torch.int32, device=dev), N, K, E)
    ref = O.grouped_gemm("fp8block", a, q, s, None, rows_l)
    torch.testing.assert_close(d.cpu().float(), ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("T", [1024, 700])
def test_fused_moe_wide8_ragged(dev, T):
    """Whole fp8 block-scaled layer through the 320x256 kernels: the w13
    epilogue re-quantises the activation to e4m3 (1x128 groups) in LDS;
    T=700 leaves about 175 slots per expert (second wave half nearly idle)."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C2"], recipe="fp8block", hidden=384, inter=256,
                              experts=8, topk=2)
    cfg, w, x, tw, ti, out, _ = _layer(cfg, T, dev)
    _close(out, _oracle_layer(cfg, w, x, tw, ti), fp8=True)


# ---------------------------------------------- K-blocked bf16 / fp8 weights
@pytest.mark.parametrize("shape", [(3, 72, 256), (2, 768, 2048), (1, 8, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
def test_pack_weights_kblock_layout(dev, shape, dtype):
    """[E, N, K] -> [E, K/B, N, B] (B = 32 for 16-bit, 128 for e4m3): element
    (e, n, k) lands at (e, k // B, n, k % B)."""
    from vllm_xpu_kernels.fused_moe_interface import pack_weights_kblock
    E, N, K = shape
    B = 128 if dtype == torch.float8_e4m3fn else 32
    g = torch.Generator().manual_seed(7)
    w = torch.randn(E, N, K, generator=g).to(dtype)
    ib = torch.uint8 if B == 128 else torch.int16
    out = pack_weights_kblock(w.to(dev)).cpu()
    assert out.shape == (E, K // B, N, B)
    e, n, k = (torch.randint(0, d, (4096,), generator=g) for d in (E, N, K))
    assert torch.equal(out.view(ib)[e, k // B, n, k % B], w.view(ib)[e, n, k])
    assert torch.equal(out.view(ib),
                       w.view(ib).view(E, N, K // B, B).permute(0, 2, 1, 3).contiguous())


def _layer_both_layouts(cfg, T, dev, monkeypatch):
    monkeypatch.setenv("MI355MOE_WEIGHT_LAYOUT", "nk")
    _, _, _, _, _, out_nk, moe_nk = _layer(cfg, T, dev)
    monkeypatch.delenv("MI355MOE_WEIGHT_LAYOUT")
    res = _layer(cfg, T, dev)
    assert moe_nk._w_layout == 0 and res[6]._w_layout == 1
    return res, out_nk


@pytest.mark.parametrize("T", [1, 16, 256, 512, 1024, 2048])
def test_fused_moe_kblock_equals_nk_c2(dev, monkeypatch, T):
    """The K-blocked layout changes addresses only: every kernel family (T=1
    split-K stream, 16 stream, 256/512 small, 1024/2048 wide) gives the
    row-major layer's output bit for bit, and that output meets the oracle."""
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(_W().CONFIGS["C2"], T, dev,
                                                             monkeypatch)
    assert torch.equal(out, out_nk)
    toks = torch.linspace(0, T - 1, min(T, 8)).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks))


@pytest.mark.parametrize("T", [8, 96, 160, 1024])
@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
def test_fused_moe_kblock_ragged(dev, monkeypatch, activation, T):
    """H=352 / I=224: K loops that end inside a 128-wide stage (stream,
    small) and GLU tiles with rows past I, over the K-blocked weights."""
    import dataclasses
    base = _W().CONFIGS["C5" if activation == "swigluoai" else "C2"]
    cfg = dataclasses.replace(base, recipe="bf16", hidden=352, inter=224, experts=8, topk=2)
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(cfg, T, dev, monkeypatch)
    assert torch.equal(out, out_nk)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
@pytest.mark.parametrize("T", [8, 32, 48, 96, 500, 1024])
def test_fused_moe_kblock_fp8_families(dev, monkeypatch, T, activation):
    """fp8 block-scaled weights K-blocked in 128-byte blocks (H=384, I=256,
    8 experts, top-2: about T/4 slots per expert): stream (T=8), small
    (32, 48), 128-slot 8-wave (96, 500) and 320-slot (1024) kernels each give
    the row-major layer's output bit for bit, within the fp8 bar of the
    oracle; swigluoai (interleaved rows, read as gate / up halves with
    64-row scale blocks) through the same kernels."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C2"], recipe="fp8block", hidden=384, inter=256,
                              experts=8, topk=2, activation=activation)
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(cfg, T, dev, monkeypatch)
    assert torch.equal(out, out_nk)
    _close(out, _oracle_layer(cfg, w, x, tw, ti), fp8=True)


@pytest.mark.parametrize("shape", [(3, 72, 256), (2, 64, 2880)])
def test_pack_mxfp4_kblock_layout(dev, shape):
    """e2m1 pairs u8 [E, N, K/2] -> [E, K/32, N, 16] and e8m0 scales
    [E, N, K/32] -> [E, K/32, N]."""
    from vllm_xpu_kernels.fused_moe_interface import pack_scales_kblock, pack_weights_kblock
    E, N, K = shape
    g = torch.Generator().manual_seed(9)
    w = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    sc = torch.randint(0, 256, (E, N, K // 32), generator=g, dtype=torch.uint8)
    pw = pack_weights_kblock(w.to(dev)).cpu()
    ps = pack_scales_kblock(sc.to(dev)).cpu()
    assert pw.shape == (E, K // 32, N, 16) and ps.shape == (E, K // 32, N)
    assert torch.equal(pw, w.view(E, N, K // 32, 16).permute(0, 2, 1, 3))
    assert torch.equal(ps, sc.permute(0, 2, 1))


@pytest.mark.parametrize("T", [8, 96, 160])
def test_fused_moe_kblock_mxfp4_families(dev, monkeypatch, T):
    """mxfp4 weights and e8m0 scales K-blocked (32-value blocks; H=320,
    I=256, swigluoai with biases, 8 experts, top-2): stream (T=8) and small
    (96: 16-slot blocks, 160: 32-slot blocks) kernels give the row-major
    layer's output bit for bit, within the bar of the oracle."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C5"], hidden=320, inter=256, experts=8, topk=2)
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(cfg, T, dev, monkeypatch)
    assert torch.equal(out, out_nk)
    _close(out, _oracle_layer(cfg, w, x, tw, ti))


def _assert_near_layouts(out, out_nk):
    """Two kernel families over the same operands: fp32 sums in different
    orders, so the bf16 outputs may differ in the last place only."""
    a, b = out.float(), out_nk.float()
    assert torch.isfinite(a).all()
    assert ((a - b).abs() <= 1e-2 * b.abs() + 1e-3).all()


@pytest.mark.parametrize("shape", [(320, 256, 1024), (320, 256, 2000), (352, 160, 700),
                                   (96, 64, 1200)])
def test_fused_moe_mxfp4_wide(dev, monkeypatch, shape):
    """K-blocked mxfp4 layers whose experts average > 96 slots run the
    320-slot mxfp4 kernel (row-major weights: the 128-slot register-staged
    one): H=320 / I=256 (10 and 8 K stages), H=352 / I=160 (11 and 5 K
    stages: GLU and STORE tiles with columns past N), H=96 / I=64 (K loops
    shorter than the DMA lookahead).  Within the oracle's bar and near the
    row-major layer's output."""
    import dataclasses
    H, I, T = shape
    cfg = dataclasses.replace(_W().CONFIGS["C5"], hidden=H, inter=I, experts=8, topk=2)
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(cfg, T, dev, monkeypatch)
    _assert_near_layouts(out, out_nk)
    toks = torch.linspace(0, T - 1, min(T, 64)).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks))


@pytest.mark.parametrize("hot", [0.0, 0.6, 1.0])
def test_fused_moe_mxfp4_wide_skewed(dev, hot):
    """Skewed routing over the 320-slot mxfp4 kernel: a share `hot` of the
    tokens put expert 3 first, so the experts hold from a few slots (blocks
    with one or two 32-row groups) to several full 320-slot blocks."""
    import dataclasses
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    T = 1500
    cfg = dataclasses.replace(W.CONFIGS["C5"], hidden=320, inter=256, experts=8, topk=2)
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, T, dev, seed=5)
    g = torch.Generator().manual_seed(17)
    first = torch.where(torch.rand(T, generator=g) < hot, torch.full((T,), 3),
                        torch.randint(0, 8, (T,), generator=g))
    second = (first + 1 + torch.randint(0, 7, (T,), generator=g)) % 8
    ti = torch.stack([first, second], 1).to(torch.int32).to(dev)
    tw = torch.rand(T, 2, generator=g) + 0.1
    tw = (tw / tw.sum(1, keepdim=True)).to(dev)
    moe = XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, cfg.activation, cfg.experts)
    assert moe._w_layout == 1
    out = torch.empty_like(x)
    moe.apply(out, x, tw, ti)
    toks = torch.linspace(0, T - 1, 96).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks))


@pytest.mark.parametrize("T", [1, 16, 48, 300, 1024])
def test_fused_moe_a1q_scale_pre_quantised(dev, T):
    """Pre-quantised hidden states (a1q_scale, fp8block; H=384, I=256, 8
    experts, top-2): the (q, s) of the layer's own 1x128 quantiser give its
    bf16-input output bit for bit in every family (T=1 split-K stream, 16
    stream, 48 small, 300 128-slot, 1024 320-slot); other scales (ue8m0)
    meet the oracle run on the same pre-quantised input."""
    import dataclasses
    from vllm_xpu_kernels import ops
    cfg = dataclasses.replace(_W().CONFIGS["C2"], recipe="fp8block", hidden=384, inter=256,
                              experts=8, topk=2)
    cfg, w, x, tw, ti, out, moe = _layer(cfg, T, dev)
    xq, xs = ops.per_token_group_fp8_quant(x, 128)
    out2 = torch.empty_like(out)
    moe.apply(out2, xq, tw, ti, a1q_scale=xs)
    assert torch.equal(out2, out)
    xq3, xs3 = ops.per_token_group_fp8_quant(x, 128, scale_ue8m0=True)
    out3 = torch.empty_like(out)
    moe.apply(out3, xq3, tw, ti, a1q_scale=xs3)
    toks = torch.linspace(0, T - 1, min(T, 64)).long().to(dev)
    _close(out3[toks], _oracle_layer(cfg, w, xq3, tw, ti, toks, a1q_scale=xs3), fp8=True)


@pytest.mark.parametrize("recipe", ["bf16", "fp8block", "mxfp4"])
@pytest.mark.parametrize("act", ["gelu", "gelu_tanh", "swiglustep", "relu2_no_mul"])
@pytest.mark.parametrize("T", [2, 48, 1024])
def test_fused_moe_generic_activations(dev, recipe, act, T):
    """Activations with no GEMM-epilogue form (w13 stores G1, one kernel
    applies the activation and, for fp8, the 1x128 re-quantisation; relu2_no_mul
    keeps 2I columns, so w2 has K = 2I): H=384, I=256, 8 experts, top-2,
    T = 2 (split-K stream), 48 (small), 1024 (320-slot) against the oracle."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C2"], recipe=recipe, hidden=384, inter=256,
                              experts=8, topk=2, activation=act)
    cfg, w, x, tw, ti, out, moe = _layer(cfg, T, dev)
    toks = torch.linspace(0, T - 1, min(T, 48)).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks), fp8=recipe == "fp8block")


def test_fused_moe_generic_activation_clamp(dev):
    """gemm1_clamp_limit on the bf16 halves before the activation."""
    import dataclasses
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    for act in ("gelu", "relu2_no_mul"):
        cfg = dataclasses.replace(W.CONFIGS["C2"], hidden=256, inter=128, experts=4, topk=2,
                                  activation=act)
        w = W.make_weights(cfg, dev)
        x = W.make_activations(cfg, 40, dev) * 30
        tw, ti = W.route(cfg, W.make_router_logits(cfg, 40, dev))
        moe = XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, act, cfg.experts,
                          gemm1_clamp_limit=0.5)
        out = torch.empty_like(x)
        moe.apply(out, x, tw, ti)
        ref = _oracle_layer(cfg, w, x, tw, ti)
        ti_c = ti.cpu().long()
        used = torch.unique(ti_c)
        remap = torch.full((cfg.experts,), -1, dtype=torch.long)
        remap[used] = torch.arange(used.numel())
        ref = O.fused_moe("bf16", x.cpu(),
                          w.w13.index_select(0, used.to(dev)).transpose(1, 2).contiguous().cpu(),
                          None, None,
                          w.w2.index_select(0, used.to(dev)).transpose(1, 2).contiguous().cpu(),
                          None, None, tw.cpu(), remap[ti_c], activation=act,
                          gemm1_clamp_limit=0.5)
        _close(out, ref)


@pytest.mark.parametrize("recipe", ["bf16", "fp8block", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("T", [1, 16, 48, 300, 1024])
def test_fused_moe_fp16(dev, recipe, T):
    """fp16 hidden states, output and biases (16-bit recipe: fp16 weights;
    mxfp4 dequantised to fp16) through every kernel family (H=384, I=256, 8
    experts, top-2; T=1 split-K stream ... 1024 320-slot), at the reference's
    fp16 bar rtol = atol = 1e-2 (tests/fused_moe/test_fused_moe.py:288-294;
    fp8 at its own bar).  mxfp4 runs swigluoai with biases, the others SiLU."""
    import dataclasses
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    cfg = dataclasses.replace(W.CONFIGS["C5" if recipe == "mxfp4" else "C2"], recipe=recipe,
                              hidden=384, inter=256, experts=8, topk=2, bias=True)
    w = W.make_weights(cfg, dev)
    h = torch.float16
    w = dataclasses.replace(w, w13=w.w13.to(h) if recipe == "bf16" else w.w13,
                            w2=w.w2.to(h) if recipe == "bf16" else w.w2,
                            w13_bias=w.w13_bias.to(h), w2_bias=w.w2_bias.to(h))
    x = W.make_activations(cfg, T, dev).to(h)
    tw, ti = W.route(cfg, W.make_router_logits(cfg, T, dev))
    moe = XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, cfg.activation, cfg.experts)
    out = torch.empty_like(x)
    moe.apply(out, x, tw, ti)
    toks = torch.linspace(0, T - 1, min(T, 48)).long().to(dev)
    ref = _oracle_layer(cfg, w, x, tw, ti, toks)
    assert ref.dtype == h
    if recipe in ("fp8block", "mxfp8"):
        _close(out[toks], ref, fp8=True)
    else:
        _close(out[toks], ref, rtol=1e-2, atol=1e-2)


def test_fused_moe_fp16_bias_follows_call_dtype(dev):
    """bf16 biases with fp16 activations (fp8 weights): converted once to the
    call's type; a bf16 call with the same layer reuses the originals."""
    import dataclasses
    W = _W()
    cfg = dataclasses.replace(W.CONFIGS["C2"], recipe="fp8block", hidden=256, inter=128,
                              experts=4, topk=2, bias=True)
    cfg, w, x, tw, ti, out, moe = _layer(cfg, 24, dev)
    out16 = torch.empty_like(x, dtype=torch.float16)
    moe.apply(out16, x.half(), tw, ti)
    _close(out16.float(), out.float(), fp8=True)
    assert torch.float16 in moe._bias_cache


def _fp8_expert_weights(E, N, K, fp8, g):
    """[E, N, K] weights randn/16 quantised per expert with power-of-two
    scales 2^-3..2^3 (the reference's tests/fused_moe/test_fused_moe.py:
    226-246 recipe); returns (q nk, scales [E])."""
    w = torch.randn(E, N, K, generator=g) / 16
    s = torch.pow(2.0, torch.randint(-3, 4, (E,), generator=g).float())
    fmax = torch.finfo(fp8).max
    return (w / s.view(E, 1, 1)).clamp(-fmax, fmax).to(fp8), s


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fp8", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("has_bias", [False, True])
def test_grouped_gemm_fp8_per_expert(dev, dt, fp8, has_bias):
    """Per-expert fp8 weights [E, K, N] (e5m2 or e4m3) with fp32 scales [E]
    (reference tests/fused_moe/test_grouped_gemm.py:153-221): D = T(s_e A W_e +
    bias), within rtol = atol = 1e-2 of the oracle."""
    g = torch.Generator().manual_seed(21)
    E, N, K = 4, 384, 512
    M = sum(ROWS)
    a = torch.randn(M, K, generator=g).to(dt)
    q, sc = _fp8_expert_weights(E, N, K, fp8, g)
    bias = (torch.randn(E, N, generator=g) * 100).to(dt) if has_bias else None
    d = torch.empty(M, N, dtype=dt, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), q.transpose(1, 2).contiguous().to(dev), sc.to(dev),
                                None if bias is None else bias.to(dev), d,
                                torch.tensor(ROWS, dtype=torch.int32, device=dev), N, K, E)
    ref = O.grouped_gemm("fp8", a, q, sc, bias, ROWS, out_dtype=dt)
    torch.testing.assert_close(d.cpu(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fp8", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("T,topk", [(1, 1), (4, 1), (16, 1), (512, 1), (2048, 2)])
def test_fused_moe_fp8_per_expert(dev, dt, fp8, T, topk):
    """The reference's per-expert fp8 layer (tests/fused_moe/test_fused_moe.py:
    179-295, Llama-4-scout structure at H=1024, I=512, 16 experts): weights
    [E, K, N] e5m2 / e4m3 with scales [E], biases, raw top-k scores as
    weights, bf16 or fp16; every element within the reference's bar (bf16
    2e-2, fp16 1e-2).  T covers the split-K stream, stream, small and 320-slot
    kernels; the oracle checks 64 sampled tokens at T=2048."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    g = torch.Generator().manual_seed(7 + T)
    E, H, I = 16, 1024, 512
    q13, s13 = _fp8_expert_weights(E, 2 * I, H, fp8, g)
    q2, s2 = _fp8_expert_weights(E, H, I, fp8, g)
    b13 = (torch.randn(E, 2 * I, generator=g) / 16).to(dt)
    b2 = (torch.randn(E, H, generator=g) / 16).to(dt)
    x = (torch.randn(T, H, generator=g) / 16).to(dt)
    tw, ti = torch.topk(torch.randn(T, E, generator=g), k=topk, dim=-1, sorted=False)
    moe = XpuFusedMoe(q13.transpose(1, 2).contiguous().to(dev), s13.to(dev), b13.to(dev),
                      q2.transpose(1, 2).contiguous().to(dev), s2.to(dev), b2.to(dev),
                      topk, "silu", E)
    assert moe.recipe == "fp8"
    out = torch.empty(T, H, dtype=dt, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, min(T, 64)).long()
    ref = O.fused_moe("fp8", x[toks], q13, s13, b13, q2, s2, b2, tw[toks], ti[toks])
    tol = 2e-2 if dt == torch.bfloat16 else 1e-2
    torch.testing.assert_close(out.cpu()[toks], ref, rtol=tol, atol=tol)


def _finite_fp8_codes(fp8):
    """Every byte whose fp8 value is finite (e4m3fn: all but 0x7f / 0xff;
    e5m2: all but the Inf / NaN codes 0x7c-0x7f, 0xfc-0xff)."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    return codes[torch.isfinite(codes.view(fp8).float())]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fp8", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("scale", [1.0, 0.125])
def test_per_expert_fp8_weight_conversion_kat(dev, dt, fp8, scale):
    """Per-expert fp8 weights read as they are (C ABI recipe FP8 / FP8E5M2,
    grouped GEMM): against one-hot activation rows every output is one
    weight times the expert scale, so each finite code's conversion to the
    16-bit type shows exactly: D[m, n] = T(s * W[n, m]).  Row n holds every
    finite code, rotated by n."""
    import ctypes
    from vllm_xpu_kernels import capi
    lib = capi.lib
    codes = _finite_fp8_codes(fp8)
    K = N = 256
    idx = (torch.arange(N).view(N, 1) + torch.arange(K).view(1, K)) % K
    wb = torch.zeros(K, dtype=torch.uint8)
    wb[:codes.numel()] = codes
    w = wb[idx].view(fp8)                                  # [N, K]
    a = torch.eye(K, dtype=dt)                             # M = K one-hot rows
    recipe = 5 if fp8 == torch.float8_e4m3fn else 6
    adt = capi.F16 if dt == torch.float16 else capi.BF16
    lib.mi355moe_grouped_gemm_workspace_size_k.restype = ctypes.c_size_t
    lib.mi355moe_grouped_gemm_workspace_size_k.argtypes = [ctypes.c_int, ctypes.c_int] + \
        [ctypes.c_int64] * 3
    lib.mi355moe_grouped_gemm.argtypes = (
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p] +
        [ctypes.c_int64] * 4 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p])
    wsb = lib.mi355moe_grouped_gemm_workspace_size_k(recipe, adt, K, K, 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    A, W = a.to(dev), w.to(dev).contiguous()
    sc = torch.tensor([scale], dtype=torch.float32, device=dev)
    rows = torch.tensor([K], dtype=torch.int32, device=dev)
    D = torch.full((K, N), float("nan"), dtype=dt, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.mi355moe_grouped_gemm(recipe, A.data_ptr(), adt, None, W.data_ptr(),
                                   sc.data_ptr(), None, D.data_ptr(), adt, rows.data_ptr(),
                                   K, N, K, 1, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, lib.mi355moe_last_error()
    torch.cuda.synchronize()
    want = (w.float() * scale).to(dt).t()                  # exact: a power-of-two scale
    assert torch.equal(D.cpu(), want)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fp8", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("shape", ["T1", "T2-k8", "T8", "C3-T1", "C2-T1", "rowmajor-T2",
                                   "k-tail-T2", "small-T256", "small-C2-T64",
                                   "small-rowmajor-T256", "prefill-T1024",
                                   "prefill-ragged-T1024", "prefill-rowmajor-T1024"])
def test_fused_moe_fp8_per_expert_reads_fp8(dev, monkeypatch, dt, fp8, shape):
    """Per-expert fp8 layers read the fp8 weights themselves (converted
    exactly in registers; no 16-bit copies are made): every element within
    the reference's bar of the oracle (bf16 2e-2, fp16 1e-2; 64 sampled
    tokens) and of the 16-bit-copy path (MI355MOE_FP8_W8A16=0).  STREAM
    shapes: split-K and self-sorting w13 (T1), 16 slots (T2-k8), C3's
    token-major w2 (C3-T1, H = 7168), C2's w2 rebuilding its rows from the
    w13 partials (C2-T1).  SMALL shapes (32 slots per expert): GLU and STORE
    kernels.  320-slot shapes (128 slots per expert): K-blocked weights,
    also with I = 544 (a last GLU tile of 32 columns, H = 1056: a 32-value K
    tail of the 128-value blocks); row-major weights (MI355MOE_WEIGHT_LAYOUT
    = nk) run the STREAM / SMALL kernels.  With H = 1000 (not % 32) the
    layer runs on the copies."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    g = torch.Generator().manual_seed(11)
    E, H, I, T, topk = 16, 1024, 512, 1, 2
    if shape == "T2-k8":
        T, topk = 2, 8
    elif shape == "T8":
        T = 8
    elif shape == "C3-T1":
        E, H, I, topk = 8, 7168, 2048, 8
    elif shape == "C2-T1":
        E, H, I, topk = 16, 2048, 768, 8
    elif shape == "rowmajor-T2":
        H, I, T = 1056, 544, 2
        monkeypatch.setenv("MI355MOE_WEIGHT_LAYOUT", "nk")
    elif shape == "k-tail-T2":
        H, I, T = 1000, 520, 2
    elif shape == "small-T256":
        T = 256
    elif shape == "small-C2-T64":
        E, H, I, T, topk = 16, 2048, 768, 64, 8
    elif shape == "small-rowmajor-T256":
        H, I, T = 1056, 544, 256
        monkeypatch.setenv("MI355MOE_WEIGHT_LAYOUT", "nk")
    elif shape == "prefill-T1024":
        T = 1024
    elif shape == "prefill-ragged-T1024":
        H, I, T = 1056, 544, 1024
    elif shape == "prefill-rowmajor-T1024":
        T = 1024
        monkeypatch.setenv("MI355MOE_WEIGHT_LAYOUT", "nk")
    q13, s13 = _fp8_expert_weights(E, 2 * I, H, fp8, g)
    q2, s2 = _fp8_expert_weights(E, H, I, fp8, g)
    b13 = (torch.randn(E, 2 * I, generator=g) / 16).to(dt)
    b2 = (torch.randn(E, H, generator=g) / 16).to(dt)
    x = (torch.randn(T, H, generator=g) / 16).to(dt)
    tw, ti = torch.topk(torch.randn(T, E, generator=g), k=topk, dim=-1, sorted=False)
    moe = XpuFusedMoe(q13.transpose(1, 2).contiguous().to(dev), s13.to(dev), b13.to(dev),
                      q2.transpose(1, 2).contiguous().to(dev), s2.to(dev), b2.to(dev),
                      topk, "silu", E)
    native = shape != "k-tail-T2"
    assert (moe._w8_recipe is not None) == native
    if native:
        assert moe._w8_layout == (0 if "rowmajor" in shape else 1)
    xd, twd, tid = x.to(dev), tw.to(dev), ti.to(dev)
    out = torch.full((T, H), float("nan"), dtype=dt, device=dev)
    moe.apply(out, xd, twd, tid)
    torch.cuda.synchronize()
    assert bool(moe._w16_cache) != native         # copies only where the layer needs them
    monkeypatch.setenv("MI355MOE_FP8_W8A16", "0")
    ref16 = torch.full_like(out, float("nan"))
    moe.apply(ref16, xd, twd, tid)
    toks = torch.linspace(0, T - 1, min(T, 64)).long()
    ref = O.fused_moe("fp8", x[toks], q13, s13, b13, q2, s2, b2, tw[toks], ti[toks])
    tol = 2e-2 if dt == torch.bfloat16 else 1e-2
    torch.testing.assert_close(out.cpu()[toks], ref, rtol=tol, atol=tol)
    torch.testing.assert_close(out, ref16, rtol=tol, atol=tol)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("grp", [128, 32])
@pytest.mark.parametrize("has_bias", [False, True])
def test_grouped_gemm_int4(dev, dt, grp, has_bias):
    """int4 weights (reference tests/fused_moe/test_grouped_gemm.py:358-420):
    u4 [E, N, K/2] with zero point 8 converted to two's complement, 16-bit
    scales [E, N, K/group]; within rtol = atol = 1e-2 of the oracle."""
    g = torch.Generator().manual_seed(31)
    E, N, K = 4, 256, 512
    M = sum(ROWS)
    a = torch.randn(M, K, generator=g).to(dt)
    u = torch.randint(0, 0xff, (E, N, K // 2), generator=g).to(torch.uint8)
    sc = torch.pow(2.0, torch.randint(-3, 4, (E, N, K // grp), generator=g).float()).to(dt)
    q = (u ^ 0x88).view(torch.int8)
    bias = (torch.randn(E, N, generator=g) * 100).to(dt) if has_bias else None
    d = torch.empty(M, N, dtype=dt, device=dev)
    _ops().cutlass_grouped_gemm(a.to(dev), q.to(dev), sc.to(dev),
                                None if bias is None else bias.to(dev), d,
                                torch.tensor(ROWS, dtype=torch.int32, device=dev), N, K, E)
    ref = O.grouped_gemm("int4", a, q, sc, bias, ROWS, out_dtype=dt)
    torch.testing.assert_close(d.cpu(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,topk", [(1, 1), (4, 1), (16, 2), (512, 1), (2048, 2)])
def test_fused_moe_int4(dev, dt, T, topk):
    """The reference's int4 layer (tests/fused_moe/test_fused_moe.py:303-420 at
    H=1024, I=512, 16 experts, group 128): u4 weights with zero point 8, scales
    2^-5 in the activation type, biases; every element within the reference's
    bar.  T covers the split-K stream, stream, small and 320-slot kernels
    (K-blocked int4 weights and scales)."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    g = torch.Generator().manual_seed(11 + T)
    E, H, I, grp = 16, 1024, 512, 128
    u13 = torch.randint(0, 0xff, (E, 2 * I, H // 2), generator=g).to(torch.uint8)
    u2 = torch.randint(0, 0xff, (E, H, I // 2), generator=g).to(torch.uint8)
    s13 = torch.full((E, 2 * I, H // grp), 2.0 ** -5).to(dt)
    s2 = torch.full((E, H, I // grp), 2.0 ** -5).to(dt)
    b13 = (torch.randn(E, 2 * I, generator=g) / 16).to(dt)
    b2 = (torch.randn(E, H, generator=g) / 16).to(dt)
    x = (torch.randn(T, H, generator=g) / 16).to(dt)
    tw, ti = torch.topk(torch.randn(T, E, generator=g), k=topk, dim=-1, sorted=False)
    moe = XpuFusedMoe(u13.to(dev), s13.to(dev), b13.to(dev), u2.to(dev), s2.to(dev), b2.to(dev),
                      topk, "silu", E)
    assert moe.recipe == "int4"
    out = torch.empty(T, H, dtype=dt, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, min(T, 64)).long()
    ref = O.fused_moe("int4", x[toks], u13 ^ 0x88, s13, b13, u2 ^ 0x88, s2, b2, tw[toks],
                      ti[toks])
    tol = 2e-2 if dt == torch.bfloat16 else 1e-2
    torch.testing.assert_close(out.cpu()[toks], ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("grp", [32, 128, 256])
@pytest.mark.parametrize("T", [2, 64, 2048])
@pytest.mark.parametrize("layout", ["kblock", "nk"])
def test_fused_moe_int4_group_scales(dev, monkeypatch, grp, T, layout):
    """int4 with a different 16-bit scale in every (row, group) and random
    biases, against the oracle (64 sampled tokens): K-blocked weights and
    scales through the stream (T=2), small (T=64) and 320-slot (T=2048)
    kernels, where one group spans 1, 4 or 8 of the 320-slot kernel's
    32-value stages and the scales of a stage move with the weights; the
    row-major layout (MI355MOE_WEIGHT_LAYOUT=nk) through the stream, small
    and 128-slot kernels."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    if layout == "nk":
        monkeypatch.setenv("MI355MOE_WEIGHT_LAYOUT", "nk")
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(31 + T + grp)
    E, H, I, topk = 16, 1024, 512, 2
    u13 = torch.randint(0, 0xff, (E, 2 * I, H // 2), generator=g).to(torch.uint8)
    u2 = torch.randint(0, 0xff, (E, H, I // 2), generator=g).to(torch.uint8)
    s13 = (torch.rand(E, 2 * I, H // grp, generator=g) * 2 ** -4 + 2 ** -7).to(dt)
    s2 = (torch.rand(E, H, I // grp, generator=g) * 2 ** -4 + 2 ** -7).to(dt)
    b13 = (torch.randn(E, 2 * I, generator=g) / 16).to(dt)
    b2 = (torch.randn(E, H, generator=g) / 16).to(dt)
    x = (torch.randn(T, H, generator=g) / 16).to(dt)
    tw, ti = torch.topk(torch.randn(T, E, generator=g), k=topk, dim=-1, sorted=False)
    moe = XpuFusedMoe(u13.to(dev), s13.to(dev), b13.to(dev), u2.to(dev), s2.to(dev), b2.to(dev),
                      topk, "silu", E)
    assert moe._w_layout == (1 if layout == "kblock" else 0)
    out = torch.full((T, H), float("nan"), dtype=dt, device=dev)
    moe.apply(out, x.to(dev), tw.to(dev), ti.to(dev))
    toks = torch.linspace(0, T - 1, min(T, 64)).long()
    ref = O.fused_moe("int4", x[toks], u13 ^ 0x88, s13, b13, u2 ^ 0x88, s2, b2, tw[toks],
                      ti[toks])
    torch.testing.assert_close(out.cpu()[toks], ref, rtol=2e-2, atol=2e-2)


def test_fused_moe_a1q_scale_rejected_outside_fp8block(dev):
    cfg, w, x, tw, ti, out, moe = _layer(_W().CONFIGS["C1"], 8, dev)
    with pytest.raises(NotImplementedError, match="fp8block, mxfp8 and mxfp4"):
        moe.apply(out, x, tw, ti, a1q_scale=torch.ones(8, 1, device=dev))


def _e8m0(scale):
    """float32 powers of two -> e8m0 bytes."""
    return (torch.log2(scale).round().to(torch.int32) + 127).to(torch.uint8)


@pytest.mark.parametrize("T", [1, 33, 200, 640])
def test_fused_moe_mxfp8_c3_32_experts(dev, T):
    """mxfp8 (e4m3 weights [E, K, N] with e8m0 scales per 32 along K; the
    input and the intermediate activation quantised to mxfp8 per 32) on
    DeepSeek-V3 shapes with 32 experts (T = 1, 33: 16-slot STREAM blocks;
    200, 640: 50 and 160 slots per expert, the 320-slot kernel with the codes
    in the MFMA); the layer's own quantisation of x equals pre-quantised
    input from the 32-group ue8m0 quantiser bit for bit."""
    import dataclasses
    from vllm_xpu_kernels import ops
    cfg = dataclasses.replace(_W().CONFIGS["C3"], recipe="mxfp8")
    cfg, w, x, tw, ti, out, moe = _layer(cfg, T, dev, E=32)
    assert moe.recipe == "mxfp8"
    toks = torch.linspace(0, T - 1, min(T, 24)).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks), fp8=True)
    xq, xs = ops.per_token_group_fp8_quant(x, 32, scale_ue8m0=True)
    out2 = torch.empty_like(out)
    moe.apply(out2, xq, tw, ti, a1q_scale=_e8m0(xs).view(torch.float8_e8m0fnu))
    assert torch.equal(out2, out)


def test_fused_moe_mxfp8_ignores_clamp_limit_like_reference(dev):
    """The reference runs mxfp8 through its torch path, which takes no
    gemm1_clamp_limit: a limit changes nothing."""
    import dataclasses
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    cfg = dataclasses.replace(_W().CONFIGS["C2"], recipe="mxfp8", experts=8, topk=2)
    cfg, w, x, tw, ti, out, moe = _layer(cfg, 16, dev)
    moe2 = XpuFusedMoe(w.w13, w.w13_scale, None, w.w2, w.w2_scale, None, cfg.topk,
                       cfg.activation, cfg.experts, gemm1_clamp_limit=1e-3)
    out2 = torch.empty_like(out)
    moe2.apply(out2, x, tw, ti)
    assert torch.equal(out2, out)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 32, 160, 1024])
def test_fused_moe_mxfp4_pre_quantised_w4a4(dev, T, dt):
    """gpt-oss shapes (H = I = 2880: K % 256 = 64 in both GEMMs, N % 128 = 64)
    with pre-quantised mxfp4 input (packed e2m1 [T, H/2] + e8m0 [T, H/32]):
    both GEMMs are e2m1 x e2m1 with the intermediate activation quantised to
    mxfp4 per 32 (the reference's quant_act_xpu).  T = 1, 32: 16-slot STREAM
    blocks; 160, 1024: the 320-slot kernel (20 and 128 slots per expert).
    The output buffer's type (bf16 or fp16) sets the call's type, as in the
    reference's kernel path (fused_moe_interface.py:368-371, 398-401): both
    GEMM outputs round to it before the activation re-quantisation, and the
    oracle is run in that type."""
    from vllm_xpu_kernels import ops
    cfg, w, x, tw, ti, out, moe = _layer(_W().CONFIGS["C5"], T, dev)
    xq, xs = ops.per_token_group_quant_mxfp4(x, 32)
    xq = xq.view(torch.uint8)
    out4 = torch.empty_like(out, dtype=dt)
    moe.apply(out4, xq.view(torch.float4_e2m1fn_x2), tw, ti,
              a1q_scale=_e8m0(xs).view(torch.float8_e8m0fnu))
    toks = torch.linspace(0, T - 1, min(T, 24)).long().to(dev)
    ref = _oracle_layer(cfg, w, xq, tw, ti, toks, a1q_scale=_e8m0(xs), compute_dtype=dt)
    _close(out4[toks], ref, fp8=True)
    # and close to the w4a16 layer on the same input
    assert (out4.float() - out.float()).abs().mean() < 0.25 * out.float().abs().mean()


@pytest.mark.parametrize("T", [1, 16])
def test_fused_moe_kblock_fp8_c3_decode(dev, monkeypatch, T):
    """DeepSeek-V3 shapes at decode (split-K stream kernels): K-blocked and
    row-major fp8 weights give the same layer output bit for bit."""
    (cfg, w, x, tw, ti, out, _), out_nk = _layer_both_layouts(_W().CONFIGS["C3"], T, dev,
                                                             monkeypatch)
    assert torch.equal(out, out_nk)
    _close(out, _oracle_layer(cfg, w, x, tw, ti), fp8=True)


def _oracle_layer_on_device(cfg, w, x, tw, ti, a1q_scale=None):
    """The oracle run on the GPU tensors themselves (every token)."""
    s13, s2 = w.w13_scale, w.w2_scale
    if cfg.recipe == "bf16":
        w13 = w.w13.transpose(1, 2)
        w2 = w.w2.transpose(1, 2)
    elif cfg.recipe == "fp8block":
        w13, w2 = w.w13, w.w2
    elif cfg.recipe == "mxfp8":   # [E, K, N] + [E, K/32, N] -> [E, N, K] + [E, N, K/32]
        w13, w2 = w.w13.transpose(1, 2), w.w2.transpose(1, 2)
        s13, s2 = s13.transpose(1, 2), s2.transpose(1, 2)
    else:
        w13, w2 = w.w13.view(torch.uint8), w.w2.view(torch.uint8)
    return O.fused_moe(cfg.recipe, x, w13, s13, w.w13_bias, w2, s2,
                       w.w2_bias, tw, ti.long(), activation=cfg.activation,
                       a1q_scale=a1q_scale)


@pytest.mark.parametrize("name,T", [("C2", 4096), ("C3", 8192), ("C4", 2048), ("C5", 4096)])
def test_fused_moe_prefill_full_size_every_token(dev, name, T):
    """Full BASELINE prefill shapes: every token against the oracle run on the
    device (fp32 matmuls, the oracle's rounding points); bf16 / mxfp4 every
    element within rtol = atol = 2e-2, fp8 the fp8 bar."""
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS[name], T, dev)
    ref = _oracle_layer_on_device(cfg, w, x, tw, ti)
    _close(out, ref, fp8=cfg.recipe == "fp8block")


def test_fused_moe_w4a4_prefill_every_token(dev):
    """mxfp4 weights with pre-quantised mxfp4 input at the C5 prefill size
    (T=4096, 512 slots per expert: the 320-slot e2m1 x e2m1 kernel, K and N
    with a 64-value tail): every token against the oracle run on the device,
    to the fp8 bar."""
    from vllm_xpu_kernels import ops
    cfg, w, x, tw, ti, _, moe = _layer(_W().CONFIGS["C5"], 4096, dev)
    xq, xs = ops.per_token_group_quant_mxfp4(x, 32)
    xq = xq.view(torch.uint8)
    out = torch.empty_like(x)
    moe.apply(out, xq.view(torch.float4_e2m1fn_x2), tw, ti,
              a1q_scale=_e8m0(xs).view(torch.float8_e8m0fnu))
    ref = _oracle_layer_on_device(cfg, w, xq, tw, ti, a1q_scale=_e8m0(xs))
    _close(out, ref, fp8=True)


@pytest.mark.parametrize("E,T", [(64, 1024), (256, 4096)])
def test_fused_moe_mxfp8_prefill_every_token(dev, E, T):
    """mxfp8 on DeepSeek-V3 shapes at prefill sizes (128 slots per expert:
    the 320-slot kernel with the e8m0 codes of both operands in the MFMA):
    every token against the oracle run on the device, to the fp8 bar."""
    import dataclasses
    cfg = dataclasses.replace(_W().CONFIGS["C3"], recipe="mxfp8")
    cfg, w, x, tw, ti, out, _ = _layer(cfg, T, dev, E=E)
    _close(out, _oracle_layer_on_device(cfg, w, x, tw, ti), fp8=True)


@pytest.mark.parametrize("name,T,sample", [("C2", 4096, 24), ("C3", 8192, 6),
                                           ("C4", 2048, 12), ("C5", 4096, 12)])
def test_fused_moe_prefill_full_size_sampled(dev, name, T, sample):
    """Full BASELINE prefill shapes through the big-tile kernels; the oracle
    checks evenly spaced sampled tokens."""
    cfg, w, x, tw, ti, out, _ = _layer(_W().CONFIGS[name], T, dev)
    toks = torch.linspace(0, T - 1, sample).long().to(dev)
    _close(out[toks], _oracle_layer(cfg, w, x, tw, ti, toks), fp8=cfg.recipe == "fp8block")


@pytest.mark.parametrize("T", [64, 1])
def test_fused_moe_hip_graph_replays(dev, T):
    """The layer captured in a HIP graph: every replay (with eager work and
    synchronisation between replays) equals the eager result.  T=1 runs the
    split-K decode GEMMs (split launch + partial-sum launch)."""
    cfg, w, x, tw, ti, out, moe = _layer(_W().CONFIGS["C2"], T, dev)
    torch.cuda.synchronize()
    eager = out.clone()
    gout = torch.empty_like(out)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        moe.apply(gout, x, tw, ti)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        moe.apply(gout, x, tw, ti)
    for i in range(4):
        gout.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, eager), f"replay {i}"
        junk = torch.randn(1 << 20, device=dev).sum()   # eager work between replays
        torch.cuda.synchronize()
        del junk


IN_PLACE = "MI355MOE_PREPARE_IN_PLACE"


@pytest.mark.parametrize("name,E", [("C1", None), ("C3", 16), ("C5", 8), ("C2-int4", 8),
                                    ("C3-mxfp8", 16), ("C3-fp8", 16)])
def test_fused_moe_prepare_in_place(dev, monkeypatch, name, E):
    """The default preparation writes the converted weights (and the mxfp4,
    mxfp8 and int4 scales) over the caller's tensors, one expert at a time:
    the layer's weights share their storage, those tensors keep shape and
    dtype, the prepared bytes and the output (T=64) equal those of
    MI355MOE_PREPARE_IN_PLACE=0 (a converted copy, the caller's tensors left
    as they were) bit for bit; a second layer on the same tensors and
    arguments reuses the preparation, one with other arguments is refused."""
    import dataclasses
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    cfg = W.config(name)
    if E is not None:
        cfg = dataclasses.replace(cfg, experts=E)
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, 64, dev)
    bias = W.make_correction_bias(cfg, dev) if cfg.routing == "grouped_sigmoid" else None
    tw, ti = W.route(cfg, W.make_router_logits(cfg, 64, dev), bias)
    args = w.layer_args(copy=True)
    snap = [None if t is None else t.clone() for t in args]

    def layer(activation=cfg.activation):
        return XpuFusedMoe(*args, cfg.topk, activation, cfg.experts)

    def run(moe):
        out = torch.full_like(x, float("nan"))
        moe.apply(out, x, tw, ti)
        return out

    monkeypatch.setenv(IN_PLACE, "0")
    moe0 = layer()
    out0 = run(moe0)
    for t, t0 in zip(args, snap):
        assert t is None or torch.equal(t.view(torch.uint8), t0.view(torch.uint8))
    monkeypatch.delenv(IN_PLACE)
    moe = layer()
    assert moe.w13.data_ptr() == args[0].data_ptr() and moe.w2.data_ptr() == args[3].data_ptr()
    for t, t0 in zip(args, snap):
        assert t is None or (t.shape == t0.shape and t.dtype == t0.dtype)
    for a0, a1 in ((moe0.w13, moe.w13), (moe0.w2, moe.w2),
                   (moe0.gemm1_wei_scales, moe.gemm1_wei_scales),
                   (moe0.gemm2_wei_scales, moe.gemm2_wei_scales)):
        assert (a0 is None) == (a1 is None)
        if a0 is not None:
            assert a0.shape == a1.shape and a0.dtype == a1.dtype
            assert torch.equal(a0.view(torch.uint8), a1.view(torch.uint8))
    out = run(moe)
    assert torch.equal(out, out0)
    moe2 = layer()
    assert moe2.w13.data_ptr() == moe.w13.data_ptr()
    assert torch.equal(run(moe2), out0)
    with pytest.raises(ValueError, match="other arguments"):
        layer("gelu" if cfg.activation != "gelu" else "silu")


def test_fused_moe_c3_weights_held_once(dev, monkeypatch):
    """DeepSeek-V3 (C3: 256 experts, fp8 block-scaled, 11.3 GB of weights):
    constructing the layer grows torch.cuda.memory_allocated() by at most 1%
    of the weight bytes (the transient peak: at most 2%), and its output at
    T=64 equals that of a layer holding a converted copy
    (MI355MOE_PREPARE_IN_PLACE=0) bit for bit."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    cfg = W.CONFIGS["C3"]
    w = W.make_weights(cfg, dev)
    x = W.make_activations(cfg, 64, dev)
    tw, ti = W.route(cfg, W.make_router_logits(cfg, 64, dev), W.make_correction_bias(cfg, dev))
    nbytes = sum(t.numel() * t.element_size() for t in w.layer_args() if t is not None)
    assert nbytes > 11e9

    def run(moe):
        out = torch.full_like(x, float("nan"))
        moe.apply(out, x, tw, ti)
        torch.cuda.synchronize()
        return out

    monkeypatch.setenv(IN_PLACE, "0")
    moe0 = XpuFusedMoe(*w.layer_args(), cfg.topk, cfg.activation, cfg.experts)
    out0 = run(moe0)
    del moe0
    monkeypatch.delenv(IN_PLACE)
    torch.cuda.synchronize()
    m0 = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    moe = XpuFusedMoe(*w.layer_args(), cfg.topk, cfg.activation, cfg.experts)
    torch.cuda.synchronize()
    grown, peak = torch.cuda.memory_allocated() - m0, torch.cuda.max_memory_allocated() - m0
    print(f"C3 weights {nbytes / 1e9:.2f} GB: layer construction grew allocated memory by "
          f"{grown / 1e6:.1f} MB, peak {peak / 1e6:.1f} MB", flush=True)
    assert grown <= 0.01 * nbytes and peak <= 0.02 * nbytes
    assert torch.equal(run(moe), out0)