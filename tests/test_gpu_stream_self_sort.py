"""Decode layers with at most 16 slots in fewer launches.  (1) The STREAM
w13 launch sorts the top-k ids itself (and quantises fp8 activations per
1 x 128 block into LDS) instead of a sort(+quantisation) launch before it:
the layer output must be the sort launch's bit for bit
(MI355MOE_STREAM_SELF_SORT=0 selects it); the w2 and reduction launches read
the sort outputs this launch writes, so any difference from the counting
sort's outputs would show in the output.  (2) Where the output columns fill
the GPU (C3 shapes), w2 runs token-major and writes the layer output itself:
bit for bit the top-k reduction launch's (MI355MOE_STREAM_TOKEN_W2=0).  (3)
With a split-K w13 and a 16-bit activation (C2, C5), the w2 launch rebuilds
its activation rows from the w13 partial tiles: bit for bit the w13
finalize launch's (MI355MOE_STREAM_W2_FINISHES_W13=0).  (4) An fp8 w13 that
would split K runs in 64-column workgroups over both K halves instead and
the token-major w2 quantises its activation rows
(MI355MOE_STREAM_KHALVES=0)."""
import dataclasses

import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _W():
    from vllm_xpu_kernels import workloads
    return workloads


def _both(call, monkeypatch, var="MI355MOE_STREAM_SELF_SORT"):
    monkeypatch.setenv(var, "0")
    ref = call()
    monkeypatch.delenv(var)
    got = call()
    again = call()
    torch.cuda.synchronize()
    return ref, got, again


def _layer_call(cfg, T, dev, dt=torch.bfloat16, ids_dtype=torch.int32, ti=None, tw=None,
                expert_map=None, prequant=False):
    from vllm_xpu_kernels import ops
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    w = W.make_weights(cfg, dev)
    if dt == torch.float16:
        w = dataclasses.replace(
            w, w13=w.w13.half() if cfg.recipe == "bf16" else w.w13,
            w2=w.w2.half() if cfg.recipe == "bf16" else w.w2,
            w13_bias=None if w.w13_bias is None else w.w13_bias.half(),
            w2_bias=None if w.w2_bias is None else w.w2_bias.half())
    x = W.make_activations(cfg, T, dev).to(dt)
    if ti is None:
        bias = W.make_correction_bias(cfg, dev) if cfg.routing == "grouped_sigmoid" else None
        tw, ti = W.route(cfg, W.make_router_logits(cfg, T, dev), bias)
    ti = ti.to(ids_dtype)
    moe = XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, cfg.activation, cfg.experts)
    kw = {} if expert_map is None else {"expert_map": expert_map}
    if prequant:
        xq, xs = ops.per_token_group_fp8_quant(x, 128)
        x, kw["a1q_scale"] = xq, xs

    def call():
        out = torch.full((T, cfg.hidden), float("nan"), dtype=dt, device=dev)
        moe.apply(out, x, tw, ti, **kw)
        return out
    return call, (cfg, w, x, tw, ti)


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_self_sort_bit_identical(dev, monkeypatch, name, T):
    call, _ = _layer_call(_W().CONFIGS[name], T, dev)
    ref, got, again = _both(call, monkeypatch)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, ref) and torch.equal(again, ref)


@pytest.mark.parametrize("variant", ["fp16", "int64_ids", "prequant", "fp16_bf16w"])
def test_self_sort_bit_identical_variants(dev, monkeypatch, variant):
    """(int4 runs the same routing through test_fused_moe_ep at T=1 and 16.)"""
    W = _W()
    if variant == "fp16":
        call, _ = _layer_call(W.CONFIGS["C3"], 1, dev, dt=torch.float16)
    elif variant == "int64_ids":
        call, _ = _layer_call(W.CONFIGS["C3"], 2, dev, ids_dtype=torch.int64)
    elif variant == "prequant":
        call, _ = _layer_call(W.CONFIGS["C3"], 2, dev, prequant=True)
    else:
        call, _ = _layer_call(W.CONFIGS["C2"], 2, dev, dt=torch.float16)
    ref, got, again = _both(call, monkeypatch)
    assert torch.equal(got, ref) and torch.equal(again, ref)


@pytest.mark.parametrize("T", [1, 2, 8])
def test_self_sort_expert_map_and_duplicates(dev, monkeypatch, T):
    """A rank holding experts 16..23 of 64 (dropped slots, tokens with no
    local slot) and ids repeated within a token."""
    W = _W()
    cfg = dataclasses.replace(W.CONFIGS["C2"], experts=8, hidden=512, inter=256, topk=2)
    g = torch.Generator(device=dev).manual_seed(11 + T)
    ti = torch.randint(12, 28, (T, 2), generator=g, device=dev)
    ti[0] = torch.tensor([17, 17], device=dev)     # the same expert twice
    if T > 1:
        ti[1] = torch.tensor([40, 3], device=dev)  # no local expert
    tw = torch.rand(T, 2, generator=g, device=dev)
    emap = torch.full((64,), -1, dtype=torch.int32, device=dev)
    emap[16:24] = torch.arange(8, dtype=torch.int32, device=dev)
    call, _ = _layer_call(cfg, T, dev, ti=ti, tw=tw, expert_map=emap)
    ref, got, again = _both(call, monkeypatch)
    assert torch.equal(got, ref) and torch.equal(again, ref)
    assert not torch.isnan(got.float()).any()
    if T > 1:
        assert torch.all(got[1] == 0)


@pytest.mark.parametrize("T", [1, 2])
def test_self_sort_matches_oracle(dev, T):
    """C3 (fp8, activations quantised in the kernel) against the oracle, and
    the in-kernel quantisation against the group quantiser: the same layer
    fed the oracle quantiser's codes and scales (a1q_scale, no quantisation
    in the kernel) gives the same output bit for bit."""
    from test_gpu_gemm_fused import _close, _oracle_layer
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    call, (cfg, w, x, tw, ti) = _layer_call(_W().CONFIGS["C3"], T, dev)
    out = call()
    _close(out, _oracle_layer(cfg, w, x, tw, ti.long()), fp8=True)
    xq, xs = O.per_token_group_fp8_quant(x.cpu(), 128)
    moe = XpuFusedMoe(w.w13, w.w13_scale, w.w13_bias, w.w2, w.w2_scale, w.w2_bias,
                      cfg.topk, cfg.activation, cfg.experts)
    out_q = torch.empty_like(out)
    moe.apply(out_q, xq.to(dev), tw, ti, a1q_scale=xs.to(dev))
    assert torch.equal(out_q, out)


TOKEN_W2 = "MI355MOE_STREAM_TOKEN_W2"


@pytest.mark.parametrize("variant", ["T1", "T2", "fp16", "int64_ids"])
def test_token_major_w2_bit_identical(dev, monkeypatch, variant):
    C3 = _W().CONFIGS["C3"]
    if variant == "T1":
        call, _ = _layer_call(C3, 1, dev)
    elif variant == "T2":
        call, _ = _layer_call(C3, 2, dev)
    elif variant == "fp16":
        call, _ = _layer_call(C3, 1, dev, dt=torch.float16)
    else:
        call, _ = _layer_call(C3, 2, dev, ids_dtype=torch.int64)
    ref, got, again = _both(call, monkeypatch, TOKEN_W2)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, ref) and torch.equal(again, ref)


@pytest.mark.parametrize("T", [1, 2])
def test_token_major_w2_expert_parallel(dev, monkeypatch, T):
    """DeepSeek-V3 shapes on a rank holding experts 64..95 of 256: dropped
    slots (their waves stream nothing), a token with no local expert (exact
    zeros), and a token listing one expert twice."""
    W = _W()
    cfg = dataclasses.replace(W.CONFIGS["C3"], experts=32)
    g = torch.Generator(device=dev).manual_seed(21 + T)
    ti = torch.randint(40, 120, (T, 8), generator=g, device=dev)
    ti[0, :3] = torch.tensor([70, 70, 5], device=dev)
    if T > 1:
        ti[1] = torch.arange(200, 208, device=dev)
    tw = torch.rand(T, 8, generator=g, device=dev)
    emap = torch.full((256,), -1, dtype=torch.int32, device=dev)
    emap[64:96] = torch.arange(32, dtype=torch.int32, device=dev)
    call, _ = _layer_call(cfg, T, dev, ti=ti, tw=tw, expert_map=emap)
    ref, got, again = _both(call, monkeypatch, TOKEN_W2)
    assert torch.equal(got, ref) and torch.equal(again, ref)
    assert not torch.isnan(got.float()).any()
    if T > 1:
        assert torch.all(got[1] == 0)


@pytest.mark.parametrize("T", [1, 2])
def test_token_major_w2_matches_oracle(dev, T):
    from test_gpu_gemm_fused import _close, _oracle_layer
    cfg = dataclasses.replace(_W().CONFIGS["C3"], bias=True)
    call, (cfg, w, x, tw, ti) = _layer_call(cfg, T, dev)
    _close(call(), _oracle_layer(cfg, w, x, tw, ti.long()), fp8=True)


KHALVES = "MI355MOE_STREAM_KHALVES"


def _c3_variant(dev, variant, T=1):
    """C3-shaped decode layer calls for the fp8 decode paths."""
    from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
    W = _W()
    C3 = W.CONFIGS["C3"]
    if variant == "T1":
        return _layer_call(C3, T, dev)[0]
    if variant == "fp16":
        return _layer_call(C3, T, dev, dt=torch.float16)[0]
    if variant == "int64_ids":
        return _layer_call(C3, T, dev, ids_dtype=torch.int64)[0]
    if variant == "prequant":
        return _layer_call(C3, T, dev, prequant=True)[0]
    if variant == "bias":
        return _layer_call(dataclasses.replace(C3, bias=True), T, dev)[0]
    if variant == "swigluoai":
        return _layer_call(dataclasses.replace(C3, activation="swigluoai", bias=True), T, dev)[0]
    if variant == "expert_map":
        cfg = dataclasses.replace(C3, experts=32)
        g = torch.Generator(device=dev).manual_seed(31)
        ti = torch.randint(40, 120, (T, 8), generator=g, device=dev)
        ti[0, :3] = torch.tensor([70, 70, 5], device=dev)
        tw = torch.rand(T, 8, generator=g, device=dev)
        emap = torch.full((256,), -1, dtype=torch.int32, device=dev)
        emap[64:96] = torch.arange(32, dtype=torch.int32, device=dev)
        return _layer_call(cfg, T, dev, ti=ti, tw=tw, expert_map=emap)[0]
    assert variant == "clamp"
    w = W.make_weights(C3, dev)
    x = W.make_activations(C3, T, dev)
    bias = W.make_correction_bias(C3, dev)
    tw, ti = W.route(C3, W.make_router_logits(C3, T, dev), bias)
    moe = XpuFusedMoe(*w.layer_args(copy=True), C3.topk, C3.activation, C3.experts,
                      gemm1_clamp_limit=0.05)

    def call():
        out = torch.empty_like(x)
        moe.apply(out, x, tw, ti)
        return out
    return call


@pytest.mark.parametrize("variant", ["T1", "fp16", "int64_ids", "prequant", "bias",
                                     "swigluoai", "expert_map", "clamp"])
def test_khalves_bit_identical(dev, monkeypatch, variant):
    """(4) fp8 decode whose w13 would split K: 64-column w13 workgroups over
    both K halves store the 16-bit activation and every token-major w2 wave
    quantises its own slot's row -- bit for bit the split launch, its
    partial-sum launch and the w13 epilogue's quantisation
    (MI355MOE_STREAM_KHALVES=0)."""
    call = _c3_variant(dev, variant)
    ref, got, again = _both(call, monkeypatch, KHALVES)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, ref) and torch.equal(again, ref)


@pytest.mark.parametrize("variant", ["T1", "bias", "swigluoai"])
def test_khalves_matches_oracle(dev, variant):
    from test_gpu_gemm_fused import _close, _oracle_layer_on_device
    W = _W()
    cfg = W.CONFIGS["C3"]
    if variant != "T1":
        cfg = dataclasses.replace(cfg, bias=True,
                                  activation="swigluoai" if variant == "swigluoai" else "silu")
    call, (cfg, w, x, tw, ti) = _layer_call(cfg, 1, dev)
    _close(call(), _oracle_layer_on_device(cfg, w, x, tw, ti), fp8=True)


W2_FIN = "MI355MOE_STREAM_W2_FINISHES_W13"


@pytest.mark.parametrize("variant", ["C2-T1", "C2-T2", "C5-T1", "C5-T2", "C1-T2", "C2-fp16",
                                     "C5-clamp"])
def test_w2_finishes_w13_bit_identical(dev, monkeypatch, variant):
    W = _W()
    name, rest = variant.split("-")
    cfg = W.CONFIGS[name]
    if rest == "fp16":
        call, _ = _layer_call(cfg, 1, dev, dt=torch.float16)
    elif rest == "clamp":
        from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
        w = W.make_weights(cfg, dev)
        x = W.make_activations(cfg, 2, dev)
        tw, ti = W.route(cfg, W.make_router_logits(cfg, 2, dev))
        moe = XpuFusedMoe(w.w13, w.w13_scale, w.w13_bias, w.w2, w.w2_scale, w.w2_bias,
                          cfg.topk, cfg.activation, cfg.experts, gemm1_clamp_limit=0.05)

        def call():
            out = torch.empty_like(x)
            moe.apply(out, x, tw, ti)
            return out
    else:
        call, _ = _layer_call(cfg, int(rest[1:]), dev)
    ref, got, again = _both(call, monkeypatch, W2_FIN)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, ref) and torch.equal(again, ref)


ALL_OFF = ("MI355MOE_STREAM_SELF_SORT", TOKEN_W2, W2_FIN, KHALVES)


@pytest.mark.parametrize("shape", ["tokw2_tail", "w2fin_tail"])
@pytest.mark.parametrize("T", [1, 2])
def test_decode_paths_ragged_shapes(dev, monkeypatch, shape, T):
    """Ragged decode shapes (row-major bf16 weights): H = 7192 (token-major
    w2 with a last column group of 24) and I = 736 (w2 rebuilding its
    activation from w13 tiles whose last one holds 96 columns), against the
    separate launches bit for bit and against the oracle."""
    from test_gpu_gemm_fused import _close, _oracle_layer
    W = _W()
    if shape == "tokw2_tail":
        cfg = dataclasses.replace(W.CONFIGS["C2"], hidden=7192, inter=512, experts=64, topk=8)
    else:
        cfg = dataclasses.replace(W.CONFIGS["C2"], hidden=2048, inter=736, experts=64, topk=8,
                                  bias=True)
    call, (cfg, w, x, tw, ti) = _layer_call(cfg, T, dev)
    for var in ALL_OFF:
        monkeypatch.setenv(var, "0")
    ref = call()
    for var in ALL_OFF:
        monkeypatch.delenv(var)
    got = call()
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    _close(got, _oracle_layer(cfg, w, x, tw, ti.long()))
