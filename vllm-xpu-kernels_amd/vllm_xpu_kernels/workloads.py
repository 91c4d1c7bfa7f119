"""Synthetic inputs of the benchmark configurations (C1-C5).

Weights, activations, router logits and correction bias are drawn from fixed
seeds (0 weights, 1 activations, 2 logits, 3 bias) with plain torch ops on the
target device; each expert has its own generator stream, so any subset of
experts can be regenerated bit-identically (used to hand the CPU checker only
the experts a sample of tokens routes to).  Nothing here depends on a
network, a checkpoint or the CPU oracle.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Optional

import torch

from . import ops


@dataclass(frozen=True)
class MoeConfig:
    name: str
    hidden: int
    inter: int
    experts: int
    topk: int
    recipe: str                 # "bf16" | "fp8block" | "mxfp4" | "mxfp8" | "fp8" | "int4"
    routing: str                # "softmax" | "grouped_sigmoid"
    activation: str = "silu"
    renormalize: bool = True
    n_group: int = 0
    topk_group: int = 0
    routed_scaling_factor: float = 1.0
    bias: bool = False          # w13/w2 biases (gpt-oss)
    zipf_tau: float = 0.0       # >0: skewed router logits
    tokens: tuple = field(default_factory=tuple)
    prequant: bool = False      # mxfp4: input handed over as e2m1 + e8m0 (w4a4)


# Calibrated once by a bisection over tau on the device generator the bench
# and tests draw logits with: the 13 busiest of 128 experts receive 50% +- 2%
# of the 16384 assignments at T=2048 (0.4980 at 0.520, 0.5059 at 0.530);
# test_moe_align_zipf_skew_c4 pins the share.
ZIPF_TAU_C4 = 0.5225

CONFIGS = {
    "C1": MoeConfig("tiny", 512, 1024, 8, 2, "bf16", "softmax", tokens=(64,)),
    "C2": MoeConfig("qwen3-30b-a3b", 2048, 768, 128, 8, "bf16", "softmax",
                    tokens=(1, 16, 64, 256, 4096)),
    "C3": MoeConfig("deepseek-v3", 7168, 2048, 256, 8, "fp8block",
                    "grouped_sigmoid", n_group=8, topk_group=4,
                    routed_scaling_factor=2.5, tokens=(1, 64, 8192)),
    "C4": MoeConfig("qwen3-235b-a22b", 4096, 1536, 128, 8, "fp8block",
                    "softmax", zipf_tau=ZIPF_TAU_C4, tokens=(2048,)),
    "C5": MoeConfig("gpt-oss-20b", 2880, 2880, 32, 4, "mxfp4", "softmax",
                    activation="swigluoai", bias=True, tokens=(1, 128, 4096)),
}


# Recipe variants on the same shapes (not BASELINE configurations): DeepSeek-V3
# with mxfp8 weights or per-expert-scaled e4m3 weights (the reference's
# recipe "fp8", w8a16), gpt-oss-20b with pre-quantised mxfp4 input (both
# GEMMs e2m1 x e2m1).
VARIANTS = {
    "C3-mxfp8": replace(CONFIGS["C3"], recipe="mxfp8"),
    "C3-fp8": replace(CONFIGS["C3"], recipe="fp8"),
    # Qwen3-30B-A3B with int4 weights (u4, zero point 8, bf16 scale per 128
    # along K: the reference's w4a16 recipe)
    "C2-int4": replace(CONFIGS["C2"], recipe="int4"),
    "C5-w4a4": replace(CONFIGS["C5"], prequant=True),
}


def config(name: str) -> MoeConfig:
    """A configuration (C1-C5) or a recipe variant by name."""
    return CONFIGS[name] if name in CONFIGS else VARIANTS[name]


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, std, seed, device, dtype=torch.float32):
    return (torch.randn(shape, generator=_gen(device, seed), device=device,
                        dtype=torch.float32) * std).to(dtype)


def fp8_block_quant(w: torch.Tensor, eps: float = 1e-6):
    """[..., N, K] -> e4m3 + fp32 [..., N/128, K/128] scales,
    s = clamp(amax/448, min=eps), q = e4m3(w/s)."""
    *lead, N, K = w.shape
    x = w.float().reshape(*lead, N // 128, 128, K // 128, 128)
    s = torch.clamp(x.abs().amax(dim=(-3, -1)) / 448.0, min=eps)
    q = (x / s.unsqueeze(-2).unsqueeze(-1)).reshape(*lead, N, K)
    return q.to(torch.float8_e4m3fn), s


def int4_quant(w: torch.Tensor, group: int = 128):
    """[N, K] fp32 -> u4 pairs uint8 [N, K/2] (zero point 8, the even K
    value in the low nibble) + bf16 scales [N, K/group]."""
    N, K = w.shape
    g = w.view(N, K // group, group)
    s = (g.abs().amax(-1) / 7.0).clamp(min=1e-8).to(torch.bfloat16)
    q = (torch.round(g / s.float().unsqueeze(-1)).clamp(-8, 7) + 8).to(torch.uint8).view(N, K)
    return q[:, 0::2] | (q[:, 1::2] << 4), s


def mxfp4_quant(w: torch.Tensor):
    """[..., K] fp32 -> packed e2m1 [..., K/2] + e8m0 [..., K/32]: RCEIL
    exponent per 32 values, value rounded to bf16 then to the e2m1 grid with
    ties to the even code (OCP MX v1.0)."""
    shp = w.shape
    K = shp[-1]
    x = w.float().reshape(-1, K // 32, 32)
    amax = x.abs().amax(-1, keepdim=True)
    e = torch.clamp(torch.ceil(torch.log2(amax / 6.0)), -127, 127) + 127
    e = torch.nan_to_num(e, nan=255.0)
    dsc = torch.where(e == 0, torch.ones_like(e), torch.exp2(127 - e))
    v = torch.clamp(x * dsc, -6.0, 6.0).to(torch.bfloat16).float()
    m = v.abs()
    code = ((m > 0.25).int() + (m >= 0.75).int() + (m > 1.25).int() +
            (m >= 1.75).int() + (m > 2.5).int() + (m >= 3.5).int() +
            (m > 5.0).int())
    code = code | ((v < 0).int() << 3)
    code = code.reshape(-1, K)
    q = (code[:, 0::2] | (code[:, 1::2] << 4)).to(torch.uint8)
    return (q.reshape(shp[:-1] + (K // 2,)),
            e.to(torch.uint8).reshape(shp[:-1] + (K // 32,)))


def mxfp8_quant(w: torch.Tensor):
    """[..., K] fp32 -> e4m3 [..., K] + e8m0 [..., K/32]: exponent
    ceil(log2(amax / 448)) per 32 values (the least power of two that keeps
    the block within e4m3's range), values rounded to nearest even."""
    shp = w.shape
    K = shp[-1]
    x = w.float().reshape(-1, K // 32, 32)
    amax = x.abs().amax(-1, keepdim=True)
    e = torch.clamp(torch.ceil(torch.log2(amax / 448.0)), -127, 127) + 127
    e = torch.nan_to_num(e, nan=255.0)
    q = torch.clamp(x * torch.exp2(127 - e), -448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(shp), e.to(torch.uint8).reshape(shp[:-1] + (K // 32,))


@dataclass
class MoeWeights:
    """Weights in the reference's constructor layouts (see XpuFusedMoe)."""
    w13: torch.Tensor
    w13_scale: Optional[torch.Tensor]
    w13_bias: Optional[torch.Tensor]
    w2: torch.Tensor
    w2_scale: Optional[torch.Tensor]
    w2_bias: Optional[torch.Tensor]

    def layer_args(self, copy: bool = False):
        """(w13, w13_scale, w13_bias, w2, w2_scale, w2_bias) for XpuFusedMoe;
        copy: new tensors, so that these keep the reference layouts (a layer
        prepares its weights over the tensors it is given)."""
        ts = (self.w13, self.w13_scale, self.w13_bias, self.w2, self.w2_scale, self.w2_bias)
        return tuple(None if t is None else t.clone() for t in ts) if copy else ts


def act_width(cfg: MoeConfig) -> int:
    """Width of the activation, and K of w2: 2I for relu2_no_mul (no gate),
    else I."""
    return 2 * cfg.inter if cfg.activation == "relu2_no_mul" else cfg.inter


def expert_weights_nk(cfg: MoeConfig, e: int, device, seed: int = 0):
    """One expert in [N, K] layout: (w13 [2I,H], s13, w2 [H,K2], s2), recipe
    encoded (K2 = act_width); biases separately via make_biases."""
    H, I = cfg.hidden, cfg.inter
    w13 = _randn((2 * I, H), 0.02, seed * 1000003 + 2 * e, device)
    w2 = _randn((H, act_width(cfg)), 0.02, seed * 1000003 + 2 * e + 1, device)
    if cfg.recipe == "bf16":
        return w13.to(torch.bfloat16), None, w2.to(torch.bfloat16), None
    if cfg.recipe == "fp8block":
        q13, s13 = fp8_block_quant(w13)
        q2, s2 = fp8_block_quant(w2)
        return q13, s13, q2, s2
    if cfg.recipe == "mxfp8":
        q13, s13 = mxfp8_quant(w13)
        q2, s2 = mxfp8_quant(w2)
        return q13, s13, q2, s2
    if cfg.recipe == "int4":  # u4 = round(w / s) + 8 in [0, 15], s = amax / 7 per 128
        return (*int4_quant(w13), *int4_quant(w2))
    if cfg.recipe == "fp8":   # one scale per expert and matrix: amax / 448
        s13, s2 = w13.abs().amax() / 448.0, w2.abs().amax() / 448.0
        return ((w13 / s13).to(torch.float8_e4m3fn), s13, (w2 / s2).to(torch.float8_e4m3fn),
                s2)
    q13, s13 = mxfp4_quant(w13)
    q2, s2 = mxfp4_quant(w2)
    return q13, s13, q2, s2


def make_biases(cfg: MoeConfig, device, seed: int = 0):
    if not cfg.bias:
        return None, None
    E, H, I = cfg.experts, cfg.hidden, cfg.inter
    b13 = _randn((E, 2 * I), 0.01, seed * 1000003 + 777777, device, torch.bfloat16)
    b2 = _randn((E, H), 0.01, seed * 1000003 + 777778, device, torch.bfloat16)
    return b13, b2


def make_weights(cfg: MoeConfig, device, seed: int = 0) -> MoeWeights:
    E, H, I, K2 = cfg.experts, cfg.hidden, cfg.inter, act_width(cfg)
    if cfg.recipe == "bf16":
        w13 = torch.empty(E, H, 2 * I, dtype=torch.bfloat16, device=device)
        w2 = torch.empty(E, K2, H, dtype=torch.bfloat16, device=device)
        s13 = s2 = None
    elif cfg.recipe == "fp8block":
        w13 = torch.empty(E, 2 * I, H, dtype=torch.float8_e4m3fn, device=device)
        w2 = torch.empty(E, H, K2, dtype=torch.float8_e4m3fn, device=device)
        s13 = torch.empty(E, 2 * I // 128, H // 128, device=device)
        s2 = torch.empty(E, H // 128, K2 // 128, device=device)
    elif cfg.recipe == "fp8":
        # reference layout [E, K, N] e4m3 + f32 [E] (its per-expert fp8 test,
        # tests/fused_moe/test_fused_moe.py:226-246)
        w13 = torch.empty(E, H, 2 * I, dtype=torch.float8_e4m3fn, device=device)
        w2 = torch.empty(E, K2, H, dtype=torch.float8_e4m3fn, device=device)
        s13 = torch.empty(E, device=device)
        s2 = torch.empty(E, device=device)
    elif cfg.recipe == "int4":
        # reference layout: u4 pairs [E, N, K/2] + 16-bit scales [E, N, K/128]
        w13 = torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=device)
        w2 = torch.empty(E, H, K2 // 2, dtype=torch.uint8, device=device)
        s13 = torch.empty(E, 2 * I, H // 128, dtype=torch.bfloat16, device=device)
        s2 = torch.empty(E, H, K2 // 128, dtype=torch.bfloat16, device=device)
    elif cfg.recipe == "mxfp8":
        # reference layout (moe_utils.py:80-82): [E, K, N] + e8m0 [E, K/32, N]
        w13 = torch.empty(E, H, 2 * I, dtype=torch.float8_e4m3fn, device=device)
        w2 = torch.empty(E, K2, H, dtype=torch.float8_e4m3fn, device=device)
        s13 = torch.empty(E, H // 32, 2 * I, dtype=torch.uint8, device=device)
        s2 = torch.empty(E, K2 // 32, H, dtype=torch.uint8, device=device)
    else:
        w13 = torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=device)
        w2 = torch.empty(E, H, K2 // 2, dtype=torch.uint8, device=device)
        s13 = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8, device=device)
        s2 = torch.empty(E, H, K2 // 32, dtype=torch.uint8, device=device)
    for e in range(E):
        a, sa, b, sb = expert_weights_nk(cfg, e, device, seed)
        if cfg.recipe == "bf16":
            w13[e].copy_(a.t())   # reference bf16 layout [E, K, N]
            w2[e].copy_(b.t())
        elif cfg.recipe == "fp8":
            w13[e].copy_(a.t())
            w2[e].copy_(b.t())
            s13[e] = sa
            s2[e] = sb
        elif cfg.recipe == "mxfp8":
            w13[e].copy_(a.t())
            w2[e].copy_(b.t())
            s13[e].copy_(sa.t())
            s2[e].copy_(sb.t())
        else:
            w13[e].copy_(a)
            w2[e].copy_(b)
            s13[e].copy_(sa)
            s2[e].copy_(sb)
    if cfg.recipe == "mxfp4":
        w13 = w13.view(torch.float4_e2m1fn_x2)
        w2 = w2.view(torch.float4_e2m1fn_x2)
    b13, b2 = make_biases(cfg, device, seed)
    return MoeWeights(w13, s13, b13, w2, s2, b2)


def make_activations(cfg: MoeConfig, T: int, device, seed: int = 1):
    return _randn((T, cfg.hidden), 1.0, seed, device, torch.bfloat16)


def make_router_logits(cfg: MoeConfig, T: int, device, seed: int = 2):
    logits = _randn((T, cfg.experts), 1.0, seed, device)
    if cfg.zipf_tau > 0:
        perm = torch.randperm(cfg.experts, generator=_gen("cpu", seed + 100))
        rank = torch.empty(cfg.experts)
        rank[perm] = torch.arange(1, cfg.experts + 1, dtype=torch.float32)
        logp = -1.1 * torch.log(rank)
        logp = logp - torch.logsumexp(logp, 0)
        logits = logits + cfg.zipf_tau * logp.to(device)
    return logits


def make_correction_bias(cfg: MoeConfig, device, seed: int = 3):
    return _randn((cfg.experts,), 0.01, seed, device)


def route(cfg: MoeConfig, logits: torch.Tensor,
          bias: Optional[torch.Tensor] = None):
    """Router of the configuration on the GPU kernels: returns
    (topk_weights f32 [T,k], topk_ids i32 [T,k])."""
    if cfg.routing == "grouped_sigmoid":
        w, ids = ops.fused_grouped_topk(logits, cfg.topk, cfg.renormalize, bias,
                                        cfg.n_group, cfg.topk_group, "sigmoid",
                                        cfg.routed_scaling_factor)
        return w, ids
    w, ids, _ = ops.topk_softmax(logits, cfg.topk, cfg.renormalize)
    return w, ids


def algorithmic_bytes(cfg: MoeConfig, T: int, active: int) -> float:
    """Roofline bytes per layer call: |A| experts' weights (+scales, biases)
    + x in + y out + logits + ids/weights; intermediates excluded."""
    H, I, E, k = cfg.hidden, cfg.inter, cfg.experts, cfg.topk
    n = 3 * H * I
    if cfg.recipe == "bf16":
        wb = 2 * n
    elif cfg.recipe == "fp8block":
        wb = n + 4 * n / (128 * 128)
    elif cfg.recipe == "mxfp8":
        wb = n + n / 32
    elif cfg.recipe == "fp8":
        wb = n + 8
    elif cfg.recipe == "int4":
        wb = n / 2 + 2 * n / 128
    else:
        wb = n / 2 + n / 32
    if cfg.bias:
        wb += 2 * (2 * I + H)
    x_in = T * (H / 2 + H / 32) if cfg.prequant else T * H * 2
    return active * wb + x_in + T * H * 2 + T * E * 4 + T * k * 8


def algorithmic_flops(cfg: MoeConfig, T: int) -> float:
    return 6.0 * T * cfg.topk * cfg.hidden * cfg.inter


PEAK_TFLOPS = {"bf16": 2500.0, "fp8block": 5000.0, "mxfp4": 2500.0, "mxfp8": 5000.0,
               "fp8": 2500.0, "int4": 2500.0}   # w8a16 / w4a16 run 16-bit MFMAs
PEAK_TFLOPS_FP4 = 10100.0   # e2m1 x e2m1 (pre-quantised mxfp4 input)
PEAK_HBM_GBS = 8000.0


def roofline_time_s(cfg: MoeConfig, T: int, active: int) -> tuple[float, float]:
    """(t_hbm, t_mfma) lower bounds in seconds.  mxfp4 with 16-bit input runs
    its MFMA in bf16 (weights dequantised in registers), so it is priced at
    the bf16 peak; with pre-quantised input at the fp4 peak."""
    peak = PEAK_TFLOPS_FP4 if cfg.prequant else PEAK_TFLOPS[cfg.recipe]
    return (algorithmic_bytes(cfg, T, active) / (PEAK_HBM_GBS * 1e9),
            algorithmic_flops(cfg, T) / (peak * 1e12))


def expected_active(E: int, slots: int) -> float:
    return E * (1.0 - (1.0 - 1.0 / E) ** slots)


__all__ = ["MoeConfig", "CONFIGS", "VARIANTS", "config", "make_weights", "make_activations",
           "make_router_logits", "make_correction_bias", "route",
           "fp8_block_quant", "mxfp4_quant", "mxfp8_quant", "expert_weights_nk",
           "algorithmic_bytes", "algorithmic_flops", "roofline_time_s",
           "math"]
