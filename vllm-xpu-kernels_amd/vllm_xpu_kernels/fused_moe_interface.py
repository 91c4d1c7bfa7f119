"""Fused MoE layer API (reference vllm_xpu_kernels/fused_moe_interface.py).

``XpuFusedMoe(...)`` keeps the reference constructor and ``apply`` signature
(:165-181, :273-281).  At construction the weights are converted once into
the layout the gfx950 kernels stream: every expert matrix [N, K] with K
contiguous, swigluoai's interleaved gate/up rows split into a gate half and an
up half, and bf16 weights with K % 32 == 0 (hidden and intermediate sizes)
or fp8 block-scaled weights with K <= 8192 further K-blocked to [E, K/B, N, B]
(B = 32 bf16 / 128 e4m3 elements, ``mi355_pack_weights_kblock``), so that
the kernels read each 16-row weight fragment of a K stage as one contiguous
1-2 KiB run.  ``MI355MOE_WEIGHT_LAYOUT=nk`` keeps the row-major [E, N, K]
layout.
``apply`` makes one call, ``torch.ops._moe_C.mi355_fused_moe``, which
launches the whole layer on the current stream without synchronising the
host.
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from . import _ops  # noqa: F401  (loads the HIP library)

REF_FUSED_MOE_ENV = "VLLM_XPU_FUSED_MOE_USE_REF"
USE_MXFP4_FP8_ENV = "VLLM_XPU_FUSED_MOE_USE_MXFP4_FP8"
FP8_BLOCK_SIZE = 128

RECIPE_BF16, RECIPE_FP8BLOCK, RECIPE_MXFP4, RECIPE_INT4, RECIPE_MXFP8 = 0, 1, 2, 3, 4
# per-expert fp8 weights read as they are (e4m3 / e5m2, converted in registers)
RECIPE_FP8, RECIPE_FP8E5M2 = 5, 6
# Per-expert fp8 weights are read as fp8 by every kernel family (hidden and
# intermediate sizes % 32 == 0; others run on exact 16-bit copies, made on
# the first call).  "0" always uses the copies.
FP8_W8A16_ENV = "MI355MOE_FP8_W8A16"
ACT_SILU, ACT_SWIGLUOAI, ACT_GELU, ACT_GELU_TANH, ACT_SWIGLUSTEP, ACT_RELU2 = range(6)
# reference fused_moe_interface.py:119-133, 239-254
_ACT_CODES = {"silu": ACT_SILU, "swigluoai": ACT_SWIGLUOAI, "gelu": ACT_GELU,
              "gelu_tanh": ACT_GELU_TANH, "swiglustep": ACT_SWIGLUSTEP,
              "relu2_no_mul": ACT_RELU2}
WLAYOUT_NK, WLAYOUT_KBLOCK = 0, 1
WEIGHT_LAYOUT_ENV = "MI355MOE_WEIGHT_LAYOUT"
# Default "1": the prepared weights (w13 / w2 and their mxfp4, mxfp8 and int4
# scales) are written over the caller's tensors, one expert at a time, so the
# weights are held once and the transient is one expert's bytes (the
# reference rewrites its int4 weights in place too, fused_moe_interface.py:
# 195-205).  Those tensors keep their shape and dtype but hold the prepared
# layout; a later XpuFusedMoe on them with the same arguments reuses it.
# "0" leaves the caller's tensors untouched and keeps a converted copy.
PREPARE_IN_PLACE_ENV = "MI355MOE_PREPARE_IN_PLACE"


def _is_env_enabled(env_name: str, default: str = "0") -> bool:
    value = os.environ.get(env_name, default).strip().upper()
    return value in ("1", "ON", "TRUE", "YES", "Y")


def _get_weights_dtype(weight, scales):
    """Recipe detection of the reference (fused_moe_interface.py:47-61)."""
    weight_dtype = weight.dtype
    is_fp8 = weight_dtype in (torch.float8_e4m3fn, torch.float8_e5m2)
    is_int4 = weight_dtype == torch.uint8 and (scales is None or
                                               scales.dtype != torch.uint8)
    is_mxfp4 = weight_dtype == torch.float4_e2m1fn_x2 or (
        weight_dtype == torch.uint8 and scales is not None and
        scales.dtype in (torch.uint8, torch.float8_e8m0fnu))
    is_mxfp8 = is_fp8 and scales is not None and scales.dtype == torch.uint8
    is_block_fp8 = (is_fp8 and scales is not None and
                    scales.dtype == torch.float32 and scales.ndim == 3)
    is_fp8 = is_fp8 and not is_mxfp8 and not is_block_fp8
    return is_fp8, is_int4, is_mxfp4, is_mxfp8, is_block_fp8


def _get_inter_size(w13, w13_scales, is_int4, is_mxfp4, is_block_fp8):
    """Reference fused_moe_interface.py:64-69."""
    if is_block_fp8:
        return w13_scales.shape[-2] * FP8_BLOCK_SIZE // 2
    if is_int4 or is_mxfp4:
        return w13.shape[-2] // 2
    return w13.shape[-1] // 2


def _bias16(b):
    if b is None:
        return None
    if b.dtype not in (torch.bfloat16, torch.float16):
        b = b.to(torch.bfloat16)
    return b.contiguous()


def _deinterleave_rows(t: torch.Tensor, dim: int) -> torch.Tensor:
    """[.., 2I, ..] with gate at even / up at odd rows -> [gate; up]."""
    even = t.narrow(dim, 0, t.shape[dim]).index_select(
        dim, torch.arange(0, t.shape[dim], 2, device=t.device))
    odd = t.index_select(dim, torch.arange(1, t.shape[dim], 2, device=t.device))
    return torch.cat([even, odd], dim=dim).contiguous()


def pack_weights_kblock(w: torch.Tensor) -> torch.Tensor:
    """[E, N, K] -> K-blocked [E, K/B, N, B] on the device: B = 32 values for
    16-bit, 128 for e4m3 weights; packed e2m1 pairs (uint8 [E, N, K/2]) go to
    [E, K/32, N, 16]."""
    E, N, Kb = w.shape
    if w.dtype == torch.uint8:        # e2m1 pairs: 16 bytes per 32 values
        B = 16
    else:
        B = 128 if w.element_size() == 1 else 32
    out = torch.empty((E, Kb // B, N, B), dtype=w.dtype, device=w.device)
    torch.ops._moe_C.mi355_pack_weights_kblock(w.contiguous(), out)
    return out


def _prepare(src: torch.Tensor, steps, in_place: bool) -> torch.Tensor:
    """Apply `steps` (maps of expert slices [e, ...] to their prepared
    layout) to src.  in_place: one expert at a time, each result written back
    over that expert's own bytes (every step keeps an expert's byte count),
    so the result shares src's storage; else a new tensor."""
    def run(t):
        for f in steps:
            t = f(t)
        return t.contiguous()
    if not in_place or not src.is_contiguous() or src.numel() == 0:
        return run(src)
    E = src.shape[0]
    flat = src.view(torch.uint8).reshape(E, -1)
    shape = dtype = None
    for e in range(E):
        p = run(src[e:e + 1])
        pb = p.view(torch.uint8).reshape(-1)
        if pb.numel() != flat.shape[1]:
            raise AssertionError("a weight preparation step changed an expert's size")
        if pb.data_ptr() != flat[e].data_ptr():
            flat[e].copy_(pb)
        shape, dtype = p.shape[1:], p.dtype
    return flat.view(dtype).view(E, *shape)


def _kblock32(w: torch.Tensor) -> torch.Tensor:
    """1-byte weights [E, N, K] -> [E, K/32, N, 32] (K % 32 == 0)."""
    E, N, K = w.shape
    b = w.view(torch.uint8).view(E, N, K // 32, 32).permute(0, 2, 1, 3).contiguous()
    return b.view(w.dtype)


def pack_scales_kblock(s: torch.Tensor) -> torch.Tensor:
    """mxfp4 e8m0 scales uint8 [E, N, K/32] -> [E, K/32, N] on the device."""
    E, N, KB = s.shape
    out = torch.empty((E, KB, N), dtype=s.dtype, device=s.device)
    torch.ops._moe_C.mi355_pack_scales_kblock(s.contiguous(), out)
    return out


# what _prepare_weights sets: a layer built on tensors prepared in place
# takes these from the layer that prepared them
_PREPARED_STATE = ("w13", "w2", "gemm1_wei_scales", "gemm2_wei_scales", "w13_bias",
                   "w2_bias", "_w_group", "_ws_rows", "_w_layout", "_kblock",
                   "_w8_recipe", "_w8_layout")


class XpuFusedMoe:
    """Drop-in for the reference's XpuFusedMoe (fused_moe_interface.py:165-419).

    Weight layouts accepted (as the reference):
      bf16 / fp16     w13 [E, H, 2I], w2 [E, I, H]            ("kn")
      fp8 block       w13 [E, 2I, H] or [E, H, 2I], w2 likewise, fp32 scales
                      [E, N/128, K/128]
      mxfp4           w13 [E, 2I, H/2] float4_e2m1fn_x2 (or uint8), e8m0
                      scales [E, 2I, H/32] uint8; w2 [E, H, I/2]
    """

    def __init__(self, w13, w13_scales, w13_bias, w2, w2_scales, w2_bias,
                 n_experts_per_token, activation, num_experts, ep_rank=0,
                 ep_size=1, expert_map=None,
                 gemm1_clamp_limit: Optional[float] = None):
        assert w13.is_contiguous() and w2.is_contiguous()
        (is_fp8, is_int4, is_mxfp4, is_mxfp8,
         is_block_fp8) = _get_weights_dtype(w13, w13_scales)
        self.inter_size = _get_inter_size(w13, w13_scales, is_int4, is_mxfp4,
                                          is_block_fp8)
        self.n_experts_per_token = n_experts_per_token
        self.activation = activation
        self.num_experts = num_experts
        self.ep_rank = ep_rank
        self.ep_size = ep_size
        self.is_fp8 = is_fp8
        self.is_int4 = is_int4
        self.is_mxfp4 = is_mxfp4
        self.is_mxfp8 = is_mxfp8
        self.is_block_fp8 = is_block_fp8
        self.gemm1_clamp_limit = gemm1_clamp_limit
        if "SWIGLUOAI" in str(activation):
            self._act = ACT_SWIGLUOAI
        elif activation in _ACT_CODES:
            self._act = _ACT_CODES[activation]
        else:
            raise ValueError(f"Unsupported FusedMoe activation: {activation}.")
        # relu2_no_mul keeps all 2I columns: the activation, and w2's K, are
        # 2I wide (reference :226)
        self.inter_size_scale = 2 if self._act == ACT_RELU2 else 1
        # per-expert fp8 (reference recipe "fp8", w8a16): the weights are
        # converted exactly to the call's 16-bit type and run the 16-bit
        # kernels with each expert's scale on the accumulators
        self._fp8_expert = is_fp8
        if is_block_fp8:
            self.recipe = "fp8block"
            self._recipe = RECIPE_FP8BLOCK
        elif is_fp8:
            self.recipe = "fp8"
            self._recipe = RECIPE_BF16
        elif is_int4:
            self.recipe = "int4"
            self._recipe = RECIPE_INT4
        elif is_mxfp4:
            # the reference's recipe selector (fused_moe_interface.py:33-44);
            # its kernel path runs mxfp4_fp8 as mxfp4
            self.recipe = "mxfp4_fp8" if _is_env_enabled(USE_MXFP4_FP8_ENV) else "mxfp4"
            self._recipe = RECIPE_MXFP4
        elif is_mxfp8:
            self.recipe = "mxfp8"
            self._recipe = RECIPE_MXFP8
        else:
            self.recipe = "bf16"
            self._recipe = RECIPE_BF16
        if _is_env_enabled(REF_FUSED_MOE_ENV):
            raise NotImplementedError(
                f"{REF_FUSED_MOE_ENV}=1 (torch reference path) is not provided "
                "by the MI355X build; the HIP kernels are the only path")
        # tensors an earlier layer prepared in place carry that preparation:
        # it is reused when every argument that shapes it is the same
        key = (self._recipe, self._fp8_expert, self._act, self.inter_size,
               os.environ.get(WEIGHT_LAYOUT_ENV, "kblock").lower(),
               _is_env_enabled(FP8_W8A16_ENV, "1"),
               bool(getattr(w13, "xpu_fused_moe", False)),
               tuple(None if t is None else (t.data_ptr(), tuple(t.shape), t.dtype)
                     for t in (w13, w13_scales, w13_bias, w2, w2_scales, w2_bias)))
        prev = [getattr(t, "mi355moe_prepared", None) for t in (w13, w2)]
        if prev[0] is not None or prev[1] is not None:
            if prev[0] is not prev[1] or prev[0][0] != key:
                raise ValueError(
                    "w13 / w2 hold weights another XpuFusedMoe prepared in place "
                    f"({PREPARE_IN_PLACE_ENV}=1) with other arguments; pass the "
                    "original tensors")
            self.__dict__.update(prev[0][1])
            self._w16_cache, self._bias_cache = {}, {}
        else:
            in_place = _is_env_enabled(PREPARE_IN_PLACE_ENV, "1")
            self._prepare_weights(w13, w13_scales, w13_bias, w2, w2_scales, w2_bias,
                                  in_place)
            if in_place:
                state = (key, {k: getattr(self, k) for k in _PREPARED_STATE})
                w13.mi355moe_prepared = w2.mi355moe_prepared = state

        self.expert_map = expert_map
        if self.expert_map is None and self.ep_size > 1:
            self.expert_map = torch.empty(self.num_experts * self.ep_size,
                                          dtype=torch.int32, device=w13.device)
            torch.ops._moe_C.init_expert_map(self.expert_map, self.num_experts,
                                             self.ep_rank, self.ep_size)
        if self.expert_map is not None:
            self.total_experts_num = self.expert_map.shape[0]
        else:
            self.total_experts_num = self.num_experts * self.ep_size
        self.local_experts_num = self.num_experts

    # ------------------------------------------------------------------
    def _prepare_weights(self, w13, s13, b13, w2, s2, b2, in_place=False):
        """Convert the reference layouts into the kernels' (see the module
        docstring); in_place: over the caller's tensors, one expert at a
        time."""
        I = self.inter_size
        K2 = I * self.inter_size_scale
        E = w13.shape[0]
        swiglu = self._act == ACT_SWIGLUOAI
        tr = lambda t: t.transpose(1, 2).contiguous()  # noqa: E731
        u8 = lambda t: t.view(torch.uint8)  # noqa: E731
        # per-tensor steps, each a map of expert slices [e, ...] that keeps an
        # expert's byte count
        f13, f2, fs13, fs2 = [], [], [], []
        self._w_group = 0
        self._ws_rows = 128
        if self._recipe == RECIPE_INT4:
            # u4 with zero point 8 -> two's-complement int4 (the reference's
            # implement_zp, :135-163, is (u4 - 8) & 0xF = u4 ^ 8 per nibble);
            # weights the reference already converted carry `xpu_fused_moe`
            f13 = [u8]
            if not getattr(w13, "xpu_fused_moe", False):
                f13 = [u8, lambda t: t ^ 0x88]
            f2 = list(f13)
            self._w_group = (w13.shape[2] * 2) // s13.shape[-1]
            if (K2 // s2.shape[-1]) != self._w_group:
                raise ValueError("w13 and w2 int4 scales must use one group size")
        elif self._fp8_expert:
            # reference layout [E, K, N] -> [E, N, K], kept in fp8 (read as
            # such by the decode kernels, K-blocked by 128 where the sizes
            # allow; exact 16-bit copies are made for larger calls)
            f13, f2 = [tr], [tr]
        elif self._recipe == RECIPE_BF16:
            if w13.dtype not in (torch.bfloat16, torch.float16):
                raise NotImplementedError("16-bit weights must be bfloat16 or float16")
            f13, f2 = [tr], [tr]      # reference layout [E, K, N] -> [E, N, K]
        elif self._recipe == RECIPE_MXFP8:
            # reference layout (moe_utils.py:80-82): w [E, K, N] e4m3 with e8m0
            # scales [E, K/32, N] -> [E, N, K] and [E, N, K/32]
            f13, f2 = [tr], [tr]
            fs13, fs2 = [u8, tr], [u8, tr]
        elif self._recipe == RECIPE_FP8BLOCK:
            # [E, N, K] preferred when ambiguous, as the reference
            # (grouped_gemm_xe2_interface.hpp:206-223)
            f13 = [] if w13.shape[1] == 2 * I else [tr]
            f2 = [] if w2.shape[2] == K2 else [tr]
        else:
            f13, f2, fs13, fs2 = [u8], [u8], [u8], [u8]
        if swiglu:
            # gate / up rows interleaved -> [gate; up] halves
            f13.append(lambda t: _deinterleave_rows(t, 1))
            if not self._fp8_expert and self._recipe != RECIPE_FP8BLOCK:
                fs13.append(lambda t: _deinterleave_rows(t, 1))
        # hidden size: K of w13 ([E, 2I, H/2] packed 4-bit, [E, 2I, H] or
        # [E, H, 2I] fp8 block, [E, H, 2I] otherwise)
        if self._recipe in (RECIPE_MXFP4, RECIPE_INT4):
            H = w13.shape[2] * 2
        elif self._recipe == RECIPE_FP8BLOCK and w13.shape[1] == 2 * I:
            H = w13.shape[2]
        else:
            H = w13.shape[1]
        self._w_layout = WLAYOUT_NK
        kblock = ((self._recipe == RECIPE_BF16 and H % 32 == 0 and I % 32 == 0) or
                  (self._recipe == RECIPE_FP8BLOCK and H <= 8192 and K2 <= 8192) or
                  (self._recipe == RECIPE_MXFP8 and H % 128 == 0 and K2 % 128 == 0) or
                  self._recipe in (RECIPE_MXFP4, RECIPE_INT4))
        self._kblock = kblock and os.environ.get(WEIGHT_LAYOUT_ENV, "kblock").lower() != "nk"
        if self._kblock and not self._fp8_expert:
            f13.append(pack_weights_kblock)
            f2.append(pack_weights_kblock)
            if self._recipe in (RECIPE_MXFP4, RECIPE_MXFP8):
                fs13.append(pack_scales_kblock)
                fs2.append(pack_scales_kblock)
            elif self._recipe == RECIPE_INT4:
                # 16-bit group scales [E, N, K/group] -> [E, K/group, N]
                fs13.append(tr)
                fs2.append(tr)
            self._w_layout = WLAYOUT_KBLOCK
        if self._fp8_expert and self._kblock:
            self._w_layout = WLAYOUT_KBLOCK   # applies to the 16-bit copies
        self._w8_recipe = None
        self._w8_layout = WLAYOUT_NK
        if self._fp8_expert and H % 32 == 0 and K2 % 32 == 0:
            self._w8_recipe = (RECIPE_FP8E5M2 if w13.dtype == torch.float8_e5m2
                               else RECIPE_FP8)
            if os.environ.get(WEIGHT_LAYOUT_ENV, "kblock").lower() != "nk":
                # K blocks of 32 bytes, [E, K/32, N, 32]: one 32-byte block
                # per lane in the STREAM / SMALL kernels, a 32-value stage of
                # 256 rows one 8 KB run in the 320-slot kernel
                f13.append(_kblock32)
                f2.append(_kblock32)
                self._w8_layout = WLAYOUT_KBLOCK
        self.w13 = _prepare(w13, f13, in_place)
        self.w2 = _prepare(w2, f2, in_place)
        if self._fp8_expert:
            s13c = s13.to(torch.float32).reshape(E).contiguous()
            s2c = s2.to(torch.float32).reshape(E).contiguous()
        elif self._recipe == RECIPE_BF16:
            s13c = s2c = None
        elif self._recipe == RECIPE_FP8BLOCK:
            s13c, s2c = s13.contiguous(), s2.contiguous()
            if swiglu:
                # 128-row scale block b of the interleaved rows holds gates and
                # ups j in [64 b, 64 b + 64): after the split, row n of either
                # half has scale row n / 64 of that half, so the kernels read
                # [E, 2I/64, K/128] scales (each half a copy of the original)
                s13c = torch.cat([s13c, s13c], dim=1)
                self._ws_rows = 64
        else:
            s13c = _prepare(s13, fs13, in_place)
            s2c = _prepare(s2, fs2, in_place)
        self.gemm1_wei_scales, self.gemm2_wei_scales = s13c, s2c
        # biases keep their 16-bit type; apply() converts them to the call's
        b13c = _bias16(b13)
        if swiglu and b13c is not None:
            b13c = _deinterleave_rows(b13c, 1)
        self.w13_bias, self.w2_bias = b13c, _bias16(b2)
        self._w16_cache = {}
        self._bias_cache = {}

    def _fp8_rows(self, w):
        """[E, N, K] view of kept per-expert fp8 weights."""
        if self._w8_layout != WLAYOUT_KBLOCK:
            return w
        E, KB, N, B = w.shape
        return w.permute(0, 2, 1, 3).reshape(E, N, KB * B)

    def _call_plan(self, dtype):
        """(recipe, w13, w2, weight layout) of a call in `dtype`: per-expert
        fp8 weights are read as they are (sizes % 32 == 0), else through
        exact 16-bit copies."""
        if self._w8_recipe is not None and _is_env_enabled(FP8_W8A16_ENV, "1"):
            return self._w8_recipe, self.w13, self.w2, self._w8_layout
        w13, w2 = self._call_weights(dtype)
        return self._recipe, w13, w2, self._w_layout

    def _call_weights(self, dtype):
        """(w13, w2) the 16-bit-recipe kernels read for a call in `dtype`:
        the prepared weights, or for per-expert fp8 their exact 16-bit copies
        (made once per dtype, K-blocked like 16-bit weights)."""
        if not self._fp8_expert:
            return self.w13, self.w2
        if dtype not in self._w16_cache:
            w13 = self._fp8_rows(self.w13).to(dtype)
            w2 = self._fp8_rows(self.w2).to(dtype)
            if self._kblock:
                w13, w2 = pack_weights_kblock(w13), pack_weights_kblock(w2)
            self._w16_cache[dtype] = (w13.contiguous(), w2.contiguous())
        return self._w16_cache[dtype]

    def _scales(self, dtype):
        """int4 group scales in the call's 16-bit type."""
        s13, s2 = self.gemm1_wei_scales, self.gemm2_wei_scales
        if self._recipe != RECIPE_INT4 or s13.dtype == dtype:
            return s13, s2
        key = ("scales", dtype)
        if key not in self._bias_cache:
            self._bias_cache[key] = (s13.to(dtype).contiguous(), s2.to(dtype).contiguous())
        return self._bias_cache[key]

    def _biases(self, dtype):
        """Biases in the call's 16-bit type (the kernels read them as such)."""
        if self.w13_bias is None and self.w2_bias is None:
            return None, None
        if all(b is None or b.dtype == dtype for b in (self.w13_bias, self.w2_bias)):
            return self.w13_bias, self.w2_bias
        if dtype not in self._bias_cache:
            self._bias_cache[dtype] = tuple(
                None if b is None else b.to(dtype).contiguous()
                for b in (self.w13_bias, self.w2_bias))
        return self._bias_cache[dtype]

    # ------------------------------------------------------------------
    def apply(self, output, hidden_states, topk_weights, topk_ids,
              expert_map=None, a1q_scale=None):
        if a1q_scale is not None:
            # hidden_states already quantised, consumed with their scales as
            # the reference's torch path dequantises them (moe_utils.py:189-199,
            # 285-300): fp8block e4m3 + f32 [T, H/128]; mxfp8 e4m3 + e8m0
            # [T, H/32]; mxfp4 packed e2m1 [T, H/2] + e8m0 [T, H/32], both GEMMs
            # then e2m1 x e2m1
            if self._recipe == RECIPE_FP8BLOCK:
                a1q_scale = a1q_scale.to(torch.float32).contiguous()
            elif self._recipe in (RECIPE_MXFP8, RECIPE_MXFP4):
                if self.recipe == "mxfp4_fp8":
                    # the reference's quant_act_xpu has no mxfp4_fp8 path
                    raise NotImplementedError(
                        "Unsupported recipe for quant_act_xpu: mxfp4_fp8")
                a1q_scale = a1q_scale.view(torch.uint8).contiguous()
                if self._recipe == RECIPE_MXFP4:
                    hidden_states = hidden_states.view(torch.uint8)
            else:
                raise NotImplementedError(
                    "pre-quantised activations (a1q_scale) are supported for the "
                    "fp8block, mxfp8 and mxfp4 recipes")
        # the call's 16-bit type: that of the activations, or of the output
        # when they come quantised; the kernels write the output, and read
        # the biases, in it
        dt16 = output.dtype if a1q_scale is not None else hidden_states.dtype
        if dt16 not in (torch.bfloat16, torch.float16):
            raise ValueError(f"output must be bfloat16 or float16, got {dt16}")
        if output.dtype != dt16:
            raise ValueError(f"output ({output.dtype}) must have hidden_states' "
                             f"dtype ({hidden_states.dtype})")
        if (self._recipe == RECIPE_BF16 and not self._fp8_expert and
                hidden_states.dtype != self.w13.dtype):
            raise ValueError(f"hidden_states ({hidden_states.dtype}) must have the "
                             f"16-bit weights' dtype ({self.w13.dtype})")
        if tuple(topk_weights.shape) != tuple(topk_ids.shape):
            raise ValueError("topk_weights and topk_ids must have the same shape")
        if expert_map is None and self.ep_size > 1:
            expert_map = self.expert_map
        clamp = float(self.gemm1_clamp_limit) if self.gemm1_clamp_limit else 0.0
        if self._recipe == RECIPE_MXFP8:
            # the reference runs mxfp8 through ref_fused_moe, which takes no
            # clamp limit (fused_moe_interface.py:27-30, 296-317)
            clamp = 0.0
        b13, b2 = self._biases(dt16)
        recipe, w13, w2, layout = self._call_plan(dt16)
        s13, s2 = self._scales(dt16)
        torch.ops._moe_C.mi355_fused_moe(
            output, hidden_states, topk_weights.to(torch.float32).contiguous(),
            topk_ids.contiguous(), w13, s13, b13, w2, s2, b2,
            recipe, self._act, self.inter_size, clamp, expert_map,
            layout, a1q_scale, self._w_group, self._ws_rows)
        return output


def xpu_fused_moe(hidden_states,
                  w13,
                  w13_scales,
                  w13_bias,
                  w2,
                  w2_scales,
                  w2_bias,
                  topk_weights,
                  topk_ids,
                  n_experts_per_token,
                  activation,
                  num_experts,
                  ep_rank=0,
                  ep_size=1,
                  expert_map=None,
                  output=None,
                  is_fp8=False,
                  is_int4=False,
                  is_mxfp4=False,
                  is_mxfp8=False,
                  is_block_fp8=False,
                  gemm1_clamp_limit: Optional[float] = None):
    """Functional entry (reference fused_moe_interface.py:421-442, same
    parameters in the same order): builds an XpuFusedMoe and applies it once.

    The is_* flags name the recipe as the reference's do; the weight and
    scale dtypes must agree with the flag that is set (the reference reads the
    flags only, this build checks them against the tensors and raises
    ValueError on a mismatch).  No flag set: the recipe follows the dtypes.
    """
    if output is None:
        output = torch.empty_like(hidden_states)
    else:
        assert output.shape == hidden_states.shape, \
            "output shape must be the same as hidden_states shape"
    flags = {"fp8": is_fp8, "int4": is_int4, "mxfp4": is_mxfp4,
             "mxfp8": is_mxfp8, "block_fp8": is_block_fp8}
    asked = [k for k, v in flags.items() if v]
    if len(asked) > 1:
        raise ValueError(f"xpu_fused_moe: more than one recipe flag set: {asked}")
    det = dict(zip(("fp8", "int4", "mxfp4", "mxfp8", "block_fp8"),
                   _get_weights_dtype(w13, w13_scales)))
    if asked and not det[asked[0]]:
        found = [k for k, v in det.items() if v] or ["bf16"]
        raise ValueError(f"xpu_fused_moe: is_{asked[0]}=True but w13 "
                         f"({w13.dtype}) with scales "
                         f"({None if w13_scales is None else w13_scales.dtype}) "
                         f"is recipe {found[0]}")
    moe = XpuFusedMoe(w13, w13_scales, w13_bias, w2, w2_scales, w2_bias,
                      n_experts_per_token, activation, num_experts, ep_rank,
                      ep_size, expert_map, gemm1_clamp_limit)
    moe.apply(output, hidden_states, topk_weights, topk_ids,
              expert_map=expert_map)
    return output
