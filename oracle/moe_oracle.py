"""CPU restatement of the reference's fused-MoE path (TEST INFRASTRUCTURE ONLY).

Every function restates the reference algorithm named in its docstring
(paths relative to the reference repository root).  It is used as the checker
by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` and nothing else; the product library never calls it.

Pinning (how each function is checked independently of a retyped formula):

* ``topk_softmax`` / ``topk_sigmoid``   brute-force stable sort, softmax
  monotonicity, invariants (ids unique, in range, ordered)  -> pinned
* ``grouped_topk``                      brute force over every subset of groups
  on small cases + invariants                               -> pinned
* ``moe_align_block_size``              docstring KAT (tests/ops/
  moe_align_block_size_ops.py:56-69), golden stable-sort restatement of
  tests/test_moe_align_block_size.py:97-183                 -> pinned
* ``silu_and_mul`` / ``swigluoai_and_mul`` closed forms at special points
  (x=0, clamp limits) and torch.nn.functional.silu           -> pinned
* ``per_token_group_fp8_quant``         exact e4m3 grid (all 254 finite codes),
  round-trip and scale closed form                          -> pinned
* ``per_token_group_quant_mxfp4``       known-value KAT
  (tests/test_mxfp4_quant.py:113-142)                       -> pinned
* ``to_mxfp4``                          RCEIL/RNE special cases, e2m1 grid
  round trip                                                -> pinned
* ``moe_sum`` / ``moe_gather``          fixed-order fp32 sums vs float64 sum  -> pinned
* ``remap_hidden_states``               un-permute invariant (tests/fused_moe/
  test_remap_hidden_states.py:204-217)                      -> pinned
* ``grouped_gemm`` / ``fused_moe``      all-finite-e4m3 identity KAT
  (tests/fused_moe/test_grouped_gemm.py:275-307), E=1 special case vs
  torch.matmul, per-expert brute force                      -> pinned

The layer functions (quantisers, dequantisers, ``grouped_gemm``,
``fused_moe``) use torch operations only and run on the tensors' device; the
GPU tests run them on the device to check every token of the full-size
prefill layers (fp32 matmuls with the same rounding points).
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch

FP8_MAX = 448.0
FP8_MIN_SCALE = 1.0 / (448.0 * 512.0)   # csrc/quantization/fp8/quant_utils.h:35-37
FP4_MAX = 6.0
E2M1_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _div_const(a: torch.Tensor, c: float) -> torch.Tensor:
    """a / c correctly rounded on every device.  torch's GPU division by a
    Python scalar multiplies by the rounded reciprocal (one ulp off for about
    half of the inputs when c = 448); a tensor divisor divides exactly, as
    the CPU path and the kernels do."""
    return a / torch.full_like(a, c)


# ----------------------------------------------------------------------------
# Routing
# ----------------------------------------------------------------------------
def _stable_topk_desc(vals: torch.Tensor, k: int):
    """Descending top-k with ties to the lower index (tests/ops/topk_op.py:11-13,
    csrc/moe/topk.cpp:536-545)."""
    v, i = torch.sort(vals, dim=-1, descending=True, stable=True)
    return v[..., :k], i[..., :k]


def topk_softmax(gating: torch.Tensor, topk: int, renormalize: bool,
                 bias: Optional[torch.Tensor] = None):
    """tests/ops/topk_op.py:16-35 with the kernel's renorm guard
    (csrc/moe/topk.cpp:573-583) and token_expert_indices (topk.cpp:563).

    Returns (weights f32 [T,k], ids i32 [T,k], token_expert_indices i32 [T,k]).
    """
    T, E = gating.shape
    p = torch.softmax(gating.float(), dim=-1)
    sel = p + bias.float().unsqueeze(0) if bias is not None else p
    _, ids = _stable_topk_desc(sel, topk)
    w = p.gather(1, ids)
    if renormalize:
        s = w.sum(dim=-1, keepdim=True)
        w = w * (1.0 / torch.where(s > 0, s, torch.ones_like(s)))
    tei = (torch.arange(topk, dtype=torch.int32).unsqueeze(0) * T +
           torch.arange(T, dtype=torch.int32).unsqueeze(1))
    return w.float(), ids.int(), tei


def sigmoid_typed(x: torch.Tensor) -> torch.Tensor:
    """sigmoid in fp32 rounded to the input dtype (csrc/moe/topk.cpp:17-23)."""
    s = 1.0 / (1.0 + torch.exp(-x.float()))
    return s.to(x.dtype).float()


def topk_sigmoid(gating: torch.Tensor, topk: int, renormalize: bool,
                 bias: Optional[torch.Tensor] = None,
                 routed_scaling_factor: float = 1.0):
    """tests/ops/topk_op.py:38-59 with csrc/moe/topk.cpp:573-583 scaling."""
    T, E = gating.shape
    p = sigmoid_typed(gating)
    sel = p + bias.float().unsqueeze(0) if bias is not None else p
    _, ids = _stable_topk_desc(sel, topk)
    w = p.gather(1, ids)
    scale = torch.full((T, 1), float(routed_scaling_factor))
    if renormalize:
        s = w.sum(dim=-1, keepdim=True)
        scale = scale / torch.where(s > 0, s, torch.ones_like(s))
    w = w * scale
    tei = (torch.arange(topk, dtype=torch.int32).unsqueeze(0) * T +
           torch.arange(T, dtype=torch.int32).unsqueeze(1))
    return w.float(), ids.int(), tei


def topk_softplus_sqrt(gating: torch.Tensor, topk: int, renormalize: bool,
                       routed_scaling_factor: float = 1.0,
                       correction_bias: Optional[torch.Tensor] = None,
                       input_ids: Optional[torch.Tensor] = None,
                       tid2eid: Optional[torch.Tensor] = None):
    """csrc/moe/topk_softplus_sqrt_kernels.cpp:233-416: s = sqrt(x if x > 20
    else log(1 + exp(x))) in fp32; top-k of s + bias (value desc, id asc),
    weight (s + b) - b; hash: ids tid2eid[input_ids[t]], weights s (non-finite
    -> 0); scale = rsf / (sum if renormalize and sum > 0, else 1 when
    renormalize), weights * scale.  Returns (weights f32, ids i64)."""
    x = gating.float()
    s = torch.sqrt(torch.where(x > 20, x, torch.log(1.0 + torch.exp(x))))
    T, E = s.shape
    if tid2eid is not None:
        ids = tid2eid.long()[input_ids.long()][:, :topk]
        w = s.gather(1, ids.clamp(0, E - 1))
        w = torch.where(torch.isfinite(w) & (ids >= 0) & (ids < E), w, torch.zeros_like(w))
    else:
        sel = s + correction_bias.float().unsqueeze(0) if correction_bias is not None else s
        _, ids = _stable_topk_desc(sel, topk)
        w = sel.gather(1, ids)
        if correction_bias is not None:
            w = w - correction_bias.float()[ids]
    scale = torch.full((T, 1), float(routed_scaling_factor))
    if renormalize:
        tot = w.sum(-1, keepdim=True)
        scale = scale / torch.where(tot > 0, tot, torch.ones_like(tot))
    return w * scale, ids


def grouped_topk(scores: torch.Tensor, scores_with_bias: torch.Tensor,
                 n_group: int, topk_group: int, topk: int, renormalize: bool,
                 routed_scaling_factor: float):
    """Kernel semantics of csrc/moe/grouped_topk.cpp:405-695 (golden
    tests/ops/grouped_topk_op.py:11-64).

    * group score = top1 + top2 of scores_with_bias inside the group, summed
      in fp32 and stored in the input dtype (:433-446);
    * keep ``topk_group`` groups by (score desc, group asc) (:556-623);
    * ids = top-k of scores_with_bias over the kept groups, (value desc,
      id asc) (:588-625, ``is_better_than`` :36-45);
    * weights = scores[ids] / (1e-20 + sum) (if renormalize) * rsf, rounded
      to the input dtype (:636-668); all-(-inf) group scores fall back to
      ids 0..k-1 with 1/k (:669-674).

    Returns (values [T,k] in scores.dtype, ids int32 [T,k]) ordered by
    descending scores_with_bias.
    """
    dt = scores.dtype
    T, E = scores.shape
    epg = E // n_group
    sb = scores_with_bias.float()
    sbv = sb.view(T, n_group, epg)
    top2 = torch.topk(sbv, 2 if epg >= 2 else 1, dim=-1).values
    gs = top2.sum(-1) if epg >= 2 else top2[..., 0] * 2
    gs = gs.to(dt).float()
    vals = torch.empty(T, topk, dtype=torch.float32)
    ids = torch.empty(T, topk, dtype=torch.int32)
    for t in range(T):
        g = gs[t].clone()
        g[~torch.isfinite(g)] = -math.inf
        order = sorted(range(n_group), key=lambda i: (-g[i].item(), i))
        kept = order[:topk_group]
        if g[kept[-1]].item() == -math.inf and g[order[0]].item() == -math.inf:
            ids[t] = torch.arange(topk, dtype=torch.int32)
            vals[t] = 1.0 / topk
            continue
        cand = []
        for gi in sorted(kept):
            for e in range(gi * epg, (gi + 1) * epg):
                v = sb[t, e].item()
                cand.append((-(v if math.isfinite(v) else -math.inf), e))
        cand.sort()
        sel = [e for _, e in cand[:topk]]
        w = scores[t, sel].float()
        if renormalize:
            ssum = np.float32(1e-20)
            for x in w.tolist():
                ssum = np.float32(ssum + np.float32(x))
            w = w / float(ssum) * routed_scaling_factor
        else:
            w = w * routed_scaling_factor
        ids[t] = torch.tensor(sel, dtype=torch.int32)
        vals[t] = w
    return vals.to(dt), ids


# ----------------------------------------------------------------------------
# Alignment / permutation
# ----------------------------------------------------------------------------
def align_buffer_sizes(numel: int, num_experts: int, block_size: int,
                       pad_sorted_ids: bool = False):
    """Caller-side buffer sizes (tests/ops/moe_align_block_size_ops.py:71-86)."""
    mx = numel + num_experts * (block_size - 1)
    if pad_sorted_ids:
        mx = (mx + block_size - 1) // block_size * block_size
    if numel < num_experts:
        mx = min(numel * block_size, mx)
    return mx, (mx + block_size - 1) // block_size


def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int,
                         block_size: int, max_num_tokens_padded: int,
                         max_num_m_blocks: int,
                         expert_map: Optional[torch.Tensor] = None):
    """Stable counting sort of the flattened ids (golden
    tests/test_moe_align_block_size.py:97-183; kernel id filtering
    csrc/moe/moe_align_sum_kernels.cpp:196-206, expert-map remap :330-336,
    tail expert ids = 0 :266-272).

    Ids outside [0, num_experts) and experts mapped to -1 are dropped.
    Returns numpy int32 arrays (sorted_token_ids, expert_ids, ntp[1]).
    """
    flat = topk_ids.reshape(-1).to(torch.int64).numpy()
    numel = flat.size
    local = flat.copy()
    valid = (flat >= 0) & (flat < num_experts)
    if expert_map is not None:
        em = expert_map.to(torch.int64).numpy()
        local = np.where(valid, em[np.clip(flat, 0, len(em) - 1)], -1)
        valid = valid & (local >= 0)
    counts = np.bincount(local[valid], minlength=num_experts)[:num_experts]
    padded = (counts + block_size - 1) // block_size * block_size
    cumsum = np.concatenate([[0], np.cumsum(padded)]).astype(np.int64)
    sorted_ids = np.full(max_num_tokens_padded, numel, dtype=np.int32)
    expert_ids = np.zeros(max_num_m_blocks, dtype=np.int32)
    order = np.argsort(np.where(valid, local, num_experts), kind="stable")
    pos = cumsum[:-1].copy()
    for i in order[:int(valid.sum())]:
        e = local[i]
        sorted_ids[pos[e]] = i
        pos[e] += 1
    for e in range(num_experts):
        expert_ids[cumsum[e] // block_size:cumsum[e + 1] // block_size] = e
    ntp = np.array([cumsum[-1]], dtype=np.int32)
    return sorted_ids, expert_ids, ntp


def moe_lora_align_block_size(topk_ids: torch.Tensor,
                              token_lora_mapping: torch.Tensor,
                              num_experts: int, block_size: int, max_loras: int,
                              max_num_tokens_padded: int, max_num_m_blocks: int,
                              sorted_token_ids: np.ndarray,
                              expert_ids: np.ndarray,
                              num_tokens_post_pad: np.ndarray,
                              adapter_enabled: torch.Tensor,
                              lora_ids: torch.Tensor,
                              expert_map: Optional[torch.Tensor] = None) -> None:
    """Multi-LoRA alignment, in place on the numpy outputs
    (csrc/moe/moe_align_sum_kernels.cpp:800-845 and :984-1025: adapter
    id = lora_ids[w] for w < max_loras + 1, skipped when -1, >= max_loras or
    disabled; token mask token_lora_mapping[i // topk] == id :196-216; row
    slices at id * max_num_tokens_padded / id * max_num_m_blocks :165-170;
    unused blocks get -1 :839,267-272; padding value numel :172-178).

    Inside one adapter's slice the slots are in flat order per expert (the
    reference scatters them in any order within an expert's blocks).
    """
    topk = topk_ids.shape[1]
    tok = token_lora_mapping.to(torch.int64).numpy()
    lids = lora_ids.to(torch.int64).numpy()
    enabled = adapter_enabled.to(torch.int64).numpy()
    flat = topk_ids.reshape(-1).to(torch.int64)
    for w in range(min(len(lids), max_loras + 1)):
        lid = int(lids[w])
        if lid == -1 or lid >= max_loras or enabled[lid] == 0:
            continue
        mask = torch.from_numpy(np.repeat(tok[:len(flat) // topk] == lid, topk))
        # masked-out slots become an out-of-range id, which the sort drops
        ids = torch.where(mask, flat, torch.full_like(flat, num_experts))
        srt, eid, ntp = moe_align_block_size(ids, num_experts, block_size,
                                             max_num_tokens_padded,
                                             max_num_m_blocks, expert_map)
        nblk = int(ntp[0]) // block_size
        eid[nblk:] = -1
        sorted_token_ids[lid * max_num_tokens_padded:
                         (lid + 1) * max_num_tokens_padded] = srt
        expert_ids[lid * max_num_m_blocks:(lid + 1) * max_num_m_blocks] = eid
        num_tokens_post_pad[lid] = ntp[0]


PROLOGUE_SECTIONS = ("permuted_row_to_unpermuted_row", "permuted_token_selected_experts",
                     "unpermuted_row_to_permuted_row", "blocked_expert_counts",
                     "blocked_expert_counts_cumsum", "blocked_row_to_unpermuted_row",
                     "expert_first_token_offset", "permuted_token_final_scales",
                     "overlapped_gemm1_gemm2_inputs", "permuted_act_scales")


def prologue_tokens_per_block(T: int, E: int) -> int:
    """csrc/moe/fused_moe_prologue.hpp:35-46."""
    tpb = 32
    while tpb <= 1024:
        if -(-T // tpb) * E <= tpb:
            return tpb
        tpb *= 2
    return 1024


def prologue_layout(T: int, k: int, hidden: int, elem_bytes: int, block_k: int,
                    scale_bytes: int, E: int):
    """Workspace sections in order, each padded to 256 bytes
    (csrc/moe/fused_moe_prologue.cpp:40-102).  Returns (total, {name: (size,
    offset)})."""
    N = T * k
    nblk = -(-T // prologue_tokens_per_block(T, E)) if T else 0
    raw = [N * 4, N * 4, N * 4, E * nblk * 4, E * nblk * 4, E * T * 4, (E + 1) * 8, N * 4,
           N * hidden * elem_bytes, (N * hidden // block_k) * scale_bytes if scale_bytes else 0]
    out, at = {}, 0
    for name, r in zip(PROLOGUE_SECTIONS, raw):
        sz = (r + 255) // 256 * 256
        out[name] = (sz, at)
        at += sz
    return at, out


def fused_moe_prologue(rows: np.ndarray, scale_rows: Optional[np.ndarray],
                       token_selected_experts: np.ndarray,
                       token_final_scales: np.ndarray, num_experts_on_rank: int,
                       ep_rank: int = 0):
    """The reference's three-step permutation and row expansion
    (csrc/moe/fused_moe_prologue.hpp:154-229 block scan: token t matches
    expert e at its FIRST top-k position j with id - start == e, expanded row
    j * T + t; :260-372 prefix sums -> expert_first_token_offset; :423-472
    merge -> the three index maps; :555-640 expand: row copy, scale-row copy,
    token scale of flat slot t * k + j).

    rows: u8 [T, row_bytes] (the input's bytes); scale_rows: u8 [T,
    srow_bytes] or None.  Returns a dict of the written section values
    (index maps over routed rows only; unpermuted_row_to_permuted_row as
    {expanded row: permuted row}).
    """
    ids = np.asarray(token_selected_experts, dtype=np.int64)
    T, k = ids.shape
    E = num_experts_on_rank
    start = E * ep_rank
    p2u, experts = [], []
    offsets = np.zeros(E + 1, dtype=np.int64)
    tok = np.arange(T, dtype=np.int64)
    for e in range(E):
        offsets[e] = sum(len(r) for r in p2u)
        match = ids - start == e                 # [T, k]
        has = match.any(axis=1)
        first = match.argmax(axis=1)             # first matching position j
        p2u.append(first[has] * T + tok[has])    # tokens ascending
        experts.append(np.full(int(has.sum()), e))
    p2u = np.concatenate(p2u).astype(np.int32) if E else np.zeros(0, np.int32)
    offsets[E] = p2u.size
    u2p = {int(r): p for p, r in enumerate(p2u)}
    src_t = p2u % T if T else p2u
    src_j = p2u // T if T else p2u
    fs = np.asarray(token_final_scales, dtype=np.float32).reshape(T, k)
    return {
        "permuted_row_to_unpermuted_row": p2u,
        "permuted_token_selected_experts": np.concatenate(experts).astype(np.int32),
        "unpermuted_row_to_permuted_row": u2p,
        "expert_first_token_offset": offsets,
        "permuted_token_final_scales": fs[src_t, src_j],
        "overlapped_gemm1_gemm2_inputs": rows[src_t],
        "permuted_act_scales": None if scale_rows is None else scale_rows[src_t],
    }


def remap_hidden_states(hidden: torch.Tensor, topk_ids: torch.Tensor,
                        local_experts_num: int,
                        expert_map: Optional[torch.Tensor] = None,
                        scales: Optional[torch.Tensor] = None):
    """tests/fused_moe/test_remap_hidden_states.py:38-83 (stable order: the
    destination of slot (t, j) is prefix[e] + rank of (t, j) among earlier
    slots of the same expert in row-major order).

    Returns (remapped [T*k,H], remapped_scales or None, rows_per_expert [E]
    int32, perm [T,k] int32 (-1 when not local)).
    """
    T, k = topk_ids.shape
    ids = topk_ids.to(torch.int64)
    if expert_map is not None:
        ids = expert_map.to(torch.int64)[ids]
    counts = torch.bincount(ids[ids >= 0].flatten(),
                            minlength=local_experts_num)[:local_experts_num]
    prefix = torch.cat([torch.zeros(1, dtype=torch.int64), counts.cumsum(0)])
    off = torch.zeros(local_experts_num, dtype=torch.int64)
    perm = torch.full((T, k), -1, dtype=torch.int32)
    out = torch.zeros((T * k,) + tuple(hidden.shape[1:]), dtype=hidden.dtype)
    out_s = None
    if scales is not None:
        out_s = torch.zeros((T * k,) + tuple(scales.shape[1:]),
                            dtype=scales.dtype)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e < 0:
                continue
            d = int(prefix[e] + off[e])
            off[e] += 1
            out[d] = hidden[t]
            if scales is not None:
                out_s[d] = scales[t]
            perm[t, j] = d
    return out, out_s, counts.to(torch.int32), perm


def init_expert_map(num_experts: int, ep_rank: int, ep_size: int):
    """csrc/moe/init_expert_map.cpp:40-60: map[g] = g - rank*E if local."""
    g = torch.arange(num_experts * ep_size, dtype=torch.int32)
    lo = ep_rank * num_experts
    return torch.where((g >= lo) & (g < lo + num_experts), g - lo,
                       torch.full_like(g, -1))


# ----------------------------------------------------------------------------
# Reductions
# ----------------------------------------------------------------------------
def moe_sum(inp: torch.Tensor, topk_ids: Optional[torch.Tensor] = None,
            expert_map: Optional[torch.Tensor] = None):
    """csrc/moe/moe_align_sum_kernels.cpp:585-664: out[t] = T(sum_j float(in[t,j]))
    in fixed j order, skipping id<0 and expert_map[id]<0."""
    T, k, H = inp.shape
    acc = torch.zeros(T, H, dtype=torch.float32)
    for j in range(k):
        x = inp[:, j].float()
        if topk_ids is not None:
            ids = topk_ids[:, j].to(torch.int64)
            ok = ids >= 0
            if expert_map is not None:
                em = expert_map.to(torch.int64)
                ok = ok & (em[ids.clamp(min=0)] >= 0)
            x = x * ok.unsqueeze(1).float()
        acc = acc + x
    return acc.to(inp.dtype)


def moe_gather(moe_output: torch.Tensor, topk_weights: torch.Tensor,
               perm: torch.Tensor):
    """csrc/moe/moe_gather.cpp:9-98: y[t] = T(sum_j w[t,j] * float(G[perm[t,j]]))
    in fixed j order, skipping perm == -1."""
    T, k = perm.shape
    H = moe_output.shape[1]
    acc = torch.zeros(T, H, dtype=torch.float32, device=moe_output.device)
    for j in range(k):
        p = perm[:, j].to(torch.int64)
        ok = p >= 0
        rows = moe_output[p.clamp(min=0)].float()
        acc = acc + torch.where(ok.unsqueeze(1),
                                topk_weights[:, j].float().unsqueeze(1) * rows,
                                torch.zeros_like(rows))
    return acc.to(moe_output.dtype)


# ----------------------------------------------------------------------------
# Activations
# ----------------------------------------------------------------------------
def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """csrc/activation.cpp:16-20,81-87: out = T(float(T(silu_f32(g))) * float(u)),
    g = x[..., :d], u = x[..., d:]."""
    d = x.shape[-1] // 2
    g = x[..., :d].float()
    u = x[..., d:].float()
    s = (g / (1.0 + torch.exp(-g))).to(x.dtype).float()
    return (s * u).to(x.dtype)


def swigluoai_and_mul(x: torch.Tensor, alpha: float = 1.702,
                      limit: float = 7.0) -> torch.Tensor:
    """csrc/activation.cpp:277-295: interleaved gate/up, fp32, one rounding."""
    g = x[..., 0::2].float().clamp(max=limit)
    u = x[..., 1::2].float().clamp(min=-limit, max=limit)
    glu = g * (1.0 / (1.0 + torch.exp(-g * alpha)))
    return ((u + 1.0) * glu).to(x.dtype)


def gelu_erf_f32(f: torch.Tensor) -> torch.Tensor:
    """csrc/activation.cpp:52-60: f * 0.5 * (1 + erf(f / sqrt(2))) in fp32."""
    return f * 0.5 * (1.0 + torch.erf(f * 0.7071067811865476))


def gelu_tanh_f32(f: torch.Tensor) -> torch.Tensor:
    """csrc/activation.cpp:62-73: 0.5 f (1 + tanh(sqrt(2/pi) (f + 0.044715
    f^3))) in fp32."""
    inner = 0.7978845608028654 * (f + 0.044715 * (f * f * f))
    return 0.5 * f * (1.0 + torch.tanh(inner))


def gelu_and_mul(x: torch.Tensor, approximate: str = "none") -> torch.Tensor:
    """csrc/activation.cpp:81-86 (act_first): out = T(float(T(gelu(g))) * u),
    g = x[..., :d], u = x[..., d:]."""
    d = x.shape[-1] // 2
    g = x[..., :d].float()
    u = x[..., d:].float()
    a = gelu_erf_f32(g) if approximate == "none" else gelu_tanh_f32(g)
    return (a.to(x.dtype).float() * u).to(x.dtype)


def swiglustep_and_mul(x: torch.Tensor, limit: float = 7.0) -> torch.Tensor:
    """csrc/activation.cpp:297-311: T(min(silu(g), limit) * clamp(u, +-limit))
    in fp32, one rounding."""
    d = x.shape[-1] // 2
    g = x[..., :d].float()
    u = x[..., d:].float()
    sg = torch.clamp(g / (1.0 + torch.exp(-g)), max=limit)
    return (sg * u.clamp(min=-limit, max=limit)).to(x.dtype)


def relu2_no_mul(x: torch.Tensor) -> torch.Tensor:
    """csrc/activation.cpp:44-50: T(max(x, 0)^2) elementwise."""
    r = torch.clamp(x.float(), min=0.0)
    return (r * r).to(x.dtype)


# ----------------------------------------------------------------------------
# Quantisation
# ----------------------------------------------------------------------------
def per_token_group_fp8_quant(x: torch.Tensor, group_size: int,
                              eps: float = 1e-10, scale_ue8m0: bool = False):
    """csrc/quantization/fp8/fp8_quant.cpp:209-255 + quant_utils.h:35-37,61-71:
    amax = max(eps, max|x|); s = max(amax/448, 1/(448*512)); optional
    s = 2^ceil(log2(max(|s|,1e-10))); q = e4m3(clamp(x * (1/s), +-448)).
    Returns (q float8_e4m3fn [M,K], s float32 [M, K/group])."""
    M, K = x.shape
    xg = x.float().reshape(M, K // group_size, group_size)
    amax = torch.clamp(xg.abs().amax(-1), min=eps)
    s = torch.clamp(_div_const(amax, FP8_MAX), min=FP8_MIN_SCALE)
    if scale_ue8m0:
        s = torch.exp2(torch.ceil(torch.log2(torch.clamp(s.abs(), min=1e-10))))
    inv = 1.0 / s
    q = torch.clamp(xg * inv.unsqueeze(-1), -FP8_MAX, FP8_MAX)
    return q.reshape(M, K).to(torch.float8_e4m3fn), s


def dequant_fp8_groups(q: torch.Tensor, s: torch.Tensor, group_size: int):
    """vllm_xpu_kernels/moe_utils.py:143-148 (dequant_fp8_block_act)."""
    M, K = q.shape
    return (q.float().reshape(M, K // group_size, group_size) *
            s.unsqueeze(-1)).reshape(M, K)


def fp4_code(a: torch.Tensor) -> torch.Tensor:
    """Strict-midpoint e2m1 code of csrc/quantization/fp4/mxfp4_quant.h:17-25
    (round-half-toward-zero in magnitude); sign bit from x < 0."""
    b = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    m = a.abs()
    code = torch.zeros_like(a, dtype=torch.int32)
    for t in b:
        code += (m > t).int()
    return code | ((a < 0).int() << 3)


def per_token_group_quant_mxfp4(x: torch.Tensor, group_size: int = 32,
                                eps: float = 1e-10):
    """csrc/quantization/fp4/mxfp4_quant.h:37-134: s = 2^ceil(log2(max(amax/6,eps)))
    with amax starting at eps; codes of clamp(x/s, +-6); byte = c[2i+1]<<4|c[2i].
    Returns (q uint8 [M, K/2], s float32 [M, K/group])."""
    M, K = x.shape
    xg = x.float().reshape(M, K // group_size, group_size)
    amax = torch.clamp(xg.abs().amax(-1), min=eps)
    s = torch.exp2(torch.ceil(torch.log2(torch.clamp(_div_const(amax, FP4_MAX).abs(),
                                                     min=eps))))
    v = torch.clamp(xg * (1.0 / s).unsqueeze(-1), -FP4_MAX, FP4_MAX)
    c = fp4_code(v).reshape(M, K)
    q = (c[:, 0::2] | (c[:, 1::2] << 4)).to(torch.uint8)
    return q, s


def silu_mul_f32(x: torch.Tensor) -> torch.Tensor:
    """csrc/quantization/fused_kernels/fused_silu_mul_block_quant.cpp:73 and
    fused_silu_mul_mxfp4_quant.cpp:77: r = (g / (1 + exp(-g))) * u in fp32
    with no intermediate rounding; g = x[:, :H], u = x[:, H:]."""
    H = x.shape[-1] // 2
    g = x[:, :H].float()
    u = x[:, H:].float()
    return (g / (1.0 + torch.exp(-g))) * u


_QMAX = {torch.float8_e4m3fn: 448.0, torch.float8_e5m2: 57344.0}


def silu_and_mul_per_block_quant(x: torch.Tensor, group_size: int,
                                 quant_dtype: torch.dtype,
                                 scale_ub: Optional[float] = None,
                                 scale_ue8m0: bool = False):
    """csrc/quantization/fused_kernels/fused_silu_mul_block_quant.cpp:80-121 +
    quant_conversions.h:19-71.  Per group of r = silu_mul_f32(x): amax =
    max|r| (from 0); fp8: s = max(amax/qmax, 1/(qmax*512)), with scale_ub
    s = max(min(s, ub), 1/(qmax*512)), with ue8m0 s = 2^ceil(log2(max(|s|,
    1e-10))); q = cast_rne(clamp(r / s, +-qmax)).  int8: s = max(amax/127,
    FLT_EPSILON) (no ub / ue8m0), q = clamp(rint(r / s), -128, 127).
    Returns (q [T, H] quant_dtype, s float32 [T, H/group_size])."""
    r = silu_mul_f32(x)
    T, H = r.shape
    rg = r.reshape(T, H // group_size, group_size)
    amax = rg.abs().amax(-1)
    if quant_dtype == torch.int8:
        s = torch.clamp(_div_const(amax, 127.0), min=torch.finfo(torch.float32).eps)
        q = torch.clamp(torch.round(rg / s.unsqueeze(-1)), -128, 127)
        return q.reshape(T, H).to(torch.int8), s
    qmax = _QMAX[quant_dtype]
    min_sf = torch.tensor(1.0, dtype=torch.float32) / (qmax * 512.0)
    s = torch.maximum(_div_const(amax, qmax), min_sf)
    if scale_ub is not None:
        s = torch.maximum(torch.clamp(s, max=scale_ub), min_sf)
    if scale_ue8m0:
        s = torch.exp2(torch.ceil(torch.log2(torch.clamp(s.abs(), min=1e-10))))
    q = torch.clamp(rg / s.unsqueeze(-1), -qmax, qmax)
    return q.reshape(T, H).to(quant_dtype), s


def silu_and_mul_mxfp4_quant(x: torch.Tensor, eps: float = 1e-10):
    """csrc/quantization/fused_kernels/fused_silu_mul_mxfp4_quant.cpp:83-115:
    per 32 columns of r = silu_mul_f32(x), amax = max|r| (from 0), s =
    2^ceil(log2(max(|amax/6|, eps))), codes of clamp(r * (1/s), +-6) with the
    strict-midpoint e2m1 rounding of mxfp4_quant.h:17-25, the even column in
    the low nibble.  Returns (q uint8 [T, H/2], s float32 [T, H/32])."""
    r = silu_mul_f32(x)
    T, H = r.shape
    rg = r.reshape(T, H // 32, 32)
    amax = rg.abs().amax(-1)
    s = torch.exp2(torch.ceil(torch.log2(torch.clamp(_div_const(amax, FP4_MAX).abs(), min=eps))))
    v = torch.clamp(rg * (1.0 / s).unsqueeze(-1), -FP4_MAX, FP4_MAX)
    c = fp4_code(v).reshape(T, H)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).to(torch.uint8), s


def _e2m1_rne(v: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even onto the e2m1 grid (OCP MX v1.0 sec. 5.3.3);
    ties go to the code with an even mantissa bit."""
    grid = torch.tensor(E2M1_VALUES, dtype=torch.float32)
    m = v.abs().clamp(max=FP4_MAX)
    d = (m.unsqueeze(-1) - grid).abs()
    best = d.argmin(-1)
    dmin = d.gather(-1, best.unsqueeze(-1)).squeeze(-1)
    # tie: two grid points at the same distance -> pick the even code
    nxt = (best + 1).clamp(max=7)
    tie = (d.gather(-1, nxt.unsqueeze(-1)).squeeze(-1) == dmin) & (nxt != best)
    best = torch.where(tie & (best % 2 == 1), nxt, best)
    return best.int() | ((v < 0).int() << 3)


def to_mxfp4(w: torch.Tensor):
    """MXFP4 weight generator, semantics of to_mxfp(format="mxfp4")
    (tests/ops/mx_utils.py:277-353): RCEIL e8m0 exponent per 32 along the last
    dim, data cast to bf16 then RNE e2m1, low nibble = even element.
    Returns (packed uint8 [..., K/2], e8m0 uint8 [..., K/32])."""
    shp = w.shape
    K = shp[-1]
    x = w.float().reshape(-1, K // 32, 32)
    amax = x.abs().amax(-1, keepdim=True)
    desc = _div_const(amax, FP4_MAX)
    e = (torch.clamp(torch.ceil(torch.log2(desc)), min=-127, max=127) + 127)
    e = torch.where(torch.isnan(desc), torch.full_like(e, 255), e)
    e_u8 = e.to(torch.uint8)
    dsc = torch.where(e == 0, torch.ones_like(e), torch.exp2(127 - e))
    v = torch.clamp(x * dsc, -FP4_MAX, FP4_MAX).to(torch.bfloat16).float()
    c = _e2m1_rne(v).reshape(-1, K)
    q = (c[:, 0::2] | (c[:, 1::2] << 4)).to(torch.uint8)
    return q.reshape(shp[:-1] + (K // 2,)), e_u8.reshape(shp[:-1] + (K // 32,))


def dequant_mxfp4(q: torch.Tensor, e8m0: torch.Tensor) -> torch.Tensor:
    """LUT dequant of tests/fused_moe/test_fused_moe.py:79-116 (e8m0 via
    (e<<7) as bf16, so e=0 -> 0) == 2^(e-127) for 0<e<255."""
    lut = torch.tensor(E2M1_VALUES + [-v for v in E2M1_VALUES],
                       dtype=torch.float32, device=q.device)
    qi = q.to(torch.int64)
    lo = lut[qi & 0xF]
    hi = lut[qi >> 4]
    vals = torch.stack([lo, hi], dim=-1).reshape(q.shape[:-1] +
                                                 (q.shape[-1] * 2,))
    sc = (e8m0.to(torch.int32) << 7).to(torch.int16).view(
        torch.bfloat16).float()
    sc = sc.repeat_interleave(32, dim=-1)
    return vals * sc


def e8m0_value(e8m0: torch.Tensor) -> torch.Tensor:
    """2^(e-127) of e8m0 bytes as the reference's _as_e8m0(s).to(float32)
    (vllm_xpu_kernels/moe_utils.py:168-174): 0 -> 2^-127, 255 -> NaN."""
    e = e8m0.view(torch.uint8).to(torch.int32)
    v = torch.exp2((e - 127).double()).float()
    return torch.where(e == 255, torch.full_like(v, float("nan")), v)


def dequant_mxfp8(q: torch.Tensor, e8m0: torch.Tensor) -> torch.Tensor:
    """e4m3 values [..., K] times their e8m0 scale per 32 along K
    (vllm_xpu_kernels/moe_utils.py:76-82, dequant_mxfp8 / dequant_mxfp8_wei
    with the weight transposed to [N, K])."""
    return q.float() * e8m0_value(e8m0).repeat_interleave(32, dim=-1)


def quant_mxfp8_act(x: torch.Tensor):
    """_quant_mxfp8_act_xpu (vllm_xpu_kernels/moe_utils.py:90-104):
    per_token_group_fp8_quant with group 32, eps 1e-10 and ue8m0 scales;
    returns (e4m3 codes [M, K], e8m0 bytes [M, K/32])."""
    q, sc = per_token_group_fp8_quant(x, 32, scale_ue8m0=True)
    e = torch.log2(sc).round().to(torch.int32) + 127
    return q, e.to(torch.uint8)


def quant_mxfp4_act(x: torch.Tensor):
    """_quant_mxfp4_act_xpu (vllm_xpu_kernels/moe_utils.py:106-120):
    per_token_group_quant_mxfp4 with group 32, eps 1e-10; returns (packed
    e2m1 [M, K/2], e8m0 bytes [M, K/32])."""
    q, sc = per_token_group_quant_mxfp4(x, 32)
    e = torch.log2(sc).round().to(torch.int32) + 127
    return q, e.to(torch.uint8)


def fp8_block_quant_weight(w: torch.Tensor, eps: float = 1e-6):
    """128x128 block quant of the last two dims (tests/ops/fp8_quant_op.py:16-78):
    s = clamp(amax/448, min=eps), q = e4m3(w / s).
    Returns (q float8_e4m3fn, s float32 [..., N/128, K/128])."""
    *lead, N, K = w.shape
    x = w.float().reshape(*lead, N // 128, 128, K // 128, 128)
    amax = x.abs().amax(dim=(-3, -1))
    s = torch.clamp(_div_const(amax, FP8_MAX), min=eps)
    q = (x / s.unsqueeze(-2).unsqueeze(-1)).reshape(*lead, N, K)
    return q.to(torch.float8_e4m3fn), s


def dequant_fp8_block_weight(q: torch.Tensor, s: torch.Tensor):
    """[N,K] e4m3 weights with [N/128, K/128] scales -> fp32 (kernel convention
    of csrc/xpu/grouped_gemm/xe_2/grouped_gemm_xe2_interface.hpp:362-376)."""
    N, K = q.shape
    x = q.float().reshape(N // 128, 128, K // 128, 128)
    return (x * s.reshape(N // 128, 1, K // 128, 1)).reshape(N, K)


# ----------------------------------------------------------------------------
# Grouped GEMM and the fused layer
# ----------------------------------------------------------------------------
def dequant_int4(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """[N, K/2] two's-complement int4 (even K value in the low nibble) with
    16-bit group scales [N, K/group] -> [N, K] fp32 of T(v * scale), T the
    scales' type (the reference kernel's 16-bit dequantisation,
    csrc/xpu/grouped_gemm/xe_2/gemm_xe2.hpp:455-470; its test's
    dequantize_uint4, tests/fused_moe/test_grouped_gemm.py:310-323, is the same
    value through (u4 - 8) * scale)."""
    b = q.view(torch.uint8).to(torch.int32)
    lo = ((b & 0xF) ^ 8) - 8
    hi = ((b >> 4) ^ 8) - 8
    v = torch.stack([lo, hi], -1).reshape(q.shape[0], -1).float()
    g = v.shape[1] // s.shape[1]
    return (v * s.float().repeat_interleave(g, dim=1)).to(s.dtype).float()


def dequant_weight(recipe: str, w_e: torch.Tensor, s_e) -> torch.Tensor:
    """[N, K] fp32 weights of one expert, per recipe
    (vllm_xpu_kernels/moe_utils.py:189-202)."""
    if recipe == "bf16":
        return w_e.float()
    if recipe == "fp8":
        # per-expert scale (moe_utils.py:212-213; gemm_xe2.hpp:192-198 applies
        # it to the accumulators, the same product up to fp32 rounding)
        return w_e.float() * float(s_e)
    if recipe == "int4":
        return dequant_int4(w_e, s_e)
    if recipe == "fp8block":
        return dequant_fp8_block_weight(w_e, s_e)
    if recipe == "mxfp4":
        return dequant_mxfp4(w_e, s_e)
    if recipe == "mxfp8":
        return dequant_mxfp8(w_e, s_e)
    raise ValueError(recipe)


def qdq_act(recipe: str, x: torch.Tensor) -> torch.Tensor:
    """Activation quant-dequant round trip of the recipe
    (vllm_xpu_kernels/moe_utils.py:176-187): fp8block -> 1x128 e4m3; mxfp8
    -> e4m3 with ue8m0 scales per 32; "mxfp4a4" (mxfp4 weights with
    pre-quantised inputs, whose intermediate activation the reference
    quantises with quant_act_xpu) -> e2m1 per 32; bf16 and mxfp4 (w4a16
    kernel semantics) -> unchanged."""
    if recipe == "fp8block":
        q, s = per_token_group_fp8_quant(x, 128)
        return dequant_fp8_groups(q, s, 128)
    if recipe == "mxfp8":
        return dequant_mxfp8(*quant_mxfp8_act(x))
    if recipe == "mxfp4a4":
        return dequant_mxfp4(*quant_mxfp4_act(x))
    return x.float()


def grouped_gemm(recipe: str, a: torch.Tensor, w: torch.Tensor, w_scale,
                 bias, rows_per_expert, out_dtype=torch.bfloat16):
    """cutlass_grouped_gemm_interface semantics (csrc/xpu/grouped_gemm/
    grouped_gemm_interface.cpp:12-60; per-expert loop of
    vllm_xpu_kernels/moe_utils.py:319-363): rows of expert e are contiguous;
    D = T(A_qdq @ deq(W_e)^T + b_e) with fp32 accumulation.  ``w`` is [E,N,K]
    (nk) for every recipe (mxfp4 packed along K)."""
    M = a.shape[0]
    E = w.shape[0]
    N = w.shape[1]
    out = torch.zeros(M, N, dtype=out_dtype, device=a.device)
    off = 0
    for e in range(E):
        n = int(rows_per_expert[e])
        if n == 0:
            continue
        x = qdq_act(recipe, a[off:off + n])
        we = dequant_weight(recipe, w[e], None if w_scale is None else w_scale[e])
        y = x @ we.t()
        if bias is not None:
            y = y + bias[e].float()
        out[off:off + n] = y.to(out_dtype)
        off += n
    return out


def fused_moe(recipe: str, hidden: torch.Tensor, w13, w13_scale, w13_bias,
              w2, w2_scale, w2_bias, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, activation: str = "silu",
              expert_map: Optional[torch.Tensor] = None,
              gemm1_clamp_limit: Optional[float] = None,
              experts=None, a1q_scale: Optional[torch.Tensor] = None,
              compute_dtype: Optional[torch.dtype] = None):
    """XpuFusedMoe.apply semantics (vllm_xpu_kernels/fused_moe_interface.py:
    319-419, reference path moe_utils.py:236-403, rounding points of
    SURVEY Appendix A):

      G1  = T(qdq(x) @ deq(W13_e)^T + b13_e)            per slot
      act = silu_and_mul(G1) | swigluoai_and_mul(G1)
      G2  = T(qdq(act) @ deq(W2_e)^T + b2_e)
      y   = T(sum_j w[t,j] * float(G2[t,j]))            fixed j order

    Weights are [E, N, K] (nk); for mxfp4 packed uint8 [E, N, K/2] with e8m0
    [E, N, K/32].  The expert loop dequantises one expert at a time.
    ``experts`` optionally restricts the computation to a subset of expert ids
    (the CPU-baseline sample); slots of other experts contribute zero.
    ``a1q_scale``: ``hidden`` is already quantised and dequantised as given,
    computed in bf16 (fused_moe_interface.py:326-360, moe_utils.py:189-199,
    285, 338-347): fp8block e4m3 with [T, H/128] f32 scales; mxfp8 e4m3
    with e8m0 [T, H/32]; mxfp4 packed e2m1 [T, H/2] with e8m0 [T, H/32],
    whose intermediate activation is then quantised to mxfp4 too.
    ``compute_dtype`` overrides that bf16 for pre-quantised input: the
    reference's kernel path rounds both GEMM outputs to the caller's output
    type (fused_moe_interface.py:368-371, 398-401), its torch path to bf16
    (moe_utils.py:285); the two differ only for an fp16 output.
    """
    T = hidden.shape[0]
    k = topk_ids.shape[1]
    if a1q_scale is None:
        dt = hidden.dtype
    else:
        dt = torch.bfloat16 if compute_dtype is None else compute_dtype
    ids = topk_ids.to(torch.int64)
    if expert_map is not None:
        ids = expert_map.to(torch.int64)[ids]
    E = w13.shape[0]
    I2 = w13.shape[1]
    flat = ids.reshape(-1)
    todo = range(E) if experts is None else experts
    act_recipe = recipe
    if a1q_scale is not None:
        if recipe == "fp8block":
            xq_all = dequant_fp8_groups(hidden, a1q_scale.float(), 128)
        elif recipe == "mxfp8":
            xq_all = dequant_mxfp8(hidden, a1q_scale)
        elif recipe == "mxfp4":
            xq_all = dequant_mxfp4(hidden.view(torch.uint8), a1q_scale.view(torch.uint8))
            act_recipe = "mxfp4a4"
        else:
            raise ValueError(f"a1q_scale with recipe {recipe}")
    else:
        xq_all = qdq_act(recipe, hidden)
    H = xq_all.shape[1]
    g2 = torch.zeros(T * k, H, dtype=dt, device=xq_all.device)
    for e in todo:
        slots = (flat == e).nonzero().flatten()
        if slots.numel() == 0:
            continue
        toks = slots // k
        x = xq_all[toks]
        w1 = dequant_weight(recipe, w13[e],
                            None if w13_scale is None else w13_scale[e])
        g1 = x @ w1.t()
        del w1
        if w13_bias is not None:
            g1 = g1 + w13_bias[e].float()
        g1 = g1.to(dt)
        if gemm1_clamp_limit is not None and gemm1_clamp_limit > 0:
            I = I2 // 2
            g1 = g1.clone()
            g1[:, :I] = g1[:, :I].clamp(max=gemm1_clamp_limit)
            g1[:, I:] = g1[:, I:].clamp(min=-gemm1_clamp_limit,
                                        max=gemm1_clamp_limit)
        if activation == "silu":
            act = silu_and_mul(g1)
        elif activation == "swigluoai":
            act = swigluoai_and_mul(g1)
        elif activation == "gelu":
            act = gelu_and_mul(g1)
        elif activation == "gelu_tanh":
            act = gelu_and_mul(g1, "tanh")
        elif activation == "swiglustep":
            act = swiglustep_and_mul(g1)
        elif activation == "relu2_no_mul":
            act = relu2_no_mul(g1)       # all 2I columns; w2 has K = 2I
        else:
            raise ValueError(activation)
        aq = qdq_act(act_recipe, act)
        wd = dequant_weight(recipe, w2[e],
                            None if w2_scale is None else w2_scale[e])
        y = aq @ wd.t()
        del wd
        if w2_bias is not None:
            y = y + w2_bias[e].float()
        g2[slots] = y.to(dt)
    perm = torch.arange(T * k, dtype=torch.int32, device=ids.device).reshape(T, k)
    perm = torch.where(ids >= 0, perm, torch.full_like(perm, -1))
    return moe_gather(g2, topk_weights.float(), perm)


def active_experts(topk_ids: torch.Tensor, num_experts: int) -> int:
    """|A| of the roofline: experts with at least one routed slot."""
    f = topk_ids.reshape(-1).to(torch.int64)
    f = f[(f >= 0) & (f < num_experts)]
    return int(torch.unique(f).numel())
