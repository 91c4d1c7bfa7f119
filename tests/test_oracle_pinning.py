"""Pins the CPU oracle (oracle/moe_oracle.py) against the reference's
known-answer vectors, closed forms and independent brute force.  CPU only."""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O


# ------------------------------------------------------------------ routing
def test_topk_softmax_ties_go_to_lower_index():
    g = torch.tensor([[1.0, 3.0, 3.0, 0.0, 3.0]])
    w, ids, tei = O.topk_softmax(g, 3, renormalize=False)
    assert ids.tolist() == [[1, 2, 4]]
    assert tei.tolist() == [[0, 1, 2]]


def test_topk_softmax_matches_logit_order_and_closed_form():
    torch.manual_seed(0)
    T, E, k = 33, 192, 8
    g = torch.randn(T, E)
    w, ids, tei = O.topk_softmax(g, k, renormalize=True)
    # softmax is monotone: ids are the stable top-k of the logits themselves
    ref_ids = torch.sort(g, dim=-1, descending=True, stable=True).indices[:, :k]
    assert torch.equal(ids.long(), ref_ids)
    for t in range(T):
        m = max(g[t].tolist())
        ex = [math.exp(float(g[t, i]) - m) for i in ids[t].tolist()]
        s = sum(ex)
        assert np.allclose(w[t].numpy(), [x / s for x in ex], rtol=1e-6)
    assert torch.equal(tei, (torch.arange(k) * T).unsqueeze(0) +
                       torch.arange(T).unsqueeze(1))


def test_topk_softmax_bias_selects_but_does_not_weight():
    g = torch.tensor([[0.0, 0.0, 0.0, 0.0]])
    bias = torch.tensor([0.0, 1.0, 0.0, 2.0])
    w, ids, _ = O.topk_softmax(g, 2, renormalize=False, bias=bias)
    assert ids.tolist() == [[3, 1]]
    assert np.allclose(w.numpy(), [[0.25, 0.25]])


def test_topk_sigmoid_rounds_to_input_dtype_and_scales():
    g = torch.tensor([[0.3, -1.2, 2.0, 0.7]], dtype=torch.bfloat16)
    w, ids, _ = O.topk_sigmoid(g, 2, renormalize=True, routed_scaling_factor=2.5)
    assert ids.tolist() == [[2, 3]]
    sig = [float(torch.tensor(1 / (1 + math.exp(-float(x))), dtype=torch.bfloat16))
           for x in g[0].float().tolist()]
    s = sig[2] + sig[3]
    assert np.allclose(w.numpy(), [[sig[2] * 2.5 / s, sig[3] * 2.5 / s]], rtol=1e-6)


def _grouped_brute(s, sb, n_group, topk_group, k):
    E = s.shape[0]
    epg = E // n_group
    gs = []
    for g in range(n_group):
        v = sorted(sb[g * epg:(g + 1) * epg].tolist(), reverse=True)
        gs.append(v[0] + v[1])
    best = None
    # brute force: the kept set is the lexicographically best subset by
    # (sorted scores desc, then lowest group ids)
    for combo in itertools.combinations(range(n_group), topk_group):
        key = (sorted([gs[c] for c in combo], reverse=True),
               [-c for c in combo])
        if best is None or key > best[0]:
            best = (key, combo)
    kept = best[1]
    cand = [(float(sb[e]), -e) for g in kept for e in range(g * epg, (g + 1) * epg)]
    cand.sort(reverse=True)
    return [-c[1] for c in cand[:k]]


def test_topk_softplus_sqrt_vs_reference_test_oracle():
    """Against the reference test's torch oracle
    (tests/test_topk_softplus_sqrt.py:19-47: F.softplus(x).sqrt(), topk of the
    biased scores, weights the unbiased scores): same ids, weights within an
    ulp-level tolerance (the kernel reports (s + b) - b, the test oracle s);
    closed forms of the softplus branches; hash routing."""
    F = torch.nn.functional
    g = torch.Generator().manual_seed(14)
    T, E, k = 33, 256, 8
    x = torch.randn(T, E, generator=g)
    b = torch.randn(E, generator=g) * 0.1
    w, ids = O.topk_softplus_sqrt(x, k, True, 1.5, b)
    s = F.softplus(x).sqrt()
    rid = torch.topk(s + b, k, dim=-1, sorted=True)[1]
    rw = s.gather(1, rid)
    rw = rw / rw.sum(-1, keepdim=True) * 1.5
    assert torch.equal(ids, rid)
    torch.testing.assert_close(w, rw, rtol=1e-5, atol=1e-6)
    one = torch.tensor([[25.0, 0.0, -30.0]])
    w1, i1 = O.topk_softplus_sqrt(one, 3, False, 1.0)
    assert i1.tolist() == [[0, 1, 2]]
    assert w1[0, 0].item() == 5.0 and w1[0, 2].item() == 0.0     # log(1 + e^-30) = 0 in fp32
    assert w1[0, 1].item() == pytest.approx(math.sqrt(math.log(2.0)), rel=1e-6)
    ids_tab = torch.randint(0, E, (50, k), generator=g)
    tok = torch.randint(0, 50, (T,), generator=g)
    wh, ih = O.topk_softplus_sqrt(x, k, True, 2.5, None, tok, ids_tab)
    assert torch.equal(ih, ids_tab[tok])
    rh = s.gather(1, ids_tab[tok])
    torch.testing.assert_close(wh, rh / rh.sum(-1, keepdim=True) * 2.5, rtol=1e-5, atol=1e-6)


def test_grouped_topk_brute_force():
    torch.manual_seed(1)
    T, E, n_group, topk_group, k = 16, 64, 8, 4, 6
    logits = torch.randn(T, E)
    s = logits.sigmoid()
    sb = s + 0.1 * torch.randn(E)
    v, ids = O.grouped_topk(s, sb, n_group, topk_group, k, True, 2.5)
    for t in range(T):
        exp_ids = _grouped_brute(s[t], sb[t], n_group, topk_group, k)
        assert ids[t].tolist() == exp_ids
        ws = s[t, exp_ids].double()
        assert np.allclose(v[t].double().numpy(),
                           (ws / (1e-20 + ws.sum()) * 2.5).numpy(), rtol=1e-6)


def test_grouped_topk_group_ties_lower_group_wins():
    # 4 groups of 2; groups 1 and 2 tie for the second slot
    sb = torch.tensor([[0.9, 0.8, 0.5, 0.5, 0.5, 0.5, 0.1, 0.1]])
    v, ids = O.grouped_topk(sb.clone(), sb, 4, 2, 2, False, 1.0)
    assert ids.tolist() == [[0, 1]]
    v, ids = O.grouped_topk(sb.clone(), sb, 4, 2, 4, False, 1.0)
    assert ids.tolist() == [[0, 1, 2, 3]]


# ---------------------------------------------------------------- alignment
def test_moe_align_docstring_kat():
    """tests/ops/moe_align_block_size_ops.py:56-69 (self-consistent for
    num_experts = 5: experts 1..4 used)."""
    ids = torch.tensor([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]])
    mx, nb = O.align_buffer_sizes(12, 5, 4)
    srt, eids, ntp = O.moe_align_block_size(ids, 5, 4, mx, nb)
    assert srt[:16].tolist() == [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]
    assert (srt[16:] == 12).all()
    assert eids.tolist()[:4] == [1, 2, 3, 4] and (eids[4:] == 0).all()
    assert ntp.tolist() == [16]


def _golden_align(topk_ids, block_size, num_experts, mx, nb, expert_map=None):
    """Restatement of the reference golden tests/test_moe_align_block_size.py:97-183."""
    flat = topk_ids.flatten()
    sorted_e, order = torch.sort(flat, stable=True)
    tok = torch.arange(flat.numel(), dtype=torch.int32)[order]
    out = torch.full((mx,), flat.numel(), dtype=torch.int32)
    eids = torch.zeros(nb, dtype=torch.int32)
    pos = blk = 0
    for e in range(num_experts):
        if expert_map is not None and expert_map[e] == -1:
            continue
        t = tok[sorted_e == e]
        if t.numel() == 0:
            continue
        padded = (t.numel() + block_size - 1) // block_size * block_size
        out[pos:pos + t.numel()] = t
        eids[blk:blk + padded // block_size] = (e if expert_map is None
                                                else int(expert_map[e]))
        pos += padded
        blk += padded // block_size
    return out, eids, pos


@pytest.mark.parametrize("m,topk,E,bs", [(1, 1, 32, 32), (3, 2, 160, 128),
                                         (256, 16, 32, 32), (257, 8, 257, 128),
                                         (64, 4, 8, 16)])
def test_moe_align_vs_reference_golden(m, topk, E, bs):
    g = torch.Generator().manual_seed(m * 1000 + E)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(m)])
    mx, nb = O.align_buffer_sizes(ids.numel(), E, bs)
    srt, eids, ntp = O.moe_align_block_size(ids, E, bs, mx, nb)
    g_srt, g_eids, g_ntp = _golden_align(ids, bs, E, mx, nb)
    assert ntp[0] == g_ntp
    assert torch.equal(torch.from_numpy(eids), g_eids)
    assert torch.equal(torch.from_numpy(srt), g_srt)


def test_moe_align_expert_map_vs_golden():
    g = torch.Generator().manual_seed(7)
    E, m, k, bs = 8, 32, 4, 64
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(m)])
    em = torch.full((E,), -1, dtype=torch.int32)
    for i, e in enumerate(range(0, E, 2)):
        em[e] = i
    mx, nb = O.align_buffer_sizes(ids.numel(), E, bs)
    srt, eids, ntp = O.moe_align_block_size(ids, E, bs, mx, nb, expert_map=em)
    g_srt, g_eids, g_ntp = _golden_align(ids, bs, E, mx, nb, expert_map=em)
    assert ntp[0] == g_ntp
    assert torch.equal(torch.from_numpy(eids), g_eids)
    assert torch.equal(torch.from_numpy(srt), g_srt)


def _lora_inputs(T, k, E, max_loras, seed, base_tokens=0):
    """Reference tests/test_moe_lora_align_sum.py:29-40 and :136-157: k
    distinct experts per token, adapters drawn from [0, max_loras) (the last
    `base_tokens` tokens are base-model tokens, adapter -1); buffer sizes as
    in its :55-60."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    tok = torch.randint(0, max_loras, (T,), generator=g, dtype=torch.int32)
    if base_tokens:
        tok[T - base_tokens:] = -1
    return ids, tok


def _lora_run(ids, tok, E, bs, max_loras, lora_ids, enabled, fill=(-7, -2, -13)):
    mx = (ids.numel() + E * (bs - 1) + bs - 1) // bs * bs
    if ids.numel() < E:
        mx = ids.numel() * bs
    nb = (mx + bs - 1) // bs
    srt = np.full(max_loras * mx, fill[0], np.int32)
    eid = np.full(max_loras * nb, fill[1], np.int32)
    ntp = np.full(max_loras, fill[2], np.int32)
    O.moe_lora_align_block_size(ids, tok, E, bs, max_loras, mx, nb, srt, eid, ntp,
                                enabled, lora_ids)
    return srt, eid, ntp, mx, nb


@pytest.mark.parametrize("T,E,max_loras", [(100, 64, 2), (200, 128, 32), (37, 64, 3)])
def test_moe_lora_align_vs_golden(T, E, max_loras):
    """Every adapter's slice equals the sort-based golden of the plain
    alignment over that adapter's tokens, and passes the reference's own
    membership check (tests/test_moe_lora_align_sum.py:98-108)."""
    bs, k = 16, 6
    ids, tok = _lora_inputs(T, k, E, max_loras, seed=T + max_loras)
    lora_ids = torch.arange(max_loras + 2, dtype=torch.int32)
    enabled = torch.ones(max_loras + 1, dtype=torch.int32)
    srt, eid, ntp, mx, nb = _lora_run(ids, tok, E, bs, max_loras, lora_ids, enabled)
    flat = ids.flatten()
    for lid in range(max_loras):
        masked = torch.where(tok.repeat_interleave(k) == lid, flat.long(), E).reshape(ids.shape)
        g_srt, g_eids, g_ntp = _golden_align(masked, bs, E, mx, nb)
        g_eids[g_ntp // bs:] = -1
        assert ntp[lid] == g_ntp
        assert np.array_equal(srt[lid * mx:(lid + 1) * mx], g_srt.numpy())
        assert np.array_equal(eid[lid * nb:(lid + 1) * nb], g_eids.numpy())
        blocks = srt[lid * mx:(lid + 1) * mx].reshape(-1, bs)
        for b in range(blocks.shape[0]):
            idx = blocks[b][blocks[b] != ids.numel()]
            if idx.size:
                assert (flat.numpy()[idx] == eid[lid * nb + b]).all()


def test_moe_lora_align_sentinels():
    """tests/test_moe_lora_align_sum.py:225-331: a mixed batch with -1 first in
    lora_ids still sorts adapter 0; a disabled adapter and an out-of-range id
    leave their rows untouched."""
    E, bs, k = 64, 16, 6
    ids, tok = _lora_inputs(16, k, E, 1, seed=1, base_tokens=8)
    tok[:8] = 0
    lora_ids = torch.tensor([-1, 0], dtype=torch.int32)
    on = torch.ones(2, dtype=torch.int32)
    srt, eid, ntp, mx, nb = _lora_run(ids, tok, E, bs, 1, lora_ids, on)
    assert 0 < ntp[0] <= mx and ntp[0] % bs == 0
    assert (srt != -7).all() and (eid != -2).all()
    # 8 adapter tokens x 6 slots, all in distinct-or-shared experts; only
    # slots of tokens 0..7 appear
    got = srt[srt != ids.numel()]
    assert sorted(got.tolist()) == list(range(48))
    off = torch.tensor([0, 1], dtype=torch.int32)
    srt, eid, ntp, mx, nb = _lora_run(ids, torch.zeros(16, dtype=torch.int32), E, bs, 1,
                                      torch.tensor([0, -1], dtype=torch.int32), off * 0)
    assert ntp[0] == -13 and (eid == -2).all() and (srt == -7).all()
    srt, eid, ntp, mx, nb = _lora_run(ids, torch.zeros(16, dtype=torch.int32), E, bs, 1,
                                      torch.tensor([0, 5], dtype=torch.int32), on)
    assert ntp[0] != -13 and sorted(srt[srt != ids.numel()].tolist()) == list(range(96))


# ------------------------------------------------------- fused_moe_prologue
def _ref_prologue_golden(x, scales, ids, k):
    """Restatement of the reference golden tests/fused_moe/test_moe_prologue.py:
    52-97 (argsort of the flat expert ids; rows of token idx // k)."""
    flat = ids.reshape(-1)
    idxs = np.argsort(flat, kind="stable")
    counts = np.bincount(flat)
    tok = idxs // k
    offsets = counts.cumsum()
    return offsets, x[tok], None if scales is None else scales[tok]


@pytest.mark.parametrize("T,k,E", [(1, 1, 16), (4, 2, 16), (16, 2, 16), (300, 2, 16), (64, 8, 64)])
@pytest.mark.parametrize("row_bytes,srow_bytes", [(512, 0), (256, 8), (128, 16)])
def test_prologue_vs_reference_golden(T, k, E, row_bytes, srow_bytes):
    g = np.random.default_rng(T * 7 + k)
    x = g.integers(0, 256, (T, row_bytes), dtype=np.uint8)
    sc = g.integers(0, 256, (T, srow_bytes), dtype=np.uint8) if srow_bytes else None
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    fs = g.standard_normal((T, k)).astype(np.float32)
    out = O.fused_moe_prologue(x, sc, ids, fs, E)
    offs, gx, gs = _ref_prologue_golden(x, sc, ids, k)
    # the reference test compares expert_first_token_offset[1:1 + n]
    assert np.array_equal(out["expert_first_token_offset"][1:1 + offs.size], offs)
    assert np.array_equal(out["overlapped_gemm1_gemm2_inputs"], gx)
    if sc is not None:
        assert np.array_equal(out["permuted_act_scales"], gs)
    p2u = out["permuted_row_to_unpermuted_row"]
    # maps are mutually inverse; experts and token scales follow the source slot
    assert all(out["unpermuted_row_to_permuted_row"][int(r)] == p for p, r in enumerate(p2u))
    assert np.array_equal(out["permuted_token_selected_experts"], ids[p2u % T, p2u // T])
    assert np.array_equal(out["permuted_token_final_scales"], fs[p2u % T, p2u // T])


def test_prologue_known_answer_ep_and_duplicates():
    """Hand-worked: E = 2 on rank 1 (experts 2, 3); token 1 lists expert 3
    twice and is routed once (first position); id 0 is another rank's."""
    ids = np.array([[2, 3], [3, 3], [0, 2]], dtype=np.int64)
    fs = np.arange(6, dtype=np.float32).reshape(3, 2)
    x = np.arange(3, dtype=np.uint8).reshape(3, 1)
    out = O.fused_moe_prologue(x, None, ids, fs, 2, ep_rank=1)
    assert out["permuted_row_to_unpermuted_row"].tolist() == [0, 5, 3, 1]
    assert out["permuted_token_selected_experts"].tolist() == [0, 0, 1, 1]
    assert out["expert_first_token_offset"].tolist() == [0, 2, 4]
    assert out["permuted_token_final_scales"].tolist() == [0.0, 5.0, 1.0, 2.0]
    assert out["overlapped_gemm1_gemm2_inputs"].ravel().tolist() == [0, 2, 0, 1]
    assert out["unpermuted_row_to_permuted_row"] == {0: 0, 5: 1, 3: 2, 1: 3}


def _ref_test_ws_map(T, k, hidden, elem_bytes, block_k, scale_bytes, E):
    """The layout as the reference test builds it
    (tests/fused_moe/test_moe_prologue.py:151-204)."""
    N = T * k
    tpb = O.prologue_tokens_per_block(T, E)
    nblk = -(-T // tpb)
    sizes = [N * 4, N * 4, k * T * 4, E * nblk * 4, E * nblk * 4, E * T * 4, (E + 1) * 8, N * 4,
             N * hidden * elem_bytes, (N * hidden) // block_k * scale_bytes if scale_bytes else 0]
    ws, at = {}, 0
    for name, sz in zip(O.PROLOGUE_SECTIONS, sizes):
        if sz % 256:
            sz += 256 - sz % 256
        ws[name] = (sz, at)
        at += sz
    return at, ws


@pytest.mark.parametrize("T,k,hidden,eb,bk,sb,E", [
    (1, 1, 128, 2, 1, 0, 2), (4, 2, 8192, 2, 1, 0, 16), (16, 2, 8192, 1, 128, 4, 16),
    (8192, 2, 8192, 1, 32, 1, 16), (8192, 1, 4096, 1, 16, 1, 16), (3000, 8, 7168, 1, 128, 4, 256)])
def test_prologue_layout_matches_reference_test(T, k, hidden, eb, bk, sb, E):
    assert O.prologue_layout(T, k, hidden, eb, bk, sb, E) == _ref_test_ws_map(T, k, hidden, eb, bk, sb, E)
    # tokens per block: the smallest power of two in [32, 1024] whose block
    # count times E fits in one block
    tpb = O.prologue_tokens_per_block(T, E)
    assert tpb == 1024 or (-(-T // tpb) * E <= tpb and (tpb == 32 or -(-T // (tpb // 2)) * E > tpb // 2))


def test_remap_unpermute_invariant():
    torch.manual_seed(3)
    T, H, k, E = 40, 16, 4, 8
    x = torch.randn(T, H)
    ids = torch.stack([torch.randperm(E)[:k] for _ in range(T)])
    out, _, rows, perm = O.remap_hidden_states(x, ids, E)
    assert rows.tolist() == torch.bincount(ids.flatten(), minlength=E).tolist()
    for t in range(T):
        for j in range(k):
            assert torch.equal(out[perm[t, j]], x[t])
    # rows of expert e are contiguous and in [prefix[e], prefix[e+1])
    pre = torch.cat([torch.zeros(1, dtype=torch.long), rows.long().cumsum(0)])
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            assert pre[e] <= perm[t, j] < pre[e + 1]


def test_init_expert_map_closed_form():
    m = O.init_expert_map(4, 1, 3)
    assert m.tolist() == [-1, -1, -1, -1, 0, 1, 2, 3, -1, -1, -1, -1]


# ---------------------------------------------------------------- reductions
def test_moe_sum_and_gather_vs_float64():
    torch.manual_seed(4)
    T, k, H = 7, 3, 33
    x = torch.randn(T, k, H)
    ids = torch.randint(0, 6, (T, k))
    ids[:, -1] = -1
    em = torch.tensor([0, 1, 2, -1, -1, 3], dtype=torch.int32)
    y = O.moe_sum(x, ids, em)
    mask = (ids >= 0) & (em[ids.clamp(min=0)] >= 0)
    ref = (x.double() * mask.unsqueeze(-1)).sum(1)
    assert torch.allclose(y.double(), ref, atol=1e-5)
    w = torch.rand(T, k)
    perm = torch.randperm(T * k).reshape(T, k).int()
    perm[0, 1] = -1
    g = torch.randn(T * k, H)
    y = O.moe_gather(g, w, perm)
    ref = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            if perm[t, j] >= 0:
                ref[t] += float(w[t, j]) * g[perm[t, j]].double()
    assert torch.allclose(y.double(), ref, atol=1e-5)


# --------------------------------------------------------------- activations
def test_silu_and_mul_closed_form():
    x = torch.tensor([[0.0, 1.0, -2.0, 3.0, 5.0, 7.0]])
    y = O.silu_and_mul(x)
    silu = torch.nn.functional.silu(torch.tensor([0.0, 1.0, -2.0]))
    assert torch.allclose(y, silu * torch.tensor([3.0, 5.0, 7.0]), rtol=1e-6)
    assert y[0, 0] == 0.0


def test_swigluoai_special_points():
    # gate clamped at +7 from above only, up clamped to [-7, 7]
    x = torch.tensor([[10.0, 10.0, -3.0, -10.0, 0.0, 2.0]])
    y = O.swigluoai_and_mul(x)
    sig = lambda v: 1 / (1 + math.exp(-v))
    exp = [(7 + 1) * 7 * sig(7 * 1.702), (-7 + 1) * -3 * sig(-3 * 1.702), 0.0]
    assert np.allclose(y[0].numpy(), exp, rtol=1e-6)


# -------------------------------------------------------------- quantisation
def test_fp8_group_quant_all_finite_e4m3_round_trip():
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)],
                         dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    # groups of 127 codes + one 448 so every group has amax 448 -> scale 1
    row = torch.cat([vals[:127], torch.tensor([448.0]), vals[127:],
                     torch.tensor([448.0])]).unsqueeze(0)
    q, s = O.per_token_group_fp8_quant(row, 128)
    assert torch.equal(s, torch.ones(1, 2))
    assert torch.equal(q.view(torch.uint8)[0, :127], codes[:127])
    assert torch.equal(q.view(torch.uint8)[0, 128:255], codes[127:])


def test_fp8_group_quant_scale_closed_form():
    x = torch.zeros(2, 128)
    x[0, 5] = 3.0
    q, s = O.per_token_group_fp8_quant(x, 128)
    assert s[0, 0].item() == pytest.approx(3.0 / 448.0, rel=1e-7)
    assert s[1, 0].item() == pytest.approx(1.0 / (448.0 * 512.0), rel=1e-7)
    assert float(q[0, 5].float()) == 448.0
    q, s = O.per_token_group_fp8_quant(x, 128, scale_ue8m0=True)
    assert s[0, 0].item() == 2.0 ** math.ceil(math.log2(3.0 / 448.0))


# ----------------------------------------------- gelu / swiglustep / relu2
def test_gelu_forms_match_torch_and_identities():
    """The erf and tanh GELU forms agree with torch's own GELU (within 2e-6:
    1 + erf(x/sqrt 2) cancels for negative x, in the reference kernel's form
    as in this one);
    the erf form satisfies gelu(x) - gelu(-x) = x (its odd part) and
    gelu(0) = 0; gelu_and_mul rounds gelu(g) to the element type before the
    multiply."""
    F = torch.nn.functional
    x = torch.linspace(-8, 8, 4001)
    torch.testing.assert_close(O.gelu_erf_f32(x), F.gelu(x), rtol=1e-6, atol=2e-6)
    torch.testing.assert_close(O.gelu_tanh_f32(x), F.gelu(x, approximate="tanh"),
                               rtol=1e-6, atol=2e-6)
    torch.testing.assert_close(O.gelu_erf_f32(x) - O.gelu_erf_f32(-x), x, rtol=1e-6, atol=1e-6)
    assert O.gelu_erf_f32(torch.zeros(1)).item() == 0.0
    g = torch.Generator().manual_seed(3)
    xx = torch.randn(16, 512, generator=g).bfloat16()
    y = O.gelu_and_mul(xx)
    unrounded = (F.gelu(xx[:, :256].float()) * xx[:, 256:].float()).bfloat16()
    assert not torch.equal(y, unrounded)
    torch.testing.assert_close(y.float(), unrounded.float(), rtol=1.6e-2, atol=1e-3)
    yt = O.gelu_and_mul(xx, "tanh")
    ref = (F.gelu(xx[:, :256].float(), approximate="tanh").bfloat16().float() *
           xx[:, 256:].float()).bfloat16()
    torch.testing.assert_close(yt.float(), ref.float(), rtol=1.6e-2, atol=1e-3)


def test_swiglustep_matches_reference_test_formula():
    """fp32 input: the reference test's forward_native
    (tests/ops/swiglustep_and_mul_op.py:23-29) up to the exp ulp; the gate
    clamps only from above, the up input both ways."""
    F = torch.nn.functional
    g = torch.Generator().manual_seed(4)
    x = torch.randn(32, 256, generator=g) * 6
    ref = F.silu(x[:, :128]).clamp(max=7.0) * x[:, 128:].clamp(min=-7.0, max=7.0)
    torch.testing.assert_close(O.swiglustep_and_mul(x), ref, rtol=2e-6, atol=1e-6)
    t = torch.tensor([[20.0, -20.0, 100.0, -100.0]])
    assert O.swiglustep_and_mul(t).tolist() == [[7.0 * 7.0, pytest.approx(-20.0 / (1 + math.exp(20.0)) * -7.0)]]


def test_relu2_exact_values():
    x = torch.tensor([-1.0, 0.0, 1.5, 3.0, -0.0]).bfloat16()
    assert O.relu2_no_mul(x).float().tolist() == [0.0, 0.0, 2.25, 9.0, 0.0]


# ------------------------------------------- fused SiLU-and-mul + quantisers
def _gate_up(T, H, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, 2 * H, generator=g) * scale).to(dtype)


def test_silu_mul_f32_gate_first_unrounded():
    """r = silu(first half) * second half in fp32: within 3 ulp of torch's
    own silu, unlike the swapped halves or a 16-bit-rounded silu."""
    x = _gate_up(8, 256, 1)
    r = O.silu_mul_f32(x)
    g, u = x[:, :256].float(), x[:, 256:].float()
    assert torch.allclose(r, torch.nn.functional.silu(g) * u, rtol=4e-7, atol=0)
    assert not torch.allclose(r, torch.nn.functional.silu(u) * g, rtol=1e-2)
    rounded = torch.nn.functional.silu(g).bfloat16().float() * u
    assert (r != rounded).float().mean().item() > 0.5


def _reference_test_group_quant(r, group_size, quant_dtype):
    """The quantiser of the reference's own test
    (tests/test_fused_silu_mul_block_quant.py:49-66) applied to fp32 r."""
    T, H = r.shape
    rg = r.reshape(T, H // group_size, group_size)
    gmax = rg.abs().amax(-1)
    if quant_dtype == torch.int8:
        s = gmax.clamp(min=1e-10) / 127.0
        q = (rg / s.unsqueeze(-1)).round().clamp(-128, 127)
    else:
        qmax = torch.finfo(quant_dtype).max
        s = gmax.clamp(min=torch.finfo(torch.float32).tiny) / qmax
        q = (rg / s.unsqueeze(-1)).clamp(-qmax, qmax)
    return q.reshape(T, H).to(quant_dtype), s


@pytest.mark.parametrize("quant_dtype", [torch.float8_e4m3fn, torch.float8_e5m2, torch.int8])
@pytest.mark.parametrize("group_size", [32, 64, 128])
def test_block_quant_matches_reference_test_quantiser(quant_dtype, group_size):
    """On unit-scale data (every group's scale above the floors) the oracle
    quantises silu(gate)*up exactly as the reference test's quantiser does."""
    x = _gate_up(16, 512, 2)
    q, s = O.silu_and_mul_per_block_quant(x, group_size, quant_dtype)
    qr, sr = _reference_test_group_quant(O.silu_mul_f32(x), group_size, quant_dtype)
    assert torch.equal(s, sr)
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8))


def test_block_quant_floors_and_qmax():
    """qmax is the format's largest finite value; an all-zero group takes
    the floor scale 1/(qmax*512) (fp8) or FLT_EPSILON (int8), codes 0."""
    assert O._QMAX[torch.float8_e4m3fn] == torch.finfo(torch.float8_e4m3fn).max
    assert O._QMAX[torch.float8_e5m2] == torch.finfo(torch.float8_e5m2).max
    x = _gate_up(2, 128, 3)
    x[0, :64] = 0.0                       # gate of group 0 of row 0: silu(0) = 0
    for dt, floor in [(torch.float8_e4m3fn, 1.0 / (448.0 * 512.0)),
                      (torch.float8_e5m2, 1.0 / (57344.0 * 512.0)),
                      (torch.int8, torch.finfo(torch.float32).eps)]:
        q, s = O.silu_and_mul_per_block_quant(x, 64, dt)
        assert s[0, 0].item() == pytest.approx(floor, rel=1e-7)
        assert not q.float()[0, :64].any()   # +-0 (0 * negative up is -0)
        assert s[0, 1].item() > floor and s[1, 0].item() > floor


def test_block_quant_scale_ub_and_ue8m0():
    """scale_ub caps the scale (the largest values then saturate at qmax) and
    never lowers it below the floor; ue8m0 rounds the scale up to a power of
    two."""
    x = _gate_up(4, 256, 4)
    q, s = O.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn)
    ub = float(s.min()) / 4
    qu, su = O.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn, scale_ub=ub)
    assert torch.all(su == torch.tensor(ub, dtype=torch.float32))
    assert torch.all(qu.float().abs().reshape(4, 2, 128).amax(-1) == 448.0)
    _, sf = O.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn, scale_ub=1e-12)
    assert torch.all(sf == torch.tensor(1.0, dtype=torch.float32) / (448.0 * 512.0))
    _, se = O.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn, scale_ue8m0=True)
    m, _ = torch.frexp(se)
    assert torch.all(m == 0.5) and torch.all(se >= s) and torch.all(se < 2 * s)


def test_mxfp4_fused_is_silu_then_pinned_quantiser():
    """The fused mxfp4 quantiser equals the pinned per-token-group mxfp4
    quantiser applied to silu(gate)*up, all-zero groups included, and its
    scales equal the reference test's RCEIL e8m0 scales
    (tests/ops/mx_utils.py:307-330)."""
    x = _gate_up(6, 256, 5)
    x[1, :32] = 0.0
    q, s = O.silu_and_mul_mxfp4_quant(x)
    q2, s2 = O.per_token_group_quant_mxfp4(O.silu_mul_f32(x), 32)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    amax = O.silu_mul_f32(x).reshape(6, 8, 32).abs().amax(-1)
    e = torch.clamp(torch.ceil(torch.log2(amax / 6.0)), -127, 127) + 127
    rceil = torch.where(e == 0, torch.ones_like(amax), torch.exp2(e - 127))
    nz = amax > 0
    assert torch.equal(s[nz], rceil[nz])


MXFP4_KNOWN = {0.5: (0.125, 6), 1.0: (0.25, 6), 1.5: (0.25, 7), 2.0: (0.5, 6),
               3.0: (0.5, 7), 4.0: (1.0, 6), 6.0: (1.0, 7)}


@pytest.mark.parametrize("val", sorted(MXFP4_KNOWN))
def test_mxfp4_quant_known_values(val):
    """tests/test_mxfp4_quant.py:113-142, expected scale/code derived by hand."""
    x = torch.zeros(1, 32)
    x[0, 0] = val
    q, s = O.per_token_group_quant_mxfp4(x)
    es, ec = MXFP4_KNOWN[val]
    assert s[0, 0].item() == es
    assert int(q[0, 0]) & 0xF == ec
    assert (q[0, 1:] == 0).all()


def test_to_mxfp4_rne_ties_and_grid():
    # block max 6 -> e8m0 127 (scale 1); midpoints tie to the even code
    v = torch.tensor([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.75, 0.5,
                      1.0, 1.5, 2.0, 3.0, 4.0, -6.0] + [0.0] * 16)
    q, e = O.to_mxfp4(v.unsqueeze(0))
    assert e.tolist() == [[127]]
    codes = torch.stack([q[0] & 0xF, q[0] >> 4], -1).flatten().tolist()
    assert codes[:16] == [7, 0, 2, 2, 4, 4, 6, 6, 0xA, 1, 2, 3, 4, 5, 6, 0xF]
    # decode round trip is exact on the grid
    d = O.dequant_mxfp4(q, e)
    assert torch.equal(d[0, 9:16], torch.tensor([0.5, 1, 1.5, 2, 3, 4, -6.0]))


# ----------------------------------------------------------- GEMM and layer
def test_grouped_gemm_fp8_block_all_finite_e4m3_kat():
    """tests/fused_moe/test_grouped_gemm.py:275-307: identity A x every finite
    e4m3 code x block scales {0.5, 2.0} is reproduced bit-exactly."""
    n, k = 128, 256
    a = torch.eye(k, dtype=torch.bfloat16)
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)],
                         dtype=torch.uint8)
    b = codes.repeat((n * k + 253) // 254)[:n * k].reshape(1, n, k)
    b = b.view(torch.float8_e4m3fn)
    scales = torch.tensor([[[0.5, 2.0]]])
    out = O.grouped_gemm("fp8block", a, b, scales, None,
                         torch.tensor([k], dtype=torch.int32))
    ref = (b.float() * scales.repeat_interleave(128, 1).repeat_interleave(128, 2))
    assert torch.equal(out.float(), ref[0].t().to(torch.bfloat16).float())


def test_grouped_gemm_single_expert_is_matmul():
    torch.manual_seed(5)
    a = torch.randn(9, 64).to(torch.bfloat16)
    w = (torch.randn(1, 32, 64) * 0.1).to(torch.bfloat16)
    bias = torch.randn(1, 32).to(torch.bfloat16)
    out = O.grouped_gemm("bf16", a, w, None, bias, [9])
    ref = (a.float() @ w[0].float().t() + bias[0].float()).to(torch.bfloat16)
    assert torch.equal(out, ref)


def _reference_test_golden(x, w13, b13, w2, b2, weights, ids, k):
    """Restatement of the reference test golden
    tests/fused_moe/test_fused_moe.py:119-176 (argsort / bincount /
    scatter_reduce structure), weights in nk layout."""
    flat_i = ids.view(-1)
    flat_w = weights.view(-1, 1)
    cache = torch.zeros_like(x)
    idxs = flat_i.argsort()
    counts = flat_i.bincount().numpy()
    ends = counts.cumsum()
    tok = idxs // k
    for e, end in enumerate(ends):
        st = 0 if e == 0 else ends[e - 1]
        if st == end:
            continue
        xt = x[tok[st:end]]
        w1, w3 = torch.split(w13[e], w13.shape[1] // 2, dim=0)
        g = xt.float() @ w1.t().float()
        u = xt.float() @ w3.t().float()
        if b13 is not None:
            b1, b3 = b13[e].chunk(2)
            g, u = g + b1.float(), u + b3.float()
        o = (torch.nn.functional.silu(g) * u) @ w2[e].t().float()
        if b2 is not None:
            o = o + b2[e].float()
        o = o.to(x.dtype)
        o.mul_(flat_w[idxs[st:end]])
        cache.scatter_reduce_(0, tok[st:end].view(-1, 1).repeat(1, x.shape[-1]),
                              o, reduce="sum")
    return cache


def test_fused_moe_oracle_vs_reference_golden():
    torch.manual_seed(6)
    T, H, I, E, k = 24, 64, 32, 6, 2
    x = torch.randn(T, H).to(torch.bfloat16) / 4
    w13 = (torch.randn(E, 2 * I, H) / 8).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I) / 8).to(torch.bfloat16)
    b13 = (torch.randn(E, 2 * I) / 16).to(torch.bfloat16)
    b2 = (torch.randn(E, H) / 16).to(torch.bfloat16)
    scores = torch.randn(T, E)
    w, ids = torch.topk(scores, k, dim=-1)
    y = O.fused_moe("bf16", x, w13, None, b13, w2, None, b2, w, ids)
    ref = _reference_test_golden(x, w13, b13, w2, b2, w, ids, k)
    torch.testing.assert_close(y.float(), ref.float(), rtol=2e-2, atol=2e-2)


def test_fp8_per_expert_is_the_16bit_layer_on_dequantised_weights():
    """Recipe "fp8" (per-expert scales, w8a16): e4m3 and e5m2 codes times a
    power-of-two scale are exact in fp32, so the grouped GEMM and the layer
    equal the 16-bit recipe run on the dequantised weights."""
    g = torch.Generator().manual_seed(12)
    E, N, K = 3, 64, 96
    rows = [5, 0, 7]
    a = torch.randn(sum(rows), K, generator=g).bfloat16()
    s = torch.tensor([0.25, 2.0, 8.0])
    for dt in (torch.float8_e4m3fn, torch.float8_e5m2):
        q = (torch.randn(E, N, K, generator=g) * 4).to(dt)
        deq = q.float() * s.view(E, 1, 1)
        y = O.grouped_gemm("fp8", a, q, s, None, rows)
        assert torch.equal(y, O.grouped_gemm("bf16", a, deq, None, None, rows))
    T, H, I, k = 10, 64, 32, 2
    x = torch.randn(T, H, generator=g).bfloat16()
    q13 = (torch.randn(E, 2 * I, H, generator=g) * 4).to(torch.float8_e5m2)
    q2 = (torch.randn(E, H, I, generator=g) * 4).to(torch.float8_e5m2)
    w, ids, _ = O.topk_softmax(torch.randn(T, E, generator=g), k, True)
    y = O.fused_moe("fp8", x, q13, s, None, q2, s * 0.5, None, w, ids)
    ref = O.fused_moe("bf16", x, q13.float() * s.view(E, 1, 1), None, None,
                      q2.float() * (s * 0.5).view(E, 1, 1), None, None, w, ids)
    assert torch.equal(y, ref)


def test_int4_zero_point_conversion_and_dequant():
    """u4 with zero point 8 -> two's-complement int4 is `byte ^ 0x88` ((u4 -
    8) mod 16 per nibble, all 256 bytes); the oracle's int4 dequantisation of
    the converted bytes equals the reference test's (u4 - 8) * scale in the
    scale's type (tests/fused_moe/test_grouped_gemm.py:310-323)."""
    b = torch.arange(256, dtype=torch.int32)
    zp = ((((b & 0xF) - 8) & 0xF) | ((((b >> 4) - 8) & 0xF) << 4))
    assert torch.equal(zp, b ^ 0x88)
    g = torch.Generator().manual_seed(13)
    N, K, grp = 48, 256, 64
    u = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    for dt in (torch.bfloat16, torch.float16):
        s = torch.pow(2.0, torch.randint(-3, 4, (N, K // grp), generator=g).float()).to(dt)
        nib = torch.stack([u.to(torch.int32) & 0xF, u.to(torch.int32) >> 4], -1).reshape(N, K)
        ref = ((nib - 8) * s.repeat_interleave(grp, 1)).to(dt).float()
        assert torch.equal(O.dequant_int4(u ^ 0x88, s), ref)
    # non-power-of-two scales round the product to the scale's type
    s = torch.full((N, K // grp), 0.3).bfloat16()
    v = O.dequant_int4(torch.full((N, K // 2), 0x77, dtype=torch.uint8), s)
    assert torch.all(v == (7 * s.float()).bfloat16().float()[0, 0])


def test_fused_moe_oracle_fp8block_close_to_dequant_fp32():
    """fp8block = dequantised fp32 layer up to activation quantisation noise."""
    torch.manual_seed(8)
    T, H, I, E, k = 12, 256, 128, 4, 2
    x = torch.randn(T, H).to(torch.bfloat16)
    w13m = torch.randn(E, 2 * I, H) * 0.02
    w2m = torch.randn(E, H, I) * 0.02
    q13, s13 = O.fp8_block_quant_weight(w13m)
    q2, s2 = O.fp8_block_quant_weight(w2m)
    scores = torch.randn(T, E)
    w, ids, _ = O.topk_softmax(scores, k, True)
    y = O.fused_moe("fp8block", x, q13, s13, None, q2, s2, None, w, ids)
    d13 = torch.stack([O.dequant_fp8_block_weight(q13[e], s13[e]) for e in range(E)])
    d2 = torch.stack([O.dequant_fp8_block_weight(q2[e], s2[e]) for e in range(E)])
    ref = O.fused_moe("bf16", x, d13, None, None, d2, None, None, w, ids)
    torch.testing.assert_close(y.float(), ref.float(), rtol=0.1, atol=0.05)
    # pre-quantised input (a1q_scale): the pinned 1x128 quantiser's own
    # (q, s) give exactly the layer that quantises x itself; other scales
    # (a power of two above) give a different but close layer
    xq, xs = O.per_token_group_fp8_quant(x, 128)
    yq = O.fused_moe("fp8block", xq, q13, s13, None, q2, s2, None, w, ids, a1q_scale=xs)
    assert yq.dtype == torch.bfloat16 and torch.equal(yq, y)
    xq2, xs2 = O.per_token_group_fp8_quant(x, 128, scale_ue8m0=True)
    y2 = O.fused_moe("fp8block", xq2, q13, s13, None, q2, s2, None, w, ids, a1q_scale=xs2)
    assert not torch.equal(y2, y)
    torch.testing.assert_close(y2.float(), y.float(), rtol=0.1, atol=0.05)
    # compute_dtype=fp16 on pre-quantised input is exactly the fp16 layer
    # that quantises its own fp16 input (the quantiser's codes and scales
    # are the same for x in bf16 and in fp16: bf16 -> fp16 is exact here)
    xh = x.half()
    yh = O.fused_moe("fp8block", xh, q13, s13, None, q2, s2, None, w, ids)
    xqh, xsh = O.per_token_group_fp8_quant(xh, 128)
    assert torch.equal(xqh.view(torch.uint8), xq.view(torch.uint8)) and torch.equal(xsh, xs)
    yqh = O.fused_moe("fp8block", xq, q13, s13, None, q2, s2, None, w, ids, a1q_scale=xs,
                      compute_dtype=torch.float16)
    assert yqh.dtype == torch.float16 and torch.equal(yqh, yh)
    assert not torch.equal(yqh.float(), yq.float())


# ------------------------------------------------------------ MX recipes
def _e4m3_grid():
    """Every finite e4m3 value, decoded from its bit fields by hand
    (sign, 4-bit exponent with bias 7, 3-bit mantissa; exponent 0 is
    subnormal; 0x7f/0xff are NaN)."""
    vals = []
    for b in range(256):
        if b & 0x7F == 0x7F:
            continue
        e, m = (b >> 3) & 0xF, b & 7
        v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        vals.append(-v if b & 0x80 else v)
    return torch.tensor(sorted(set(vals)), dtype=torch.float64)


def test_e8m0_value_special_codes():
    e = torch.tensor([0, 1, 126, 127, 128, 254, 255], dtype=torch.uint8)
    v = O.e8m0_value(e)
    assert v[:6].tolist() == [2.0 ** -127, 2.0 ** -126, 0.5, 1.0, 2.0, 2.0 ** 127]
    assert math.isnan(v[6].item())


def test_dequant_mxfp8_kat_per_32_along_k():
    """Group g of row r is scaled by 2^(s[r, g] - 127); nothing else."""
    q = torch.ones(2, 64).to(torch.float8_e4m3fn)
    q[1, 33] = torch.tensor(-448.0).to(torch.float8_e4m3fn)
    s = torch.tensor([[127, 130], [120, 127]], dtype=torch.uint8)
    d = O.dequant_mxfp8(q, s)
    assert torch.all(d[0, :32] == 1.0) and torch.all(d[0, 32:] == 8.0)
    assert torch.all(d[1, :32] == 2.0 ** -7)
    assert d[1, 33].item() == -448.0 and d[1, 32].item() == 1.0


def test_mxfp8_act_quant_scale_is_least_power_of_two_and_codes_nearest():
    """Brute force on the e4m3 grid: the e8m0 scale s is the least power of
    two with amax / s <= 448 for groups whose amax / 448 is above the
    1 / (448 * 512) scale floor, 2^ceil(log2(floor)) = 2^-17 for the others,
    and every code is a nearest grid value of x / s."""
    torch.manual_seed(21)
    x = (torch.randn(6, 256) * torch.logspace(-6, 4, 6).unsqueeze(1)).to(torch.bfloat16)
    x[2, 64:96] = 0.0
    q, e = O.quant_mxfp8_act(x)
    assert q.dtype == torch.float8_e4m3fn and e.dtype == torch.uint8
    assert e.shape == (6, 8)
    xf = x.double().reshape(6, 8, 32)
    s = torch.exp2(e.double() - 127)
    amax = xf.abs().amax(-1)
    live = amax > 1.0 / 512.0
    assert live.any() and (~live).any()
    assert torch.all(amax[live] / s[live] <= 448.0)
    assert torch.all(amax[live] / (s[live] / 2) > 448.0)
    assert torch.all(s[~live] == 2.0 ** -17)
    grid = _e4m3_grid()
    y = (xf / s.unsqueeze(-1)).flatten()
    qd = q.double().flatten()
    dist = (y.unsqueeze(1) - grid.unsqueeze(0)).abs()
    best = dist.min(1).values
    assert torch.all((qd - y).abs() <= best + 1e-300)
    # the all-zero group dequantises to zero; the round trip moves the
    # group amax by at most half a 3-bit-mantissa ulp
    d = O.dequant_mxfp8(q, e)
    assert torch.all(d[2, 64:96] == 0)
    da = d.double().reshape(6, 8, 32).abs().amax(-1)
    assert torch.all((da[live] - amax[live]).abs() <= amax[live] * 2.0 ** -4)


def test_mxfp4_act_quant_matches_rceil_and_grid_brute_force():
    """e8m0 scale = 2^ceil(log2(amax / 6)); every e2m1 code is the nearest
    grid point of x / s, a midpoint going to the smaller magnitude
    (csrc/quantization/fp4/mxfp4_quant.h:17-25 compares with strict >)."""
    torch.manual_seed(22)
    x = torch.randn(5, 128).to(torch.bfloat16) * 3
    q, e = O.quant_mxfp4_act(x)
    assert q.shape == (5, 64) and e.shape == (5, 4)
    xf = x.double().reshape(5, 4, 32)
    amax = xf.abs().amax(-1)
    assert torch.equal(e.long(), (torch.ceil(torch.log2(amax / 6.0)) + 127).long())
    grid = torch.tensor([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=torch.float64)
    y = (xf / torch.exp2(e.double() - 127).unsqueeze(-1)).flatten()
    codes = torch.stack([q & 0xF, q >> 4], -1).reshape(-1).long()
    mag = (y.abs().unsqueeze(1) - grid).abs()
    best = mag.min(1).values
    got = grid[codes & 7]
    assert torch.all((got - y.abs()).abs() <= best + 1e-12)
    tie = (mag == best.unsqueeze(1)).sum(1) > 1
    assert tie.any()
    lower = grid[(mag == best.unsqueeze(1)).int().argmax(1)]
    assert torch.all(got[tie] == lower[tie])
    nz = got != 0
    assert torch.all(((codes[nz] >> 3) == 1) == (y[nz] < 0))


def _mx_weights(E, N, K, seed, fmt):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(E, N, K, generator=g) * 0.05
    if fmt == "mxfp8":
        q, e = O.quant_mxfp8_act(w.reshape(E * N, K))
        return q.reshape(E, N, K), e.reshape(E, N, K // 32)
    q, e = O.quant_mxfp4_act(w.reshape(E * N, K))
    return q.reshape(E, N, K // 2), e.reshape(E, N, K // 32)


def test_fused_moe_oracle_mxfp8_is_bf16_layer_on_qdq_input_and_act():
    """mxfp8 = the 16-bit layer on exactly dequantised weights whose input
    and intermediate activation went through the pinned mxfp8 round trip;
    a1q_scale with the quantiser's own (q, e) gives the same layer."""
    torch.manual_seed(23)
    T, H, I, E, k = 9, 128, 64, 4, 2
    x = torch.randn(T, H).to(torch.bfloat16)
    q13, s13 = _mx_weights(E, 2 * I, H, 1, "mxfp8")
    q2, s2 = _mx_weights(E, H, I, 2, "mxfp8")
    w, ids, _ = O.topk_softmax(torch.randn(T, E), k, True)
    y = O.fused_moe("mxfp8", x, q13, s13, None, q2, s2, None, w, ids)
    d13 = torch.stack([O.dequant_mxfp8(q13[e], s13[e]) for e in range(E)])
    d2 = torch.stack([O.dequant_mxfp8(q2[e], s2[e]) for e in range(E)])
    xq = O.dequant_mxfp8(*O.quant_mxfp8_act(x)).to(torch.bfloat16)
    # 16-bit layer with the intermediate round trip spelled out per slot
    flat = ids.reshape(-1).long()
    g2 = torch.zeros(T * k, H, dtype=torch.bfloat16)
    for e in range(E):
        sl = (flat == e).nonzero().flatten()
        if sl.numel() == 0:
            continue
        g1 = (xq[sl // k].float() @ d13[e].t()).to(torch.bfloat16)
        a = O.silu_and_mul(g1)
        aq = O.dequant_mxfp8(*O.quant_mxfp8_act(a))
        g2[sl] = (aq @ d2[e].t()).to(torch.bfloat16)
    ref = (g2.float().reshape(T, k, H) * w.float().unsqueeze(-1))
    acc = torch.zeros(T, H)
    for j in range(k):
        acc = acc + ref[:, j]
    assert torch.equal(y, acc.to(torch.bfloat16))
    xq8, xe8 = O.quant_mxfp8_act(x)
    ya = O.fused_moe("mxfp8", xq8, q13, s13, None, q2, s2, None, w, ids, a1q_scale=xe8)
    assert ya.dtype == torch.bfloat16 and torch.equal(ya, y)


def test_fused_moe_oracle_mxfp4_a1q_quantises_both_gemm_inputs():
    """mxfp4 with pre-quantised input: GEMM1 reads the dequantised packed
    input, GEMM2 the mxfp4 round trip of the activation; without a1q_scale
    the recipe is w4a16 (activation unrounded)."""
    torch.manual_seed(24)
    T, H, I, E, k = 7, 128, 64, 3, 2
    x = torch.randn(T, H).to(torch.bfloat16)
    q13, s13 = _mx_weights(E, 2 * I, H, 3, "mxfp4")
    q2, s2 = _mx_weights(E, H, I, 4, "mxfp4")
    w, ids, _ = O.topk_softmax(torch.randn(T, E), k, True)
    xq, xe = O.quant_mxfp4_act(x)
    ya = O.fused_moe("mxfp4", xq, q13, s13, None, q2, s2, None, w, ids, a1q_scale=xe)
    xd = O.dequant_mxfp4(xq, xe).to(torch.bfloat16)
    y16 = O.fused_moe("mxfp4", xd, q13, s13, None, q2, s2, None, w, ids)
    assert ya.shape == (T, H) and not torch.equal(ya, y16)
    torch.testing.assert_close(ya.float(), y16.float(), rtol=0.25, atol=0.05)
    flat = ids.reshape(-1).long()
    g2 = torch.zeros(T * k, H, dtype=torch.bfloat16)
    for e in range(E):
        sl = (flat == e).nonzero().flatten()
        if sl.numel() == 0:
            continue
        g1 = (xd[sl // k].float() @ O.dequant_mxfp4(q13[e], s13[e]).t()).to(torch.bfloat16)
        a = O.silu_and_mul(g1)
        aq = O.dequant_mxfp4(*O.quant_mxfp4_act(a))
        g2[sl] = (aq @ O.dequant_mxfp4(q2[e], s2[e]).t()).to(torch.bfloat16)
    acc = torch.zeros(T, H)
    for j in range(k):
        acc = acc + g2.float().reshape(T, k, H)[:, j] * w.float()[:, j:j + 1]
    assert torch.equal(ya, acc.to(torch.bfloat16))
