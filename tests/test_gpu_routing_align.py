"""GPU parity: routing and token->expert alignment are bit-exact against the
CPU oracle on the same inputs."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _ops():
    from vllm_xpu_kernels import ops
    return ops


@pytest.mark.parametrize("T", [1, 33, 64])
@pytest.mark.parametrize("E", [16, 128, 192, 512, 1024])
@pytest.mark.parametrize("k", [2, 8])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("has_bias", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_softmax(dev, T, E, k, renorm, has_bias, dtype):
    g = torch.Generator().manual_seed(T * 7919 + E * 31 + k)
    logits = torch.randn(T, E, generator=g).to(dtype)
    bias = torch.randn(E, generator=g) if has_bias else None
    w, ids, tei = _ops().topk_softmax(logits.to(dev), k, renorm,
                                      bias.to(dev) if has_bias else None)
    rw, rids, rtei = O.topk_softmax(logits, k, renorm, bias)
    assert torch.equal(ids.cpu(), rids)
    assert torch.equal(tei.cpu(), rtei)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T", [1, 64])
@pytest.mark.parametrize("E", [16, 256])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("rsf", [1.0, 2.5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_topk_sigmoid(dev, T, E, renorm, rsf, dtype):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g).to(dtype)
    bias = torch.randn(E, generator=g)
    w, ids, _ = _ops().topk_sigmoid(logits.to(dev), 8, renorm, bias.to(dev),
                                    routed_scaling_factor=rsf)
    rw, rids, _ = O.topk_sigmoid(logits, 8, renorm, bias, rsf)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-7)


# reference tests/test_topk_softplus_sqrt.py:250-349 parameter grid
@pytest.mark.parametrize("T", [1, 33, 128])
@pytest.mark.parametrize("E", [128, 256, 384, 512])
@pytest.mark.parametrize("k", [6, 8, 16])
@pytest.mark.parametrize("renorm,rsf", [(True, 1.0), (False, 1.5), (True, 1.5)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_softplus_sqrt(dev, T, E, k, renorm, rsf, dtype):
    """With a correction bias (biased selection, (s + b) - b weights): the
    same experts per row as the oracle (the reference test's criterion,
    sorted ids), weights matched by expert within fp32 ulps of exp / log /
    sqrt, and the same order in at least 95 % of rows (scores an ulp apart
    may swap places, as they may between the reference kernel and torch)."""
    g = torch.Generator().manual_seed(T * 7 + E + k)
    logits = torch.randn(T, E, generator=g).to(dtype)
    bias = torch.randn(E, generator=g) * 0.1
    w, ids = _ops().topk_softplus_sqrt(logits.to(dev), k, renorm, rsf, bias.to(dev))
    rw, rids = O.topk_softplus_sqrt(logits, k, renorm, rsf, bias)
    gi, gw = ids.cpu().long(), w.cpu()
    assert torch.equal(gi.sort(-1).values, rids.sort(-1).values)
    assert (gi == rids).all(-1).float().mean().item() >= 0.95
    torch.testing.assert_close(gw.gather(1, gi.argsort(1)), rw.gather(1, rids.argsort(1)),
                               rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T", [1, 33, 1024])
@pytest.mark.parametrize("E", [256, 576])
@pytest.mark.parametrize("k", [6, 16])
@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_topk_softplus_sqrt_hash(dev, T, E, k, idt):
    """Hash routing: experts tid2eid[input_ids[t]] (of the indices' dtype),
    weights their sqrt(softplus) scores, renormalised and scaled by 2.5."""
    g = torch.Generator().manual_seed(T + E + k)
    logits = torch.randn(T, E, generator=g)
    tab = torch.randint(0, E, (4096, k), generator=g).to(idt)
    tok = torch.randint(0, 4096, (T,), generator=g).to(idt)
    w = torch.empty(T, k, device=dev)
    ids = torch.empty(T, k, dtype=idt, device=dev)
    src = torch.empty(T, k, dtype=torch.int32, device=dev)
    torch.ops._moe_C.topk_softplus_sqrt(w, ids, src, logits.to(dev), True, 2.5, None,
                                        tok.to(dev), tab.to(dev))
    rw, rids = O.topk_softplus_sqrt(logits, k, True, 2.5, None, tok, tab)
    assert torch.equal(ids.cpu().long(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-7)
    assert torch.equal(src.cpu(), (torch.arange(k).view(1, k) * T + torch.arange(T).view(T, 1))
                       .int())


def test_topk_softplus_sqrt_rejects_unsupported_expert_count(dev):
    x = torch.randn(4, 100, device=dev)
    with pytest.raises(RuntimeError, match="Unsupported expert number"):
        _ops().topk_softplus_sqrt(x, 4, True)


def test_topk_softmax_int64_ids_and_ties(dev):
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.0, 3.0, -1.0, 3.0, 2.0]])
    w, ids, _ = _ops().topk_softmax(logits.to(dev), 3, False,
                                    indices_type=torch.int64)
    assert ids.dtype == torch.int64
    assert ids.cpu().tolist() == [[1, 2, 4]]


@pytest.mark.parametrize("T", [1, 64, 512])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("renorm", [True, False])
def test_grouped_topk_deepseek_shape(dev, T, dtype, renorm):
    """C3 routing: sigmoid scores, +bias N(0,0.01), 8 groups keep 4, top-8,
    rsf 2.5."""
    g = torch.Generator().manual_seed(T)
    logits = torch.randn(T, 256, generator=g)
    bias = torch.randn(256, generator=g) * 0.01
    s = logits.sigmoid().to(dtype)
    sb = (s.float() + bias).to(dtype)
    v, ids = _ops().grouped_topk(s.to(dev), sb.to(dev), 8, 4, 8, renorm, 2.5)
    rv, rids = O.grouped_topk(s, sb, 8, 4, 8, renorm, 2.5)
    assert torch.equal(ids.cpu(), rids)
    assert v.dtype == dtype
    torch.testing.assert_close(v.cpu().float(), rv.float(), rtol=4e-6 if dtype == torch.float32 else 8e-3, atol=1e-7)


@pytest.mark.parametrize("T", [1, 33, 2051, 8192])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("E,n_group,topk_group,k", [(256, 8, 4, 8), (128, 4, 2, 6),
                                                    (512, 16, 8, 8), (256, 1, 1, 16),
                                                    (96, 3, 2, 4), (64, 1, 1, 8),
                                                    (256, 32, 4, 8)])
def test_fused_grouped_topk_equals_torch_scoring(dev, T, dtype, E, n_group, topk_group, k):
    """One-launch sigmoid + correction bias + grouped top-k equals the
    reference's caller-side torch ops followed by the grouped top-k op
    (tests/ops/grouped_topk_op.py:67-92) bit for bit: same ids, same values,
    both against the oracle.  From 2048 tokens (2051: a ragged last wave),
    E 128 / 256 / 512 with n_group dividing 16 run four tokens per wave;
    n_group 3 takes the serial group scan, 32 and E 64 / 96 the
    one-token-per-wave shuffle merge."""
    g = torch.Generator(device=dev).manual_seed(T + E)
    logits = torch.randn(T, E, generator=g, device=dev).to(dtype)
    bias = torch.randn(E, generator=g, device=dev) * 0.01
    v, ids = _ops().fused_grouped_topk(logits, k, True, bias, n_group, topk_group,
                                       "sigmoid", 2.5)
    s = logits.sigmoid()
    sb = (s + bias.unsqueeze(0)).to(dtype)
    rv, rids = _ops().grouped_topk(s, sb, n_group, topk_group, k, True, 2.5)
    assert torch.equal(ids, rids)
    assert torch.equal(v, rv.float())
    toks = torch.linspace(0, T - 1, min(T, 64)).long().to(dev)
    ov, oids = O.grouped_topk(s[toks].cpu(), sb[toks].cpu(), n_group, topk_group, k, True, 2.5)
    assert torch.equal(ids[toks].cpu(), oids)
    tol = 4e-6 if dtype == torch.float32 else 8e-3
    torch.testing.assert_close(v[toks].cpu(), ov.float(), rtol=tol, atol=1e-7)


def test_fused_grouped_topk_without_bias(dev):
    logits = torch.randn(33, 256, device=dev)
    v, ids = _ops().fused_grouped_topk(logits, 8, False, None, 8, 4, "sigmoid", 1.0)
    s = logits.sigmoid()
    rv, rids = _ops().grouped_topk(s, s.clone(), 8, 4, 8, False, 1.0)
    assert torch.equal(ids, rids) and torch.equal(v, rv)


@pytest.mark.parametrize("name,T", [("C2", 4096), ("C4", 2048), ("C5", 4096), ("C3", 8192)])
def test_route_full_size_bit_exact(dev, name, T):
    """Each configuration's router at its prefill size on the benchmark's own
    logits (C4 Zipf-skewed): every token's expert ids equal the oracle's bit
    for bit, the weights within fp32 ulps.  C3 scores with the sigmoid the
    reference's caller applies (tests/ops/grouped_topk_op.py:67-92), taken
    from the device as the oracle's input."""
    from vllm_xpu_kernels import workloads as W
    cfg = W.CONFIGS[name]
    logits = W.make_router_logits(cfg, T, dev)
    bias = W.make_correction_bias(cfg, dev) if cfg.routing == "grouped_sigmoid" else None
    tw, ti = W.route(cfg, logits, bias)
    if cfg.routing == "grouped_sigmoid":
        s = logits.sigmoid()
        sb = s + bias.unsqueeze(0)
        rw, rids = O.grouped_topk(s.cpu(), sb.cpu(), cfg.n_group, cfg.topk_group, cfg.topk,
                                  cfg.renormalize, cfg.routed_scaling_factor)
        tol = 4e-6
    else:
        rw, rids, _ = O.topk_softmax(logits.cpu(), cfg.topk, cfg.renormalize)
        tol = 2e-6
    assert torch.equal(ti.cpu(), rids)
    torch.testing.assert_close(tw.cpu(), rw.float(), rtol=tol, atol=1e-7)


def test_grouped_topk_full_size_invariants(dev):
    """T=8192 (C3 prefill): every id lies in one of the 4 kept groups and the
    kept groups are the top-4 by top-2 sums; ids unique per token."""
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(8192, 256, generator=g)
    bias = torch.randn(256, generator=g) * 0.01
    s = logits.sigmoid()
    sb = s + bias
    v, ids = _ops().grouped_topk(s.to(dev), sb.to(dev), 8, 4, 8, True, 2.5)
    ids = ids.cpu().long()
    gs = sb.view(8192, 8, 32).topk(2, dim=-1).values.sum(-1)
    kept = torch.sort(gs, dim=-1, descending=True, stable=True).indices[:, :4]
    grp = ids // 32
    assert all(set(grp[t].tolist()) <= set(kept[t].tolist()) for t in range(0, 8192, 97))
    assert (torch.sort(ids, dim=-1).values[:, 1:] != torch.sort(ids, dim=-1).values[:, :-1]).all()
    torch.testing.assert_close(v.cpu().sum(-1), torch.full((8192,), 2.5), rtol=1e-5, atol=1e-5)
    # sampled exact parity at full size
    rv, rids = O.grouped_topk(s[:256], sb[:256], 8, 4, 8, True, 2.5)
    assert torch.equal(ids[:256].int(), rids)


# ---------------------------------------------------------------- alignment
# above 4096 ids the sort runs in chunks of workgroups: 4097 leaves a
# one-id last chunk, E=990 a large key space
ALIGN_CASES = [(1, 1, 32, 32), (3, 2, 160, 128), (256, 16, 256, 32),
               (2256, 32, 257, 128), (4096, 2, 32, 128), (4096, 8, 256, 16),
               (8192, 8, 256, 64), (4097, 1, 64, 32), (1700, 3, 990, 8)]


@pytest.mark.parametrize("m,topk,E,bs", ALIGN_CASES)
@pytest.mark.parametrize("id_dtype", [torch.int32, torch.int64])
def test_moe_align_block_size_bit_exact(dev, m, topk, E, bs, id_dtype):
    g = torch.Generator().manual_seed(m + 13 * E + bs)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(m)]).to(id_dtype)
    srt, eids, ntp = _ops().moe_align_block_size(ids.to(dev), bs, E)
    mx, nb = O.align_buffer_sizes(ids.numel(), E, bs)
    rs, re, rn = O.moe_align_block_size(ids, E, bs, mx, nb)
    assert ntp.cpu().tolist() == rn.tolist()
    assert np.array_equal(eids.cpu().numpy(), re)
    assert np.array_equal(srt.cpu().numpy(), rs)


def test_moe_align_zipf_skew_c4(dev):
    from vllm_xpu_kernels import workloads as W
    cfg = W.CONFIGS["C4"]
    logits = W.make_router_logits(cfg, 2048, dev)
    _, ids = W.route(cfg, logits)
    cnt = torch.bincount(ids.flatten().long(), minlength=128).sort(descending=True).values
    assert 0.48 <= float(cnt[:13].sum()) / ids.numel() <= 0.52
    srt, eids, ntp = _ops().moe_align_block_size(ids, 64, 128)
    mx, nb = O.align_buffer_sizes(ids.numel(), 128, 64)
    rs, re, rn = O.moe_align_block_size(ids.cpu(), 128, 64, mx, nb)
    assert np.array_equal(srt.cpu().numpy(), rs) and np.array_equal(eids.cpu().numpy(), re)


@pytest.mark.parametrize("m", [32, 2048])
def test_moe_align_expert_map(dev, m):
    E, k, bs = 8, 4, 64
    g = torch.Generator().manual_seed(5)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(m)]).int()
    em = torch.full((E,), -1, dtype=torch.int32)
    em[0::2] = torch.arange(4, dtype=torch.int32)
    srt, eids, ntp = _ops().moe_align_block_size(ids.to(dev), bs, E, em.to(dev),
                                                 ignore_invalid_experts=True)
    mx, nb = O.align_buffer_sizes(ids.numel(), E, bs)
    rs, re, rn = O.moe_align_block_size(ids, E, bs, mx, nb, expert_map=em)
    assert ntp.cpu().tolist() == rn.tolist()
    assert np.array_equal(eids.cpu().numpy(), re)
    assert np.array_equal(srt.cpu().numpy(), rs)


def test_moe_align_deterministic(dev):
    g = torch.Generator().manual_seed(42)
    ids = torch.randint(0, 32, (4096, 8), generator=g, dtype=torch.int32).to(dev)
    outs = [_ops().moe_align_block_size(ids, 64, 32) for _ in range(5)]
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert torch.equal(a, b)


# ----------------------------------------------------------- LoRA alignment
def _lora_case(T, k, E, max_loras, bs, seed, id_dtype=torch.int32, base_tokens=0):
    """Inputs and buffers as tests/test_moe_lora_align_sum.py:29-40, :55-80
    builds them (k distinct experts per token, adapters in [0, max_loras))."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(id_dtype)
    tok = torch.randint(0, max_loras, (T,), generator=g, dtype=torch.int32)
    if base_tokens:
        tok[T - base_tokens:] = -1
    mx = (ids.numel() + E * (bs - 1) + bs - 1) // bs * bs
    if ids.numel() < E:
        mx = ids.numel() * bs
    nb = (mx + bs - 1) // bs
    return ids, tok, mx, nb


def _lora_both(dev, ids, tok, E, bs, max_loras, mx, nb, lora_ids, enabled, em=None,
               fill=(-7, -2, -13)):
    """Run the op and the oracle on outputs pre-filled with sentinels."""
    srt = torch.full((max_loras * mx,), fill[0], dtype=torch.int32)
    eid = torch.full((max_loras * nb,), fill[1], dtype=torch.int32)
    ntp = torch.full((max_loras,), fill[2], dtype=torch.int32)
    d = [t.to(dev) for t in (srt, eid, ntp)]
    _ops().moe_lora_align_block_size(ids.to(dev), tok.to(dev), E, bs, max_loras, mx, nb,
                                     d[0], d[1], d[2], enabled.to(dev), lora_ids.to(dev),
                                     em.to(dev) if em is not None else None)
    r = [srt.numpy().copy(), eid.numpy().copy(), ntp.numpy().copy()]
    O.moe_lora_align_block_size(ids, tok, E, bs, max_loras, mx, nb, r[0], r[1], r[2],
                                enabled, lora_ids, em)
    return [t.cpu().numpy() for t in d], r


@pytest.mark.parametrize("T", [100, 200, 1024, 4096])
@pytest.mark.parametrize("E", [64, 128, 256, 512])
@pytest.mark.parametrize("max_loras", [2, 32])
def test_moe_lora_align_block_size(dev, T, E, max_loras):
    """The reference grid (tests/test_moe_lora_align_sum.py:43-108), bit-exact
    against the oracle, which also checks its block-membership property."""
    bs, k = 16, 6
    ids, tok, mx, nb = _lora_case(T, k, E, max_loras, bs, seed=T + E + max_loras)
    lora_ids = torch.arange(max_loras + 2, dtype=torch.int32)
    enabled = torch.ones(max_loras + 1, dtype=torch.int32)
    got, ref = _lora_both(dev, ids, tok, E, bs, max_loras, mx, nb, lora_ids, enabled)
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)
    flat = ids.flatten().numpy()
    blocks = got[0].reshape(max_loras, -1, bs)
    eid = got[1].reshape(max_loras, -1)
    for lid in range(max_loras):
        for b in range(blocks.shape[1]):
            idx = blocks[lid, b][blocks[lid, b] != ids.numel()]
            if idx.size:
                assert (flat[idx] == eid[lid, b]).all()


@pytest.mark.parametrize("T,k,E,bs,max_loras", [(33, 8, 256, 64, 4), (700, 8, 128, 128, 3)])
def test_moe_lora_align_int64_ids_and_expert_map(dev, T, k, E, bs, max_loras):
    ids, tok, mx, nb = _lora_case(T, k, E, max_loras, bs, seed=T, id_dtype=torch.int64,
                                  base_tokens=5)
    em = torch.full((E,), -1, dtype=torch.int32)
    em[1::2] = torch.arange(E // 2, dtype=torch.int32)
    # -1 in the middle, one disabled adapter, an out-of-range id at the end
    lora_ids = torch.tensor([0, -1] + list(range(1, max_loras - 1)) + [max_loras + 3],
                            dtype=torch.int32)[:max_loras + 1]
    enabled = torch.ones(max_loras + 1, dtype=torch.int32)
    enabled[1] = 0
    for m in (None, em):
        got, ref = _lora_both(dev, ids, tok, E, bs, max_loras, mx, nb, lora_ids, enabled, m)
        for a, b in zip(got, ref):
            assert np.array_equal(a, b)
    assert got[2][1] == -13  # the disabled adapter's row stays as it was


@pytest.mark.parametrize("max_loras", [1, 2])
def test_moe_lora_align_mixed_base_and_lora(dev, max_loras):
    """tests/test_moe_lora_align_sum.py:225-261: -1 first in lora_ids."""
    E, bs, k = 64, 16, 6
    ids, tok, mx, nb = _lora_case(16, k, E, 1, bs, seed=1, base_tokens=8)
    lora_ids = torch.full((max_loras + 1,), -1, dtype=torch.int32)
    lora_ids[1] = 0
    enabled = torch.ones(max_loras + 1, dtype=torch.int32)
    got, ref = _lora_both(dev, ids, tok, E, bs, max_loras, mx, nb, lora_ids, enabled)
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)
    assert 0 < got[2][0] <= mx and got[2][0] % bs == 0
    assert (got[1].reshape(max_loras, -1)[0] != -2).all()
    assert (got[0].reshape(max_loras, -1)[0] != -7).all()


def test_moe_lora_align_disabled_and_out_of_range(dev):
    """tests/test_moe_lora_align_sum.py:264-331."""
    E, bs, k = 64, 16, 6
    ids, _, mx, nb = _lora_case(16, k, E, 1, bs, seed=1)
    tok = torch.zeros(16, dtype=torch.int32)
    got, _ = _lora_both(dev, ids, tok, E, bs, 1, mx, nb, torch.tensor([0, -1], dtype=torch.int32),
                        torch.zeros(2, dtype=torch.int32))
    assert got[2][0] == -13 and (got[1] == -2).all() and (got[0] == -7).all()
    got, ref = _lora_both(dev, ids, tok, E, bs, 1, mx, nb, torch.tensor([0, 5], dtype=torch.int32),
                          torch.ones(2, dtype=torch.int32))
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)
    assert got[2][0] != -13


def test_moe_lora_align_rejects_bad_buffers(dev):
    ids, tok, mx, nb = _lora_case(8, 2, 64, 2, 16, seed=0)
    small = torch.empty(mx, dtype=torch.int32, device=dev)  # one slice, two adapters
    with pytest.raises(RuntimeError, match="smaller than max_loras"):
        _ops().moe_lora_align_block_size(
            ids.to(dev), tok.to(dev), 64, 16, 2, mx, nb, small,
            torch.empty(2 * nb, dtype=torch.int32, device=dev),
            torch.empty(2, dtype=torch.int32, device=dev),
            torch.ones(3, dtype=torch.int32, device=dev),
            torch.arange(3, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="padded_num_experts"):
        _ops().moe_lora_align_block_size(
            ids.to(dev), tok.to(dev), 1000, 16, 2, mx, nb, small, small, small, small, small)


@pytest.mark.parametrize("T,k,E,with_map", [(32, 1, 16, False), (257, 8, 64, True),
                                             (1024, 4, 128, False), (2048, 8, 128, True)])
def test_remap_hidden_states(dev, T, k, E, with_map):
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, 128, generator=g).to(torch.bfloat16)
    total = E * 2 if with_map else E
    ids = torch.stack([torch.randperm(total, generator=g)[:k] for _ in range(T)]).int()
    em = None
    if with_map:
        em = torch.full((total,), -1, dtype=torch.int32)
        em[E:] = torch.arange(E, dtype=torch.int32)
    scales = torch.randn(T, 1, generator=g)
    out, osc, rows, perm = _ops().remap_hidden_states(
        x.to(dev), ids.to(dev), total, E, em.to(dev) if em is not None else None,
        scales.to(dev))
    ro, rsc, rrows, rperm = O.remap_hidden_states(x, ids, E, em, scales)
    assert torch.equal(rows.cpu(), rrows)
    assert torch.equal(perm.cpu(), rperm)
    valid = int(rrows.sum())
    assert torch.equal(out.cpu()[:valid], ro[:valid])
    assert torch.equal(osc.cpu()[:valid], rsc[:valid])


def test_init_expert_map(dev):
    m = _ops().init_expert_map(32, 2, 4, dev)
    assert torch.equal(m.cpu(), O.init_expert_map(32, 2, 4))
