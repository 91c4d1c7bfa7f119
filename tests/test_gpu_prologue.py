"""GPU parity of fused_moe_prologue: every written section of the workspace
is bit-exact against the CPU oracle (which is pinned to the reference test's
argsort golden), on the reference test's grid
(tests/fused_moe/test_moe_prologue.py:10-265), plus expert-parallel ranks,
duplicate experts, int32 ids, unaligned rows and the bytes it must leave
untouched."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5

# recipe -> (input dtype, scale dtype, block_k) as the reference test sets
# them (fp4: hidden counts packed bytes, block_k 16 bytes = 32 values)
RECIPES = {
    "bf16": (torch.bfloat16, None, 1),
    "fp16": (torch.float16, None, 1),
    "mxfp8": (torch.float8_e4m3fn, torch.float8_e8m0fnu, 32),
    "fp8block": (torch.float8_e4m3fn, torch.float32, 128),
    "mxfp4": (torch.float4_e2m1fn_x2, torch.float8_e8m0fnu, 16),
}


def _inputs(recipe, T, hidden, g):
    dt, sdt, bk = RECIPES[recipe]
    if dt in (torch.bfloat16, torch.float16):
        x = (torch.randn(T, hidden, generator=g) / 16).to(dt)
        return x, None, bk
    if dt == torch.float4_e2m1fn_x2:
        x = torch.randint(0, 256, (T, hidden), generator=g, dtype=torch.uint8).view(dt)
    else:
        x = torch.randn(T, hidden, generator=g).to(dt)
    if sdt == torch.float32:
        sc = torch.randn(T, hidden // bk, generator=g)
    else:
        sc = torch.randint(1, 256, (T, hidden // bk), generator=g, dtype=torch.uint8).view(sdt)
    return x, sc, bk


def _u8(t):
    return t.contiguous().view(torch.uint8).reshape(t.shape[0], -1).numpy()


def _run_and_check(dev, x, sc, bk, ids, fs, E, ep_rank=0, ep_size=1, inter=512):
    from vllm_xpu_kernels import capi, ops
    T, hidden = x.shape
    k = ids.shape[1]
    eb = x.element_size()
    sb = 0 if sc is None or eb == 2 else sc.element_size()
    total, ws_map = capi.prologue_layout(T, k, hidden, eb, bk, sb, E)
    ws = torch.full((total,), SENTINEL, dtype=torch.uint8, device=dev)
    ops.fused_moe_prologue(x.to(dev), sc.to(dev) if sc is not None else None, ids.to(dev),
                           fs.to(dev), ws, hidden, inter, bk, ep_rank, ep_size, E)
    w = ws.cpu().numpy()
    ref = O.fused_moe_prologue(_u8(x), _u8(sc) if sb else None, ids.numpy(), fs.numpy(), E,
                               ep_rank)

    def sec(name, dtype):
        size, off = ws_map[name]
        return w[off:off + size].view(dtype)

    rows = int(ref["expert_first_token_offset"][-1])
    N = T * k
    assert np.array_equal(sec("expert_first_token_offset", np.int64)[:E + 1],
                          ref["expert_first_token_offset"])
    for name, dt in (("permuted_row_to_unpermuted_row", np.int32),
                     ("permuted_token_selected_experts", np.int32),
                     ("permuted_token_final_scales", np.float32)):
        got = sec(name, dt)
        assert np.array_equal(got[:rows], ref[name]), name
        # rows past the routed ones are not written
        assert (got[rows:N].view(np.uint8) == SENTINEL).all(), name
    u2p = sec("unpermuted_row_to_permuted_row", np.int32)[:N]
    routed = np.zeros(N, dtype=bool)
    for r, p in ref["unpermuted_row_to_permuted_row"].items():
        routed[r] = True
        assert u2p[r] == p
    # slots not routed to this rank: -1 (the reference leaves them as they were)
    assert (u2p[~routed] == -1).all()
    size, off = ws_map["overlapped_gemm1_gemm2_inputs"]
    data = w[off:off + N * hidden * eb].reshape(N, hidden * eb)
    assert np.array_equal(data[:rows], ref["overlapped_gemm1_gemm2_inputs"])
    assert (data[rows:] == SENTINEL).all()
    if sb:
        size, off = ws_map["permuted_act_scales"]
        srow = hidden // bk * sb
        scl = w[off:off + N * srow].reshape(N, srow)
        assert np.array_equal(scl[:rows], ref["permuted_act_scales"])
    return ref, sec


@pytest.mark.parametrize("m,n,k", [(1, 5120, 8192), (4, 5120, 8192), (16, 5120, 8192),
                                   (8192, 5120, 8192)])
@pytest.mark.parametrize("topk", [1, 2])
@pytest.mark.parametrize("recipe", ["bf16", "fp16", "mxfp8", "mxfp4", "fp8block"])
def test_prologue(dev, m, n, k, topk, recipe):
    """The reference grid: 16 experts, distinct experts per token from
    torch.topk, one rank."""
    g = torch.Generator().manual_seed(7 + m + topk)
    hidden = k // 2 if recipe == "mxfp4" else k
    x, sc, bk = _inputs(recipe, m, hidden, g)
    scores = torch.randn(m, 16, generator=g)
    fs, ids = torch.topk(scores, k=topk, dim=-1, sorted=False)
    ref, sec = _run_and_check(dev, x, sc, bk, ids.to(torch.int64).contiguous(),
                              fs.contiguous(), 16, inter=n)
    # the reference test's own check: offsets [1:] are the cumulative counts
    counts = np.bincount(ids.reshape(-1).numpy(), minlength=16).cumsum()
    assert np.array_equal(sec("expert_first_token_offset", np.int64)[1:17], counts)


@pytest.mark.parametrize("T,k,E,ep_rank,ep_size", [(37, 8, 32, 1, 4), (513, 6, 64, 0, 2),
                                                    (5000, 8, 256, 2, 3)])
@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_prologue_ep_ranks_and_duplicates(dev, T, k, E, ep_rank, ep_size, id_dtype):
    """Ids over all ranks' experts, drawn with repeats: other ranks' experts
    are dropped and a token's repeated expert is routed once."""
    g = torch.Generator().manual_seed(T + E)
    x, sc, bk = _inputs("fp8block", T, 256, g)
    ids = torch.randint(0, E * ep_size, (T, k), generator=g).to(id_dtype)
    ids[0, :] = ep_rank * E  # one token repeats one local expert k times
    fs = torch.randn(T, k, generator=g)
    ref, _ = _run_and_check(dev, x, sc, bk, ids, fs, E, ep_rank, ep_size)
    assert (ref["permuted_row_to_unpermuted_row"] == 0).sum() == 1


@pytest.mark.parametrize("recipe,hidden,bk", [("bf16", 100, 1), ("mxfp8", 40, 8),
                                              ("fp8block", 24, 8)])
def test_prologue_unaligned_rows(dev, recipe, hidden, bk):
    """Rows whose byte length is not a multiple of 16 (4-byte and byte
    copies)."""
    g = torch.Generator().manual_seed(hidden)
    dt, sdt, _ = RECIPES[recipe]
    T = 33
    if dt == torch.bfloat16:
        x, sc = torch.randn(T, hidden, generator=g).to(dt), None
    else:
        x = torch.randn(T, hidden, generator=g).to(dt)
        sc = (torch.randn(T, hidden // bk, generator=g) if sdt == torch.float32 else
              torch.randint(1, 256, (T, hidden // bk), generator=g, dtype=torch.uint8).view(sdt))
    ids = torch.stack([torch.randperm(8, generator=g)[:3] for _ in range(T)])
    _run_and_check(dev, x, sc, bk, ids, torch.randn(T, 3, generator=g), 8)


def test_prologue_rejects_small_workspace_and_bad_scales(dev):
    from vllm_xpu_kernels import ops
    x = torch.randn(4, 256, device=dev).to(torch.float8_e4m3fn)
    ids = torch.zeros(4, 2, dtype=torch.int64, device=dev)
    fs = torch.ones(4, 2, device=dev)
    ws = torch.empty(64, dtype=torch.uint8, device=dev)
    sc = torch.ones(4, 2, device=dev)
    with pytest.raises(RuntimeError, match="smaller than the prologue layout"):
        ops.fused_moe_prologue(x, sc, ids, fs, ws, 256, 512, 128, 0, 1, 16)
    with pytest.raises(RuntimeError, match="need input_scales"):
        ops.fused_moe_prologue(x, None, ids, fs, ws, 256, 512, 128, 0, 1, 16)
    with pytest.raises(RuntimeError, match="hidden_size / block_k"):
        ops.fused_moe_prologue(x, sc, ids, fs, ws, 256, 512, 32, 0, 1, 16)
