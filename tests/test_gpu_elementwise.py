"""GPU parity: activations, activation quantisers and top-k reductions."""
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _ops():
    from vllm_xpu_kernels import ops
    return ops


DT = [torch.float32, torch.bfloat16, torch.float16]


def _tol(dt):
    # one rounding of the element type (silu is rounded before the multiply,
    # so an ulp flip there can move the result by one more ulp)
    return {torch.float32: (2e-6, 1e-6), torch.bfloat16: (1.6e-2, 1e-3),
            torch.float16: (2e-3, 1e-4)}[dt]


@pytest.mark.parametrize("rows,d", [(7, 1024), (64, 768), (3, 1000), (1, 2880)])
@pytest.mark.parametrize("dt", DT)
def test_silu_and_mul(dev, rows, d, dt):
    x = torch.randn(rows, 2 * d, generator=torch.Generator().manual_seed(d)).to(dt)
    y = _ops().silu_and_mul(x.to(dev)).cpu()
    rtol, atol = _tol(dt)
    torch.testing.assert_close(y, O.silu_and_mul(x), rtol=rtol, atol=atol)


@pytest.mark.parametrize("rows,d", [(7, 1024), (33, 2880)])
@pytest.mark.parametrize("dt", DT)
def test_swigluoai_and_mul(dev, rows, d, dt):
    x = (torch.randn(rows, 2 * d, generator=torch.Generator().manual_seed(d)) * 4).to(dt)
    y = _ops().swigluoai_and_mul(x.to(dev)).cpu()
    rtol, atol = _tol(dt)
    torch.testing.assert_close(y, O.swigluoai_and_mul(x), rtol=rtol, atol=atol)


@pytest.mark.parametrize("rows,cols,group", [(1, 7168, 128), (64, 2048, 128),
                                             (5, 256, 32), (3, 512, 64)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ue8m0", [False, True])
def test_per_token_group_fp8_quant_bit_exact(dev, rows, cols, group, dt, ue8m0):
    x = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(cols)) * 3).to(dt)
    x[0, :group] = 0.0                      # all-zero group -> minimum scale
    q, s = _ops().per_token_group_fp8_quant(x.to(dev), group, scale_ue8m0=ue8m0)
    rq, rs = O.per_token_group_fp8_quant(x, group, scale_ue8m0=ue8m0)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))


def test_fp8_quant_every_e4m3_code(dev):
    """The device e4m3 encoder reproduces all 254 finite codes and rounds
    midpoints to even like torch's conversion."""
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    row = torch.cat([vals[:127], torch.tensor([448.0]), vals[127:], torch.tensor([448.0])])
    q, s = _ops().per_token_group_fp8_quant(row.unsqueeze(0).to(dev), 128)
    assert torch.equal(q.cpu().view(torch.uint8)[0, :127], codes[:127])
    # random values with scale 1: device rounding == torch RNE
    x = torch.randn(16, 128, generator=torch.Generator().manual_seed(3)) * 100
    x[:, 0] = 448.0
    q, s = _ops().per_token_group_fp8_quant(x.to(dev), 128)
    assert torch.equal(q.cpu().view(torch.uint8), x.to(torch.float8_e4m3fn).view(torch.uint8))


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 2880), (64, 4096)])
def test_per_token_group_quant_mxfp4_bit_exact(dev, rows, cols):
    x = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(rows)) * 2).to(torch.bfloat16)
    q, s = _ops().per_token_group_quant_mxfp4(x.to(dev))
    rq, rs = O.per_token_group_quant_mxfp4(x)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(q.cpu().view(torch.uint8), rq)


@pytest.mark.parametrize("val", [0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
def test_mxfp4_known_values(dev, val):
    x = torch.zeros(1, 32)
    x[0, 0] = val
    q, s = _ops().per_token_group_quant_mxfp4(x.to(dev))
    rq, rs = O.per_token_group_quant_mxfp4(x)
    assert torch.equal(s.cpu(), rs) and torch.equal(q.cpu().view(torch.uint8), rq)


@pytest.mark.parametrize("m,topk,k", [(1, 2, 128), (33, 8, 511), (222, 4, 1024)])
@pytest.mark.parametrize("dt", DT)
def test_moe_sum(dev, m, topk, k, dt):
    x = torch.randn(m, topk, k, generator=torch.Generator().manual_seed(m)).to(dt)
    out = torch.empty(m, k, dtype=dt, device=dev)
    _ops().moe_sum(x.to(dev), out)
    torch.testing.assert_close(out.cpu(), O.moe_sum(x), rtol=1e-5 if dt == torch.float32 else 8e-3, atol=1e-5)


@pytest.mark.parametrize("dt", DT)
def test_moe_sum_expert_map_and_padding(dev, dt):
    m, topk, k, E = 33, 4, 256, 8
    g = torch.Generator().manual_seed(9)
    x = torch.randn(m, topk, k, generator=g).to(dt)
    ids = torch.randint(0, E, (m, topk), generator=g, dtype=torch.int32)
    ids[:, -1] = -1
    em = torch.arange(E, dtype=torch.int32)
    em[E // 2:] = -1
    out = torch.empty(m, k, dtype=dt, device=dev)
    _ops().moe_sum(x.to(dev), out, ids.to(dev), em.to(dev))
    torch.testing.assert_close(out.cpu(), O.moe_sum(x, ids, em),
                               rtol=1e-5 if dt == torch.float32 else 8e-3, atol=1e-5)


def test_moe_sum_validation_messages(dev):
    x = torch.randn(4, 2, 128, device=dev)
    with pytest.raises(RuntimeError, match="expert_map requires topk_ids"):
        _ops().moe_sum(x, torch.empty(4, 128, device=dev), None,
                       torch.zeros(8, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="same dtype"):
        _ops().moe_sum(x, torch.empty(4, 128, device=dev, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="num_tokens, topk"):
        _ops().moe_sum(x, torch.empty(4, 128, device=dev),
                       torch.zeros(4, 3, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="expert_map must be int32"):
        _ops().moe_sum(x, torch.empty(4, 128, device=dev),
                       torch.zeros(4, 2, dtype=torch.int32, device=dev),
                       torch.zeros(8, dtype=torch.int64, device=dev))


@pytest.mark.parametrize("T,k,H", [(1, 8, 7168), (64, 2, 512), (100, 4, 2880)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_moe_gather(dev, T, k, H, dt):
    g = torch.Generator().manual_seed(T * k)
    src = torch.randn(T * k, H, generator=g).to(dt)
    w = torch.rand(T, k, generator=g)
    perm = torch.randperm(T * k, generator=g).reshape(T, k).int()
    perm[0, 0] = -1
    out = torch.empty(T, H, dtype=dt, device=dev)
    _ops().moe_gather(out, src.to(dev), w.to(dev), perm.to(dev), 8)
    torch.testing.assert_close(out.cpu(), O.moe_gather(src, w, perm),
                               rtol=1e-5 if dt == torch.float32 else 8e-3, atol=1e-5)
