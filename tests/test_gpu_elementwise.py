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


# reference tests/test_activation.py:13-15 shapes, plus an odd d (scalar path)
@pytest.mark.parametrize("rows,d", [(7, 512), (83, 13824), (2048, 512), (3, 1000)])
@pytest.mark.parametrize("dt", DT)
@pytest.mark.parametrize("act", ["gelu", "gelu_tanh", "swiglustep", "relu2"])
def test_gelu_swiglustep_relu2(dev, rows, d, dt, act):
    scale = 4.0 if act == "swiglustep" else 1.0
    x = (torch.randn(rows, 2 * d, generator=torch.Generator().manual_seed(d + rows)) * scale).to(dt)
    ops = _ops()
    if act == "gelu":
        y, ref = ops.gelu_and_mul(x.to(dev)), O.gelu_and_mul(x)
    elif act == "gelu_tanh":
        y, ref = ops.gelu_tanh_and_mul(x.to(dev)), O.gelu_and_mul(x, "tanh")
    elif act == "swiglustep":
        y, ref = ops.swiglustep_and_mul(x.to(dev), 3.0), O.swiglustep_and_mul(x, 3.0)
    else:
        y, ref = ops.relu2_no_mul(x.to(dev)), O.relu2_no_mul(x)
    rtol, atol = _tol(dt)
    if act == "relu2":
        assert torch.equal(y.cpu(), ref)     # one product, one rounding
    else:
        torch.testing.assert_close(y.cpu(), ref, rtol=rtol, atol=atol)


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


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [0, -3, 5])
def test_mxfp4_quant_every_16bit_value(dev, dt, k):
    """Every finite 16-bit value of magnitude <= 6, in groups of 32 led by a 6
    (group scale 1), times 2^k (scale 2^k): the device's e2m1 codes for
    16-bit input (the hardware conversion, round to nearest even, after the
    operands are moved 2^-12 of themselves toward zero) equal the oracle's
    strict-midpoint rounding -- every midpoint tie, values that round to a
    signed zero, and -0 included."""
    x = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(dt).float()
    x = x[torch.isfinite(x) & (x.abs() <= 6)]
    pad = (-x.numel()) % 31
    x = torch.cat([x, torch.zeros(pad)]).reshape(-1, 31)
    x = torch.cat([torch.full((x.shape[0], 1), 6.0), x], dim=1)
    x = (x * 2.0 ** k).to(dt)
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


# ------------------------------------------- fused SiLU-and-mul + quantisers
# Shapes of the reference's tests (tests/test_fused_silu_mul_block_quant.py:
# 16-26, tests/test_fused_silu_mul_mxfp4_quant.py:11-19), hidden % group == 0.
BQ_SHAPES = [(1, 64), (1, 1024), (1, 2048), (1, 5120), (16, 64), (16, 1024), (16, 5120),
             (128, 64), (128, 1024), (512, 64), (512, 5120)]
QDT = [torch.float8_e4m3fn, torch.float8_e5m2, torch.int8]
_STEP = {torch.float8_e4m3fn: (0.125, 2.0 ** -9), torch.float8_e5m2: (0.25, 2.0 ** -16),
         torch.int8: (0.0, 1.0)}


def _gate_up(T, H, seed, dt, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, 2 * H, generator=g) * scale).to(dt)


def _assert_block_quant_close(q, s, qr, sr, qdt):
    """The GPU's exp and the CPU oracle's may differ by an ulp, so a group's
    amax, and with it its scale, by a few ulp and a code sitting on a
    rounding boundary by one step: scales within rtol 1e-6, at least 99.9 %
    of the codes identical and every code within one step of the oracle's
    (relative 1/8 for e4m3, 1/4 for e5m2 above their subnormal steps; one
    unit for int8)."""
    s = s.cpu().contiguous()
    torch.testing.assert_close(s, sr, rtol=1e-6, atol=0)
    qb, qrb = q.cpu().view(torch.uint8), qr.view(torch.uint8)
    assert (qb == qrb).float().mean().item() >= 0.999
    qf, qrf = q.cpu().float(), qr.float()
    rel, sub = _STEP[qdt]
    assert torch.all((qf - qrf).abs() <= torch.maximum(qrf.abs() * rel, torch.tensor(sub)) * 1.001)


@pytest.mark.parametrize("T,H", BQ_SHAPES)
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("qdt", QDT)
def test_silu_and_mul_per_block_quant(dev, T, H, group, transposed, qdt):
    if H % group:
        pytest.skip("hidden_size not divisible by group_size (the op rejects it)")
    x = _gate_up(T, H, 31 * T + H, torch.bfloat16)
    q, s = _ops().silu_and_mul_per_block_quant(x.to(dev), group, qdt, None, transposed)
    assert q.dtype == qdt and q.shape == (T, H) and s.shape == (T, H // group)
    if transposed:
        assert s.stride() == (1, T)
    qr, sr = O.silu_and_mul_per_block_quant(x, group, qdt)
    _assert_block_quant_close(q, s, qr, sr, qdt)


@pytest.mark.parametrize("T,H", [(1, 1024), (16, 5120), (128, 64)])
@pytest.mark.parametrize("qdt", QDT)
def test_silu_and_mul_per_block_quant_fp16_and_reference_scale(dev, T, H, qdt):
    """fp16 input, and the reference test's data scale (x / hidden), which
    puts the fp8 scales on their 1/(qmax*512) floor."""
    for scale in (1.0, 1.0 / H):
        x = _gate_up(T, H, 7 * T + H, torch.float16, scale)
        q, s = _ops().silu_and_mul_per_block_quant(x.to(dev), 64, qdt)
        qr, sr = O.silu_and_mul_per_block_quant(x, 64, qdt)
        _assert_block_quant_close(q, s, qr, sr, qdt)


@pytest.mark.parametrize("qdt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_silu_and_mul_per_block_quant_scale_ub_ue8m0(dev, qdt):
    x = _gate_up(64, 1024, 5, torch.bfloat16)
    _, sr = O.silu_and_mul_per_block_quant(x, 128, qdt)
    ub = float(sr.median())
    q, s = _ops().silu_and_mul_per_block_quant(
        x.to(dev), 128, qdt, torch.tensor([ub], device=dev))
    qr, sr2 = O.silu_and_mul_per_block_quant(x, 128, qdt, scale_ub=ub)
    _assert_block_quant_close(q, s, qr, sr2, qdt)
    assert (s.cpu() == ub).float().mean().item() >= 0.4
    q, s = _ops().silu_and_mul_per_block_quant(x.to(dev), 128, qdt, None, False, True)
    qr, sr3 = O.silu_and_mul_per_block_quant(x, 128, qdt, scale_ue8m0=True)
    assert (s.cpu() == sr3).float().mean().item() >= 0.999
    m, _ = torch.frexp(s.cpu())
    assert torch.all(m == 0.5)


@pytest.mark.parametrize("B", [1, 16, 256])
@pytest.mark.parametrize("H", [1024, 5120, 14336])
def test_silu_and_mul_per_block_quant_edge_cases(dev, B, H):
    """Reference edge-case shapes (tests/test_fused_silu_mul_block_quant.py:
    165-190): unit-variance fp16, group 128, finite outputs, oracle parity."""
    x = _gate_up(B, H, B + H, torch.float16)
    q, s = _ops().silu_and_mul_per_block_quant(x.to(dev), 128, torch.float8_e4m3fn)
    assert not torch.isnan(q.float()).any() and torch.isfinite(s).all()
    qr, sr = O.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn)
    _assert_block_quant_close(q, s, qr, sr, torch.float8_e4m3fn)


def _nibbles(q):
    q = q.cpu()
    return torch.stack([q & 0xF, q >> 4], -1).reshape(q.shape[0], -1).long()


@pytest.mark.parametrize("T", [1, 7, 83, 2048])
@pytest.mark.parametrize("H", [128, 1024, 5120])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
def test_silu_and_mul_mxfp4_quant(dev, T, H, dt, transposed):
    """Scales are powers of two equal to the oracle's except where an ulp of
    exp moves amax/6 across a power of two (then a factor of 2, and that
    group's codes are not compared); at least 99.9 % of the codes identical,
    the rest one e2m1 step away with the same sign."""
    x = _gate_up(T, H, 13 * T + H, dt)
    G = H // 32
    q = torch.empty(T, H // 2, dtype=torch.uint8, device=dev)
    s = (torch.empty(G, T, dtype=torch.float32, device=dev).t() if transposed
         else torch.empty(T, G, dtype=torch.float32, device=dev))
    torch.ops._C.silu_and_mul_mxfp4_quant(q, x.to(dev), s, 32, 1e-10)
    qr, sr = O.silu_and_mul_mxfp4_quant(x)
    s = s.cpu().contiguous()
    same = s == sr
    assert same.float().mean().item() >= 0.999
    assert torch.all(torch.where(same, torch.ones_like(s), s / sr).log2().abs() <= 1)
    c, cr = _nibbles(q), _nibbles(qr)
    keep = same.repeat_interleave(32, dim=1)
    assert (c[keep] == cr[keep]).float().mean().item() >= 0.999
    d = c[keep] - cr[keep]
    assert torch.all((d.abs() <= 1) & ((c[keep] >> 3) == (cr[keep] >> 3)) | (d == 0))


def test_fused_quant_validation_messages(dev):
    x = torch.randn(4, 256, device=dev).bfloat16()
    q = torch.empty(4, 128, device=dev, dtype=torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="group_size must be 32, 64, or 128"):
        torch.ops._C.silu_and_mul_per_block_quant(q, x, torch.empty(4, 3, device=dev), 48)
    with pytest.raises(RuntimeError, match="out must be float8_e4m3fn, float8_e5m2, or int8"):
        torch.ops._C.silu_and_mul_per_block_quant(
            torch.empty(4, 128, device=dev, dtype=torch.bfloat16), x,
            torch.empty(4, 2, device=dev), 64)
    with pytest.raises(RuntimeError, match="scale_ub is only supported for FP8 output"):
        torch.ops._C.silu_and_mul_per_block_quant(
            q.view(torch.int8), x, torch.empty(4, 2, device=dev), 64,
            torch.ones(1, device=dev))
    with pytest.raises(RuntimeError, match="scales must have logical shape"):
        torch.ops._C.silu_and_mul_per_block_quant(q, x, torch.empty(4, 3, device=dev), 64)
    with pytest.raises(RuntimeError, match="scales must be row-major"):
        torch.ops._C.silu_and_mul_per_block_quant(
            q, x, torch.empty(4, 2, device=dev), 64, None, True)
    with pytest.raises(RuntimeError, match="MXFP4 requires group_size == 32"):
        torch.ops._C.silu_and_mul_mxfp4_quant(
            torch.empty(4, 64, device=dev, dtype=torch.uint8), x, torch.empty(4, 2, device=dev), 64)
