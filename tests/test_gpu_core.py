"""GPU parity of the tcfp.core primitives beyond the per-tensor casts:
stochastic-rounding casts (to_fp8_e4m3_sr, stochastic_round_to_fp8_e4m3),
compute_block_scales and the FP8 matmuls (fp8_matmul, fp8_matmul_nn), all
reached through the reference's import names.

The SR random bits come from this build's Philox stream instead of
torch.rand_like, so SR parity is statistical, as in the reference's own
tests (tests/test_fused_dual_quant.py:494-526): every code is one of the
oracle's two candidates, exact values keep theirs, and the up-rounding rate
matches the oracle's probability.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import gemm as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


# ------------------------------------------------------------ SR casts
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 256), (37, 100), (1, 7)])
def test_to_fp8_e4m3_sr_candidates_scale_and_rate(dev, dtype, shape):
    from tcfp.core import to_fp8_e4m3, to_fp8_e4m3_sr

    g = torch.Generator().manual_seed(shape[0] * 1000 + shape[1])
    x = (torch.randn(shape, generator=g) * 3.0).to(dtype)
    xd = x.to(dev)
    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    scale = oq.per_tensor_scale(x.float().numpy(), dt)
    c = np.clip(x.float().numpy() * scale, -448, 448).astype(np.float32)
    lo, hi, frac, exact = oq.sr_candidates_per_tensor(c)
    _, inv_rne = to_fp8_e4m3(xd)
    n = 300
    ups = np.zeros(c.shape, np.float64)
    for _ in range(n):
        q, inv = to_fp8_e4m3_sr(xd)
        assert q.dtype == torch.float8_e4m3fn and q.shape == x.shape
        assert inv.shape == (1,) and inv.item() == inv_rne.item()
        code = u8(q)
        assert np.all((code == lo) | (code == hi)), "code outside the candidate pair"
        assert np.all(code[exact] == lo[exact])
        ups += (code == hi) & (hi != lo)
    m = ~exact & (hi != lo) & np.isfinite(frac)
    p = ups[m] / n
    # binomial z-test of the pooled up-rounding count against sum(frac)
    var = float((frac[m] * (1 - frac[m])).sum()) * n
    z = (float(ups[m].sum()) - n * float(frac[m].sum())) / max(var, 1e-9) ** 0.5
    assert abs(z) < 5, z
    if p.size >= 1000:  # mean error of the per-element rates (sd ~0.03/sqrt(size))
        assert abs(float((p - frac[m]).mean())) < 0.01


def test_to_fp8_e4m3_sr_explicit_scale_and_empty(dev):
    from tcfp.core import to_fp8_e4m3_sr

    x = torch.ones(64, device=dev) * 100.0
    s = torch.tensor(448.0 / 100.0, device=dev)
    q, inv = to_fp8_e4m3_sr(x, scale=s)
    assert torch.allclose(q.float() * inv, x, atol=1.0)
    assert inv.item() == float(np.float32(1.0) / np.float32(448.0 / 100.0))
    q, inv = to_fp8_e4m3_sr(torch.empty(0, 16, device=dev))
    assert q.shape == (0, 16)
    assert inv.item() == float(oq.to_fp8_per_tensor(np.zeros((0, 16), np.float32))[1])


def test_stochastic_round_to_fp8_e4m3_unbiased(dev):
    """E[dequant(SR(x))] = x within 10% over 500 draws (the reference's own
    bar, tests/test_fused_dual_quant.py:494-526), codes always candidates."""
    from tcfp.core import stochastic_round_to_fp8_e4m3

    g = torch.Generator().manual_seed(5)
    x = torch.empty(4096).uniform_(-400, 400, generator=g)
    x[:64] = torch.tensor(ofp8.DECODE[ofp8.E4M3][:64])  # exact codes stay
    lo, hi, frac, exact = oq.sr_candidates_per_tensor(x.numpy())
    xd = x.to(dev)
    acc = torch.zeros_like(xd, dtype=torch.float64)
    for _ in range(500):
        q = stochastic_round_to_fp8_e4m3(xd)
        c = u8(q)
        assert np.all((c == lo) | (c == hi))
        assert np.all(c[exact] == lo[exact])
        acc += q.double()
    mean = (acc / 500).cpu().numpy()
    xs = x.numpy()
    gap = np.abs(ofp8.decode(hi, ofp8.E4M3) - ofp8.decode(lo, ofp8.E4M3))
    m = ~exact & np.isfinite(gap) & (gap > 0)
    # per element: the mean of 500 draws lies within 6 standard errors of x
    # (sd of one draw <= gap / 2), i.e. within ~0.13 gap; round-to-nearest
    # would miss by |x - lo|, up to gap / 2
    assert np.all(np.abs(mean[m] - xs[m]) <= 6 * 0.5 * gap[m] / np.sqrt(500))
    assert np.all(mean[exact] == xs[exact])
    # and no drift across elements
    assert abs(float(((mean[m] - xs[m]) / gap[m]).mean())) < 0.01


# ------------------------------------------------------------ block scales
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bs", [16, 32, 64, 128])
@pytest.mark.parametrize("fm", [448.0, 57344.0])
def test_compute_block_scales_bitexact(dev, dtype, bs, fm):
    from tcfp.core import compute_block_scales

    g = torch.Generator().manual_seed(bs)
    x = torch.randn(3, 40, 256, generator=g) * torch.exp2(torch.randint(-60, 60, (3, 40, 1),
                                                                          generator=g).float())
    x[0, 0] = 0.0
    x[0, 1] = 1e-20
    x[1, 2, 5] = float("nan")
    x[2, 3, 7] = float("inf")
    x = x.to(dtype)
    s = compute_block_scales(x.to(dev), bs, fm)
    assert s.dtype == dtype and s.shape == (3, 40, 256 // bs)
    ref = oq.compute_block_scales(x.float().numpy(), bs, fm, "bf16" if dtype == torch.bfloat16
                                  else "f32")
    assert np.array_equal(s.float().cpu().numpy(), ref, equal_nan=True)


def test_compute_block_scales_every_bf16_quotient(dev):
    """With fp8_max = 1 and one-element blocks the quotient is the element:
    every positive finite bf16 value goes through the bf16 log2 rounding."""
    from tcfp.core import compute_block_scales

    bits = np.arange(1, 0x7F80, dtype=np.uint32)
    q = (bits << 16).view(np.float32)
    x = torch.from_numpy(q.copy()).bfloat16().reshape(-1, 1)
    s = compute_block_scales(x.to(dev), 1, 1.0).float().cpu().numpy().ravel()
    ref = oq.compute_block_scales(q.reshape(-1, 1), 1, 1.0, "bf16").ravel()
    assert np.array_equal(s, ref)


# ------------------------------------------------------------ FP8 matmuls
@pytest.mark.parametrize("mkn", [(64, 128, 32), (32, 64, 16), (300, 256, 208)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_fp8_matmul_matches_dequant_matmul(dev, mkn, out_dtype):
    from tcfp.core import fp8_matmul, fp8_matmul_nn, to_fp8_e4m3

    M, K, N = mkn
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(K, N, generator=g)
    a8, sa = to_fp8_e4m3(a.to(dev))
    b8, sb = to_fp8_e4m3(b.to(dev))
    ref = og.gemm_nt(u8(a8), ofp8.E4M3, u8(b8).T.copy(), ofp8.E4M3, float(sa.item()),
                     float(sb.item()))
    tol = 1e-4 if out_dtype == torch.float32 else 5e-3
    out = fp8_matmul(a8, b8, sa, sb, out_dtype=out_dtype)
    assert out.shape == (M, N) and out.dtype == out_dtype
    assert og.rel_fro(out.float().cpu().numpy(), ref) < tol
    # column-major B is used without a copy, same result
    b_cm = b8.t().contiguous().t()
    assert torch.equal(fp8_matmul(a8, b_cm, sa, sb, out_dtype=out_dtype), out)
    # B given transposed
    assert torch.equal(fp8_matmul_nn(a8, b8.t().contiguous(), sa, sb, out_dtype=out_dtype), out)
    # the reference's own accuracy bar against the fp32 product
    exact = (a @ b).numpy()
    assert og.rel_fro(out.float().cpu().numpy(), exact) < 0.15


def test_fused_block_scaled_backward_dx_is_the_dispatcher(dev):
    from tcfp.kernels import (
        block_quantize_fp8,
        fused_block_scaled_backward_dx,
        fused_block_scaled_dual_gemm_backward_dx,
        fused_dual_quantize_fp8,
    )

    g = torch.Generator().manual_seed(9)
    W = (torch.randn(256, 384, generator=g) * 0.02).to(dev)
    G = torch.randn(128, 256, generator=g).to(dev)
    hi, lo, sh, sl = fused_dual_quantize_fp8(W, 64)
    g8, sg = block_quantize_fp8(G, 64, torch.float8_e5m2)
    a = fused_block_scaled_backward_dx(g8, hi, lo, sg, sh, sl, 64, persistent=False,
                                       launch_mult=2)
    b = fused_block_scaled_dual_gemm_backward_dx(g8, hi, lo, sg, sh, sl, 64)
    assert a.shape == (128, 384) and torch.equal(a, b)
    ref = og.block_dgrad(u8(g8), sg.cpu().numpy(), u8(hi), u8(lo), sh.cpu().numpy(),
                         sl.cpu().numpy(), 64)
    assert og.rel_fro(a.cpu().numpy(), ref) < 1e-4
