"""GPU parity of NF-aware (sigma-based) per-tensor scaling against the oracle.

The reference's ``to_fp8_e4m3_nf_aware`` (tcfp/core.py:161-193) and the NF
branches of the tensor-core forward (tcfp/nn/__init__.py:263-275, 356-359).
Codes, scales and error buffers are compared bit for bit.  The std is the
real one rounded once to fp32 on both sides (fp64 sums here, a float64
two-pass in the oracle): the two agree unless the real std lies within about
1e-16 (relative) of an fp32 rounding boundary, which none of the seeded
inputs below does.  Stochastic W_hi codes are checked against the candidate
pair and for consistency of everything computed from them.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import quant as oq
from tcfp_amd import kernels as K
from tcfp_amd.core import ErrorFeedbackState, to_fp8_e4m3_nf_aware
from tcfp_amd.nn import TCFPLinear

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def f32bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _weight(shape, seed, kind):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(shape, generator=g) * 0.02
    if kind == "outliers":
        W.view(-1)[:: max(1, W.numel() // 7)] *= 40.0
    elif kind == "shifted":
        W = W * 0.05 + 3.0  # mean far above the spread
    elif kind == "constant":
        W = torch.full(shape, -0.375)
    return W


# ------------------------------------------------------ codes and scales
CASES = [((s, k)) for s in [(1, 7), (33, 1000), (256, 512)]
         for k in ["gauss", "outliers", "shifted", "constant"]] + [((4096, 1024), "gauss")]


@pytest.mark.parametrize("shape,kind", CASES)
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_nf_dual_quant_matches_oracle(dev, shape, wdt, kind):
    W = _weight(shape, sum(shape), kind).to(wdt)
    Wf = W.float().numpy()
    g = torch.Generator().manual_seed(7)
    ef0 = (torch.randn(shape, generator=g) * 1e-4).numpy()
    transposed = shape[1] % 8 == 0
    for sigma in (3.0, 2.2):
        ef_d = torch.from_numpy(ef0.copy()).to(dev)
        res = K.dual_quantize_per_tensor(W.to(dev), ef_d, transposed=transposed,
                                         sigma_factor=sigma)
        hi, lo, ih, il, ef_new, _ = oq.dual_quant_per_tensor(Wf, ef0, sigma_factor=sigma)
        tag = f"{shape} {wdt} {kind} sigma={sigma}"
        assert res[2].item() == float(ih) or (np.isnan(ih) and np.isnan(res[2].item())), tag
        assert res[3].item() == float(il) or (np.isnan(il) and np.isnan(res[3].item())), tag
        assert np.array_equal(u8(res[0]), hi), tag
        assert np.array_equal(u8(res[1]), lo), tag
        assert np.array_equal(f32bits(ef_d.cpu().numpy()), f32bits(ef_new)), tag
        if transposed:
            assert np.array_equal(u8(res[4]), hi.T) and np.array_equal(u8(res[5]), lo.T), tag


def test_nf_scale_differs_from_amax_rule(dev):
    # on Gaussian data 3 sigma sits well below the amax: the NF scale is
    # larger, and the outliers saturate at +-448 in W_hi
    W = _weight((512, 512), 3, "outliers").to(dev)
    _, _, ih_nf, _ = K.dual_quantize_per_tensor(W, None, sigma_factor=3.0)
    _, _, ih, _ = K.dual_quantize_per_tensor(W, None)
    assert ih_nf.item() < ih.item() / 10
    h, _, _, _ = K.dual_quantize_per_tensor(W, None, sigma_factor=3.0)
    assert (u8(h) & 0x7F == 0x7E).sum() >= 7


def test_nf_multi_step_ef_and_nan(dev):
    shape = (300, 200)
    W = _weight(shape, 9, "gauss")
    ef_d = torch.zeros(shape, device=dev)
    ef_o = np.zeros(shape, np.float32)
    g = torch.Generator().manual_seed(10)
    for step in range(4):
        res = K.dual_quantize_per_tensor(W.to(dev), ef_d, sigma_factor=3.0)
        hi, lo, ih, il, ef_new, _ = oq.dual_quant_per_tensor(W.numpy(), ef_o, sigma_factor=3.0)
        assert np.array_equal(u8(res[0]), hi) and np.array_equal(u8(res[1]), lo), step
        assert res[2].item() == float(ih) and res[3].item() == float(il), step
        assert np.array_equal(f32bits(ef_d.cpu().numpy()), f32bits(ef_new)), step
        ef_o = ef_new
        W = W + torch.randn(shape, generator=g) * 0.003
    # a NaN makes the std, and so the scale, NaN (torch.std propagates it)
    Wn = W.clone()
    Wn[5, 5] = float("nan")
    _, _, ih, _ = K.dual_quantize_per_tensor(Wn.to(dev), None, sigma_factor=3.0)
    assert torch.isnan(ih).all()
    with pytest.raises(RuntimeError, match="empty"):
        K.dual_quantize_per_tensor(torch.empty(0, 16, device=dev), None, sigma_factor=3.0)


@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(256, 512), (33, 1000)])
def test_nf_delayed_matches_oracle_over_steps(dev, wdt, shape):
    state = ErrorFeedbackState(ema_decay=0.9, residual_validation_interval=3)
    ost = oq.new_delayed_state()
    g = torch.Generator().manual_seed(sum(shape) + 1)
    W = torch.randn(shape, generator=g) * 0.02
    ef_dev = torch.zeros(shape, device=dev)
    ef_np = np.zeros(shape, np.float32)
    transposed = shape[1] % 8 == 0
    for step in range(7):
        Wd = W.to(wdt)
        res = K.dual_quantize_per_tensor_delayed(Wd.to(dev), ef_dev, state, "lin",
                                                 transposed=transposed, sigma_factor=3.0)
        hi, lo, ih, il, ef_new, val = oq.dual_quant_per_tensor_delayed(
            Wd.float().numpy(), ef_np, ost, "lin", decay=0.9, interval=3, sigma_factor=3.0)
        tag = f"step {step} validated={val}"
        assert np.array_equal(u8(res[0]), hi), tag
        assert np.array_equal(u8(res[1]), lo), tag
        assert res[2].item() == float(ih) and res[3].item() == float(il), tag
        assert np.array_equal(f32bits(ef_dev.cpu().numpy()), f32bits(ef_new)), tag
        assert state._delayed_amax["lin.w_hi"].item() == float(ost["amax"]["lin.w_hi"]), tag
        assert state._residual_ratio["lin.ratio"].item() == float(ost["ratio"]["lin.ratio"]), tag
        if transposed:
            assert np.array_equal(u8(res[4]), hi.T) and np.array_equal(u8(res[5]), lo.T), tag
        ef_np = ef_new
        W = W + torch.randn(shape, generator=g) * 0.004


# --------------------------------------------------- stochastic W_hi codes
@pytest.mark.parametrize("shape", [(128, 256), (37, 101)])
def test_nf_stochastic_hi_candidates_and_consistency(dev, shape):
    W = _weight(shape, 4, "gauss")
    Wn = W.numpy()
    _, _, ih_o, _, _, _ = oq.dual_quant_per_tensor(Wn, None, sigma_factor=3.0)
    scale = oq._scale_of(oq.nf_target(Wn, 3.0))
    x = np.clip(Wn * scale, -448, 448).astype(np.float32)
    lo_c, hi_c, frac, exact = oq.sr_candidates_per_tensor(x)
    transposed = shape[1] % 8 == 0
    acc = np.zeros(x.shape, np.float64)
    n = 100
    for i in range(n):
        ef = torch.zeros(shape, device=dev)
        res = K.dual_quantize_per_tensor(W.to(dev), ef, sigma_factor=3.0, stochastic_hi=True,
                                         seed=500 + i, transposed=transposed)
        h = u8(res[0])
        assert res[2].item() == float(ih_o)
        assert np.all((h == lo_c) | (h == hi_c)), "SR picked a code outside the candidate pair"
        assert np.all(h[exact] == lo_c[exact])
        # W_lo, its scale and the EF are the deterministic functions of the
        # stochastic W_hi codes (the residual pass recomputes the same draws)
        res_o = (Wn - ofp8.decode(h, ofp8.E4M3) * res[2].item()).astype(np.float32)
        lo, il, _ = oq.to_fp8_per_tensor(res_o, "f32")
        assert np.array_equal(u8(res[1]), lo) and res[3].item() == float(il)
        ef_o = Wn - (ofp8.decode(h, ofp8.E4M3) * res[2].item() + ofp8.decode(lo, ofp8.E4M3) * il)
        assert np.array_equal(f32bits(ef.cpu().numpy()), f32bits(ef_o))
        if transposed:
            assert np.array_equal(u8(res[4]), h.T) and np.array_equal(u8(res[5]), lo.T)
        acc += (h == hi_c) & (hi_c != lo_c)
    p = acc / n
    m = ~exact & (hi_c != lo_c) & np.isfinite(frac)
    assert abs(float((p[m] - frac[m]).mean())) < 0.02
    # the same seed repeats; W_lo's stochastic rounding draws independently
    a = K.dual_quantize_per_tensor(W.to(dev), None, sigma_factor=3.0, stochastic_hi=True,
                                   seed=77)
    b = K.dual_quantize_per_tensor(W.to(dev), None, sigma_factor=3.0, stochastic_hi=True,
                                   seed=77)
    assert np.array_equal(u8(a[0]), u8(b[0])) and np.array_equal(u8(a[1]), u8(b[1]))
    c = K.dual_quantize_per_tensor(W.to(dev), None, sigma_factor=3.0, stochastic_hi=True,
                                   stochastic_lo=True, seed=77)
    assert np.array_equal(u8(a[0]), u8(c[0]))


def test_nf_stochastic_hi_under_delayed_two_pass(dev):
    # on predicted (non-validation) steps the residual pass writes W_hi
    # itself: its stochastic codes must be the ones a validation step draws
    shape = (64, 256)
    W = _weight(shape, 12, "gauss").to(dev)
    s1 = ErrorFeedbackState(ema_decay=0.0, residual_validation_interval=1000)
    s2 = ErrorFeedbackState(ema_decay=0.0, residual_validation_interval=1)
    for st in (s1, s2):
        K.dual_quantize_per_tensor_delayed(W, None, st, "w", sigma_factor=3.0)
    a = K.dual_quantize_per_tensor_delayed(W, None, s1, "w", sigma_factor=3.0,
                                           stochastic_hi=True, seed=5)
    b = K.dual_quantize_per_tensor_delayed(W, None, s2, "w", sigma_factor=3.0,
                                           stochastic_hi=True, seed=5)
    assert np.array_equal(u8(a[0]), u8(b[0])) and a[2].item() == b[2].item()


# ------------------------------------------------ to_fp8_e4m3_nf_aware
@pytest.mark.parametrize("shape", [(256, 256), (3, 5, 7), (1000,)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_to_fp8_e4m3_nf_aware_matches_oracle(dev, shape, dtype):
    g = torch.Generator().manual_seed(len(shape))
    x = torch.randn(shape, generator=g).to(dtype)
    q, inv = to_fp8_e4m3_nf_aware(x.to(dev))
    codes, inv_o, _ = oq.to_fp8_nf_aware(x.float().numpy(), 3.0)
    assert q.shape == x.shape and q.dtype == torch.float8_e4m3fn
    assert inv.shape == (1,) and inv.dtype == torch.float32
    assert np.array_equal(u8(q), codes) and inv.item() == float(inv_o)


def test_to_fp8_e4m3_nf_aware_reference_properties(dev):
    # tests/test_tensor_cores.py:27-68 upstream
    x = torch.randn(256, 256, device=dev)
    fp8, inv = to_fp8_e4m3_nf_aware(x)
    recon = fp8.float() * inv
    assert (x - recon).abs().mean() / x.abs().mean() < 0.15
    torch.manual_seed(42)
    x = torch.randn(1024, 1024, device=dev)
    fp8, inv = to_fp8_e4m3_nf_aware(x)
    assert (x - fp8.float() * inv).pow(2).mean().item() / x.pow(2).mean().item() < 0.01
    x = torch.randn(64, 64, device=dev)
    a, _ = to_fp8_e4m3_nf_aware(x, stochastic=True)
    b, _ = to_fp8_e4m3_nf_aware(x, stochastic=True)
    assert not torch.equal(a.float(), b.float())
    x = torch.ones(64, 64, device=dev) * 0.5
    fp8, inv = to_fp8_e4m3_nf_aware(x)
    assert torch.isfinite(inv).all() and torch.isfinite(fp8.float()).all()
    q, inv = to_fp8_e4m3_nf_aware(torch.empty(0, 4, device=dev))
    assert q.shape == (0, 4) and torch.isnan(inv).all()


# ------------------------------------------------------------- the layer
def test_nf_layer_forward_backward_and_training(dev):
    # tests/test_tcfp12_tensor_cores.py:396-405 upstream, plus parity of the
    # output with the fp64 product of the oracle's dequantised operands
    torch.manual_seed(0)
    layer = TCFPLinear(128, 64, use_tensor_cores=True, nf_aware_scaling=True).to(dev)
    assert "nf_aware_scaling=True" in repr(layer)
    x = torch.randn(8, 128, device=dev)
    w0 = layer.weight.detach().float().cpu().numpy()
    out = layer(x)
    assert out.shape == (8, 64) and torch.isfinite(out).all()
    hi, lo, ih, il, _, _ = oq.dual_quant_per_tensor(w0, np.zeros_like(w0), sigma_factor=3.0)
    xq, xinv, _ = oq.to_fp8_per_tensor(x.cpu().numpy(), "f32")
    wd = (ofp8.decode(hi, ofp8.E4M3).astype(np.float64) * ih
          + ofp8.decode(lo, ofp8.E4M3).astype(np.float64) * il)
    ref = (ofp8.decode(xq, ofp8.E4M3).astype(np.float64) * xinv) @ wd.T
    ref += layer.bias.detach().double().cpu().numpy()
    got = out.detach().double().cpu().numpy()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2
    out.sum().backward()
    assert torch.isfinite(layer.weight.grad).all()
    # a few SGD steps on a regression target reduce the loss, in every NF mode
    for kw in ({}, {"stochastic_rounding": True}, {"delayed_scaling": True}):
        torch.manual_seed(1)
        lin = TCFPLinear(256, 128, use_tensor_cores=True, nf_aware_scaling=True, **kw).to(dev)
        xt = torch.randn(64, 256, device=dev)
        yt = xt @ (torch.randn(256, 128, device=dev) * 0.05)
        # the loss's curvature in W is about 2 * 256 / (64 * 128) = 1/16
        opt = torch.optim.SGD(lin.parameters(), lr=2.0)
        losses = []
        for _ in range(30):
            loss = (lin(xt) - yt).pow(2).mean()
            opt.zero_grad()
            loss.backward()
            opt.step()
            losses.append(loss.item())
        assert losses[-1] < 0.5 * losses[0], (kw, losses[0], losses[-1])
