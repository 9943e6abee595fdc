"""GPU tests of the producer-fused GELU quantisation and the fused MLP.

The fused path claims bit-identity, so every check here is ``torch.equal``
on raw bits:

* the GELU (erf form) and its gradient equal torch's on the GPU;
* the fused quantisation of gelu(h) / of the GELU's input gradient equals
  the plain per-tensor quantisation (codes, inverse scales, transposed codes,
  bias column sums) of torch's gelu(h) / gradient;
* ``TCFPMLP`` (TCFPLinear -> GELU -> TCFPLinear as one autograd node) gives
  the outputs, gradients and EF buffers of the plain sequence over several
  AdamW steps.
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import quant as oq
from tcfp_amd import kernels as K
from tcfp_amd.nn import TCFPLinear, TCFPMLP, convert_to_tcfp, fuse_tcfp_mlp

pytestmark = pytest.mark.gpu


def bits(t):
    t = t.contiguous()
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.uint8)


def same_scalar(a, b):
    a, b = float(a.item()), float(b.item())
    return a == b or (a != a and b != b)


def _specials(t):
    v = torch.tensor([0.0, -0.0, -0.7518, 10.0, -10.0, 1e-30, 3.5, -3.5])
    n = min(v.numel(), t.numel())
    t.view(-1)[:n] = v[:n]
    return t


@pytest.mark.parametrize("shape", [(8192, 4096), (300, 208), (33, 130), (5, 3), (1, 8), (0, 64)])
def test_gelu_quantize_equals_torch_gelu_then_quantize(dev, shape):
    print(f"gelu quant {shape}", flush=True)
    g = torch.Generator().manual_seed(shape[0] * 7 + shape[1])
    h = _specials(torch.randn(shape, generator=g) * 3).to(dev)
    dg_ok = shape[-1] % 8 == 0
    res = K.gelu_quantize_per_tensor(h, transpose=True, return_act=True, return_dgelu=dg_ok)
    q, inv, q_t, act = res[:4]
    ref = F.gelu(h)
    assert torch.equal(bits(act), bits(ref))
    q2, inv2, q2_t = K.quantize_per_tensor(ref, transpose=True)
    assert torch.equal(bits(q), bits(q2)) and torch.equal(bits(q_t), bits(q2_t))
    assert same_scalar(inv, inv2)
    # and directly against the oracle's to_fp8_e4m3 of torch's gelu(h)
    if ref.numel() and torch.isfinite(ref).all():
        oc, oinv, _ = oq.to_fp8_per_tensor(ref.cpu().numpy(), "f32")
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oc)
        assert np.array_equal(q_t.view(torch.uint8).cpu().numpy(), oc.T)
        assert float(inv.item()) == float(oinv)
    if dg_ok:
        # torch's GELU backward is dy * (derivative factor), bit for bit
        dy = torch.randn(shape, generator=g).to(dev)
        hr = h.clone().requires_grad_(True)
        F.gelu(hr).backward(dy)
        assert torch.equal(bits(dy * res[-1]), bits(hr.grad))
        # and without act the same codes
        q3, inv3 = K.gelu_quantize_per_tensor(h)
        assert torch.equal(bits(q3), bits(q)) and same_scalar(inv3, inv)


@pytest.mark.parametrize("shape", [(8192, 4096), (300, 208), (8, 8), (1000, 24), (0, 64)])
def test_gelu_backward_quantize_colsum_equals_torch(dev, shape):
    print(f"gelu bwd quant {shape}", flush=True)
    g = torch.Generator().manual_seed(shape[0] + 11 * shape[1])
    h = _specials(torch.randn(shape, generator=g) * 3).to(dev)
    dy = (torch.randn(shape, generator=g) * 1e-3).to(dev)
    hr = h.clone().requires_grad_(True)
    F.gelu(hr).backward(dy)
    ref = hr.grad
    q, inv, q_t, cs, gr = K.gelu_backward_quantize_per_tensor_colsum(
        dy, h, transpose=True, return_grad=True)
    assert torch.equal(bits(gr), bits(ref))
    q2, inv2, q2_t, cs2 = K.quantize_per_tensor_colsum(ref, torch.float8_e5m2, transpose=True)
    assert torch.equal(bits(q), bits(q2)) and torch.equal(bits(q_t), bits(q2_t))
    assert same_scalar(inv, inv2)
    assert torch.equal(bits(cs), bits(cs2))
    # and directly against the oracle: to_fp8_e5m2 of torch's GELU backward,
    # and the column sums in this build's fixed order
    if ref.numel():
        r = ref.cpu().numpy()
        oc, oinv, _ = oq.to_fp8_per_tensor(r, "f32", "e5m2")
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oc)
        assert float(inv.item()) == float(oinv)
        assert np.array_equal(cs.cpu().numpy(), oq.column_sums(r))


def test_gelu_quantize_nan_propagates(dev):
    h = torch.randn(64, 64, device=dev)
    h[3, 5] = float("nan")
    q, inv = K.gelu_quantize_per_tensor(h)
    assert torch.isnan(inv).all()


def test_gelu_wrappers_reject_bad_inputs(dev):
    with pytest.raises(AssertionError, match="float32"):
        K.gelu_quantize_per_tensor(torch.randn(8, 8, device=dev).bfloat16())
    with pytest.raises(AssertionError, match="shape"):
        K.gelu_backward_quantize_per_tensor_colsum(torch.randn(8, 8, device=dev),
                                                   torch.randn(8, 16, device=dev))
    with pytest.raises(ValueError, match="divisible"):
        K.gelu_backward_quantize_per_tensor_colsum(torch.randn(8, 12, device=dev),
                                                   torch.randn(8, 12, device=dev))


# ------------------------------------ GELU and its amax in the GEMM epilogue
def _fp8_layer(dev, m, k, n, seed, a_dtype=torch.float8_e4m3fn):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * (1e-3 if a_dtype == torch.float8_e5m2 else 1.0)
    W = torch.randn(n, k, generator=g) * 0.05
    a, a_inv = K.quantize_per_tensor(x.to(dev), a_dtype)
    hi, lo, ih, il = K.dual_quantize_per_tensor(W.to(dev))
    return a, hi, lo, a_inv, ih, il


# (m, k, n): persistent launches (more 256 x 128 tiles than CUs, the C4
# layer shapes) and shapes that take the unfused fallback
EPI_SHAPES = [(4096, 256, 4096), (8192, 1024, 4096), (2048, 512, 4224), (300, 64, 208),
              (512, 256, 1024)]


def _bias_case(case, h0, n, dev):
    """Biases that steer the GELU amax rule: the rule holds ("normal"), or
    the device falls back to the full pass (every h negative, a NaN, a -inf,
    or max h so small that gelu(max h) is below the negative-side bound)."""
    g = torch.Generator().manual_seed(n)
    b = (torch.randn(n, generator=g) * 0.1).to(dev)
    if case == "all_negative":
        b = torch.full((n,), -1e4, device=dev)
    elif case == "nan":
        b[5] = float("nan")
    elif case == "neg_inf":
        b[7] = float("-inf")
    elif case == "small_max":
        b = torch.full((n,), -1e4, device=dev)
        b[3] = 0.1 - h0[:, 3].max()
    return b


@pytest.mark.parametrize("case", ["normal", "all_negative", "nan", "neg_inf", "small_max"])
@pytest.mark.parametrize("shape", EPI_SHAPES)
def test_dual_gemm_gelu_quantize_equals_unfused(dev, shape, case):
    m, k, n = shape
    if case != "normal" and m * n > 2**25:
        pytest.skip("fallback cases at the smaller shapes")
    print(f"gemm+gelu quant {shape} {case}", flush=True)
    a, hi, lo, a_inv, ih, il = _fp8_layer(dev, m, k, n, seed=m + k + n)
    h0 = K._dual_gemm(a, hi, lo, a_inv, ih, il, None, torch.float32)
    bias = _bias_case(case, h0, n, dev)
    h, q, inv, q_t, act, dg = K.dual_gemm_gelu_quantize(
        a, hi, lo, a_inv, ih, il, bias=bias, transpose=True, return_act=True, return_dgelu=True)
    h_ref = K._dual_gemm(a, hi, lo, a_inv, ih, il, bias, torch.float32)
    q2, inv2, q2_t, act2, dg2 = K.gelu_quantize_per_tensor(h_ref, transpose=True,
                                                            return_act=True, return_dgelu=True)
    assert torch.equal(bits(h), bits(h_ref))
    assert torch.equal(bits(act), bits(act2)) and torch.equal(bits(dg), bits(dg2))
    assert torch.equal(bits(q), bits(q2)) and torch.equal(bits(q_t), bits(q2_t))
    assert same_scalar(inv, inv2)
    # and against torch's GELU of the same h
    ref = F.gelu(h_ref)
    assert torch.equal(bits(act), bits(ref))
    q3, inv3 = K.quantize_per_tensor(ref)
    assert torch.equal(bits(q), bits(q3)) and same_scalar(inv, inv3)
    # without the optional outputs: the same codes
    h4, q4, inv4 = K.dual_gemm_gelu_quantize(a, hi, lo, a_inv, ih, il, bias=bias)
    assert torch.equal(bits(q4), bits(q)) and same_scalar(inv4, inv)


def test_gelu_amax_rule_premises_hold(dev):
    a, hi, lo, a_inv, ih, il = _fp8_layer(dev, 4096, 256, 4096, seed=0)
    K.dual_gemm_gelu_quantize(a, hi, lo, a_inv, ih, il)
    torch.cuda.synchronize()
    checked, holds, bound = K.gelu_amax_rule_status()
    print(f"gelu amax rule: checked={checked} holds={holds} T={bound!r}", flush=True)
    assert checked and holds
    # max |gelu| over the negatives: 0.16997 at x = -0.7518
    x = torch.linspace(-0.80, -0.70, 200001, device=dev)
    assert abs(bound - float(F.gelu(x).abs().max())) < 1e-6


@pytest.mark.parametrize("col_sum", [True, False])
@pytest.mark.parametrize("shape", EPI_SHAPES + [(1000, 128, 24)])
def test_dual_gemm_dgelu_quantize_colsum_equals_unfused(dev, shape, col_sum):
    m, k, n = shape
    print(f"dgrad+dgelu quant {shape} col_sum={col_sum}", flush=True)
    a, hi, lo, a_inv, ih, il = _fp8_layer(dev, m, k, n, seed=3 * m + k, a_dtype=torch.float8_e5m2)
    g = torch.Generator().manual_seed(m * 5 + n)
    h = _specials(torch.randn(m, n, generator=g) * 3).to(dev)
    dg = K.gelu_quantize_per_tensor(h, return_dgelu=True)[-1]
    res = K.dual_gemm_dgelu_quantize_colsum(a, hi, lo, a_inv, ih, il, dg, transpose=True,
                                            col_sum=col_sum, return_grad=True)
    dh = K._dual_gemm(a, hi, lo, a_inv, ih, il, None, torch.float32)
    hr = h.clone().requires_grad_(True)
    F.gelu(hr).backward(dh)
    g_ref = hr.grad
    # the gradient is torch's GELU backward of the dgrad output
    assert torch.equal(bits(res[-1]), bits(g_ref))
    q2, inv2, q2_t, cs2 = K.quantize_per_tensor_colsum(g_ref, torch.float8_e5m2, transpose=True)
    q, inv, q_t = res[:3]
    assert torch.equal(bits(q), bits(q2)) and torch.equal(bits(q_t), bits(q2_t))
    assert same_scalar(inv, inv2)
    if col_sum:
        assert torch.equal(bits(res[3]), bits(cs2))
        # the fixed summation order, restated on the CPU
        assert np.array_equal(res[3].cpu().numpy(), oq.column_sums(g_ref.cpu().numpy()))


def test_gemm_epilogue_replaces_the_gelu_passes_at_c4(dev):
    """At the C4 layer shapes the GELU's amax comes from the persistent
    GEMM's epilogue, and its backward, amax and bias partials from the dgrad
    GEMM's: no separate GELU or amax pass over h or its gradient runs."""
    a, hi, lo, a_inv, ih, il = _fp8_layer(dev, 8192, 1024, 4096, seed=1)
    fwd = lambda: K.dual_gemm_gelu_quantize(a, hi, lo, a_inv, ih, il, transpose=True,  # noqa: E731
                                            return_dgelu=True)
    fwd()
    torch.cuda.synchronize()  # the premise check has run
    names = _kernel_names(fwd)
    assert any("gemm_nt_persist_kernel<0, 0, float, 1, 0, 8, 128, false>" in n for n in names), names
    assert not any("gelu_amax_kernel" in n or "amax_part_kernel" in n for n in names), names
    g8, hi2, lo2, g_inv, ih2, il2 = _fp8_layer(dev, 8192, 1024, 4096, seed=2,
                                               a_dtype=torch.float8_e5m2)
    dg = torch.rand(8192, 4096, device=dev)
    names = _kernel_names(lambda: K.dual_gemm_dgelu_quantize_colsum(
        g8, hi2, lo2, g_inv, ih2, il2, dg, transpose=True))
    assert any("gemm_nt_persist_kernel<1, 0, float, 2, 0, 6, 64, false>" in n for n in names), names
    assert not any("amax" in n for n in names), names


def _pair(dev, d_in, d_h, d_out, bias=True, seed=0, **kw):
    torch.manual_seed(seed)
    base = nn.Sequential(nn.Linear(d_in, d_h, bias=bias), nn.GELU(),
                         nn.Linear(d_h, d_out, bias=bias)).to(dev)
    plain = convert_to_tcfp(copy.deepcopy(base), use_tensor_cores=True, **kw)
    fused = fuse_tcfp_mlp(convert_to_tcfp(copy.deepcopy(base), use_tensor_cores=True, **kw))
    assert type(plain) is nn.Sequential and isinstance(fused, TCFPMLP)
    assert list(plain.state_dict()) == list(fused.state_dict())
    return plain, fused


def _kernel_names(fn):
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return [e.name for e in prof.events()]


def _run_steps(model, x, y, steps, x_grad):
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    rec = []
    for _ in range(steps):
        xx = x.clone().requires_grad_(x_grad)
        out = model(xx)
        loss = (out.float() - y).square().mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        r = [out.detach().clone()] + [p.grad.clone() for p in model.parameters()]
        if x_grad:
            r.append(xx.grad.clone())
        rec.append(r)
        opt.step()
    efs = [m._error_state._buffers[m._param_name].clone()
           for m in model.modules() if isinstance(m, TCFPLinear)]
    return rec, efs


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("x_grad", [False, True])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float32])
def test_fused_mlp_bit_identical_to_plain_sequence(dev, bias, x_grad, xdtype):
    print(f"fused mlp bias={bias} x_grad={x_grad} {xdtype}", flush=True)
    plain, fused = _pair(dev, 256, 1024, 384, bias)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 128, 256, generator=g).to(xdtype).to(dev)
    y = torch.randn(4, 128, 384, generator=g).to(dev)
    with torch.no_grad():  # no EF update: the runs below start from the same state
        names = _kernel_names(lambda: fused(x))
    assert any("gelu_amax_kernel" in n for n in names), names
    rp, ep = _run_steps(plain, x, y, 3, x_grad)
    rf, ef = _run_steps(fused, x, y, 3, x_grad)
    for step, (a, b) in enumerate(zip(rp, rf)):
        assert len(a) == len(b)
        for i, (u, v) in enumerate(zip(a, b)):
            assert u.dtype == v.dtype and u.shape == v.shape, (step, i)
            assert torch.equal(u.float().view(torch.int32), v.float().view(torch.int32)), (step, i)
    for u, v in zip(ep, ef):
        assert torch.equal(bits(u), bits(v))


def test_fused_mlp_c4_shape_one_step(dev):
    # BASELINE configs[3] shape: 8192 tokens, 1024 -> 4096 -> 1024
    plain, fused = _pair(dev, 1024, 4096, 1024, seed=3)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(8192, 1024, generator=g).bfloat16().to(dev)
    y = torch.randn(8192, 1024, generator=g).to(dev)
    rp, ep = _run_steps(plain, x, y, 2, False)
    rf, ef = _run_steps(fused, x, y, 2, False)
    for a, b in zip(rp, rf):
        for u, v in zip(a, b):
            assert torch.equal(bits(u.float()), bits(v.float()))
    for u, v in zip(ep, ef):
        assert torch.equal(bits(u), bits(v))


def test_fused_mlp_falls_back_to_plain_sequence(dev):
    # options the fused path leaves out, a tanh GELU or a ragged token count
    # run the plain sequence (same results, no fused kernel)
    cases = [dict(delayed_scaling=True), dict(hp_grad_weight=True)]
    for kw in cases:
        plain, fused = _pair(dev, 128, 256, 128, **kw)
        x = torch.randn(64, 128, device=dev)
        names = _kernel_names(lambda: fused(x))
        plain(x)  # the same number of calls on both (EF and scaling state advance per call)
        assert not any("gelu_amax_kernel" in n for n in names), kw
        assert torch.equal(bits(fused(x).detach()), bits(plain(x).detach())), kw
    plain, fused = _pair(dev, 128, 256, 128)
    assert not any("gelu_amax_kernel" in n
                   for n in _kernel_names(lambda: fused(torch.randn(40, 128, device=dev))))
    fused[1] = nn.GELU(approximate="tanh")
    assert not any("gelu_amax_kernel" in n
                   for n in _kernel_names(lambda: fused(torch.randn(64, 128, device=dev))))


def test_fuse_tcfp_mlp_replaces_nested_sequences(dev):
    torch.manual_seed(0)
    model = nn.Module()
    model.blocks = nn.ModuleList([
        nn.Sequential(nn.Linear(64, 256), nn.GELU(), nn.Linear(256, 64)) for _ in range(2)])
    model.head = nn.Sequential(nn.Linear(64, 64), nn.ReLU(), nn.Linear(64, 64))
    model = fuse_tcfp_mlp(convert_to_tcfp(model.to(dev), use_tensor_cores=True,
                                          skip_patterns=("none",)))
    assert all(isinstance(b, TCFPMLP) for b in model.blocks)
    assert type(model.head) is nn.Sequential


@pytest.mark.parametrize("shape", [(300, 208), (1000, 24)])
def test_gelu_e5m2_and_colsum_e4m3_quantisation(dev, shape):
    """The entry points take either FP8 format (the layers use E4M3 for
    gelu(h) and E5M2 for gradients): gelu(h) quantised to E5M2, and the
    column-sum quantisation to E4M3 from fp32 and bf16, held to the
    oracle's casts and column sums."""
    print(f"gelu e5m2 / colsum e4m3 {shape}", flush=True)
    g = torch.Generator().manual_seed(shape[0] + 3 * shape[1])
    h = (torch.randn(shape, generator=g) * 3).to(dev)
    q, inv, q_t = K.gelu_quantize_per_tensor(h, torch.float8_e5m2, transpose=True)
    ref = F.gelu(h).cpu().numpy()
    oc, oinv, _ = oq.to_fp8_per_tensor(ref, "f32", "e5m2")
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oc)
    assert np.array_equal(q_t.view(torch.uint8).cpu().numpy(), oc.T)
    assert float(inv.item()) == float(oinv)
    for dt, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        x = torch.randn(shape, generator=g).to(dt).to(dev)
        q, inv, q_t, cs = K.quantize_per_tensor_colsum(x, torch.float8_e4m3fn, transpose=True)
        xn = x.float().cpu().numpy()
        oc, oinv, _ = oq.to_fp8_per_tensor(xn, tag, "e4m3")
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oc), tag
        assert np.array_equal(q_t.view(torch.uint8).cpu().numpy(), oc.T), tag
        assert float(inv.item()) == float(oinv), tag
        assert np.array_equal(cs.cpu().numpy(), oq.column_sums(xn)), tag


@pytest.mark.parametrize("m,k,n", [(8192, 1024, 4096), (4096, 512, 2048), (2048, 256, 8192),
                                   (8192, 2048, 4096)])
def test_dgelu_epilogue_narrow_tile_matches_wide(dev, m, k, n):
    """Layer 2's dgrad with the GELU backward in its epilogue: the 256 x 64
    tile with the derivative factors brought into LDS during the K loop
    (taken for K <= 2048) against the 256 x 128 tile that loads them in the
    epilogue (tile policy "large"), bit for bit: gradient, codes, transposed
    codes, inverse scale and bias column sums; and the kernel each takes."""
    print(f"dgelu narrow vs wide {m}x{k}x{n}", flush=True)
    a, hi, lo, a_inv, ih, il = _fp8_layer(dev, m, k, n, seed=m + 7 * k,
                                          a_dtype=torch.float8_e5m2)
    dg = torch.rand(m, n, generator=torch.Generator().manual_seed(n)).to(dev) * 1.2 - 0.15
    run = lambda: K.dual_gemm_dgelu_quantize_colsum(a, hi, lo, a_inv, ih, il, dg,  # noqa: E731
                                                    transpose=True, col_sum=True,
                                                    return_grad=True)
    names = _kernel_names(run)
    assert any("gemm_nt_persist_kernel<1, 0, float, 2, 0, 6, 64, false>" in x for x in names), names
    p = run()
    try:
        K.set_gemm_tile_policy("large")
        assert not any(", 6, 64>" in x for x in _kernel_names(run))
        q = run()
    finally:
        K.set_gemm_tile_policy("auto")
    for x, y in zip(p, q):
        assert torch.equal(bits(x), bits(y))
