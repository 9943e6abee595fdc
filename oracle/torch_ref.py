"""Torch restatement of the reference's TCFP-12 training steps
(TEST INFRASTRUCTURE ONLY; see the package docstring).

The reference's ``_TCFP12TensorCoreFunction`` (tcfp/nn/__init__.py:312-566)
with its non-fused tier, and its ``_TCFP12BlockScaledFunction``
(tcfp/nn/__init__.py:574-761) with the block quantisation rules of
tcfp/kernels.py:205-275 and :288-459, evaluated with plain torch ops on
whatever device the tensors live on:

* ``to_fp8`` is ``to_fp8_e4m3`` / ``to_fp8_e5m2`` (tcfp/core.py:85-106,
  137-158) op for op;
* every ``torch._scaled_mm(a, b, scale_a, scale_b, out_dtype=float32)`` of
  the reference is the fp32 matmul of the dequantised operands
  (``(a.float() * s_a) @ (b.float() * s_b)``), the product it defines;
* dual quantisation + error feedback as tcfp/nn/__init__.py:343-383, the
  error-feedback update guard as :983-994.

* the block exponent is ``max(ceil(log2(max(amax, 1e-12) / FP8_MAX)),
  -126)`` with log2 evaluated in float64 and rounded once to fp32 (a
  correctly rounded fp32 log2, the rule the numpy oracle pins against
  torch's CPU log2), and the zero-residual W_lo sentinel -128.

Used by the GPU tests to hold the HIP path's training loss to the
reference algorithm's (BASELINE's "loss within 1% after 100 steps").
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

E4M3_MAX = 448.0
E5M2_MAX = 57344.0


def to_fp8(t: torch.Tensor, fmax: float, dtype: torch.dtype):
    """tcfp/core.py:99-106: amax -> scale = fmax / amax (in t's dtype) ->
    clamp(t.float() * scale) -> cast; returns (codes, inv_scale (1,))."""
    amax = t.abs().max().clamp(min=1e-12)
    scale = (fmax / amax).to(torch.float32)
    scaled = (t.float() * scale).clamp(-fmax, fmax)
    q = scaled.to(dtype)
    inv = torch.ones(1, device=t.device, dtype=torch.float32) / scale
    return q, inv


def _deq(q: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    return q.float() * inv


class RefTCFP12Function(torch.autograd.Function):
    """Forward/backward of tcfp/nn/__init__.py:325-566 (no ABD, no delayed
    scaling), FP8 GEMMs as fp32 matmuls of the dequantised operands."""

    @staticmethod
    def forward(ctx, x, weight, bias, ef_store, name, update_ef):
        # dual quantisation with error feedback (nn:343-383)
        w = weight.float()
        err = ef_store.get(name)
        if err is None or err.shape != weight.shape:
            err = torch.zeros_like(w)
        w = w + err
        hi, inv_hi = to_fp8(w, E4M3_MAX, torch.float8_e4m3fn)
        residual = w - hi.float() * inv_hi
        lo, inv_lo = to_fp8(residual, E4M3_MAX, torch.float8_e4m3fn)
        if update_ef:
            ef_store[name] = (weight.float() - (hi.float() * inv_hi + lo.float() * inv_lo)).detach()
        x2 = x.reshape(-1, x.shape[-1]) if x.ndim == 3 else x
        act, act_inv = to_fp8(x2, E4M3_MAX, torch.float8_e4m3fn)
        A = _deq(act, act_inv)
        out = A @ _deq(hi, inv_hi).t() + A @ _deq(lo, inv_lo).t()
        if bias is not None:
            out = out + bias
        ctx.save_for_backward(act, act_inv, hi, lo, inv_hi, inv_lo)
        ctx.in_shape = x.shape
        ctx.has_bias = bias is not None
        return out.reshape(*x.shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, grad_out):
        act, act_inv, hi, lo, inv_hi, inv_lo = ctx.saved_tensors
        g2 = grad_out.reshape(-1, grad_out.shape[-1]) if grad_out.ndim == 3 else grad_out
        gq, g_inv = to_fp8(g2, E5M2_MAX, torch.float8_e5m2)
        G = _deq(gq, g_inv)
        dx = (G @ _deq(hi, inv_hi) + G @ _deq(lo, inv_lo)).reshape(ctx.in_shape)
        if g2.shape[0] % 16 == 0:
            dw = G.t() @ _deq(act, act_inv)
        else:
            dw = g2.t() @ _deq(act, act_inv)
        db = g2.sum(0) if ctx.has_bias else None
        return dx, dw, db, None, None, None


class RefTCFPLinear(nn.Linear):
    """nn.Linear running RefTCFP12Function, with the reference's EF guard
    (update only when the weight changed and autograd records)."""

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.ef: dict[str, torch.Tensor] = {}
        self._last_version = -1

    def forward(self, x):
        v = self.weight._version
        upd = v != self._last_version and torch.is_grad_enabled()
        if upd:
            self._last_version = v
        return RefTCFP12Function.apply(x, self.weight, self.bias, self.ef, "", upd)


def gelu_mlp_step_losses(make_linear, d_in, d_hidden, tokens, steps, seed, device,
                         autocast_bf16=False):
    """Losses of ``steps`` AdamW(lr 1e-3) steps of Linear -> GELU -> Linear
    on seeded bf16 inputs and an MSE target, with ``make_linear(i, o)``
    building the linears (weights re-initialised from ``seed``).
    ``autocast_bf16``: run the forward under ``torch.autocast(bfloat16)``
    (the BF16 mixed-precision baseline with ``nn.Linear``)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, d_in, generator=g).bfloat16().to(device)
    y = torch.randn(tokens, d_in, generator=g).to(device)
    l1, l2 = make_linear(d_in, d_hidden), make_linear(d_hidden, d_in)
    torch.manual_seed(seed + 1)
    for lin in (l1, l2):
        nn.init.kaiming_uniform_(lin.weight, a=5**0.5)
        nn.init.uniform_(lin.bias, -lin.weight.shape[1] ** -0.5, lin.weight.shape[1] ** -0.5)
    model = nn.Sequential(l1, nn.GELU(), l2).to(device)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    losses = []
    for _ in range(steps):
        with torch.autocast(device.type if isinstance(device, torch.device) else "cuda",
                            dtype=torch.bfloat16, enabled=autocast_bf16):
            out = model(x)
        loss = (out.float() - y).square().mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        losses.append(loss.detach())
    return [float(v) for v in torch.stack(losses).cpu()]


# ------------------------------------------------------------ block-scaled
def block_quant(t: torch.Tensor, bs: int, fmax: float, dtype: torch.dtype,
                sentinel: bool = False):
    """Per-(row, bs-block) power-of-two quantisation of a 2-D tensor
    (tcfp/kernels.py:205-275; the W_lo variant :381-396 when ``sentinel``):
    returns (codes [M, K], exponents int8 [K/bs, M])."""
    M, K = t.shape
    blocks = t.float().reshape(M, K // bs, bs)
    raw = blocks.abs().amax(-1)
    amax = raw.clamp(min=1e-12)
    e = torch.ceil(torch.log2((amax / fmax).double()).float()).clamp(min=-126)
    if sentinel:
        zero = raw < 1e-12
        div = torch.where(zero, torch.ones_like(e), torch.exp2(e))
        e = torch.where(zero, torch.full_like(e, -128.0), e)
    else:
        div = torch.exp2(e)
    q = (blocks / div[..., None]).clamp(-fmax, fmax).to(dtype).reshape(M, K)
    return q, e.to(torch.int8).t().contiguous()


def block_deq(q: torch.Tensor, e: torch.Tensor, bs: int) -> torch.Tensor:
    """``fp8 * exp2(e)`` per block (tcfp/kernels.py:1725-1746)."""
    M, K = q.shape
    s = torch.exp2(e.t().float())  # [M, K/bs]
    return (q.float().reshape(M, K // bs, bs) * s[..., None]).reshape(M, K)


class RefBlockTCFP12Function(torch.autograd.Function):
    """Forward/backward of tcfp/nn/__init__.py:583-761 (no ABD, hp_grad_weight
    False, error feedback, no SRR): the FP8 GEMMs as fp32 matmuls of the
    dequantised operands, which is what its kernels compute."""

    @staticmethod
    def forward(ctx, x, weight, bias, ef_store, name, update_ef, bs, mm_dtype=torch.float32,
                out_noise=0.0):
        # dual quantisation with in-place error feedback (kernels.py:1749-1875)
        err = ef_store.get(name)
        if err is None or err.shape != weight.shape:
            err = torch.zeros(weight.shape, dtype=torch.float32, device=weight.device)
            ef_store[name] = err
        w = weight.float() + err
        hi, e_hi = block_quant(w, bs, E4M3_MAX, torch.float8_e4m3fn)
        d_hi = block_deq(hi, e_hi, bs)
        lo, e_lo = block_quant(w - d_hi, bs, E4M3_MAX, torch.float8_e4m3fn, sentinel=True)
        d_lo = block_deq(lo, e_lo, bs)
        if update_ef:
            ef_store[name] = ((weight.float() - d_hi) - d_lo).detach()
        x2 = x.reshape(-1, x.shape[-1])
        act, e_act = block_quant(x2, bs, E4M3_MAX, torch.float8_e4m3fn)
        A = block_deq(act, e_act, bs)
        Am = A.to(mm_dtype)
        out = (Am @ d_hi.t().to(mm_dtype) + Am @ d_lo.t().to(mm_dtype)).float()
        if out_noise:
            out = out + out_noise * out.std() * torch.randn_like(out)
        if bias is not None:
            out = out + bias
        ctx.save_for_backward(A, d_hi, d_lo)
        ctx.in_shape, ctx.has_bias, ctx.bs = x.shape, bias is not None, bs
        return out.reshape(*x.shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, grad_out):
        A, d_hi, d_lo = ctx.saved_tensors
        g2 = grad_out.reshape(-1, grad_out.shape[-1]).float()
        gq, e_g = block_quant(g2, ctx.bs, E5M2_MAX, torch.float8_e5m2)
        G = block_deq(gq, e_g, ctx.bs)
        dx = (G @ (d_hi + d_lo)).reshape(ctx.in_shape)
        dw = g2.t() @ A
        db = g2.sum(0) if ctx.has_bias else None
        return dx, dw, db, None, None, None, None, None, None


class RefBlockTCFPLinear(nn.Linear):
    """nn.Linear running RefBlockTCFP12Function with the reference's EF
    guard (tcfp/nn/__init__.py:983-994).  ``mm_dtype`` sets the forward
    matmuls' precision and ``out_noise`` adds Gaussian noise of that
    relative size to each forward product: controls for how a network
    amplifies summation differences through its re-quantisations."""

    def __init__(self, *a, block_size: int = 64, mm_dtype=torch.float32, out_noise: float = 0.0,
                 **kw):
        super().__init__(*a, **kw)
        self.bs = block_size
        self.mm_dtype = mm_dtype
        self.out_noise = out_noise
        self.ef: dict[str, torch.Tensor] = {}
        self._last_version = -1

    def forward(self, x):
        v = self.weight._version
        upd = v != self._last_version and torch.is_grad_enabled()
        if upd:
            self._last_version = v
        return RefBlockTCFP12Function.apply(x, self.weight, self.bias, self.ef, "", upd, self.bs,
                                            self.mm_dtype, self.out_noise)


def swap_linears(model: nn.Module, make, skip: tuple[str, ...] = ("head",)) -> nn.Module:
    """Replace every nn.Linear child (depth first, names containing a
    ``skip`` pattern left alone) by ``make(linear)``."""
    for name, child in model.named_children():
        swap_linears(child, make, skip)
        if any(p in name for p in skip):
            continue
        if type(child) is nn.Linear:
            setattr(model, name, make(child))
    return model
