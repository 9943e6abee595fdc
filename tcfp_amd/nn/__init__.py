"""TCFP-12 modules and autograd Functions (drop-in for ``tcfp.nn``'s tensor-core path).

``TCFPLinear`` / ``convert_to_tcfp`` keep the reference's constructor and
conversion API (``tcfp/nn/__init__.py:769-1077, 1190-1351``).  The two
autograd Functions keep the reference's positional signatures and
saved-state semantics:

* ``_TCFP12TensorCoreFunction.apply`` -- 15 args (``tcfp/nn/__init__.py:312-566``)
* ``_TCFP12BlockScaledFunction.apply`` -- 10 args (``tcfp/nn/__init__.py:574-761``)

but their bodies call the HIP operator layer (``tcfp_amd.kernels``):

* per-tensor forward: one dual-quant launch chain (W + EF -> W_hi, W_lo,
  scales, new EF, and the transposed copies dgrad needs), one act-quant
  chain (codes + the transposed copy wgrad needs), one fused dual FP8 GEMM
  with the bias in its epilogue;
* per-tensor backward: E5M2 grad quant (+ transposed copy), dual FP8 dgrad,
  single FP8 wgrad, all on the same K-contiguous MFMA kernel.  dX is
  skipped when autograd does not need it (the reference always computes it;
  the results of the gradients that are returned are unchanged).

Delayed scaling and NF-aware scaling run inside the same dual-quant
kernels.  The reference's fake-quantise path (``use_tensor_cores=False``,
int4/NF4 residual via ``tcfp.tcfp12``) is not part of this build and raises
``NotImplementedError``.
"""
from __future__ import annotations

import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import kernels as K
from ..core import DEFAULT_BLOCK_SIZE, ErrorFeedbackState, TCFPMode

__all__ = [
    "TCFPLinear",
    "TCFPMLP",
    "convert_to_tcfp",
    "fuse_tcfp_mlp",
    "set_block_dgrad",
    "set_block_wgrad",
    "_TCFP12TensorCoreFunction",
    "_TCFP12BlockScaledFunction",
    "_TCFP12FusedMLPFunction",
]


def _flatten(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1]) if t.ndim != 2 else t


def _ef_buffer(state: ErrorFeedbackState | None, name: str, weight: torch.Tensor):
    if state is None:
        return None
    return state.get_error(name, weight)


class _TCFP12TensorCoreFunction(torch.autograd.Function):
    """TCFP-12 per-tensor dual-FP8 linear (reference ``tcfp/nn/__init__.py:312-566``).

    Forward: ``out = X W_hi^T s_x s_hi + X W_lo^T s_x s_lo (+ bias)`` in fp32.
    Backward: ``dX`` = dual FP8 dgrad with E5M2 gradients (W_hi only under
    ABD); ``dW`` = FP8 wgrad, or ``grad^T @ input`` when ``hp_grad_weight``,
    or ``grad^T @ dequant(act)`` when the token count is not a multiple of
    16 (reference ``:540-555``).
    """

    @staticmethod
    def forward(  # noqa: PLR0913
        ctx,
        input: torch.Tensor,
        weight: torch.Tensor,
        bias: torch.Tensor | None,
        nf_aware_scaling: bool,
        sigma_factor: float,
        stochastic_rounding: bool,
        hp_grad_weight: bool,
        error_state: ErrorFeedbackState | None,
        param_name: str,
        delayed_scaling: bool = False,
        use_fused_kernel: bool = True,
        use_cuda_ext: bool = True,
        abd: bool = False,
        srr: bool = False,
        update_ef: bool = True,
    ) -> torch.Tensor:
        need_dx = ctx.needs_input_grad[0]
        need_dw = ctx.needs_input_grad[1]

        # 1-4. dual quantisation of W (+ EF read and in-place update); with
        # delayed scaling (and an EF state to hold it) the scales follow the
        # reference's predictive dual-track rule (nn:250-309, 350-374);
        # NF-aware scaling sets the W_hi scale from sigma_factor * std, with
        # stochastic W_hi rounding when stochastic_rounding (nn:356-359)
        error_buf = _ef_buffer(error_state, param_name, weight)
        sigma = float(sigma_factor) if nf_aware_scaling else None
        sr_hi = bool(nf_aware_scaling and stochastic_rounding)
        delayed = delayed_scaling and error_state is not None
        input_shape = input.shape
        input_2d = _flatten(input)
        M = input_2d.shape[0]
        fp8_wgrad = need_dw and not hp_grad_weight and M % 16 == 0
        # (5. below) With no delayed, NF-aware or stochastic option and a
        # weight below 2^23 elements (where the single call also makes three
        # passes), W's dual quantisation and the activation quantisation run
        # as one batch: the same results in fewer launches.
        if not delayed and sigma is None and not srr and weight.numel() < (1 << 23):
            (res,), (ra,) = K.quantize_batch(
                dual=[(weight, error_buf, update_ef, need_dx)],
                act=[(input_2d, torch.float8_e4m3fn, fp8_wgrad)],
            )
        else:
            if delayed:
                res = K.dual_quantize_per_tensor_delayed(
                    weight, error_buf, error_state, param_name, update_ef=update_ef,
                    transposed=need_dx, sigma_factor=sigma, stochastic_hi=sr_hi,
                )
            else:
                res = K.dual_quantize_per_tensor(
                    weight, error_buf, update_ef=update_ef, stochastic_lo=srr,
                    transposed=need_dx, sigma_factor=sigma, stochastic_hi=sr_hi,
                )
            ra = K.quantize_per_tensor(input_2d, transpose=fp8_wgrad)
        w_hi, w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t = res if need_dx else (*res, None, None)

        # 5. activation quantisation (and the transposed copy FP8 wgrad reads)
        act_fp8, act_inv, act_t = ra if fp8_wgrad else (*ra, None)

        # 6-7. fused dual GEMM, bias in the epilogue
        out_2d = K.fused_dual_gemm_forward(
            act_fp8, w_hi, w_lo, act_inv, inv_hi, inv_lo, bias=bias
        )
        output = out_2d.reshape(*input_shape[:-1], out_2d.shape[-1])

        # 8. save for backward
        ctx.hp_grad_weight = hp_grad_weight
        ctx.input_shape = input_shape
        ctx.has_bias = bias is not None
        ctx.abd = abd
        ctx.fp8_wgrad = fp8_wgrad
        if not need_dw:
            saved_act = None
        elif hp_grad_weight:
            saved_act = input_2d
        elif fp8_wgrad:
            saved_act = act_t
        else:
            saved_act = act_fp8
        ctx.save_for_backward(
            saved_act, act_inv, w_hi_t, None if abd else w_lo_t, inv_hi, inv_lo
        )
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        saved_act, act_inv, w_hi_t, w_lo_t, inv_hi, inv_lo = ctx.saved_tensors
        need_dx, need_dw, need_db = ctx.needs_input_grad[:3]
        grad_2d = _flatten(grad_output)
        if not grad_2d.is_contiguous():
            grad_2d = grad_2d.contiguous()

        grad_input = grad_weight = grad_bias = None
        # the bias gradient comes out of the gradient's amax pass when the
        # gradient is quantised anyway (fp32 sums, as the reference's sum(0))
        fuse_db = need_db and ctx.has_bias and grad_2d.shape[-1] % 8 == 0
        if need_dx or (need_dw and ctx.fp8_wgrad):
            want_t = need_dw and ctx.fp8_wgrad
            if fuse_db:
                res = K.quantize_per_tensor_colsum(grad_2d, torch.float8_e5m2, transpose=want_t)
                grad_bias = res[-1].to(grad_2d.dtype)
                res = res[:-1]
            else:
                res = K.quantize_per_tensor(grad_2d, torch.float8_e5m2, transpose=want_t)
            if want_t:
                grad_fp8, grad_inv, grad_t = res
            else:
                (grad_fp8, grad_inv), grad_t = res, None
            if need_dx:
                if ctx.abd:
                    gi = K.fp8_gemm_nt(grad_fp8, w_hi_t, grad_inv, inv_hi)
                else:
                    gi = K._dual_gemm(grad_fp8, w_hi_t, w_lo_t, grad_inv, inv_hi, inv_lo,
                                      None, torch.float32)
                grad_input = gi.reshape(ctx.input_shape)
        if need_dw:
            if ctx.hp_grad_weight:
                grad_weight = grad_2d.t() @ saved_act.to(grad_2d.dtype)
            elif ctx.fp8_wgrad:
                grad_weight = K.fp8_gemm_nt(grad_t, saved_act, grad_inv, act_inv)
            else:
                grad_weight = grad_2d.t() @ (saved_act.float() * act_inv).to(grad_2d.dtype)
        if need_db and ctx.has_bias and grad_bias is None:
            grad_bias = grad_2d.sum(dim=0)
        return (grad_input, grad_weight, grad_bias) + (None,) * 12


_BLOCK_DGRAD = "exact"


def set_block_dgrad(mode: str) -> None:
    """Numerics of the block-scaled layers' input gradient (default
    ``"exact"``).

    ``"exact"``: the reference's ``dX = deq(G) @ (deq(W_hi) + deq(W_lo))``
    with every product exact (bf16 MFMA on exactly representable operands),
    at least as accurate as its fp32 dot.  ``"fp8"``: W re-blocked along
    D_out and the block dual FP8 GEMM (``kernels.fp8_block_dgrad``), which
    adds one dual-FP8 rounding of W (relative ~2^-9 of a block's maximum) and
    runs at FP8 rate.  Read when a layer's forward runs; the backward of that
    call uses the mode in force then.
    """
    global _BLOCK_DGRAD
    if mode not in ("exact", "fp8"):
        raise ValueError(f"block dgrad mode must be 'exact' or 'fp8', got {mode!r}")
    _BLOCK_DGRAD = mode


_BLOCK_WGRAD = "split"


def set_block_wgrad(mode: str) -> None:
    """Numerics of the block-scaled layers' weight gradient (default
    ``"split"``).

    ``"split"``: the reference's ``dW = G^T @ deq(X)`` with G in fp32,
    computed as two exact bf16 passes over ``[bf16(G) | bf16(G - bf16(G))]``
    (the reference's fp32 product to within fp32 accumulation).
    ``"bf16"``: one pass over ``bf16(G)`` (relative error ~2^-9 per gradient
    element, within the reference's 1e-2 GEMM contract): half the MFMA
    work, and the gradient's low half is never stored.  Token counts that
    are not a multiple of 64 keep the split.  Read when a layer's forward
    runs, like :func:`set_block_dgrad`.
    """
    global _BLOCK_WGRAD
    if mode not in ("split", "bf16"):
        raise ValueError(f"block wgrad mode must be 'split' or 'bf16', got {mode!r}")
    _BLOCK_WGRAD = mode


class _TCFP12BlockScaledFunction(torch.autograd.Function):
    """TCFP-12 with per-block (32/64/128 along K) power-of-two scales
    (reference ``tcfp/nn/__init__.py:574-761``)."""

    @staticmethod
    def forward(
        ctx,
        input: torch.Tensor,
        weight: torch.Tensor,
        bias: torch.Tensor | None,
        scale_block_size: int,
        hp_grad_weight: bool,
        error_state: ErrorFeedbackState | None,
        param_name: str,
        abd: bool = False,
        srr: bool = False,
        update_ef: bool = True,
    ) -> torch.Tensor:
        bs = scale_block_size
        error_buf = _ef_buffer(error_state, param_name, weight)
        w = weight if weight.is_contiguous() else weight.contiguous()
        input_shape = input.shape
        input_2d = _flatten(input)
        # W's dual quantisation (EF is read, and rewritten in place only when
        # update_ef; the reference clones the buffer instead, :597-608), then
        # the reference's dispatch (:617-650): the fused act-quant GEMM for
        # narrow layers, separate activation quantisation otherwise -- the
        # launches of K.fused_dual_quantize_fp8, K.fused_act_quant_dual_gemm_forward
        # / K.block_quantize_fp8 + K.fused_block_scaled_dual_gemm_forward in
        # one host call
        out_2d, w_hi, w_lo, sh, sl, act_fp8, act_scales = K.block_linear_forward(
            input_2d, w, bias, bs, error_buf=error_buf, srr=srr, update_ef=update_ef
        )
        output = out_2d.reshape(*input_shape[:-1], out_2d.shape[-1])

        ctx.hp_grad_weight = hp_grad_weight
        ctx.input_shape = input_shape
        ctx.has_bias = bias is not None
        ctx.bs = bs
        ctx.abd = abd
        ctx.fp8_dgrad = _BLOCK_DGRAD == "fp8"
        ctx.bf16_wgrad = _BLOCK_WGRAD == "bf16"
        # only what the backward will use is kept: the activation codes for
        # dW, the weight codes for dX
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        saved_act = (input_2d if hp_grad_weight else act_fp8) if need_dw else None
        saved_act_scales = None if (hp_grad_weight or not need_dw) else act_scales
        w_lo_b, sl_b = (None, None) if abd else (w_lo, sl)
        if not need_dx:
            w_hi = w_lo_b = sh = sl_b = None
        elif ctx.fp8_dgrad:
            # the FP8 dgrad's weight operand, re-blocked along D_out once per
            # forward; the backward needs nothing else of W
            w_hi, w_lo_b, sh, sl_b = K.block_requant_t(w_hi, w_lo_b, sh, sl_b, bs)
        ctx.save_for_backward(saved_act, saved_act_scales, w_hi, w_lo_b, sh, sl_b)
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        saved_act, act_scales, w_hi, w_lo, sh, sl = ctx.saved_tensors
        need_dx, need_dw, need_db = ctx.needs_input_grad[:3]
        bs = ctx.bs
        grad_2d = _flatten(grad_output)
        if not grad_2d.is_contiguous():
            grad_2d = grad_2d.contiguous()
        grad_input = grad_weight = grad_bias = None
        # one pass over the gradient prepares what the reference derives from
        # it separately (nn:700-761): the E5M2 block-quantised G for the
        # dgrad (as bf16 values), the split gradient for the fp32-accuracy
        # wgrad, and the bias gradient
        fp8_wgrad = need_dw and not ctx.hp_grad_weight and grad_2d.shape[0] % 4 == 0
        want_db = need_db and ctx.has_bias
        split_lo = not (ctx.bf16_wgrad and grad_2d.shape[0] % 64 == 0)
        if (not ctx.fp8_dgrad and not ctx.hp_grad_weight and (fp8_wgrad or not need_dw)
                and (need_dx or need_dw or want_db)):
            # the default modes: the prep pass, the wgrad, the exact dgrad
            # in one host call (the same launches as below)
            dx, dw, db = K.block_linear_backward(
                grad_2d, saved_act, act_scales, w_hi, w_lo, sh, sl, bs, need_dx, need_dw,
                want_db, split_lo=split_lo)
            if dx is not None:
                grad_input = dx.reshape(ctx.input_shape)
            if dw is not None:
                grad_weight = dw.to(grad_2d.dtype)
            if want_db:
                grad_bias = db.to(grad_2d.dtype)
            return (grad_input, grad_weight, grad_bias) + (None,) * 7
        g_deq = g_split = db = g_codes = None
        exact_dx = need_dx and not ctx.fp8_dgrad
        fp8_dx = need_dx and ctx.fp8_dgrad
        if exact_dx or fp8_wgrad or want_db or fp8_dx:
            res = K.block_backward_prep(
                grad_2d, bs, dequant=exact_dx, split=fp8_wgrad, bias=want_db, fp8=fp8_dx,
                split_lo=split_lo,
            )
            g_deq, g_split, db = res[:3]
            if fp8_dx:
                g_codes = (res[3], res[4])
            del res  # (the buffers are released as soon as their users are done)
        # the wgrad first: its split gradient is released before the dgrad
        # allocates dX (the two never coexist at the layer's peak)
        if need_dw:
            if ctx.hp_grad_weight:
                grad_weight = grad_2d.t() @ saved_act.to(grad_2d.dtype)
            elif fp8_wgrad:
                grad_weight = K.block_wgrad_from_prep(g_split, saved_act, act_scales, bs)
                grad_weight = grad_weight.to(grad_2d.dtype)
            else:
                grad_weight = K.block_scaled_wgrad(grad_2d, saved_act, act_scales, bs)
                grad_weight = grad_weight.to(grad_2d.dtype)
        g_split = None
        if exact_dx:
            grad_input = K.block_dgrad_from_prep(
                g_deq, w_hi, w_lo, sh, sl, block_size=bs
            ).reshape(ctx.input_shape)
        elif need_dx:
            # (the saved weight operands are the forward's re-blocked ones)
            grad_input = K.fp8_block_dgrad(None, None, None, None, None, bs,
                                           reblocked=(w_hi, w_lo, sh, sl),
                                           grad_fp8=g_codes).reshape(ctx.input_shape)
        g_deq = g_codes = None
        if want_db:
            grad_bias = db.to(grad_2d.dtype)
        return (grad_input, grad_weight, grad_bias) + (None,) * 7


class TCFPLinear(nn.Module):
    """Drop-in ``nn.Linear`` on the TCFP-12 dual-FP8 tensor-core path.

    Same constructor as the reference (``tcfp/nn/__init__.py:810-832``).
    ``use_tensor_cores`` must be True (the fake-quantise path is not part of
    this build); ``use_fused_kernel`` / ``use_cuda_ext`` are accepted and
    ignored -- every call runs the HIP kernels.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = True,
        mode: TCFPMode = TCFPMode.TCFP12,
        block_size: int = DEFAULT_BLOCK_SIZE,
        *,
        nf4_residual: bool = False,
        nf_aware_scaling: bool = False,
        sigma_factor: float = 3.0,
        stochastic_rounding: bool = False,
        warmup_steps: int = 0,
        use_tensor_cores: bool = False,
        hp_grad_weight: bool = False,
        error_feedback: bool = True,
        delayed_scaling: bool = False,
        use_fused_kernel: bool = True,
        use_cuda_ext: bool = True,
        scale_block_size: int | None = None,
        abd: bool = False,
        srr: bool = False,
        device=None,
        dtype=None,
    ) -> None:
        super().__init__()
        if not use_tensor_cores:
            raise NotImplementedError(
                "TCFPLinear(use_tensor_cores=False) is the fake-quantise path, which is "
                "not part of this build; pass use_tensor_cores=True"
            )
        if nf4_residual:
            warnings.warn(
                "nf4_residual is ignored in tensor core mode — NF4 cannot "
                "run on tensor cores. The residual uses FP8 E4M3 instead.",
                stacklevel=2,
            )
        if scale_block_size is not None:
            if scale_block_size not in (32, 64, 128):
                raise ValueError(
                    f"scale_block_size must be 32, 64, or 128, got {scale_block_size}"
                )
            if in_features % scale_block_size != 0:
                raise ValueError(
                    f"in_features ({in_features}) must be divisible by "
                    f"scale_block_size ({scale_block_size})"
                )
            if out_features % scale_block_size != 0:
                raise ValueError(
                    f"out_features ({out_features}) must be divisible by "
                    f"scale_block_size ({scale_block_size}). Backward pass "
                    f"block-quantizes gradients along the output dimension."
                )
            if delayed_scaling:
                warnings.warn(
                    "Per-block scaling (scale_block_size) and delayed_scaling "
                    "are mutually exclusive. Ignoring delayed_scaling.",
                    stacklevel=2,
                )
                delayed_scaling = False
        if srr and delayed_scaling:
            warnings.warn(
                "srr=True is mutually exclusive with delayed_scaling=True. "
                "Disabling delayed_scaling.",
                stacklevel=2,
            )
            delayed_scaling = False

        self.in_features = in_features
        self.out_features = out_features
        self.mode = mode
        self.block_size = block_size
        self.nf4_residual = nf4_residual
        self.nf_aware_scaling = nf_aware_scaling
        self.sigma_factor = sigma_factor
        self.stochastic_rounding = stochastic_rounding
        self._warmup_steps = warmup_steps
        self._warmup_remaining = warmup_steps
        self.use_tensor_cores = use_tensor_cores
        self.hp_grad_weight = hp_grad_weight
        self.use_fused_kernel = use_fused_kernel
        self.use_cuda_ext = use_cuda_ext
        self.scale_block_size = scale_block_size
        self.delayed_scaling = delayed_scaling
        self.abd = abd
        self.srr = srr
        self._error_state: ErrorFeedbackState | None = (
            ErrorFeedbackState() if (error_feedback and not srr) else None
        )
        self._param_name: str = ""
        self._last_weight_version: int = -1
        self._bf16_fallback: bool = False

        factory = {"device": device, "dtype": dtype}
        self.weight = nn.Parameter(torch.empty(out_features, in_features, **factory))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, **factory))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.kaiming_uniform_(self.weight, a=5**0.5)
        if self.bias is not None:
            fan_in = self.weight.shape[1]
            bound = 1 / fan_in**0.5
            nn.init.uniform_(self.bias, -bound, bound)

    def fallback_to_bf16(self) -> None:
        """Switch this layer to the unquantised pass-through."""
        self._bf16_fallback = True

    def restore_tcfp(self) -> None:
        self._bf16_fallback = False

    @torch.compiler.disable
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._bf16_fallback:
            return F.linear(x, self.weight, self.bias)
        if self._warmup_remaining > 0:
            self._warmup_remaining -= 1
            return F.linear(x, self.weight, self.bias)
        update_ef = self._ef_update_flag()
        if self.scale_block_size is not None:
            return _TCFP12BlockScaledFunction.apply(
                x, self.weight, self.bias, self.scale_block_size, self.hp_grad_weight,
                self._error_state, self._param_name, self.abd, self.srr, update_ef,
            )
        return _TCFP12TensorCoreFunction.apply(
            x, self.weight, self.bias, self.nf_aware_scaling, self.sigma_factor,
            self.stochastic_rounding, self.hp_grad_weight, self._error_state,
            self._param_name, self.delayed_scaling, self.use_fused_kernel, self.use_cuda_ext,
            self.abd, self.srr, update_ef,
        )

    def _ef_update_flag(self) -> bool:
        """EF guard (reference :983-994): update only when the weight changed
        since the last update and autograd is recording."""
        ver = self.weight._version
        update_ef = ver != self._last_weight_version and torch.is_grad_enabled()
        if update_ef:
            self._last_weight_version = ver
        return update_ef

    def _plain_per_tensor(self) -> bool:
        """True when forward takes the default per-tensor path (EF or not)
        with no option the fused MLP path leaves out."""
        return (
            self.scale_block_size is None and not self.delayed_scaling
            and not self.nf_aware_scaling and not self.srr and not self.abd
            and not self.hp_grad_weight and not self._bf16_fallback
            and self._warmup_remaining == 0
        )

    def extra_repr(self) -> str:
        parts = [
            f"in_features={self.in_features}",
            f"out_features={self.out_features}",
            f"bias={self.bias is not None}",
            f"mode={self.mode.name}",
            f"block_size={self.block_size}",
            "use_tensor_cores=True",
        ]
        if self.hp_grad_weight:
            parts.append("hp_grad_weight=True")
        if self.nf4_residual:
            parts.append("nf4_residual=True")
        if self.nf_aware_scaling:
            parts.append("nf_aware_scaling=True")
        if self.stochastic_rounding:
            parts.append("stochastic_rounding=True")
        if self.delayed_scaling:
            parts.append("delayed_scaling=True")
        if self.use_fused_kernel:
            parts.append("use_fused_kernel=True")
        if self.use_cuda_ext:
            parts.append("use_cuda_ext=True")
        if self.scale_block_size is not None:
            parts.append(f"scale_block_size={self.scale_block_size}")
        if self.abd:
            parts.append("abd=True")
        if self.srr:
            parts.append("srr=True")
        if self._warmup_steps > 0:
            parts.append(f"warmup_steps={self._warmup_steps}")
        if self._bf16_fallback:
            parts.append("bf16_fallback=True")
        return ", ".join(parts)


class _TCFP12FusedMLPFunction(torch.autograd.Function):
    """``TCFPLinear -> GELU -> TCFPLinear`` (both per-tensor, EF as each layer
    has it) as one autograd node, with the GELU fused into the
    quantisation on either side of it.

    No reference counterpart: the reference runs ``torch.nn.functional.gelu``
    between two ``_TCFP12TensorCoreFunction`` calls
    (``tcfp/nn/__init__.py:325-566``).  Every step here is that sequence's
    step -- same operands, same order of rounding -- except that the
    amax of ``gelu(h)`` comes from the maximum of h recorded in the epilogue
    of layer 1's GEMM (exact under premises checked once per device, with a
    full pass otherwise), ``gelu(h)`` is evaluated in layer 2's activation
    quantisation, which also saves the GELU derivative factors in place of
    h, and the GELU backward (one multiply by those factors), the amax of
    its result and the bias column partials run in the epilogue of layer 2's
    dgrad GEMM.  GELU and its backward are evaluated as torch evaluates
    them, bit for bit, so outputs, gradients and EF updates are identical to
    the unfused sequence; the separate GELU and amax passes over the hidden
    activation and its gradient disappear.
    """

    @staticmethod
    def forward(  # noqa: PLR0913
        ctx, x, w1, b1, w2, b2, st1, name1, st2, name2, update_ef1, update_ef2,
    ):
        need_dx, need_dw1, need_db1, need_dw2, need_db2 = ctx.needs_input_grad[:5]
        need_h = need_dx or need_dw1 or need_db1  # a gradient flows into layer 1

        # both layers' dual quantisation (nn:343-383) and layer 1's
        # activation quantisation (nn:390): independent per-tensor
        # quantisations, run as one batch (three launches in all)
        ef1 = _ef_buffer(st1, name1, w1)
        ef2 = _ef_buffer(st2, name2, w2)
        input_shape = x.shape
        x2d = _flatten(x)
        (res, res2), (ra,) = K.quantize_batch(
            dual=[(w1, ef1, update_ef1, need_dx), (w2, ef2, update_ef2, need_h)],
            act=[(x2d, torch.float8_e4m3fn, need_dw1)],
        )
        w1_hi, w1_lo, ih1, il1, w1_hi_t, w1_lo_t = res if need_dx else (*res, None, None)
        a1, a1_inv, a1_t = ra if need_dw1 else (*ra, None)
        # layer 1's GEMM, whose epilogue records max h for the GELU's amax,
        # then layer 2's activation quantisation (nn:390 on gelu(h)), which
        # also writes the GELU derivative factors the backward needs
        res = K.dual_gemm_gelu_quantize(a1, w1_hi, w1_lo, a1_inv, ih1, il1, bias=b1,
                                        transpose=need_dw2, return_dgelu=need_h)
        _, a2, a2_inv = res[:3]
        a2_t = res[3] if need_dw2 else None
        dgelu = res[-1] if need_h else None

        # layer 2
        w2_hi, w2_lo, ih2, il2, w2_hi_t, w2_lo_t = res2 if need_h else (*res2, None, None)
        out = K.fused_dual_gemm_forward(a2, w2_hi, w2_lo, a2_inv, ih2, il2, bias=b2)

        ctx.input_shape = input_shape
        ctx.has_b1, ctx.has_b2 = b1 is not None, b2 is not None
        ctx.save_for_backward(
            a1_t, a1_inv, w1_hi_t, w1_lo_t, ih1, il1,
            dgelu, a2_t, a2_inv, w2_hi_t, w2_lo_t, ih2, il2,
        )
        return out.reshape(*input_shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, grad_output):
        (a1_t, a1_inv, w1_hi_t, w1_lo_t, ih1, il1,
         dgelu, a2_t, a2_inv, w2_hi_t, w2_lo_t, ih2, il2) = ctx.saved_tensors
        need_dx, need_dw1, need_db1, need_dw2, need_db2 = ctx.needs_input_grad[:5]
        need_h = need_dx or need_dw1 or need_db1
        g2 = _flatten(grad_output)
        if not g2.is_contiguous():
            g2 = g2.contiguous()
        grad_x = dw1 = db1 = dw2 = db2 = None

        # layer 2 (nn:462-566): E5M2 grad + bias sums, dual dgrad, FP8 wgrad
        fuse_db2 = need_db2 and ctx.has_b2 and g2.shape[-1] % 8 == 0
        q2 = g2_inv = None
        if need_h or need_dw2:
            if fuse_db2:
                res = K.quantize_per_tensor_colsum(g2, torch.float8_e5m2, transpose=need_dw2)
                db2 = res[-1].to(g2.dtype)
                res = res[:-1]
            else:
                res = K.quantize_per_tensor(g2, torch.float8_e5m2, transpose=need_dw2)
            (q2, g2_inv, q2_t) = res if need_dw2 else (*res, None)
            if need_dw2:
                dw2 = K.fp8_gemm_nt(q2_t, a2_t, g2_inv, a2_inv)
        if need_db2 and ctx.has_b2 and db2 is None:
            db2 = g2.sum(dim=0)

        # layer 2's dgrad with the GELU backward, its amax and layer 1's
        # bias column sums in the epilogue, then layer 1's E5M2 gradient
        # quantisation; layer 1
        if need_h:
            sums = need_db1 and ctx.has_b1
            # (layer 1's gradient codes feed its dX, their transposed copy its
            # dW: the codes are written only when dX is needed)
            res = K.dual_gemm_dgelu_quantize_colsum(
                q2, w2_hi_t, w2_lo_t, g2_inv, ih2, il2, dgelu, transpose=need_dw1, col_sum=sums,
                codes=need_dx or not need_dw1,
            )
            q1, g1_inv = res[0], res[1]
            q1_t = res[2] if need_dw1 else None
            if sums:
                db1 = res[-1]
            if need_dx:
                grad_x = K._dual_gemm(q1, w1_hi_t, w1_lo_t, g1_inv, ih1, il1, None,
                                      torch.float32).reshape(ctx.input_shape)
            if need_dw1:
                dw1 = K.fp8_gemm_nt(q1_t, a1_t, g1_inv, a1_inv)
        return (grad_x, dw1, db1, dw2, db2) + (None,) * 6


class TCFPMLP(nn.Sequential):
    """``TCFPLinear -> nn.GELU() -> TCFPLinear`` with the GELU fused into the
    quantisation around it (``_TCFP12FusedMLPFunction``).

    A ``nn.Sequential`` of exactly those three children (same parameter
    names as the plain sequence, so state dicts and optimizers carry over).
    When both layers take the default per-tensor path, the GELU is the exact
    (``approximate="none"``) form, the hidden size is a multiple of 8 and the
    token count a multiple of 16, forward runs the fused Function, whose
    results equal the plain sequence's bit for bit; otherwise it runs the
    plain sequence.  Each layer keeps its own EF state and EF guard.
    """

    def _fusable(self, x: torch.Tensor) -> bool:
        if len(self) != 3:
            return False
        fc1, act, fc2 = self[0], self[1], self[2]
        if not (isinstance(fc1, TCFPLinear) and isinstance(fc2, TCFPLinear)):
            return False
        if not isinstance(act, nn.GELU) or act.approximate != "none":
            return False
        if not (fc1._plain_per_tensor() and fc2._plain_per_tensor()):
            return False
        if fc1.out_features != fc2.in_features or fc1.out_features % 8 != 0:
            return False
        if x.device.type != "cuda" or x.dtype not in (torch.float32, torch.bfloat16):
            return False
        if x.dim() == 0 or x.shape[-1] != fc1.in_features:
            return False
        tokens = x.numel() // x.shape[-1]
        return tokens % 16 == 0 and tokens > 0

    @torch.compiler.disable
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._fusable(x):
            return super().forward(x)
        fc1, fc2 = self[0], self[2]
        u1 = fc1._ef_update_flag()
        u2 = fc2._ef_update_flag()
        return _TCFP12FusedMLPFunction.apply(
            x, fc1.weight, fc1.bias, fc2.weight, fc2.bias,
            fc1._error_state, fc1._param_name, fc2._error_state, fc2._param_name, u1, u2,
        )


def _is_mlp_triplet(m: nn.Module) -> bool:
    return (
        type(m) is nn.Sequential and len(m) == 3
        and isinstance(m[0], TCFPLinear) and isinstance(m[2], TCFPLinear)
        and isinstance(m[1], nn.GELU) and m[1].approximate == "none"
    )


def fuse_tcfp_mlp(model: nn.Module) -> nn.Module:
    """Turn every ``nn.Sequential(TCFPLinear, nn.GELU(), TCFPLinear)`` in
    ``model`` into a ``TCFPMLP`` holding the same three modules (run it after
    ``convert_to_tcfp``).  Children are replaced in place; if ``model`` itself
    is such a sequence, the new ``TCFPMLP`` is returned, else ``model``."""
    if _is_mlp_triplet(model):
        return TCFPMLP(*model)
    for name, child in model.named_children():
        new = fuse_tcfp_mlp(child)
        if new is not child:
            setattr(model, name, new)
    return model


def convert_to_tcfp(
    model: nn.Module,
    mode: TCFPMode = TCFPMode.TCFP12,
    block_size: int = DEFAULT_BLOCK_SIZE,
    skip_patterns: tuple[str, ...] = ("head",),
    *,
    nf4_residual: bool = False,
    nf_aware_scaling: bool = False,
    stochastic_rounding: bool = False,
    warmup_steps: int = 0,
    use_tensor_cores: bool = False,
    hp_grad_weight: bool = False,
    error_feedback: bool = True,
    delayed_scaling: bool = False,
    use_fused_kernel: bool = True,
    use_cuda_ext: bool = True,
    scale_block_size: int | None = None,
    abd: bool = False,
    srr: bool = False,
    _parent_path: str = "",
) -> nn.Module:
    """Replace ``nn.Linear`` layers with ``TCFPLinear`` in place
    (reference ``tcfp/nn/__init__.py:1190-1351``).

    Same eligibility rules: children are converted depth-first, names
    matching ``skip_patterns`` are skipped, a layer is converted only when
    ``in_features % block_size == 0`` and both dims are multiples of 16,
    and ``scale_block_size`` is dropped per layer when it does not divide
    both dims.  The new module shares the original Parameters and gets
    ``_param_name`` = its module path.  Layers the reference would put on
    the fake-quantise path (``use_tensor_cores=False`` or dims not multiples
    of 16) stay ``nn.Linear``; ``nn.LayerNorm`` / ``nn.Embedding`` are left
    unchanged for the same reason.
    """
    for name, module in model.named_children():
        full_path = f"{_parent_path}.{name}" if _parent_path else name
        convert_to_tcfp(
            module, mode, block_size, skip_patterns,
            nf4_residual=nf4_residual, nf_aware_scaling=nf_aware_scaling,
            stochastic_rounding=stochastic_rounding, warmup_steps=warmup_steps,
            use_tensor_cores=use_tensor_cores, hp_grad_weight=hp_grad_weight,
            error_feedback=error_feedback, delayed_scaling=delayed_scaling,
            use_fused_kernel=use_fused_kernel, use_cuda_ext=use_cuda_ext,
            scale_block_size=scale_block_size, abd=abd, srr=srr, _parent_path=full_path,
        )
        if any(pat in name for pat in skip_patterns):
            continue
        if not isinstance(module, nn.Linear) or isinstance(module, TCFPLinear):
            continue
        if module.in_features % block_size != 0:
            continue
        layer_tc = use_tensor_cores and (
            module.in_features % 16 == 0 and module.out_features % 16 == 0
        )
        if not layer_tc:
            continue
        layer_sbs = scale_block_size
        if layer_sbs is not None and (
            module.in_features % layer_sbs != 0 or module.out_features % layer_sbs != 0
        ):
            layer_sbs = None
        new_module = TCFPLinear(
            module.in_features, module.out_features, bias=module.bias is not None,
            mode=mode, block_size=block_size, nf4_residual=nf4_residual,
            nf_aware_scaling=nf_aware_scaling, stochastic_rounding=stochastic_rounding,
            warmup_steps=warmup_steps, use_tensor_cores=True, hp_grad_weight=hp_grad_weight,
            error_feedback=error_feedback, delayed_scaling=delayed_scaling,
            use_fused_kernel=use_fused_kernel, use_cuda_ext=use_cuda_ext,
            scale_block_size=layer_sbs, abd=abd, srr=srr,
            device="meta",
        )
        new_module._param_name = full_path
        new_module.weight = module.weight
        if module.bias is not None:
            new_module.bias = module.bias
        setattr(model, name, new_module)
    return model
