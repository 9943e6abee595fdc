"""Operator API of the TCFP-12 hot path, backed by hand-written HIP (gfx950).

Names, argument meaning, output layouts and error behaviour follow the
reference's Python wrappers (``tcfp/kernels.py:1545-2469``) so that
``tcfp_amd.nn`` -- and users of the reference's operator layer -- can switch
over unchanged.  Every op runs the HIP kernels in ``libtcfp_hip.so`` on the
tensors' GPU and current stream; there is no CPU or Triton path.

Additions over the reference interface, all keyword-only:

* ``out_dtype`` on the GEMMs (bf16 output for the raw-GEMM benchmark),
* ``bias`` fused into the GEMM epilogue,
* transposed operand copies (``w_hi_t``/``w_lo_t``) so dgrad and wgrad use
  the same K-contiguous MFMA kernel as the forward.
"""
from __future__ import annotations

import torch

from . import _hip
from ._hip import DTYPE_BF16, DTYPE_F32, FP8_E4M3, FP8_E5M2, check, ptr

_FP8_E4M3_MAX = 448.0
_FP8_E5M2_MAX = 57344.0

_FMT = {torch.float8_e4m3fn: FP8_E4M3, torch.float8_e5m2: FP8_E5M2}


def is_hip_available() -> bool:
    """HIP library built and a GPU visible."""
    return _hip.is_available()


def is_triton_available() -> bool:
    """The reference's gate for its fused-kernel tier
    (``tcfp/kernels.py:1537-1539``, used at ``tcfp/nn/__init__.py:40-55``);
    here the tier is the HIP library, so this is :func:`is_hip_available`."""
    return _hip.is_available()


def _fmt(dtype: torch.dtype) -> int:
    try:
        return _FMT[dtype]
    except KeyError:
        raise TypeError(f"unsupported fp8 dtype {dtype}") from None


def _in_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"unsupported input dtype {t.dtype}: expected float32 or bfloat16")


def _out_dtype(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"unsupported output dtype {dtype}")


def _bias_f32(bias: torch.Tensor, n: int) -> torch.Tensor:
    """fp32, contiguous, 16-byte aligned copy of the bias (the GEMM epilogue
    reads it as 16-byte vectors)."""
    b = bias.to(torch.float32).contiguous()
    assert b.shape == (n,), f"bias shape {tuple(b.shape)} != ({n},)"
    if b.data_ptr() % 16 != 0:
        b = b.clone()
    return b


def _scalar(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.numel() != 1 or t.dtype != torch.float32:
        raise ValueError(f"{name} must be a single-element float32 tensor")
    return t if t.is_contiguous() else t.contiguous()


# ---------------------------------------------------------------------------
# Per-tensor quantisation
# ---------------------------------------------------------------------------


def quantize_per_tensor(
    x: torch.Tensor,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    scale: torch.Tensor | None = None,
    transpose: bool = False,
    return_scale: bool = False,
):
    """Per-tensor FP8 cast with amax scaling (``to_fp8_e4m3`` / ``to_fp8_e5m2``
    semantics, reference ``tcfp/core.py:85-158``).

    Returns ``(q, inv)``, plus ``q_t`` ([cols, rows], the transposed codes of
    the 2-D view) when ``transpose``, plus the fp32 ``scale`` when
    ``return_scale``.  ``x`` is viewed as ``[numel / x.shape[-1], x.shape[-1]]``.
    """
    dev = _hip.require_gpu(x, scale)
    xc = x if x.is_contiguous() else x.contiguous()
    cols = xc.shape[-1] if xc.dim() > 0 else 1
    rows = xc.numel() // cols if cols else 0
    q = torch.empty(x.shape, dtype=fp8_dtype, device=dev)
    q_t = torch.empty((cols, rows), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    scale_out = torch.empty(1, dtype=torch.float32, device=dev) if return_scale else None
    s_in = _scalar(scale.to(torch.float32), "scale") if scale is not None else None
    ws = _hip.workspace(dev) if scale is None else None
    check(
        _hip.lib().tcfp_quantize_per_tensor(
            ptr(xc), _in_dtype(xc), rows, cols, _fmt(fp8_dtype), ptr(s_in), ptr(q), ptr(q_t),
            ptr(scale_out), ptr(inv), ptr(ws), _hip.stream_of(dev),
        ),
        "quantize_per_tensor",
    )
    out = (q, inv)
    if transpose:
        out = out + (q_t,)
    if return_scale:
        out = out + (scale_out,)
    return out


def quantize_per_tensor_sr(
    x: torch.Tensor,
    scale: torch.Tensor | None = None,
    seed: int | None = None,
    return_scale: bool = False,
):
    """Per-tensor FP8 E4M3 cast with stochastic rounding (``to_fp8_e4m3_sr``
    semantics, reference ``tcfp/core.py:109-134`` -> ``stochastic_round_to_
    fp8_e4m3``, ``:418-464``).  The scale follows the amax rule of
    :func:`quantize_per_tensor` (or ``scale``); each code is the round-to-
    nearest candidate or its neighbour toward the scaled value, chosen with
    the reference's probability from a Philox4x32-10 stream keyed by
    ``seed`` (drawn from torch's CPU generator when None).  Returns ``(q,
    inv)`` (plus the fp32 ``scale`` with ``return_scale``)."""
    dev = _hip.require_gpu(x, scale)
    xc = x if x.is_contiguous() else x.contiguous()
    cols = xc.shape[-1] if xc.dim() > 0 else 1
    rows = xc.numel() // cols if cols else 0
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=dev)
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    scale_out = torch.empty(1, dtype=torch.float32, device=dev) if return_scale else None
    s_in = _scalar(scale.to(torch.float32), "scale") if scale is not None else None
    ws = _hip.workspace(dev) if scale is None else None
    if seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    check(
        _hip.lib().tcfp_quantize_per_tensor_sr(
            ptr(xc), _in_dtype(xc), rows, cols, ptr(s_in), int(seed), 0, ptr(q), ptr(scale_out),
            ptr(inv), ptr(ws), _hip.stream_of(dev),
        ),
        "quantize_per_tensor_sr",
    )
    return (q, inv, scale_out) if return_scale else (q, inv)


def block_scales(
    x: torch.Tensor,
    block_size: int,
    fp8_max: float = _FP8_E4M3_MAX,
) -> torch.Tensor:
    """Power-of-two block scales ``2^ceil(log2(amax / fp8_max))`` per run of
    ``block_size`` elements along the last axis, in ``x``'s dtype (fp32 or
    bf16), shape ``x.shape[:-1] + (D // block_size,)`` (reference
    ``compute_block_scales``, ``tcfp/core.py:221-252``)."""
    dev = _hip.require_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"block scales support float32 and bfloat16 tensors, got {x.dtype}")
    if x.dim() == 0:
        raise ValueError("block scales need at least one dimension")
    d = x.shape[-1]
    xc = x if x.is_contiguous() else x.contiguous()
    rows = xc.numel() // d if d else 0
    out = torch.empty((*x.shape[:-1], d // block_size), dtype=x.dtype, device=dev)
    check(
        _hip.lib().tcfp_block_scales(
            ptr(xc), _in_dtype(xc), rows, d, int(block_size), float(fp8_max), ptr(out),
            _hip.stream_of(dev),
        ),
        "block_scales",
    )
    return out


def quantize_per_tensor_colsum(
    x: torch.Tensor,
    fp8_dtype: torch.dtype = torch.float8_e5m2,
    transpose: bool = False,
):
    """Per-tensor FP8 cast (amax scaling, as ``quantize_per_tensor``) that
    also returns the column sums of the 2-D view, read in the same pass.

    For a gradient this gives the bias gradient (the reference's
    ``grad_2d.sum(0)``, ``tcfp/nn/__init__.py:558``) alongside the E5M2
    codes (``:494``).  Returns ``(q, inv, col_sum)`` or, with ``transpose``,
    ``(q, inv, q_t, col_sum)``.  Needs ``x.shape[-1] % 8 == 0``.
    """
    dev = _hip.require_gpu(x)
    xc = x if x.is_contiguous() else x.contiguous()
    cols = xc.shape[-1]
    rows = xc.numel() // cols if cols else 0
    if cols % 8 != 0:
        raise ValueError(f"column count ({cols}) must be divisible by 8")
    q = torch.empty(x.shape, dtype=fp8_dtype, device=dev)
    q_t = torch.empty((cols, rows), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    cs = torch.empty(cols, dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_colsum_workspace_bytes(rows, cols))
    cws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_quantize_per_tensor_colsum(
            ptr(xc), _in_dtype(xc), rows, cols, _fmt(fp8_dtype), ptr(q), ptr(q_t), ptr(inv),
            ptr(cs), ptr(_hip.workspace(dev)), ptr(cws), nbytes, _hip.stream_of(dev),
        ),
        "quantize_per_tensor_colsum",
    )
    if transpose:
        return q, inv, q_t, cs
    return q, inv, cs


def gelu_quantize_per_tensor(
    h: torch.Tensor,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    transpose: bool = False,
    return_act: bool = False,
    return_dgelu: bool = False,
):
    """``quantize_per_tensor(torch.nn.functional.gelu(h))`` with the GELU
    evaluated inside the amax and quantising passes (the producer of the next
    layer's activation quantisation, ``tcfp/nn/__init__.py:390`` applied to a
    GELU output).

    ``h`` is fp32.  ``gelu(h)`` is computed as torch computes it (erf form,
    bit for bit) and quantised with the per-tensor amax rule.  Returns
    ``(q, inv)``, plus ``q_t`` when ``transpose``, plus the fp32 activation
    when ``return_act``, plus the GELU derivative factor ``d`` (torch's GELU
    backward is ``dy * d`` bit for bit) when ``return_dgelu``.
    """
    dev = _hip.require_gpu(h)
    if h.dtype != torch.float32:
        raise AssertionError(f"h must be float32, got {h.dtype}")
    hc = h if h.is_contiguous() else h.contiguous()
    cols = hc.shape[-1] if hc.dim() > 0 else 1
    rows = hc.numel() // cols if cols else 0
    if return_dgelu and cols % 8 != 0:
        raise ValueError(f"return_dgelu needs a last dim divisible by 8, got {cols}")
    # a ragged last dim quantises gelu(h) from a stored copy
    store = return_act or cols % 8 != 0
    act = torch.empty(h.shape, dtype=torch.float32, device=dev) if store else None
    dg = torch.empty(h.shape, dtype=torch.float32, device=dev) if return_dgelu else None
    q = torch.empty(h.shape, dtype=fp8_dtype, device=dev)
    q_t = torch.empty((cols, rows), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    check(
        _hip.lib().tcfp_gelu_quantize_per_tensor(
            ptr(hc), rows, cols, _fmt(fp8_dtype), ptr(act), ptr(dg), ptr(q), ptr(q_t), ptr(inv),
            ptr(_hip.workspace(dev)), _hip.stream_of(dev),
        ),
        "gelu_quantize_per_tensor",
    )
    out = (q, inv)
    if transpose:
        out = out + (q_t,)
    if return_act:
        out = out + (act,)
    if return_dgelu:
        out = out + (dg,)
    return out


def gelu_backward_quantize_per_tensor_colsum(
    dy: torch.Tensor,
    h: torch.Tensor,
    fp8_dtype: torch.dtype = torch.float8_e5m2,
    transpose: bool = False,
    return_grad: bool = False,
):
    """The gradient of a GELU's input, ``g = gelu'(h) * dy`` (as torch's GELU
    backward computes it, bit for bit), quantised per tensor with its column
    sums from the same pass (``quantize_per_tensor_colsum(g)``: the E5M2
    gradient quantisation at ``tcfp/nn/__init__.py:494`` and the bias
    gradient ``grad_2d.sum(0)`` at ``:558``).

    ``dy`` and ``h`` are fp32 of one shape, last dim divisible by 8.  Returns
    ``(q, inv, col_sum)`` or, with ``transpose``, ``(q, inv, q_t, col_sum)``;
    ``return_grad`` appends ``g``.
    """
    dev = _hip.require_gpu(dy, h)
    if dy.dtype != torch.float32 or h.dtype != torch.float32:
        raise AssertionError("dy and h must be float32")
    if dy.shape != h.shape:
        raise AssertionError(f"shape mismatch: dy {tuple(dy.shape)} vs h {tuple(h.shape)}")
    dc = dy if dy.is_contiguous() else dy.contiguous()
    hc = h if h.is_contiguous() else h.contiguous()
    cols = dc.shape[-1]
    rows = dc.numel() // cols if cols else 0
    if cols % 8 != 0:
        raise ValueError(f"column count ({cols}) must be divisible by 8")
    g = torch.empty(dy.shape, dtype=torch.float32, device=dev)
    q = torch.empty(dy.shape, dtype=fp8_dtype, device=dev)
    q_t = torch.empty((cols, rows), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    cs = torch.empty(cols, dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_colsum_workspace_bytes(rows, cols))
    cws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_gelu_backward_quantize_per_tensor_colsum(
            ptr(dc), ptr(hc), rows, cols, _fmt(fp8_dtype), ptr(g), ptr(q), ptr(q_t), ptr(inv),
            ptr(cs), ptr(_hip.workspace(dev)), ptr(cws), nbytes, _hip.stream_of(dev),
        ),
        "gelu_backward_quantize_per_tensor_colsum",
    )
    out = (q, inv, q_t, cs) if transpose else (q, inv, cs)
    if return_grad:
        out = out + (g,)
    return out


def dual_quantize_per_tensor(
    weight: torch.Tensor,
    error_buf: torch.Tensor | None = None,
    update_ef: bool = True,
    stochastic_lo: bool = False,
    transposed: bool = False,
    seed: int | None = None,
    sigma_factor: float | None = None,
    stochastic_hi: bool = False,
):
    """W (+ error feedback) -> (W_hi, W_lo, inv_hi, inv_lo[, W_hi^T, W_lo^T]).

    The per-tensor decomposition of ``_TCFP12TensorCoreFunction.forward``
    (reference ``tcfp/nn/__init__.py:343-383``).  ``error_buf`` ([N, K]
    fp32) is read as the previous error and, when ``update_ef``, overwritten
    in place with ``W - (deq(hi) + deq(lo))``.  ``stochastic_lo`` rounds
    W_lo stochastically (SRR); the Philox key is drawn from torch's CPU
    generator unless ``seed`` is given.

    ``sigma_factor`` selects NF-aware W_hi scaling (``nf_aware_scaling``,
    reference ``:356-359`` -> ``to_fp8_e4m3_nf_aware``, ``tcfp/core.py:
    161-193``): the W_hi scale is ``448 / (sigma_factor * std(W + ef))``, or
    the amax rule when that std is below 1e-6.  ``stochastic_hi`` (only with
    ``sigma_factor``) rounds the W_hi codes stochastically.
    """
    dev = _hip.require_gpu(weight, error_buf)
    assert weight.dim() == 2, "weight must be 2-D (N, K)"
    w = weight if weight.is_contiguous() else weight.contiguous()
    n, k = w.shape
    if error_buf is not None:
        assert error_buf.dtype == torch.float32, "error_buf must be float32"
        assert error_buf.shape == (n, k), (
            f"error_buf shape {tuple(error_buf.shape)} != weight shape {(n, k)}"
        )
        assert error_buf.is_contiguous(), "error_buf must be contiguous"
    w_hi = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
    w_lo = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
    inv_hi = torch.empty(1, dtype=torch.float32, device=dev)
    inv_lo = torch.empty(1, dtype=torch.float32, device=dev)
    w_hi_t = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if transposed else None
    w_lo_t = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if transposed else None
    if stochastic_hi and sigma_factor is None:
        raise ValueError("stochastic_hi applies to NF-aware scaling only (pass sigma_factor)")
    if (stochastic_lo or stochastic_hi) and seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    if sigma_factor is not None:
        _dual_quantize_nf(
            w, n, k, error_buf, update_ef, sigma_factor, stochastic_hi, stochastic_lo, seed,
            None, None, 0.0, False, None, None, w_hi, w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t, dev,
        )
        if transposed:
            return w_hi, w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t
        return w_hi, w_lo, inv_hi, inv_lo
    check(
        _hip.lib().tcfp_dual_quantize_per_tensor(
            ptr(w), _in_dtype(w), n, k, ptr(error_buf), int(bool(update_ef)),
            int(bool(stochastic_lo)), int(seed or 0), 0, ptr(w_hi), ptr(w_lo), ptr(inv_hi),
            ptr(inv_lo), ptr(w_hi_t), ptr(w_lo_t), ptr(_hip.workspace(dev)),
            _hip.stream_of(dev),
        ),
        "dual_quantize_per_tensor",
    )
    if transposed:
        return w_hi, w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t
    return w_hi, w_lo, inv_hi, inv_lo


def quantize_batch(dual=(), act=()):
    """Several independent per-tensor quantisations in three launches in all
    (``tcfp_quantize_batch``; no reference counterpart).

    ``dual``: ``(weight, error_buf, update_ef, transposed)`` tuples, each
    quantised as ``dual_quantize_per_tensor(weight, error_buf, update_ef,
    transposed=transposed)`` (no stochastic rounding); ``act``: ``(x,
    fp8_dtype, transpose)`` tuples, each as ``quantize_per_tensor(x,
    fp8_dtype, transpose=transpose)`` (2-D ``x``).  Returns the two lists
    of result tuples, bit for bit those calls' results.  Tensors the batch
    does not take (empty, a last dimension not divisible by 8, more than
    four in all) are quantised by those calls instead.
    """
    dual, act = list(dual), list(act)
    fits = (0 < len(dual) + len(act) <= _hip.MAX_BATCH_JOBS
            and all(w.dim() == 2 and w.numel() > 0 and w.shape[1] % 8 == 0 for w, *_ in dual)
            and all(x.dim() == 2 and x.numel() > 0 and x.shape[1] % 8 == 0 for x, *_ in act))
    if not fits:
        return ([dual_quantize_per_tensor(w, e, u, transposed=t) for w, e, u, t in dual],
                [quantize_per_tensor(x, f, transpose=t) for x, f, t in act])
    dev = _hip.require_gpu(*[t for w, e, _, _ in dual for t in (w, e)],
                           *[x for x, _, _ in act])
    jobs = (_hip.QuantJob * (len(dual) + len(act)))()
    res_d, res_a = [], []
    for i, (w, e, u, t) in enumerate(dual):
        w = w if w.is_contiguous() else w.contiguous()
        n, k = w.shape
        if e is not None:
            assert e.dtype == torch.float32, "error_buf must be float32"
            assert e.shape == (n, k), f"error_buf shape {tuple(e.shape)} != weight shape {(n, k)}"
            assert e.is_contiguous(), "error_buf must be contiguous"
        hi = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
        lo = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
        ih = torch.empty(1, dtype=torch.float32, device=dev)
        il = torch.empty(1, dtype=torch.float32, device=dev)
        ht = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if t else None
        lt = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if t else None
        jobs[i] = _hip.QuantJob(_hip.JOB_DUAL, ptr(w), _in_dtype(w), n, k, ptr(e), int(bool(u)),
                                0, ptr(hi), ptr(ht), ptr(ih), ptr(lo), ptr(lt), ptr(il))
        res_d.append((hi, lo, ih, il, ht, lt) if t else (hi, lo, ih, il))
    for i, (x, f, t) in enumerate(act, start=len(dual)):
        x = x if x.is_contiguous() else x.contiguous()
        rows, cols = x.shape
        q = torch.empty((rows, cols), dtype=f, device=dev)
        qt = torch.empty((cols, rows), dtype=f, device=dev) if t else None
        inv = torch.empty(1, dtype=torch.float32, device=dev)
        jobs[i] = _hip.QuantJob(_hip.JOB_ACT, ptr(x), _in_dtype(x), rows, cols, None, 0, _fmt(f),
                                ptr(q), ptr(qt), ptr(inv), None, None, None)
        res_a.append((q, inv, qt) if t else (q, inv))
    ws = _hip.batch_workspace(dev)
    check(_hip.lib().tcfp_quantize_batch(len(jobs), jobs, ptr(ws), ws.numel(),
                                         _hip.stream_of(dev)), "quantize_batch")
    return res_d, res_a


def _dual_quantize_nf(w, n, k, error_buf, update_ef, sigma_factor, stochastic_hi, stochastic_lo,
                      seed, prev, ratio_prev, decay, validate, amax_out, ratio_out, w_hi, w_lo,
                      inv_hi, inv_lo, w_hi_t, w_lo_t, dev) -> None:
    """``tcfp_dual_quantize_per_tensor_nf`` (``amax_out`` None: no delayed
    scaling)."""
    if n * k == 0:
        raise RuntimeError(
            "NF-aware dual quantisation of an empty weight (the reference's residual amax "
            "of an empty tensor raises)"
        )
    check(
        _hip.lib().tcfp_dual_quantize_per_tensor_nf(
            ptr(w), _in_dtype(w), n, k, ptr(error_buf), int(bool(update_ef)),
            float(sigma_factor), int(bool(stochastic_hi)), int(bool(stochastic_lo)),
            int(seed or 0), 0, ptr(prev), ptr(ratio_prev), float(decay), 1.0 - float(decay),
            int(bool(validate)), ptr(amax_out), ptr(ratio_out), ptr(w_hi), ptr(w_lo),
            ptr(inv_hi), ptr(inv_lo), ptr(w_hi_t), ptr(w_lo_t), ptr(_hip.workspace(dev)),
            _hip.stream_of(dev),
        ),
        "dual_quantize_per_tensor (NF-aware)",
    )


def dual_quantize_per_tensor_delayed(
    weight: torch.Tensor,
    error_buf: torch.Tensor | None,
    state,
    name: str,
    update_ef: bool = True,
    transposed: bool = False,
    sigma_factor: float | None = None,
    stochastic_hi: bool = False,
    seed: int | None = None,
):
    """Per-tensor dual quantisation with delayed scaling, updating ``state``.

    ``_delayed_quantise_w_hi`` / ``_delayed_quantise_w_lo`` of the reference
    (``tcfp/nn/__init__.py:250-309``) on an :class:`ErrorFeedbackState`:
    the W_hi scale comes from the EMA of the amax (``_delayed_amax[name +
    ".w_hi"]``), the W_lo scale from the measured residual amax on
    validation steps (``should_validate_residual``; the ratio EMA
    ``_residual_ratio[name + ".ratio"]`` is updated) and from the predicted
    one otherwise.  The state tensors are replaced by new 0-dim fp32
    tensors, as the reference's EMA rebinds them.  Returns what
    :func:`dual_quantize_per_tensor` returns.  ``sigma_factor`` /
    ``stochastic_hi``: the NF branch of ``_delayed_quantise_w_hi``
    (``:263-275``), the sigma target in place of the amax.
    """
    dev = _hip.require_gpu(weight, error_buf)
    assert weight.dim() == 2, "weight must be 2-D (N, K)"
    w = weight if weight.is_contiguous() else weight.contiguous()
    n, k = w.shape
    if error_buf is not None:
        assert error_buf.dtype == torch.float32, "error_buf must be float32"
        assert error_buf.shape == (n, k), (
            f"error_buf shape {tuple(error_buf.shape)} != weight shape {(n, k)}"
        )
        assert error_buf.is_contiguous(), "error_buf must be contiguous"
    validate = state.should_validate_residual(name)
    amax_key, ratio_key = name + ".w_hi", f"{name}.ratio"

    def _scalar_state(t):
        if t is None:
            return None
        return t.detach().to(device=dev, dtype=torch.float32).reshape(()).contiguous()

    prev = _scalar_state(state._delayed_amax.get(amax_key))
    ratio_prev = _scalar_state(state._residual_ratio.get(ratio_key))
    amax_out = torch.empty((), dtype=torch.float32, device=dev)
    ratio_out = torch.empty((), dtype=torch.float32, device=dev) if validate else None
    w_hi = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
    w_lo = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
    inv_hi = torch.empty(1, dtype=torch.float32, device=dev)
    inv_lo = torch.empty(1, dtype=torch.float32, device=dev)
    w_hi_t = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if transposed else None
    w_lo_t = torch.empty((k, n), dtype=torch.float8_e4m3fn, device=dev) if transposed else None
    decay = float(state._ema_decay)
    if stochastic_hi and sigma_factor is None:
        raise ValueError("stochastic_hi applies to NF-aware scaling only (pass sigma_factor)")
    if sigma_factor is not None:
        if stochastic_hi and seed is None:
            seed = int(torch.randint(0, 2**62, (1,)).item())
        _dual_quantize_nf(
            w, n, k, error_buf, update_ef, sigma_factor, stochastic_hi, False, seed, prev,
            ratio_prev, decay, validate, amax_out, ratio_out, w_hi, w_lo, inv_hi, inv_lo,
            w_hi_t, w_lo_t, dev,
        )
    else:
        check(
            _hip.lib().tcfp_dual_quantize_per_tensor_delayed(
                ptr(w), _in_dtype(w), n, k, ptr(error_buf), int(bool(update_ef)), ptr(prev),
                ptr(ratio_prev), decay, 1.0 - decay, int(validate), ptr(amax_out),
                ptr(ratio_out), ptr(w_hi), ptr(w_lo), ptr(inv_hi), ptr(inv_lo), ptr(w_hi_t),
                ptr(w_lo_t), ptr(_hip.workspace(dev)), _hip.stream_of(dev),
            ),
            "dual_quantize_per_tensor_delayed",
        )
    state._delayed_amax[amax_key] = amax_out
    if validate:
        state._residual_ratio[ratio_key] = ratio_out
    if transposed:
        return w_hi, w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t
    return w_hi, w_lo, inv_hi, inv_lo


def transpose_fp8(t: torch.Tensor) -> torch.Tensor:
    """Contiguous transpose of a 2-D 8-bit tensor (HIP, LDS-tiled)."""
    dev = _hip.require_gpu(t)
    assert t.dim() == 2 and t.element_size() == 1, "expects a 2-D 8-bit tensor"
    src = t if t.is_contiguous() else t.contiguous()
    rows, cols = src.shape
    out = torch.empty((cols, rows), dtype=t.dtype, device=dev)
    check(
        _hip.lib().tcfp_transpose_u8(ptr(src), rows, cols, ptr(out), _hip.stream_of(dev)),
        "transpose_fp8",
    )
    return out


# ---------------------------------------------------------------------------
# GEMMs
# ---------------------------------------------------------------------------


def _gemm_operand(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype not in _FMT:
        raise TypeError(f"{name} must be float8_e4m3fn or float8_e5m2, got {t.dtype}")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D")
    if t.stride(1) != 1 or t.stride(0) % 16 != 0 or t.data_ptr() % 16 != 0:
        t = t.contiguous()
    return t


def _dual_gemm(a, b_hi, b_lo, s_a, s_hi, s_lo, bias, out_dtype):
    dev = _hip.require_gpu(a, b_hi, b_lo, s_a, s_hi, s_lo, bias)
    a = _gemm_operand(a, "A")
    b_hi = _gemm_operand(b_hi, "B_hi")
    b_lo = _gemm_operand(b_lo, "B_lo") if b_lo is not None else None
    m, k = a.shape
    n = b_hi.shape[0]
    if k % 16 != 0:
        raise ValueError(f"K ({k}) must be divisible by 16")
    if b_hi.stride(0) != (b_lo.stride(0) if b_lo is not None else b_hi.stride(0)):
        b_lo = b_lo.contiguous()
        b_hi = b_hi.contiguous()
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    if bias is not None:
        bias = _bias_f32(bias, n)
    check(
        _hip.lib().tcfp_dual_gemm(
            ptr(a), _fmt(a.dtype), a.stride(0), ptr(b_hi), ptr(b_lo), _fmt(b_hi.dtype),
            b_hi.stride(0), m, n, k, ptr(_scalar(s_a, "scale_a")), ptr(_scalar(s_hi, "scale_hi")),
            ptr(_scalar(s_lo, "scale_lo")) if s_lo is not None else None, ptr(bias), ptr(out),
            _out_dtype(out_dtype), n, _hip.stream_of(dev),
        ),
        "dual_gemm",
    )
    return out


def _gemm_operands(a, b_hi, b_lo):
    a = _gemm_operand(a, "A")
    b_hi = _gemm_operand(b_hi, "B_hi")
    b_lo = _gemm_operand(b_lo, "B_lo")
    if a.shape[1] != b_hi.shape[1] or b_hi.shape != b_lo.shape:
        raise AssertionError(
            f"Shape mismatch: A{tuple(a.shape)}, B_hi{tuple(b_hi.shape)}, B_lo{tuple(b_lo.shape)}"
        )
    if a.shape[1] % 16 != 0:
        raise ValueError(f"K ({a.shape[1]}) must be divisible by 16")
    if b_hi.stride(0) != b_lo.stride(0):
        b_hi, b_lo = b_hi.contiguous(), b_lo.contiguous()
    return a, b_hi, b_lo


def dual_gemm_gelu_quantize(
    act_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    act_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
    *,
    bias: torch.Tensor | None = None,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    transpose: bool = False,
    return_act: bool = False,
    return_dgelu: bool = False,
):
    """``h = fused_dual_gemm_forward(...)`` (fp32) and
    ``gelu_quantize_per_tensor(h)`` in one call, the GELU's amax taken from
    the maximum of h the GEMM's epilogue records where the persistent launch
    runs (the first layer of a TCFP -> GELU -> TCFP pair:
    ``tcfp/kernels.py:1545-1601``, then ``tcfp/nn/__init__.py:390`` on the
    GELU output).  Same bits as the two calls.

    Returns ``(h, q, inv)``, then ``q_t`` when ``transpose``, then gelu(h)
    when ``return_act``, then the GELU derivative factor when
    ``return_dgelu`` (what ``dual_gemm_dgelu_quantize_colsum`` takes).
    """
    dev = _hip.require_gpu(act_fp8, w_hi_fp8, w_lo_fp8, act_inv, w_hi_inv, w_lo_inv, bias)
    a, b_hi, b_lo = _gemm_operands(act_fp8, w_hi_fp8, w_lo_fp8)
    m, k = a.shape
    n = b_hi.shape[0]
    if return_dgelu and n % 8 != 0:
        raise ValueError(f"return_dgelu needs N divisible by 8, got {n}")
    h = torch.empty((m, n), dtype=torch.float32, device=dev)
    store = return_act or n % 8 != 0
    act = torch.empty((m, n), dtype=torch.float32, device=dev) if store else None
    dg = torch.empty((m, n), dtype=torch.float32, device=dev) if return_dgelu else None
    q = torch.empty((m, n), dtype=fp8_dtype, device=dev)
    q_t = torch.empty((n, m), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    if bias is not None:
        bias = _bias_f32(bias, n)
    check(
        _hip.lib().tcfp_dual_gemm_gelu_quantize(
            ptr(a), _fmt(a.dtype), a.stride(0), ptr(b_hi), ptr(b_lo), _fmt(b_hi.dtype),
            b_hi.stride(0), m, n, k, ptr(_scalar(act_inv, "scale_a")),
            ptr(_scalar(w_hi_inv, "scale_hi")), ptr(_scalar(w_lo_inv, "scale_lo")), ptr(bias),
            ptr(h), ptr(act), ptr(dg), _fmt(fp8_dtype), ptr(q), ptr(q_t), ptr(inv),
            ptr(_hip.workspace(dev)), _hip.stream_of(dev),
        ),
        "dual_gemm_gelu_quantize",
    )
    out = (h, q, inv)
    if transpose:
        out = out + (q_t,)
    if return_act:
        out = out + (act,)
    if return_dgelu:
        out = out + (dg,)
    return out


def gelu_amax_rule_status() -> tuple[bool, bool, float]:
    """``(checked, holds, bound)`` of the once-per-device premise check of
    ``dual_gemm_gelu_quantize``'s amax rule (synchronous)."""
    import ctypes

    c, h, b = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_float(0.0)
    check(_hip.lib().tcfp_gelu_amax_rule_status(ctypes.addressof(c), ctypes.addressof(h),
                                                 ctypes.addressof(b)), "gelu_amax_rule_status")
    return bool(c.value), bool(h.value), float(b.value)


def dual_gemm_dgelu_quantize_colsum(
    grad_fp8: torch.Tensor,
    w_hi_t: torch.Tensor,
    w_lo_t: torch.Tensor,
    grad_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
    dgelu: torch.Tensor,
    *,
    fp8_dtype: torch.dtype = torch.float8_e5m2,
    transpose: bool = False,
    col_sum: bool = True,
    return_grad: bool = False,
    codes: bool = True,
):
    """The dgrad of the second layer of a TCFP -> GELU -> TCFP pair with the
    GELU backward in the GEMM's epilogue: ``g = (grad @ W) * dgelu``
    (``fused_dual_gemm_backward_dx``, ``tcfp/kernels.py:1604-1666``, with the
    transposed weight codes ``w_*_t`` [d_in, d_out], then torch's GELU
    backward from the derivative factors ``dual_gemm_gelu_quantize`` /
    ``gelu_quantize_per_tensor`` return) quantised per tensor with its column
    sums (``tcfp/nn/__init__.py:494, 558`` on the first layer's gradient).
    Same bits as ``_dual_gemm`` followed by torch's GELU backward and
    ``quantize_per_tensor_colsum``.

    Returns ``(q, inv)``, then ``q_t`` when ``transpose``, then the column
    sums when ``col_sum``, then ``g`` when ``return_grad``.  ``codes=False``
    (with ``transpose``) writes only the transposed codes; ``q`` is then
    None.
    """
    if not codes and not transpose:
        raise ValueError("codes=False needs transpose=True (the codes are written one way or both)")
    dev = _hip.require_gpu(grad_fp8, w_hi_t, w_lo_t, grad_inv, w_hi_inv, w_lo_inv, dgelu)
    a, b_hi, b_lo = _gemm_operands(grad_fp8, w_hi_t, w_lo_t)
    m, k = a.shape
    n = b_hi.shape[0]
    if dgelu.dtype != torch.float32 or tuple(dgelu.shape) != (m, n):
        raise AssertionError(
            f"dgelu must be float32 of shape {(m, n)}, got {dgelu.dtype} {tuple(dgelu.shape)}")
    if n % 8 != 0:
        raise ValueError(f"column count ({n}) must be divisible by 8")
    dc = dgelu if dgelu.is_contiguous() else dgelu.contiguous()
    g = torch.empty((m, n), dtype=torch.float32, device=dev)
    q = torch.empty((m, n), dtype=fp8_dtype, device=dev) if codes else None
    q_t = torch.empty((n, m), dtype=fp8_dtype, device=dev) if transpose else None
    inv = torch.empty(1, dtype=torch.float32, device=dev)
    cs = torch.empty(n, dtype=torch.float32, device=dev) if col_sum else None
    nbytes = int(_hip.lib().tcfp_colsum_workspace_bytes(m, n)) if col_sum else 0
    cws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev) if col_sum else None
    check(
        _hip.lib().tcfp_dual_gemm_dgelu_quantize_colsum(
            ptr(a), _fmt(a.dtype), a.stride(0), ptr(b_hi), ptr(b_lo), _fmt(b_hi.dtype),
            b_hi.stride(0), m, n, k, ptr(_scalar(grad_inv, "scale_a")),
            ptr(_scalar(w_hi_inv, "scale_hi")), ptr(_scalar(w_lo_inv, "scale_lo")), ptr(dc),
            ptr(g), _fmt(fp8_dtype), ptr(q), ptr(q_t), ptr(inv), ptr(cs),
            ptr(_hip.workspace(dev)), ptr(cws), nbytes, _hip.stream_of(dev),
        ),
        "dual_gemm_dgelu_quantize_colsum",
    )
    out = (q, inv)
    if transpose:
        out = out + (q_t,)
    if col_sum:
        out = out + (cs,)
    if return_grad:
        out = out + (g,)
    return out


def fused_dual_gemm_forward(
    act_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    act_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
    *,
    bias: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``(act @ W_hi.T) * s_a s_hi + (act @ W_lo.T) * s_a s_lo`` (+ bias).

    Reference: ``fused_dual_gemm_forward`` (``tcfp/kernels.py:1545-1601``)
    and ``cuda_ext_dual_gemm_forward`` (``tcfp/cuda_ext.py:241-259``).
    act [M, K], W [N, K] FP8; returns [M, N] (fp32 by default).
    """
    M, K = act_fp8.shape
    N, K2 = w_hi_fp8.shape
    assert K == K2 and tuple(w_lo_fp8.shape) == (N, K), (
        f"Shape mismatch: act({M},{K}), w_hi({N},{K2}), w_lo{tuple(w_lo_fp8.shape)}"
    )
    return _dual_gemm(act_fp8, w_hi_fp8, w_lo_fp8, act_inv, w_hi_inv, w_lo_inv, bias, out_dtype)


def fused_dual_gemm_backward_dx(
    grad_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    grad_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
    *,
    w_hi_t: torch.Tensor | None = None,
    w_lo_t: torch.Tensor | None = None,
) -> torch.Tensor:
    """``dX = (grad @ W_hi) s_g s_hi + (grad @ W_lo) s_g s_lo`` (fp32 [M, D_in]).

    Reference: ``fused_dual_gemm_backward_dx`` (``tcfp/kernels.py:1604-1666``).
    grad [M, D_out] (E5M2), W [D_out, D_in].  ``w_hi_t``/``w_lo_t`` are the
    [D_in, D_out] copies emitted by the dual-quant kernel; without them the
    transposes are made here.
    """
    M, D_out = grad_fp8.shape
    D_out2, D_in = w_hi_fp8.shape
    assert D_out == D_out2 and tuple(w_lo_fp8.shape) == (D_out, D_in), (
        f"Shape mismatch: grad({M},{D_out}), "
        f"w_hi({D_out2},{D_in}), w_lo{tuple(w_lo_fp8.shape)}"
    )
    if w_hi_t is None:
        w_hi_t = transpose_fp8(w_hi_fp8)
    if w_lo_t is None:
        w_lo_t = transpose_fp8(w_lo_fp8)
    return _dual_gemm(grad_fp8, w_hi_t, w_lo_t, grad_inv, w_hi_inv, w_lo_inv, None, torch.float32)


def fp8_gemm_nt(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    *,
    out_dtype: torch.dtype = torch.float32,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """Single scaled FP8 GEMM ``(A @ B.T) * s_a s_b`` with A [M, K], B [N, K].

    The FP8 wgrad of ``tcfp/nn/__init__.py:546-555`` is
    ``fp8_gemm_nt(grad^T, act^T, grad_inv, act_inv)``; it also stands in for
    ``torch._scaled_mm`` in the reference's ABD dgrad (``:499-508``).
    """
    assert a_fp8.shape[1] == b_fp8.shape[1], (
        f"K mismatch: A {tuple(a_fp8.shape)} vs B {tuple(b_fp8.shape)}"
    )
    return _dual_gemm(a_fp8, b_fp8, None, scale_a, scale_b, None, bias, out_dtype)


# ---------------------------------------------------------------------------
# Block quantisation
# ---------------------------------------------------------------------------


_SCALE_FORMATS = ("exponent", "fp32")


def _scale_format(scale_format: str) -> bool:
    """True for fp32 block multipliers, False for the reference's exponents."""
    if scale_format not in _SCALE_FORMATS:
        raise ValueError(f"scale_format must be one of {_SCALE_FORMATS}, got {scale_format!r}")
    return scale_format == "fp32"


def block_quantize_fp8(
    tensor: torch.Tensor,
    block_size: int = 128,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    *,
    scale_format: str = "exponent",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(row, K-block) FP8 quantisation; returns ``(fp8 [M,K], scales
    [K // block_size, M])``.

    Reference: ``block_quantize_fp8`` (``tcfp/kernels.py:1675-1722``).
    ``scale_format="exponent"`` (the reference's format): int8 exponents,
    block value = fp8 * 2^exp.  ``scale_format="fp32"``: ``to_fp8_e4m3`` /
    ``to_fp8_e5m2`` (``tcfp/core.py:85-106, 137-158``) applied per block
    (scale = FP8_MAX / amax, not a power of two); the scales returned are
    the fp32 dequantisation multipliers ``1 / scale``, block value =
    fp8 * multiplier.
    """
    f32s = _scale_format(scale_format)
    dev = _hip.require_gpu(tensor)
    M, K = tensor.shape
    assert K % block_size == 0, f"K ({K}) must be divisible by block_size ({block_size})"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    x = tensor if tensor.is_contiguous() else tensor.contiguous()
    q = torch.empty((M, K), dtype=fp8_dtype, device=dev)
    scales = torch.empty((K // block_size, M), dtype=torch.float32 if f32s else torch.int8,
                         device=dev)
    fn = _hip.lib().tcfp_block_quantize_f32s if f32s else _hip.lib().tcfp_block_quantize
    check(
        fn(ptr(x), _in_dtype(x), M, K, block_size, _fmt(fp8_dtype), ptr(q), ptr(scales),
           _hip.stream_of(dev)),
        "block_quantize_fp8",
    )
    return q, scales


def block_dequantize_fp8(
    fp8_tensor: torch.Tensor,
    block_scales: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """``fp8 * 2^exp`` (int8 exponents) or ``fp8 * multiplier`` (fp32
    multipliers) -> fp32 [M, K] (reference ``tcfp/kernels.py:1725-1746``)."""
    dev = _hip.require_gpu(fp8_tensor, block_scales)
    M, K = fp8_tensor.shape
    q = fp8_tensor.contiguous()
    e = block_scales.contiguous()
    assert e.dtype in (torch.int8, torch.float32) and tuple(e.shape) == (K // block_size, M), (
        f"block_scales must be int8 or float32 ({K // block_size}, {M})"
    )
    out = torch.empty((M, K), dtype=torch.float32, device=dev)
    fn = (_hip.lib().tcfp_block_dequantize_f32s if e.dtype == torch.float32
          else _hip.lib().tcfp_block_dequantize)
    check(
        fn(ptr(q), _fmt(q.dtype), ptr(e), M, K, block_size, ptr(out), _hip.stream_of(dev)),
        "block_dequantize_fp8",
    )
    return out


def fused_dual_quantize_fp8(
    weight: torch.Tensor,
    block_size: int = 128,
    error_buf: torch.Tensor | None = None,
    stochastic_lo: bool = False,
    update_ef: bool = True,
    seed: int | None = None,
    *,
    scale_format: str = "exponent",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """W (+ EF) -> ``(w_hi, w_lo, scales_hi, scales_lo)``, one HBM pass.

    Reference: ``fused_dual_quantize_fp8`` (``tcfp/kernels.py:1749-1875``).
    The error update the reference runs afterwards in Python
    (``:1867-1873``) happens inside the same kernel here; ``error_buf`` is
    modified in place (unless ``update_ef=False``).  Scales are int8
    exponents [K // block_size, N]; W_lo blocks with zero residual carry
    the -128 sentinel.  ``scale_format="fp32"`` quantises both components
    with the per-block ``to_fp8_e4m3`` rule of :func:`block_quantize_fp8`
    and returns fp32 multipliers (no sentinel).
    """
    f32s = _scale_format(scale_format)
    assert weight.is_contiguous(), "Weight must be contiguous (N, K) row-major"
    N, K = weight.shape
    assert K % block_size == 0, f"K ({K}) must be divisible by block_size ({block_size})"
    if stochastic_lo and error_buf is not None:
        raise ValueError(
            "stochastic_lo and error_buf are mutually exclusive: "
            "SRR eliminates the need for error feedback buffers."
        )
    if error_buf is not None:
        assert error_buf.dtype == torch.float32, "error_buf must be float32"
        assert tuple(error_buf.shape) == (N, K), (
            f"error_buf shape {tuple(error_buf.shape)} != weight shape {(N, K)}"
        )
        assert error_buf.is_contiguous(), "error_buf must be contiguous"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    dev = _hip.require_gpu(weight, error_buf)
    num_kb = K // block_size
    w_hi = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=dev)
    w_lo = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=dev)
    sdt = torch.float32 if f32s else torch.int8
    sh = torch.empty((num_kb, N), dtype=sdt, device=dev)
    sl = torch.empty((num_kb, N), dtype=sdt, device=dev)
    if stochastic_lo and seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    fn = _hip.lib().tcfp_block_dual_quantize_f32s if f32s else _hip.lib().tcfp_block_dual_quantize
    check(
        fn(
            ptr(weight), _in_dtype(weight), N, K, block_size, ptr(error_buf),
            int(bool(update_ef)), int(bool(stochastic_lo)), int(seed or 0), 0, ptr(w_hi),
            ptr(w_lo), ptr(sh), ptr(sl), _hip.stream_of(dev),
        ),
        "fused_dual_quantize_fp8",
    )
    return w_hi, w_lo, sh, sl


# ---------------------------------------------------------------------------
# Block-scaled GEMMs
# ---------------------------------------------------------------------------


def _block_exps(e: torch.Tensor, rows: int, num_kb: int, name: str,
                dtype: torch.dtype = torch.int8) -> torch.Tensor:
    if e.dtype != dtype:
        what = "int8 power-of-two exponents" if dtype == torch.int8 else "float32 multipliers"
        raise TypeError(f"{name} must be {what} like the other scales, got {e.dtype}")
    if tuple(e.shape) != (num_kb, rows):
        raise ValueError(f"{name} must have shape ({num_kb}, {rows}), got {tuple(e.shape)}")
    return e if e.is_contiguous() else e.contiguous()


def _block_gemm(a, e_a, b_hi, b_lo, e_hi, e_lo, block_size, bias, out_dtype):
    dev = _hip.require_gpu(a, e_a, b_hi, b_lo, e_hi, e_lo, bias)
    a = _gemm_operand(a, "A")
    b_hi = _gemm_operand(b_hi, "B_hi")
    b_lo = _gemm_operand(b_lo, "B_lo") if b_lo is not None else None
    m, k = a.shape
    n = b_hi.shape[0]
    assert k % block_size == 0, f"K ({k}) not divisible by block_size ({block_size})"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    num_kb = k // block_size
    # int8 exponents (the reference's format) or fp32 multipliers, not mixed
    sdt = torch.float32 if e_a.dtype == torch.float32 else torch.int8
    e_a = _block_exps(e_a, m, num_kb, "scales_a", sdt)
    e_hi = _block_exps(e_hi, n, num_kb, "scales_b", sdt)
    e_lo = _block_exps(e_lo, n, num_kb, "scales_lo", sdt) if b_lo is not None else None
    if b_lo is not None and b_hi.stride(0) != b_lo.stride(0):
        b_hi, b_lo = b_hi.contiguous(), b_lo.contiguous()
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    if bias is not None:
        bias = _bias_f32(bias, n)
    fn = (_hip.lib().tcfp_block_dual_gemm_f32s if sdt == torch.float32
          else _hip.lib().tcfp_block_dual_gemm)
    check(
        fn(
            ptr(a), _fmt(a.dtype), a.stride(0), ptr(e_a), ptr(b_hi), ptr(b_lo),
            _fmt(b_hi.dtype), b_hi.stride(0), ptr(e_hi), ptr(e_lo), m, n, k, block_size,
            ptr(bias), ptr(out), _out_dtype(out_dtype), n, _hip.stream_of(dev),
        ),
        "block_dual_gemm",
    )
    return out


def block_scaled_gemm(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scales_a: torch.Tensor,
    scales_b: torch.Tensor,
    block_size: int = 128,
    *,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``C = sum_kb 2^sa[kb,m] 2^sb[kb,n] (A_kb @ B_kb^T)``, fp32 [M, N].

    Reference: ``block_scaled_gemm`` (``tcfp/kernels.py:1878-1936``).
    A [M, K], B [N, K] FP8; scales are the int8 exponents
    ``[K // block_size, rows]`` produced by ``block_quantize_fp8``.  The
    exponents enter the MFMA as hardware E8M0 block scales.  fp32
    multipliers (``scale_format="fp32"``; both operands) are accepted too:
    ``C = sum_kb sa[kb,m] sb[kb,n] (A_kb @ B_kb^T)``.
    """
    M, K = a_fp8.shape
    N, K2 = b_fp8.shape
    assert K == K2, f"K mismatch: A ({K}) vs B ({K2})"
    return _block_gemm(a_fp8, scales_a, b_fp8, None, scales_b, None, block_size, None, out_dtype)


def _lo_threshold(w_lo: torch.Tensor, lo_scales: torch.Tensor, threshold: float,
                  block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The W_lo sparsity rule for ``sparse_threshold > 0``
    (``tcfp/kernels.py:766-776, 997-1008``): the W_lo part of K-block kb is
    dropped for a tile of weight rows when the largest of the tile's W_lo
    scales (2^e, 0 for the -128 sentinel) is at most the threshold.  The
    reference's tile width is its autotuned ``BLOCK_N`` (64 or 128), so its
    result depends on the configuration it picked; this build fixes the
    rule at 64-row tiles.  Dropped blocks become zero codes under the
    sentinel, which the GEMM skips.  Threshold <= 0 changes nothing (only
    sentinel blocks qualify, and the GEMM skips wave tiles of those)."""
    if threshold <= 0.0:
        return w_lo, lo_scales
    n = w_lo.shape[0]
    num_kb = lo_scales.shape[0]
    sc = torch.where(lo_scales == -128, torch.zeros((), device=lo_scales.device),
                     torch.exp2(lo_scales.float()))
    g = (n + 63) // 64
    pad = torch.zeros((num_kb, g * 64), dtype=sc.dtype, device=sc.device)
    pad[:, :n] = sc
    drop = (pad.view(num_kb, g, 64).amax(-1) <= threshold)              # [num_kb, g]
    drop_rows = drop.repeat_interleave(64, dim=1)[:, :n]                # [num_kb, n]
    lo_scales = lo_scales.masked_fill(drop_rows, -128)
    codes = w_lo.view(torch.uint8).reshape(n, num_kb, block_size)
    codes = codes.masked_fill(drop_rows.t().unsqueeze(-1), 0)
    return codes.reshape(n, num_kb * block_size).view(w_lo.dtype), lo_scales


def block_linear_forward(x2d, weight, bias, block_size, error_buf=None, srr=False,
                         update_ef=True):
    """The launches of a block-scaled TCFP layer's forward, as the public ops
    run them and with the same results bit for bit: ``fused_dual_quantize_fp8``
    of W (EF or SRR, the same seed draw), then ``fused_act_quant_dual_gemm_forward``
    for layers of at most four 128-column tiles, else ``block_quantize_fp8``
    of X and ``fused_block_scaled_dual_gemm_forward`` (the reference's
    dispatch, ``tcfp/nn/__init__.py:617-650``).

    For ``tcfp_amd.nn``'s block-scaled layer, whose W, EF buffer and bias are
    its own: it skips the per-op argument checks and Python calls (one host
    call instead of three; the layer's forward enqueues ~11 us faster, which
    small host-bound models see).  ``x2d`` [M, K] fp32/bf16, ``weight``
    [N, K] contiguous.  Returns ``(out fp32 [M, N], w_hi, w_lo, e_hi, e_lo,
    act_fp8, act_e)``."""
    bs = block_size
    if bs not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {bs}")
    M, Kd = x2d.shape
    N = weight.shape[0]
    assert weight.is_contiguous() and weight.shape[1] == Kd and Kd % bs == 0, (
        f"weight {tuple(weight.shape)} vs input ({M}, {Kd}), block {bs}")
    if srr and error_buf is not None:
        raise ValueError("stochastic_lo and error_buf are mutually exclusive")
    dev = _hip.require_gpu(x2d, weight, error_buf, bias)
    lib = _hip.lib()
    st = _hip.stream_of(dev)
    nkb = Kd // bs
    e4 = torch.float8_e4m3fn
    w_hi = torch.empty((N, Kd), dtype=e4, device=dev)
    w_lo = torch.empty((N, Kd), dtype=e4, device=dev)
    e_hi = torch.empty((nkb, N), dtype=torch.int8, device=dev)
    e_lo = torch.empty((nkb, N), dtype=torch.int8, device=dev)
    seed = int(torch.randint(0, 2**62, (1,)).item()) if srr else 0
    check(lib.tcfp_block_dual_quantize(
        ptr(weight), _in_dtype(weight), N, Kd, bs, ptr(error_buf), int(bool(update_ef)),
        int(bool(srr)), seed, 0, ptr(w_hi), ptr(w_lo), ptr(e_hi), ptr(e_lo), st),
        "fused_dual_quantize_fp8")
    act = x2d
    if not act.is_contiguous() or act.data_ptr() % 16 != 0:
        act = act.contiguous()
    b = _bias_f32(bias, N) if bias is not None else None
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    act_fp8 = torch.empty((M, Kd), dtype=e4, device=dev)
    act_e = torch.empty((nkb, M), dtype=torch.int8, device=dev)
    if (N + 127) // 128 <= 4:
        check(lib.tcfp_act_quant_block_dual_gemm(
            ptr(act), _in_dtype(act), Kd, ptr(w_hi), ptr(w_lo), Kd, ptr(e_hi), ptr(e_lo), M, N,
            Kd, bs, ptr(b), ptr(out), N, ptr(act_fp8), ptr(act_e), st),
            "fused_act_quant_dual_gemm_forward")
    else:
        check(lib.tcfp_block_quantize(ptr(act), _in_dtype(act), M, Kd, bs, FP8_E4M3,
                                      ptr(act_fp8), ptr(act_e), st), "block_quantize_fp8")
        check(lib.tcfp_block_dual_gemm(
            ptr(act_fp8), FP8_E4M3, Kd, ptr(act_e), ptr(w_hi), ptr(w_lo), FP8_E4M3, Kd,
            ptr(e_hi), ptr(e_lo), M, N, Kd, bs, ptr(b), ptr(out), DTYPE_F32, N, st),
            "block_dual_gemm")
    return out, w_hi, w_lo, e_hi, e_lo, act_fp8, act_e


def fused_block_scaled_dual_gemm_forward(
    act_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    act_scales: torch.Tensor,
    w_hi_scales: torch.Tensor,
    w_lo_scales: torch.Tensor,
    block_size: int,
    sparse_threshold: float = 0.0,
    persistent: bool = True,
    launch_mult: int = 1,
    *,
    bias: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``sum_kb sa (shi A Whi^T + slo A Wlo^T)`` over K-blocks, fp32 [M, N].

    Reference: ``fused_block_scaled_dual_gemm_forward``
    (``tcfp/kernels.py:1939-2028``).  W_lo exponents of -128 (zero residual
    blocks) contribute nothing, and on the 128 x 64 tile a wave tile whose
    W_lo exponents are all the sentinel skips its W_lo MFMAs (the
    reference's sparsity fast path at its default threshold 0).  ``sparse_threshold > 0`` drops the
    W_lo blocks the reference's rule drops (``_lo_threshold``).
    ``persistent`` and ``launch_mult`` are scheduling hints of the
    reference's Triton kernel, accepted and without effect on the result.
    fp32 block multipliers for all three operands (``scale_format="fp32"``
    quantisers) select the fp32-scale kernel: the same sum with the
    multipliers in place of 2^exp.
    """
    M, K = act_fp8.shape
    N, K2 = w_hi_fp8.shape
    assert K == K2 and tuple(w_lo_fp8.shape) == (N, K), (
        f"Shape mismatch: act({M},{K}), w_hi({N},{K2}), w_lo{tuple(w_lo_fp8.shape)}"
    )
    if sparse_threshold > 0.0 and w_lo_scales.dtype == torch.int8:
        w_lo_fp8, w_lo_scales = _lo_threshold(w_lo_fp8, w_lo_scales, sparse_threshold,
                                              block_size)
    return _block_gemm(act_fp8, act_scales, w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales,
                       block_size, bias, out_dtype)


def fused_act_quant_dual_gemm_forward(
    act: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    w_hi_scales: torch.Tensor,
    w_lo_scales: torch.Tensor,
    block_size: int,
    sparse_threshold: float = 0.0,
    persistent: bool = True,
    launch_mult: int = 1,
    save_side_outputs: bool = True,
    *,
    bias: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """Activation block-quantisation + block-scaled dual GEMM, one launch.

    Reference: ``fused_act_quant_dual_gemm_forward`` (``tcfp/kernels.py:
    2031-2149``, kernel ``:826-1041``).  ``act`` [M, K] bf16/fp32 is
    quantised per (row, K-block) to E4M3 with the ``block_quantize_fp8``
    exponent rule inside the GEMM (each workgroup quantises its activation
    tile in registers and stages the codes in LDS), then multiplied with
    W_hi/W_lo as ``fused_block_scaled_dual_gemm_forward``.  Returns ``(out
    fp32 [M, N], act_fp8, act_scales)`` -- the side outputs, written by the
    workgroups of the first output-column tile, are bitwise what
    ``block_quantize_fp8`` returns -- or ``(out, None, None)`` when
    ``save_side_outputs`` is False (nothing is written for them).
    ``sparse_threshold`` as ``fused_block_scaled_dual_gemm_forward``.
    """
    M, K = act.shape
    N, K2 = w_hi_fp8.shape
    assert K == K2 and tuple(w_lo_fp8.shape) == (N, K), (
        f"Shape mismatch: act({M},{K}), w_hi({N},{K2}), w_lo{tuple(w_lo_fp8.shape)}"
    )
    assert K % block_size == 0, f"K ({K}) must be divisible by block_size ({block_size})"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    if act.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"act must be float32 or bfloat16, got {act.dtype}")
    dev = _hip.require_gpu(act, w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales, bias)
    num_kb = K // block_size
    e_hi = _block_exps(w_hi_scales, N, num_kb, "w_hi_scales")
    e_lo = _block_exps(w_lo_scales, N, num_kb, "w_lo_scales")
    if sparse_threshold > 0.0:
        w_lo_fp8, e_lo = _lo_threshold(w_lo_fp8, e_lo, sparse_threshold, block_size)
    w_hi_fp8 = _gemm_operand(w_hi_fp8, "w_hi")
    w_lo_fp8 = _gemm_operand(w_lo_fp8, "w_lo")
    if w_hi_fp8.stride(0) != w_lo_fp8.stride(0):
        w_hi_fp8, w_lo_fp8 = w_hi_fp8.contiguous(), w_lo_fp8.contiguous()
    es = act.element_size()
    if act.stride(1) != 1 or (act.stride(0) * es) % 16 != 0 or act.data_ptr() % 16 != 0:
        act = act.contiguous()
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    act_fp8 = act_scales = None
    if save_side_outputs:
        act_fp8 = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=dev)
        act_scales = torch.empty((num_kb, M), dtype=torch.int8, device=dev)
    if bias is not None:
        bias = _bias_f32(bias, N)
    check(
        _hip.lib().tcfp_act_quant_block_dual_gemm(
            ptr(act), _in_dtype(act), act.stride(0), ptr(w_hi_fp8), ptr(w_lo_fp8),
            w_hi_fp8.stride(0), ptr(e_hi), ptr(e_lo), M, N, K, block_size, ptr(bias), ptr(out),
            N, ptr(act_fp8), ptr(act_scales), _hip.stream_of(dev),
        ),
        "fused_act_quant_dual_gemm_forward",
    )
    return out, act_fp8, act_scales


def fused_wtquant_block_scaled_dual_gemm_forward(
    act_fp8: torch.Tensor,
    weight: torch.Tensor,
    act_scales: torch.Tensor,
    block_size: int,
    error_buf: torch.Tensor | None = None,
    stochastic_lo: bool = False,
    save_w_lo: bool = True,
    sparse_threshold: float = 0.0,
    persistent: bool = True,
    launch_mult: int = 1,
    *,
    seed: int | None = None,
    bias: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor, torch.Tensor | None]:
    """Weight dual-quantisation (+ EF) and block-scaled dual GEMM.

    Reference: ``fused_wtquant_block_scaled_dual_gemm_forward``
    (``tcfp/kernels.py:2152-2323``, kernel ``:1233-1531``).  W [N, K]
    bf16/fp32 (+ ``error_buf``) is dual-quantised exactly as
    ``fused_dual_quantize_fp8`` (error buffer rewritten in place with
    ``W - deq(hi) - deq(lo)``, the reference's post-step ``:2311-2319``),
    then ``out = fused_block_scaled_dual_gemm_forward``.  Returns ``(out
    fp32 [M, N], w_hi, w_lo | None, scales_hi, scales_lo | None)``; W_lo and
    its scales are None when ``save_w_lo`` is False (ABD).  One C-ABI call,
    two launches (the streaming weight pass and the GEMM).
    ``sparse_threshold``, ``persistent`` and ``launch_mult`` are the
    reference's scheduling hints and do not change the result.
    """
    assert act_fp8.is_contiguous() and weight.is_contiguous(), (
        "Activations and weight must be contiguous"
    )
    M, K = act_fp8.shape
    N, K2 = weight.shape
    assert K == K2, f"K mismatch: act ({K}) vs weight ({K2})"
    assert K % block_size == 0, f"K ({K}) must be divisible by block_size ({block_size})"
    if stochastic_lo and error_buf is not None:
        raise ValueError(
            "stochastic_lo and error_buf are mutually exclusive "
            "(SRR eliminates the error-feedback buffer)"
        )
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    if error_buf is not None:
        assert error_buf.dtype == torch.float32 and tuple(error_buf.shape) == (N, K), (
            "error_buf must be float32 with the weight's shape"
        )
        assert error_buf.is_contiguous(), "error_buf must be contiguous"
    dev = _hip.require_gpu(act_fp8, weight, act_scales, error_buf, bias)
    num_kb = K // block_size
    e_a = _block_exps(act_scales, M, num_kb, "act_scales")
    if sparse_threshold > 0.0:
        # the threshold rule rewrites W_lo between the two launches
        w_hi, w_lo, s_hi, s_lo = fused_dual_quantize_fp8(
            weight, block_size, error_buf=error_buf, stochastic_lo=stochastic_lo, seed=seed)
        out = fused_block_scaled_dual_gemm_forward(
            act_fp8, w_hi, w_lo, e_a, s_hi, s_lo, block_size, sparse_threshold, bias=bias)
        if save_w_lo:
            return out, w_hi, w_lo, s_hi, s_lo
        return out, w_hi, None, s_hi, None
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    w_hi = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=dev)
    w_lo = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=dev)
    s_hi = torch.empty((num_kb, N), dtype=torch.int8, device=dev)
    s_lo = torch.empty((num_kb, N), dtype=torch.int8, device=dev)
    if bias is not None:
        bias = _bias_f32(bias, N)
    if stochastic_lo and seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    check(
        _hip.lib().tcfp_wtquant_block_dual_gemm(
            ptr(act_fp8), _fmt(act_fp8.dtype), act_fp8.stride(0), ptr(e_a), ptr(weight),
            _in_dtype(weight), M, N, K, block_size, ptr(error_buf), int(bool(stochastic_lo)),
            int(seed or 0), 0, ptr(w_hi), ptr(w_lo), ptr(s_hi), ptr(s_lo), ptr(bias), ptr(out),
            _out_dtype(torch.float32), N, _hip.stream_of(dev),
        ),
        "fused_wtquant_block_scaled_dual_gemm_forward",
    )
    if save_w_lo:
        return out, w_hi, w_lo, s_hi, s_lo
    return out, w_hi, None, s_hi, None


def fused_block_scaled_backward_dx(
    grad_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor | None,
    grad_scales: torch.Tensor,
    w_hi_scales: torch.Tensor,
    w_lo_scales: torch.Tensor | None,
    block_size: int,
    persistent: bool = True,
    launch_mult: int = 1,
) -> torch.Tensor:
    """``dX = deq(grad) @ (deq(W_hi) + deq(W_lo))``, fp32 [M, D_in].

    Reference: ``fused_block_scaled_backward_dx`` (``tcfp/kernels.py:
    2326-2425``, kernel ``:1051-1205``); ``persistent`` / ``launch_mult`` are
    its scheduling hints and do not change the result.  grad [M, D_out]
    (E5M2 or E4M3) with exponents [D_out // bs, M]; W [D_out, D_in] E4M3
    with exponents [D_in // bs, D_out].  The W exponents change along the
    contraction index, so the operands are dequantised exactly into bf16
    and multiplied on the bf16 MFMA (fp32 accumulation); ``w_lo_fp8=None``
    (ABD) uses W_hi alone.
    """
    M, D_out = grad_fp8.shape
    D_out2, D_in = w_hi_fp8.shape
    assert D_out == D_out2, f"Shape mismatch: grad({M},{D_out}), w_hi({D_out2},{D_in})"
    if w_lo_fp8 is not None:
        assert tuple(w_lo_fp8.shape) == (D_out, D_in), "w_lo shape mismatch"
    assert D_out % block_size == 0, f"D_out ({D_out}) not divisible by block_size ({block_size})"
    assert D_in % block_size == 0, f"D_in ({D_in}) not divisible by block_size ({block_size})"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    dev = _hip.require_gpu(grad_fp8, w_hi_fp8, w_lo_fp8, grad_scales, w_hi_scales, w_lo_scales)
    g = grad_fp8.contiguous()
    wh = w_hi_fp8.contiguous()
    wl = w_lo_fp8.contiguous() if w_lo_fp8 is not None else None
    eg = _block_exps(grad_scales, M, D_out // block_size, "grad_scales")
    eh = _block_exps(w_hi_scales, D_out, D_in // block_size, "w_hi_scales")
    el = (_block_exps(w_lo_scales, D_out, D_in // block_size, "w_lo_scales")
          if wl is not None else None)
    if wh.dtype != torch.float8_e4m3fn or (wl is not None and wl.dtype != torch.float8_e4m3fn):
        raise TypeError("W_hi / W_lo must be float8_e4m3fn")
    out = torch.empty((M, D_in), dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_block_dual_gemm_dx_workspace_bytes(M, D_out, D_in))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_block_dual_gemm_dx(
            ptr(g), _fmt(g.dtype), ptr(eg), ptr(wh), ptr(wl), ptr(eh), ptr(el), M, D_out, D_in,
            block_size, ptr(out), ptr(ws), nbytes, _hip.stream_of(dev),
        ),
        "block_dual_gemm_dx",
    )
    return out


def fused_block_scaled_dual_gemm_backward_dx(
    grad_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor | None,
    grad_scales: torch.Tensor,
    w_hi_scales: torch.Tensor,
    w_lo_scales: torch.Tensor | None,
    block_size: int,
) -> torch.Tensor:
    """Block dgrad dispatcher (reference ``tcfp/kernels.py:2428-2469``): the
    reference sends it to :func:`fused_block_scaled_backward_dx` whenever its
    fused tier is available, and here that tier always is."""
    return fused_block_scaled_backward_dx(grad_fp8, w_hi_fp8, w_lo_fp8, grad_scales, w_hi_scales,
                                          w_lo_scales, block_size)


def block_scaled_wgrad(
    grad: torch.Tensor,
    act_fp8: torch.Tensor,
    act_scales: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """``grad.t() @ block_dequantize_fp8(act)`` in fp32 accuracy, [N, K].

    The block path's weight gradient (reference ``tcfp/nn/__init__.py:
    743-750``, an fp32 matmul there).  grad [M, N] (fp32; other dtypes are
    promoted), act [M, K] FP8 with exponents [K // block_size, M].  The
    fp32 gradient is split into two bf16 parts and both products run as one
    bf16-MFMA GEMM; every product is exact and the split's relative
    representation error is at most 2^-17.  Token counts that are not a
    multiple of 4 use the dequantise + fp32 matmul form.
    """
    M, N = grad.shape
    M2, Kd = act_fp8.shape
    assert M == M2, f"token mismatch: grad {tuple(grad.shape)} vs act {tuple(act_fp8.shape)}"
    dev = _hip.require_gpu(grad, act_fp8, act_scales)
    g = grad.float().contiguous()
    if M % 4 != 0:
        return g.t() @ block_dequantize_fp8(act_fp8, act_scales, block_size)
    a = act_fp8.contiguous()
    e = _block_exps(act_scales, M, Kd // block_size, "act_scales")
    out = torch.empty((N, Kd), dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_block_wgrad_workspace_bytes(M, N, Kd))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_block_wgrad(
            ptr(g), M, N, ptr(a), _fmt(a.dtype), ptr(e), Kd, block_size, ptr(out), ptr(ws),
            nbytes, _hip.stream_of(dev),
        ),
        "block_wgrad",
    )
    return out


def block_backward_prep(
    grad: torch.Tensor,
    block_size: int,
    *,
    dequant: bool = True,
    split: bool = True,
    bias: bool = False,
    fp8: bool = False,
    split_lo: bool = True,
):
    """One pass over the fp32 gradient [M, N] for the block backward.

    Returns ``(g_deq, g_split_t, bias_grad)`` (None where not requested),
    plus ``(g_fp8, g_exps)`` when ``fp8``: ``g_deq`` [M, N] bf16 is the
    gradient block-quantised to E5M2 exactly as
    ``block_quantize_fp8(grad, block_size, float8_e5m2)`` and dequantised
    (the exact dgrad's operand); ``g_fp8`` / ``g_exps`` are those codes and
    exponents themselves (the FP8 dgrad's operand); ``g_split_t`` [N, 2M]
    bf16 is the transposed hi/lo split the block wgrad uses (``split_lo``
    False: [N, M], the transposed bf16(grad) of the single-pass wgrad); ``bias_grad``
    [N] fp32 is ``grad.sum(0)`` summed per 64-row tile.  These replace the
    quantise, dequantise, split and reduce passes the backward would
    otherwise make.
    """
    M, N = grad.shape
    assert N % block_size == 0, f"N ({N}) must be divisible by block_size ({block_size})"
    dev = _hip.require_gpu(grad)
    g = grad if (grad.dtype == torch.float32 and grad.is_contiguous()) else grad.float().contiguous()
    g_deq = torch.empty((M, N), dtype=torch.bfloat16, device=dev) if dequant else None
    g_split = (torch.empty((N, 2 * M if split_lo else M), dtype=torch.bfloat16, device=dev)
               if split else None)
    bias_grad = torch.empty((N,), dtype=torch.float32, device=dev) if bias else None
    g_fp8 = torch.empty((M, N), dtype=torch.float8_e5m2, device=dev) if fp8 else None
    g_exps = torch.empty((N // block_size, M), dtype=torch.int8, device=dev) if fp8 else None
    nbytes = int(_hip.lib().tcfp_block_grad_prep_workspace_bytes(M, N)) if bias else 0
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if bias else None
    check(
        _hip.lib().tcfp_block_grad_prep(
            ptr(g), M, N, block_size, ptr(g_deq), ptr(g_split), int(split_lo), ptr(bias_grad),
            ptr(g_fp8),
            ptr(g_exps), ptr(ws), nbytes, _hip.stream_of(dev),
        ),
        "block_backward_prep",
    )
    if fp8:
        return g_deq, g_split, bias_grad, g_fp8, g_exps
    return g_deq, g_split, bias_grad


_BWD_WS: dict[tuple, tuple[int, int, int]] = {}


def block_linear_backward(grad_2d, act_fp8, act_e, w_hi, w_lo, e_hi, e_lo, block_size,
                          need_dx, need_dw, want_db, split_lo=True):
    """The launches of a block-scaled TCFP layer's default backward, as
    :func:`block_backward_prep`, :func:`block_wgrad_from_prep` and
    :func:`block_dgrad_from_prep` run them, with the same results bit for
    bit: one pass over the gradient, then the wgrad from the split gradient
    (released before dX is allocated), then the exact dgrad.

    For ``tcfp_amd.nn``'s block-scaled layer (its saved operands): one host
    call without the per-op checks, the workspace sizes cached per shape.
    ``grad_2d`` [M, D_out]; ``act_fp8`` / ``act_e`` the forward's activation
    codes and exponents (``need_dw``; M % 4 == 0, and M % 64 == 0 without
    ``split_lo``); ``w_hi`` .. ``e_lo`` the forward's weight operands
    (``need_dx``).  Returns ``(dx fp32 [M, D_in], dw fp32 [D_out, D_in],
    db fp32 [D_out])``, None where not requested."""
    bs = block_size
    M, Nout = grad_2d.shape
    Kin = w_hi.shape[1] if need_dx else (act_fp8.shape[1] if need_dw else 0)
    dev = _hip.require_gpu(grad_2d, act_fp8, w_hi)
    lib = _hip.lib()
    st = _hip.stream_of(dev)
    key = (M, Nout, Kin, bool(split_lo), bool(want_db), bool(need_dw), bool(need_dx))
    sizes = _BWD_WS.get(key)
    if sizes is None:
        sizes = (int(lib.tcfp_block_grad_prep_workspace_bytes(M, Nout)) if want_db else 0,
                 int(lib.tcfp_block_wgrad_presplit_workspace_bytes(M, Nout, Kin, int(split_lo)))
                 if need_dw else 0,
                 int(lib.tcfp_block_dual_gemm_dx_bf16_workspace_bytes(Nout, Kin)) if need_dx else 0)
        _BWD_WS[key] = sizes
    n_prep, n_w, n_d = sizes
    g = grad_2d if (grad_2d.dtype == torch.float32 and grad_2d.is_contiguous()) else (
        grad_2d.float().contiguous())
    bf = torch.bfloat16
    g_deq = torch.empty((M, Nout), dtype=bf, device=dev) if need_dx else None
    g_split = (torch.empty((Nout, 2 * M if split_lo else M), dtype=bf, device=dev)
               if need_dw else None)
    db = torch.empty((Nout,), dtype=torch.float32, device=dev) if want_db else None
    ws = torch.empty(max(n_prep, 1), dtype=torch.uint8, device=dev) if want_db else None
    check(lib.tcfp_block_grad_prep(ptr(g), M, Nout, bs, ptr(g_deq), ptr(g_split), int(split_lo),
                                   ptr(db), None, None, ptr(ws), n_prep, st),
          "block_backward_prep")
    # (the gradient copy and each scratch are released before the next
    # allocation, as the per-op calls release theirs on return)
    g = dw = dx = ws = None
    if need_dw:
        dw = torch.empty((Nout, Kin), dtype=torch.float32, device=dev)
        ws = torch.empty(max(n_w, 1), dtype=torch.uint8, device=dev)
        check(lib.tcfp_block_wgrad_presplit(
            ptr(g_split), int(split_lo), M, Nout, ptr(act_fp8), _fmt(act_fp8.dtype), ptr(act_e),
            Kin, bs, ptr(dw), ptr(ws), n_w, st), "block_wgrad_from_prep")
    g_split = ws = None  # (released before dX is allocated)
    if need_dx:
        dx = torch.empty((M, Kin), dtype=torch.float32, device=dev)
        ws = torch.empty(max(n_d, 1), dtype=torch.uint8, device=dev)
        check(lib.tcfp_block_dual_gemm_dx_bf16(
            ptr(g_deq), ptr(w_hi), ptr(w_lo), ptr(e_hi), ptr(e_lo), M, Nout, Kin, bs, ptr(dx),
            ptr(ws), n_d, st), "block_dgrad_from_prep")
    return dx, dw, db


def block_dgrad_from_prep(g_deq, w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales, block_size):
    """``fused_block_scaled_dual_gemm_backward_dx`` from the bf16 gradient of
    :func:`block_backward_prep` (same result bit for bit)."""
    M, D_out = g_deq.shape
    D_out2, D_in = w_hi_fp8.shape
    assert D_out == D_out2, f"Shape mismatch: grad({M},{D_out}), w_hi({D_out2},{D_in})"
    dev = _hip.require_gpu(g_deq, w_hi_fp8, w_lo_fp8)
    nkb = D_in // block_size
    wh = w_hi_fp8.contiguous()
    wl = w_lo_fp8.contiguous() if w_lo_fp8 is not None else None
    eh = _block_exps(w_hi_scales, D_out, nkb, "w_hi_scales")
    el = _block_exps(w_lo_scales, D_out, nkb, "w_lo_scales") if wl is not None else None
    out = torch.empty((M, D_in), dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_block_dual_gemm_dx_bf16_workspace_bytes(D_out, D_in))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_block_dual_gemm_dx_bf16(
            ptr(g_deq), ptr(wh), ptr(wl), ptr(eh), ptr(el), M, D_out, D_in, block_size, ptr(out),
            ptr(ws), nbytes, _hip.stream_of(dev),
        ),
        "block_dgrad_from_prep",
    )
    return out


def block_requant_t(w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales, block_size):
    """Block dual-quantised W [D_out, D_in] (exponents [D_in // bs, D_out])
    re-blocked along D_out: ``v = deq(W_hi) + deq(W_lo)`` in fp32, then
    ``fused_dual_quantize_fp8`` of ``v.T`` (RNE, no error buffer).  Returns
    ``(wt_hi, wt_lo, et_hi, et_lo)`` with codes [D_in, D_out] and exponents
    [D_out // bs, D_in]: the weight operands of an FP8 block dgrad
    (:func:`fp8_block_dgrad`).  ``w_lo_fp8=None`` re-blocks W_hi alone."""
    D_out, D_in = w_hi_fp8.shape
    assert D_out % block_size == 0, f"D_out ({D_out}) not divisible by block_size ({block_size})"
    assert D_in % block_size == 0, f"D_in ({D_in}) not divisible by block_size ({block_size})"
    if block_size not in (32, 64, 128):
        raise ValueError(f"block_size must be 32, 64, or 128, got {block_size}")
    dev = _hip.require_gpu(w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales)
    if w_hi_fp8.dtype != torch.float8_e4m3fn or (
            w_lo_fp8 is not None and w_lo_fp8.dtype != torch.float8_e4m3fn):
        raise TypeError("W_hi / W_lo must be float8_e4m3fn")
    nkb = D_in // block_size
    wh = w_hi_fp8.contiguous()
    wl = w_lo_fp8.contiguous() if w_lo_fp8 is not None else None
    if wl is not None:
        assert tuple(wl.shape) == (D_out, D_in), "w_lo shape mismatch"
    eh = _block_exps(w_hi_scales, D_out, nkb, "w_hi_scales")
    el = _block_exps(w_lo_scales, D_out, nkb, "w_lo_scales") if wl is not None else None
    wt_hi = torch.empty((D_in, D_out), dtype=torch.float8_e4m3fn, device=dev)
    wt_lo = torch.empty((D_in, D_out), dtype=torch.float8_e4m3fn, device=dev)
    et_hi = torch.empty((D_out // block_size, D_in), dtype=torch.int8, device=dev)
    et_lo = torch.empty((D_out // block_size, D_in), dtype=torch.int8, device=dev)
    check(
        _hip.lib().tcfp_block_requant_t(
            ptr(wh), ptr(wl), ptr(eh), ptr(el), D_out, D_in, block_size, ptr(wt_hi), ptr(wt_lo),
            ptr(et_hi), ptr(et_lo), _hip.stream_of(dev),
        ),
        "block_requant_t",
    )
    return wt_hi, wt_lo, et_hi, et_lo


def fp8_block_dgrad(grad, w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales, block_size, *,
                    reblocked=None, grad_fp8=None):
    """Opt-in FP8 block dgrad ``dX ~ grad @ (deq(W_hi) + deq(W_lo))``, fp32
    [M, D_in]: the gradient block-quantised to E5M2 along D_out (the
    reference's ``block_quantize_fp8`` of the gradient, ``nn:700-712``),
    W re-blocked along D_out (:func:`block_requant_t`), then the block dual
    FP8 GEMM.  The reference multiplies the dequantised operands in fp32
    (``fused_block_scaled_dual_gemm_backward_dx``); here W carries one more
    dual-FP8 rounding (relative ~2^-9 of a block's maximum).

    ``reblocked`` (the four outputs of :func:`block_requant_t`, e.g. built
    once in the forward) and ``grad_fp8`` (codes and exponents, e.g. from
    :func:`block_backward_prep`) skip those steps; ``grad`` and the
    original weight operands may then be None."""
    if grad_fp8 is None:
        g_fp8, g_exps = block_quantize_fp8(grad, block_size, torch.float8_e5m2)
    else:
        g_fp8, g_exps = grad_fp8
    if reblocked is None:
        assert g_fp8.shape[1] == w_hi_fp8.shape[0], (
            f"Shape mismatch: grad{tuple(g_fp8.shape)}, w_hi{tuple(w_hi_fp8.shape)}")
        reblocked = block_requant_t(w_hi_fp8, w_lo_fp8, w_hi_scales, w_lo_scales, block_size)
    wt_hi, wt_lo, et_hi, et_lo = reblocked
    return _block_gemm(g_fp8, g_exps, wt_hi, wt_lo, et_hi, et_lo, block_size, None,
                       torch.float32)


def block_wgrad_from_prep(g_split_t, act_fp8, act_scales, block_size):
    """``block_scaled_wgrad`` from the split gradient of
    :func:`block_backward_prep` (same result bit for bit; M % 4 == 0).  A
    [N, M] operand (``split_lo=False``) gives the single-pass wgrad
    ``bf16(grad)^T deq(act)`` (M % 64 == 0)."""
    N, M2 = g_split_t.shape
    M, Kd = act_fp8.shape
    lo = M2 == 2 * M
    assert (lo and M % 4 == 0) or (M2 == M and M % 64 == 0), (
        "split gradient must be [N, 2M] with M % 4 == 0 or [N, M] with M % 64 == 0")
    dev = _hip.require_gpu(g_split_t, act_fp8, act_scales)
    a = act_fp8.contiguous()
    e = _block_exps(act_scales, M, Kd // block_size, "act_scales")
    out = torch.empty((N, Kd), dtype=torch.float32, device=dev)
    nbytes = int(_hip.lib().tcfp_block_wgrad_presplit_workspace_bytes(M, N, Kd, int(lo)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(
        _hip.lib().tcfp_block_wgrad_presplit(
            ptr(g_split_t), int(lo), M, N, ptr(a), _fmt(a.dtype), ptr(e), Kd, block_size, ptr(out),
            ptr(ws), nbytes, _hip.stream_of(dev),
        ),
        "block_wgrad_from_prep",
    )
    return out


def set_gemm_tile_policy(policy: str) -> None:
    """Tuning hook: ``"auto"`` (default), ``"large"`` (256 x 128 tiles),
    ``"small"`` (128 x 64 tiles, two workgroups per CU), ``"small8"``
    (128 x 64 with eight waves where the grid fits one round) or
    ``"large_nonpersistent"`` (256 x 128 with one workgroup per tile, never
    the persistent launch) or ``"large4"`` (the persistent 256 x 128 tile
    with four waves, one per SIMD, for per-tensor dual GEMMs with bf16
    output).  Results do not depend on the policy."""
    code = {"auto": 0, "large": 1, "small": 2, "small8": 3, "large_nonpersistent": 4,
            "large4": 5}[policy]
    check(_hip.lib().tcfp_gemm_set_tile_policy(code), "set_gemm_tile_policy")


def set_dual_quant_candidates(on: bool) -> None:
    """Tuning hook of the per-tensor dual quantisation on tensors of 2^23
    elements or more: True (default) keeps the candidates for the residual
    amax in the amax pass and skips the full residual pass whenever they
    decide it; False always runs the full pass.  Results do not depend on
    it."""
    check(_hip.lib().tcfp_dual_quantize_set_candidates(int(bool(on))),
          "set_dual_quant_candidates")
