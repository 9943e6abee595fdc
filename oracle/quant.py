"""Quantisation restatement in numpy (test oracle; see package docstring).

All arrays are float32 holding the exact values of the reference tensor's
dtype ("f32" or "bf16"); the dtype tag only changes where the reference's
scale arithmetic rounds.
"""
from __future__ import annotations

import numpy as np

from .fp8 import E4M3, FP8_MAX, bf16_round, decode, encode

F32 = np.float32

# Largest mantissa offset j (q = 2^k (1 + j 2^-23)) for which a correctly
# rounded fp32 log2(q) still rounds to the integer k, indexed by p, the
# binade exponent of the fp32 numbers adjacent to k on the side of k + L.
_J_TABLE = np.array([0, 0, 1, 2, 5, 11, 22], dtype=np.int64)


def ceil_log2_f32(q: np.ndarray) -> np.ndarray:
    """``torch.ceil(torch.log2(q))`` for positive normal fp32 ``q`` (int64 out).

    Restates the exponent rule of ``tcfp/kernels.py:257-260`` /
    ``tcfp/core.py:250`` *as evaluated by a correctly rounded fp32 log2*
    (which is what torch's CPU ``log2`` gives at every boundary input):
    for ``q = 2^k (1 + f)`` with small ``f > 0`` the fp32 log2 can round to
    exactly ``k``, so ``ceil`` returns ``k`` instead of ``k + 1``.
    Subnormal inputs return -127 (callers clamp to -126).
    """
    q = np.ascontiguousarray(q, dtype=F32)
    bits = q.view(np.uint32).astype(np.int64)
    ef = (bits >> 23) & 0xFF
    j = bits & 0x7FFFFF
    k = ef - 127
    a = np.abs(k)
    safe_a = np.maximum(a, 1)
    p = np.floor(np.log2(safe_a)).astype(np.int64)
    pow2 = (safe_a & (safe_a - 1)) == 0
    p = np.where((k < 0) & pow2, p - 1, p)
    p = np.where(k == 0, 0, p)
    jmax = np.where(p < 0, 0, _J_TABLE[np.clip(p, 0, 6)])
    e = np.where(j == 0, k, np.where(j <= jmax, k, k + 1))
    return np.where(ef == 0, -127, e)


def _round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf16_round(x) if dtype == "bf16" else np.asarray(x, dtype=F32)


def per_tensor_scale(t: np.ndarray, dtype: str, fmt: str = E4M3) -> np.float32:
    """``scale = (FP8_MAX / amax.clamp(min=1e-12)).to(float32)`` (core.py:100-101).

    ``python_float / tensor`` is ``tensor.reciprocal() * python_float``
    (torch ``Tensor.__rtruediv__``), each op rounded to the tensor's dtype.
    """
    amax = np.max(np.abs(t)) if t.size else F32(0)
    amax = np.maximum(F32(amax), _round_dtype(np.array([1e-12], F32), dtype)[0])
    rcp = _round_dtype(np.array([F32(1.0) / F32(amax)], F32), dtype)[0]
    scale = _round_dtype(np.array([F32(rcp) * F32(FP8_MAX[fmt])], F32), dtype)[0]
    return F32(scale)


def to_fp8_per_tensor(t: np.ndarray, dtype: str = "f32", fmt: str = E4M3,
                      scale: np.float32 | None = None):
    """``to_fp8_e4m3`` / ``to_fp8_e5m2`` (core.py:85-106, :137-158).

    Returns ``(codes uint8, inv_scale float32, scale float32)``.
    """
    t = np.asarray(t, dtype=F32)
    if scale is None:
        scale = per_tensor_scale(t, dtype, fmt)
    mx = F32(FP8_MAX[fmt])
    scaled = np.clip(t * F32(scale), -mx, mx)
    codes = encode(scaled, fmt)
    inv = F32(F32(1.0) / F32(scale))
    return codes, inv, F32(scale)


def nf_std_f32(t: np.ndarray) -> np.float32:
    """``t.std()`` of an fp32 tensor (unbiased, torch's default correction)
    as the real standard deviation rounded to fp32: float64 mean, float64
    sum of squared deviations, one rounding at the end.  Fewer than two
    elements give NaN, as torch.std does.
    """
    v = np.asarray(t, dtype=F32).ravel().astype(np.float64)
    if v.size < 2:
        return F32(np.nan)
    d = v - v.mean()
    return F32(np.sqrt(np.dot(d, d) / (v.size - 1)))


def _clamp_min(v, lo: float) -> np.float32:
    """``clamp(min=lo)`` of an fp32 scalar; NaN passes through."""
    v = F32(v)
    return v if np.isnan(v) else np.maximum(v, F32(lo))


def nf_target(t: np.ndarray, sigma_factor: float = 3.0) -> np.float32:
    """The effective max of ``to_fp8_e4m3_nf_aware`` (core.py:181-184):
    ``sigma_factor * std`` (fp32 product with the fp32-rounded factor), or
    the clamped amax when the clamped std is below 1e-6 (compared in fp32).
    """
    t = np.asarray(t, dtype=F32)
    std = _clamp_min(nf_std_f32(t), 1e-12)
    if std < F32(1e-6):
        return _clamp_min(np.max(np.abs(t)), 1e-12)
    return F32(F32(sigma_factor) * std)


def to_fp8_nf_aware(t: np.ndarray, sigma_factor: float = 3.0):
    """``to_fp8_e4m3_nf_aware`` without SR (core.py:161-193): the scale is
    ``(448 / target).to(float32)``, values beyond +-448 saturate.  Returns
    ``(codes, inv_scale, scale)``."""
    return to_fp8_per_tensor(t, "f32", scale=_scale_of(nf_target(t, sigma_factor)))


def dual_quant_per_tensor(W: np.ndarray, ef: np.ndarray | None = None,
                          sigma_factor: float | None = None):
    """Per-tensor dual-quant + error feedback (nn/__init__.py:343-383).

    ``W`` holds the weight's values as float32.  Returns
    ``(hi, lo, inv_hi, inv_lo, ef_new, residual)``; ``ef_new`` is relative
    to the original W, not to ``W + ef`` (nn/__init__.py:378-383).
    ``sigma_factor`` selects NF-aware W_hi scaling (nn/__init__.py:356-359).
    """
    W = np.asarray(W, dtype=F32)
    w = W + ef if ef is not None else W
    if sigma_factor is None:
        hi, inv_hi, _ = to_fp8_per_tensor(w, "f32")
    else:
        hi, inv_hi, _ = to_fp8_nf_aware(w, sigma_factor)
    deq_hi = decode(hi, E4M3) * inv_hi
    residual = w - deq_hi
    lo, inv_lo, _ = to_fp8_per_tensor(residual, "f32")
    deq_lo = decode(lo, E4M3) * inv_lo
    ef_new = W - (deq_hi + deq_lo)
    return hi, lo, F32(inv_hi), F32(inv_lo), ef_new, residual


def _ema_f32(prev, cur, decay: float) -> np.float32:
    """torch's ``decay * prev + (1 - decay) * cur`` on fp32 scalars: the
    Python floats are rounded to fp32 and each op rounds (core.py:352-355)."""
    a, b = F32(decay), F32(1.0 - decay)
    return F32(F32(a * F32(prev)) + F32(b * F32(cur)))


def _scale_of(v) -> np.float32:
    """``(448 / v).to(float32)`` for an fp32 tensor v: reciprocal, then
    product (``Tensor.__rtruediv__``)."""
    return F32(F32(F32(1.0) / F32(v)) * F32(FP8_MAX[E4M3]))


def new_delayed_state() -> dict:
    """The delayed-scaling parts of ``ErrorFeedbackState`` (core.py:309-314)."""
    return {"amax": {}, "ratio": {}, "steps": {}}


def dual_quant_per_tensor_delayed(W: np.ndarray, ef: np.ndarray | None, state: dict,
                                  name: str, decay: float = 0.999, interval: int = 100,
                                  sigma_factor: float | None = None):
    """Per-tensor dual quantisation with delayed (predictive dual-track)
    scaling: ``_delayed_quantise_w_hi`` / ``_delayed_quantise_w_lo``
    (nn/__init__.py:250-309) inside the forward's steps 1-4 (:343-383), with
    ErrorFeedbackState's EMA bookkeeping (core.py:341-403).  With
    ``sigma_factor`` the NF branch (:263-275): the sigma target replaces the
    amax in the EMA.

    ``state`` is updated in place.  Returns ``(hi, lo, inv_hi, inv_lo,
    ef_new, validated)``.
    """
    W = np.asarray(W, dtype=F32)
    w = W + ef if ef is not None else W
    # W_hi: scale from the EMA of the clamped amax (first call: the amax)
    if sigma_factor is None:
        cur = np.maximum(F32(np.max(np.abs(w))), F32(1e-12))
    else:
        cur = nf_target(w, sigma_factor)
    key = name + ".w_hi"
    if key not in state["amax"]:
        delayed = F32(cur)
    else:
        delayed = _ema_f32(state["amax"][key], cur, decay)
    state["amax"][key] = delayed
    hi, inv_hi, _ = to_fp8_per_tensor(w, "f32", scale=_scale_of(delayed))
    residual = (w - decode(hi, E4M3) * inv_hi).astype(F32)
    # W_lo: measured on validation steps (first call, every `interval`),
    # predicted from the ratio EMA otherwise
    skey, rkey = f"{name}.steps", f"{name}.ratio"
    count = state["steps"].get(skey, 0) + 1
    state["steps"][skey] = count
    validate = count == 1 or count % interval == 0
    if validate:
        actual = np.maximum(F32(np.max(np.abs(residual))), F32(1e-12))
        ratio = F32(actual / np.maximum(delayed, F32(1e-12)))
        state["ratio"][rkey] = ratio if rkey not in state["ratio"] else _ema_f32(
            state["ratio"][rkey], ratio, decay)
        lo_amax = actual
    elif rkey in state["ratio"]:
        lo_amax = np.maximum(F32(delayed * state["ratio"][rkey]), F32(1e-12))
    else:
        lo_amax = np.maximum(F32(delayed / F32(8.0)), F32(1e-12))
    lo, inv_lo, _ = to_fp8_per_tensor(residual, "f32", scale=_scale_of(lo_amax))
    ef_new = W - (decode(hi, E4M3) * inv_hi + decode(lo, E4M3) * inv_lo)
    return hi, lo, F32(inv_hi), F32(inv_lo), ef_new.astype(F32), validate


def sr_candidates_per_tensor(x: np.ndarray):
    """Deterministic part of ``stochastic_round_to_fp8_e4m3`` (core.py:418-464).

    ``x`` is the already scaled and clamped tensor.  Returns
    ``(lo_codes, hi_codes, frac, exact)``: the result is ``lo`` where
    ``exact``, else ``hi`` with probability ``frac``.  Note ``hi`` can be
    NaN-coded (0x7F) near the top of the range; ``rand < NaN`` is false, so
    such elements always keep ``lo``.
    """
    x = np.asarray(x, dtype=F32)
    lo = encode(x, E4M3)
    lo_f = decode(lo, E4M3)
    d = np.sign(x - lo_f).astype(F32)
    exact = x == lo_f
    nudge = d * F32(2.0 ** -6) * F32(0.5)
    hi = encode(lo_f + nudge, E4M3)
    same = (decode(hi, E4M3) == lo_f) & ~exact
    abs_lo = np.maximum(np.abs(lo_f), F32(2.0 ** -6))
    larger = d * abs_lo * F32(0.25)
    hi_retry = encode(lo_f + larger, E4M3)
    hi = np.where(same, hi_retry, hi)
    with np.errstate(invalid="ignore"):
        gap = np.maximum(np.abs(decode(hi, E4M3) - lo_f), F32(1e-45))
        gap = np.where(np.isnan(decode(hi, E4M3)), np.nan, gap).astype(F32)
        frac = np.clip(np.abs(x - lo_f) / gap, F32(0), F32(1))
    return lo, hi.astype(np.uint8), frac.astype(F32), exact


def compute_block_scales(x: np.ndarray, bs: int, fp8_max: float = 448.0,
                         dtype: str = "f32") -> np.ndarray:
    """``compute_block_scales`` (core.py:221-252): ``2^ceil(log2(amax / fp8_max))``
    per run of ``bs`` elements along the last axis, in the tensor's dtype.

    Every step rounds to ``dtype`` as torch's ops on that dtype do:
    ``amax.clamp(min=1e-12)`` (the bound itself rounded to the dtype; NaN
    passes), ``amax / fp8_max`` (fp32 quotient, rounded), ``log2`` (an fp32
    log2 rounded to the dtype: for bf16 that 8-bit rounding can pull a value
    just above an integer down onto it), ``ceil`` and ``exp2``.  fp32
    ``ceil(log2)`` follows :func:`ceil_log2_f32` for normal quotients.
    Returns float32 arrays holding the dtype's values, shape
    ``x.shape[:-1] + (x.shape[-1] // bs,)``.
    """
    x = np.asarray(x, dtype=F32)
    *lead, d = x.shape
    assert d % bs == 0
    blocks = x.reshape(*lead, d // bs, bs)
    with np.errstate(invalid="ignore"):
        amax = np.max(np.abs(blocks), axis=-1) if bs else np.zeros(blocks.shape[:-1], F32)
    lo = _round_dtype(np.array([1e-12], F32), dtype)[0]
    amax = np.where(np.isnan(amax), amax, np.maximum(amax, lo)).astype(F32)
    q = _round_dtype((amax / F32(fp8_max)).astype(F32), dtype)
    with np.errstate(divide="ignore", invalid="ignore"):
        l32 = np.log2(q.astype(np.float64)).astype(F32)
    if dtype == "bf16":
        e = np.ceil(bf16_round(l32).astype(np.float64))
    else:
        normal = np.isfinite(q) & (q >= F32(2.0 ** -126))
        e = np.where(normal, ceil_log2_f32(np.where(normal, q, F32(1))).astype(np.float64),
                     np.ceil(l32.astype(np.float64)))
    with np.errstate(over="ignore"):
        out = np.exp2(e).astype(F32)
    return _round_dtype(out, dtype).reshape(*lead, d // bs)


def _blocks(x: np.ndarray, bs: int) -> np.ndarray:
    m, k = x.shape
    assert k % bs == 0
    return x.reshape(m, k // bs, bs)


def block_exponent(amax: np.ndarray, fmt: str = E4M3) -> np.ndarray:
    """``max(ceil(log2(max(amax, 1e-12) / FP8_MAX)), -126)`` (kernels.py:253-260)."""
    a = np.maximum(np.asarray(amax, dtype=F32), F32(1e-12))
    q = (a / F32(FP8_MAX[fmt])).astype(F32)
    return np.maximum(ceil_log2_f32(q), -126)


def _pow2(e: np.ndarray) -> np.ndarray:
    return np.ldexp(np.ones_like(e, dtype=F32), e.astype(np.int32)).astype(F32)


def block_quantize(x: np.ndarray, bs: int, fmt: str = E4M3):
    """``block_quantize_fp8`` (kernels.py:1675-1722, kernel :205-275).

    ``x`` [M, K] float32 values.  Returns ``(codes [M,K] uint8, exps int8
    [K/bs, M])`` with ``scale = 2^exp`` (divide before the cast).
    """
    x = np.asarray(x, dtype=F32)
    xb = _blocks(x, bs)
    e = block_exponent(np.max(np.abs(xb), axis=-1), fmt)
    mx = F32(FP8_MAX[fmt])
    scaled = np.clip(xb * _pow2(-e)[..., None], -mx, mx)
    codes = encode(scaled, fmt).reshape(x.shape)
    return codes, np.ascontiguousarray(e.T.astype(np.int8))


def block_dequantize(codes: np.ndarray, exps: np.ndarray, bs: int,
                     fmt: str = E4M3) -> np.ndarray:
    """``block_dequantize_fp8`` (kernels.py:1725-1746): ``fp8 * exp2(e)``."""
    m, k = codes.shape
    vals = decode(codes, fmt).reshape(m, k // bs, bs)
    scl = np.exp2(exps.astype(F32)).astype(F32).T[..., None]
    return (vals * scl).reshape(m, k).astype(F32)


def block_dual_quantize(w: np.ndarray, bs: int, ef: np.ndarray | None = None):
    """``fused_dual_quantize_fp8`` without SR (kernels.py:1749-1875, :288-459).

    Returns ``(hi, lo, e_hi int8 [K/bs,N], e_lo int8 [K/bs,N], ef_new|None)``.
    ``e_lo`` is -128 for blocks whose residual amax is below 1e-12; the new
    error is ``w - deq(hi) - deq(lo)`` evaluated left to right
    (kernels.py:1870-1873).
    """
    w = np.asarray(w, dtype=F32)
    wc = w + ef if ef is not None else w
    wb = _blocks(wc, bs)
    e_hi = block_exponent(np.max(np.abs(wb), axis=-1))
    mx = F32(448.0)
    hi = encode(np.clip(wb * _pow2(-e_hi)[..., None], -mx, mx), E4M3)
    deq_hi = decode(hi, E4M3) * _pow2(e_hi)[..., None]
    r = (wb - deq_hi).astype(F32)
    amax_lo = np.max(np.abs(r), axis=-1)
    zero = amax_lo < F32(1e-12)
    e_lo = block_exponent(amax_lo)
    div = np.where(zero, F32(1.0), _pow2(e_lo))
    lo = encode(np.clip(r / div[..., None], -mx, mx), E4M3)
    e_lo_store = np.where(zero, -128, e_lo)
    shape = w.shape
    hi = hi.reshape(shape)
    lo = lo.reshape(shape)
    e_hi8 = np.ascontiguousarray(e_hi.T.astype(np.int8))
    e_lo8 = np.ascontiguousarray(e_lo_store.T.astype(np.int8))
    ef_new = None
    if ef is not None:
        ef_new = (w - block_dequantize(hi, e_hi8, bs)) - block_dequantize(lo, e_lo8, bs)
    return hi, lo, e_hi8, e_lo8, ef_new


def block_requant_t(hi: np.ndarray, lo: np.ndarray | None, e_hi: np.ndarray,
                    e_lo: np.ndarray | None, bs: int):
    """A block dual-quantised W [D_out, D_in] re-blocked along D_out (the
    weight operand of an FP8 block dgrad; the reference has no such step:
    its dgrad multiplies ``block_dequantize_fp8`` outputs, kernels.py:
    2326-2425).  ``v = deq(hi) + deq(lo)`` in float32 (kernels.py:1725-1746),
    then ``fused_dual_quantize_fp8`` of ``v.T`` without EF or SR
    (kernels.py:1749-1875).  Returns ``(hi_t, lo_t, e_hi_t, e_lo_t)``, codes
    [D_in, D_out], exponents [D_out/bs, D_in].
    """
    v = block_dequantize(hi, e_hi, bs)
    if lo is not None:
        v = (v + block_dequantize(lo, e_lo, bs)).astype(F32)
    hi_t, lo_t, eh_t, el_t, _ = block_dual_quantize(np.ascontiguousarray(v.T), bs)
    return hi_t, lo_t, eh_t, el_t


def block_scale_f32(amax: np.ndarray, dtype: str = "f32", fmt: str = E4M3) -> np.ndarray:
    """fp32 block scales: ``per_tensor_scale``'s rule (core.py:100-101) on
    each block's amax -- clamp to 1e-12, reciprocal and product with
    FP8_MAX each rounded to ``dtype``."""
    a = np.maximum(np.asarray(amax, dtype=F32), _round_dtype(np.array([1e-12], F32), dtype)[0])
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        rcp = _round_dtype((F32(1.0) / a).astype(F32), dtype)
        return _round_dtype((rcp * F32(FP8_MAX[fmt])).astype(F32), dtype).astype(F32)


def block_quantize_f32s(x: np.ndarray, bs: int, dtype: str = "f32", fmt: str = E4M3):
    """Block quantisation with fp32 scales: ``to_fp8_e4m3`` / ``to_fp8_e5m2``
    (core.py:85-106, :137-158) applied to every (row, K-block).  The
    reference has no such format (its blocks use power-of-two exponents,
    kernels.py:205-275); this is the non-power-of-two ``448 / amax`` block
    scaling run beside it.

    Returns ``(codes [M,K] uint8, inv [K/bs, M] float32)`` where ``inv`` is
    ``1 / scale``, the block's dequantisation multiplier.
    """
    x = np.asarray(x, dtype=F32)
    xb = _blocks(x, bs)
    scale = block_scale_f32(np.max(np.abs(xb), axis=-1), dtype, fmt)
    mx = F32(FP8_MAX[fmt])
    codes = encode(np.clip(xb * scale[..., None], -mx, mx), fmt).reshape(x.shape)
    with np.errstate(divide="ignore"):
        inv = (F32(1.0) / scale).astype(F32)
    return codes, np.ascontiguousarray(inv.T)


def block_dequantize_f32s(codes: np.ndarray, inv: np.ndarray, bs: int,
                          fmt: str = E4M3) -> np.ndarray:
    """``fp8 * inv[kb, row]`` in float32."""
    m, k = codes.shape
    vals = decode(codes, fmt).reshape(m, k // bs, bs)
    return (vals * inv.T[..., None].astype(F32)).reshape(m, k).astype(F32)


def block_dual_quantize_f32s(w: np.ndarray, bs: int, ef: np.ndarray | None = None):
    """Dual quantisation with fp32 block scales: the fused block kernel's
    structure (kernels.py:288-459) with :func:`block_quantize_f32s`'s rule
    for both components (fp32 rule on ``w + ef`` and on the residual
    ``r = w' - hi * inv_hi``; no zero-block sentinel) and the block path's
    error update order ``(w - deq(hi)) - deq(lo)`` (kernels.py:1870-1873).

    Returns ``(hi, lo, inv_hi [K/bs,N], inv_lo [K/bs,N], ef_new|None)``.
    """
    w = np.asarray(w, dtype=F32)
    wc = w + ef if ef is not None else w
    hi, inv_hi = block_quantize_f32s(wc, bs)
    deq_hi = block_dequantize_f32s(hi, inv_hi, bs)
    r = (wc - deq_hi).astype(F32)
    lo, inv_lo = block_quantize_f32s(r, bs)
    ef_new = None
    if ef is not None:
        ef_new = ((w - deq_hi) - block_dequantize_f32s(lo, inv_lo, bs)).astype(F32)
    return hi, lo, inv_hi, inv_lo, ef_new


def sr_candidates_block(x: np.ndarray):
    """Deterministic part of the in-kernel SR of kernels.py:398-423.

    ``x`` is the scaled and clamped residual.  Returns ``(rtn, other, frac,
    exact)``.  The Triton cast saturates (``satfinite``) so ``other`` never
    leaves +-448.
    """
    x = np.asarray(x, dtype=F32)
    mx = F32(448.0)
    rtn = encode(x, E4M3)
    rtn_f = decode(rtn, E4M3)
    diff = x - rtn_f
    d = np.where(diff >= 0, F32(1), F32(-1))
    abs_rtn = np.maximum(np.abs(rtn_f), F32(1e-12))
    nudge = d * abs_rtn * F32(0.25)
    other = encode(np.clip(rtn_f + nudge, -mx, mx), E4M3)
    other_f = decode(other, E4M3)
    gap = np.maximum(np.abs(other_f - rtn_f), F32(1e-45))
    with np.errstate(over="ignore"):
        frac = np.minimum(np.abs(diff) / gap, F32(1))
    boundary = np.abs(other_f - rtn_f) < F32(1e-45)
    exact = (np.abs(diff) < F32(1e-45)) | boundary
    return rtn, other, frac.astype(F32), exact


def column_sums(x: np.ndarray) -> np.ndarray:
    """The bias gradient ``grad_2d.sum(0)`` (``tcfp/nn/__init__.py:558``) in
    the fixed fp32 order of this build's column-sum producers.

    The reference leaves the order to torch's reduction; this build fixes
    one so that its two producers (the quantising pass and the dgrad GEMM's
    GELU epilogue) agree bit for bit, and the result agrees with the
    reference's within fp32 rounding:

    1. per 64-row group (missing rows +0): ``y = x[0:32] + x[32:64]``, then
       the halving folds ``y = y[:d] + y[d:2d]`` for d = 16, 8, 4, 2, 1;
    2. the group sums P[q] are added by eight lanes (lane r takes the groups
       q = r mod 8: four accumulators over q, q + 8, q + 16, q + 24 for each
       32 groups, then the remaining groups into the first), each lane's
       ``(s0 + s1) + (s2 + s3)``, then the lanes in turn.
    """
    x = np.asarray(x, dtype=F32)
    rows, cols = x.shape
    groups = -(-rows // 64)
    xp = np.zeros((groups * 64, cols), F32)
    xp[:rows] = x
    y = xp.reshape(groups, 64, cols)
    y = y[:, :32] + y[:, 32:]
    while y.shape[1] > 1:
        d = y.shape[1] // 2
        y = y[:, :d] + y[:, d:]
    p = y[:, 0]
    lanes = []
    for lane in range(8):
        s = [np.zeros(cols, F32) for _ in range(4)]
        r = lane
        while r + 24 < groups:
            for j in range(4):
                s[j] = s[j] + p[r + 8 * j]
            r += 32
        while r < groups:
            s[0] = s[0] + p[r]
            r += 8
        lanes.append((s[0] + s[1]) + (s[2] + s[3]))
    out = lanes[0]
    for v in lanes[1:]:
        out = out + v
    return out
