"""Dequantised GEMM references in float64 (test oracle; see package docstring).

Each function is the textbook matmul of the *same* FP8 operands the kernel
consumes, dequantised exactly, accumulated in float64.  The reference's
tests hold its kernels to these at 1e-2 (``tests/test_fused_kernels.py:
115-150``) and 1e-3 (``tests/test_block_scaling_kernels.py:146-290``).
"""
from __future__ import annotations

import numpy as np

from .fp8 import E4M3, decode


def _deq(codes, fmt):
    return decode(codes, fmt).astype(np.float64)


def dual_gemm_nt(a, a_fmt, w_hi, w_lo, s_a, s_hi, s_lo, w_fmt=E4M3):
    """``out = (A @ W_hi^T) s_a s_hi + (A @ W_lo^T) s_a s_lo``.

    Forward of ``fused_dual_gemm_forward`` (kernels.py:1545-1601) with
    ``A`` [M,K] and ``W`` [N,K]; the dgrad ``fused_dual_gemm_backward_dx``
    (kernels.py:1604-1666) is this with ``W`` transposed to [D_in, D_out].
    """
    A = _deq(a, a_fmt)
    hi = A @ _deq(w_hi, w_fmt).T
    lo = A @ _deq(w_lo, w_fmt).T
    return hi * (float(s_a) * float(s_hi)) + lo * (float(s_a) * float(s_lo))


def gemm_nt(a, a_fmt, b, b_fmt, s_a, s_b):
    """Single scaled FP8 GEMM ``(A @ B^T) s_a s_b``; the FP8 wgrad of
    nn/__init__.py:546-555 is this with A = G^T and B = X^T."""
    return (_deq(a, a_fmt) @ _deq(b, b_fmt).T) * (float(s_a) * float(s_b))


def block_deq64(codes, exps, bs, fmt=E4M3, lo_sentinel=False):
    """Block dequantisation in float64; ``exps`` is [K/bs, rows] int8.

    ``lo_sentinel``: exponent -128 means "zero block" (kernels.py:757-764).
    """
    m, k = codes.shape
    vals = _deq(codes, fmt).reshape(m, k // bs, bs)
    e = exps.astype(np.float64).T
    s = np.exp2(e)
    if lo_sentinel:
        s = np.where(exps.T == -128, 0.0, s)
    return (vals * s[..., None]).reshape(m, k)


def block_scale_deq64(codes, scales, bs, fmt=E4M3):
    """Dequantise with float32 multiplicative block scales [K/bs, rows]."""
    m, k = codes.shape
    vals = _deq(codes, fmt).reshape(m, k // bs, bs)
    return (vals * scales.astype(np.float64).T[..., None]).reshape(m, k)


def block_dual_gemm_nt(a, a_exps, w_hi, w_lo, e_hi, e_lo, bs):
    """``fused_block_scaled_dual_gemm_forward`` (kernels.py:1939-2028)."""
    A = block_deq64(a, a_exps, bs)
    W = block_deq64(w_hi, e_hi, bs) + block_deq64(w_lo, e_lo, bs, lo_sentinel=True)
    return A @ W.T


def lo_threshold_exps(e_lo, threshold, tile=64):
    """The W_lo sparsity rule of the reference's block GEMMs
    (``tcfp/kernels.py:766-776``, ``:997-1008``, ``:1497``): for every
    K-block and every tile of ``tile`` consecutive weight rows, the W_lo
    part is dropped when the largest W_lo scale of the tile (2^e, 0 for the
    -128 sentinel) is ``<= threshold``.  Returns the exponents with the
    dropped blocks set to the sentinel (which ``block_deq64(...,
    lo_sentinel=True)`` reads as zero)."""
    e = np.asarray(e_lo).copy()
    scale = np.where(e == -128, 0.0, np.exp2(e.astype(np.float64)))
    nkb, n = e.shape
    for t0 in range(0, n, tile):
        drop = scale[:, t0:t0 + tile].max(axis=1) <= threshold
        e[drop, t0:t0 + tile] = -128
    return e


def block_dual_gemm_f32s_nt(a, s_a, w_hi, w_lo, s_hi, s_lo, bs, a_fmt=E4M3):
    """Block dual GEMM with fp32 block multipliers (no sentinel):
    ``sum_kb s_a (s_hi A W_hi^T + s_lo A W_lo^T)``; ``w_lo=None`` gives the
    single GEMM."""
    A = block_scale_deq64(a, s_a, bs, a_fmt)
    W = block_scale_deq64(w_hi, s_hi, bs)
    if w_lo is not None:
        W = W + block_scale_deq64(w_lo, s_lo, bs)
    return A @ W.T


def block_dgrad(g, g_exps, w_hi, w_lo, e_hi, e_lo, bs, g_fmt="e5m2"):
    """``fused_block_scaled_dual_gemm_backward_dx`` (kernels.py:2428-2469)."""
    G = block_deq64(g, g_exps, bs, g_fmt)
    W = block_deq64(w_hi, e_hi, bs) + block_deq64(w_lo, e_lo, bs, lo_sentinel=True)
    return G @ W


def rel_fro(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-300))
