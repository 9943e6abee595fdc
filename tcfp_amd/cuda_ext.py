"""The reference's ``tcfp.cuda_ext`` operator surface on MI355X.

In the reference this module JIT-builds a cuBLASLt extension and exposes
its dual GEMMs (``tcfp/cuda_ext.py:236-283``); ``tcfp.nn`` prefers it for
the forward when it loads (``tcfp/nn/__init__.py:58-66, 405-421``).  Here
the same names route to the hand-written HIP dual GEMM of
``libtcfp_hip.so`` (the one backend), with the reference's interface and
its ``RuntimeError`` when the backend is unavailable.
"""
from __future__ import annotations

import torch

from . import _hip
from . import kernels as _k


def is_cuda_ext_available() -> bool:
    """True when the HIP library loads and a GPU is visible
    (``tcfp/cuda_ext.py:236-238``)."""
    return _hip.is_available()


def _require() -> None:
    if not is_cuda_ext_available():
        raise RuntimeError(
            "HIP dual GEMM backend not available: build tcfp_amd (python -m tcfp_amd.build) "
            "and run on an MI355X (gfx950)."
        )


def cuda_ext_dual_gemm_forward(
    act_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    act_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
) -> torch.Tensor:
    """Same interface and result as ``fused_dual_gemm_forward``
    (``tcfp/cuda_ext.py:241-259``)."""
    _require()
    return _k.fused_dual_gemm_forward(act_fp8, w_hi_fp8, w_lo_fp8, act_inv, w_hi_inv, w_lo_inv)


def cuda_ext_dual_gemm_backward_dx(
    grad_fp8: torch.Tensor,
    w_hi_fp8: torch.Tensor,
    w_lo_fp8: torch.Tensor,
    grad_inv: torch.Tensor,
    w_hi_inv: torch.Tensor,
    w_lo_inv: torch.Tensor,
) -> torch.Tensor:
    """Same interface and result as ``fused_dual_gemm_backward_dx``
    (``tcfp/cuda_ext.py:262-283``)."""
    _require()
    return _k.fused_dual_gemm_backward_dx(grad_fp8, w_hi_fp8, w_lo_fp8, grad_inv, w_hi_inv,
                                          w_lo_inv)
