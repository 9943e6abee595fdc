"""FP8 primitives of the TCFP-12 path (drop-in for ``tcfp.core``).

``to_fp8_e4m3`` / ``to_fp8_e5m2`` keep the reference's exact semantics
(``tcfp/core.py:85-158``) -- codes and scales bit-identical -- but run as
HIP kernels (one amax pass, one quantise pass, no host synchronisation);
so do the stochastic-rounding casts (``to_fp8_e4m3_sr``,
``stochastic_round_to_fp8_e4m3``), ``compute_block_scales`` and the FP8
matmuls ``fp8_matmul`` / ``fp8_matmul_nn`` (the hand-written FP8 GEMM in
place of ``torch._scaled_mm``).  ``ErrorFeedbackState`` is the reference's
per-parameter buffer store (``tcfp/core.py:298-326``), keyed by parameter
name.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum, auto

import torch

from . import _hip
from . import kernels as _k

FP8_E4M3_MAX: float = 448.0
FP8_E4M3_MIN: float = -448.0
FP8_E4M3_SMALLEST_NORMAL: float = 2**-6
FP8_E5M2_MAX: float = 57344.0
FP8_E5M2_MIN: float = -57344.0

DEFAULT_BLOCK_SIZE: int = 32
VALID_BLOCK_SIZES: tuple[int, ...] = (16, 32, 64, 128)

SCALE_EXPONENT_BIAS: int = 127


class TCFPMode(Enum):
    """Available TCFP precision modes (reference ``tcfp/core.py:46-49``)."""

    TCFP12 = auto()


@dataclass
class FP8Config:
    """Configuration record (reference ``tcfp/core.py:52-77``)."""

    mode: TCFPMode = TCFPMode.TCFP12
    block_size: int = DEFAULT_BLOCK_SIZE
    e4m3_for_weights: bool = True
    e5m2_for_grads: bool = True
    error_feedback: bool = True
    stochastic_rounding: bool = False

    def __post_init__(self) -> None:
        if self.block_size not in VALID_BLOCK_SIZES:
            raise ValueError(
                f"block_size must be one of {VALID_BLOCK_SIZES}, got {self.block_size}"
            )


def to_fp8_e4m3(
    tensor: torch.Tensor,
    scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor FP8 E4M3 cast; returns ``(fp8, inv_scale)`` with inv_scale (1,) fp32.

    Without ``scale``: ``amax = |t|.max().clamp(min=1e-12)``,
    ``scale = 448 / amax`` evaluated as torch does (reciprocal then product,
    both in t's dtype), ``fp8 = RNE(clamp(t.float() * scale))``,
    ``inv = 1 / scale``.
    """
    q, inv = _k.quantize_per_tensor(tensor, torch.float8_e4m3fn, scale)
    return q, inv


def to_fp8_e4m3_sr(
    tensor: torch.Tensor,
    scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor FP8 E4M3 cast with stochastic rounding
    (``tcfp/core.py:109-134``): the scale of :func:`to_fp8_e4m3`, then
    :func:`stochastic_round_to_fp8_e4m3` on the scaled, clamped values, so
    that ``E[dequant(quant(x))] = x``.  Returns ``(fp8, inv_scale)``."""
    q, inv = _k.quantize_per_tensor_sr(tensor, scale)
    return q, inv


def stochastic_round_to_fp8_e4m3(tensor: torch.Tensor) -> torch.Tensor:
    """FP8 E4M3 with stochastic rounding of values already in range
    (``tcfp/core.py:418-464``): each value goes to its round-to-nearest code
    or that code's neighbour toward it, the neighbour with probability
    ``|x - lo| / |hi - lo|``; exact values keep their code.  (Values past
    +-448, outside the reference's contract, saturate here.)"""
    one = torch.ones(1, dtype=torch.float32, device=tensor.device)
    q, _ = _k.quantize_per_tensor_sr(tensor, one)
    return q


def to_fp8_e5m2(
    tensor: torch.Tensor,
    scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor FP8 E5M2 cast (``tcfp/core.py:137-158``), FP8_MAX = 57344."""
    q, inv = _k.quantize_per_tensor(tensor, torch.float8_e5m2, scale)
    return q, inv


def to_fp8_e4m3_nf_aware(
    tensor: torch.Tensor,
    sigma_factor: float = 3.0,
    stochastic: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor FP8 E4M3 cast with NF-aware (sigma-based) scaling
    (``tcfp/core.py:161-193``); returns ``(fp8, inv_scale)``, inv_scale (1,).

    ``target = sigma_factor * std(t)`` (unbiased std, clamped to 1e-12), or
    the clamped amax when that std is below 1e-6; ``scale = 448 / target``;
    values beyond +-448 saturate; ``stochastic`` rounds each code up or down
    with probability proportional to its distance.  The std is the real one
    rounded once to fp32.  Runs the NF-aware dual quantisation kernels and
    keeps their W_hi half.  An empty tensor gives a NaN scale, as the
    reference's ``std`` of nothing does.
    """
    dev = _hip.require_gpu(tensor)
    t = tensor if tensor.dtype in (torch.float32, torch.bfloat16) else tensor.float()
    if t.numel() == 0:
        return (
            torch.empty(tensor.shape, dtype=torch.float8_e4m3fn, device=dev),
            torch.full((1,), float("nan"), dtype=torch.float32, device=dev),
        )
    flat = t.contiguous().reshape(1, -1)
    hi, _, inv_hi, _ = _k.dual_quantize_per_tensor(
        flat, None, update_ef=False, sigma_factor=sigma_factor, stochastic_hi=stochastic
    )
    return hi.reshape(tensor.shape), inv_hi


def ensure_column_major(t: torch.Tensor) -> torch.Tensor:
    """Column-major view (or copy) of a 2-D tensor (``tcfp/core.py:196-213``)."""
    assert t.ndim == 2, f"ensure_column_major requires 2-D tensor, got {t.ndim}-D"
    if t.stride(0) == 1 and t.stride(1) == t.shape[0]:
        return t
    return t.t().contiguous().t()


def compute_block_scales(
    tensor: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
    fp8_max: float = FP8_E4M3_MAX,
) -> torch.Tensor:
    """Power-of-two block scales ``2^ceil(log2(amax / fp8_max))`` of each
    run of ``block_size`` elements along the last dimension
    (``tcfp/core.py:221-252``), shape ``(..., D // block_size)``, in the
    tensor's dtype (fp32 or bf16; each step rounds as torch's ops on that
    dtype round)."""
    *_, D = tensor.shape
    assert D % block_size == 0, f"D ({D}) must be divisible by block_size ({block_size})"
    return _k.block_scales(tensor, block_size, fp8_max)


def apply_block_scales(
    tensor: torch.Tensor,
    scales: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
) -> torch.Tensor:
    """``tensor / scales`` broadcast over each block (``tcfp/core.py:467-490``)."""
    *batch_dims, D = tensor.shape
    blocked = tensor.reshape(*batch_dims, D // block_size, block_size)
    return (blocked / scales.unsqueeze(-1)).reshape(*batch_dims, D)


def reverse_block_scales(
    tensor: torch.Tensor,
    scales: torch.Tensor,
    block_size: int = DEFAULT_BLOCK_SIZE,
) -> torch.Tensor:
    """``tensor * scales`` broadcast over each block (``tcfp/core.py:493-513``)."""
    *batch_dims, D = tensor.shape
    blocked = tensor.reshape(*batch_dims, D // block_size, block_size)
    return (blocked * scales.unsqueeze(-1)).reshape(*batch_dims, D)


def fp8_matmul(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``(a_fp8 * scale_a) @ (b_fp8 * scale_b)`` on the FP8 MFMA
    (``tcfp/core.py:519-553``, where ``torch._scaled_mm`` does it).

    a [M, K], b [K, N] FP8 (E4M3 or E5M2); per-tensor (single-element) fp32
    scales, i.e. the inverse scales the casts return; fp32 or bf16 output.
    The GEMM reads both operands K-contiguous, so a row-major b is
    transposed once (a column-major b is used as is)."""
    b_t = b_fp8.t()
    if not b_t.is_contiguous():
        b_t = _k.transpose_fp8(b_fp8)
    return _k.fp8_gemm_nt(a_fp8, b_t, scale_a, scale_b, out_dtype=out_dtype)


def fp8_matmul_nn(
    a_fp8: torch.Tensor,
    b_fp8_t: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """:func:`fp8_matmul` with B given transposed, ``b_fp8_t`` [N, K]
    (``tcfp/core.py:556-578``): ``(a * scale_a) @ (b_fp8_t * scale_b).T``."""
    return _k.fp8_gemm_nt(a_fp8, b_fp8_t, scale_a, scale_b, out_dtype=out_dtype)


def bits_per_value(mode: TCFPMode, block_size: int = DEFAULT_BLOCK_SIZE) -> float:
    """Effective bits per value (``tcfp/core.py:586-603``): 8 + 4 plus two
    8-bit block scales amortised over ``block_size`` values."""
    if mode == TCFPMode.TCFP12:
        return 8.0 + 4.0 + 2 * (8.0 / block_size)
    raise ValueError(f"Unknown mode: {mode}")


class ErrorFeedbackState:
    """Per-parameter FP32 error-feedback buffers (``tcfp/core.py:298-326``)
    and the delayed-scaling state (``:328-403``).

    ``get_error`` lazily creates a zero buffer shaped like ``like`` (fp32);
    ``update_error`` rebinds the stored tensor.  The HIP dual-quant kernels
    update the stored buffer in place, which is observationally the same
    for the state machine (``tcfp/nn/__init__.py:375-383``).  Under delayed
    scaling the HIP kernel computes the EMAs on the device and the
    dictionaries are rebound to its outputs
    (``kernels.dual_quantize_per_tensor_delayed``); the methods below give
    the same state transitions with torch ops for callers that drive the
    state themselves.
    """

    def __init__(
        self,
        ema_decay: float = 0.999,
        residual_validation_interval: int = 100,
    ) -> None:
        self._buffers: dict[str, torch.Tensor] = {}
        self._amax_ema: dict[str, torch.Tensor] = {}
        self._ema_decay: float = ema_decay
        self._delayed_amax: dict[str, torch.Tensor] = {}
        self._residual_ratio: dict[str, torch.Tensor] = {}
        self._step_count: dict[str, int] = {}
        self._residual_validation_interval: int = residual_validation_interval

    def get_error(self, name: str, like: torch.Tensor) -> torch.Tensor:
        buf = self._buffers.get(name)
        if buf is None or buf.shape != like.shape:
            buf = torch.zeros(like.shape, dtype=torch.float32, device=like.device)
            self._buffers[name] = buf
        return buf

    def update_error(self, name: str, error: torch.Tensor) -> None:
        self._buffers[name] = error.detach()

    def get_amax_ema(self, name: str, current_amax: torch.Tensor) -> torch.Tensor:
        """EMA of ``current_amax`` (``tcfp/core.py:328-339``)."""
        if name not in self._amax_ema:
            self._amax_ema[name] = current_amax.detach().clone()
        else:
            self._amax_ema[name] = (
                self._ema_decay * self._amax_ema[name]
                + (1 - self._ema_decay) * current_amax.detach()
            )
        return self._amax_ema[name]

    def get_delayed_amax(self, name: str, current_amax: torch.Tensor) -> torch.Tensor:
        """EMA-smoothed amax for delayed scaling; the first call returns
        ``current_amax`` (``tcfp/core.py:341-356``)."""
        if name not in self._delayed_amax:
            self._delayed_amax[name] = current_amax.detach().clone()
            return current_amax
        prev = self._delayed_amax[name]
        self._delayed_amax[name] = (
            self._ema_decay * prev + (1 - self._ema_decay) * current_amax.detach()
        )
        return self._delayed_amax[name]

    def predict_residual_amax(self, name: str, main_amax: torch.Tensor) -> torch.Tensor:
        """``main_amax * ratio`` (``main_amax / 8`` before any ratio),
        clamped to 1e-12 (``tcfp/core.py:358-372``)."""
        ratio_key = f"{name}.ratio"
        if ratio_key not in self._residual_ratio:
            return (main_amax / 8.0).clamp(min=1e-12)
        return (main_amax * self._residual_ratio[ratio_key]).clamp(min=1e-12)

    def update_residual_ratio(self, name: str, main_amax: torch.Tensor,
                              actual_residual_amax: torch.Tensor) -> None:
        """EMA of ``amax_lo / amax_hi`` (``tcfp/core.py:374-393``)."""
        ratio = (actual_residual_amax / main_amax.clamp(min=1e-12)).detach()
        ratio_key = f"{name}.ratio"
        if ratio_key not in self._residual_ratio:
            self._residual_ratio[ratio_key] = ratio
        else:
            self._residual_ratio[ratio_key] = (
                self._ema_decay * self._residual_ratio[ratio_key]
                + (1 - self._ema_decay) * ratio
            )

    def should_validate_residual(self, name: str) -> bool:
        """True on the first call and every ``residual_validation_interval``
        calls (``tcfp/core.py:395-403``)."""
        key = f"{name}.steps"
        count = self._step_count.get(key, 0) + 1
        self._step_count[key] = count
        return count == 1 or count % self._residual_validation_interval == 0

    def reset(self) -> None:
        self._buffers.clear()
        self._amax_ema.clear()
        self._delayed_amax.clear()
        self._residual_ratio.clear()
        self._step_count.clear()
