"""Error-feedback state on disk, in the reference's ``ef_state.pt`` format.

The reference's ``TCFPCheckpointer`` writes, for every ``TCFPLinear`` with an
``ErrorFeedbackState``, ``{outer_key: {"_buffers", "_amax_ema",
"_delayed_amax", "_residual_ratio", "_step_count", "_ema_decay"}}`` with the
tensors on the CPU, where ``outer_key`` is the layer's ``_param_name`` or,
when that is empty, its ``named_modules()`` path
(``tcfp/training/checkpointing.py:200-224``); restoring moves the tensors to
the layer's weight device (``:226-271``).  These functions produce and
consume the same structure, so EF buffers trained here resume under the
reference's checkpointer and vice versa.

The snapshot holds only tensors, ints, floats and dicts, so it loads with
``torch.load(..., weights_only=True)``.
"""
from __future__ import annotations

from pathlib import Path

import torch
import torch.nn as nn

from .nn import TCFPLinear

_DICTS = ("_buffers", "_amax_ema", "_delayed_amax", "_residual_ratio")


def _layers(model: nn.Module) -> dict[str, TCFPLinear]:
    return {
        (m._param_name if m._param_name else name): m
        for name, m in model.named_modules()
        if isinstance(m, TCFPLinear) and m._error_state is not None
    }


def ef_state_dict(model: nn.Module) -> dict[str, dict]:
    """The reference's EF snapshot of ``model`` (tensors copied to the CPU)."""
    snap: dict[str, dict] = {}
    for key, m in _layers(model).items():
        ef = m._error_state
        entry = {d: {k: v.detach().cpu().clone() for k, v in getattr(ef, d).items()}
                 for d in _DICTS}
        entry["_step_count"] = dict(ef._step_count)
        entry["_ema_decay"] = float(ef._ema_decay)
        snap[key] = entry
    return snap


def load_ef_state_dict(model: nn.Module, snap: dict[str, dict]) -> int:
    """Restore a snapshot into ``model``'s layers (tensors moved to each
    layer's weight device); keys without a matching layer are skipped, as
    in the reference.  Returns the number of layers restored."""
    layers = _layers(model)
    n = 0
    for key, state in snap.items():
        m = layers.get(str(key))
        if m is None:
            continue
        ef = m._error_state
        dev = m.weight.device
        for d in _DICTS:
            src = state.get(d, {})
            assert isinstance(src, dict), f"{key}.{d} must be a dict"
            getattr(ef, d).update({k: v.to(dev) for k, v in src.items()})
        steps = state.get("_step_count", {})
        assert isinstance(steps, dict), f"{key}._step_count must be a dict"
        ef._step_count.update(steps)
        if state.get("_ema_decay") is not None:
            ef._ema_decay = float(state["_ema_decay"])
        n += 1
    return n


def save_ef_state(model: nn.Module, path: str | Path) -> None:
    """``torch.save`` of :func:`ef_state_dict` (the reference's
    ``ef_state.pt``)."""
    torch.save(ef_state_dict(model), Path(path))


def load_ef_state(model: nn.Module, path: str | Path) -> int:
    """Load an ``ef_state.pt`` (written here or by the reference) into
    ``model``; returns the number of layers restored."""
    snap = torch.load(Path(path), map_location="cpu", weights_only=True)
    return load_ef_state_dict(model, snap)
