"""ctypes binding of ``libtcfp_hip.so`` (the C ABI declared in include/tcfp_hip.h).

The product path has no fallback: if the library is missing or no GPU is
visible, every op raises.  Device tensors cross the boundary as raw
pointers; work is enqueued on torch's current HIP stream.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libtcfp_hip.so")

FP8_E4M3 = 0
FP8_E5M2 = 1
DTYPE_F32 = 0
DTYPE_BF16 = 1

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64

JOB_DUAL = 0
JOB_ACT = 1


class QuantJob(ctypes.Structure):
    """``tcfp_quant_job`` (include/tcfp_hip.h): one tensor of
    ``tcfp_quantize_batch``."""

    _fields_ = [
        ("kind", _i32), ("x", _c_void_p), ("x_dtype", _i32), ("rows", _i64), ("cols", _i64),
        ("ef", _c_void_p), ("update_ef", _i32), ("fp8_fmt", _i32), ("q", _c_void_p),
        ("q_t", _c_void_p), ("inv", _c_void_p), ("q_lo", _c_void_p), ("q_lo_t", _c_void_p),
        ("inv_lo", _c_void_p),
    ]

# name -> argtypes (all return int status unless listed in _RESTYPE)
_SIGNATURES = {
    "tcfp_status_string": [_i32],
    "tcfp_workspace_bytes": [],
    "tcfp_quantize_per_tensor": [_c_void_p, _i32, _i64, _i64, _i32, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_quantize_per_tensor_sr": [_c_void_p, _i32, _i64, _i64, _c_void_p, _u64, _u64,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_block_scales": [_c_void_p, _i32, _i64, _i64, _i32, ctypes.c_float, _c_void_p,
                          _c_void_p],
    "tcfp_colsum_workspace_bytes": [_i64, _i64],
    "tcfp_quantize_per_tensor_colsum": [_c_void_p, _i32, _i64, _i64, _i32, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                        ctypes.c_size_t, _c_void_p],
    "tcfp_gelu_quantize_per_tensor": [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_gelu_backward_quantize_per_tensor_colsum": [_c_void_p, _c_void_p, _i64, _i64, _i32,
                                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                                      _c_void_p, _c_void_p, _c_void_p,
                                                      ctypes.c_size_t, _c_void_p],
    "tcfp_dual_quantize_per_tensor": [_c_void_p, _i32, _i64, _i64, _c_void_p, _i32, _i32, _u64,
                                      _u64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_dual_quantize_per_tensor_noalloc": [_c_void_p, _i32, _i64, _i64, _c_void_p, _i32,
                                              _i32, _u64, _u64, _c_void_p, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                              _c_void_p],
    "tcfp_dual_quantize_per_tensor_delayed": [_c_void_p, _i32, _i64, _i64, _c_void_p, _i32,
                                              _c_void_p, _c_void_p, ctypes.c_float,
                                              ctypes.c_float, _i32, _c_void_p, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_dual_quantize_per_tensor_nf": [_c_void_p, _i32, _i64, _i64, _c_void_p, _i32,
                                         ctypes.c_float, _i32, _i32, _u64, _u64, _c_void_p,
                                         _c_void_p, ctypes.c_float, ctypes.c_float, _i32,
                                         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _c_void_p],
    "tcfp_block_quantize": [_c_void_p, _i32, _i64, _i64, _i32, _i32, _c_void_p, _c_void_p,
                            _c_void_p],
    "tcfp_block_dual_quantize": [_c_void_p, _i32, _i64, _i64, _i32, _c_void_p, _i32, _i32, _u64,
                                 _u64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_block_dequantize": [_c_void_p, _i32, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p],
    "tcfp_block_requant_t": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32,
                             _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_block_quantize_f32s": [_c_void_p, _i32, _i64, _i64, _i32, _i32, _c_void_p, _c_void_p,
                                 _c_void_p],
    "tcfp_block_dual_quantize_f32s": [_c_void_p, _i32, _i64, _i64, _i32, _c_void_p, _i32, _i32,
                                      _u64, _u64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p],
    "tcfp_block_dequantize_f32s": [_c_void_p, _i32, _c_void_p, _i64, _i64, _i32, _c_void_p,
                                   _c_void_p],
    "tcfp_dual_gemm": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _i64,
                       _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64,
                       _c_void_p],
    "tcfp_dual_gemm_gelu_quantize": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32, _i64,
                                     _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                     _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32,
                                     _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_gelu_amax_rule_status": [_c_void_p, _c_void_p, _c_void_p],
    "tcfp_dual_gemm_dgelu_quantize_colsum": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32,
                                             _i64, _i64, _i64, _i64, _c_void_p, _c_void_p,
                                             _c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p,
                                             _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                             _c_void_p, ctypes.c_size_t, _c_void_p],
    "tcfp_block_dual_gemm": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _i32, _i64,
                             _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p,
                             _i32, _i64, _c_void_p],
    "tcfp_block_dual_gemm_f32s": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _i32,
                                  _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p,
                                  _c_void_p, _i32, _i64, _c_void_p],
    "tcfp_act_quant_block_dual_gemm": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i64,
                                       _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p,
                                       _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p],
    "tcfp_wtquant_block_dual_gemm": [_c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32, _i64,
                                     _i64, _i64, _i32, _c_void_p, _i32, _u64, _u64, _c_void_p,
                                     _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32,
                                     _i64, _c_void_p],
    "tcfp_block_dual_gemm_dx": [_c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                _c_void_p, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p,
                                ctypes.c_size_t, _c_void_p],
    "tcfp_block_dual_gemm_dx_workspace_bytes": [_i64, _i64, _i64],
    "tcfp_block_wgrad": [_c_void_p, _i64, _i64, _c_void_p, _i32, _c_void_p, _i64, _i32, _c_void_p,
                         _c_void_p, ctypes.c_size_t, _c_void_p],
    "tcfp_block_wgrad_workspace_bytes": [_i64, _i64, _i64],
    "tcfp_block_grad_prep": [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p, _i32, _c_void_p,
                             _c_void_p, _c_void_p, _c_void_p, ctypes.c_size_t, _c_void_p],
    "tcfp_block_grad_prep_workspace_bytes": [_i64, _i64],
    "tcfp_block_dual_gemm_dx_bf16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                     _i64, _i64, _i32, _c_void_p, _c_void_p, ctypes.c_size_t,
                                     _c_void_p],
    "tcfp_block_dual_gemm_dx_bf16_workspace_bytes": [_i64, _i64],
    "tcfp_block_wgrad_presplit": [_c_void_p, _i32, _i64, _i64, _c_void_p, _i32, _c_void_p, _i64,
                                  _i32, _c_void_p, _c_void_p, ctypes.c_size_t, _c_void_p],
    "tcfp_block_wgrad_presplit_workspace_bytes": [_i64, _i64, _i64, _i32],
    "tcfp_quantize_batch_workspace_bytes": [_i32],
    "tcfp_quantize_batch": [_i32, ctypes.POINTER(QuantJob), _c_void_p, ctypes.c_size_t, _c_void_p],
    "tcfp_gemm_set_tile_policy": [_i32],
    "tcfp_dual_quantize_set_candidates": [_i32],
    "tcfp_transpose_u8": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "tcfp_selftest_fp8_cvt": [_u32, _u32, _i32, _c_void_p, _c_void_p],
    "tcfp_selftest_sr_block": [_u32, _u32, ctypes.c_float, _c_void_p, _c_void_p],
    "tcfp_selftest_philox": [_u32, _u32, _u32, _u32, _u32, _u32, _i64, _c_void_p, _c_void_p],
}
_RESTYPE = {
    "tcfp_status_string": ctypes.c_char_p,
    "tcfp_workspace_bytes": ctypes.c_size_t,
    "tcfp_colsum_workspace_bytes": ctypes.c_size_t,
    "tcfp_block_dual_gemm_dx_workspace_bytes": ctypes.c_size_t,
    "tcfp_block_wgrad_workspace_bytes": ctypes.c_size_t,
    "tcfp_block_grad_prep_workspace_bytes": ctypes.c_size_t,
    "tcfp_block_dual_gemm_dx_bf16_workspace_bytes": ctypes.c_size_t,
    "tcfp_block_wgrad_presplit_workspace_bytes": ctypes.c_size_t,
    "tcfp_quantize_batch_workspace_bytes": ctypes.c_size_t,
}

_lib = None
_lock = threading.Lock()


def exported_symbols() -> tuple[str, ...]:
    return tuple(_SIGNATURES)


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load and type the library (no GPU needed to load)."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"tcfp_amd HIP library not found at {p}; build it with "
                "`python -m tcfp_amd.build` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(p))
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        if path is None:
            _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load_library()


def is_available() -> bool:
    """True when the library is built and a GPU is visible."""
    if not LIB_PATH.exists():
        return False
    try:
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch without a GPU runtime
        return False


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().tcfp_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Raw handle of torch's current stream on ``device`` (the stream every
    op here enqueues on).  torch's own raw-stream query costs ~0.1 us
    against ~2 us for ``torch.cuda.current_stream``; both give the same
    handle."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


_ws: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device) -> torch.Tensor:
    """Reduction scratch for the current stream of ``device``.

    Per-tensor reductions pass per-workgroup partial maxima from one launch
    to the next through it.  Stream order makes one buffer per (device,
    stream) safe for every call on that stream.
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, stream_of(device))
    ws = _ws.get(key)
    if ws is None:
        nbytes = int(lib().tcfp_workspace_bytes())
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _ws[key] = ws
    return ws


_bws: dict[tuple[int, int], torch.Tensor] = {}
MAX_BATCH_JOBS = 4


def batch_workspace(device: torch.device) -> torch.Tensor:
    """``tcfp_quantize_batch``'s reduction scratch (room for its largest
    batch) for the current stream of ``device``; stream order makes one per
    (device, stream) safe."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, stream_of(device))
    ws = _bws.get(key)
    if ws is None:
        nbytes = int(lib().tcfp_quantize_batch_workspace_bytes(MAX_BATCH_JOBS))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _bws[key] = ws
    return ws


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU; raise otherwise (there is no CPU path)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "tcfp_amd ops run only on the GPU (hand-written HIP kernels); got a "
                f"{t.device} tensor"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    lib()
    return dev
