"""tcfp_amd -- MI355X-native (gfx950) TCFP-12 dual-FP8 training path.

Drop-in for the reference's tensor-core path (bwiemz/tcfp): the top level
exports what ``tcfp/__init__.py:12-34`` exports, ``tcfp_amd.core`` mirrors
``tcfp.core``'s FP8 casts, block scales, FP8 matmuls and error-feedback
state, ``tcfp_amd.kernels`` mirrors ``tcfp.kernels``' operator API,
``tcfp_amd.cuda_ext`` its ``tcfp.cuda_ext`` entry points, and
``tcfp_amd.nn`` ``tcfp.nn``'s ``TCFPLinear`` / ``convert_to_tcfp`` and
autograd Functions.  ``import tcfp`` (the sibling ``tcfp`` package) binds
this package under the reference's import name.  All device work runs in
hand-written HIP kernels (``libtcfp_hip.so``, C ABI in
``include/tcfp_hip.h``).
"""
from . import core, cuda_ext, kernels, nn  # noqa: F401
from .core import (  # noqa: F401
    ErrorFeedbackState,
    FP8Config,
    TCFPMode,
    ensure_column_major,
    fp8_matmul,
    to_fp8_e4m3,
    to_fp8_e4m3_nf_aware,
    to_fp8_e4m3_sr,
    to_fp8_e5m2,
)
from .nn import TCFPLinear, TCFPMLP, convert_to_tcfp, fuse_tcfp_mlp  # noqa: F401

__all__ = [
    "ErrorFeedbackState",
    "FP8Config",
    "TCFPMode",
    "ensure_column_major",
    "fp8_matmul",
    "to_fp8_e4m3",
    "to_fp8_e4m3_nf_aware",
    "to_fp8_e4m3_sr",
    "to_fp8_e5m2",
]

__version__ = "0.1.0"
