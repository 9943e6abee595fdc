"""tcfp_amd -- MI355X-native (gfx950) TCFP-12 dual-FP8 training path.

Drop-in for the reference's tensor-core path (bwiemz/tcfp):
``tcfp_amd.core`` mirrors ``tcfp.core``'s FP8 casts and error-feedback
state, ``tcfp_amd.kernels`` mirrors ``tcfp.kernels``' operator API, and
``tcfp_amd.nn`` mirrors ``tcfp.nn``'s ``TCFPLinear`` / ``convert_to_tcfp``
and autograd Functions.  All device work runs in hand-written HIP kernels
(``libtcfp_hip.so``, C ABI in ``include/tcfp_hip.h``).
"""
from . import core, cuda_ext, kernels, nn  # noqa: F401
from .core import (  # noqa: F401
    ErrorFeedbackState,
    TCFPMode,
    to_fp8_e4m3,
    to_fp8_e4m3_nf_aware,
    to_fp8_e5m2,
)
from .nn import TCFPLinear, TCFPMLP, convert_to_tcfp, fuse_tcfp_mlp  # noqa: F401

__version__ = "0.1.0"
