"""The reference's import name for this build.

Code written against bwiemz/tcfp imports ``tcfp``, ``tcfp.core``,
``tcfp.nn``, ``tcfp.kernels`` and ``tcfp.cuda_ext``.  Importing this package
registers the MI355X-native package ``tcfp_amd`` and its submodules under
those names in ``sys.modules``, so ``import tcfp`` binds ``tcfp_amd`` itself
and ``from tcfp.nn import TCFPLinear`` returns ``tcfp_amd.nn.TCFPLinear``:
the same module objects, not copies, so module state (``set_block_dgrad``,
tile policy, the HIP library handle) is shared between the two names.
"""
import sys

import tcfp_amd as _pkg
from tcfp_amd import core, cuda_ext, kernels, nn  # noqa: F401

for _name in ("core", "cuda_ext", "kernels", "nn"):
    sys.modules[f"{__name__}.{_name}"] = getattr(_pkg, _name)
sys.modules[__name__] = _pkg
