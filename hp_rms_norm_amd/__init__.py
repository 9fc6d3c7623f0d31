"""MI355X (gfx950) fused residual-add + RMSNorm.

Importing the package imports its extension module ``_C`` (``_C.so``, built
by ``python hp_rms_norm_amd/build.py``), which registers
``torch.ops.hp_rms_norm.*`` and calls the HIP kernels of ``libhprms.so``
through their C ABI.  Mirrors the reference package's loader
(hp_rms_norm/__init__.py:1-3): ``import torch``, import ``_C``, re-export the
ops.  There is no CPU implementation: a missing library is an ImportError,
and the ops accept HIP tensors only.
"""
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNEL_LIB = os.path.join(_HERE, "libhprms.so")
TORCH_LIB = os.path.join(_HERE, "_C.so")

if not os.path.exists(TORCH_LIB) or not os.path.exists(KERNEL_LIB):
    raise ImportError(
        f"hp_rms_norm_amd: native libraries not built ({TORCH_LIB}, {KERNEL_LIB}); "
        "run `python hp_rms_norm_amd/build.py`")

from . import _C  # noqa: E402  (registers torch.ops.hp_rms_norm.*)
from .ops import *  # noqa: E402,F401,F403
from . import ops  # noqa: E402,F401
