"""Import-compatible alias of hp_rms_norm_amd under the reference's package
name, so ``import hp_rms_norm; hp_rms_norm.hp_rms_norm(x, w, r, eps)`` and
``hp_rms_norm.relu(out, x)`` work unchanged (reference: hp_rms_norm/__init__.py:1-3)."""
import torch  # noqa: F401

from hp_rms_norm_amd import _C  # noqa: F401
from hp_rms_norm_amd import ops  # noqa: F401
from hp_rms_norm_amd.ops import *  # noqa: F401,F403
