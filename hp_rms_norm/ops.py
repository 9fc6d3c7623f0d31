"""The reference's ``hp_rms_norm.ops`` module (hp_rms_norm/ops.py:1-24):
``hp_rms_norm(input, weight, residual, eps)`` and ``relu(output, input)``,
with the same positional arguments, in-place semantics and ``None`` return,
plus this build's further operators, all from ``hp_rms_norm_amd.ops``."""
from hp_rms_norm_amd.ops import *  # noqa: F401,F403
from hp_rms_norm_amd.ops import __all__  # noqa: F401
