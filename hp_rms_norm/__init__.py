"""Import-compatible alias of hp_rms_norm_amd under the reference's package
name (reference: hp_rms_norm/__init__.py:1-3), so existing callers work
unchanged: ``import hp_rms_norm; hp_rms_norm.hp_rms_norm(x, w, r, eps)``,
``hp_rms_norm.relu(out, x)``, ``from hp_rms_norm.ops import hp_rms_norm`` and
``from hp_rms_norm import _C`` (the extension module that registers
``torch.ops.hp_rms_norm.*``)."""
import sys

import torch  # noqa: F401

from hp_rms_norm_amd import _C

sys.modules.setdefault(__name__ + "._C", _C)

from .ops import *  # noqa: E402,F401,F403
from . import ops  # noqa: E402,F401
