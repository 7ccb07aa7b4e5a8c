"""The reference's import path for this build (reference
``flashslice/__init__.py:1-27``)::

    from flashslice import Transolver
    from flashslice.kernels import fused_slice, fused_deslice, unsupported_dims

``flashslice`` and its submodules -- ``kernels`` (``slice_ops``,
``blocked``, plus this build's ``tied``, ``coupling`` and ``varlen``), ``layers``
(``basic``, ``physics_attention``, ``norm``) and ``models``
(``transolver``) -- are bound to the modules of ``flashslice_amd``, the
package that holds the HIP operators. They are the same module objects, not
copies: a setting made through either name (``set_dot_mode``,
``set_kernel_mode``, ...) is one process-wide state, and the
``torch.ops.flashslice`` operators are registered once. Code written
against the reference therefore runs unchanged on the MI355X kernels.
"""

import importlib
import sys

import flashslice_amd as _impl

_SUBMODULES = ("kernels", "kernels.slice_ops", "kernels.blocked", "kernels.tied",
               "kernels.coupling", "kernels.varlen", "layers", "layers.basic", "layers.physics_attention",
               "layers.norm", "models", "models.transolver")

for _name in _SUBMODULES:
    _mod = importlib.import_module(_impl.__name__ + "." + _name)
    sys.modules[__name__ + "." + _name] = _mod
    if "." not in _name:
        globals()[_name] = _mod

from flashslice_amd.layers.physics_attention import Physics_Attention_Irregular_Mesh  # noqa: E402
from flashslice_amd.models.transolver import (  # noqa: E402
    TokenTransformerBlock, Transolver, TransolverBlock)

__version__ = _impl.__version__
__all__ = ["Transolver", "TransolverBlock", "TokenTransformerBlock",
           "Physics_Attention_Irregular_Mesh"]
