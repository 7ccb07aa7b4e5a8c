"""flashslice_amd: FlashSlice's fused slice/deslice operators for AMD MI355X.

    from flashslice_amd.kernels import fused_slice, fused_deslice

The operators keep the reference's ``flashslice.kernels`` API and
``torch.ops.flashslice`` custom-operator boundary; underneath they run
hand-written HIP kernels for gfx950 (``flashslice_amd/csrc``), built in-tree
into ``flashslice_amd/_lib/libflashslice_hip.so`` by
``python -m flashslice_amd.build``.
"""

__version__ = "0.1.0"

# The reference package root exports its model and layer classes
# (reference flashslice/__init__.py:18-27); loaded on first use, so that
# ``python -m flashslice_amd.build`` does not import torch.
_LAYER_NAMES = ("Transolver", "TransolverBlock", "TokenTransformerBlock",
                "Physics_Attention_Irregular_Mesh")
__all__ = list(_LAYER_NAMES) + ["__version__"]


def __getattr__(name):
    if name == "Physics_Attention_Irregular_Mesh":
        from . import layers
        return layers.Physics_Attention_Irregular_Mesh
    if name in _LAYER_NAMES:
        from . import models
        return getattr(models, name)
    raise AttributeError("module 'flashslice_amd' has no attribute %r" % name)
