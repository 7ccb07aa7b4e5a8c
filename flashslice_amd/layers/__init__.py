"""Callers of the slice/deslice path: the physics-attention layer, its MLP
and the Transolver model (reference ``flashslice/layers`` and
``flashslice/models``), with ``use_fused_slice=True`` running on the HIP
operators of ``flashslice_amd.kernels``."""

from .basic import ACTIVATION, MLP, PointLinear
from .norm import PointLayerNorm
from .physics_attention import Physics_Attention_Irregular_Mesh
from .transolver import TokenTransformerBlock, Transolver, TransolverBlock

__all__ = ["ACTIVATION", "MLP", "Physics_Attention_Irregular_Mesh", "PointLayerNorm",
           "PointLinear", "Transolver", "TransolverBlock", "TokenTransformerBlock"]
