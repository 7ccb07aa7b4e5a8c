"""Callers of the slice/deslice path: the physics-attention layer and its MLP
(reference ``flashslice/layers``), with ``use_fused_slice=True`` running on
the HIP operators of ``flashslice_amd.kernels``; the point-stream LayerNorm
and Linear the Transolver model (``flashslice_amd.models``) builds on."""

from .basic import ACTIVATION, MLP, PointLinear
from .norm import PointLayerNorm
from .physics_attention import Physics_Attention_Irregular_Mesh

__all__ = ["ACTIVATION", "MLP", "Physics_Attention_Irregular_Mesh", "PointLayerNorm",
           "PointLinear"]
