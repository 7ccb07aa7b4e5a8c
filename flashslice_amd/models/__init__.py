"""The Transolver model (reference ``flashslice/models``): blocks of
physics-attention and MLP over a point stream, with ``use_fused_slice=True``
running the slice/deslice path on the HIP operators."""

from .transolver import TokenTransformerBlock, Transolver, TransolverBlock

__all__ = ["Transolver", "TransolverBlock", "TokenTransformerBlock"]
