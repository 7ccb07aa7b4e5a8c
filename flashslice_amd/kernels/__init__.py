"""Fused slice/deslice operators for MI355X (gfx950), behind the reference's
``flashslice.kernels`` API.

``fused_slice`` and ``fused_deslice`` are registered ``torch.library``
custom operators (namespace ``flashslice``), so they compose with autograd
and stay single opaque nodes in a ``torch.compile`` graph. Their
implementations call hand-written HIP kernels through the C ABI of
``libflashslice_hip.so`` (``include/flashslice_hip.h``); there is no CPU
implementation.

The eleven public names are those of the reference package
(``flashslice/kernels/__init__.py:44-59``). Additions: ``fused_deslice_slice``
(a deslice -> slice coupling with one fused backward pass, ``tied.py``),
``fused_coupling`` (a slice/deslice coupling in either order with any step
between the two ops, its backward merged into one pass, ``coupling.py``) and
``fused_slice_varlen`` / ``fused_deslice_varlen`` (ragged batches through
row splits, ``varlen.py``).
"""

from .slice_ops import (
    fused_slice,
    fused_deslice,
    unsupported_dims,
    single_tile_dims,
    set_dot_mode,
    set_kernel_mode,
    set_tile_table,
    tile_table,
)
from . import blocked  # noqa: F401  -- registers the flashslice::*_blk ops
from .blocked import set_block_g, set_stats_mode, stats_mode
from .tied import fused_deslice_slice
from .coupling import fused_coupling
from .varlen import fused_deslice_varlen, fused_slice_varlen

__all__ = ["fused_slice", "fused_deslice", "unsupported_dims", "single_tile_dims",
           "set_dot_mode", "set_kernel_mode", "set_block_g", "set_stats_mode",
           "stats_mode", "set_tile_table", "tile_table", "fused_deslice_slice",
           "fused_coupling", "fused_slice_varlen", "fused_deslice_varlen"]
