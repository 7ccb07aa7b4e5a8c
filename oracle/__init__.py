"""CPU oracle for the fused slice/deslice path -- TEST INFRASTRUCTURE ONLY.

This package restates, on CPU tensors, the math of the reference FlashSlice
slice/deslice operators (Shizheng-Wen/flashslice v0.3.0). It exists to
*check* the HIP implementation and to time the eager CPU baseline. It is
never the thing that is measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
it. The product package ``flashslice_amd`` never imports it, and its ops
raise when the HIP library is missing instead of falling back to the CPU.

Every function cites the reference file:line it follows (paths relative to
the reference repository root). How each function is pinned (autograd,
finite differences, invariants, closed-form special cases, brute-force
loops) is listed in ``oracle/eager.py``'s module docstring.
"""

from .eager import (  # noqa: F401
    membership, logits, stats, slice_fwd, deslice_fwd, deslice_fwd_online,
    slice_bwd, deslice_bwd, reduce_param_grad, coupling, coupling_loss,
    EPS_TOKEN,
)
