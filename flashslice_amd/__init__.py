"""flashslice_amd: FlashSlice's fused slice/deslice operators for AMD MI355X.

    from flashslice_amd.kernels import fused_slice, fused_deslice

The operators keep the reference's ``flashslice.kernels`` API and
``torch.ops.flashslice`` custom-operator boundary; underneath they run
hand-written HIP kernels for gfx950 (``flashslice_amd/csrc``), built in-tree
into ``flashslice_amd/_lib/libflashslice_hip.so`` by
``python -m flashslice_amd.build``.
"""

__version__ = "0.1.0"
