"""The reference's import lines resolve unchanged (CPU).

Each statement below is one the reference's README or tests write
(reference README.md:78-103; flashslice/__init__.py:8-15; tests/test_dims.py:21-24;
bench/parity_ops.py:35-42), run verbatim in a fresh interpreter, so that the
``flashslice`` names are found through ``import`` alone.
"""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

REFERENCE_LINES = """
import torch
from flashslice import Transolver
from flashslice.kernels import fused_slice, fused_deslice
from flashslice.kernels import fused_slice, fused_deslice, unsupported_dims
from flashslice.kernels import unsupported_dims, single_tile_dims
from flashslice.kernels import set_kernel_mode, single_tile_dims
from flashslice.kernels import set_tile_table, tile_table
from flashslice.kernels import slice_ops as fs
from flashslice.kernels import blocked as fb
from flashslice.kernels.blocked import compute_stats
from flashslice.kernels.blocked import tiles
from flashslice.layers import Physics_Attention_Irregular_Mesh
from flashslice.layers.physics_attention import Physics_Attention_Irregular_Mesh
from flashslice.models.transolver import Transolver, TransolverBlock, TokenTransformerBlock
from flashslice.models import Transolver
"""

CHECKS = """
import flashslice, flashslice_amd
assert Transolver is flashslice_amd.models.Transolver is flashslice.Transolver
assert fs is flashslice_amd.kernels.slice_ops and fb is flashslice_amd.kernels.blocked
assert fused_slice is flashslice_amd.kernels.fused_slice
# one process-wide state through either name
fs.set_dot_mode("tf32")
assert flashslice_amd.kernels.slice_ops._DOT_ENV == "tf32"
fs.set_dot_mode("")
assert hasattr(torch.ops.flashslice, "flash_slice") and hasattr(torch.ops.flashslice, "slice_blk")
assert unsupported_dims(300, 32) is not None and single_tile_dims(32, 32)
assert tiles(32, 32) == fb.tiles(32, 32)
# the README's model (its fused route needs the GPU; the eager route runs here)
Transolver(space_dim=3, fun_dim=1, out_dim=4, n_hidden=64, n_heads=4, n_layers=1,
           slice_num=8, use_fused_slice=True)
model = Transolver(space_dim=3, fun_dim=1, out_dim=4, n_hidden=64, n_heads=4, n_layers=1,
                   slice_num=8)
x = torch.randn(1, 50, 3)
fx = torch.randn(1, 50, 1)
y = model(x, fx)
assert y.shape == (1, 50, 4)
print("IMPORTS_OK")
"""


def test_reference_import_lines_resolve():
    env = dict(os.environ, PYTHONPATH=ROOT + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", REFERENCE_LINES + CHECKS], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "IMPORTS_OK" in r.stdout, r.stderr[-3000:]
