"""The C ABI library (CPU-only checks: no kernel is launched).

* the in-tree library loads and exports every entry point that the headers
  in ``include/`` declare;
* argument validation happens before any launch and reports through
  ``fs_last_error`` (these calls never reach the GPU);
* workspace sizing and family routing are pure functions of the shape.
"""

import ctypes
import os
import re

import pytest
import torch

from flashslice_amd.kernels import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("flashslice_hip.h", "flashslice_layer.h")]


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"\b(fs_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    names = _declared()
    assert set(names) == set(_hip.EXPORTS), names
    for n in names:
        assert hasattr(lib, n), n
    assert b"gfx950" in lib.fs_version()


def test_nm_lists_the_symbols():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _hip.LIB_PATH],
                         capture_output=True, text=True).stdout
    for n in _declared():
        assert re.search(r"\bT %s$" % n, out, re.M), n


def _params(B=1, N=100, H=2, D=32, DV=32, G=32, dot=0):
    w = torch.zeros(G, D)
    b = torch.zeros(G)
    tau = torch.ones(H)
    p = _hip.FsSliceParams(B, N, H, D, DV, G, w.data_ptr(), 0, 0, b.data_ptr(), 0, 0,
                           tau.data_ptr(), dot, 0)
    return p, (w, b, tau)


def test_validation_before_launch():
    lib = _hip.lib()
    p, keep = _params()
    x = _hip.FsPoints(None, 0, 0, 0, 0, 32)
    rc = lib.fs_slice_fwd(ctypes.byref(x), ctypes.byref(x), ctypes.byref(p), None, None,
                          None, None, None, 0, None)
    assert rc == _hip.FS_ERR_INVALID
    assert b"x_mid is NULL" in lib.fs_last_error()
    bad, keep2 = _params(D=300)
    rc = lib.fs_deslice_fwd(ctypes.byref(x), ctypes.byref(bad), None, None, None,
                            ctypes.byref(x), None, 0, None)
    assert rc == _hip.FS_ERR_INVALID and b"[1, 256]" in lib.fs_last_error()
    bad, keep3 = _params(G=0)
    rc = lib.fs_slice_bwd(ctypes.byref(x), ctypes.byref(x), ctypes.byref(bad), None, None,
                          None, ctypes.byref(x), ctypes.byref(x), None, None, None, None, 0,
                          None)
    assert rc == _hip.FS_ERR_INVALID and b"G must be" in lib.fs_last_error()
    bad, keep4 = _params(dot=7)
    rc = lib.fs_deslice_bwd(ctypes.byref(x), ctypes.byref(bad), None, None, ctypes.byref(x),
                            ctypes.byref(x), None, None, None, None, None, 0, None)
    assert rc == _hip.FS_ERR_INVALID and b"dot level" in lib.fs_last_error()


def test_dtype_and_width_mismatch_rejected():
    lib = _hip.lib()
    p, keep = _params()
    buf = torch.zeros(16)
    x = _hip.FsPoints(buf.data_ptr(), 0, 0, 0, 0, 32)
    fx = _hip.FsPoints(buf.data_ptr(), 0, 0, 0, 1, 32)
    z = ctypes.c_void_p(buf.data_ptr())
    rc = lib.fs_slice_fwd(ctypes.byref(x), ctypes.byref(fx), ctypes.byref(p), None, None, z, z,
                          None, 0, None)
    assert rc == _hip.FS_ERR_INVALID and b"dtypes differ" in lib.fs_last_error()
    fx = _hip.FsPoints(buf.data_ptr(), 0, 0, 0, 0, 31)
    rc = lib.fs_slice_fwd(ctypes.byref(x), ctypes.byref(fx), ctypes.byref(p), None, None, z, z,
                          None, 0, None)
    assert rc == _hip.FS_ERR_INVALID and b"width 31" in lib.fs_last_error()


def test_workspace_too_small_rejected():
    lib = _hip.lib()
    p, keep = _params(N=4096)
    need = lib.fs_workspace_bytes(_hip.OP_SLICE_FWD, ctypes.byref(p))
    assert need > 0
    buf = torch.zeros(16)
    x = _hip.FsPoints(buf.data_ptr(), 0, 0, 0, 0, 32)
    z = ctypes.c_void_p(buf.data_ptr())
    rc = lib.fs_slice_fwd(ctypes.byref(x), ctypes.byref(x), ctypes.byref(p), None, None, z, z,
                          z, need - 4, None)
    assert rc == _hip.FS_ERR_WORKSPACE and b"workspace" in lib.fs_last_error()


@pytest.mark.parametrize("N,B,H,G,DV", [(4096, 1, 8, 32, 32), (1_000_000, 1, 8, 32, 32),
                                        (262144, 4, 8, 64, 64), (17, 2, 4, 256, 32)])
def test_workspace_is_a_function_of_the_shape(N, B, H, G, DV):
    lib = _hip.lib()
    p, keep = _params(B=B, N=N, H=H, G=G, DV=DV)
    a = lib.fs_workspace_bytes(_hip.OP_SLICE_BWD, ctypes.byref(p))
    b = lib.fs_workspace_bytes(_hip.OP_SLICE_BWD, ctypes.byref(p))
    assert a == b and a % 4 == 0
    # deslice forward: nothing on the whole-G family; the prepared operand
    # fragments (O(B H G (D + DV))) on the G-blocked one
    d = lib.fs_workspace_bytes(_hip.OP_DESLICE_FWD, ctypes.byref(p))
    if lib.fs_family(ctypes.byref(p)) == 1:
        assert d == 0
    else:
        assert 0 < d <= B * H * ((G + 31) // 32) * 64 * 1024
    # partials are O(B H P G (D+1)), far below the N x H x G tensor at scale
    if N >= 262144:
        assert a < B * N * H * G * 4 / 10


def test_family_routing():
    lib = _hip.lib()
    for (D, DV, G), fam in (((32, 32, 32), 1), ((32, 64, 64), 1), ((32, 32, 128), 1),
                            ((32, 32, 256), 2), ((32, 32, 1024), 2), ((256, 32, 32), 2)):
        p, keep = _params(D=D, DV=DV, G=G)
        assert lib.fs_family(ctypes.byref(p)) == fam, (D, DV, G)


def test_layernorm_validation_before_launch():
    """The layer's LayerNorm entry points (include/flashslice_layer.h):
    workspace sizing is a function of the shape, and bad shapes or pointers
    are refused before any launch."""
    lib = _hip.lib()
    assert lib.fs_layernorm_workspace_bytes(2_000_000, 256) > 0
    assert lib.fs_layernorm_workspace_bytes(2_000_000, 258) == 0
    assert lib.fs_layernorm_workspace_bytes(0, 256) == 0
    assert lib.fs_layernorm_workspace_bytes(10, 4096) == 0
    V = ctypes.c_void_p
    p = V(4096)  # never dereferenced: validation fails first
    rc = lib.fs_layernorm_fwd(p, p, p, p, p, p, 100, 6, 1e-5, None)
    assert rc == _hip.FS_ERR_INVALID and b"multiple of 4" in lib.fs_last_error()
    rc = lib.fs_layernorm_fwd(p, None, p, p, p, p, 100, 256, 1e-5, None)
    assert rc == _hip.FS_ERR_INVALID and b"NULL" in lib.fs_last_error()
    rc = lib.fs_layernorm_fwd(V(4100), p, p, p, p, p, 100, 256, 1e-5, None)
    assert rc == _hip.FS_ERR_INVALID and b"aligned" in lib.fs_last_error()
    rc = lib.fs_layernorm_bwd(p, p, p, p, p, p, p, p, p, 0, 100, 256, None)
    assert rc == _hip.FS_ERR_WORKSPACE


def _pts(t, width):
    return _hip.FsPoints(t.data_ptr(), 0, width, width, 0, width)


def test_tied_and_row_splits_refused_before_launch():
    """fs_tied_bwd serves the whole-G family only; row splits need their
    total rows, and are served with statistics and by the G-blocked family.
    All of it is decided before a launch (the host buffers passed here are
    never touched)."""
    lib = _hip.lib()
    buf = torch.zeros(64)
    x = _pts(buf, 32)
    p, keep = _params()
    p.family = 2
    rc = lib.fs_tied_bwd(ctypes.byref(x), ctypes.byref(x), ctypes.byref(x), ctypes.byref(p),
                         *([ctypes.c_void_p(buf.data_ptr())] * 3), ctypes.byref(x), ctypes.byref(x),
                         *([ctypes.c_void_p(buf.data_ptr())] * 4), None, 0, None)
    assert rc == _hip.FS_ERR_UNSUPPORTED and b"whole-G kernels only" in lib.fs_last_error()
    assert lib.fs_workspace_bytes(_hip.OP_TIED_BWD, ctypes.byref(p)) == 0
    splits = torch.tensor([0, 60, 100], dtype=torch.int64)
    p, keep = _params(B=2)
    p.row_splits = splits.data_ptr()
    # the rows of the point tensors bound the device-side clamp of the splits
    rc = lib.fs_deslice_fwd(ctypes.byref(x), ctypes.byref(p), ctypes.c_void_p(buf.data_ptr()),
                            None, None, ctypes.byref(x), None, 0, None)
    assert rc == _hip.FS_ERR_INVALID and b"total_rows" in lib.fs_last_error()
    p.total_rows = 100
    # row splits are served with statistics and by the G-blocked family: these
    # calls pass validation and stop at the (missing) workspace
    rc = lib.fs_slice_fwd(ctypes.byref(x), ctypes.byref(x), ctypes.byref(p), None,
                          ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(buf.data_ptr()),
                          ctypes.c_void_p(buf.data_ptr()), None, 0, None)
    assert rc == _hip.FS_ERR_WORKSPACE
    p.family = 2
    rc = lib.fs_compute_stats(ctypes.byref(x), ctypes.byref(p), ctypes.c_void_p(buf.data_ptr()),
                              0, None, 0, None)
    assert rc == _hip.FS_ERR_WORKSPACE
    rc = lib.fs_deslice_fwd(ctypes.byref(x), ctypes.byref(p), ctypes.c_void_p(buf.data_ptr()),
                            None, None, ctypes.byref(x), None, 0, None)
    assert rc == _hip.FS_ERR_WORKSPACE
    # a ragged batch's per-point buffers are sized by its total rows, H planes
    nws = lib.fs_workspace_bytes(_hip.OP_DESLICE_BWD, ctypes.byref(p))
    p.total_rows = 100_000
    assert lib.fs_workspace_bytes(_hip.OP_DESLICE_BWD, ctypes.byref(p)) > nws + 3 * 2 * 99_900 * 4
