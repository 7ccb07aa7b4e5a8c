"""fs_slice_fwd_static -- the slice forward that allocates nothing -- against
fs_slice_fwd with a caller-owned workspace, through the C ABI (GPU).

The static entry point keeps its partials in the library's per-GPU scratch
array, which holds the previous call's contents: two calls in a row (the
second on a smaller input) must each equal the workspace entry point
bitwise. Shapes whose workspace exceeds the array are refused before any
launch.
"""

import ctypes

import pytest
import torch

from flashslice_amd.kernels import _hip

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _inputs(B, N, H, D, DV, G, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, H, D, generator=g).cuda()
    fx = torch.randn(B, N, H, DV, generator=g).cuda()
    w = (torch.randn(H, G, D, generator=g) / D ** 0.5).cuda()
    b = (0.02 * torch.randn(H, G, generator=g)).cuda()
    tau = (0.3 + 0.7 * torch.rand(H, generator=g)).cuda()
    return x, fx, w, b, tau


def _params(x, fx, w, b, tau, family):
    B, N, H, D = x.shape
    G = w.shape[-2]
    return _hip.FsSliceParams(B, N, H, D, fx.shape[3], G, w.data_ptr(), 0, G * D,
                              b.data_ptr(), 0, G, tau.data_ptr(), 0, family, None, 0)


def _run(static, x, fx, w, b, tau, family, want_stats):
    lib = _hip.lib()
    B, N, H, D = x.shape
    DV, G = fx.shape[3], w.shape[-2]
    p = _params(x, fx, w, b, tau, family)
    z = torch.full((B, H, G, DV), float("nan"), device="cuda")
    s = torch.full((B, H, G), float("nan"), device="cuda")
    st = torch.full((B, H, 2, N), float("nan"), device="cuda") if want_stats else None
    px, pf = _hip.points(x, D), _hip.points(fx, DV)
    stream = _hip.stream_of(x.device)
    if static:
        rc = lib.fs_slice_fwd_static(ctypes.byref(px), ctypes.byref(pf), ctypes.byref(p), None,
                                     _hip.ptr(st), _hip.ptr(z), _hip.ptr(s), stream)
    else:
        nws = lib.fs_workspace_bytes(_hip.OP_SLICE_FWD, ctypes.byref(p))
        ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
        rc = lib.fs_slice_fwd(ctypes.byref(px), ctypes.byref(pf), ctypes.byref(p), None,
                              _hip.ptr(st), _hip.ptr(z), _hip.ptr(s), _hip.ptr(ws), nws, stream)
    _hip.check(rc)
    torch.cuda.synchronize()
    return z, s, st


# (B, N, H, D, DV, G, family): each pair is called larger first, then smaller
PAIRS = {
    "whole-g": [(1, 200_000, 8, 32, 32, 32, 0), (1, 3001, 8, 32, 32, 32, 0)],
    "whole-g-c4-shape": [(2, 40_000, 8, 32, 64, 64, 0), (1, 777, 8, 32, 64, 64, 0)],
    "g-blocked": [(1, 4000, 2, 32, 32, 256, 0), (1, 1025, 2, 32, 32, 256, 0)],
    "g-blocked-forced": [(1, 30_000, 4, 32, 32, 32, 2), (1, 517, 4, 32, 32, 32, 2)],
}


@pytest.mark.parametrize("name", list(PAIRS))
def test_static_matches_workspace_entry_point(name):
    for i, (B, N, H, D, DV, G, family) in enumerate(PAIRS[name]):
        print("[no-alloc] %s call %d: B=%d N=%d H=%d D=%d DV=%d G=%d family=%d"
              % (name, i, B, N, H, D, DV, G, family), flush=True)
        inp = _inputs(B, N, H, D, DV, G, seed=10 + i)
        lib = _hip.lib()
        need = lib.fs_workspace_bytes(_hip.OP_SLICE_FWD, ctypes.byref(_params(*inp, family)))
        assert 0 < need <= SCRATCH_BYTES, need
        want_stats = family == 2 or G > 128
        ref = _run(False, *inp, family, want_stats)
        got = _run(True, *inp, family, want_stats)
        for r, g_ in zip(ref, got):
            if r is None:
                continue
            assert torch.isfinite(r).all()
            assert torch.equal(r, g_)


def test_static_refuses_shapes_beyond_its_scratch():
    """A shape whose workspace exceeds the static array: FS_ERR_WORKSPACE
    before any launch (the host pointers below are never touched)."""
    lib = _hip.lib()
    B, N, H, D, G = 1, 1_000_000, 8, 32, 256
    w, b, tau = torch.zeros(H, G, D), torch.zeros(H, G), torch.ones(H)
    p = _hip.FsSliceParams(B, N, H, D, D, G, w.data_ptr(), 0, G * D, b.data_ptr(), 0, G,
                           tau.data_ptr(), 0, 0, None, 0)
    need = lib.fs_workspace_bytes(_hip.OP_SLICE_FWD, ctypes.byref(p))
    assert need > SCRATCH_BYTES
    buf = torch.zeros(64)
    x = _hip.FsPoints(buf.data_ptr(), 0, H * D, D, 0, D)
    rc = lib.fs_slice_fwd_static(ctypes.byref(x), ctypes.byref(x), ctypes.byref(p), None, None,
                                 ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(buf.data_ptr()),
                                 None)
    assert rc == _hip.FS_ERR_WORKSPACE
    assert b"static buffer" in lib.fs_last_error()
