"""Error paths of the operators on the GPU: every refusal happens on the host,
before any launch (reference: every shape, layout or mode error is a
``ValueError`` raised before the Triton launch, slice_ops.py:503-526).

A tensor on the wrong device would reach the kernels as a host pointer, so
the operators refuse it; ragged row splits that do not describe the point
tensors (device splits are never read on the host) are clamped by the
kernels to the tensors' rows, so they give wrong sums but stay in bounds.
"""

import pytest
import torch

from flashslice_amd.kernels import (fused_deslice, fused_deslice_slice, fused_deslice_varlen,
                                    fused_slice, fused_slice_varlen)

pytestmark = pytest.mark.gpu


def _inputs(G=32, N=257, H=4, D=32):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, N, H, D, generator=g).cuda()
    fx = torch.randn(1, N, H, D, generator=g).cuda()
    w = (torch.randn(H, G, D, generator=g) / D ** 0.5).cuda()
    b = (0.02 * torch.randn(H, G, generator=g)).cuda()
    tau = (0.3 + 0.7 * torch.rand(H, generator=g)).cuda()
    tok = torch.randn(1, H, G, D, generator=g).cuda()
    return x, fx, w, b, tau, tok


@pytest.mark.parametrize("G", [32, 256], ids=["whole-g", "g-blocked"])
def test_host_tensors_refused(G):
    x, fx, w, b, tau, tok = _inputs(G)
    cases = {
        "tau": lambda: fused_slice(x, fx, w, b, tau.cpu()),
        "weight": lambda: fused_slice(x, fx, w.cpu(), b, tau),
        "bias": lambda: fused_deslice(x, w, b.cpu(), tau, tok),
        "fx_mid": lambda: fused_slice(x, fx.cpu(), w, b, tau),
        "tokens": lambda: fused_deslice(x, w, b, tau, tok.cpu()),
        "tied tokens": lambda: fused_deslice_slice(x, fx, w, b, tau, tok.cpu()),
    }
    for name, fn in cases.items():
        with pytest.raises(ValueError, match="device"):
            fn()
    # statistics from the host
    _, _, st = fused_slice(x, fx, w, b, tau, return_stats=True)
    if st is not None:
        with pytest.raises(ValueError, match="device"):
            fused_deslice(x, w, b, tau, tok, stats=st.cpu())
    # and a host upstream gradient in the backward
    xr = x.clone().requires_grad_(True)
    out = fused_deslice(xr, w, b, tau, tok)
    with pytest.raises(ValueError, match="device"):
        torch.ops.flashslice.flash_deslice_bwd(x, w, b, tau, tok, torch.zeros_like(out).cpu(), 0)
    torch.cuda.synchronize()
    # the library is still usable: nothing was launched with a host pointer
    z, s = fused_slice(x, fx, w, b, tau)
    torch.cuda.synchronize()
    assert torch.isfinite(z).all()


def test_malformed_device_row_splits_stay_in_bounds():
    """Device row splits are not read on the host; splits that decrease or
    run past the point tensors' rows are clamped on the device to them (and
    to max_rows per sample): the call completes and writes only its own
    outputs."""
    H, D, G = 4, 32, 32
    rows = 100
    g = torch.Generator().manual_seed(2)
    x = torch.randn(rows, H, D, generator=g).cuda()
    fx = torch.randn(rows, H, D, generator=g).cuda()
    w = (torch.randn(H, G, D, generator=g) / D ** 0.5).cuda()
    tau = torch.full((H,), 0.5).cuda()
    splits = torch.tensor([0, 50, 10, 400], dtype=torch.int64).cuda()
    z, s = fused_slice_varlen(x, fx, w, None, tau, splits, max_rows=60)
    tok = torch.randn(3, H, G, D).cuda()
    out = fused_deslice_varlen(x, w, None, tau, tok, splits, max_rows=60)
    torch.cuda.synchronize()
    assert torch.isfinite(z).all() and torch.isfinite(s).all()
    # sample 1 (rows 50 .. 10) is empty after the clamp
    assert float(s[1].abs().sum()) == 0.0
    # sample 2 covers rows 10 .. 69 (clamped to the tensors' 100 rows, then
    # to max_rows = 60 rows): every point's weights sum to one
    assert torch.allclose(s[2].sum(-1), torch.full((H,), 60.0, device="cuda"), rtol=1e-5)
    assert out.shape == (rows, H, D) and torch.isfinite(out[:70]).all()
