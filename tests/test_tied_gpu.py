"""Parity of the tied deslice -> slice operator (``fused_deslice_slice``,
one fused backward kernel ``fs_tied_bwd``) on the GPU.

Each case runs the coupling in the deslice-first order -- out from the given
tokens, then (z_num, s) from fx_mid on the same logits -- forward and
backward through the tied op, against the CPU oracle in float64 and float32
with the gates of ``tests/parity.py`` (the same as the two separate ops are
held to), and twice for bitwise determinism. The G-blocked shapes and kernel
mode "blocked" exercise the tied op's fallback (the two backward ops summed).
A further test holds the tied kernel to the two separate ops' own
gradients, at small size and at BASELINE config 4's full size.
"""

import math

import pytest
import torch

from parity import Case, check_case, relerr
from flashslice_amd.kernels import fused_deslice, fused_deslice_slice, fused_slice

pytestmark = pytest.mark.gpu


def _report(name, fails, rows):
    print("\ncase %s" % name, flush=True)
    for k, ee, ef, fe in rows:
        print("  %-10s eager %.3e  fused %.3e  fused-vs-eager %.3e" % (k, ee, ef, fe))
    assert not fails, "\n".join(fails)


CASES = [
    ("c4-shape-bhgd", dict(B=4, N=2048, H=8, D=32, DV=64, G=64, mode="bhgd"), {}),
    ("hgd-d32-g32-ragged", dict(B=2, N=3001, H=4, D=32, G=32, mode="hgd"), {}),
    ("gd-nobias", dict(B=1, N=2049, H=4, D=32, G=32, mode="gd", bias=False), {}),
    ("tiny-N17", dict(B=2, N=17, H=4, D=32, G=32, mode="hgd"), {}),
    ("one-point", dict(B=1, N=1, H=2, D=32, G=32, mode="hgd"), {}),
    ("masked-g40-d40-dv24", dict(B=2, N=1537, H=4, D=40, DV=24, G=40, mode="hgd"), {}),
    ("g128", dict(B=1, N=2049, H=2, D=32, G=128, mode="hgd"), {}),
    ("d64-dv128-g32", dict(B=1, N=1025, H=2, D=64, DV=128, G=32, mode="hgd"), {}),
    ("g8-padded", dict(B=1, N=2049, H=4, D=32, G=8, mode="hgd"), {}),
    # the fallback: G-blocked shapes and the forced blocked kernel mode
    ("fallback-g256", dict(B=1, N=2049, H=2, D=32, G=256, mode="hgd"), dict(blocked=True)),
    ("fallback-forced-blocked", dict(B=2, N=1025, H=4, D=32, DV=64, G=64, mode="bhgd"),
     dict(kernel_mode="blocked", blocked=True)),
    # 16-bit point tensors, fp32-accurate and bf16 dots
    ("bf16-inputs", dict(B=1, N=2049, H=4, D=32, DV=64, G=64, mode="hgd"),
     dict(inputs="bf16")),
    ("bf16-dots", dict(B=1, N=2049, H=4, D=32, DV=64, G=64, mode="hgd"), dict(dot="bf16")),
]


@pytest.mark.parametrize("name,kw,opts", CASES, ids=[c[0] for c in CASES])
def test_tied_parity(name, kw, opts):
    fails, rows = check_case(Case(**kw), order="tied", **opts)
    _report(name, fails, rows)


def _two_ops_vs_tied(B, N, H, D, DV, G, seed=0):
    """Gradients of one deslice-first coupling through the two ops and
    through the tied op, on the same GPU inputs."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, H, D, generator=g)
    fx = torch.randn(B, N, H, DV, generator=g)
    W = torch.randn(B, H, G, D, generator=g) / math.sqrt(D)
    b = torch.randn(B, H, G, generator=g) / math.sqrt(D)
    tau = 0.3 + 0.7 * torch.rand(H, generator=g)
    tok = torch.randn(B, H, G, DV, generator=g)
    ups = [torch.randn(B, N, H, DV, generator=g), torch.randn(B, H, G, DV, generator=g),
           torch.randn(B, H, G, generator=g)]
    dev = [t.cuda() for t in (x, fx, W, b, tau, tok)]
    ups = [u.cuda() for u in ups]
    res = []
    for tied in (False, True):
        leaves = [t.clone().requires_grad_(True) for t in dev]
        xl, fl, Wl, bl, tl, kl = leaves
        if tied:
            out, z, s = fused_deslice_slice(xl, fl, Wl, bl, tl, kl)
        else:
            out, st = fused_deslice(xl, Wl, bl, tl, kl, return_stats=True)
            z, s = fused_slice(xl, fl, Wl, bl, tl, stats=st)
        loss = (out * ups[0]).sum() + (z * ups[1]).sum() + (s * ups[2]).sum()
        loss.backward()
        res.append({"out": out.detach(), "z": z.detach(), "s": s.detach(),
                    **{"d" + n: t.grad for n, t in zip(("x", "fx", "W", "b", "tau", "tok"),
                                                        leaves)}})
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("shape", [(2, 5003, 4, 32, 64, 64), (1, 4097, 8, 32, 32, 32),
                                   (4, 262_144, 8, 32, 64, 64)],
                         ids=["small-c4-shape", "c2-shape", "c4-full"])
def test_tied_matches_two_ops(shape):
    """The tied kernel's gradients equal the two backward ops' summed ones
    up to summation order: forward outputs bitwise (the same kernels),
    gradients within 1e-5 relative (2e-5 for the cancellation sums db and
    dtau)."""
    two, tied = _two_ops_vs_tied(*shape)
    print("\nshape", shape, flush=True)
    for k in two:
        e = relerr(tied[k], two[k])
        print("  %-5s tied vs two ops %.3e" % (k, e), flush=True)
        assert tied[k].shape == two[k].shape and tied[k].dtype == two[k].dtype, k
        if k in ("out", "z", "s"):
            assert torch.equal(tied[k], two[k]), k
        else:
            assert e <= (2e-5 if k in ("db", "dtau") else 1e-5), (k, e)


def test_operand_shapes_checked_before_launch():
    """The library reads tokens, dz_num, ds, statistics and the second point
    tensors through raw pointers: every op refuses a wrong shape with a
    ValueError before anything is launched."""
    ops = torch.ops.flashslice
    B, N, H, D, G = 1, 300, 2, 32, 32
    c = lambda *s: torch.randn(*s, device="cuda")  # noqa: E731
    x, fx, W, b, tau = c(B, N, H, D), c(B, N, H, D), c(H, G, D), c(H, G), torch.ones(H).cuda()
    tok, dz, ds = c(B, H, G, D), c(B, H, G, D), c(B, H, G)
    with pytest.raises(ValueError, match="fx_mid has shape"):
        ops.flash_slice(x, c(B, N - 1, H, D), W, b, tau, 0)
    with pytest.raises(ValueError, match="tokens has shape"):
        ops.flash_deslice(x, W, b, tau, c(B, H, G - 1, D), 0)
    with pytest.raises(ValueError, match="dz_num has shape"):
        ops.flash_slice_bwd(x, fx, W, b, tau, c(B, H, G, D - 1), ds, 0)
    with pytest.raises(ValueError, match="ds has shape"):
        ops.flash_slice_bwd(x, fx, W, b, tau, dz, c(B, H), 0)
    with pytest.raises(ValueError, match="d_out has shape"):
        ops.flash_deslice_bwd(x, W, b, tau, tok, c(B, N, H + 1, D), 0)
    with pytest.raises(ValueError, match="stats has shape"):
        ops.slice_blk(x, fx, W, b, tau, c(B, H, 2, N + 5), 0)
    with pytest.raises(ValueError, match="d_out has shape"):
        ops.deslice_slice_bwd(x, fx, W, b, tau, tok, c(B, 2 * N, H, D), dz, ds, 0)
    with pytest.raises(ValueError, match="tokens has shape"):
        ops.deslice_slice_bwd(x, fx, W, b, tau, c(2, H, G, D), x, dz, ds, 0)
    torch.cuda.synchronize()
