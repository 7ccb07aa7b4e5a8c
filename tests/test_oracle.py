"""Pins the CPU oracle (``oracle/eager.py``) without trusting its formulas.

Each check is chosen so that a plausible mistake in the restatement -- a
dropped bias, the bias after the temperature instead of before, a wrong
sign on the temperature gradient, a transposed einsum, a missing sum over a
shared axis -- fails at least one of them:

* the backward closed forms against float64 autograd of the forward
  restatement and against finite differences (``gradcheck``);
* forward special cases with known answers (W = 0, D = 1, G = 1, tau -> inf,
  constant tokens) and invariants (sum_g s = N, shift of the bias,
  (W, b, tau) scaling, point and slot permutations);
* a pure-Python brute-force loop at N = 17 written from the definition;
* the shared-parameter reduction against autograd through a broadcast leaf.
"""

import math

import pytest
import torch

import oracle


@pytest.fixture(autouse=True)
def _float64_default():
    """Every tensor these checks create without a dtype is float64; the
    process-wide default is restored afterwards for the other test files."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(B=2, N=17, H=3, D=5, DV=4, G=6, wmode="hgd", bias=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    x, fx = r(B, N, H, D), r(B, N, H, DV)
    W = {"gd": r(G, D), "hgd": r(H, G, D), "bhgd": r(B, H, G, D)}[wmode] / math.sqrt(D)
    b = None
    if bias:
        b = {"gd": r(G), "hgd": r(H, G), "bhgd": r(B, H, G)}[wmode] * 0.3
    tau = 0.3 + torch.rand(H, generator=g, dtype=torch.float64) * 0.7
    tok = r(B, H, G, DV)
    return x, fx, W, b, tau, tok


# --------------------------------------------------------------------------- forward
def test_logits_bias_before_tau_closed_form():
    x, fx, W, b, tau, tok = _inputs(wmode="hgd")
    Wz = torch.zeros_like(W)
    L = oracle.logits(x, Wz, b, tau)
    want = (b / tau[:, None])[None, :, None, :].expand_as(L)
    assert torch.allclose(L, want)
    w = oracle.membership(x, Wz, b, tau)
    assert torch.allclose(w, torch.softmax(want, -1))


def test_logits_d1_by_hand():
    x = torch.tensor([[[[2.0]], [[-1.0]]]])          # B=1, N=2, H=1, D=1
    W = torch.tensor([[1.5], [0.5], [-2.0]])         # G=3, D=1
    b = torch.tensor([0.1, -0.2, 0.3])
    tau = torch.tensor([0.5])
    L = oracle.logits(x, W, b, tau)
    want = torch.tensor([[[[ (3.0 + 0.1) / 0.5, (1.0 - 0.2) / 0.5, (-4.0 + 0.3) / 0.5],
                           [(-1.5 + 0.1) / 0.5, (-0.5 - 0.2) / 0.5, (2.0 + 0.3) / 0.5]]]])
    assert torch.allclose(L, want)


def test_brute_force_loop_n17():
    x, fx, W, b, tau, tok = _inputs(B=1, N=17, H=2, D=3, DV=2, G=4, wmode="bhgd")
    z, s = oracle.slice_fwd(x, fx, W, b, tau)
    out = oracle.deslice_fwd(x, W, b, tau, tok)
    B, N, H, D = x.shape
    G, DV = W.shape[-2], fx.shape[-1]
    for bb in range(B):
        for h in range(H):
            zz = [[0.0] * DV for _ in range(G)]
            ss = [0.0] * G
            for n in range(N):
                lg = []
                for g in range(G):
                    a = sum(float(x[bb, n, h, d]) * float(W[bb, h, g, d]) for d in range(D))
                    lg.append((a + float(b[bb, h, g])) / float(tau[h]))
                mx = max(lg)
                ex = [math.exp(v - mx) for v in lg]
                tot = sum(ex)
                wv = [e / tot for e in ex]
                for g in range(G):
                    ss[g] += wv[g]
                    for v in range(DV):
                        zz[g][v] += wv[g] * float(fx[bb, n, h, v])
                for v in range(DV):
                    o = sum(wv[g] * float(tok[bb, h, g, v]) for g in range(G))
                    assert abs(o - float(out[bb, n, h, v])) < 1e-12
            assert torch.allclose(z[bb, h], torch.tensor(zz), atol=1e-12)
            assert torch.allclose(s[bb, h], torch.tensor(ss), atol=1e-12)


def test_slice_sums_to_n_and_g1():
    x, fx, W, b, tau, tok = _inputs(G=7)
    z, s = oracle.slice_fwd(x, fx, W, b, tau)
    assert torch.allclose(s.sum(-1), torch.full_like(s.sum(-1), x.shape[1]))
    x, fx, W, b, tau, tok = _inputs(G=1)
    z, s = oracle.slice_fwd(x, fx, W, b, tau)
    assert torch.allclose(s, torch.full_like(s, x.shape[1]))
    assert torch.allclose(z[:, :, 0, :], fx.sum(1))
    out = oracle.deslice_fwd(x, W, b, tau, tok)
    assert torch.allclose(out, tok[:, :, 0, :][:, None].expand_as(out))


def test_invariances():
    x, fx, W, b, tau, tok = _inputs(wmode="hgd")
    w0 = oracle.membership(x, W, b, tau)
    # a uniform shift of the bias along g leaves w unchanged
    assert torch.allclose(oracle.membership(x, W, b + 1.7, tau), w0)
    # (W, b, tau) -> (cW, cb, c tau) leaves w unchanged
    assert torch.allclose(oracle.membership(x, 2.5 * W, 2.5 * b, 2.5 * tau), w0)
    # tau -> inf: uniform weights
    wu = oracle.membership(x, W, b, torch.full_like(tau, 1e12))
    assert torch.allclose(wu, torch.full_like(wu, 1.0 / W.shape[-2]))
    # constant tokens give a constant out
    c = torch.randn(x.shape[0], x.shape[2], 1, tok.shape[-1])
    out = oracle.deslice_fwd(x, W, b, tau, c.expand_as(tok))
    assert torch.allclose(out, c[:, :, 0, :][:, None].expand_as(out))


def test_permutations():
    x, fx, W, b, tau, tok = _inputs(wmode="bhgd")
    perm = torch.randperm(x.shape[1], generator=torch.Generator().manual_seed(3))
    z, s = oracle.slice_fwd(x, fx, W, b, tau)
    zp, sp = oracle.slice_fwd(x[:, perm], fx[:, perm], W, b, tau)
    assert torch.allclose(z, zp) and torch.allclose(s, sp)
    out = oracle.deslice_fwd(x, W, b, tau, tok)
    assert torch.allclose(oracle.deslice_fwd(x[:, perm], W, b, tau, tok), out[:, perm])
    gp = torch.randperm(W.shape[-2], generator=torch.Generator().manual_seed(4))
    z2, s2 = oracle.slice_fwd(x, fx, W[:, :, gp], b[:, :, gp], tau)
    assert torch.allclose(z2, z[:, :, gp]) and torch.allclose(s2, s[:, :, gp])
    out2 = oracle.deslice_fwd(x, W[:, :, gp], b[:, :, gp], tau, tok[:, :, gp])
    assert torch.allclose(out2, out)


def test_stats():
    x, fx, W, b, tau, tok = _inputs(G=9)
    st = oracle.stats(x, W, b, tau)
    L = oracle.logits(x, W, b, tau)
    w = oracle.membership(x, W, b, tau)
    m, l = st[:, :, 0], st[:, :, 1]
    assert torch.equal(m, L.max(-1).values)
    assert torch.allclose(torch.exp(L - m[..., None]) / l[..., None], w)
    # the online (rescaling) form of l equals the two-pass form
    B, H, N, G = L.shape
    mo = torch.full((B, H, N), -math.inf)
    lo = torch.zeros(B, H, N)
    for g0 in range(0, G, 4):
        blk = L[..., g0:g0 + 4]
        mn = torch.maximum(mo, blk.max(-1).values)
        lo = lo * torch.exp(mo - mn) + torch.exp(blk - mn[..., None]).sum(-1)
        mo = mn
    assert torch.equal(mo, m) and torch.allclose(lo, l)


# --------------------------------------------------------------------------- backward
@pytest.mark.parametrize("wmode,bias", [("gd", True), ("hgd", True), ("bhgd", True),
                                        ("gd", False), ("bhgd", False)])
def test_backward_closed_forms_match_autograd(wmode, bias):
    x, fx, W, b, tau, tok = _inputs(wmode=wmode, bias=bias)
    g = torch.Generator().manual_seed(11)
    dz = torch.randn(x.shape[0], x.shape[2], W.shape[-2], fx.shape[-1], generator=g)
    ds = torch.randn(x.shape[0], x.shape[2], W.shape[-2], generator=g)
    do = torch.randn(*fx.shape, generator=g)
    leaves = [t.clone().requires_grad_(True) for t in (x, fx, W, tau, tok)]
    bl = None if b is None else b.clone().requires_grad_(True)
    xl, fl, Wl, tl, kl = leaves
    # autograd through an independent float64 softmax/einsum chain
    B, N, H, D = x.shape
    w4 = Wl.reshape((1,) * (4 - Wl.dim()) + tuple(Wl.shape)).expand(B, H, -1, -1)
    a = torch.einsum("bnhd,bhgd->bhng", xl, w4)
    if bl is not None:
        a = a + bl.reshape((1,) * (3 - bl.dim()) + tuple(bl.shape))[:, :, None, :]
    w = torch.softmax(a / tl.view(1, H, 1, 1), -1)
    z = torch.einsum("bhng,bnhv->bhgv", w, fl)
    s = w.sum(2)
    loss = (z * dz).sum() + (s * ds).sum()
    grads = torch.autograd.grad(loss, [xl, fl, Wl, tl] + ([bl] if bl is not None else []),
                                retain_graph=True)
    dx, dfx, dW, db, dtau = oracle.slice_bwd(x, fx, W, b, tau, dz, ds)
    assert torch.allclose(dx, grads[0]) and torch.allclose(dfx, grads[1])
    assert torch.allclose(dW, grads[2]) and torch.allclose(dtau, grads[3])
    if b is not None:
        assert torch.allclose(db, grads[4])
    out = torch.einsum("bhgv,bhng->bnhv", kl, w)
    grads = torch.autograd.grad((out * do).sum(), [xl, Wl, tl, kl] + ([bl] if bl is not None else []))
    dx, dtok, dW, db, dtau = oracle.deslice_bwd(x, W, b, tau, tok, do)
    assert torch.allclose(dx, grads[0]) and torch.allclose(dW, grads[1])
    assert torch.allclose(dtau, grads[2]) and torch.allclose(dtok, grads[3])
    if b is not None:
        assert torch.allclose(db, grads[4])


def test_backward_gradcheck_finite_differences():
    x, fx, W, b, tau, tok = _inputs(B=1, N=5, H=2, D=3, DV=2, G=4, wmode="hgd")
    g = torch.Generator().manual_seed(5)
    dz = torch.randn(1, 2, 4, 2, generator=g)
    ds = torch.randn(1, 2, 4, generator=g)
    do = torch.randn(*fx.shape, generator=g)

    # finite differences of the forward restatement pin the closed form
    def f_slice(x_, fx_, W_, b_, tau_):
        z, s = oracle.slice_fwd(x_, fx_, W_, b_, tau_)
        return (z * dz).sum() + (s * ds).sum()

    def f_deslice(x_, W_, b_, tau_, tok_):
        return (oracle.deslice_fwd(x_, W_, b_, tau_, tok_) * do).sum()

    args = [t.clone().requires_grad_(True) for t in (x, fx, W, b, tau)]
    assert torch.autograd.gradcheck(f_slice, args)
    eps = 1e-6
    dx, dfx, dW, db, dtau = oracle.slice_bwd(x, fx, W, b, tau, dz, ds)
    # one-sided spot checks of the closed form against central differences
    for t, gt, idx in ((x, dx, (0, 3, 1, 2)), (W, dW, (1, 2, 0)), (tau, dtau, (1,)),
                       (b, db, (0, 3))):
        tp, tm = t.clone(), t.clone()
        tp[idx] += eps
        tm[idx] -= eps
        kw = {id(x): 0, id(W): 2, id(b): 3, id(tau): 4}[id(t)]
        ap = [x, fx, W, b, tau]
        am = [x, fx, W, b, tau]
        ap[kw], am[kw] = tp, tm
        fd = (f_slice(*ap) - f_slice(*am)) / (2 * eps)
        assert abs(float(fd) - float(gt[idx])) < 1e-6
    args = [t.clone().requires_grad_(True) for t in (x, W, b, tau, tok)]
    assert torch.autograd.gradcheck(f_deslice, args)


def test_jacobian_rows_sum_to_zero_and_g1():
    x, fx, W, b, tau, tok = _inputs(wmode="hgd", G=8)
    g = torch.Generator().manual_seed(2)
    dz = torch.randn(x.shape[0], x.shape[2], 8, fx.shape[-1], generator=g)
    ds = torch.randn(x.shape[0], x.shape[2], 8, generator=g)
    dx, dfx, dW, db, dtau = oracle.slice_bwd(x, fx, W, b, tau, dz, ds)
    assert torch.allclose(db.sum(-1), torch.zeros(x.shape[2]), atol=1e-12)
    assert torch.allclose(dW.sum(-2), torch.zeros(x.shape[2], x.shape[3]), atol=1e-12)
    # G = 1: the softmax is constant, every logits-side gradient vanishes
    x, fx, W, b, tau, tok = _inputs(wmode="hgd", G=1)
    dz = torch.randn(x.shape[0], x.shape[2], 1, fx.shape[-1], generator=g)
    ds = torch.randn(x.shape[0], x.shape[2], 1, generator=g)
    dx, dfx, dW, db, dtau = oracle.slice_bwd(x, fx, W, b, tau, dz, ds)
    for t in (dx, dW, db, dtau):
        assert torch.allclose(t, torch.zeros_like(t), atol=1e-12)
    assert torch.allclose(dfx, dz[:, :, 0, :][:, None].expand_as(dfx))


@pytest.mark.parametrize("wmode", ["gd", "hgd", "bhgd"])
def test_reduce_param_grad_matches_broadcast_leaf(wmode):
    x, fx, W, b, tau, tok = _inputs(wmode=wmode)
    do = torch.randn(*fx.shape)
    Wl, bl = W.clone().requires_grad_(True), b.clone().requires_grad_(True)
    out = oracle.deslice_fwd(x, Wl, bl, tau, tok)
    gW, gb = torch.autograd.grad((out * do).sum(), [Wl, bl])
    _, _, dW, db, _ = oracle.deslice_bwd(x, W, b, tau, tok, do)
    assert dW.shape == W.shape and db.shape == b.shape
    assert torch.allclose(dW, gW) and torch.allclose(db, gb)


def test_coupling_orders():
    x, fx, W, b, tau, tok = _inputs(wmode="hgd", DV=4)
    tm = torch.randn(4, 4)
    out, z, s = oracle.coupling(x, fx, W, b, tau, tm=tm, order="slice-first")
    z2, s2 = oracle.slice_fwd(x, fx, W, b, tau)
    tk = (z2 / (s2 + oracle.EPS_TOKEN)[..., None]) @ tm
    assert torch.allclose(out, oracle.deslice_fwd(x, W, b, tau, tk))
    out, z, s = oracle.coupling(x, fx, W, b, tau, tokens=tok, order="deslice-first")
    assert torch.allclose(out, oracle.deslice_fwd(x, W, b, tau, tok))
    assert torch.allclose(z, z2) and torch.allclose(s, s2)
