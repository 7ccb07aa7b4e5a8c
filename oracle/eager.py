"""Eager CPU restatement of the reference slice/deslice math (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``. Nothing in the
``flashslice_amd`` package imports this module.

Notation, per sample b and head h (reference ``slice_ops.py:9-18``):

    a[n,g] = x[n].W[g] + beta[g]        L = a / tau      (bias before tau)
    w      = softmax_g(L)
    slice   z_num[g] = sum_n w[n,g] fx[n]      s[g] = sum_n w[n,g]
    deslice out[n]   = sum_g w[n,g] T[g]

Backward (reference ``slice_ops.py:679-705`` and ``:749-770``):

    slice   fx_bar = w Zb          omega[n,g] = fx[n].Zb[g] + sb[g]
    deslice T_bar  = w^T Ob        omega[n,g] = Ob[n].T[g]
    both    delta = sum_g w omega   Lb = w (omega - delta)   ab = Lb / tau
            x_bar = ab W   W_bar = ab^T x   beta_bar = sum_n ab
            tau_bar = -(1/tau) sum_n sum_g Lb L

Every function computes in the dtype of its inputs (pass float64 tensors for
the truth, float32 for "eager fp32"), exactly as the reference's eager path
does (``bench/parity_ops.py:59-79``).

How each function is pinned (tests/test_oracle.py):
  * ``logits`` / ``membership``: closed forms (W = 0 gives softmax(beta/tau);
    D = 1 by hand), a pure-Python brute-force loop at N = 17, the
    shift invariance of beta, the (W, beta, tau) -> (cW, c beta, c tau)
    invariance, tau -> inf giving 1/G, and G = 1 giving w = 1.
  * ``slice_fwd``: sum_g s[g] = N, G = 1 gives z_num = sum_n fx and s = N,
    point permutation invariance, slot permutation equivariance, a brute
    loop at N = 17.
  * ``deslice_fwd``: constant tokens give out = c, point permutation
    equivariance, G = 1 gives out = T.
  * ``stats``: m is the row max and sum_g exp(L - m) = l against the
    membership (w = exp(L - m) / l), and the online form equals the
    two-pass form.
  * ``slice_bwd`` / ``deslice_bwd``: float64 autograd of the forward
    restatement (an independent derivation of the closed forms), and
    ``torch.autograd.gradcheck`` finite differences on tiny shapes;
    sum_g beta_bar = 0 and sum_g W_bar[g] = 0 (the softmax Jacobian's
    rows sum to zero); G = 1 makes every logits-side gradient zero.
  * ``reduce_param_grad``: the shared-weight gradient equals autograd's
    gradient for a broadcast (G, D) / (H, G, D) leaf.
"""

import torch

#: the token normaliser eps of ``z_num / (s + eps)`` (reference
#: ``flashslice/layers/physics_attention.py:112``, ``bench/parity_ops.py:73``).
EPS_TOKEN = 1e-5


def _w4(weight, B, H):
    """Weight (G, D) | (H, G, D) | (B, H, G, D) broadcast to (B, H, G, D).
    Reference ``bench/parity_ops.py:60-61`` (leading dims read from the
    right: heads, then batch; ``slice_ops.py:461-478``)."""
    w = weight.reshape((1,) * (4 - weight.dim()) + tuple(weight.shape))
    return w.expand(B, H, -1, -1)


def _b3(bias, B, H, G, like):
    """Bias None | (G,) | (H, G) | (B, H, G) broadcast to (B, H, G); None is
    zeros (reference ``slice_ops.py:517-518``)."""
    if bias is None:
        return like.new_zeros(B, H, G)
    b = bias.reshape((1,) * (3 - bias.dim()) + tuple(bias.shape))
    return b.expand(B, H, G)


def logits(x, weight, bias, tau):
    """(B, H, N, G) slice logits L = (x . W + b) / tau, bias added before the
    temperature division (reference ``bench/parity_ops.py:59-65``,
    ``slice_ops.py:588-589``). x is (B, N, H, D), tau (H,)."""
    B, N, H, D = x.shape
    w4 = _w4(weight, B, H)
    a = torch.einsum("bnhd,bhgd->bhng", x, w4.to(x.dtype))
    a = a + _b3(bias, B, H, w4.shape[2], x).to(x.dtype)[:, :, None, :]
    return a / tau.to(x.dtype).view(1, H, 1, 1)


def membership(x, weight, bias, tau):
    """(B, H, N, G) slice weights w = softmax_G(L) (reference
    ``bench/parity_ops.py:59-65``)."""
    return torch.softmax(logits(x, weight, bias, tau), dim=-1)


def stats(x, weight, bias, tau):
    """(B, H, 2, N) per-point softmax statistics of the logits:
    [..., 0, :] = max_g L, [..., 1, :] = sum_g exp(L - max) (reference
    ``flashslice/kernels/blocked.py:1329-1343`` layout, ``:302-346`` math)."""
    L = logits(x, weight, bias, tau)
    m = L.max(dim=-1).values
    l = torch.exp(L - m[..., None]).sum(-1)
    return torch.stack((m, l), dim=2)


def slice_fwd(x, fx, weight, bias, tau):
    """z_num (B, H, G, DV) and s (B, H, G) (reference
    ``slice_ops.py:585-595``; eager form ``bench/parity_ops.py:67-68``)."""
    w = membership(x, weight, bias, tau)
    z_num = torch.einsum("bhng,bnhd->bhgd", w, fx.to(w.dtype))
    return z_num, w.sum(2)


def deslice_fwd(x, weight, bias, tau, tokens):
    """out (B, N, H, DV) = sum_g w[n, g] tokens[g] (reference
    ``slice_ops.py:632-637``; eager form ``bench/parity_ops.py:71``)."""
    w = membership(x, weight, bias, tau)
    return torch.einsum("bhgd,bhng->bnhd", tokens.to(w.dtype), w)


def deslice_fwd_online(x, weight, bias, tau, tokens):
    """(out, stats): the deslice together with the statistics of its own
    logits (reference ``blocked.py:513-573``, whose online pass yields both)."""
    return deslice_fwd(x, weight, bias, tau, tokens), stats(x, weight, bias, tau)


def _jacobian(x, weight, bias, tau, w, L, omega):
    """Shared softmax-Jacobian tail of both backward passes (reference
    ``slice_ops.py:698-705`` / ``:763-770``). Returns dx (B, N, H, D), the
    per-(b, h) dW4 (B, H, G, D), db3 (B, H, G), and dtau (H,) summed over b
    (``slice_ops.py:843``)."""
    B, N, H, D = x.shape
    delta = (w * omega).sum(-1, keepdim=True)
    Lb = w * (omega - delta)
    tv = tau.to(w.dtype).view(1, H, 1, 1)
    ab = Lb / tv
    w4 = _w4(weight, B, H).to(w.dtype)
    dx = torch.einsum("bhng,bhgd->bnhd", ab, w4)
    dW4 = torch.einsum("bhng,bnhd->bhgd", ab, x.to(w.dtype))
    db3 = ab.sum(2)
    dtau = -(Lb * L).sum(dim=(0, 2, 3)) / tau.to(w.dtype)
    return dx, dW4, db3, dtau


def reduce_param_grad(dW4, db3, weight_shape, bias_shape):
    """Per-(b, h) gradients summed over the axes the parameter is shared
    along, returned in the parameter's shape (reference
    ``slice_ops.py:481-500``). ``bias_shape`` None means the bias was None
    (its gradient is then the (G,) gradient of the zeros bias)."""
    dW = dW4
    if len(weight_shape) < 4:
        dW = dW.sum(0)
    if len(weight_shape) < 3:
        dW = dW.sum(0)
    db = db3
    bshape = (db3.shape[-1],) if bias_shape is None else tuple(bias_shape)
    if len(bshape) < 3:
        db = db.sum(0)
    if len(bshape) < 2:
        db = db.sum(0)
    return dW.reshape(weight_shape), db.reshape(bshape)


def slice_bwd(x, fx, weight, bias, tau, dz_num, ds):
    """(dx, dfx, dW, db, dtau) of ``slice_fwd`` given upstream dz_num
    (B, H, G, DV) and ds (B, H, G) (reference ``slice_ops.py:643-710``,
    ``:822-843``). dW/db come back in the weight's/bias's own shape."""
    L = logits(x, weight, bias, tau)
    w = torch.softmax(L, dim=-1)
    dz = dz_num.to(w.dtype)
    dfx = torch.einsum("bhng,bhgv->bnhv", w, dz)
    omega = torch.einsum("bnhv,bhgv->bhng", fx.to(w.dtype), dz) \
        + ds.to(w.dtype)[:, :, None, :]
    dx, dW4, db3, dtau = _jacobian(x, weight, bias, tau, w, L, omega)
    dW, db = reduce_param_grad(dW4, db3, tuple(weight.shape),
                               None if bias is None else tuple(bias.shape))
    return dx, dfx, dW, db, dtau


def deslice_bwd(x, weight, bias, tau, tokens, d_out):
    """(dx, dtokens, dW, db, dtau) of ``deslice_fwd`` given upstream d_out
    (B, N, H, DV) (reference ``slice_ops.py:713-776``, ``:862-885``)."""
    L = logits(x, weight, bias, tau)
    w = torch.softmax(L, dim=-1)
    do = d_out.to(w.dtype)
    dtok = torch.einsum("bhng,bnhv->bhgv", w, do)
    omega = torch.einsum("bnhv,bhgv->bhng", do, tokens.to(w.dtype))
    dx, dW4, db3, dtau = _jacobian(x, weight, bias, tau, w, L, omega)
    dW, db = reduce_param_grad(dW4, db3, tuple(weight.shape),
                               None if bias is None else tuple(bias.shape))
    return dx, dtok, dW, db, dtau


def coupling(x, fx, weight, bias, tau, tm=None, tokens=None,
             order="slice-first"):
    """One tied slice/deslice coupling in either call order (reference
    ``bench/parity_ops.py:67-79``): slice-first forms the tokens
    (z_num / (s + eps)) @ tm and deslices them; deslice-first deslices the
    given tokens, then slices. Returns (out, z_num, s)."""
    w = membership(x, weight, bias, tau)
    z_num = torch.einsum("bhng,bnhd->bhgd", w, fx.to(w.dtype))
    s = w.sum(2)
    if order == "slice-first":
        tok = z_num / (s + EPS_TOKEN)[..., None]
        if tm is not None:
            tok = tok @ tm.to(tok.dtype)
    else:
        tok = tokens
    out = torch.einsum("bhgd,bhng->bnhd", tok.to(w.dtype), w)
    return out, z_num, s


def coupling_loss(out, z_num, s, up_out, up_z, up_s):
    """The scalar the parity gates differentiate: upstream gradients
    (up_out, up_z, up_s) contracted with (out, z_num, s) (reference
    ``bench/parity_ops.py:148-151``)."""
    return ((out * up_out.to(out.dtype)).sum()
            + (z_num * up_z.to(z_num.dtype)).sum()
            + (s * up_s.to(s.dtype)).sum())
