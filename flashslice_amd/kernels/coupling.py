"""A slice/deslice coupling with its backward merged into one pass, in either
order and with any differentiable step between the two ops.

The reference plans this as its "tied backward fusion" (ROADMAP.md:58-65:
"In a deslice -> MLP -> slice coupling both ops share x_mid, W and the
statistics. The slice's dfx pass must run before the MLP's backward, but its
dx_mid, dW and dtau can be deferred and merged into the deslice's backward
... Needs a custom autograd node that stitches the two ops") and does not
implement it. ``fused_coupling(x_mid, W, b, tau)`` returns a handle whose
``.slice(fx_mid)`` and ``.deslice(tokens)`` are called once each, in either
order, with anything between them::

    c = fused_coupling(x_mid, W, b, tau)      # deslice -> MLP -> slice
    out = c.deslice(tokens)
    z_num, s = c.slice(mlp(out))

    c = fused_coupling(x_mid, W, b, tau)      # slice -> tokens -> deslice
    z_num, s = c.slice(fx_mid)                # (the Transolver layer's order)
    out = c.deslice(mix(z_num / (s + 1e-5)[..., None]))

Both return what ``fused_slice`` / ``fused_deslice`` return, and their
gradients equal those of the two plain ops. The backward of the op that ran
second does only what the step between them needs before it can run -- dfx
= w dz_num (deslice-first), or dtokens = w^T d_out (slice-first), each one
pass of the forward kernels -- and hands its remaining inputs to the first
op's backward, which forms both ops' dx_mid, dW, db and dtau in one pass
(``fs_tied_bwd``: one logits recompute, one softmax Jacobian over the summed
Jacobian inputs, one dx_mid / dW product). Point passes of a backward at
DV = D: deslice-first 2 + 4 = 6, slice-first 2 + 5 = 7 (the merged pass
also writes the slice's dfx), against the two ops' 3 + 4 plus autograd's 3
for summing their dx_mid. Where the whole-G kernels serve the shape the
first op forms no softmax statistics (they read none) and hands on a
zero-stride placeholder instead.

The hand-over rides on autograd itself: the first op also outputs two
"link" tensors (zero-stride, no memory) that the second op takes as inputs.
The second op's backward returns, as the links' gradients, the tensors the
first op's backward needs (fx_mid and dz_num / ds, or d_out and the
tokens), so autograd orders the two backward calls and carries the data,
and the pair stays two opaque nodes of one graph under ``torch.compile``.
If the second op never runs or gets no gradient, the first op's backward
is the plain one. Shapes the whole-G kernels do not serve (G > 128, wide D
or DV) run the two plain backward ops inside the merged node.
"""

import torch

from .slice_ops import (_LIB, _check_dims, _dot_mode, _hip_deslice_bwd, _hip_deslice_fwd,
                        _hip_slice_bwd, _hip_slice_fwd, _prep_wb, _whole_g, stats_placeholder)
from .tied import _hip_tied_bwd

_LIB.define(
    "tied_deslice(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "int dot) -> (Tensor, Tensor, Tensor, Tensor)")
_LIB.define(
    "tied_slice_after(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor stats, Tensor link_pt, Tensor link_small, int dot) -> (Tensor, Tensor)")
_LIB.define(
    "tied_deslice_bwd(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor stats, Tensor d_out, Tensor fx_mid, Tensor dz_num, Tensor ds, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_LIB.define(
    "tied_slice(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "int dot) -> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_LIB.define(
    "tied_deslice_after(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor stats, Tensor link_pt, Tensor link_tok, int dot) -> Tensor")
_LIB.define(
    "tied_slice_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor stats, Tensor dz_num, Tensor ds, Tensor d_out, Tensor tokens, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")


def _link(shape, like, dtype):
    """A zero-stride tensor of ``shape``: it carries no data, only the
    gradient autograd hands from the second op's backward to the first's."""
    return torch.empty_strided(tuple(shape), (0,) * len(shape), device=like.device, dtype=dtype)


# --------------------------------------------------------------- deslice first

def _first_stats(x_mid, weight, dv):
    """Whether the first op of a coupling forms softmax statistics for the
    second op and the backward: the G-blocked kernels need them; where the
    whole-G kernels serve the shape they hand on ``stats_placeholder``."""
    return not _whole_g(x_mid.shape[3], dv, weight.shape[-2])


def _tied_deslice_impl(x_mid, weight, bias, tau, tokens, dot):
    B, N, H, _ = x_mid.shape
    G, DV = weight.shape[-2], tokens.shape[3]
    want = _first_stats(x_mid, weight, DV)
    out, st = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot, want_stats=want)
    if not want:
        st = stats_placeholder(B, H, N, x_mid)
    return (out, st, _link((B, N, H, DV), x_mid, x_mid.dtype),
            _link((B, H, G, DV + 1), x_mid, torch.float32))


def _tied_slice_after_impl(x_mid, fx_mid, weight, bias, tau, stats, link_pt, link_small, dot):
    z_num, s, _ = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot, stats_in=stats)
    return z_num, s


def _sum_grads(a, b):
    return tuple(u + v for u, v in zip(a, b))


def _tied_deslice_bwd_impl(x_mid, weight, bias, tau, tokens, stats, d_out, fx_mid, dz_num, ds,
                           dot):
    """dx_mid, dtokens, dW, db, dtau of the deslice and of the slice that ran
    after it on fx_mid (its dz_num, ds), in one pass; the slice's dfx is
    already formed."""
    res = _hip_tied_bwd(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot,
                        want_dfx=False)
    if res is not None:
        dx, _, dw, db, dtau, dtok = res
        return dx, dtok, dw, db, dtau
    dxd, dtok, dwd, dbd, dtd = _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot,
                                                stats_in=stats)
    dxs, _, dws, dbs, dts = _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot,
                                           stats_in=stats)
    dx, dw, db, dtau = _sum_grads((dxd, dwd, dbd, dtd), (dxs, dws, dbs, dts))
    return dx, dtok, dw, db, dtau


_LIB.impl("tied_deslice", _tied_deslice_impl, "CUDA")
_LIB.impl("tied_slice_after", _tied_slice_after_impl, "CUDA")
_LIB.impl("tied_deslice_bwd", _tied_deslice_bwd_impl, "CUDA")


@torch.library.register_fake("flashslice::tied_deslice")
def _(x_mid, weight, bias, tau, tokens, dot):
    B, N, H, _ = x_mid.shape
    G, DV = weight.shape[-2], tokens.shape[3]
    return (x_mid.new_empty((B, N, H, DV)),
            x_mid.new_empty((B, H, 2, N), dtype=torch.float32)
            if _first_stats(x_mid, weight, DV) else stats_placeholder(B, H, N, x_mid),
            _link((B, N, H, DV), x_mid, x_mid.dtype),
            _link((B, H, G, DV + 1), x_mid, torch.float32))


@torch.library.register_fake("flashslice::tied_slice_after")
def _(x_mid, fx_mid, weight, bias, tau, stats, link_pt, link_small, dot):
    B, N, H, _ = x_mid.shape
    G = weight.shape[-2]
    return (x_mid.new_empty((B, H, G, fx_mid.shape[3]), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32))


@torch.library.register_fake("flashslice::tied_deslice_bwd")
def _(x_mid, weight, bias, tau, tokens, stats, d_out, fx_mid, dz_num, ds, dot):
    return (torch.empty_like(x_mid), torch.empty_like(tokens), torch.empty_like(weight),
            torch.empty_like(bias), torch.empty_like(tau))


def _tied_deslice_setup(ctx, inputs, output):
    # an output without a gradient arrives as None, not as zeros: no hand-over
    ctx.set_materialize_grads(False)
    x_mid, weight, bias, tau, tokens, dot = inputs
    ctx.save_for_backward(x_mid, weight, bias, tau, tokens, output[1])
    ctx.dot = dot


def _tied_deslice_grad(ctx, d_out, d_stats, fx_mid, d_link_small):
    """The deslice's backward: merged with the slice's deferred part when the
    slice's backward handed it over through the links (fx_mid, and dz_num
    and ds packed as (B, H, G, DV + 1)), else the plain deslice backward."""
    x_mid, weight, bias, tau, tokens, stats = ctx.saved_tensors
    handed = d_link_small is not None and fx_mid is not None
    if d_out is None:
        if not handed:
            return None, None, None, None, None, None
        d_out = torch.zeros(x_mid.shape[:3] + (tokens.shape[3],), device=x_mid.device,
                            dtype=x_mid.dtype)
    if not handed:
        dx, dtok, dw, db, dtau = torch.ops.flashslice.deslice_blk_bwd(
            x_mid, weight, bias, tau, tokens, stats, d_out, ctx.dot)
    else:
        DV = tokens.shape[3]
        dx, dtok, dw, db, dtau = torch.ops.flashslice.tied_deslice_bwd(
            x_mid, weight, bias, tau, tokens, stats, d_out, fx_mid,
            d_link_small[..., :DV], d_link_small[..., DV], ctx.dot)
    return dx, dw, db, dtau, dtok, None


def _tied_slice_after_setup(ctx, inputs, output):
    # an output without a gradient arrives as None, not as zeros: no hand-over
    ctx.set_materialize_grads(False)
    x_mid, fx_mid, weight, bias, tau, stats, link_pt, link_small, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau, stats)
    ctx.dot = dot


def _tied_slice_after_grad(ctx, dz_num, ds):
    """The slice's backward when it ran second: only dfx = w dz_num (the
    step before it needs it now); x_mid, W, b, tau get their gradient from
    the deslice's backward, which receives fx_mid, dz_num and ds as the
    links' gradients."""
    x_mid, fx_mid, weight, bias, tau, stats = ctx.saved_tensors
    B, H, G, DV = x_mid.shape[0], x_mid.shape[2], weight.shape[-2], fx_mid.shape[3]
    if dz_num is None and ds is None:
        return (None,) * 9
    if dz_num is None:
        dz_num = torch.zeros(B, H, G, DV, device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(B, H, G, device=x_mid.device, dtype=torch.float32)
    dfx, _ = torch.ops.flashslice.deslice_blk(x_mid, weight, bias, tau,
                                              dz_num.to(torch.float32), stats, ctx.dot)
    link_small = torch.cat([dz_num.to(torch.float32), ds.to(torch.float32).unsqueeze(-1)], -1)
    return (None, dfx.to(fx_mid.dtype), None, None, None, None, fx_mid.detach(), link_small,
            None)


torch.library.register_autograd("flashslice::tied_deslice", _tied_deslice_grad,
                                setup_context=_tied_deslice_setup)
torch.library.register_autograd("flashslice::tied_slice_after", _tied_slice_after_grad,
                                setup_context=_tied_slice_after_setup)


# ----------------------------------------------------------------- slice first

def _tied_slice_impl(x_mid, fx_mid, weight, bias, tau, dot):
    B, N, H, _ = x_mid.shape
    G, DV = weight.shape[-2], fx_mid.shape[3]
    want = _first_stats(x_mid, weight, DV)
    z_num, s, st = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot, want_stats=want)
    if not want:
        st = stats_placeholder(B, H, N, x_mid)
    return (z_num, s, st, _link((B, N, H, DV), x_mid, x_mid.dtype),
            _link((B, H, G, DV), x_mid, torch.float32))


def _tied_deslice_after_impl(x_mid, weight, bias, tau, tokens, stats, link_pt, link_tok, dot):
    out, _ = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot, stats_in=stats)
    return out


def _tied_slice_bwd_impl(x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, d_out, tokens,
                         dot):
    """dx_mid, dfx, dW, db, dtau of the slice and of the deslice that ran
    after it (its d_out, tokens), in one pass; the deslice's dtokens are
    already formed."""
    res = _hip_tied_bwd(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot,
                        want_dtok=False)
    if res is not None:
        return res[:5]
    dxs, dfx, dws, dbs, dts = _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot,
                                             stats_in=stats)
    dxd, _, dwd, dbd, dtd = _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot,
                                             stats_in=stats)
    dx, dw, db, dtau = _sum_grads((dxs, dws, dbs, dts), (dxd, dwd, dbd, dtd))
    return dx, dfx, dw, db, dtau


_LIB.impl("tied_slice", _tied_slice_impl, "CUDA")
_LIB.impl("tied_deslice_after", _tied_deslice_after_impl, "CUDA")
_LIB.impl("tied_slice_bwd", _tied_slice_bwd_impl, "CUDA")


@torch.library.register_fake("flashslice::tied_slice")
def _(x_mid, fx_mid, weight, bias, tau, dot):
    B, N, H, _ = x_mid.shape
    G, DV = weight.shape[-2], fx_mid.shape[3]
    return (x_mid.new_empty((B, H, G, DV), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32),
            x_mid.new_empty((B, H, 2, N), dtype=torch.float32)
            if _first_stats(x_mid, weight, DV) else stats_placeholder(B, H, N, x_mid),
            _link((B, N, H, DV), x_mid, x_mid.dtype),
            _link((B, H, G, DV), x_mid, torch.float32))


@torch.library.register_fake("flashslice::tied_deslice_after")
def _(x_mid, weight, bias, tau, tokens, stats, link_pt, link_tok, dot):
    B, N, H, _ = x_mid.shape
    return x_mid.new_empty((B, N, H, tokens.shape[3]))


@torch.library.register_fake("flashslice::tied_slice_bwd")
def _(x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, d_out, tokens, dot):
    return (torch.empty_like(x_mid), torch.empty_like(fx_mid), torch.empty_like(weight),
            torch.empty_like(bias), torch.empty_like(tau))


def _tied_slice_setup(ctx, inputs, output):
    # an output without a gradient arrives as None, not as zeros: no hand-over
    ctx.set_materialize_grads(False)
    x_mid, fx_mid, weight, bias, tau, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau, output[2])
    ctx.dot = dot


def _tied_slice_grad(ctx, dz_num, ds, d_stats, d_out, tokens):
    """The slice's backward: merged with the deslice's deferred part when the
    deslice's backward handed over d_out and its tokens through the links,
    else the plain slice backward."""
    x_mid, fx_mid, weight, bias, tau, stats = ctx.saved_tensors
    B, H, G, DV = x_mid.shape[0], x_mid.shape[2], weight.shape[-2], fx_mid.shape[3]
    handed = d_out is not None and tokens is not None
    if dz_num is None and ds is None and not handed:
        return (None,) * 6
    if dz_num is None:
        dz_num = torch.zeros(B, H, G, DV, device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(B, H, G, device=x_mid.device, dtype=torch.float32)
    if not handed:
        dx, dfx, dw, db, dtau = torch.ops.flashslice.slice_blk_bwd(
            x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, ctx.dot)
    else:
        dx, dfx, dw, db, dtau = torch.ops.flashslice.tied_slice_bwd(
            x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, d_out, tokens, ctx.dot)
    return dx, dfx, dw, db, dtau, None


def _tied_deslice_after_setup(ctx, inputs, output):
    # an output without a gradient arrives as None, not as zeros: no hand-over
    ctx.set_materialize_grads(False)
    x_mid, weight, bias, tau, tokens, stats, link_pt, link_tok, dot = inputs
    ctx.save_for_backward(x_mid, weight, bias, tau, tokens, stats)
    ctx.dot = dot


def _tied_deslice_after_grad(ctx, d_out):
    """The deslice's backward when it ran second: only dtokens = w^T d_out
    (the token step before it needs them now); d_out and the tokens go to
    the slice's backward as the links' gradients."""
    x_mid, weight, bias, tau, tokens, stats = ctx.saved_tensors
    if d_out is None:
        return (None,) * 9
    dtok, _, _ = torch.ops.flashslice.slice_blk(x_mid, d_out, weight, bias, tau, stats, ctx.dot)
    return (None, None, None, None, dtok.to(tokens.dtype), None, d_out,
            tokens.detach().to(torch.float32), None)


torch.library.register_autograd("flashslice::tied_slice", _tied_slice_grad,
                                setup_context=_tied_slice_setup)
torch.library.register_autograd("flashslice::tied_deslice_after", _tied_deslice_after_grad,
                                setup_context=_tied_deslice_after_setup)


# ------------------------------------------------------------------ public API

class Coupling:
    """One slice and one deslice on the same x_mid, weight, bias and tau, in
    either order (module docstring). Made by ``fused_coupling``."""

    def __init__(self, x_mid, weight, bias, tau):
        weight, bias, G = _prep_wb(x_mid, weight, bias)
        self.x_mid, self.weight, self.bias, self.tau, self.G = x_mid, weight, bias, tau, G
        self.dot = _dot_mode(x_mid)
        self._first = None      # "slice" or "deslice", once one has run
        self._pending = None    # (stats, links, DV) the second op consumes
        self._done = False

    def _second(self, name, dv):
        if self._done or self._first == name:
            raise RuntimeError("a coupling runs one slice and one deslice; %s was called twice"
                               % name)
        stats, links, DV = self._pending
        if dv != DV:
            raise ValueError("the coupling's %s has value width %d, the first op had %d"
                             % (name, dv, DV))
        self._done = True
        return stats, links

    def deslice(self, tokens):
        """``fused_deslice(x_mid, weight, bias, tau, tokens)``: out
        (B, N, H, DV) in x_mid's dtype."""
        DV = tokens.shape[3]
        _check_dims(self.x_mid.shape[3], self.G, DV)
        args = (self.x_mid, self.weight, self.bias, self.tau, tokens)
        if self._first is None:
            out, stats, lp, ls = torch.ops.flashslice.tied_deslice(*args, self.dot)
            self._first, self._pending = "deslice", (stats, (lp, ls), DV)
            return out
        stats, (lp, lt) = self._second("deslice", DV)
        return torch.ops.flashslice.tied_deslice_after(*args, stats, lp, lt, self.dot)

    def slice(self, fx_mid):
        """``fused_slice(x_mid, fx_mid, weight, bias, tau)``: fp32 z_num
        (B, H, G, DV) and s (B, H, G)."""
        DV = fx_mid.shape[3]
        _check_dims(self.x_mid.shape[3], self.G, DV)
        args = (self.x_mid, fx_mid, self.weight, self.bias, self.tau)
        if self._first is None:
            z_num, s, stats, lp, lt = torch.ops.flashslice.tied_slice(*args, self.dot)
            self._first, self._pending = "slice", (stats, (lp, lt), DV)
            return z_num, s
        stats, (lp, ls) = self._second("slice", DV)
        return torch.ops.flashslice.tied_slice_after(*args, stats, lp, ls, self.dot)


def fused_coupling(x_mid, weight, bias, tau):
    """A slice/deslice coupling on one x_mid (B, N, H, D), weight, bias and
    tau (the shapes ``fused_slice`` documents) whose backward is one merged
    pass: call ``.slice(fx_mid)`` and ``.deslice(tokens)`` once each, in
    either order, with any differentiable step between them (module
    docstring). Both ops share one value width DV."""
    return Coupling(x_mid, weight, bias, tau)


__all__ = ["fused_coupling", "Coupling"]
