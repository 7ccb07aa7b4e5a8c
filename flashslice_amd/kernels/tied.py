"""Tied deslice -> slice coupling with one fused backward pass.

The reference lists this as its "tied backward fusion" (ROADMAP.md:58-65)
and does not implement it. In a persistent point stream a layer deslices
tokens onto the points and slices a point stream back, both through the
same ``x_mid``, slice projection and temperature::

    out        = fused_deslice(x_mid, W, b, tau, tokens, return_stats=True)
    z_num, s   = fused_slice(x_mid, fx_mid, W, b, tau, stats=...)

(BASELINE config 4's order). Autograd then runs the two backward ops --
each recomputes the softmax weights, forms a softmax Jacobian and writes its
own dx_mid -- and sums the two dx_mid (reference ``_deslice_bwd_impl`` and
``_slice_bwd_impl``, ``slice_ops.py:822-885``). ``fused_deslice_slice``
computes the same three outputs as one custom operator whose backward is one
HIP kernel (``fs_tied_bwd``): one logits recompute per tile, the two ops'
Jacobian inputs summed before the Jacobian (it is linear in them), one
dx_mid / dW product, and one dx_mid written. Point passes of the backward:
read x_mid, fx_mid, d_out, write dx_mid, dfx_mid -- five, against the two
ops' seven plus autograd's three for the dx_mid sum.

``fx_mid`` is an input of the op, so it cannot depend on ``out``; a deslice
-> MLP -> slice chain, whose slice input is computed from ``out``, keeps
using the two ops. Shapes outside the whole-G kernel family (G > 128, wide
D / DV) and kernel mode ``"blocked"`` run the two backward ops inside this
op's backward and sum their gradients, so every shape the two ops accept is
accepted here too.
"""

import torch

from . import _hip
from .slice_ops import (
    _Call, _LIB, _as_points, _check_dims, _check_points, _dot_mode, _grads_out, _hip_deslice_bwd,
    _hip_deslice_fwd, _hip_slice_bwd, _hip_slice_fwd, _param_grad_buffers, _point_dtype,
    _prep_wb, _small,
)

_LIB.define(
    "deslice_slice(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor tokens, int dot) -> (Tensor, Tensor, Tensor)")
_LIB.define(
    "deslice_slice_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor tokens, Tensor d_out, Tensor dz_num, Tensor ds, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")


def _family(x_mid, weight, bias, tau, dv, dot):
    """1 = the whole-G kernels serve this call, 2 = the G-blocked ones."""
    call = _Call(x_mid, weight, bias, tau, dv, dot)
    return _hip.lib().fs_family(call.prm)


def _deslice_slice_impl(x_mid, fx_mid, weight, bias, tau, tokens, dot):
    """flashslice::deslice_slice: the deslice, then the slice on the same
    logits. The G-blocked kernels hand the deslice's softmax statistics to
    the slice (as ``fused_slice(..., stats=)`` does); the whole-G kernels
    form the softmax exactly in each op's one pass and need none."""
    DV = fx_mid.shape[3]
    with torch.cuda.device(x_mid.device):
        blocked = _family(x_mid, weight, bias, tau, DV, dot) == 2
    out, st = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot, want_stats=blocked)
    z_num, s, _ = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot, stats_in=st)
    return out, z_num, s


def _hip_tied_bwd(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot,
                  want_dfx=True, want_dtok=True):
    """Both ops' gradients from fs_tied_bwd; None where the whole-G kernels
    do not serve the shape. ``want_dfx`` / ``want_dtok`` False: that output
    is not formed (None in its place)."""
    B, N, H, D = x_mid.shape
    DV = fx_mid.shape[3]
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, DV, dot)
        if _hip.lib().fs_family(call.prm) != 1:
            return None
        _check_points(x_mid, fx_mid, DV, "fx_mid")
        _check_points(x_mid, d_out, DV, "d_out")
        dt = _point_dtype(x_mid, fx_mid, d_out)
        x, fx, do = _as_points(x_mid, dt), _as_points(fx_mid, dt), _as_points(d_out, dt)
        dxm = torch.empty_like(x_mid, dtype=dt) if x_mid.stride(3) == 1 else \
            torch.empty(x_mid.shape, device=x.device, dtype=dt)
        dfx = None
        if want_dfx:
            dfx = torch.empty_like(fx_mid, dtype=dt) if fx_mid.stride(3) == 1 else \
                torch.empty(fx_mid.shape, device=x.device, dtype=dt)
        tok = _small(tokens, (B, H, call.G, DV), "tokens", x.device)
        dz = _small(dz_num, (B, H, call.G, DV), "dz_num", x.device)
        dsv = _small(ds, (B, H, call.G), "ds", x.device)
        dtok = (torch.empty(B, H, call.G, DV, device=x.device, dtype=torch.float32)
                if want_dtok else None)
        dW, db, dtau = _param_grad_buffers(call)
        ws, nws = call.workspace(_hip.OP_TIED_BWD)
        _hip.check(_hip.lib().fs_tied_bwd(
            _hip.points(x, D), _hip.points(fx, DV), _hip.points(do, DV), call.prm,
            _hip.ptr(tok), _hip.ptr(dz), _hip.ptr(dsv), _hip.points(dxm, D),
            _hip.points(dfx, DV) if want_dfx else None, _hip.ptr(dtok), _hip.ptr(dW),
            _hip.ptr(db), _hip.ptr(dtau), _hip.ptr(ws), nws, call.stream()))
    if dxm.dtype != x_mid.dtype:
        dxm = dxm.to(x_mid.dtype)
    if dfx is not None and dfx.dtype != fx_mid.dtype:
        dfx = dfx.to(fx_mid.dtype)
    return ((dxm, dfx) + _grads_out(call, weight, bias, tau, dW, db, dtau)
            + (None if dtok is None else dtok.to(tokens.dtype),))


def _deslice_slice_bwd_impl(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot):
    """flashslice::deslice_slice_bwd -> (dx_mid, dfx_mid, dweight, dbias,
    dtau, dtokens): the tied kernel, or the two backward ops and the sum of
    their gradients where it does not serve the shape."""
    res = _hip_tied_bwd(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot)
    if res is not None:
        return res
    dxd, dtok, dwd, dbd, dtd = _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot)
    dxs, dfx, dws, dbs, dts = _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot)
    return dxd + dxs, dfx, dwd + dws, dbd + dbs, dtd + dts, dtok


_LIB.impl("deslice_slice", _deslice_slice_impl, "CUDA")
_LIB.impl("deslice_slice_bwd", _deslice_slice_bwd_impl, "CUDA")


@torch.library.register_fake("flashslice::deslice_slice")
def _(x_mid, fx_mid, weight, bias, tau, tokens, dot):
    B, N, H, D = x_mid.shape
    G, DV = weight.shape[-2], fx_mid.shape[3]
    return (x_mid.new_empty((B, N, H, tokens.shape[3])),
            x_mid.new_empty((B, H, G, DV), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32))


@torch.library.register_fake("flashslice::deslice_slice_bwd")
def _(x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, dot):
    return (torch.empty_like(x_mid), torch.empty_like(fx_mid), torch.empty_like(weight),
            torch.empty_like(bias), torch.empty_like(tau), torch.empty_like(tokens))


def _tied_setup(ctx, inputs, output):
    x_mid, fx_mid, weight, bias, tau, tokens, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau, tokens)
    ctx.dot = dot


def _tied_grad(ctx, d_out, dz_num, ds):
    """Saves the inputs, never w; an output without a gradient contributes
    zeros (as the two ops' own formulas, reference slice_ops.py:928-948)."""
    x_mid, fx_mid, weight, bias, tau, tokens = ctx.saved_tensors
    B, N, H, D = x_mid.shape
    G, DV = weight.shape[-2], fx_mid.shape[3]
    if d_out is None:
        d_out = torch.zeros(B, N, H, DV, device=x_mid.device, dtype=x_mid.dtype)
    if dz_num is None:
        dz_num = torch.zeros(B, H, G, DV, device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(B, H, G, device=x_mid.device, dtype=torch.float32)
    dxm, dfx, dw, db, dtau, dtok = torch.ops.flashslice.deslice_slice_bwd(
        x_mid, fx_mid, weight, bias, tau, tokens, d_out, dz_num, ds, ctx.dot)
    return dxm, dfx, dw, db, dtau, dtok, None


torch.library.register_autograd("flashslice::deslice_slice", _tied_grad,
                                setup_context=_tied_setup)


def fused_deslice_slice(x_mid, fx_mid, weight, bias, tau, tokens):
    """``out = fused_deslice(x_mid, weight, bias, tau, tokens)`` and
    ``z_num, s = fused_slice(x_mid, fx_mid, weight, bias, tau)`` on one set
    of logits, as one operator whose backward is a single pass over the
    points (module docstring). Arguments take the shapes ``fused_slice`` /
    ``fused_deslice`` document; ``tokens`` (B, H, G, DV) share fx_mid's value
    width DV. Returns ``(out, z_num, s)``: out (B, N, H, DV) in x_mid's
    dtype, z_num (B, H, G, DV) and s (B, H, G) fp32."""
    weight, bias, G = _prep_wb(x_mid, weight, bias)
    D, DV = x_mid.shape[3], fx_mid.shape[3]
    if tokens.shape[3] != DV:
        raise ValueError("fused_deslice_slice: tokens have width %d, fx_mid %d"
                         % (tokens.shape[3], DV))
    _check_dims(D, G, DV)
    dot = _dot_mode(x_mid)
    return torch.ops.flashslice.deslice_slice(x_mid, fx_mid, weight, bias, tau, tokens, dot)
