"""Ragged batches: samples of different point counts in one launch.

The reference plans this (ROADMAP.md:66-68: "samples of different N in one
launch through row splits, so that small meshes fill the GPU instead of
running one sample per device behind a fixed per-step floor") and does not
implement it. Here the B samples' points are concatenated along the point
axis -- x_mid (rows, H, D), fx_mid (rows, H, DV) -- and ``row_splits``
(B + 1 non-decreasing offsets, first 0, last = rows) says which rows are
sample b's. Every sample gets its own slice sums (z_num, s of shape
(B, H, G, DV), (B, H, G)); the slice projection may be shared (G, D),
per head (H, G, D) or per sample (B, H, G, D), as in ``fused_slice``. Each
(sample, head) block of every kernel reads its row range from the splits,
so no sample is padded and one launch covers all.

``row_splits`` on the CPU (a list or an int64 tensor) is validated and
copied to the device; a device tensor is used as is, with ``max_rows`` (the
longest sample, which sizes the launch) required and the splits not read
back (that would synchronise): the kernels clamp them to the point tensors'
rows, so malformed splits give wrong sums but stay in bounds.

Every shape the plain ops serve is served here, on both kernel families:
the whole-G kernels where the slot axis fits in registers, the G-blocked
ones (any G, widths up to 256) otherwise. The softmax statistics of a
ragged batch are (1, H, 2, rows) fp32, indexed by row like the points;
``return_stats`` / ``stats`` hand them from one op to the other as
``fused_slice`` / ``fused_deslice`` do.
"""

import torch

from .slice_ops import (
    _LIB, _check_dims, _dot_mode, _hip_deslice_bwd, _hip_deslice_fwd, _hip_slice_bwd,
    _hip_slice_fwd, _prep_wb,
)

_LIB.define(
    "slice_varlen(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor row_splits, int max_rows, Tensor? stats, int dot) -> (Tensor, Tensor, Tensor)")
_LIB.define(
    "slice_varlen_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor row_splits, int max_rows, Tensor stats, Tensor dz_num, Tensor ds, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_LIB.define(
    "deslice_varlen(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor row_splits, int max_rows, Tensor? stats, int dot) -> (Tensor, Tensor)")
_LIB.define(
    "deslice_varlen_bwd(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor row_splits, int max_rows, Tensor stats, Tensor d_out, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")


def _rows(row_splits, max_rows):
    return (row_splits, row_splits.shape[0] - 1, max_rows)


def _pts(t):
    """(rows, H, C) -> the (1, rows, H, C) view the library addresses."""
    return t.unsqueeze(0)


def _slice_varlen_impl(x_mid, fx_mid, weight, bias, tau, row_splits, max_rows, stats, dot):
    return _hip_slice_fwd(_pts(x_mid), _pts(fx_mid), weight, bias, tau, dot, stats_in=stats,
                          want_stats=True, rows=_rows(row_splits, max_rows))


def _slice_varlen_bwd_impl(x_mid, fx_mid, weight, bias, tau, row_splits, max_rows, stats, dz_num,
                           ds, dot):
    dx, dfx, dw, db, dtau = _hip_slice_bwd(_pts(x_mid), _pts(fx_mid), weight, bias, tau, dz_num,
                                           ds, dot, stats_in=stats,
                                           rows=_rows(row_splits, max_rows))
    return dx[0], dfx[0], dw, db, dtau


def _deslice_varlen_impl(x_mid, weight, bias, tau, tokens, row_splits, max_rows, stats, dot):
    out, st = _hip_deslice_fwd(_pts(x_mid), weight, bias, tau, tokens, dot, stats_in=stats,
                               want_stats=True, rows=_rows(row_splits, max_rows))
    return out[0], st


def _deslice_varlen_bwd_impl(x_mid, weight, bias, tau, tokens, row_splits, max_rows, stats, d_out,
                             dot):
    dx, dtok, dw, db, dtau = _hip_deslice_bwd(_pts(x_mid), weight, bias, tau, tokens,
                                              _pts(d_out), dot, stats_in=stats,
                                              rows=_rows(row_splits, max_rows))
    return dx[0], dtok, dw, db, dtau


_LIB.impl("slice_varlen", _slice_varlen_impl, "CUDA")
_LIB.impl("slice_varlen_bwd", _slice_varlen_bwd_impl, "CUDA")
_LIB.impl("deslice_varlen", _deslice_varlen_impl, "CUDA")
_LIB.impl("deslice_varlen_bwd", _deslice_varlen_bwd_impl, "CUDA")


def _stats_fake(x_mid):
    return x_mid.new_empty((1, x_mid.shape[1], 2, x_mid.shape[0]), dtype=torch.float32)


@torch.library.register_fake("flashslice::slice_varlen")
def _(x_mid, fx_mid, weight, bias, tau, row_splits, max_rows, stats, dot):
    B, H, G = row_splits.shape[0] - 1, x_mid.shape[1], weight.shape[-2]
    return (x_mid.new_empty((B, H, G, fx_mid.shape[2]), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32), _stats_fake(x_mid))


@torch.library.register_fake("flashslice::slice_varlen_bwd")
def _(x_mid, fx_mid, weight, bias, tau, row_splits, max_rows, stats, dz_num, ds, dot):
    return (torch.empty_like(x_mid), torch.empty_like(fx_mid), torch.empty_like(weight),
            torch.empty_like(bias), torch.empty_like(tau))


@torch.library.register_fake("flashslice::deslice_varlen")
def _(x_mid, weight, bias, tau, tokens, row_splits, max_rows, stats, dot):
    return (x_mid.new_empty((x_mid.shape[0], x_mid.shape[1], tokens.shape[3])),
            _stats_fake(x_mid))


@torch.library.register_fake("flashslice::deslice_varlen_bwd")
def _(x_mid, weight, bias, tau, tokens, row_splits, max_rows, stats, d_out, dot):
    return (torch.empty_like(x_mid), torch.empty_like(tokens), torch.empty_like(weight),
            torch.empty_like(bias), torch.empty_like(tau))


def _slice_setup(ctx, inputs, output):
    x_mid, fx_mid, weight, bias, tau, row_splits, max_rows, stats, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau, row_splits, output[2])
    ctx.max_rows, ctx.dot = max_rows, dot


def _slice_grad(ctx, dz_num, ds, dstats):
    """The statistics are saved intermediates: an incoming gradient on them
    is ignored (as the blocked ops', reference blocked.py:1538-1550)."""
    x_mid, fx_mid, weight, bias, tau, row_splits, stats = ctx.saved_tensors
    B, H, G, DV = row_splits.shape[0] - 1, x_mid.shape[1], weight.shape[-2], fx_mid.shape[2]
    if dz_num is None:
        dz_num = torch.zeros(B, H, G, DV, device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(B, H, G, device=x_mid.device, dtype=torch.float32)
    dxm, dfx, dw, db, dtau = torch.ops.flashslice.slice_varlen_bwd(
        x_mid, fx_mid, weight, bias, tau, row_splits, ctx.max_rows, stats, dz_num, ds, ctx.dot)
    return dxm, dfx, dw, db, dtau, None, None, None, None


def _deslice_setup(ctx, inputs, output):
    x_mid, weight, bias, tau, tokens, row_splits, max_rows, stats, dot = inputs
    ctx.save_for_backward(x_mid, weight, bias, tau, tokens, row_splits, output[1])
    ctx.max_rows, ctx.dot = max_rows, dot


def _deslice_grad(ctx, d_out, dstats):
    x_mid, weight, bias, tau, tokens, row_splits, stats = ctx.saved_tensors
    dxm, dtok, dw, db, dtau = torch.ops.flashslice.deslice_varlen_bwd(
        x_mid, weight, bias, tau, tokens, row_splits, ctx.max_rows, stats, d_out, ctx.dot)
    return dxm, dw, db, dtau, dtok, None, None, None, None


torch.library.register_autograd("flashslice::slice_varlen", _slice_grad,
                                setup_context=_slice_setup)
torch.library.register_autograd("flashslice::deslice_varlen", _deslice_grad,
                                setup_context=_deslice_setup)


def _splits(row_splits, rows, device, max_rows):
    """The row splits on ``device`` and the longest sample."""
    if isinstance(row_splits, torch.Tensor) and row_splits.device.type != "cpu":
        if max_rows is None:
            raise ValueError("row_splits on the device need max_rows (the longest sample)")
        if row_splits.dtype != torch.int64 or row_splits.dim() != 1 or row_splits.numel() < 2:
            raise ValueError("row_splits must be a 1-d int64 tensor of B + 1 offsets")
        return row_splits, int(max_rows)
    rs = torch.as_tensor(row_splits, dtype=torch.int64)
    if rs.dim() != 1 or rs.numel() < 2:
        raise ValueError("row_splits must hold B + 1 offsets, got shape %s" % (tuple(rs.shape),))
    n = rs[1:] - rs[:-1]
    if int(rs[0]) != 0 or int(rs[-1]) != rows or bool((n < 0).any()):
        raise ValueError("row_splits must rise from 0 to the %d rows of x_mid, got %s"
                         % (rows, rs.tolist()))
    longest = int(n.max())
    if max_rows is not None and int(max_rows) < longest:
        raise ValueError("max_rows=%d is below the longest sample (%d rows)"
                         % (max_rows, longest))
    return rs.to(device), max(1, longest if max_rows is None else int(max_rows))


def _prep(x_mid, weight, bias, row_splits, max_rows, dv):
    if x_mid.dim() != 3:
        raise ValueError("x_mid must be (rows, H, D) for a ragged batch, got shape %s"
                         % (tuple(x_mid.shape),))
    rs, longest = _splits(row_splits, x_mid.shape[0], x_mid.device, max_rows)
    B = rs.shape[0] - 1
    view = torch.empty((B, 1) + tuple(x_mid.shape[1:]), device="meta")  # (B, ., H, D) for _prep_wb
    weight, bias, G = _prep_wb(view, weight, bias)
    _check_dims(x_mid.shape[2], G, dv)
    return weight, bias, rs, longest


def fused_slice_varlen(x_mid, fx_mid, weight, bias, tau, row_splits, max_rows=None,
                       return_stats=False, stats=None):
    """Slice of a ragged batch: x_mid (rows, H, D), fx_mid (rows, H, DV),
    sample b = rows row_splits[b] .. row_splits[b+1]-1; weight (G, D),
    (H, G, D) or (B, H, G, D); bias None, (G,), (H, G) or (B, H, G); tau
    (H,). Returns fp32 z_num (B, H, G, DV) and s (B, H, G), each sample's
    equal to ``fused_slice`` on that sample alone (an empty sample gives
    zeros). ``stats`` (1, H, 2, rows): statistics of these very logits from
    a tied ``fused_deslice_varlen(..., return_stats=True)``; with
    ``return_stats=True`` the statistics are returned third (detached)."""
    weight, bias, rs, longest = _prep(x_mid, weight, bias, row_splits, max_rows,
                                      fx_mid.shape[2])
    if fx_mid.dim() != 3 or fx_mid.shape[:2] != x_mid.shape[:2]:
        raise ValueError("fx_mid must be (rows, H, DV) with x_mid's rows and heads")
    z_num, s, st = torch.ops.flashslice.slice_varlen(x_mid, fx_mid, weight, bias, tau, rs,
                                                     longest, stats, _dot_mode(x_mid))
    return (z_num, s, st.detach()) if return_stats else (z_num, s)


def fused_deslice_varlen(x_mid, weight, bias, tau, tokens, row_splits, max_rows=None,
                         stats=None, return_stats=False):
    """Deslice of a ragged batch: tokens (B, H, G, DV) per sample; returns out
    (rows, H, DV) in x_mid's dtype, each sample's rows equal to
    ``fused_deslice`` on that sample alone; ``stats`` / ``return_stats`` as
    in ``fused_slice_varlen``."""
    weight, bias, rs, longest = _prep(x_mid, weight, bias, row_splits, max_rows,
                                      tokens.shape[3])
    if tokens.dim() != 4 or tokens.shape[0] != rs.shape[0] - 1:
        raise ValueError("tokens must be (B, H, G, DV) with B = %d samples, got shape %s"
                         % (rs.shape[0] - 1, tuple(tokens.shape)))
    out, st = torch.ops.flashslice.deslice_varlen(x_mid, weight, bias, tau, tokens, rs, longest,
                                                  stats, _dot_mode(x_mid))
    return (out, st.detach()) if return_stats else out


__all__ = ["fused_slice_varlen", "fused_deslice_varlen"]
