"""The G-blocked ("blocked") operators: any slot count, head widths up to 256,
with per-point softmax statistics.

Mirrors the reference's ``flashslice.kernels.blocked``
(``flashslice/kernels/blocked.py``): the same public functions
(``set_block_g``, ``set_stats_mode``, ``stats_mode``, ``tiles``,
``compute_stats``) and the same four ``torch.ops.flashslice`` custom
operators (``slice_blk``, ``slice_blk_bwd``, ``deslice_blk``,
``deslice_blk_bwd``) with their schemas, fakes and autograd. The ops carry
the statistics tensor (B, H, 2, N) fp32 -- [..., 0, n] the row max of the
logits, [..., 1, n] the sum of exponentials against it -- which a tied op
reuses (reference ``blocked.py:1329-1335``).

Underneath, the HIP library decides by shape which kernels serve a call
(``fs_family``): shapes whose slot axis fits in registers run the whole-G
kernels, which recompute the membership exactly in one pass and write the
statistics when asked; the others run the G-blocked kernels.
"""

import os

import torch

from . import _hip
from .slice_ops import (set_tile_table, tile_table,  # noqa: F401
                        _hip_slice_fwd, _hip_deslice_fwd, _hip_slice_bwd, _hip_deslice_bwd,
                        _Call, _as_points, _point_dtype, stats_placeholder)

_BLOCK_G = None  # None = automatic; set_block_g overrides


def set_block_g(gb):
    """Force the G-block size (a power of two >= 16), or None for automatic
    (reference ``blocked.py:87-94``). The value is validated as the
    reference's and reported by ``tiles()``; the HIP kernels always work in
    slot blocks of 32 (one MFMA tile), so it does not change them."""
    global _BLOCK_G
    if gb is not None and (gb < 16 or (gb & (gb - 1)) != 0):
        raise ValueError("block size must be a power of two >= 16, got %r" % gb)
    _BLOCK_G = gb


def _pow2_at_least_16(v):
    p = 16
    while p < v:
        p *= 2
    return p


_STATS_MODES = ("online", "two-pass")
_STATS_MODE = os.environ.get("FLASHSLICE_STATS_MODE", "").lower() or "online"


def set_stats_mode(mode):
    """How the statistics (m, l) are formed when none are handed in:
    ``"online"`` (default, one pass over G) or ``"two-pass"`` (max first,
    then the sum against it). Overrides FLASHSLICE_STATS_MODE (reference
    ``blocked.py:105-116``)."""
    global _STATS_MODE
    if mode not in _STATS_MODES:
        raise ValueError("stats mode must be one of %s, got %r" % (_STATS_MODES, mode))
    _STATS_MODE = mode


def stats_mode():
    return _STATS_MODE


def tiles(d, g, dot=0):
    """(D_tile, G_block) the reference's blocked Triton kernels use at head
    width d, slot count g and dot level ``dot`` (reference
    ``blocked.py:123-133``): D padded to a power of two >= 16, a block
    budget GB * D_tile of 2048 on FMA paths and 4096 on tensor-core paths,
    GB in [16, 64]. Kept as the API's pure function; the HIP kernels tile
    slots in blocks of 32 and D in blocks of 32."""
    dt = _pow2_at_least_16(d)
    budget = 4096 if dot >= 3 else 2048
    gb = _BLOCK_G or max(16, min(64, budget // dt))
    return dt, min(gb, _pow2_at_least_16(g))


def compute_stats(x_mid, weight, bias, tau, dot=0):
    """(B, H, 2, N) fp32 softmax statistics of the slice logits per point:
    [..., 0, :] the row max, [..., 1, :] the sum of exponentials (reference
    ``blocked.py:1329-1343``)."""
    B, N, H, D = x_mid.shape
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, D, dot)
        x = _as_points(x_mid, _point_dtype(x_mid))
        stats = torch.empty(B, H, 2, N, device=x.device, dtype=torch.float32)
        ws, nws = call.workspace(_hip.OP_STATS)
        _hip.check(_hip.lib().fs_compute_stats(
            _hip.points(x, D), call.prm, _hip.ptr(stats), 1 if _STATS_MODE == "two-pass" else 0,
            _hip.ptr(ws), nws, call.stream()))
    return stats


# --------------------------------------------------------------------------- #
# custom ops (reference blocked.py:1477-1568)
# --------------------------------------------------------------------------- #

torch.library.define(
    "flashslice::slice_blk",
    "(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor? stats, int dot) -> (Tensor, Tensor, Tensor)")
torch.library.define(
    "flashslice::slice_blk_bwd",
    "(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor stats, Tensor dz_num, Tensor ds, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
torch.library.define(
    "flashslice::deslice_blk",
    "(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor? stats, int dot) -> (Tensor, Tensor)")
torch.library.define(
    "flashslice::deslice_blk_bwd",
    "(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, Tensor tokens, "
    "Tensor stats, Tensor d_out, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")


def _is_placeholder(stats):
    return stats is not None and all(st == 0 for st in stats.stride())


def _slice_blk_impl(x_mid, fx_mid, weight, bias, tau, stats, dot):
    """flashslice::slice_blk (reference ``_slice_blk_impl``, blocked.py:1346-1368).
    Given a coupling's placeholder for statistics no whole-G pass formed
    (``stats_placeholder``), it returns that placeholder and forms none."""
    if _is_placeholder(stats):
        z_num, s, _ = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot, stats_in=stats)
        return z_num, s, stats
    if stats is None and _STATS_MODE == "two-pass":
        stats = compute_stats(x_mid, weight, bias, tau, dot)
    z_num, s, st = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot,
                                  stats_in=stats, want_stats=True)
    return z_num, s, st


def _slice_blk_bwd_impl(x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, dot):
    """flashslice::slice_blk_bwd (reference blocked.py:1371-1403)."""
    return _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot, stats_in=stats)


def _deslice_blk_impl(x_mid, weight, bias, tau, tokens, stats, dot):
    """flashslice::deslice_blk (reference blocked.py:1406-1433): with no
    statistics in hand one online pass forms out and (m, l) both."""
    if _is_placeholder(stats):
        out, _ = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot, stats_in=stats)
        return out, stats
    if stats is None and _STATS_MODE == "two-pass":
        stats = compute_stats(x_mid, weight, bias, tau, dot)
    out, st = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot,
                               stats_in=stats, want_stats=True)
    return out, st


def _deslice_blk_bwd_impl(x_mid, weight, bias, tau, tokens, stats, d_out, dot):
    """flashslice::deslice_blk_bwd (reference blocked.py:1436-1469)."""
    return _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot, stats_in=stats)


torch.library.impl("flashslice::slice_blk", "CUDA", _slice_blk_impl)
torch.library.impl("flashslice::slice_blk_bwd", "CUDA", _slice_blk_bwd_impl)
torch.library.impl("flashslice::deslice_blk", "CUDA", _deslice_blk_impl)
torch.library.impl("flashslice::deslice_blk_bwd", "CUDA", _deslice_blk_bwd_impl)


@torch.library.register_fake("flashslice::slice_blk")
def _(x_mid, fx_mid, weight, bias, tau, stats, dot):
    B, N, H, D = x_mid.shape
    G = weight.shape[-2]
    return (x_mid.new_empty((B, H, G, fx_mid.shape[3]), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32),
            stats_placeholder(B, H, N, x_mid) if _is_placeholder(stats)
            else x_mid.new_empty((B, H, 2, N), dtype=torch.float32))


@torch.library.register_fake("flashslice::slice_blk_bwd")
def _(x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, dot):
    return (torch.empty_like(x_mid), torch.empty_like(fx_mid),
            torch.empty_like(weight), torch.empty_like(bias),
            torch.empty_like(tau))


@torch.library.register_fake("flashslice::deslice_blk")
def _(x_mid, weight, bias, tau, tokens, stats, dot):
    B, N, H, D = x_mid.shape
    return (x_mid.new_empty((B, N, H, tokens.shape[3])),
            stats_placeholder(B, H, N, x_mid) if _is_placeholder(stats)
            else x_mid.new_empty((B, H, 2, N), dtype=torch.float32))


@torch.library.register_fake("flashslice::deslice_blk_bwd")
def _(x_mid, weight, bias, tau, tokens, stats, d_out, dot):
    return (torch.empty_like(x_mid), torch.empty_like(tokens),
            torch.empty_like(weight), torch.empty_like(bias),
            torch.empty_like(tau))


def _slice_setup(ctx, inputs, output):
    x_mid, fx_mid, weight, bias, tau, stats, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau, output[2])
    ctx.dot = dot


def _slice_grad(ctx, dz_num, ds, dstats):
    """The statistics are saved intermediates, not a differentiable output:
    an incoming gradient on them is ignored (reference blocked.py:1538-1550)."""
    x_mid, fx_mid, weight, bias, tau, stats = ctx.saved_tensors
    if dz_num is None:
        dz_num = torch.zeros(x_mid.shape[0], x_mid.shape[2], weight.shape[-2],
                             fx_mid.shape[3], device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(dz_num.shape[:-1], device=dz_num.device, dtype=torch.float32)
    dxm, dfx, dw, db, dtau = torch.ops.flashslice.slice_blk_bwd(
        x_mid, fx_mid, weight, bias, tau, stats, dz_num, ds, ctx.dot)
    return dxm, dfx, dw, db, dtau, None, None


def _deslice_setup(ctx, inputs, output):
    x_mid, weight, bias, tau, tokens, stats, dot = inputs
    ctx.save_for_backward(x_mid, weight, bias, tau, tokens, output[1])
    ctx.dot = dot


def _deslice_grad(ctx, d_out, dstats):
    x_mid, weight, bias, tau, tokens, stats = ctx.saved_tensors
    dxm, dtok, dw, db, dtau = torch.ops.flashslice.deslice_blk_bwd(
        x_mid, weight, bias, tau, tokens, stats, d_out, ctx.dot)
    return dxm, dw, db, dtau, dtok, None, None


torch.library.register_autograd("flashslice::slice_blk", _slice_grad,
                                setup_context=_slice_setup)
torch.library.register_autograd("flashslice::deslice_blk", _deslice_grad,
                                setup_context=_deslice_setup)

__all__ = ["tiles", "set_block_g", "compute_stats", "set_stats_mode", "stats_mode"]
