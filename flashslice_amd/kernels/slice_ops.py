"""FlashSlice's fused slice/deslice operators, served by hand-written HIP
kernels for MI355X (gfx950).

This module mirrors the reference's ``flashslice.kernels.slice_ops``
(Shizheng-Wen/flashslice v0.3.0, ``flashslice/kernels/slice_ops.py``): the
same public functions, the same shape contract and error messages, the same
four ``torch.ops.flashslice`` custom operators with the same schemas, fake
(meta) implementations and autograd formulas. Only what runs underneath
differs: every op's CUDA-key implementation (PyTorch-ROCm routes HIP tensors
through that key) calls the C ABI of ``libflashslice_hip.so``
(``include/flashslice_hip.h``) through ctypes, on the current stream.

The math, per sample b and head h (reference ``slice_ops.py:9-18``)::

    w = softmax_G((x_mid @ W.T + b) / tau)        never written to memory
    slice:   z_num[g] = sum_n w[n, g] fx_mid[n],  s[g] = sum_n w[n, g]
    deslice: out[n]   = sum_g w[n, g] tokens[g]

Backward recomputes w and applies the softmax Jacobian per point; the
cross-tile sums (z_num, s, dtokens, dW, db, dtau) are per-wave partials
reduced in a fixed order inside the library, so repeated runs are bitwise
identical.

Routing is kept exactly as the reference's (``single_tile_dims`` /
``_use_blocked``): it selects which custom op is called -- the "single-tile"
ops here, the "blocked" ops (which carry softmax statistics) in
``blocked.py``. Which HIP kernel family serves a call is the library's own
decision by shape (``fs_family``): the whole-G family (slot axis in
registers, one pass per op) or the G-blocked family.
"""

import os

import torch

from . import _hip

# --------------------------------------------------------------------------- #
# tile tables (API shim)
# --------------------------------------------------------------------------- #
# The reference picks Triton tile tables per NVIDIA GPU class
# (slice_ops.py:270-301). The HIP kernels here have one MI355X launch
# geometry; the API is kept (validation and reporting) so code that sets or
# reads the table keeps working.

_TILE_TABLES = ("hopper", "ada", "cdna4")
_TILE_TABLE = os.environ.get("FLASHSLICE_TILE_TABLE", "").lower() or "auto"


def set_tile_table(name):
    """'auto' (default), 'hopper', 'ada' or 'cdna4' -- overrides
    FLASHSLICE_TILE_TABLE (reference ``slice_ops.py:281-289``). The HIP
    kernels have a single MI355X geometry; the value is reported by
    ``tile_table`` and otherwise has no effect."""
    global _TILE_TABLE
    if name not in ("auto",) + _TILE_TABLES:
        raise ValueError("tile table must be 'auto', 'hopper', 'ada' or 'cdna4', got %r"
                         % (name,))
    _TILE_TABLE = name


def tile_table(device=None):
    """The tile-table class in use: the forced one, else ``"cdna4"`` (the
    MI355X geometry of the HIP kernels). Reference ``slice_ops.py:292-301``."""
    if _TILE_TABLE != "auto":
        return _TILE_TABLE
    return "cdna4"


# --------------------------------------------------------------------------- #
# dot precision
# --------------------------------------------------------------------------- #

_DOT_ENV = os.environ.get("FLASHSLICE_DOT_MODE", "").lower()

# 0 = ieee fp32, 1 = tf32 value dots, 2 = bf16 value dots, 3 = all dots
# bf16, 4 = tf32x3 (reference slice_ops.py:338-343). gfx950 has no xf32
# MFMA: levels 0, 1 and 4 all run the exact fp32 MFMA
# (v_mfma_f32_32x32x2_f32), which is at least as accurate as tf32 / tf32x3.
# Level 2 runs the value dots on bf16 MFMA, level 3 every dot; both only for
# 16-bit inputs (fp32 inputs fall back to level 1, as in the reference).
_DOT_LEVELS = {"": 0, "ieee": 0, "tf32": 1, "bf16v": 2, "bf16": 3, "tf32x3": 4}


def set_dot_mode(mode):
    """'ieee' (default), 'tf32', 'bf16v', 'bf16' or 'tf32x3' -- overrides
    FLASHSLICE_DOT_MODE (reference ``slice_ops.py:346-352``)."""
    global _DOT_ENV
    if mode not in _DOT_LEVELS:
        raise ValueError("dot mode must be one of %s, got %r"
                         % (tuple(k for k in _DOT_LEVELS if k), mode))
    _DOT_ENV = mode


def _dot_mode(t):
    """The dot level baked into an op call (reference ``slice_ops.py:355-359``):
    bf16 levels only for 16-bit inputs, fp32 inputs fall back to tf32 (1)."""
    lvl = _DOT_LEVELS[_DOT_ENV]
    if lvl in (2, 3) and t.dtype == torch.float32:
        return 1
    return lvl


# --------------------------------------------------------------------------- #
# shape contract and routing (reference slice_ops.py:368-444)
# --------------------------------------------------------------------------- #

_D_MAX = 256

_KERNEL_MODES = ("auto", "single-tile", "blocked")
_KERNEL_MODE = os.environ.get("FLASHSLICE_KERNEL_MODE", "").lower() or "auto"


def set_kernel_mode(mode):
    """'auto' (default), 'single-tile' or 'blocked' -- overrides
    FLASHSLICE_KERNEL_MODE. 'auto' calls the single-tile ops wherever
    ``single_tile_dims`` holds and the blocked ops elsewhere; the other two
    force one (for parity and timing runs); 'single-tile' raises on a shape
    it cannot serve rather than silently switching."""
    global _KERNEL_MODE
    if mode not in _KERNEL_MODES:
        raise ValueError("kernel mode must be one of %s, got %r" % (_KERNEL_MODES, mode))
    _KERNEL_MODE = mode


def single_tile_dims(d, g, dv=None):
    """True when the single-tile ops serve (D, G): both powers of two in
    [16, 128] and the value width ``dv`` equal to D (reference
    ``slice_ops.py:386-393``)."""
    if dv is not None and dv != d:
        return False
    return all(16 <= v <= 128 and (v & (v - 1)) == 0 for v in (d, g))


def unsupported_dims(d, g, dv=None):
    """Why the fused ops cannot serve these dims, or None if they can
    (reference ``slice_ops.py:396-420``). ``d`` is the logits width (x_mid,
    weight), ``dv`` the value width (fx_mid, tokens, out; None = d). Only D
    or DV outside [1, 256] and G < 1 are refused."""
    if not 1 <= d <= _D_MAX:
        return ("dim_head=%d is outside the fused kernels' supported range "
                "[1, %d]" % (d, _D_MAX))
    if dv is not None and not 1 <= dv <= _D_MAX:
        return ("value width %d is outside the fused kernels' supported range "
                "[1, %d]" % (dv, _D_MAX))
    if g < 1:
        return "slice_num=%d is not a positive slice count" % g
    return None


def _check_dims(d, g, dv=None):
    why = unsupported_dims(d, g, dv)
    if why:
        raise ValueError("fused_slice: " + why)


def _use_blocked(d, g, dv=None, dot=0, device=None):
    """Route a shape: False = the single-tile ops, True = the blocked ops
    (reference ``slice_ops.py:429-444``)."""
    if _KERNEL_MODE == "blocked":
        return True
    if _KERNEL_MODE == "single-tile":
        if not single_tile_dims(d, g, dv):
            raise ValueError("kernel mode 'single-tile' cannot serve dim_head=%d, "
                             "slice_num=%d, value width %s (powers of two in "
                             "[16, 128], equal widths)" % (d, g, dv))
        return False
    return not single_tile_dims(d, g, dv)


# --------------------------------------------------------------------------- #
# weight / bias layouts (reference slice_ops.py:455-526)
# --------------------------------------------------------------------------- #

def _lead2(t, trailing):
    """(batch, heads) extent of a weight-like tensor's leading dims: 1 where
    a dim is absent (reference ``slice_ops.py:455-458``)."""
    return ((1, 1) + tuple(t.shape[:-trailing]))[-2:]


def _wb_layout(weight, bias, B, H):
    """Element strides (swb, swh, sbb, sbh) of a contiguous weight (.., G, D)
    and bias (.., G) along x_mid's batch and head axes, zero where shared
    (reference ``slice_ops.py:461-478``)."""
    assert weight.is_contiguous() and bias.is_contiguous()
    G, D = weight.shape[-2:]
    Bw, Hw = _lead2(weight, 2)
    Bb, Hb = _lead2(bias, 1)
    for name, got in (("weight", (Bw, Hw)), ("bias", (Bb, Hb))):
        if got[0] not in (1, B) or got[1] not in (1, H):
            raise ValueError("%s has (batch, heads) = %s, x_mid has (%d, %d)"
                             % (name, got, B, H))
    if bias.shape[-1] != G:
        raise ValueError("bias has %d slices, weight %d" % (bias.shape[-1], G))
    return (Hw * G * D if Bw > 1 else 0, G * D if Hw > 1 else 0,
            Hb * G if Bb > 1 else 0, G if Hb > 1 else 0)


def _prep_wb(x_mid, weight, bias):
    """Validate weight (G, D) | (H, G, D) | (B, H, G, D) and bias None | (G,)
    | (H, G) | (B, H, G) against x_mid (B, N, H, D); a None bias becomes
    zeros (G,). Returns (weight, bias, G). Reference ``slice_ops.py:503-526``."""
    B, N, H, D = x_mid.shape
    if weight.dim() not in (2, 3, 4):
        raise ValueError("weight must be (G, D), (H, G, D) or (B, H, G, D), "
                         "got shape %s" % (tuple(weight.shape),))
    G = weight.shape[-2]
    if weight.shape[-1] != D:
        raise ValueError("weight's last dim is %d, x_mid's head width is %d"
                         % (weight.shape[-1], D))
    if bias is None:
        bias = _zero_bias(weight, G)
    elif bias.dim() not in (1, 2, 3) or bias.shape[-1] != G:
        raise ValueError("bias must be (G,), (H, G) or (B, H, G) with G=%d, "
                         "got shape %s" % (G, tuple(bias.shape)))
    for name, t, trailing in (("weight", weight, 2), ("bias", bias, 1)):
        for got, want, axis in zip(tuple(t.shape[:-trailing])[::-1], (H, B),
                                   ("heads", "batch")):
            if got not in (1, want):
                raise ValueError("%s has %d along %s, x_mid has %d"
                                 % (name, got, axis, want))
    return weight, bias, G


# --------------------------------------------------------------------------- #
# the HIP calls (shared with blocked.py)
# --------------------------------------------------------------------------- #

_POINT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _point_dtype(*ts):
    """The one dtype the library reads and writes every point tensor of a
    call in: their common dtype when it is fp32/bf16/fp16, else fp32 (a
    mixed or other-dtype call is served exactly, in fp32)."""
    dts = {t.dtype for t in ts if t is not None}
    if len(dts) == 1 and next(iter(dts)) in _POINT_DTYPES:
        return next(iter(dts))
    return torch.float32


def _as_points(t, dtype):
    """``t`` in ``dtype`` with a unit stride on the last dim (a copy only
    when needed)."""
    if t.dtype != dtype:
        t = t.to(dtype)
    if t.stride(3) != 1:
        t = t.contiguous()
    return t


def _same_device(x_mid, **tensors):
    """Every tensor operand of a call on x_mid's device. The library takes
    raw device pointers: a host tensor handed to a kernel would be read (or
    written) from the GPU and fault it, so it is refused before any launch
    (the reference's Triton launch raises on it too)."""
    dev = x_mid.device
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError("%s is on %s, x_mid on %s: every tensor of a fused call must be "
                             "on x_mid's device" % (name, t.device, dev))


_ZERO_BIAS = {}


def _zero_bias(weight, G):
    """zeros(G) in weight's dtype and device for a None bias, cached per
    (device, dtype, G) outside compiled regions (an allocation less per op
    call); the tensor is only read by the kernels."""
    if torch.compiler.is_compiling():
        return weight.new_zeros(G)
    key = (weight.device, weight.dtype, G)
    z = _ZERO_BIAS.get(key)
    if z is None:
        z = _ZERO_BIAS[key] = weight.new_zeros(G)
    return z


_WS_BYTES = {}


class _Call:
    """The fp32 small operands and the FsSliceParams of one call (holding
    references so the converted tensors outlive the launch)."""

    def __init__(self, x_mid, weight, bias, tau, dv, dot, rows=None):
        B, N, H, D = x_mid.shape
        _same_device(x_mid, weight=weight, bias=bias, tau=tau,
                     row_splits=None if rows is None else rows[0])
        total_rows = 0
        if rows is not None:
            total_rows = N
            # ragged batch (varlen.py): x_mid is the (1, rows, H, D) view of the
            # concatenated samples; rows = (row splits on the device, samples,
            # longest sample)
            B, N = rows[1], rows[2]
        self.device = x_mid.device
        self.weight = weight.detach().to(torch.float32).contiguous()
        self.bias = bias.detach().to(torch.float32).contiguous()
        self.tau = tau.detach().to(torch.float32).contiguous()
        if self.tau.numel() != H:
            raise ValueError("tau must have H=%d elements, got %d" % (H, self.tau.numel()))
        swb, swh, sbb, sbh = _wb_layout(self.weight, self.bias, B, H)
        G = self.weight.shape[-2]
        # kernel mode 'blocked' also forces the G-blocked HIP kernels, so
        # both families can be held to the same gates on any shape
        family = 2 if _KERNEL_MODE == "blocked" else 0
        self.prm = _hip.FsSliceParams(B, N, H, D, dv, G,
                                      self.weight.data_ptr(), swb, swh,
                                      self.bias.data_ptr(), sbb, sbh,
                                      self.tau.data_ptr(), int(dot), family,
                                      None if rows is None else rows[0].data_ptr(),
                                      total_rows)
        self.rows = rows  # keeps the row splits alive across the launch
        self.B, self.N, self.H, self.D, self.DV, self.G = B, N, H, D, dv, G
        self._key = (B, N, H, D, dv, G, swb, swh, sbb, sbh, int(dot), family, rows is not None,
                     total_rows)

    def workspace(self, op):
        """A workspace of fs_workspace_bytes for this op; the size is a
        function of the shape, layout, dot level and family only, so it is
        asked for once per such key."""
        key = (op,) + self._key
        n = _WS_BYTES.get(key)
        if n is None:
            n = _WS_BYTES[key] = _hip.lib().fs_workspace_bytes(op, self.prm)
        if n == 0:
            return None, 0
        return torch.empty(n, dtype=torch.uint8, device=self.device), n

    def stream(self):
        return _hip.stream_of(self.device)


def _small(t, shape, name, device):
    """A small per-slot tensor (tokens, dz_num, ds, stats) as fp32
    contiguous, after checking its shape and device: the library reads it
    through a raw pointer, so a wrong size or a host tensor must be refused
    before the launch."""
    if t.device != device:
        raise ValueError("%s is on %s, x_mid on %s: every tensor of a fused call must be "
                         "on x_mid's device" % (name, t.device, device))
    if tuple(t.shape) != tuple(shape):
        raise ValueError("%s has shape %s, expected %s" % (name, tuple(t.shape), tuple(shape)))
    return t.detach().to(torch.float32).contiguous()


def _stats_arg(stats_in, shape, device):
    """Handed-in statistics as the library reads them; None for none, and
    for the placeholder of statistics a whole-G call never formed
    (``stats_placeholder``: every stride 0), so that a G-blocked kernel
    given it forms its own."""
    if stats_in is None or all(st == 0 for st in stats_in.stride()):
        return None
    return _small(stats_in, shape, "stats", device)


def stats_placeholder(B, H, N, like):
    """A (B, H, 2, N) stand-in that carries no values (zero strides, no
    memory) for the softmax statistics a coupling hands from its first op to
    its second and to the backward when the whole-G kernels serve the shape:
    they form the softmax exactly in each pass and read no statistics."""
    return torch.empty_strided((B, H, 2, N), (0, 0, 0, 0), device=like.device,
                               dtype=torch.float32)


_WHOLE_G = {}


def _whole_g(D, DV, G):
    """True where the whole-G kernels serve a call of this shape (the
    library's ``fs_family``, which depends on D, DV, G and the kernel mode
    only)."""
    family = 2 if _KERNEL_MODE == "blocked" else 0
    key = (int(D), int(DV), int(G), family)
    r = _WHOLE_G.get(key)
    if r is None:
        prm = _hip.FsSliceParams(1, 1, 1, int(D), int(DV), int(G), None, 0, 0, None, 0, 0,
                                 None, 0, family, None, 0)
        r = _WHOLE_G[key] = _hip.lib().fs_family(prm) == 1
    return r


def _check_points(x_mid, t, width, name):
    """A second point tensor of a call: x_mid's (B, N, H), ``width`` and
    device."""
    _same_device(x_mid, **{name: t})
    if t.dim() != 4 or tuple(t.shape[:3]) != tuple(x_mid.shape[:3]) or t.shape[3] != width:
        raise ValueError("%s has shape %s, expected %s" % (
            name, tuple(t.shape), tuple(x_mid.shape[:3]) + (width,)))


def _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot, stats_in=None, want_stats=False,
                   rows=None):
    B, N, H, D = x_mid.shape
    DV = fx_mid.shape[3]
    # statistics: (B, H, 2, N), or (1, H, 2, rows) for a ragged batch's
    # (1, rows, H, D) view of its points
    sshape = (B, H, 2, N)
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, DV, dot, rows)
        B = call.B
        _check_points(x_mid, fx_mid, DV, "fx_mid")
        dt = _point_dtype(x_mid, fx_mid)
        x, fx = _as_points(x_mid, dt), _as_points(fx_mid, dt)
        z_num = torch.empty(B, H, call.G, DV, device=x.device, dtype=torch.float32)
        s = torch.empty(B, H, call.G, device=x.device, dtype=torch.float32)
        st_in = _stats_arg(stats_in, sshape, x.device)
        st_out = (torch.empty(sshape, device=x.device, dtype=torch.float32)
                  if want_stats and st_in is None else None)
        ws, nws = call.workspace(_hip.OP_SLICE_FWD)
        _hip.check(_hip.lib().fs_slice_fwd(
            _hip.points(x, D), _hip.points(fx, DV), call.prm, _hip.ptr(st_in), _hip.ptr(st_out),
            _hip.ptr(z_num), _hip.ptr(s), _hip.ptr(ws), nws, call.stream()))
    return z_num, s, (st_in if st_in is not None else st_out)


def _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot, stats_in=None, want_stats=False,
                     rows=None):
    B, N, H, D = x_mid.shape
    DV = tokens.shape[3]
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, DV, dot, rows)
        dt = _point_dtype(x_mid)
        x = _as_points(x_mid, dt)
        tok = _small(tokens, (call.B, H, call.G, DV), "tokens", x.device)
        out = torch.empty(B, N, H, DV, device=x.device, dtype=dt)
        st_in = _stats_arg(stats_in, (B, H, 2, N), x.device)
        st_out = (torch.empty(B, H, 2, N, device=x.device, dtype=torch.float32)
                  if want_stats and st_in is None else None)
        ws, nws = call.workspace(_hip.OP_DESLICE_FWD)
        _hip.check(_hip.lib().fs_deslice_fwd(
            _hip.points(x, D), call.prm, _hip.ptr(tok), _hip.ptr(st_in), _hip.ptr(st_out),
            _hip.points(out, DV), _hip.ptr(ws), nws, call.stream()))
    if out.dtype != x_mid.dtype:
        out = out.to(x_mid.dtype)
    return out, (st_in if st_in is not None else st_out)


def _grads_out(call, weight, bias, tau, dW, db, dtau):
    """Parameter gradients in the parameter's own shape and dtype
    (reference ``slice_ops.py:497-500``); dtau in tau's dtype."""
    return (dW.reshape(weight.shape).to(weight.dtype),
            db.reshape(bias.shape).to(bias.dtype),
            dtau.to(tau.dtype))


def _param_grad_buffers(call):
    Bw, Hw = _lead2(call.weight, 2)
    Bb, Hb = _lead2(call.bias, 1)
    dev = call.device
    dW = torch.empty(Bw, Hw, call.G, call.D, device=dev, dtype=torch.float32)
    db = torch.empty(Bb, Hb, call.G, device=dev, dtype=torch.float32)
    dtau = torch.empty(call.H, device=dev, dtype=torch.float32)
    return dW, db, dtau


def _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot, stats_in=None,
                   rows=None):
    B, N, H, D = x_mid.shape
    DV = fx_mid.shape[3]
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, DV, dot, rows)
        _check_points(x_mid, fx_mid, DV, "fx_mid")
        dt = _point_dtype(x_mid, fx_mid)
        x, fx = _as_points(x_mid, dt), _as_points(fx_mid, dt)
        dxm = torch.empty_like(x_mid, dtype=dt) if x_mid.stride(3) == 1 else \
            torch.empty(x_mid.shape, device=x.device, dtype=dt)
        dfx = torch.empty_like(fx_mid, dtype=dt) if fx_mid.stride(3) == 1 else \
            torch.empty(fx_mid.shape, device=x.device, dtype=dt)
        dz = _small(dz_num, (call.B, H, call.G, DV), "dz_num", x.device)
        dsv = _small(ds, (call.B, H, call.G), "ds", x.device)
        st_in = _stats_arg(stats_in, (B, H, 2, N), x.device)
        dW, db, dtau = _param_grad_buffers(call)
        ws, nws = call.workspace(_hip.OP_SLICE_BWD)
        _hip.check(_hip.lib().fs_slice_bwd(
            _hip.points(x, D), _hip.points(fx, DV), call.prm, _hip.ptr(st_in), _hip.ptr(dz),
            _hip.ptr(dsv), _hip.points(dxm, D), _hip.points(dfx, DV), _hip.ptr(dW), _hip.ptr(db),
            _hip.ptr(dtau), _hip.ptr(ws), nws, call.stream()))
    if dxm.dtype != x_mid.dtype:
        dxm = dxm.to(x_mid.dtype)
    if dfx.dtype != fx_mid.dtype:
        dfx = dfx.to(fx_mid.dtype)
    return (dxm, dfx) + _grads_out(call, weight, bias, tau, dW, db, dtau)


def _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot, stats_in=None,
                     rows=None):
    B, N, H, D = x_mid.shape
    DV = tokens.shape[3]
    with torch.cuda.device(x_mid.device):
        call = _Call(x_mid, weight, bias, tau, DV, dot, rows)
        B = call.B
        _check_points(x_mid, d_out, DV, "d_out")
        dt = _point_dtype(x_mid, d_out)
        x, do = _as_points(x_mid, dt), _as_points(d_out, dt)
        dxm = torch.empty_like(x_mid, dtype=dt) if x_mid.stride(3) == 1 else \
            torch.empty(x_mid.shape, device=x.device, dtype=dt)
        tok = _small(tokens, (B, H, call.G, DV), "tokens", x.device)
        st_in = _stats_arg(stats_in, (x_mid.shape[0], H, 2, N), x.device)
        dtok = torch.empty(B, H, call.G, DV, device=x.device, dtype=torch.float32)
        dW, db, dtau = _param_grad_buffers(call)
        ws, nws = call.workspace(_hip.OP_DESLICE_BWD)
        _hip.check(_hip.lib().fs_deslice_bwd(
            _hip.points(x, D), call.prm, _hip.ptr(tok), _hip.ptr(st_in), _hip.points(do, DV),
            _hip.points(dxm, D), _hip.ptr(dtok), _hip.ptr(dW), _hip.ptr(db), _hip.ptr(dtau),
            _hip.ptr(ws), nws, call.stream()))
    if dxm.dtype != x_mid.dtype:
        dxm = dxm.to(x_mid.dtype)
    return (dxm, dtok.to(tokens.dtype)) + _grads_out(call, weight, bias, tau, dW, db, dtau)


# --------------------------------------------------------------------------- #
# custom ops (reference slice_ops.py:787-954): opaque to torch.compile,
# autograd- and fake-registered
# --------------------------------------------------------------------------- #

_LIB = torch.library.Library("flashslice", "DEF")
_LIB.define(
    "flash_slice(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
    "Tensor tau, int dot) -> (Tensor, Tensor)")
_LIB.define(
    "flash_slice_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
    "Tensor tau, Tensor dz_num, Tensor ds, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_LIB.define(
    "flash_deslice(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor tokens, int dot) -> Tensor")
_LIB.define(
    "flash_deslice_bwd(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, "
    "Tensor tokens, Tensor d_out, int dot) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")


def _slice_impl(x_mid, fx_mid, weight, bias, tau, dot):
    """flashslice::flash_slice (reference ``_slice_impl``, slice_ops.py:804-819)."""
    z_num, s, _ = _hip_slice_fwd(x_mid, fx_mid, weight, bias, tau, dot)
    return z_num, s


def _slice_bwd_impl(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot):
    """flashslice::flash_slice_bwd (reference slice_ops.py:822-843)."""
    return _hip_slice_bwd(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot)


def _deslice_impl(x_mid, weight, bias, tau, tokens, dot):
    """flashslice::flash_deslice (reference slice_ops.py:846-859)."""
    out, _ = _hip_deslice_fwd(x_mid, weight, bias, tau, tokens, dot)
    return out


def _deslice_bwd_impl(x_mid, weight, bias, tau, tokens, d_out, dot):
    """flashslice::flash_deslice_bwd (reference slice_ops.py:862-885)."""
    return _hip_deslice_bwd(x_mid, weight, bias, tau, tokens, d_out, dot)


_LIB.impl("flash_slice", _slice_impl, "CUDA")
_LIB.impl("flash_slice_bwd", _slice_bwd_impl, "CUDA")
_LIB.impl("flash_deslice", _deslice_impl, "CUDA")
_LIB.impl("flash_deslice_bwd", _deslice_bwd_impl, "CUDA")


@torch.library.register_fake("flashslice::flash_slice")
def _(x_mid, fx_mid, weight, bias, tau, dot):
    B, N, H, D = x_mid.shape
    G = weight.shape[-2]
    return (x_mid.new_empty((B, H, G, fx_mid.shape[3]), dtype=torch.float32),
            x_mid.new_empty((B, H, G), dtype=torch.float32))


@torch.library.register_fake("flashslice::flash_slice_bwd")
def _(x_mid, fx_mid, weight, bias, tau, dz_num, ds, dot):
    return (torch.empty_like(x_mid), torch.empty_like(fx_mid),
            torch.empty_like(weight), torch.empty_like(bias),
            torch.empty_like(tau))


@torch.library.register_fake("flashslice::flash_deslice")
def _(x_mid, weight, bias, tau, tokens, dot):
    B, N, H, D = x_mid.shape
    return x_mid.new_empty((B, N, H, tokens.shape[3]))


@torch.library.register_fake("flashslice::flash_deslice_bwd")
def _(x_mid, weight, bias, tau, tokens, d_out, dot):
    return (torch.empty_like(x_mid), torch.empty_like(tokens),
            torch.empty_like(weight), torch.empty_like(bias),
            torch.empty_like(tau))


def _slice_setup(ctx, inputs, output):
    x_mid, fx_mid, weight, bias, tau, dot = inputs
    ctx.save_for_backward(x_mid, fx_mid, weight, bias, tau)
    ctx.dot = dot


def _slice_grad(ctx, dz_num, ds):
    """Reference ``_slice_grad`` (slice_ops.py:928-935): saves inputs, never
    w; a None ds becomes zeros; no gradient for ``dot``."""
    x_mid, fx_mid, weight, bias, tau = ctx.saved_tensors
    if dz_num is None:
        dz_num = torch.zeros(x_mid.shape[0], x_mid.shape[2], weight.shape[-2],
                             fx_mid.shape[3], device=x_mid.device, dtype=torch.float32)
    if ds is None:
        ds = torch.zeros(dz_num.shape[:-1], device=dz_num.device, dtype=torch.float32)
    dxm, dfx, dw, db, dtau = torch.ops.flashslice.flash_slice_bwd(
        x_mid, fx_mid, weight, bias, tau, dz_num, ds, ctx.dot)
    return dxm, dfx, dw, db, dtau, None


def _deslice_setup(ctx, inputs, output):
    x_mid, weight, bias, tau, tokens, dot = inputs
    ctx.save_for_backward(x_mid, weight, bias, tau, tokens)
    ctx.dot = dot


def _deslice_grad(ctx, d_out):
    """Reference ``_deslice_grad`` (slice_ops.py:944-948)."""
    x_mid, weight, bias, tau, tokens = ctx.saved_tensors
    dxm, dtok, dw, db, dtau = torch.ops.flashslice.flash_deslice_bwd(
        x_mid, weight, bias, tau, tokens, d_out, ctx.dot)
    return dxm, dw, db, dtau, dtok, None


torch.library.register_autograd("flashslice::flash_slice", _slice_grad,
                                setup_context=_slice_setup)
torch.library.register_autograd("flashslice::flash_deslice", _deslice_grad,
                                setup_context=_deslice_setup)


# --------------------------------------------------------------------------- #
# public API (reference slice_ops.py:961-1022)
# --------------------------------------------------------------------------- #

def fused_slice(x_mid, fx_mid, weight, bias, tau, return_stats=False, stats=None):
    """x_mid (B, N, H, D); fx_mid (B, N, H, DV); weight (G, D), (H, G, D) or
    (B, H, G, D); bias None, (G,), (H, G) or (B, H, G); tau (H,). Returns
    fp32 z_num (B, H, G, DV) and s (B, H, G); normalise outside as
    ``z_num / (s + eps)[..., None]``.

    ``stats`` are the per-point softmax statistics of these very logits from
    an op that ran before on the same x_mid, weight, bias and tau (a tied
    ``fused_deslice(..., return_stats=True)``). With ``return_stats=True`` a
    third value is returned: the (B, H, 2, N) fp32 statistics (row max and
    sum of exponentials, detached) on the blocked path, None on the
    single-tile path. Either value is accepted by either op (reference
    ``slice_ops.py:961-996``)."""
    weight, bias, G = _prep_wb(x_mid, weight, bias)
    D, DV = x_mid.shape[3], fx_mid.shape[3]
    _check_dims(D, G, DV)
    dot = _dot_mode(x_mid)
    if _use_blocked(D, G, DV, dot, x_mid.device):
        z_num, s, st = torch.ops.flashslice.slice_blk(
            x_mid, fx_mid, weight, bias, tau, stats, dot)
        return (z_num, s, st.detach()) if return_stats else (z_num, s)
    z_num, s = torch.ops.flashslice.flash_slice(x_mid, fx_mid, weight, bias, tau, dot)
    return (z_num, s, None) if return_stats else (z_num, s)


def fused_deslice(x_mid, weight, bias, tau, tokens, stats=None, return_stats=False):
    """tokens (B, H, G, DV). Returns out (B, N, H, DV) in x_mid's dtype, the
    layout ``to_out`` expects after a reshape; weight and bias take the
    shapes ``fused_slice`` documents. ``stats`` from a tied
    ``fused_slice(..., return_stats=True)`` skip recomputing them; with
    ``return_stats=True`` returns ``(out, stats)`` (stats None on the
    single-tile path). Reference ``slice_ops.py:999-1022``."""
    weight, bias, G = _prep_wb(x_mid, weight, bias)
    D, DV = x_mid.shape[3], tokens.shape[3]
    _check_dims(D, G, DV)
    dot = _dot_mode(x_mid)
    if _use_blocked(D, G, DV, dot, x_mid.device):
        out, st = torch.ops.flashslice.deslice_blk(x_mid, weight, bias, tau, tokens, stats, dot)
        return (out, st.detach()) if return_stats else out
    out = torch.ops.flashslice.flash_deslice(x_mid, weight, bias, tau, tokens, dot)
    return (out, None) if return_stats else out
