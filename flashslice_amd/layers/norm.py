"""LayerNorm of the point streams on the HIP kernels (``fs_layernorm_fwd`` /
``fs_layernorm_bwd``, include/flashslice_layer.h).

The Transolver blocks normalise every point's features before the
physics-attention and the MLP (reference
``flashslice/models/transolver.py:51-63``, ``torch.nn.LayerNorm``). At
config 5 each such LayerNorm moves 2 GB forward and 4 GB backward, and
torch's kernels for it ran at ~1.9 TB/s on MI355X. ``PointLayerNorm`` keeps
``nn.LayerNorm``'s parameters, defaults and state dict and routes fp32 CUDA
inputs with an elementwise affine over one trailing axis (a multiple of 4,
at most 2048 wide, at least ``MIN_ROWS`` rows) to the HIP kernels; every
other case takes ``nn.LayerNorm``'s own path.
"""

import ctypes

import torch
import torch.nn as nn

from ..kernels import _hip

MIN_ROWS = 65536

# Custom operators (own namespace; the reference defines none for this), so
# that torch.compile keeps them as single opaque nodes: the CUDA-key
# implementations call the C entry points, the fakes give shapes and dtypes.
_LIB = torch.library.Library("flashslice_layer", "DEF")
_LIB.define("layer_norm(Tensor x, Tensor weight, Tensor bias, float eps) "
            "-> (Tensor, Tensor, Tensor)")
_LIB.define("layer_norm_bwd(Tensor dy, Tensor x, Tensor weight, Tensor mean, Tensor rstd) "
            "-> (Tensor, Tensor, Tensor)")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ln_impl(x, weight, bias, eps):
    """x (..., C) contiguous fp32 -> y, mean (rows,), rstd (rows,)."""
    C = x.shape[-1]
    rows = x.numel() // C
    y = torch.empty_like(x)
    mean = torch.empty(rows, device=x.device, dtype=torch.float32)
    rstd = torch.empty_like(mean)
    _hip.check(_hip.lib().fs_layernorm_fwd(
        _ptr(x), _ptr(weight), _ptr(bias), _ptr(y), _ptr(mean), _ptr(rstd), rows, C,
        float(eps), _stream()))
    return y, mean, rstd


def _ln_bwd_impl(dy, x, weight, mean, rstd):
    C = x.shape[-1]
    rows = x.numel() // C
    dx = torch.empty_like(x)
    dw = torch.empty_like(weight)
    db = torch.empty_like(weight)
    nws = _hip.lib().fs_layernorm_workspace_bytes(rows, C)
    ws = torch.empty(nws, device=x.device, dtype=torch.uint8)
    _hip.check(_hip.lib().fs_layernorm_bwd(
        _ptr(dy), _ptr(x), _ptr(weight), _ptr(mean), _ptr(rstd), _ptr(dx), _ptr(dw), _ptr(db),
        _ptr(ws), nws, rows, C, _stream()))
    return dx, dw, db


_LIB.impl("layer_norm", _ln_impl, "CUDA")
_LIB.impl("layer_norm_bwd", _ln_bwd_impl, "CUDA")


@torch.library.register_fake("flashslice_layer::layer_norm")
def _(x, weight, bias, eps):
    rows = x.numel() // x.shape[-1]
    return (torch.empty_like(x), x.new_empty(rows, dtype=torch.float32),
            x.new_empty(rows, dtype=torch.float32))


@torch.library.register_fake("flashslice_layer::layer_norm_bwd")
def _(dy, x, weight, mean, rstd):
    return torch.empty_like(x), torch.empty_like(weight), torch.empty_like(weight)


def _ln_setup(ctx, inputs, output):
    x, weight, _, _ = inputs
    _, mean, rstd = output
    ctx.save_for_backward(x, weight, mean, rstd)


def _ln_grad(ctx, gy, gmean, grstd):
    x, weight, mean, rstd = ctx.saved_tensors
    gy = gy.contiguous()
    if gy.data_ptr() % 16:
        gy = gy.clone()  # the kernels read rows as 16-byte words
    dx, dw, db = torch.ops.flashslice_layer.layer_norm_bwd(gy, x, weight, mean, rstd)
    return dx, dw, db, None


torch.library.register_autograd("flashslice_layer::layer_norm", _ln_grad,
                                setup_context=_ln_setup)


class PointLayerNorm(nn.LayerNorm):
    """``nn.LayerNorm`` whose large fp32 GPU rows run on the HIP kernels."""

    def _hip_ok(self, x):
        C = x.shape[-1] if x.dim() else 0
        return (x.is_cuda and x.dtype == torch.float32 and self.elementwise_affine
                and self.bias is not None and self.weight.dtype == torch.float32
                and len(self.normalized_shape) == 1 and C == self.normalized_shape[0]
                and C % 4 == 0 and 4 <= C <= 2048 and x.numel() // C >= MIN_ROWS
                and not torch.is_autocast_enabled()
                # the kernels read rows as 16-byte words: a view whose storage
                # offset is not a multiple of 4 floats takes nn.LayerNorm
                and (not x.is_contiguous() or x.data_ptr() % 16 == 0))

    def forward(self, x):
        if self._hip_ok(x):
            y, _, _ = torch.ops.flashslice_layer.layer_norm(
                x.contiguous(), self.weight.contiguous(), self.bias.contiguous(), self.eps)
            return y
        return super().forward(x)
