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


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class _LayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        C = x.shape[-1]
        rows = x.numel() // C
        y = torch.empty_like(x)
        mean = torch.empty(rows, device=x.device, dtype=torch.float32)
        rstd = torch.empty_like(mean)
        _hip.check(_hip.lib().fs_layernorm_fwd(
            _ptr(x), _ptr(weight), _ptr(bias), _ptr(y), _ptr(mean), _ptr(rstd), rows, C,
            float(eps), _stream()))
        ctx.save_for_backward(x, weight, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight, mean, rstd = ctx.saved_tensors
        gy = gy.contiguous()
        C = x.shape[-1]
        rows = x.numel() // C
        dx = torch.empty_like(x)
        dw = torch.empty_like(weight)
        db = torch.empty_like(weight)
        nws = _hip.lib().fs_layernorm_workspace_bytes(rows, C)
        ws = torch.empty(nws, device=x.device, dtype=torch.uint8)
        _hip.check(_hip.lib().fs_layernorm_bwd(
            _ptr(gy), _ptr(x), _ptr(weight), _ptr(mean), _ptr(rstd), _ptr(dx), _ptr(dw),
            _ptr(db), _ptr(ws), nws, rows, C, _stream()))
        return dx, dw, db, None


class PointLayerNorm(nn.LayerNorm):
    """``nn.LayerNorm`` whose large fp32 GPU rows run on the HIP kernels."""

    def _hip_ok(self, x):
        C = x.shape[-1] if x.dim() else 0
        return (x.is_cuda and x.dtype == torch.float32 and self.elementwise_affine
                and self.bias is not None and self.weight.dtype == torch.float32
                and len(self.normalized_shape) == 1 and C == self.normalized_shape[0]
                and C % 4 == 0 and 4 <= C <= 2048 and x.numel() // C >= MIN_ROWS
                and not torch.is_autocast_enabled())

    def forward(self, x):
        if self._hip_ok(x):
            return _LayerNormFn.apply(x.contiguous(), self.weight.contiguous(),
                                      self.bias.contiguous(), self.eps)
        return super().forward(x)
