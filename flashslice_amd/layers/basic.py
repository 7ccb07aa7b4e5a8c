"""Pointwise MLP of the Transolver blocks (a caller of the hot path, not part
of it; reference ``flashslice/layers/basic.py:28-53``), and the per-point
Linear with split-K weight gradients that the callers use.

Module and parameter names are the reference's (``linear_pre``,
``linears``, ``linear_post``), so state dicts interchange with models built
from the reference package.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

# Activation factories by the reference's names (``basic.py:17-26``). The
# reference stores an *instance* for "leaky_relu", which its MLP then calls
# with no input; here every entry is a zero-argument factory, so "leaky_relu"
# builds LeakyReLU(0.1) like the others.
ACTIVATION = {
    "gelu": nn.GELU,
    "tanh": nn.Tanh,
    "sigmoid": nn.Sigmoid,
    "relu": nn.ReLU,
    "leaky_relu": lambda: nn.LeakyReLU(0.1),
    "softplus": nn.Softplus,
    "ELU": nn.ELU,
    "silu": nn.SiLU,
}


# Split-K weight gradients of the per-point Linears. A point stream is a
# (M, in) x (M, out) product with M in the millions and a 256 x 256 or
# 256 x 512 result: hipBLASLt's single GEMM for it covers the result with a
# few dozen tiles and ran at 60-75 TFLOP/s on MI355X; as a batched product
# over SPLIT_K chunks of the points plus a fixed-order sum of the chunk
# results it runs at ~150 TFLOP/s (95 % of the fp32 matrix peak).
SPLIT_K = 64
SPLIT_K_MIN_ROWS = 65536


def _split_k_wgrad(g2, x2):
    """g2^T x2 for (M, out) and (M, in) point streams: a batched product over
    SPLIT_K point chunks plus a fixed-order sum of the chunk results."""
    M, n_out = g2.shape
    n_in = x2.shape[1]
    Mk = (M // SPLIT_K) * SPLIT_K
    gw = torch.bmm(g2[:Mk].view(SPLIT_K, Mk // SPLIT_K, n_out).transpose(1, 2),
                   x2[:Mk].view(SPLIT_K, Mk // SPLIT_K, n_in)).sum(0)
    if Mk < M:
        gw = gw + g2[Mk:].t() @ x2[Mk:]
    return gw


class _PointLinearFn(torch.autograd.Function):
    """y = x W^T + b; the backward forms dW over SPLIT_K point chunks."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, gy):
        x, weight = ctx.saved_tensors
        n_in, n_out = weight.shape[1], weight.shape[0]
        g2 = gy.reshape(-1, n_out)
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            gx = (g2 @ weight).view(x.shape)
        if ctx.needs_input_grad[1]:
            gw = _split_k_wgrad(g2, x.reshape(-1, n_in))
        if ctx.has_bias and ctx.needs_input_grad[2]:
            gb = g2.sum(0)
        return gx, gw, gb


class _PointLinearPairFn(torch.autograd.Function):
    """(x W1^T + b1, x W2^T + b2), two projections of one point stream, as
    one GEMM against the stacked weights; the outputs are the two column
    halves of its result (views: the kernels downstream read strided rows).
    The backward forms dx = g1 W1 + g2 W2 as one product and one
    accumulating product (the second GEMM adds into the first's result, so
    the two input gradients are never summed in a separate pass) and each
    weight's gradient split-K."""

    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2):
        ctx.save_for_backward(x, w1, w2)
        ctx.n1 = w1.shape[0]
        ctx.has_bias = (b1 is not None, b2 is not None)
        bias = None
        if b1 is not None or b2 is not None:
            bias = torch.cat([b1 if b1 is not None else w1.new_zeros(w1.shape[0]),
                              b2 if b2 is not None else w2.new_zeros(w2.shape[0])])
        y = F.linear(x, torch.cat([w1, w2]), bias)
        return y[..., :ctx.n1], y[..., ctx.n1:]

    @staticmethod
    def backward(ctx, g1, g2):
        x, w1, w2 = ctx.saved_tensors
        n_in = w1.shape[1]
        x2 = x.reshape(-1, n_in)
        g1 = (torch.zeros(x2.shape[0], w1.shape[0], device=x.device, dtype=x.dtype)
              if g1 is None else g1.reshape(-1, w1.shape[0]))
        g2 = (torch.zeros(x2.shape[0], w2.shape[0], device=x.device, dtype=x.dtype)
              if g2 is None else g2.reshape(-1, w2.shape[0]))
        gx = gw1 = gb1 = gw2 = gb2 = None
        if ctx.needs_input_grad[0]:
            gx = torch.addmm(g1 @ w1, g2, w2).view(x.shape)
        if ctx.needs_input_grad[1]:
            gw1 = _split_k_wgrad(g1, x2)
        if ctx.has_bias[0] and ctx.needs_input_grad[2]:
            gb1 = g1.sum(0)
        if ctx.needs_input_grad[3]:
            gw2 = _split_k_wgrad(g2, x2)
        if ctx.has_bias[1] and ctx.needs_input_grad[4]:
            gb2 = g2.sum(0)
        return gx, gw1, gb1, gw2, gb2


class PointLinear(nn.Linear):
    """nn.Linear (same parameters and state dict) whose weight gradient is
    formed split-K for fp32 point streams on the GPU (>= SPLIT_K_MIN_ROWS
    rows); anything else takes nn.Linear's own path."""

    def point_stream(self, x):
        return (x.is_cuda and x.dtype == torch.float32 and self.weight.dtype == torch.float32
                and torch.is_grad_enabled() and x.numel() >= SPLIT_K_MIN_ROWS * self.in_features
                and not torch.is_autocast_enabled())

    def forward(self, x):
        if self.point_stream(x):
            x = x.contiguous()
            return _PointLinearFn.apply(x, self.weight, self.bias)
        return super().forward(x)


def point_linear_pair(x, lin1, lin2):
    """(lin1(x), lin2(x)) for two PointLinears on the same input: one GEMM
    against the stacked weights on a GPU point stream (_PointLinearPairFn;
    the outputs are column halves of one result), else the two modules."""
    if lin1.point_stream(x) and lin2.point_stream(x) and lin1.in_features == lin2.in_features:
        return _PointLinearPairFn.apply(x.contiguous(), lin1.weight, lin1.bias, lin2.weight,
                                        lin2.bias)
    return lin1(x), lin2(x)


class MLP(nn.Module):
    """Linear -> act, ``n_layers`` x (Linear -> act, with a residual when
    ``res``), Linear. Unknown activations raise ``NotImplementedError``."""

    def __init__(self, n_input, n_hidden, n_output, n_layers=1, act="gelu", res=True):
        super().__init__()
        if act not in ACTIVATION:
            raise NotImplementedError("unknown activation %r" % (act,))
        make = ACTIVATION[act]
        self.n_input, self.n_hidden, self.n_output = n_input, n_hidden, n_output
        self.n_layers, self.res = n_layers, res
        # registration order (pre, post, hidden) fixes the order of the init
        # draws: the reference's, so one seed gives the same weights
        self.linear_pre = nn.Sequential(PointLinear(n_input, n_hidden), make())
        self.linear_post = PointLinear(n_hidden, n_output)
        self.linears = nn.ModuleList(
            nn.Sequential(PointLinear(n_hidden, n_hidden), make()) for _ in range(n_layers))

    def forward(self, x):
        h = self.linear_pre(x)
        for block in self.linears:
            h = block(h) + h if self.res else block(h)
        return self.linear_post(h)
