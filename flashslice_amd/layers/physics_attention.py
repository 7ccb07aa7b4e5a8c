"""Physics-attention on irregular meshes: the layer around the slice/deslice
path (reference ``flashslice/layers/physics_attention.py:28-181``).

One layer per head h: project the points twice (``in_project_x`` gives the
logits input x_mid, ``in_project_fx`` the values fx_mid), slice the points
into G tokens, mix the tokens with a small softmax attention, deslice the
tokens back onto the points, project out (``to_out``).

``use_fused_slice=True`` runs slice and deslice through the HIP operators of
``flashslice_amd.kernels``: x_mid and fx_mid go to the kernels as (B, N, H, D)
views of the Linear outputs (no permuted copies); when the deslice shares
the slice's projection the two run as one ``fused_coupling``, whose
backward is one merged pass over the points; the
(B, H, N, G) membership tensor is never formed -- on the eager route it is
formed and kept for the backward (2 GB per layer at N = 2e6, H = 8, G = 32).
The fused route has no CPU implementation: on CPU tensors its operators
raise. The eager route is the reference's formulation (``:138-181``) as
batched matrix products.

Constructor arguments, flags and parameter names are the reference's, so
state dicts interchange between the two routes and with the reference's
models.
"""

import logging

import torch
import torch.nn as nn

from ..kernels.coupling import fused_coupling
from ..kernels.slice_ops import fused_deslice, fused_slice, unsupported_dims
from .basic import PointLinear, point_linear_pair

logger = logging.getLogger(__name__)

#: token normaliser of z_num / (s + eps) (reference ``physics_attention.py:112``)
TOKEN_EPS = 1e-5


class Physics_Attention_Irregular_Mesh(nn.Module):  # noqa: N801 (reference name)
    """Physics-attention for point clouds.

    dim: model width C; heads, dim_head: H and D; slice_num: G per head.
    Flags (reference ``physics_attention.py:30-38``): ``untied_deslice`` --
    the deslice has its own projection and temperature; ``no_token_attention``
    -- tokens pass through ``to_v`` only; ``slice_dim_head`` -- width of the
    token attention (``slice_down`` maps back to dim_head). ``shapelist`` is
    accepted and unused (structured meshes are not served).

    ``use_fused_slice``: an implementation switch, same outputs. Dims the
    fused operators refuse (``unsupported_dims``: D outside [1, 256]) fall
    back to the eager route with a warning, recorded in
    ``fused_slice_fallback``.
    """

    def __init__(self, dim, heads=8, dim_head=64, dropout=0., slice_num=64, shapelist=None,
                 untied_deslice=False, no_token_attention=False, slice_dim_head=None,
                 use_fused_slice=False):
        super().__init__()
        del shapelist
        self.use_fused_slice = bool(use_fused_slice)
        self.fused_slice_fallback = None
        if self.use_fused_slice:
            why = unsupported_dims(dim_head, slice_num)
            if why:
                logger.warning("use_fused_slice=True but %s; this layer runs the eager "
                               "slice/deslice (same outputs).", why)
                self.use_fused_slice = False
                self.fused_slice_fallback = why
        inner = heads * dim_head
        self.heads, self.dim_head = heads, dim_head
        self.slice_dim_head = dim_head if slice_dim_head is None else slice_dim_head
        self.scale = self.slice_dim_head ** -0.5
        self.untied_deslice = untied_deslice
        self.no_token_attention = no_token_attention
        self.softmax = nn.Softmax(dim=-1)
        self.dropout = nn.Dropout(dropout)
        self.temperature = nn.Parameter(torch.full((1, heads, 1, 1), 0.5))
        self.in_project_x = PointLinear(dim, inner)
        self.in_project_fx = PointLinear(dim, inner)
        self.in_project_slice = nn.Linear(dim_head, slice_num)
        nn.init.orthogonal_(self.in_project_slice.weight)
        if untied_deslice:
            self.deslice_temperature = nn.Parameter(torch.full((1, heads, 1, 1), 0.5))
            self.in_project_deslice = nn.Linear(dim_head, slice_num)
            nn.init.orthogonal_(self.in_project_deslice.weight)
        sd = self.slice_dim_head
        self.to_q = nn.Linear(dim_head, sd, bias=False)
        self.to_k = nn.Linear(dim_head, sd, bias=False)
        self.to_v = nn.Linear(dim_head, sd, bias=False)
        self.slice_down = nn.Identity() if sd == dim_head else nn.Linear(sd, dim_head, bias=False)
        self.to_out = nn.Sequential(PointLinear(inner, dim), nn.Dropout(dropout))

    # tokens (B, H, G, dim_head) -> mixed tokens (B, H, G, dim_head)
    def _mix_tokens(self, tokens):
        if self.no_token_attention:
            return self.slice_down(self.to_v(tokens))
        q, k, v = self.to_q(tokens), self.to_k(tokens), self.to_v(tokens)
        attn = self.softmax(torch.matmul(q, k.transpose(-1, -2).contiguous()) * self.scale)
        return self.slice_down(torch.matmul(self.dropout(attn), v))

    def _forward_fused(self, x):
        B, N, _ = x.shape
        H, D = self.heads, self.dim_head
        # both projections as one GEMM: x_mid and fx_mid are the column
        # halves of its (B, N, 2 H D) result, read through their strides
        xm, fm = point_linear_pair(x, self.in_project_x, self.in_project_fx)
        x_mid = xm.view(B, N, H, D)
        fx_mid = fm.view(B, N, H, D)
        tau = self.temperature.view(H)
        W, b = self.in_project_slice.weight, self.in_project_slice.bias
        if self.untied_deslice:
            z_num, s = fused_slice(x_mid, fx_mid, W, b, tau)
            tokens = self._mix_tokens(z_num / (s + TOKEN_EPS).unsqueeze(-1))
            out = fused_deslice(x_mid, self.in_project_deslice.weight,
                                self.in_project_deslice.bias,
                                self.deslice_temperature.view(H), tokens)
        else:
            # slice and deslice on one x_mid, W, b, tau: one coupling, whose
            # backward is one merged pass (the deslice's dx, dW, db, dtau
            # formed in the slice's backward) and no autograd sum of two dx
            c = fused_coupling(x_mid, W, b, tau)
            z_num, s = c.slice(fx_mid)
            tokens = self._mix_tokens(z_num / (s + TOKEN_EPS).unsqueeze(-1))
            out = c.deslice(tokens)
        return self.to_out(out.reshape(B, N, H * D)), None

    def forward(self, x, slice_weights_in=None):
        """x (B, N, dim) -> (out (B, N, dim), slice weights (B, H, N, G) or
        None on the fused route). ``slice_weights_in``: externally given
        slice weights (eager route only)."""
        if self.use_fused_slice:
            if slice_weights_in is not None:
                raise ValueError("use_fused_slice cannot consume externally provided "
                                 "slice weights")
            return self._forward_fused(x)
        B, N, _ = x.shape
        H, D = self.heads, self.dim_head
        fx_mid = self.in_project_fx(x).view(B, N, H, D)
        x_mid = None
        if slice_weights_in is None or self.untied_deslice:
            x_mid = self.in_project_x(x).view(B, N, H, D).transpose(1, 2)  # B H N D
        if slice_weights_in is None:
            w = self.softmax(self.in_project_slice(x_mid) / self.temperature)  # B H N G
        else:
            w = slice_weights_in
        # batched products with contiguous right operands (bmm on a transposed
        # right operand has faulted on this part in bf16)
        z_num = torch.matmul(w.transpose(-1, -2), fx_mid.transpose(1, 2).contiguous())
        tokens = self._mix_tokens(z_num / (w.sum(2) + TOKEN_EPS).unsqueeze(-1))
        if self.untied_deslice:
            wd = self.softmax(self.in_project_deslice(x_mid) / self.deslice_temperature)
        else:
            wd = w
        out = torch.matmul(wd, tokens.contiguous()).transpose(1, 2).reshape(B, N, H * D)
        return self.to_out(out), w
