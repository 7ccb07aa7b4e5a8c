"""Transolver on unstructured point clouds: the model that calls the
slice/deslice path once per layer (reference
``flashslice/models/transolver.py:41-215``).

Blocks are pre-LayerNorm residual pairs -- physics-attention, then a
pointwise MLP -- over a per-point embedding of the coordinates and inputs;
the last block ends in a LayerNorm and a Linear head. The ablation flags of
the reference are kept (at most one at a time): ``no_token_attention``,
``untie_slice_weights``, ``share_slice_across_layers`` (slice weights of the
first layer reused by all), ``slice_once`` (one slice, a transformer over the
G tokens, one deslice), ``mlp_only``. ``use_fused_slice`` routes every
layer's slice/deslice through the HIP operators; the two flags that need the
slice weights themselves (``share_slice_across_layers``, ``slice_once``)
refuse it. Constructor arguments and parameter names are the reference's,
so state dicts interchange.
"""

from typing import Optional

import torch
import torch.nn as nn
from torch.nn.init import trunc_normal_

from ..layers.basic import MLP, PointLinear
from ..layers.norm import PointLayerNorm
from ..layers.physics_attention import TOKEN_EPS, Physics_Attention_Irregular_Mesh


class TransolverBlock(nn.Module):
    """x + Attn(ln_1 x), then + mlp(ln_2 x); the last block maps through
    ln_3 and mlp2 to ``out_dim``. Returns (x, slice weights or None)."""

    def __init__(self, num_heads, hidden_dim, dropout, act="gelu", mlp_ratio=4,
                 last_layer=False, out_dim=1, slice_num=32, untied_deslice=False,
                 no_token_attention=False, mlp_only=False, dim_head=None,
                 slice_dim_head=None, use_fused_slice=False):
        super().__init__()
        self.last_layer, self.mlp_only = last_layer, mlp_only
        self.ln_1 = PointLayerNorm(hidden_dim)
        if not mlp_only:
            self.Attn = Physics_Attention_Irregular_Mesh(
                hidden_dim, heads=num_heads,
                dim_head=hidden_dim // num_heads if dim_head is None else dim_head,
                dropout=dropout, slice_num=slice_num, untied_deslice=untied_deslice,
                no_token_attention=no_token_attention, slice_dim_head=slice_dim_head,
                use_fused_slice=use_fused_slice)
        self.ln_2 = PointLayerNorm(hidden_dim)
        self.mlp = MLP(hidden_dim, hidden_dim * mlp_ratio, hidden_dim, n_layers=0, res=False,
                       act=act)
        if last_layer:
            self.ln_3 = PointLayerNorm(hidden_dim)
            self.mlp2 = PointLinear(hidden_dim, out_dim)

    def forward(self, fx, slice_weights_in=None):
        weights = None
        if not self.mlp_only:
            a, weights = self.Attn(self.ln_1(fx), slice_weights_in=slice_weights_in)
            fx = fx + a
        fx = fx + self.mlp(self.ln_2(fx))
        if self.last_layer:
            fx = self.mlp2(self.ln_3(fx))
        return fx, weights


class TokenTransformerBlock(nn.Module):
    """Pre-LN transformer block over the G slice tokens (``slice_once``)."""

    def __init__(self, num_heads, hidden_dim, dropout, act="gelu", mlp_ratio=4):
        super().__init__()
        self.ln_1 = nn.LayerNorm(hidden_dim)
        self.attn = nn.MultiheadAttention(hidden_dim, num_heads, dropout=dropout,
                                          batch_first=True)
        self.ln_2 = nn.LayerNorm(hidden_dim)
        self.mlp = MLP(hidden_dim, hidden_dim * mlp_ratio, hidden_dim, n_layers=0, res=False,
                       act=act)

    def forward(self, tokens):
        h = self.ln_1(tokens)
        tokens = tokens + self.attn(h, h, h, need_weights=False)[0]
        return tokens + self.mlp(self.ln_2(tokens))


class Transolver(nn.Module):
    """``model(x, fx)``: coordinates x (B, N, space_dim), per-point inputs fx
    (B, N, fun_dim) or None -> (B, N, out_dim). ``slice_num`` is G per head;
    ``dim_head`` defaults to n_hidden // n_heads; ``slice_dim_head`` is the
    token attention's width (default dim_head).

    ``use_fused_slice`` reports the effective state: False when any layer
    fell back to the eager route (its ``Attn.fused_slice_fallback`` says why).
    """

    def __init__(self, space_dim=3, fun_dim=1, out_dim=1, n_hidden=256, n_heads=8,
                 n_layers=8, slice_num=32, mlp_ratio=2, dropout=0.0, act="gelu",
                 dim_head: Optional[int] = None, slice_dim_head: Optional[int] = None,
                 untie_slice_weights=False, share_slice_across_layers=False,
                 slice_once=False, no_token_attention=False, mlp_only=False,
                 use_fused_slice=False):
        super().__init__()
        flags = (untie_slice_weights, share_slice_across_layers, slice_once,
                 no_token_attention, mlp_only)
        if sum(bool(f) for f in flags) > 1:
            raise ValueError("At most one ablation flag may be enabled at a time.")
        if use_fused_slice and (share_slice_across_layers or slice_once):
            raise ValueError("use_fused_slice is incompatible with share_slice_across_layers "
                             "and slice_once: both need the slice weights, which the fused "
                             "operators never form.")
        self.n_hidden = n_hidden
        self.untied_deslice = untie_slice_weights
        self.share_slice_across_layers = share_slice_across_layers
        self.slice_once = slice_once
        self.no_token_attention = no_token_attention
        self.mlp_only = mlp_only
        self.use_fused_slice = use_fused_slice
        self.preprocess = MLP(fun_dim + space_dim, n_hidden * 2, n_hidden, n_layers=0,
                              res=False, act=act)
        if slice_once:
            self.slice_proj = nn.Linear(n_hidden, slice_num)
            self.slice_temperature = nn.Parameter(torch.tensor(0.5))
            self.token_blocks = nn.ModuleList(
                TokenTransformerBlock(n_heads, n_hidden, dropout, act=act, mlp_ratio=mlp_ratio)
                for _ in range(n_layers))
            self.out_norm = nn.LayerNorm(n_hidden)
            self.out_head = nn.Linear(n_hidden, out_dim)
        else:
            self.blocks = nn.ModuleList(
                TransolverBlock(n_heads, n_hidden, dropout, act=act, mlp_ratio=mlp_ratio,
                                last_layer=i == n_layers - 1, out_dim=out_dim,
                                slice_num=slice_num, untied_deslice=untie_slice_weights,
                                no_token_attention=no_token_attention, mlp_only=mlp_only,
                                dim_head=dim_head, slice_dim_head=slice_dim_head,
                                use_fused_slice=use_fused_slice)
                for i in range(n_layers))
            if use_fused_slice and any(
                    getattr(getattr(b, "Attn", None), "fused_slice_fallback", None)
                    for b in self.blocks):
                self.use_fused_slice = False
        self.placeholder = nn.Parameter(torch.rand(n_hidden) / n_hidden)
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(m):
        """Linear: truncated normal (std 0.02), zero bias; LayerNorm: 1, 0
        (reference ``transolver.py:174-182``; applied after construction, so
        it also replaces the slice projections' orthogonal start)."""
        if isinstance(m, nn.Linear):
            trunc_normal_(m.weight, std=0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, (nn.LayerNorm, nn.BatchNorm1d)):
            nn.init.ones_(m.weight)
            nn.init.zeros_(m.bias)

    def _slice_once_forward(self, fx):
        w = torch.softmax(self.slice_proj(fx) / self.slice_temperature, dim=-1)  # B N G
        tokens = torch.matmul(w.transpose(1, 2), fx.contiguous())
        tokens = tokens / (w.sum(1) + TOKEN_EPS).unsqueeze(-1)
        for block in self.token_blocks:
            tokens = block(tokens)
        out = torch.matmul(w, tokens.contiguous()) + fx
        return self.out_head(self.out_norm(out))

    def forward(self, x, fx=None):
        h = self.preprocess(x if fx is None else torch.cat((x, fx), dim=-1))
        h = h + self.placeholder
        if self.slice_once:
            return self._slice_once_forward(h)
        shared = None
        for block in self.blocks:
            h, weights = block(h, slice_weights_in=shared)
            if self.share_slice_across_layers and shared is None:
                shared = weights
        return h
