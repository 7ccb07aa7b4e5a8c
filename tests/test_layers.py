"""The callers of the path on the CPU: the eager physics-attention layer
against the oracle's slice/deslice, the checkpoint format (parameter names of
the reference's layer, MLP and model), the flag rules and the fallback of
unsupported dims. The fused route is covered on the GPU
(tests/test_layers_gpu.py)."""

import pytest
import torch

import oracle
from flashslice_amd.layers import MLP, Physics_Attention_Irregular_Mesh
from flashslice_amd.models import Transolver, TransolverBlock
from flashslice_amd.layers.physics_attention import TOKEN_EPS


def _layer_by_oracle(layer, x):
    """The layer's output recomputed with the oracle's slice and deslice
    (float64): the projections and the token mixing are the layer's own
    modules, the slice/deslice math is the oracle's."""
    B, N, _ = x.shape
    H, D = layer.heads, layer.dim_head
    x_mid = layer.in_project_x(x).view(B, N, H, D)
    fx_mid = layer.in_project_fx(x).view(B, N, H, D)
    W, b = layer.in_project_slice.weight, layer.in_project_slice.bias
    tau = layer.temperature.view(H)
    z_num, s = oracle.slice_fwd(x_mid, fx_mid, W, b, tau)
    tokens = layer._mix_tokens(z_num / (s + TOKEN_EPS)[..., None])
    if layer.untied_deslice:
        out = oracle.deslice_fwd(x_mid, layer.in_project_deslice.weight,
                                 layer.in_project_deslice.bias,
                                 layer.deslice_temperature.view(H), tokens)
    else:
        out = oracle.deslice_fwd(x_mid, W, b, tau, tokens)
    return layer.to_out(out.reshape(B, N, H * D)), oracle.membership(x_mid, W, b, tau)


@pytest.mark.parametrize("kw", [{}, {"untied_deslice": True}, {"no_token_attention": True},
                                {"slice_dim_head": 4}])
def test_eager_layer_matches_oracle(kw):
    torch.manual_seed(0)
    layer = Physics_Attention_Irregular_Mesh(24, heads=3, dim_head=8, slice_num=5, **kw).double()
    with torch.no_grad():
        layer.temperature.uniform_(0.3, 1.0)
        if layer.untied_deslice:
            layer.deslice_temperature.uniform_(0.3, 1.0)
    x = torch.randn(2, 37, 24, dtype=torch.float64)
    out, w = layer(x)
    ref, w_ref = _layer_by_oracle(layer, x)
    assert out.shape == (2, 37, 24) and w.shape == (2, 3, 37, 5)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(w, w_ref, rtol=1e-12, atol=1e-12)


def test_eager_layer_takes_given_slice_weights():
    torch.manual_seed(1)
    layer = Physics_Attention_Irregular_Mesh(16, heads=2, dim_head=8, slice_num=4).double()
    x = torch.randn(1, 20, 16, dtype=torch.float64)
    _, w = layer(x)
    out2, w2 = layer(torch.randn_like(x), slice_weights_in=w)
    assert w2 is w and out2.shape == x.shape


def test_mlp():
    torch.manual_seed(2)
    m = MLP(5, 16, 3, n_layers=2, act="leaky_relu", res=True)
    assert m(torch.randn(4, 5)).shape == (4, 3)
    h = m.linear_pre(torch.ones(1, 5))
    for blk in m.linears:
        h = blk(h) + h
    torch.testing.assert_close(m(torch.ones(1, 5)), m.linear_post(h))
    with pytest.raises(NotImplementedError):
        MLP(2, 4, 2, act="swish")


def _expected_keys(n_layers):
    """The state-dict names of the reference's Transolver with default flags
    (reference transolver.py:41-78, 100-172; physics_attention.py:62-93;
    basic.py:28-44)."""
    keys = {"placeholder"}
    for lin in ("preprocess.linear_pre.0", "preprocess.linear_post"):
        keys |= {lin + ".weight", lin + ".bias"}
    for i in range(n_layers):
        p = "blocks.%d." % i
        for ln in ("ln_1", "ln_2") + (("ln_3",) if i == n_layers - 1 else ()):
            keys |= {p + ln + ".weight", p + ln + ".bias"}
        keys.add(p + "Attn.temperature")
        for lin in ("in_project_x", "in_project_fx", "in_project_slice", "to_out.0"):
            keys |= {p + "Attn." + lin + ".weight", p + "Attn." + lin + ".bias"}
        keys |= {p + "Attn.to_q.weight", p + "Attn.to_k.weight", p + "Attn.to_v.weight"}
        for lin in ("mlp.linear_pre.0", "mlp.linear_post") + (("mlp2",) if i == n_layers - 1
                                                              else ()):
            keys |= {p + lin + ".weight", p + lin + ".bias"}
    return keys


def test_checkpoint_format_and_interchange():
    torch.manual_seed(3)
    eager = Transolver(space_dim=2, fun_dim=1, out_dim=3, n_hidden=32, n_heads=4, n_layers=3,
                       slice_num=8)
    assert set(eager.state_dict()) == _expected_keys(3)
    fused = Transolver(space_dim=2, fun_dim=1, out_dim=3, n_hidden=32, n_heads=4, n_layers=3,
                       slice_num=8, use_fused_slice=True)
    fused.load_state_dict(eager.state_dict(), strict=True)
    assert fused.use_fused_slice and all(b.Attn.use_fused_slice for b in fused.blocks)


def test_same_seed_same_initial_weights():
    torch.manual_seed(11)
    m1 = Transolver(n_hidden=32, n_heads=4, n_layers=2, slice_num=8)
    torch.manual_seed(11)
    m2 = Transolver(n_hidden=32, n_heads=4, n_layers=2, slice_num=8, use_fused_slice=True)
    for (k1, v1), (k2, v2) in zip(m1.state_dict().items(), m2.state_dict().items()):
        assert k1 == k2 and torch.equal(v1, v2)


def test_flag_rules_and_fallback():
    with pytest.raises(ValueError):
        Transolver(n_hidden=16, n_heads=2, n_layers=1, untie_slice_weights=True, mlp_only=True)
    for flag in ("share_slice_across_layers", "slice_once"):
        with pytest.raises(ValueError):
            Transolver(n_hidden=16, n_heads=2, n_layers=1, use_fused_slice=True, **{flag: True})
    layer = Physics_Attention_Irregular_Mesh(16, heads=2, dim_head=512, slice_num=4,
                                             use_fused_slice=True)
    assert not layer.use_fused_slice and "dim_head" in layer.fused_slice_fallback
    m = Transolver(n_hidden=16, n_heads=2, n_layers=2, dim_head=300, use_fused_slice=True)
    assert m.use_fused_slice is False
    blk = TransolverBlock(2, 16, 0.0, mlp_only=True)
    out, w = blk(torch.randn(1, 5, 16))
    assert out.shape == (1, 5, 16) and w is None


def test_fused_route_refuses_cpu_tensors():
    layer = Physics_Attention_Irregular_Mesh(16, heads=2, dim_head=8, slice_num=4,
                                             use_fused_slice=True)
    with pytest.raises(NotImplementedError):
        layer(torch.randn(1, 8, 16))
    with pytest.raises(ValueError):
        layer(torch.randn(1, 8, 16), slice_weights_in=torch.rand(1, 2, 8, 4))


@pytest.mark.parametrize("flag", ["share_slice_across_layers", "slice_once",
                                  "no_token_attention", "untie_slice_weights", "mlp_only"])
def test_ablations_run_eager(flag):
    torch.manual_seed(4)
    m = Transolver(space_dim=3, fun_dim=2, out_dim=2, n_hidden=16, n_heads=2, n_layers=2,
                   slice_num=4, **{flag: True})
    y = m(torch.rand(2, 9, 3), torch.randn(2, 9, 2))
    assert y.shape == (2, 9, 2) and torch.isfinite(y).all()
    y.square().mean().backward()


def test_layernorm_op_compiles_to_one_graph():
    """The HIP LayerNorm is a custom operator with a fake: torch.compile traces
    it (forward and the registered backward's shapes) without graph breaks,
    on meta tensors so that no kernel runs."""
    import torch._dynamo
    import flashslice_amd.layers.norm  # noqa: F401 -- registers the operators

    def f(x, w, b):
        y, _, _ = torch.ops.flashslice_layer.layer_norm(x, w, b, 1e-5)
        return y * 2.0

    torch._dynamo.reset()
    x = torch.empty(70000, 256, device="meta")
    w = torch.empty(256, device="meta")
    explain = torch._dynamo.explain(f)(x, w, w)
    assert explain.graph_break_count == 0, explain.break_reasons
    y, mean, rstd = torch.ops.flashslice_layer.layer_norm(x, w, w, 1e-5)
    assert y.shape == x.shape and mean.shape == (70000,) and rstd.dtype == torch.float32


def test_package_root_exports_the_models():
    """``from flashslice_amd import Transolver`` as the reference's
    ``from flashslice import Transolver`` (reference flashslice/__init__.py:18-27)."""
    import flashslice_amd
    from flashslice_amd import layers, models
    for name in ("Transolver", "TransolverBlock", "TokenTransformerBlock"):
        assert getattr(flashslice_amd, name) is getattr(models, name)
    assert flashslice_amd.Physics_Attention_Irregular_Mesh is layers.Physics_Attention_Irregular_Mesh
    assert flashslice_amd.__version__
