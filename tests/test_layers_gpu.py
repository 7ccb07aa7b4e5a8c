"""The callers of the path on the GPU: the physics-attention layer and the
Transolver model with ``use_fused_slice=True`` (HIP operators) against the
same modules on their eager route, fp32 and float64 (truth), forward and
every gradient.

Gate per compared tensor, as for the operators (tests/parity.py): the fused
result's error against float64 within 1.25x eager fp32's own error + 1e-6
(or 3x where eager's own error exceeds 1e-4), and fused vs eager fp32 within
1e-5 + eager's error wherever eager's error is below
1e-5. Two documented exceptions: the temperature gradient on the G-blocked
kernels is held to 10x (measured 2.3e-6 against eager's 3.3e-7 at a
near-uniform softmax over G = 256 slots, a strongly cancelling global sum;
the 1e-5 bound holds), and a gradient that is numerically zero (norm below
1e-9, e.g. the deslice temperature of an untied layer whose softmax is near
uniform) is held to an absolute bound. The config-5-shaped model, 8 layers
deep where rounding differences compound, is held to 2x. The config-5 model
(N = 2e6, 8 layers) runs forward and backward on the fused route: finite,
two runs bitwise equal; its memory is compared with the eager route at a
smaller N, where the eager route keeps a (B, H, N, G) membership tensor per
layer and the fused route none.
"""

import copy

import pytest
import torch

from parity import relerr
from flashslice_amd.layers import Physics_Attention_Irregular_Mesh
from flashslice_amd.models import Transolver
from flashslice_amd.layers.basic import PointLinear, point_linear_pair
from flashslice_amd.layers.norm import PointLayerNorm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(module, inputs, loss_fn):
    """Output and the gradients of every parameter and input (in order)."""
    module.zero_grad(set_to_none=True)
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    out = module(*leaves)
    out = out[0] if isinstance(out, tuple) else out
    loss_fn(out).backward()
    grads = [p.grad for _, p in module.named_parameters()] + [t.grad for t in leaves]
    return [out.detach()] + [g.detach() if g is not None else None for g in grads]


def _gate(name, fused, eager32, truth, blocked=False, ratio=1.25):
    assert (fused is None) == (eager32 is None), name
    if fused is None:
        return
    assert fused.shape == eager32.shape and fused.dtype == eager32.dtype, name
    t = truth.detach().double().cpu()
    if t.norm() < 1e-9:
        d_f = (fused.detach().double().cpu() - t).norm()
        d_e = (eager32.detach().double().cpu() - t).norm()
        assert d_f <= 10 * d_e + 1e-12, (name, d_f.item(), d_e.item())
        return
    ee, ef, fe = relerr(eager32, truth), relerr(fused, truth), relerr(fused, eager32)
    # the temperature gradient is a cancelling sum (sum_g Lb = 0 per point)
    # whose error sits at fp32's noise floor (~1e-6) on both routes; the fused
    # route forms it from one merged Jacobian (the layer's coupling) or in
    # G-blocked passes, a summation order of its own: 2x, as the reference
    # allows dtau on its G-blocked shapes (bench/parity_ops.py:190-200)
    g = 10.0 if (blocked and "temperature" in name) else (
        max(ratio, 2.0) if "temperature" in name else ratio)
    assert ef <= g * ee + 1e-6 or (ee > 1e-4 and ef <= 3.0 * ee), (name, ef, ee)
    if ee < 1e-5:
        assert fe <= 1e-5 + ee, (name, fe, ee)


def _compare(make, inputs, loss_fn, blocked=False):
    torch.manual_seed(0)
    eager = make(False).to(DEV)
    fused = make(True).to(DEV)
    fused.load_state_dict(eager.state_dict())
    truth_mod = copy.deepcopy(eager).double()
    names = ["out"] + [n for n, _ in eager.named_parameters()] + \
        ["input%d" % i for i in range(len(inputs))]
    r_f = _run(fused, inputs, loss_fn)
    r_e = _run(eager, inputs, loss_fn)
    r_t = _run(truth_mod, [t.double() for t in inputs], loss_fn)
    for n, f, e, t in zip(names, r_f, r_e, r_t):
        _gate(n, f, e, t, blocked)
    return r_f


def test_point_linear_split_k():
    """The per-point Linear's split-K weight gradient against nn.Linear's and
    float64 (the same gate), on a row count that is no multiple of the chunk
    count (the remainder path), and bitwise equal over two runs."""
    torch.manual_seed(6)
    M = 200_003
    print("[point-linear] M=%d" % M, flush=True)
    lin = PointLinear(256, 512).to(DEV)
    ref = torch.nn.Linear(256, 512).to(DEV)
    ref.load_state_dict(lin.state_dict())
    truth = copy.deepcopy(ref).double()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, M, 256, generator=g).to(DEV)
    up = torch.randn(1, M, 512, generator=g).to(DEV)
    loss = lambda out: (out * up.to(out.dtype)).sum()  # noqa: E731
    r1 = _run(lin, [x], loss)
    r2 = _run(lin, [x], loss)
    assert all(torch.equal(a, b) for a, b in zip(r1, r2))
    re_ = _run(ref, [x], loss)
    rt = _run(truth, [x.double()], loss)
    for n, a, b, t in zip(["out", "weight", "bias", "x"], r1, re_, rt):
        _gate(n, a, b, t)


def test_point_linear_pair():
    """Two projections of one point stream as one GEMM (point_linear_pair:
    the layer's in_project_x / in_project_fx) against the two nn.Linears and
    float64 (the same gate): both outputs, every weight and bias gradient and
    the summed input gradient; bitwise equal over two runs."""
    torch.manual_seed(9)
    M = 200_003
    print("[point-linear-pair] M=%d" % M, flush=True)
    l1, l2 = PointLinear(256, 256).to(DEV), PointLinear(256, 256).to(DEV)
    r1m, r2m = torch.nn.Linear(256, 256).to(DEV), torch.nn.Linear(256, 256).to(DEV)
    r1m.load_state_dict(l1.state_dict())
    r2m.load_state_dict(l2.state_dict())
    g = torch.Generator().manual_seed(10)
    x = torch.randn(1, M, 256, generator=g).to(DEV)
    u1 = torch.randn(1, M, 256, generator=g).to(DEV)
    u2 = torch.randn(1, M, 256, generator=g).to(DEV)

    def run(a, b, xx, pair):
        xx = xx.detach().requires_grad_(True)
        params = [a.weight, a.bias, b.weight, b.bias]
        for p_ in params:
            p_.grad = None
        o1, o2 = point_linear_pair(xx, a, b) if pair else (a(xx), b(xx))
        ((o1 * u1.to(o1.dtype)).sum() + (o2 * u2.to(o2.dtype)).sum()).backward()
        return [o1.detach(), o2.detach(), xx.grad] + [p_.grad for p_ in params]

    f1 = run(l1, l2, x, True)
    f2 = run(l1, l2, x, True)
    assert all(torch.equal(a, b) for a, b in zip(f1, f2))
    e = run(r1m, r2m, x, False)
    t = run(copy.deepcopy(r1m).double(), copy.deepcopy(r2m).double(), x.double(), False)
    for n, a, b, tt in zip(["out1", "out2", "x", "w1", "b1", "w2", "b2"], f1, e, t):
        _gate(n, a, b, tt)


@pytest.mark.parametrize("C", [256, 512])
def test_point_layernorm(C):
    """The HIP LayerNorm (include/flashslice_layer.h) against nn.LayerNorm and
    float64 (the same gate) for output and every gradient, on an odd row
    count, with a non-trivial affine; bitwise equal over two runs."""
    torch.manual_seed(8)
    M = 200_003
    print("[layernorm] M=%d C=%d" % (M, C), flush=True)
    ln = PointLayerNorm(C).to(DEV)
    with torch.no_grad():
        ln.weight.uniform_(0.5, 1.5)
        ln.bias.uniform_(-0.2, 0.2)
    ref = torch.nn.LayerNorm(C).to(DEV)
    ref.load_state_dict(ln.state_dict())
    truth = copy.deepcopy(ref).double()
    g = torch.Generator().manual_seed(9)
    x = (3.0 + 2.0 * torch.randn(M, C, generator=g)).to(DEV)
    up = torch.randn(M, C, generator=g).to(DEV)
    loss = lambda out: (out * up.to(out.dtype)).sum()  # noqa: E731
    r1 = _run(ln, [x], loss)
    r2 = _run(ln, [x], loss)
    assert all(torch.equal(a, b) for a, b in zip(r1, r2))
    re_ = _run(ref, [x], loss)
    rt = _run(truth, [x.double()], loss)
    for n, a, b, t in zip(["out", "weight", "bias", "x"], r1, re_, rt):
        _gate(n, a, b, t)


def _mse(target):
    return lambda out: (out - target.to(out.dtype)).square().mean()


LAYER_CASES = {
    "default": dict(),
    "untied": dict(untied_deslice=True),
    "no-token-attn": dict(no_token_attention=True),
    "slice-dim-16": dict(slice_dim_head=16),
    "g256-blocked": dict(slice_num=256),
    "g256-untied": dict(slice_num=256, untied_deslice=True),
    "b2": dict(B=2),
}


@pytest.mark.parametrize("case", sorted(LAYER_CASES))
def test_layer_fused_matches_eager(case):
    kw = dict(LAYER_CASES[case])
    B = kw.pop("B", 1)
    kw.setdefault("slice_num", 32)
    N, dim = 4096, 256
    print("[layer] %s B=%d N=%d %s" % (case, B, N, kw), flush=True)

    def make(fused):
        m = Physics_Attention_Irregular_Mesh(dim, heads=8, dim_head=32, use_fused_slice=fused,
                                             **kw)
        with torch.no_grad():  # per-head temperatures away from the 0.5 start
            m.temperature.copy_(torch.linspace(0.3, 1.0, 8).view(1, 8, 1, 1))
        return m

    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, N, dim, generator=g).to(DEV)
    target = torch.randn(B, N, dim, generator=g).to(DEV)
    _compare(make, [x], _mse(target), blocked=kw["slice_num"] > 128)


def test_transolver_fused_matches_eager():
    N = 8192
    print("[model] small Transolver N=%d" % N, flush=True)

    def make(fused):
        return Transolver(space_dim=3, fun_dim=1, out_dim=4, n_hidden=128, n_heads=8,
                          n_layers=3, slice_num=32, use_fused_slice=fused)

    g = torch.Generator().manual_seed(2)
    pos = torch.rand(1, N, 3, generator=g).to(DEV)
    f = torch.randn(1, N, 1, generator=g).to(DEV)
    target = torch.randn(1, N, 4, generator=g).to(DEV)
    _compare(make, [pos, f], _mse(target))


def _c5(N, fused, seed=5):
    torch.manual_seed(seed)
    m = Transolver(space_dim=3, fun_dim=1, out_dim=4, n_hidden=256, n_heads=8, n_layers=8,
                   slice_num=32, use_fused_slice=fused).to(DEV)
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(1, N, 3, generator=g).to(DEV)
    f = torch.randn(1, N, 1, generator=g).to(DEV)
    target = torch.randn(1, N, 4, generator=g).to(DEV)
    return m, pos, f, target


def _step(m, pos, f, target):
    m.zero_grad(set_to_none=True)
    loss = (m(pos, f) - target).square().mean()
    loss.backward()
    return loss.detach(), [p.grad.detach().clone() for p in m.parameters()]


def test_config5_model_runs_deterministic():
    """the full Transolver (n_hidden 256, 8 heads, 8 layers,
    G = 32) forward and backward on 2e6 points through the fused operators."""
    N = 2_000_000
    print("[model] config 5, N=%d, fused" % N, flush=True)
    m, pos, f, target = _c5(N, True)
    assert m.use_fused_slice
    l1, g1 = _step(m, pos, f, target)
    l2, g2 = _step(m, pos, f, target)
    assert torch.isfinite(l1) and all(torch.isfinite(g).all() for g in g1)
    assert torch.equal(l1, l2) and all(torch.equal(a, b) for a, b in zip(g1, g2))


def test_config5_shape_memory_vs_eager():
    """At N = 262144 the eager route keeps each layer's (B, H, N, G) fp32
    membership for the backward; the fused route keeps none: its peak is
    lower by at least the 8 layers' memberships. Loss and every gradient
    pass the gate above against the eager route in fp32 and float64."""
    N = 262_144
    peaks, res = {}, {}
    m, pos, f, target = _c5(N, False)
    truth = copy.deepcopy(m).double()
    names = [n for n, _ in m.named_parameters()]
    state = m.state_dict()
    del m
    for fused in (True, False):
        print("[model] config-5 shape, N=%d, fused=%s" % (N, fused), flush=True)
        m = _c5(N, fused)[0]
        m.load_state_dict(state)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        res[fused] = _step(m, pos, f, target)
        torch.cuda.synchronize()
        peaks[fused] = torch.cuda.max_memory_allocated() - base
        del m
    w_bytes = 8 * 1 * 8 * N * 32 * 4
    assert peaks[True] + w_bytes <= peaks[False], (peaks, w_bytes)
    print("[model] config-5 shape, N=%d, float64 eager" % N, flush=True)
    lt, gt = _step(truth, pos.double(), f.double(), target.double())
    (lf, gf), (le, ge) = res[True], res[False]
    # 8 layers deep, rounding differences compound (the token-attention
    # weights' gradients sit near 6e-5 for both routes): ratio 2x
    _gate("loss", lf, le, lt, ratio=2.0)
    for n, a, b, t in zip(names, gf, ge, gt):
        _gate(n, a, b, t, ratio=2.0)
