"""The operators under torch.compile on the GPU, forward and backward.

``torch.compile(..., backend="aot_eager", fullgraph=True)`` traces the
public API through Dynamo and AOTAutograd -- the custom operators' fakes,
their registered backward formulas and the functionalised graph -- and runs
the traced graphs (no code generation, so nothing but these kernels and
ATen runs). The compiled results must equal the uncompiled ones bitwise:
the same deterministic kernels run on the same inputs.
"""

import math

import pytest
import torch

from flashslice_amd.kernels import (fused_deslice, fused_deslice_slice, fused_deslice_varlen,
                                    fused_slice, fused_slice_varlen)

pytestmark = pytest.mark.gpu


def _leaves(*shapes, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g).cuda() for s in shapes]


def _grads(fn, inputs, ups):
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    outs = fn(*leaves)
    loss = sum((o * u).sum() for o, u in zip(outs, ups))
    loss.backward()
    torch.cuda.synchronize()
    return [o.detach() for o in outs] + [t.grad for t in leaves]


def _check(fn, inputs, ups):
    torch._dynamo.reset()
    eager = _grads(fn, inputs, ups)
    compiled = _grads(torch.compile(fn, backend="aot_eager", fullgraph=True), inputs, ups)
    for i, (a, b) in enumerate(zip(eager, compiled)):
        if a is None and b is None:
            continue  # a leaf the function does not use
        assert a.shape == b.shape and a.dtype == b.dtype, i
        assert torch.equal(a, b), (i, (a - b).abs().max().item())


def test_compiled_coupling():
    B, N, H, D, G = 1, 3001, 4, 32, 32

    def coupling(x, fx, w, b, tau):
        z, s, st = fused_slice(x, fx, w, b, tau, return_stats=True)
        tok = z / (s + 1e-5)[..., None]
        return fused_deslice(x, w, b, tau, tok, stats=st), z, s

    x, fx, w, b = _leaves((B, N, H, D), (B, N, H, D), (H, G, D), (H, G))
    w = w / math.sqrt(D)
    tau = torch.linspace(0.4, 0.9, H).cuda()
    ups = _leaves((B, N, H, D), (B, H, G, D), (B, H, G), seed=1)
    _check(coupling, [x, fx, w, b, tau], ups)


def test_compiled_blocked_coupling():
    """G = 256: the G-blocked operators (statistics handed between them)."""
    B, N, H, D, G = 1, 1025, 2, 32, 256

    def coupling(x, fx, w, b, tau):
        z, s, st = fused_slice(x, fx, w, b, tau, return_stats=True)
        return fused_deslice(x, w, b, tau, z / (s + 1e-5)[..., None], stats=st), z, s

    x, fx, w, b = _leaves((B, N, H, D), (B, N, H, D), (H, G, D), (H, G))
    tau = torch.linspace(0.4, 0.9, H).cuda()
    ups = _leaves((B, N, H, D), (B, H, G, D), (B, H, G), seed=1)
    _check(coupling, [x, fx, w / math.sqrt(D), b, tau], ups)


def test_compiled_tied_and_ragged():
    B, N, H, D, DV, G = 2, 1500, 4, 32, 64, 64
    x, fx, w, b, tok = _leaves((B, N, H, D), (B, N, H, DV), (B, H, G, D), (B, H, G),
                               (B, H, G, DV))
    tau = torch.linspace(0.4, 0.9, H).cuda()
    ups = _leaves((B, N, H, DV), (B, H, G, DV), (B, H, G), seed=1)
    _check(lambda *a: fused_deslice_slice(*a), [x, fx, w / math.sqrt(D), b, tau, tok], ups)

    rows, splits = 2600, torch.tensor([0, 1000, 1000, 2600], dtype=torch.int64).cuda()
    xr, fr, wr, br = _leaves((rows, H, D), (rows, H, D), (H, G, D), (H, G), seed=2)

    def ragged(x, fx, w, b, tau):
        z, s = fused_slice_varlen(x, fx, w, b, tau, splits, max_rows=1600)
        out = fused_deslice_varlen(x, w, b, tau, z / (s + 1e-5)[..., None], splits,
                                   max_rows=1600)
        return out, z, s

    ups = _leaves((rows, H, D), (3, H, G, D), (3, H, G), seed=3)
    _check(ragged, [xr, fr, wr / math.sqrt(D), br, tau], ups)


def test_compiled_layer():
    """The fused physics-attention layer under torch.compile (graph breaks
    allowed around the layer's own code), output and every parameter
    gradient equal to the uncompiled layer's."""
    from flashslice_amd.layers import Physics_Attention_Irregular_Mesh
    torch.manual_seed(0)
    layer = Physics_Attention_Irregular_Mesh(128, heads=4, dim_head=32, slice_num=32,
                                             use_fused_slice=True).cuda()
    x = torch.randn(1, 2049, 128).cuda()

    def run(fn):
        layer.zero_grad(set_to_none=True)
        out, _ = fn(x)
        out.square().mean().backward()
        torch.cuda.synchronize()
        return [out.detach()] + [p.grad.clone() for p in layer.parameters()]

    torch._dynamo.reset()
    eager = run(layer)
    compiled = run(torch.compile(layer, backend="aot_eager"))
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b), (a - b).abs().max().item()


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_compiled_merged_coupling(order):
    """fused_coupling with a step between the ops: the link tensors that
    carry the hand-over between the two backward calls survive Dynamo and
    AOTAutograd, and the compiled gradients equal the eager ones bitwise."""
    from flashslice_amd.kernels import fused_coupling
    B, N, H, D, G = 1, 3001, 4, 32, 32

    def chain(x, fx, w, b, tau, tok, lin):
        c = fused_coupling(x, w, b, tau)
        if order == "deslice-first":
            out = c.deslice(tok)
            z, s = c.slice(torch.tanh(out @ lin))
        else:
            z, s = c.slice(fx)
            out = c.deslice((z / (s + 1e-5)[..., None]) @ lin)
        return out, z, s

    x, fx, w, b, tok, lin = _leaves((B, N, H, D), (B, N, H, D), (H, G, D), (H, G),
                                    (B, H, G, D), (D, D))
    w = w / math.sqrt(D)
    lin = lin / math.sqrt(D)
    tau = torch.linspace(0.4, 0.9, H).cuda()
    ups = _leaves((B, N, H, D), (B, H, G, D), (B, H, G), seed=1)
    _check(chain, [x, fx, w, b, tau, tok, lin], ups)
