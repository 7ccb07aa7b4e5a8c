"""The custom-operator boundary on the CPU (no kernel runs).

* the eight ``torch.ops.flashslice`` ops exist with the reference's schemas
  (reference ``slice_ops.py:787-801``, ``blocked.py:1477-1494``);
* their fake (meta) implementations give every output's shape and dtype
  (reference ``slice_ops.py:894-919``, ``blocked.py:1502-1529``);
* they are registered for the CUDA dispatch key only: a CPU tensor raises,
  there is no CPU fallback;
* ``torch.compile`` sees them as single opaque nodes (traced on meta
  tensors).
"""

import pytest
import torch

import flashslice_amd.kernels  # noqa: F401  -- registers the ops

SCHEMAS = {
    "flash_slice": "flash_slice(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
                   "Tensor tau, int dot) -> (Tensor, Tensor)",
    "flash_slice_bwd": "flash_slice_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, "
                       "Tensor bias, Tensor tau, Tensor dz_num, Tensor ds, int dot) -> "
                       "(Tensor, Tensor, Tensor, Tensor, Tensor)",
    "flash_deslice": "flash_deslice(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, "
                     "Tensor tokens, int dot) -> Tensor",
    "flash_deslice_bwd": "flash_deslice_bwd(Tensor x_mid, Tensor weight, Tensor bias, "
                         "Tensor tau, Tensor tokens, Tensor d_out, int dot) -> "
                         "(Tensor, Tensor, Tensor, Tensor, Tensor)",
    "slice_blk": "slice_blk(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
                 "Tensor tau, Tensor? stats, int dot) -> (Tensor, Tensor, Tensor)",
    "slice_blk_bwd": "slice_blk_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
                     "Tensor tau, Tensor stats, Tensor dz_num, Tensor ds, int dot) -> "
                     "(Tensor, Tensor, Tensor, Tensor, Tensor)",
    "deslice_blk": "deslice_blk(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, "
                   "Tensor tokens, Tensor? stats, int dot) -> (Tensor, Tensor)",
    "deslice_blk_bwd": "deslice_blk_bwd(Tensor x_mid, Tensor weight, Tensor bias, Tensor tau, "
                       "Tensor tokens, Tensor stats, Tensor d_out, int dot) -> "
                       "(Tensor, Tensor, Tensor, Tensor, Tensor)",
}


def _norm(s):
    return " ".join(s.replace("flashslice::", "").split())


@pytest.mark.parametrize("name", sorted(SCHEMAS))
def test_schema(name):
    op = getattr(torch.ops.flashslice, name).default
    assert _norm(str(op._schema)) == _norm(SCHEMAS[name])


def _meta_inputs(B=2, N=37, H=3, D=8, DV=12, G=5):
    m = lambda *s, dtype=torch.float32: torch.empty(*s, device="meta", dtype=dtype)  # noqa: E731
    return dict(x=m(B, N, H, D, dtype=torch.bfloat16), fx=m(B, N, H, DV, dtype=torch.bfloat16),
                w=m(H, G, D), b=m(H, G), tau=m(H), tok=m(B, H, G, DV),
                dz=m(B, H, G, DV), ds=m(B, H, G), dout=m(B, N, H, DV, dtype=torch.bfloat16),
                st=m(B, H, 2, N))


def test_fake_shapes_and_dtypes():
    t = _meta_inputs()
    ops = torch.ops.flashslice
    z, s = ops.flash_slice(t["x"], t["fx"], t["w"], t["b"], t["tau"], 0)
    assert z.shape == (2, 3, 5, 12) and z.dtype == torch.float32
    assert s.shape == (2, 3, 5) and s.dtype == torch.float32
    out = ops.flash_deslice(t["x"], t["w"], t["b"], t["tau"], t["tok"], 0)
    assert out.shape == (2, 37, 3, 12) and out.dtype == torch.bfloat16
    g = ops.flash_slice_bwd(t["x"], t["fx"], t["w"], t["b"], t["tau"], t["dz"], t["ds"], 0)
    assert [x.shape for x in g] == [t["x"].shape, t["fx"].shape, t["w"].shape, t["b"].shape,
                                    t["tau"].shape]
    assert [x.dtype for x in g] == [torch.bfloat16, torch.bfloat16] + [torch.float32] * 3
    g = ops.flash_deslice_bwd(t["x"], t["w"], t["b"], t["tau"], t["tok"], t["dout"], 0)
    assert [x.shape for x in g] == [t["x"].shape, t["tok"].shape, t["w"].shape, t["b"].shape,
                                    t["tau"].shape]
    z, s, st = ops.slice_blk(t["x"], t["fx"], t["w"], t["b"], t["tau"], None, 0)
    assert st.shape == (2, 3, 2, 37) and st.dtype == torch.float32
    out, st = ops.deslice_blk(t["x"], t["w"], t["b"], t["tau"], t["tok"], None, 0)
    assert out.shape == (2, 37, 3, 12) and st.shape == (2, 3, 2, 37)
    g = ops.slice_blk_bwd(t["x"], t["fx"], t["w"], t["b"], t["tau"], t["st"], t["dz"], t["ds"], 0)
    assert len(g) == 5 and g[2].shape == t["w"].shape
    g = ops.deslice_blk_bwd(t["x"], t["w"], t["b"], t["tau"], t["tok"], t["st"], t["dout"], 0)
    assert len(g) == 5 and g[1].shape == t["tok"].shape


def test_no_cpu_fallback():
    """The ops have only a CUDA-key (HIP) implementation: CPU tensors raise
    instead of silently running some other code."""
    x = torch.randn(1, 8, 2, 4)
    w, b, tau = torch.randn(3, 4), torch.zeros(3), torch.ones(2)
    with pytest.raises(NotImplementedError):
        torch.ops.flashslice.flash_slice(x, x, w, b, tau, 0)
    with pytest.raises(NotImplementedError):
        torch.ops.flashslice.deslice_blk(x, w, b, tau, torch.randn(1, 2, 3, 4), None, 0)


def test_autograd_registered():
    """setup_context saves inputs; the forward on meta tensors records an
    autograd node whose backward is the registered formula (shape-checked
    through the fakes)."""
    B, N, H, D, G = 1, 16, 2, 4, 3
    x = torch.empty(B, N, H, D, device="meta", requires_grad=True)
    fx = torch.empty(B, N, H, D, device="meta", requires_grad=True)
    w = torch.empty(G, D, device="meta", requires_grad=True)
    b = torch.empty(G, device="meta", requires_grad=True)
    tau = torch.empty(H, device="meta", requires_grad=True)
    z, s = torch.ops.flashslice.flash_slice(x, fx, w, b, tau, 0)
    assert z.grad_fn is not None
    gx, gfx, gw, gb, gt = torch.autograd.grad((z.sum() + s.sum()), [x, fx, w, b, tau])
    assert gx.shape == x.shape and gw.shape == w.shape and gt.shape == tau.shape
    tok = torch.empty(B, H, G, D, device="meta", requires_grad=True)
    out = torch.ops.flashslice.flash_deslice(x, w, b, tau, tok, 0)
    gs = torch.autograd.grad(out.sum(), [x, w, b, tau, tok])
    assert [g.shape for g in gs] == [x.shape, w.shape, b.shape, tau.shape, tok.shape]
    z, s, st = torch.ops.flashslice.slice_blk(x, fx, w, b, tau, None, 0)
    gs = torch.autograd.grad(z.sum(), [x, fx, w, b, tau])
    assert gs[0].shape == x.shape


def test_compile_keeps_one_graph():
    """torch.compile traces the public API into a single graph with the ops
    as opaque nodes (no graph breaks); traced on meta tensors so that no
    kernel runs."""
    import torch._dynamo
    from flashslice_amd.kernels import fused_deslice, fused_slice

    def coupling(x, fx, w, b, tau):
        z, s, st = fused_slice(x, fx, w, b, tau, return_stats=True)
        tok = z / (s + 1e-5)[..., None]
        return fused_deslice(x, w, b, tau, tok, stats=st)

    torch._dynamo.reset()
    t = _meta_inputs(D=8, DV=8, G=8)
    x32 = torch.empty(2, 37, 3, 8, device="meta")
    explain = torch._dynamo.explain(coupling)(x32, x32, t["w"][:, :, :8].contiguous(),
                                              t["b"], t["tau"])
    assert explain.graph_break_count == 0, explain.break_reasons
    assert explain.graph_count == 1


# ---------------------------------------------------------------- tied op
TIED_SCHEMAS = {
    "deslice_slice": "deslice_slice(Tensor x_mid, Tensor fx_mid, Tensor weight, Tensor bias, "
                     "Tensor tau, Tensor tokens, int dot) -> (Tensor, Tensor, Tensor)",
    "deslice_slice_bwd": "deslice_slice_bwd(Tensor x_mid, Tensor fx_mid, Tensor weight, "
                         "Tensor bias, Tensor tau, Tensor tokens, Tensor d_out, Tensor dz_num, "
                         "Tensor ds, int dot) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
}


@pytest.mark.parametrize("name", sorted(TIED_SCHEMAS))
def test_tied_schema(name):
    op = getattr(torch.ops.flashslice, name).default
    assert _norm(str(op._schema)) == _norm(TIED_SCHEMAS[name])


def test_tied_fakes_and_autograd():
    """fused_deslice_slice: (out, z_num, s) with the two ops' shapes and
    dtypes; its backward node gives every input's gradient in that input's
    shape and dtype (meta tensors: the fakes only)."""
    from flashslice_amd.kernels import fused_deslice_slice
    B, N, H, D, DV, G = 2, 37, 3, 8, 12, 5
    m = lambda *s, dtype=torch.float32: torch.empty(  # noqa: E731
        *s, device="meta", dtype=dtype, requires_grad=True)
    x, fx = m(B, N, H, D, dtype=torch.bfloat16), m(B, N, H, DV, dtype=torch.bfloat16)
    w, b, tau, tok = m(B, H, G, D), m(H, G), m(H), m(B, H, G, DV)
    out, z, s = fused_deslice_slice(x, fx, w, b, tau, tok)
    assert out.shape == (B, N, H, DV) and out.dtype == torch.bfloat16
    assert z.shape == (B, H, G, DV) and z.dtype == torch.float32
    assert s.shape == (B, H, G) and s.dtype == torch.float32
    gs = torch.autograd.grad(out.float().sum() + z.sum() + s.sum(), [x, fx, w, b, tau, tok])
    assert [g.shape for g in gs] == [t.shape for t in (x, fx, w, b, tau, tok)]
    assert [g.dtype for g in gs] == [t.dtype for t in (x, fx, w, b, tau, tok)]
    # only some outputs used: the others' gradients are taken as zeros
    out, z, s = fused_deslice_slice(x, fx, w, b, tau, tok)
    gs = torch.autograd.grad(s.sum(), [x, w])
    assert gs[0].shape == x.shape


def test_tied_errors_and_no_cpu_fallback():
    from flashslice_amd.kernels import fused_deslice_slice
    x = torch.randn(1, 8, 2, 4)
    w, b, tau = torch.randn(3, 4), torch.zeros(3), torch.ones(2)
    with pytest.raises(ValueError, match="tokens have width 5, fx_mid 4"):
        fused_deslice_slice(x, x, w, b, tau, torch.randn(1, 2, 3, 5))
    with pytest.raises(ValueError, match="weight's last dim"):
        fused_deslice_slice(x, x, torch.randn(3, 5), b, tau, torch.randn(1, 2, 3, 4))
    with pytest.raises(NotImplementedError):
        fused_deslice_slice(x, x, w, b, tau, torch.randn(1, 2, 3, 4))


def test_tied_compile_keeps_one_graph():
    import torch._dynamo
    from flashslice_amd.kernels import fused_deslice_slice

    def stream(x, fx, w, b, tau, tok):
        out, z, s = fused_deslice_slice(x, fx, w, b, tau, tok)
        return out, z / (s + 1e-5)[..., None]

    torch._dynamo.reset()
    m = lambda *s: torch.empty(*s, device="meta")  # noqa: E731
    explain = torch._dynamo.explain(stream)(m(2, 37, 3, 8), m(2, 37, 3, 8), m(3, 5, 8), m(3, 5),
                                            m(3), m(2, 3, 5, 8))
    assert explain.graph_break_count == 0, explain.break_reasons
    assert explain.graph_count == 1


# ------------------------------------------------------------ ragged batches
def test_varlen_fakes_autograd_and_validation():
    """fused_slice_varlen / fused_deslice_varlen: per-sample slot sums
    (B, H, G, DV), per-row outputs (rows, H, DV); every input's gradient in
    its own shape; row splits validated on the host."""
    from flashslice_amd.kernels import fused_deslice_varlen, fused_slice_varlen
    m = lambda *s: torch.empty(*s, device="meta", requires_grad=True)  # noqa: E731
    x, fx, W, b, tau, tok = m(100, 4, 32), m(100, 4, 64), m(3, 4, 64, 32), m(4, 64), m(4), \
        m(3, 4, 64, 64)
    rs = [0, 40, 40, 100]  # the middle sample is empty
    z, s = fused_slice_varlen(x, fx, W, b, tau, rs)
    assert z.shape == (3, 4, 64, 64) and s.shape == (3, 4, 64) and z.dtype == torch.float32
    out = fused_deslice_varlen(x, W, b, tau, tok, rs)
    assert out.shape == (100, 4, 64)
    gs = torch.autograd.grad(z.sum() + s.sum() + out.sum(), [x, fx, W, b, tau, tok])
    assert [g.shape for g in gs] == [t.shape for t in (x, fx, W, b, tau, tok)]
    for bad, msg in (([0, 40, 30, 100], "rise from 0"), ([1, 40, 100], "rise from 0"),
                     ([0, 40, 99], "rise from 0"), ([0], "B \\+ 1 offsets")):
        with pytest.raises(ValueError, match=msg):
            fused_slice_varlen(x, fx, W, b, tau, bad)
    with pytest.raises(ValueError, match="max_rows=10 is below"):
        fused_slice_varlen(x, fx, W, b, tau, rs, max_rows=10)
    with pytest.raises(ValueError, match="weight has 3 along batch"):
        fused_slice_varlen(x, fx, W, b, tau, [0, 50, 100])
    with pytest.raises(ValueError, match="tokens must be"):
        fused_deslice_varlen(x, W, b, tau, m(2, 4, 64, 64), rs)
    with pytest.raises(ValueError, match="rows, H, D"):
        fused_slice_varlen(m(1, 100, 4, 32), fx, W, b, tau, rs)
    with pytest.raises(NotImplementedError):  # no CPU fallback
        fused_slice_varlen(torch.randn(10, 2, 4), torch.randn(10, 2, 4), torch.randn(3, 4),
                           None, torch.ones(2), [0, 4, 10])


def test_varlen_compile_keeps_one_graph():
    import torch._dynamo
    from flashslice_amd.kernels import fused_deslice_varlen, fused_slice_varlen

    def coupling(x, fx, w, b, tau, rs):
        z, s = fused_slice_varlen(x, fx, w, b, tau, rs, max_rows=60)
        return fused_deslice_varlen(x, w, b, tau, z / (s + 1e-5)[..., None], rs, max_rows=60)

    torch._dynamo.reset()
    m = lambda *s, **k: torch.empty(*s, device="meta", **k)  # noqa: E731
    explain = torch._dynamo.explain(coupling)(m(100, 3, 8), m(100, 3, 8), m(3, 5, 8), m(3, 5),
                                              m(3), m(4, dtype=torch.int64))
    assert explain.graph_break_count == 0, explain.break_reasons
    assert explain.graph_count == 1


def test_varlen_device_splits_need_max_rows():
    from flashslice_amd.kernels import fused_slice_varlen
    m = lambda *s, **k: torch.empty(*s, device="meta", **k)  # noqa: E731
    x, w, b, tau = m(100, 3, 8), m(3, 5, 8), m(3, 5), m(3)
    with pytest.raises(ValueError, match="need max_rows"):
        fused_slice_varlen(x, x, w, b, tau, m(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="1-d int64"):
        fused_slice_varlen(x, x, w, b, tau, m(4, dtype=torch.int32), max_rows=50)
    z, s = fused_slice_varlen(x, x, w, b, tau, m(4, dtype=torch.int64), max_rows=50)
    assert z.shape == (3, 3, 5, 8) and s.shape == (3, 3, 5)


# ------------------------------------------------- coupling with merged backward
COUPLING_OPS = ("tied_deslice", "tied_slice_after", "tied_deslice_bwd", "tied_slice",
                "tied_deslice_after", "tied_slice_bwd")


def _coupling_meta(B=2, N=37, H=3, D=8, DV=12, G=5, dtype=torch.float32):
    m = lambda *s, dt=torch.float32: torch.empty(  # noqa: E731
        *s, device="meta", dtype=dt, requires_grad=True)
    return (m(B, N, H, D, dt=dtype), m(B, N, H, DV, dt=dtype), m(B, H, G, D), m(H, G), m(H),
            m(B, H, G, DV))


def test_coupling_ops_registered():
    for name in COUPLING_OPS:
        assert hasattr(torch.ops.flashslice, name), name


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_coupling_fakes_and_autograd(order, dtype):
    """fused_coupling in either order, with a differentiable step between the
    ops: outputs with the plain ops' shapes and dtypes, and every leaf's
    gradient in its shape and dtype (meta tensors: the fakes and the
    hand-over through the links)."""
    from flashslice_amd.kernels import fused_coupling
    x, fx, w, b, tau, tok = _coupling_meta(dtype=dtype)
    B, N, H, D = x.shape
    G, DV = w.shape[-2], fx.shape[3]
    lin = torch.empty(DV, DV, device="meta", requires_grad=True)
    c = fused_coupling(x, w, b, tau)
    if order == "deslice-first":
        out = c.deslice(tok)
        z, s = c.slice(torch.tanh(out.float() @ lin).to(dtype))
    else:
        z, s = c.slice(fx)
        out = c.deslice((z / (s + 1e-5)[..., None]) @ lin)
    assert out.shape == (B, N, H, DV) and out.dtype == dtype
    assert z.shape == (B, H, G, DV) and z.dtype == torch.float32
    assert s.shape == (B, H, G) and s.dtype == torch.float32
    leaves = [x, w, b, tau, lin] + ([tok] if order == "deslice-first" else [fx])
    gs = torch.autograd.grad(out.float().sum() + z.sum() + s.sum(), leaves)
    assert [g.shape for g in gs] == [t.shape for t in leaves]
    assert [g.dtype for g in gs] == [t.dtype for t in leaves]


def test_coupling_misuse_refused():
    from flashslice_amd.kernels import fused_coupling
    x, fx, w, b, tau, tok = _coupling_meta(DV=12)
    c = fused_coupling(x, w, b, tau)
    c.deslice(tok)
    with pytest.raises(RuntimeError, match="called twice"):
        c.deslice(tok)
    with pytest.raises(ValueError, match="value width 8"):
        c.slice(torch.empty(2, 37, 3, 8, device="meta"))
    c.slice(fx)
    with pytest.raises(RuntimeError, match="one slice and one deslice"):
        c.slice(fx)


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_coupling_compile_keeps_one_graph(order):
    import torch._dynamo
    from flashslice_amd.kernels import fused_coupling

    def layer(x, fx, w, b, tau, tok, lin):
        c = fused_coupling(x, w, b, tau)
        if order == "deslice-first":
            out = c.deslice(tok)
            z, s = c.slice(torch.nn.functional.gelu(out @ lin))
        else:
            z, s = c.slice(fx)
            out = c.deslice((z / (s + 1e-5)[..., None]) @ lin)
        return out, z, s

    torch._dynamo.reset()
    m = lambda *s: torch.empty(*s, device="meta")  # noqa: E731
    explain = torch._dynamo.explain(layer)(m(2, 37, 3, 8), m(2, 37, 3, 8), m(3, 5, 8), m(3, 5),
                                           m(3), m(2, 3, 5, 8), m(8, 8))
    assert explain.graph_break_count == 0, explain.break_reasons
    assert explain.graph_count == 1


def test_varlen_statistics_layout():
    """A ragged batch's statistics are (1, H, 2, rows), indexed by row, on
    both routes (G <= 128 and the G-blocked G > 128); either op accepts the
    other's."""
    from flashslice_amd.kernels import fused_deslice_varlen, fused_slice_varlen
    m = lambda *s: torch.empty(*s, device="meta", requires_grad=True)  # noqa: E731
    for G in (32, 256):
        x, fx, W, b, tau, tok = m(100, 4, 32), m(100, 4, 32), m(4, G, 32), m(4, G), m(4), \
            m(3, 4, G, 32)
        rs = [0, 40, 40, 100]
        z, s, st = fused_slice_varlen(x, fx, W, b, tau, rs, return_stats=True)
        assert st.shape == (1, 4, 2, 100) and st.dtype == torch.float32
        out, st2 = fused_deslice_varlen(x, W, b, tau, tok, rs, stats=st, return_stats=True)
        assert out.shape == (100, 4, 32) and st2.shape == st.shape
        z, s = fused_slice_varlen(x, fx, W, b, tau, rs, stats=st2)
        gs = torch.autograd.grad(z.sum() + s.sum() + out.sum(), [x, fx, W, b, tau, tok])
        assert [g.shape for g in gs] == [t.shape for t in (x, fx, W, b, tau, tok)]
