"""The coupling with a merged backward (``fused_coupling``), in both orders
and with a differentiable step between the two ops, against the CPU oracle
(GPU).

deslice -> MLP -> slice is the reference's planned "tied backward fusion"
(ROADMAP.md:58-65): ``fx_mid = tanh(out @ lin)``, so the slice's dfx must
reach the MLP's backward before the deslice's backward runs.
slice -> tokens -> deslice is the Transolver layer's order
(physics_attention.py:95-136): ``tokens = (z_num / (s + eps)) @ lin``.
``lin`` is a leaf, so its gradient checks the hand-over between the two
backward calls as well. Every result and gradient is held to the gates of
``tests/parity.py`` (float64 oracle, eager fp32, two runs bitwise equal)
and compared with the same chain through the two plain operators.
"""

import pytest
import torch

import oracle
from parity import Case, compare, relerr
from flashslice_amd.kernels import (fused_coupling, fused_deslice, fused_slice, set_dot_mode,
                                    set_kernel_mode)

pytestmark = pytest.mark.gpu


class Chain(Case):
    """A coupling whose second op's input depends on the first op's output."""

    def __init__(self, *a, order="deslice-first", unaligned=False, **k):
        super().__init__(*a, **k)
        self.order = order
        self.unaligned = unaligned
        g = torch.Generator().manual_seed(99)
        self.leaves["lin"] = torch.randn(self.DV, self.DV, generator=g) / self.DV ** 0.5

    def run(self, dtype, path, device="cpu", amp=False):
        # fx (deslice-first) or tok (slice-first) stay unused: no gradient
        L = {k: v.detach().to(device=device, dtype=dtype).requires_grad_(True)
             for k, v in self.leaves.items()}
        x, fx, w, b, tau, tok = self.build(L, amp)
        if self.unaligned:
            # views one element into a wider buffer: rows that are not 16-byte
            # aligned (the kernels' element-wise load path)
            x = torch.cat([x[..., :1], x], -1)[..., 1:]
            fx = torch.cat([fx[..., :1], fx], -1)[..., 1:]
        lin = L["lin"]
        if path == "oracle":
            f32 = (lambda t: None if t is None else (t.float() if amp else t))  # noqa: E731
            x, fx, w, b = f32(x), f32(fx), f32(w), f32(b)
            slice_ = lambda f: oracle.slice_fwd(x, f, w, b, tau)  # noqa: E731
            deslice_ = lambda t: oracle.deslice_fwd(x, w, b, tau, t)  # noqa: E731
        elif path == "coupling":
            c = fused_coupling(x, w, b, tau)
            slice_, deslice_ = c.slice, c.deslice
        else:  # the two plain operators
            slice_ = lambda f: fused_slice(x, f, w, b, tau)  # noqa: E731
            deslice_ = lambda t: fused_deslice(x, w, b, tau, t)  # noqa: E731
        # the step between the ops runs in float64 on every path, so that
        # lin's gradient measures the hand-over, not the GPU's fp32 GEMMs
        if self.order == "deslice-first":
            out = deslice_(tok if path == "oracle" else tok.float())
            z, s = slice_(torch.tanh(out.double() @ lin.double()).to(out.dtype))
        else:
            z, s = slice_(fx)
            tk = (z.double() / (s.double() + oracle.EPS_TOKEN)[..., None]) @ lin.double()
            out = deslice_(tk.to(z.dtype))
        res = {"out": out.detach(), "z_num": z.detach(), "s": s.detach()}
        up = {k: v.to(device) for k, v in self.up.items()}
        loss = oracle.coupling_loss(out.float(), z.float(), s.float(), up["out"], up["z"],
                                    up["s"])
        loss.backward()
        for k, v in L.items():
            if v.grad is not None:
                res["grad:" + k] = v.grad.detach()
        return res


def _check(chain, dot="", kernel_mode="auto", ref_device="cpu", amp=False, blocked=False):
    ref = chain.run(torch.float64, "oracle", ref_device)
    ea = chain.run(torch.float32, "oracle", ref_device, amp=amp)
    set_kernel_mode(kernel_mode)
    set_dot_mode(dot)
    try:
        fu = chain.run(torch.float32, "coupling", "cuda", amp=amp)
        fu2 = chain.run(torch.float32, "coupling", "cuda", amp=amp)
        two = chain.run(torch.float32, "plain", "cuda", amp=amp)
    finally:
        set_dot_mode("")
        set_kernel_mode("auto")
    fails, rows = compare(ref, ea, fu, fu2, amp=amp, blocked=blocked)
    print("\n%s chain" % chain.order, flush=True)
    for k, ee, ef, fe in rows:
        # the merged backward against the two plain operators' backward
        print("  %-10s eager %.3e  fused %.3e  fused-vs-eager %.3e  vs-two-ops %.3e"
              % (k, ee, ef, fe, relerr(fu[k], two[k])))
        if not amp and relerr(fu[k], two[k]) > 2e-6 + ee:
            fails.append("%s: coupling vs the two plain ops %.3e" % (k, relerr(fu[k], two[k])))
    assert not fails, "\n".join(fails)


CASES = [
    # name, Case kwargs
    ("c2-shape-hgd", dict(B=1, N=4097, H=8, D=32, G=32, mode="hgd")),
    ("gd-B2-nobias", dict(B=2, N=2049, H=4, D=32, G=32, mode="gd", bias=False)),
    ("c4-shape-bhgd-dv64-g64", dict(B=2, N=3001, H=8, D=32, DV=64, G=64, mode="bhgd")),
    ("masked-g40-d40-dv24", dict(B=1, N=1537, H=4, D=40, DV=24, G=40, mode="hgd")),
    ("tiny-N17", dict(B=2, N=17, H=4, D=32, G=32, mode="hgd")),
    # one block of 32 on every axis with padded slots and masked columns
    ("padded-g8-d16-dv24", dict(B=1, N=1025, H=2, D=16, DV=24, G=8, mode="hgd")),
    # G-blocked shapes: the merged node runs the two plain backward ops
    ("g256-blocked", dict(B=1, N=2049, H=4, D=32, G=256, mode="hgd")),
]


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_coupling_parity(name, kw, order):
    _check(Chain(**kw, order=order), blocked=kw["G"] > 128)


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_coupling_forced_blocked(order):
    """kernel mode 'blocked': the G-blocked kernels with the statistics the
    first op hands to the second."""
    _check(Chain(B=1, N=2049, H=4, D=32, G=32, mode="hgd", order=order),
           kernel_mode="blocked", blocked=True)


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_coupling_bf16(order):
    """bf16 point tensors with bf16 dots: within 2x of eager on the same
    bf16 inputs."""
    _check(Chain(B=1, N=4097, H=8, D=32, G=32, mode="hgd", order=order), dot="bf16",
           amp=torch.bfloat16)


@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_coupling_unaligned_rows(order):
    """x_mid and fx_mid rows that are not 16-byte aligned: the merged
    kernels' element-wise load path."""
    _check(Chain(B=1, N=2049, H=4, D=32, G=32, mode="hgd", order=order, unaligned=True))


@pytest.mark.parametrize("inputs,dot", [(torch.float16, ""), (torch.bfloat16, "bf16v")],
                         ids=["fp16-ieee-dots", "bf16-bf16v-dots"])
@pytest.mark.parametrize("order", ["deslice-first", "slice-first"])
def test_coupling_half_inputs(order, inputs, dot):
    """16-bit point tensors with fp32-accurate dots, and bf16 with bf16 value
    dots (fp32-accurate logits): within 2x of eager on the same inputs."""
    _check(Chain(B=1, N=4097, H=8, D=32, G=32, mode="hgd", order=order), dot=dot, amp=inputs)


@pytest.mark.parametrize("name,kw,order", [
    ("c2", dict(B=1, N=1_000_000, H=8, D=32, G=32, mode="hgd"), "slice-first"),
    ("c4", dict(B=4, N=262_144, H=8, D=32, DV=64, G=64, mode="bhgd"), "deslice-first"),
], ids=["c2-slice-first", "c4-deslice-first"])
def test_coupling_full_size(name, kw, order):
    """BASELINE configs 2 and 4 at full size, the oracle on the GPU's ATen."""
    _check(Chain(**kw, order=order), ref_device="cuda")


def test_coupling_only_first_op_used():
    """A coupling whose second op never runs: the first op's backward is the
    plain one."""
    case = Case(B=1, N=2049, H=4, D=32, G=32, mode="hgd")
    x, fx, w, b, tau, tok = case.build({k: v.cuda().requires_grad_(True)
                                        for k, v in case.leaves.items()}, False)
    d_out = case.up["out"].cuda()
    c = fused_coupling(x, w, b, tau)
    out = c.deslice(tok)
    g1 = torch.autograd.grad(out, [x, w, b, tau, tok], d_out)
    out2 = fused_deslice(x, w, b, tau, tok)
    g2 = torch.autograd.grad(out2, [x, w, b, tau, tok], d_out)
    assert torch.equal(out, out2)
    for a_, b_ in zip(g1, g2):
        assert torch.equal(a_, b_)
