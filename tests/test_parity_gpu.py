"""Parity of the HIP path against the CPU oracle on seeded inputs (GPU).

Each case runs a full coupling forward and backward through the public API
(``fused_slice`` / ``fused_deslice`` and autograd), in fp64 and fp32 on the
CPU oracle and twice through the HIP kernels, and applies the gates in
``tests/parity.py``. The cases follow the reference's own op-level gate
(``bench/parity_ops.py:402-438``): weight layouts gd / hgd / bhgd, bias or
none, ragged and tiny N, both call orders, masked G, DV != D, and the bf16
dot mode.
"""

import pytest
import torch

from parity import Case, check_case, relerr

pytestmark = pytest.mark.gpu


def _report(name, fails, rows):
    print("\ncase %s" % name, flush=True)
    for k, ee, ef, fe in rows:
        print("  %-10s eager %.3e  fused %.3e  fused-vs-eager %.3e" % (k, ee, ef, fe))
    assert not fails, "\n".join(fails)


CASES = [
    # name, Case kwargs, order
    ("c1-shape-gd-nobias", dict(B=1, N=4096, H=8, D=32, G=32, mode="gd", bias=False, tau=0.5),
     "slice-first"),
    ("c2-shape-hgd-ragged", dict(B=1, N=4097, H=8, D=32, G=32, mode="hgd"), "slice-first"),
    ("hgd-deslice-first", dict(B=2, N=3001, H=4, D=32, G=32, mode="hgd"), "deslice-first"),
    ("gd-B2", dict(B=2, N=2049, H=4, D=32, G=32, mode="gd"), "slice-first"),
    ("bhgd-g64", dict(B=2, N=2049, H=4, D=32, G=64, mode="bhgd"), "slice-first"),
    ("bhgd-nobias", dict(B=2, N=1025, H=4, D=32, G=32, mode="bhgd", bias=False),
     "deslice-first"),
    ("tiny-N17", dict(B=2, N=17, H=4, D=32, G=32, mode="hgd"), "slice-first"),
    ("one-point", dict(B=1, N=1, H=2, D=32, G=32, mode="hgd"), "slice-first"),
    ("g16-d16", dict(B=1, N=3001, H=4, D=16, G=16, mode="hgd"), "slice-first"),
    ("g128", dict(B=1, N=2049, H=2, D=32, G=128, mode="hgd"), "slice-first"),
    ("d64-g64", dict(B=1, N=2049, H=4, D=64, G=64, mode="hgd"), "slice-first"),
    ("d128-g32", dict(B=1, N=1025, H=2, D=128, G=32, mode="hgd"), "slice-first"),
    ("c4-shape-dv64-g64", dict(B=4, N=2048, H=8, D=32, DV=64, G=64, mode="bhgd"),
     "deslice-first"),
    ("masked-g40-d40-dv24", dict(B=2, N=1537, H=4, D=40, DV=24, G=40, mode="hgd"),
     "deslice-first"),
    ("g8-padded", dict(B=1, N=2049, H=4, D=32, G=8, mode="hgd"), "slice-first"),
    ("g1", dict(B=1, N=1025, H=2, D=32, G=1, mode="hgd"), "slice-first"),
    # the deslice backward's head pairs (B * H even): a pair spanning two
    # samples (B = 2, H = 3), and B * H odd (one head per block)
    ("head-pair-across-samples", dict(B=2, N=2049, H=3, D=32, G=32, mode="bhgd"),
     "slice-first"),
    ("odd-heads", dict(B=1, N=3001, H=3, D=32, G=32, mode="hgd"), "deslice-first"),
]


@pytest.mark.parametrize("name,kw,order", CASES, ids=[c[0] for c in CASES])
def test_coupling_parity(name, kw, order):
    fails, rows = check_case(Case(**kw), order=order)
    _report(name, fails, rows)


@pytest.mark.parametrize("dot", ["bf16", "bf16v"])
def test_bf16_dot_modes(dot):
    case = Case(B=1, N=4097, H=8, D=32, G=32, mode="hgd")
    fails, rows = check_case(case, dot=dot)
    _report("bf16-" + dot, fails, rows)
    for k, ee, ef, fe in rows:
        if k in ("out", "z_num", "grad:x", "grad:fx"):
            assert ef < 2e-2, (k, ef)
    bf16_gate(rows)


@pytest.mark.parametrize("inputs", ["bf16", "fp16"])
@pytest.mark.parametrize("G", [32, 256], ids=["whole-g", "g-blocked"])
def test_half_point_tensors(inputs, G):
    """16-bit x_mid, fx_mid, W and b with the default (fp32-accurate) dots:
    the reference's bf16-autocast case (bench/parity_test.py:130-138), fwd
    and bwd. out, dx and dfx come back in the input dtype; every output and
    gradient within 2x of eager fp32 run on the same 16-bit inputs (errors of
    the bf16 class; the reference's forward gate is 1.5x + 1e-3)."""
    case = Case(B=1, N=2049, H=4, D=32, G=G, mode="hgd")
    fails, rows = check_case(case, inputs=inputs, blocked=G > 128)
    _report("%s-inputs-g%d" % (inputs, G), fails, rows)
    for k, ee, ef, fe in rows:
        assert ef < 0.05, (k, ef)


@pytest.mark.parametrize("dot,kw,kmode", [
    ("tf32", dict(B=1, N=4097, H=8, D=32, G=32, mode="hgd"), "auto"),
    ("tf32", dict(B=1, N=2049, H=4, D=32, G=256, mode="hgd"), "blocked"),
    ("tf32x3", dict(B=1, N=4097, H=8, D=32, G=32, mode="hgd"), "auto"),
    ("tf32x3", dict(B=1, N=2049, H=2, D=32, G=128, mode="hgd"), "auto"),
    ("tf32x3", dict(B=1, N=2049, H=4, D=32, G=256, mode="hgd"), "blocked"),
], ids=["tf32", "blk-tf32-g256", "tf32x3", "tf32x3-g128", "blk-tf32x3-g256"])
def test_tf32_levels(dot, kw, kmode):
    """The opt-in tf32 levels (reference bench/parity_test.py:230-245, gate
    10x). gfx950 has no tf32 MFMA: both run the fp32-accurate split, so they
    also meet the ieee gates."""
    fails, rows = check_case(Case(**kw), dot=dot, kernel_mode=kmode, gate=10.0,
                             blocked=kmode == "blocked")
    _report(dot, fails, rows)
    strict, _ = check_case(Case(**kw), dot=dot, kernel_mode=kmode, blocked=kmode == "blocked")
    assert not strict, strict


def test_forced_blocked_mode_small_g():
    """kernel mode 'blocked' routes through the stats-carrying ops."""
    fails, rows = check_case(Case(B=1, N=2049, H=4, D=32, G=32, mode="bhgd"),
                             kernel_mode="blocked", blocked=True)
    _report("forced-blocked-g32", fails, rows)


def test_stats_match_oracle():
    import oracle
    from flashslice_amd.kernels import fused_deslice, fused_slice, set_kernel_mode
    case = Case(B=2, N=1537, H=4, D=32, G=48, mode="hgd")
    x, fx, w, b, tau, tok = case.build({k: v.cuda() for k, v in case.leaves.items()}, False)
    set_kernel_mode("blocked")
    try:
        _, _, st1 = fused_slice(x, fx, w, b, tau, return_stats=True)
        _, st2 = fused_deslice(x, w, b, tau, tok, return_stats=True)
    finally:
        set_kernel_mode("auto")
    ref = oracle.stats(*(t.double().cpu() for t in (x, w, b, tau)))
    assert st1.shape == ref.shape and st1.dtype == torch.float32
    assert relerr(st1[:, :, 0], ref[:, :, 0]) < 1e-6
    assert relerr(st1[:, :, 1], ref[:, :, 1]) < 1e-5
    # the row max agrees bitwise between the statistics pass and the online
    # deslice; the sums agree to rounding (reference bench/parity_ops.py:231-235)
    assert torch.equal(st1[:, :, 0], st2[:, :, 0])
    assert ((st1[:, :, 1] - st2[:, :, 1]).abs() / st1[:, :, 1]).max() < 1e-5


# ------------------------------------------------------------- G-blocked family
# Shapes only the G-blocked kernels serve (G > 128, D = 256), and shapes the
# whole-G kernels serve forced onto the G-blocked ones (kernel mode
# 'blocked'), held to the same gates (dtau at 2x, reference
# bench/parity_ops.py:190-200). Follows the reference's blocked cases
# (bench/parity_test.py:218-228, bench/parity_ops.py:406-431).
BLOCKED = [
    ("blk-forced-g32", dict(B=1, N=2049, H=4, D=32, G=32, mode="hgd"), "slice-first", "blocked"),
    ("blk-forced-g32-deslice-first", dict(B=2, N=1025, H=4, D=32, G=32, mode="bhgd"),
     "deslice-first", "blocked"),
    ("blk-g256", dict(B=1, N=2049, H=4, D=32, G=256, mode="hgd"), "slice-first", "auto"),
    ("blk-g256-deslice-first", dict(B=2, N=1025, H=4, D=32, G=256, mode="gd"),
     "deslice-first", "auto"),
    ("blk-g512-tinyN17", dict(B=2, N=17, H=4, D=32, G=512, mode="gd"), "deslice-first", "auto"),
    ("blk-g1024-d56-dv32", dict(B=1, N=513, H=4, D=56, DV=32, G=1024, mode="bhgd", bias=False),
     "deslice-first", "auto"),
    ("blk-g48-masked", dict(B=1, N=1537, H=4, D=32, G=48, mode="hgd"), "slice-first", "blocked"),
    ("blk-g8-padded", dict(B=1, N=1537, H=4, D=32, G=8, mode="hgd"), "slice-first", "blocked"),
    ("blk-d256-g32", dict(B=1, N=1025, H=2, D=256, G=32, mode="hgd"), "slice-first", "auto"),
    ("blk-d128-g64-forced", dict(B=1, N=1537, H=2, D=128, DV=96, G=64, mode="hgd"),
     "deslice-first", "blocked"),
    ("blk-d24-g40-dv24", dict(B=1, N=1537, H=4, D=24, DV=24, G=40, mode="hgd"),
     "deslice-first", "blocked"),
    ("blk-g1", dict(B=1, N=1025, H=2, D=56, DV=32, G=1, mode="bhgd", bias=False),
     "slice-first", "blocked"),
    ("blk-tinyN17-g256-d56-dv32", dict(B=2, N=17, H=4, D=56, DV=32, G=256, mode="bhgd",
                                       bias=False), "slice-first", "auto"),
]


@pytest.mark.parametrize("name,kw,order,kmode", BLOCKED, ids=[c[0] for c in BLOCKED])
def test_blocked_parity(name, kw, order, kmode):
    fails, rows = check_case(Case(**kw), order=order, kernel_mode=kmode, blocked=True)
    _report(name, fails, rows)


def test_blocked_bf16_g256():
    fails, rows = check_case(Case(B=1, N=2049, H=4, D=56, DV=32, G=256, mode="bhgd", bias=False),
                             dot="bf16", blocked=True)
    _report("blk-bf16-g256", fails, rows)


def bf16_gate(rows):
    """The bf16 dot levels' absolute bound (fused vs eager on the same bf16
    inputs within 2e-2) for every output whose eager-bf16 error against
    float64 is itself below 1e-2; the ratio gate (2x eager-bf16's error,
    reference bench/parity_test.py:191) is applied by check_case."""
    bad = [(k, fe) for k, ee, ef, fe in rows if ee < 1e-2 and not fe <= 2e-2]
    assert not bad, bad


@pytest.mark.parametrize("dot", ["bf16", "bf16v"])
@pytest.mark.parametrize("G,N", [(256, 2049), (1024, 1025)], ids=["g256", "g1024"])
def test_blocked_bf16_c3_shape(dot, G, N):
    """C3's own shape on the bf16 dot levels: D = DV = 32 (the G-blocked
    prepared-fragment kernels with all rows aligned), per-head W, with bias
    -- the cases whose bf16 MFMA sums span the most slots."""
    case = Case(B=1, N=N, H=4, D=32, G=G, mode="hgd")
    fails, rows = check_case(case, dot=dot, blocked=True)
    _report("blk-%s-c3shape-g%d" % (dot, G), fails, rows)
    bf16_gate(rows)


def test_stats_modes_agree():
    """Online and two-pass statistics (reference bench/parity_ops.py:213-235):
    the row max agrees bitwise, the sums to rounding; the online deslice
    emits the same statistics."""
    import oracle
    from flashslice_amd.kernels import fused_deslice, set_stats_mode
    from flashslice_amd.kernels.blocked import compute_stats
    case = Case(B=1, N=1537, H=4, D=56, DV=32, G=300, mode="hgd")
    x, fx, w, b, tau, tok = case.build({k: v.cuda() for k, v in case.leaves.items()}, False)
    try:
        set_stats_mode("online")
        _, st_online = fused_deslice(x, w, b, tau, tok, return_stats=True)
        st_stats = compute_stats(x, w.contiguous(), b.contiguous(), tau)
        set_stats_mode("two-pass")
        st_two = compute_stats(x, w.contiguous(), b.contiguous(), tau)
    finally:
        set_stats_mode("online")
    assert torch.equal(st_online[:, :, 0], st_two[:, :, 0])
    assert torch.equal(st_stats[:, :, 0], st_two[:, :, 0])
    for st in (st_online, st_stats):
        assert ((st[:, :, 1] - st_two[:, :, 1]).abs() / st_two[:, :, 1]).max() < 1e-5
    ref = oracle.stats(*(t.double().cpu() for t in (x, w, b, tau)))
    assert relerr(st_two[:, :, 0], ref[:, :, 0]) < 1e-6
    assert relerr(st_two[:, :, 1], ref[:, :, 1]) < 1e-5


# ------------------------------------------------ block-cooperative kernels
# bf16 dots on bf16 point tensors at 128 < G <= 256 (D, DV <= 32) run the
# G-blocked family's block-cooperative kernels (both forward and both
# backward passes in one pass each); these cases cover partial last waves
# (G not a multiple of 32 * 8), narrow widths, tiny N, both call orders
# (statistics formed in the slice's pass, or handed in by the deslice) and
# per-sample weights, against the same gates as every bf16 case.
COOP = [
    ("coop-g256-hgd", dict(B=1, N=4097, H=4, D=32, G=256, mode="hgd"), "slice-first"),
    ("coop-g160-gd-deslice-first", dict(B=2, N=1025, H=4, D=32, G=160, mode="gd"),
     "deslice-first"),
    ("coop-g200-d24-dv16", dict(B=1, N=2049, H=2, D=24, DV=16, G=200, mode="hgd"),
     "slice-first"),
    ("coop-g256-bhgd-tinyN17", dict(B=2, N=17, H=4, D=32, G=256, mode="bhgd"), "slice-first"),
]


@pytest.mark.parametrize("name,kw,order", COOP, ids=[c[0] for c in COOP])
def test_coop_bf16_parity(name, kw, order):
    fails, rows = check_case(Case(**kw), order=order, dot="bf16", blocked=True)
    _report(name, fails, rows)
    bf16_gate(rows)
