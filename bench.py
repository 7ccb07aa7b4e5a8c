"""Benchmark of the fused slice/deslice hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload c1|c2|c2-df|c3-256|c3-1024|c4|c5|c5-262k|ragged|layer|layer-1m-fwd]
                    [--backward auto|tied|two-op]

One step is the coupling the metric names ("slice+deslice
fwd+bwd ms & Mpoints/s at N=1M, H=8, D=32, G=32; peak HBM") on one batch of
synthetic points already resident in HBM, through the ``torch.ops.flashslice``
operators, in the order autograd runs them:

    z_num, s   = slice(x, fx, W, b, tau)                 slice forward
    tokens     = z_num / (s + 1e-5)                      (torch, tiny)
    out        = deslice(x, W, b, tau, tokens)           deslice forward
    backward of both, with upstream gradients d_out, dz_num, ds ~ N(0, 1)
    (the loss of reference bench/parity_ops.py:148-151) and the chain rule
    through the tokens (torch, tiny)

The backward takes one of two forms, with the same gradients:
  * tied (the default where the whole-G kernels serve the shape, as at C2):
    the operators ``fused_coupling`` runs -- the deslice's dtokens (the slice
    forward kernel on d_out), then one merged pass for the rest of both
    backwards (dx of both ops summed, dfx, dW, db, dtau);
  * two ops (reference slice_ops.py:822-885): flash_deslice_bwd, then
    flash_slice_bwd (whose two dx autograd would still have to add).
Either way the step moves the same 11 x-sized passes of algorithmic bytes.
Where both forms exist the line reports the other one too
(``other_backward``). Inputs follow BASELINE.json config 2: x, fx ~ N(0, 1)
(1, 1e6, 8, 32) fp32; per-head W ~ N(0, 1/D); b ~ N(0, 0.02^2); tau ~
U[0.3, 1.0]. ``value`` is points per second of the whole step.

Printed: ONE JSON line with the driver's fields, plus ``roofline`` (the
dominant op's algorithmic bytes per launch over its HIP-event time on its
stream -- the op is its point kernel and the small fixed-order reduction of
its partials; ``traffic`` is the HBM bytes rocprofv3 counted for it, from
the committed profiles/<workload>[-tied]_hbm_traffic.txt), ``step_roofline``
(the step's algorithmic bytes over its time), ``cpu_baseline`` (the CPU
oracle -- the eager PyTorch softmax/einsum path -- timed on a bounded sample
on this host's cores), ``peak_hbm_gb``, ``per_op_ms``, ``deterministic`` and
``public_api`` (the same step through the public API and autograd).

The timed steps carry one HIP event at each step boundary and a pair around
the dominant op only; ``per_op_ms`` comes from K steps with events around
every op, run before them (a timing event is a marker the GPU waits on:
eight per step cost ~30 us of the C2 step).
"""

import argparse
import functools
import json
import os
import sys
import subprocess
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
MFMA_PEAK_TFLOPS = {"ieee": 157.3, "bf16": 2500.0}  # MI355X dense fp32 / bf16 MFMA, published
EPS = 1e-5

WORKLOADS = {
    # name: (B, N, H, D, DV, G, weight layout, order, description)
    # C2 is bounded by HBM; C3 and C4 by the matrix cores
    "c2": (1, 1_000_000, 8, 32, 32, 32, "hgd", "slice-first",
           "C2: slice->deslice fwd+bwd, B=1 N=1e6 H=8 D=DV=32 G=32 fp32 ieee, per-head W"),
    "c3-256": (1, 1_000_000, 8, 32, 32, 256, "hgd", "slice-first",
               "C3: slice->deslice fwd+bwd, B=1 N=1e6 H=8 D=DV=32 G=256 fp32 ieee, per-head W"),
    "c3-1024": (1, 1_000_000, 8, 32, 32, 1024, "hgd", "slice-first",
                "C3: slice->deslice fwd+bwd, B=1 N=1e6 H=8 D=DV=32 G=1024 fp32 ieee, per-head W"),
    # C2's shape in the persistent-stream order (deslice, then slice): where
    # the tied backward (--tied) applies at this shape
    "c2-df": (1, 1_000_000, 8, 32, 32, 32, "hgd", "deslice-first",
              "C2 shape, deslice->slice fwd+bwd, B=1 N=1e6 H=8 D=DV=G=32 fp32 ieee, per-head W, "
              "given tokens"),
    "c4": (4, 262_144, 8, 32, 64, 64, "bhgd", "deslice-first",
           "C4: deslice->slice fwd+bwd, B=4 N=262144 H=8 D=32 DV=64 G=64 fp32 ieee, "
           "per-sample W, given tokens"),
}
# model-level workload: the Transolver that calls the path
# once per layer, forward + backward of an MSE loss; reported on its own line
MODEL_WORKLOADS = {
    "c5": dict(B=1, N=2_000_000, space_dim=3, fun_dim=1, out_dim=4, n_hidden=256, n_heads=8,
               n_layers=8, slice_num=32,
               desc="C5: Transolver fwd+bwd (MSE), B=1 N=2e6, n_hidden=256, 8 heads, 8 layers, "
                    "G=32, fp32, use_fused_slice=True"),
    # the same model at the point count of the reference's published model
    # number (README.md:137-142, N = 262k)
    "c5-262k": dict(B=1, N=262_144, space_dim=3, fun_dim=1, out_dim=4, n_hidden=256, n_heads=8,
                    n_layers=8, slice_num=32,
                    desc="C5 model at N=262144: Transolver fwd+bwd (MSE), n_hidden=256, 8 heads, "
                         "8 layers, G=32, fp32, use_fused_slice=True"),
}
# ragged batch (reference ROADMAP.md:66-68): many small meshes of different N
# in one launch through row splits, against the per-sample loop it replaces
RAGGED_WORKLOADS = {
    "ragged": dict(B=64, n_min=2_000, n_max=40_000, H=8, D=32, DV=32, G=32,
                   desc="ragged: 64 meshes of N ~ U[2000, 40000] (1.34M points), H=8 "
                        "D=DV=G=32 fp32 ieee, per-head W, slice->deslice fwd+bwd in one "
                        "launch per op through row splits"),
}
# one physics-attention layer, eager and fused in the same process (reference
# bench/bench_layer.py: its default shape, training step)
LAYER_WORKLOADS = {
    "layer": dict(N=262_144, H=8, D=32, G=32, mode="train",
                  desc="layer: Physics_Attention_Irregular_Mesh(256, heads=8, dim_head=32, "
                       "slice_num=32), B=1 N=262144, fp32, training step (fwd + mean-square "
                       "loss + bwd), fused vs eager"),
    "layer-1m-fwd": dict(N=1_000_000, H=8, D=32, G=32, mode="fwd",
                         desc="layer: Physics_Attention_Irregular_Mesh(256, heads=8, dim_head=32, "
                              "slice_num=32), B=1 N=1e6, fp32, forward (no grad), fused vs eager"),
}
# dot level per run (reference slice_ops.py:336-343): 0 ieee; 3 bf16 (bf16 inputs)
DOTS = {"ieee": 0, "bf16": 3}


def timing_events(n):
    """n timing events, each recorded once already: the runtime creates an
    event on its first record, so the timed loop must not be the first to
    record them (measured: one host stall of ~38 ms inside one op of the
    timed steps when 200 fresh events were first recorded there)."""
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    return ev


def event_pairs(n):
    ev = timing_events(2 * n)
    return list(zip(ev[0::2], ev[1::2]))


class quiet_gc:
    """Collect, then keep Python's garbage collector out of the timed region
    (a full collection in a torch process is tens of ms of host time, which
    the GPU spends idle once the launch queue has drained)."""

    def __enter__(self):
        import gc
        gc.collect()
        self.was = gc.isenabled()
        gc.disable()

    def __exit__(self, *exc):
        import gc
        if self.was:
            gc.enable()


def make_inputs(B, N, H, D, DV, G, layout, device, seed=0):
    """Synthetic inputs of BASELINE.json's configs, generated on the CPU from
    one seed (so the CPU baseline and the GPU see the same values)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, H, D, generator=g)
    fx = torch.randn(B, N, H, DV, generator=g)
    wshape = {"gd": (G, D), "hgd": (H, G, D), "bhgd": (B, H, G, D)}[layout]
    W = torch.randn(*wshape, generator=g) / D ** 0.5
    b = 0.02 * torch.randn(*wshape[:-1], generator=g)
    tau = 0.3 + 0.7 * torch.rand(H, generator=g)
    d_out = torch.randn(B, N, H, DV, generator=g)
    dzb = torch.randn(B, H, G, DV, generator=g)
    dsb = torch.randn(B, H, G, generator=g)
    tok = torch.randn(B, H, G, DV, generator=g)
    to = lambda t: t.to(device)  # noqa: E731
    return tuple(map(to, (x, fx, W, b, tau, d_out, dzb, dsb, tok)))


def alg_bytes(B, N, H, D, DV, e=4):
    """Algorithmic HBM bytes per op (x-sized passes; reference
    bench/bench_kernels.py:45): slice fwd reads x, fx; deslice fwd reads x,
    writes out; deslice bwd reads x, d_out, writes dx; slice bwd reads x, fx,
    writes dx, dfx."""
    pts = B * N * H
    return {"slice_fwd": pts * (D + DV) * e, "deslice_fwd": pts * (D + DV) * e,
            "deslice_bwd": pts * (2 * D + DV) * e, "slice_bwd": pts * (2 * D + 2 * DV) * e,
            # the tied backward (--tied): reads x, fx, d_out, writes dx, dfx;
            # slice-first, the dtokens pass before it reads x, d_out
            "tied_bwd": pts * (2 * D + 3 * DV) * e, "dtok_pass": pts * (D + DV) * e}


def alg_flops(B, N, H, D, DV, G):
    """Algorithmic FLOPs per op (14 dots per step: logits recomputed in each
    op, 1 value dot per forward, 3 more dots per backward)."""
    u = 2 * B * N * H * G
    return {"slice_fwd": u * (D + DV), "deslice_fwd": u * (D + DV),
            "deslice_bwd": u * (3 * D + 2 * DV),  # logits, dtokens, omega, dx, dW
            "slice_bwd": u * (3 * D + 2 * DV),
            # logits, omega (two value dots), dfx, dtokens, dx, dW (slice-first
            # the dtokens dot is the dtokens pass's: logits and w^T d_out)
            "tied_bwd": u * (3 * D + 4 * DV), "tied_bwd_sf": u * (3 * D + 3 * DV),
            "dtok_pass": u * (D + DV)}


def measured_traffic(workload):
    """HBM bytes per launch of each op's kernels as rocprofv3 counted them
    (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of known size), read
    from the committed summary profiles/<workload>_hbm_traffic.txt (its
    ``hbm_bytes_per_launch`` block); None where no summary exists."""
    path = os.path.join(ROOT, "profiles", "%s_hbm_traffic.txt" % workload)
    if not os.path.exists(path):
        return None
    out, on = {}, False
    with open(path) as f:
        for ln in f:
            if ln.startswith("hbm_bytes_per_launch"):
                on = True
                continue
            if on:
                parts = ln.split()
                if len(parts) != 2:
                    if out:
                        break
                    continue
                out[parts[0]] = int(float(parts[1]))
    return out or None


OPS = ("slice_fwd", "deslice_fwd", "deslice_bwd", "slice_bwd")


def token_grads(dzb, dsb, dtok, tok, den):
    """The chain rule through tokens = z_num / den (den = s + eps, (..., 1)):
    dz_num = dzb + dtok / den, ds = dsb - sum_v dtok tok / den."""
    dz = torch.addcdiv(dzb, dtok, den)
    ds = torch.addcdiv(dsb, (dtok * tok).sum(-1), den[..., 0], value=-1.0)
    return dz, ds


def step_ops(x, fx, W, b, tau, d_out, dzb, dsb, tok0, order="slice-first", dot=0,
             blocked=False, ev=None, tied=False):
    """One coupling step, forward and backward, through the operators the
    public API routes the shape to (reference slice_ops.py:961-1022): the
    single-tile ops, or (``blocked``) the blocked ops, which carry the
    forward's softmax statistics into the other pass and the backward.
    slice-first: tokens come from the slice (tokens = z / (s + eps)) and the
    upstream gradients reach z and s through them too; deslice-first: the
    given tokens are deslided, then the points are slided again (config 4's
    persistent point stream), and the backward runs in autograd's order
    (slice, then deslice). ``ev``: a (start, end) event pair per op name,
    recorded around exactly that op (ops it does not name run bare). ``tied``: the backward as
    ``fused_coupling`` runs it instead of the two backward ops (whose two dx
    autograd would still have to add): deslice-first the one tied operator
    (flashslice::deslice_slice_bwd, one pass for both ops' gradients and a
    single dx); slice-first the deslice's dtokens (w^T d_out, a slice pass
    over x and d_out with the saved statistics: the token step needs them
    before the slice's backward can start), then one tied pass
    (flashslice::tied_slice_bwd) for everything else. The forward ops carry
    the slice's statistics to the deslice and the backward."""
    ops = torch.ops.flashslice
    from flashslice_amd.kernels.slice_ops import _whole_g, stats_placeholder

    def timed(name, fn, *args):
        if ev is None or name not in ev:
            return fn(*args)
        ev[name][0].record()
        r = fn(*args)
        ev[name][1].record()
        return r

    if blocked:
        slice_f = lambda st: ops.slice_blk(x, fx, W, b, tau, st, dot)  # noqa: E731
        deslice_f = lambda tk, st: ops.deslice_blk(x, W, b, tau, tk, st, dot)  # noqa: E731
        slice_b = lambda st, dz, ds: ops.slice_blk_bwd(x, fx, W, b, tau, st, dz, ds, dot)  # noqa
        deslice_b = lambda tk, st: ops.deslice_blk_bwd(x, W, b, tau, tk, st, d_out, dot)  # noqa
    else:
        slice_f = lambda st: ops.flash_slice(x, fx, W, b, tau, dot) + (None,)  # noqa: E731
        deslice_f = lambda tk, st: (ops.flash_deslice(x, W, b, tau, tk, dot), None)  # noqa
        slice_b = lambda st, dz, ds: ops.flash_slice_bwd(x, fx, W, b, tau, dz, ds, dot)  # noqa
        deslice_b = lambda tk, st: ops.flash_deslice_bwd(x, W, b, tau, tk, d_out, dot)  # noqa

    if order == "deslice-first":
        # the tied form as fused_deslice_slice runs it: where the whole-G
        # kernels serve the shape they read no statistics, so none are formed
        st0 = None
        if tied and blocked and _whole_g(x.shape[3], fx.shape[3], W.shape[-2]):
            st0 = stats_placeholder(x.shape[0], x.shape[2], x.shape[1], x)
        out, st = timed("deslice_fwd", deslice_f, tok0, st0)
        z, s, _ = timed("slice_fwd", slice_f, st)
        if tied:
            dx, dfx, dW, db, dt, dtok = timed("tied_bwd", ops.deslice_slice_bwd, x, fx, W, b,
                                              tau, tok0, d_out, dzb, dsb, dot)
            return z, s, out, dx, dtok, dW, db, dt, dfx
        dx2, dfx, dW2, db2, dt2 = timed("slice_bwd", slice_b, st, dzb, dsb)
        dx1, dtok, dW1, db1, dt1 = timed("deslice_bwd", deslice_b, tok0, st)
        return z, s, out, dx1, dtok, dW1, db1, dt1, dx2, dfx, dW2, db2, dt2
    if tied:
        # the operators fused_coupling runs (kernels/coupling.py): the slice
        # first (statistics for the G-blocked kernels, a placeholder where the
        # whole-G kernels serve the shape), the deslice after it, then the
        # deslice's backward (dtokens: the slice forward kernel on d_out) and
        # one merged pass for the rest of both backwards
        z, s, st, lp, lt = timed("slice_fwd", ops.tied_slice, x, fx, W, b, tau, dot)
        den = (s + EPS)[..., None]
        tok = z / den
        out = timed("deslice_fwd", ops.tied_deslice_after, x, W, b, tau, tok, st, lp, lt, dot)
        dtok, _, _ = timed("dtok_pass", ops.slice_blk, x, d_out, W, b, tau, st, dot)
        dz, ds = token_grads(dzb, dsb, dtok, tok, den)
        dx, dfx, dW, db, dt = timed("tied_bwd", ops.tied_slice_bwd, x, fx, W, b, tau, st, dz,
                                    ds, d_out, tok, dot)
        return z, s, out, dx, dtok, dW, db, dt, dfx
    z, s, st = timed("slice_fwd", slice_f, None)
    den = (s + EPS)[..., None]
    tok = z / den
    out, _ = timed("deslice_fwd", deslice_f, tok, st)
    dx1, dtok, dW1, db1, dt1 = timed("deslice_bwd", deslice_b, tok, st)
    dz, ds = token_grads(dzb, dsb, dtok, tok, den)
    dx2, dfx, dW2, db2, dt2 = timed("slice_bwd", slice_b, st, dz, ds)
    return z, s, out, dx1, dtok, dW1, db1, dt1, dx2, dfx, dW2, db2, dt2


def public_step(x, fx, W, b, tau, d_out, dzb, dsb, tok0, order, coupling):
    """The coupling step as a user writes it: the public API on leaves that
    require grad, and autograd for the backward (its host cost, and for the
    two plain ops the sum of their two dx, included). slice-first: tokens =
    z / (s + eps); deslice-first: the given tokens are deslided and the
    slice pools fx = tanh(out), a pointwise stand-in for the MLP of the
    deslice -> MLP -> slice chain (its dfx must reach the step's backward
    before the deslice's backward). ``coupling``: ``fused_coupling`` (merged
    backward) instead of the two plain ops. Returns the leaves' gradients."""
    from flashslice_amd.kernels import fused_coupling, fused_deslice, fused_slice
    x, fx, W, b, tau, tok0 = [t.detach().requires_grad_(True) for t in (x, fx, W, b, tau, tok0)]
    if coupling:
        c = fused_coupling(x, W, b, tau)
        slice_, deslice_ = c.slice, c.deslice
    else:
        slice_ = lambda f: fused_slice(x, f, W, b, tau)  # noqa: E731
        deslice_ = lambda t: fused_deslice(x, W, b, tau, t)  # noqa: E731
    if order == "slice-first":
        z, s = slice_(fx)
        out = deslice_(z / (s + EPS)[..., None])
        want = [x, fx, W, b, tau]
    else:
        out = deslice_(tok0)
        z, s = slice_(torch.tanh(out))
        want = [x, W, b, tau, tok0]
    return torch.autograd.grad([out, z, s], want, [d_out, dzb, dsb])


def time_public(inputs, order, steps, warmup):
    """Median ms per step of ``public_step`` with the two plain ops and with
    ``fused_coupling``, and the largest relative difference of their
    gradients."""
    res = {}
    grads = {}
    for name, cp in (("two_ops", False), ("coupling", True)):
        for _ in range(warmup):
            public_step(*inputs, order, cp)
        grads[name] = public_step(*inputs, order, cp)
        ts = event_pairs(steps)
        with quiet_gc():
            for e0, e1 in ts:
                e0.record()
                public_step(*inputs, order, cp)
                e1.record()
            torch.cuda.synchronize()
        ms = sorted(e0.elapsed_time(e1) for e0, e1 in ts)
        res[name + "_ms"] = round(ms[len(ms) // 2], 4)
    diff = max(float((u.double() - v.double()).norm() / v.double().norm().clamp_min(1e-30))
               for u, v in zip(grads["coupling"], grads["two_ops"]))
    res["coupling_vs_two_ops_relerr"] = float("%.3e" % diff)
    return res


def cpu_model():
    """The host CPU's model name (lscpu), for the CPU baseline's record."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return None


def cpu_baseline(B, N, H, D, DV, G, layout, order, budget_s=20.0):
    """The eager PyTorch softmax/einsum path (the CPU oracle, fp32) on this
    host's cores, forward + backward of the same coupling on a bounded
    sample of points; returns points/s."""
    import oracle
    torch.set_num_threads(os.cpu_count() or 1)
    n = min(32768, N)
    x, fx, W, b, tau, d_out, dzb, dsb, tok = make_inputs(B, n, H, D, DV, G, layout, "cpu")

    def run():
        leaves = [t.clone().requires_grad_(True) for t in (x, fx, W, b, tau, tok)]
        out, z, s = oracle.coupling(*leaves[:5], tokens=leaves[5], order=order)
        oracle.coupling_loss(out, z, s, d_out, dzb, dsb).backward()

    run()
    t0 = time.perf_counter()
    run()
    one = time.perf_counter() - t0
    # grow the sample (up to the workload's N) until one run is ~1/8 of the
    # budget, then time 3 runs
    while one < budget_s / 8 and n < N:
        n = min(2 * n, N)
        x, fx, W, b, tau, d_out, dzb, dsb, tok = make_inputs(B, n, H, D, DV, G, layout, "cpu")
        t0 = time.perf_counter()
        run()
        one = time.perf_counter() - t0
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return B * n / ts[1], n, torch.get_num_threads()


def bench_ragged(a, cfg):
    """One step = the slice -> deslice coupling of every mesh, forward and
    backward (the four ops of the C2 step), as ONE launch per op through row
    splits (``flashslice::*_varlen``); beside it the same work as a loop of
    per-mesh calls of the regular ops (B = 1 each), the fixed per-call floor
    that ragged batching removes. Inputs as C2's, per mesh."""
    ops = torch.ops.flashslice
    g = torch.Generator().manual_seed(0)
    B, H, D, DV, G = cfg["B"], cfg["H"], cfg["D"], cfg["DV"], cfg["G"]
    lens = torch.randint(cfg["n_min"], cfg["n_max"] + 1, (B,), generator=g).tolist()
    rows = sum(lens)
    splits = [0]
    for n in lens:
        splits.append(splits[-1] + n)
    dev = torch.device("cuda:0")
    x, fx, W, b, tau, d_out, dzb, dsb, _ = make_inputs(1, rows, H, D, DV, G, "hgd", dev)
    x, fx, d_out = x[0], fx[0], d_out[0]
    dzb = torch.randn(B, H, G, DV, generator=g).to(dev)
    dsb = torch.randn(B, H, G, generator=g).to(dev)
    rs = torch.tensor(splits, dtype=torch.int64, device=dev)
    nmax = max(lens)

    def ragged():
        z, s, st = ops.slice_varlen(x, fx, W, b, tau, rs, nmax, None, 0)
        den = (s + EPS)[..., None]
        tok = z / den
        out, _ = ops.deslice_varlen(x, W, b, tau, tok, rs, nmax, st, 0)
        dx1, dtok, dW1, db1, dt1 = ops.deslice_varlen_bwd(x, W, b, tau, tok, rs, nmax, st, d_out,
                                                          0)
        dz = dzb + dtok / den
        ds = dsb - (dtok * tok).sum(-1) / den[..., 0]
        dx2, dfx, dW2, db2, dt2 = ops.slice_varlen_bwd(x, fx, W, b, tau, rs, nmax, st, dz, ds, 0)
        return z, s, out, dx1, dtok, dx2, dfx

    def looped():
        res = []
        for i in range(B):
            sl = slice(splits[i], splits[i + 1])
            xi, fi, oi = x[sl][None], fx[sl][None], d_out[sl][None]
            z, s = ops.flash_slice(xi, fi, W, b, tau, 0)
            den = (s + EPS)[..., None]
            tok = z / den
            out = ops.flash_deslice(xi, W, b, tau, tok, 0)
            dx1, dtok, dW1, db1, dt1 = ops.flash_deslice_bwd(xi, W, b, tau, tok, oi, 0)
            dz = dzb[i:i + 1] + dtok / den
            ds = dsb[i:i + 1] - (dtok * tok).sum(-1) / den[..., 0]
            res.append(ops.flash_slice_bwd(xi, fi, W, b, tau, dz, ds, 0))
        return res

    def timed(fn, k):
        for _ in range(a.warmup):
            fn()
        with quiet_gc():
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(k):
                fn()
            torch.cuda.synchronize()
            return 1e3 * (time.perf_counter() - t0) / k

    r1 = [t.clone() for t in ragged()]
    deterministic = all(torch.equal(u, v) for u, v in zip(r1, ragged()))
    del r1
    ms = timed(ragged, a.steps)
    ms_loop = timed(looped, max(1, a.steps // 5))
    nbytes = rows * H * (6 * D + 5 * DV) * 4
    ach = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "ragged slice+deslice fwd+bwd Mpoints/s", "value": round(rows / (ms * 1e-3) / 1e6, 3),
        "unit": "Mpoints/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg["desc"], "samples": B, "rows": rows, "min_n": min(lens),
                   "max_n": nmax, "H": H, "D": D, "DV": DV, "G": G},
        "roofline": {"bound": "hbm", "kernel": "step (4 ops)", "achieved": round(ach, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": None, "alg_bytes_per_step": nbytes},
        "per_sample_loop": {"ms_per_step": round(ms_loop, 4),
                            "Mpoints_per_s": round(rows / (ms_loop * 1e-3) / 1e6, 3),
                            "launches_per_step": 4 * B},
        "deterministic": deterministic, "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def bench_c1(a):
    """BASELINE config 1, the reference's CPU-runnable case: slice then
    deslice, forward only, B=1, N=4096, H=8, D=DV=G=32, shared W ~ N(0, 1/D),
    no bias, tau = 0.5, tokens = z_num / (s + 1e-5); seed 0. Reports the
    step's time (launch-bound at this size), its error against the CPU
    oracle in float64 and the oracle's own fp32 time on this host."""
    import oracle
    from flashslice_amd.kernels import fused_deslice, fused_slice
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, N, H, D, G = 1, 4096, 8, 32, 32
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, N, H, D, generator=g)
    fx = torch.randn(B, N, H, D, generator=g)
    W = torch.randn(G, D, generator=g) / D ** 0.5
    tau = torch.full((H,), 0.5)
    xd, fd, Wd, td = (t.to(dev) for t in (x, fx, W, tau))

    def step():
        z, s_ = fused_slice(xd, fd, Wd, None, td)
        return fused_deslice(xd, Wd, None, td, z / (s_ + 1e-5)[..., None]), z, s_

    for _ in range(a.warmup):
        step()
    ev = event_pairs(a.steps)
    with quiet_gc():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for e0, e1 in ev:
            e0.record()
            res = step()
            e1.record()
        torch.cuda.synchronize()
        ms = 1e3 * (time.perf_counter() - t0) / a.steps
    ms_med = sorted(e0.elapsed_time(e1) for e0, e1 in ev)[a.steps // 2]
    ref = oracle.coupling(x.double(), fx.double(), W.double(), None, tau.double(),
                          order="slice-first")
    err = {k: float((r.detach().double().cpu() - t.double()).norm() / t.norm())
           for k, r, t in zip(("out", "z_num", "s"), res, ref)}
    torch.set_num_threads(os.cpu_count() or 1)
    ts = []
    for _ in range(4):
        t1 = time.perf_counter()
        oracle.coupling(x, fx, W, None, tau, order="slice-first")
        ts.append(time.perf_counter() - t1)
    cpu_s = sorted(ts[1:])[1]
    nbytes = B * N * H * 4 * D * 4
    line = {
        "metric": "slice+deslice forward Mpoints/s (config 1)",
        "value": round(B * N / (ms_med * 1e-3) / 1e6, 3), "unit": "Mpoints/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4),
        "ms_per_step_median": round(ms_med, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "C1: slice->deslice forward only, B=1 N=4096 H=8 D=DV=G=32, "
                               "shared W, no bias, tau=0.5", "B": B, "N": N, "H": H, "D": D,
                   "G": G},
        "roofline": {"bound": "launch latency", "achieved": round(nbytes / (ms_med * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(nbytes / (ms_med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "alg_bytes_per_step": nbytes},
        "relerr_vs_float64_oracle": {k: float("%.3g" % v) for k, v in err.items()},
        "cpu_baseline": {"value": round(B * N / cpu_s / 1e6, 4), "unit": "Mpoints/s",
                         "cores": torch.get_num_threads(), "kind": "port",
                         "sample": "eager PyTorch softmax/einsum oracle (oracle/eager.py), fp32 "
                                   "forward of the whole config, median of 3 runs after 1"},
    }
    print(json.dumps(line), flush=True)


def bench_layer(a, cfg):
    """The reference's layer-level number (bench/bench_layer.py:27-63): one
    Physics_Attention_Irregular_Mesh training step, fused and eager in the
    same process on the same weights and input, median of K event-timed
    steps, and the peak memory one step allocates above what is resident."""
    import statistics
    from flashslice_amd.layers import Physics_Attention_Irregular_Mesh
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    N, H, D, G = cfg["N"], cfg["H"], cfg["D"], cfg["G"]
    torch.manual_seed(0)
    layer = Physics_Attention_Irregular_Mesh(H * D, heads=H, dim_head=D, slice_num=G,
                                             use_fused_slice=True).to(dev)
    assert layer.use_fused_slice
    x = torch.randn(1, N, H * D, generator=torch.Generator().manual_seed(1)).to(dev)

    def step():
        if cfg["mode"] == "fwd":
            with torch.no_grad():
                layer(x)
            return
        out, _ = layer(x)
        out.float().square().mean().backward()
        layer.zero_grad(set_to_none=True)

    res = {}
    for fused in (True, False):
        layer.use_fused_slice = fused
        for _ in range(a.warmup):
            step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        step()
        torch.cuda.synchronize()
        peak = (torch.cuda.max_memory_allocated() - base) / 1e9
        ts = []
        for _ in range(a.steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            step()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        res[fused] = (statistics.median(ts), peak)
        torch.cuda.empty_cache()
    (fm, fp), (em, ep) = res[True], res[False]
    line = {
        "metric": "physics-attention layer %s Mpoints/s (fused)"
                  % ("training step" if cfg["mode"] == "train" else "forward"),
        "value": round(N / (fm * 1e-3) / 1e6, 3), "unit": "Mpoints/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(fm, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["desc"], "N": N, "H": H, "D": D, "G": G},
        "eager_ms_per_step": round(em, 4), "speedup_vs_eager": round(em / fm, 3),
        "peak_gb": {"fused": round(fp, 3), "eager": round(ep, 3)},
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def model_inputs(cfg, N, device, seed=0):
    """Coordinates uniform in the unit cube, per-point inputs and MSE targets
    ~N(0, 1), generated on the CPU from one seed."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(cfg["B"], N, cfg["space_dim"], generator=g)
    f = torch.randn(cfg["B"], N, cfg["fun_dim"], generator=g)
    y = torch.randn(cfg["B"], N, cfg["out_dim"], generator=g)
    return pos.to(device), f.to(device), y.to(device)


def model_flops(model, cfg, N):
    """Algorithmic flops of one forward + backward: every Linear applied per
    point (2 in out forward, 4 in out for dX and dW) and the path's own dots
    per layer (alg_flops); token-level products (on G tokens) and elementwise
    work are left out."""
    import torch.nn as nn
    token_level = ("to_q", "to_k", "to_v", "slice_down", "in_project_slice",
                   "in_project_deslice")
    per_point = sum(6 * m.in_features * m.out_features for n, m in model.named_modules()
                    if isinstance(m, nn.Linear) and not n.split(".")[-1] in token_level)
    H = cfg["n_heads"]
    D = cfg["n_hidden"] // H
    path = cfg["n_layers"] * sum(alg_flops(cfg["B"], N, H, D, D, cfg["slice_num"]).values())
    return cfg["B"] * N * per_point + path


def bench_model(a, cfg):
    """The config-5 model step on the fused operators: warmup, a determinism
    check (two steps, bitwise equal loss and gradients), peak memory, then K
    timed steps; the CPU baseline is the same model on its eager route on a
    bounded sample of points."""
    from flashslice_amd.models import Transolver
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kw = {k: cfg[k] for k in ("space_dim", "fun_dim", "out_dim", "n_hidden", "n_heads",
                              "n_layers", "slice_num")}
    torch.manual_seed(0)
    model = Transolver(use_fused_slice=True, **kw).to(dev)
    assert model.use_fused_slice
    B, N = cfg["B"], cfg["N"]
    pos, f, y = model_inputs(cfg, N, dev)
    print("[bench] %s" % cfg["desc"], file=sys.stderr, flush=True)

    def step():
        model.zero_grad(set_to_none=True)
        loss = (model(pos, f) - y).square().mean()
        loss.backward()
        return loss.detach()

    for _ in range(a.warmup):
        step()
    l1 = step()
    g1 = [p.grad.clone() for p in model.parameters()]
    l2 = step()
    deterministic = bool(torch.equal(l1, l2) and all(
        torch.equal(u, p.grad) for u, p in zip(g1, model.parameters())))
    del g1
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    peak_gb = (torch.cuda.max_memory_allocated() - base) / 1e9
    ev = event_pairs(a.steps)
    with quiet_gc():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for e0, e1 in ev:
            e0.record()
            step()
            e1.record()
        torch.cuda.synchronize()
        ms_step = 1e3 * (time.perf_counter() - t0) / a.steps
    ms_ev = sum(e0.elapsed_time(e1) for e0, e1 in ev) / a.steps
    flops = model_flops(model, cfg, N)
    tf = flops / (ms_ev * 1e-3) / 1e12

    cpu = None
    if not a.no_cpu_baseline:
        torch.set_num_threads(os.cpu_count() or 1)
        cmodel = Transolver(use_fused_slice=False, **kw)
        cmodel.load_state_dict({k: v.cpu() for k, v in model.state_dict().items()})
        n_s = 16384
        cp, cf, cy = model_inputs(cfg, n_s, "cpu")

        def cstep():
            cmodel.zero_grad(set_to_none=True)
            (cmodel(cp, cf) - cy).square().mean().backward()
        cstep()
        ts = []
        for _ in range(3):
            t = time.perf_counter()
            cstep()
            ts.append(time.perf_counter() - t)
        ts.sort()
        cpu = {"value": round(B * n_s / ts[1] / 1e6, 5), "unit": "Mpoints/s",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": "the same model (same weights) on its eager route, fp32 fwd+bwd of "
                         "the MSE loss on %d of the %d points, median of 3 runs" % (n_s, N)}

    line = {
        "metric": "Transolver fwd+bwd Mpoints/s (config 5)",
        "value": round(B * N / (ms_step * 1e-3) / 1e6, 3), "unit": "Mpoints/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init weights)",
        "config": {"workload": cfg["desc"], **kw, "B": B, "N": N},
        "roofline": {"bound": "mfma", "kernel": "whole step (hipBLASLt GEMMs + path)",
                     "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS["ieee"],
                     "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS["ieee"], 4),
                     "traffic": None, "alg_flops": flops},
        "peak_hbm_gb": round(peak_gb, 2),
        "deterministic": deterministic,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 50; 5 for the model workload)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 5; 2 for the model workload)")
    ap.add_argument("--workload", default="c2",
                    choices=sorted(WORKLOADS) + sorted(MODEL_WORKLOADS) + sorted(RAGGED_WORKLOADS)
                    + sorted(LAYER_WORKLOADS) + ["c1"])
    ap.add_argument("--dot", default="ieee", choices=sorted(DOTS),
                    help="dot level: ieee (fp32 inputs) or bf16 (x_mid, fx_mid, W in bf16)")
    ap.add_argument("--backward", default="auto", choices=("auto", "tied", "two-op"),
                    help="tied: the backward as fused_coupling runs it (deslice-first one tied "
                         "pass; slice-first the dtokens pass, then one tied pass); two-op: the "
                         "two backward ops (reference slice_ops.py:822-885); auto (default): "
                         "tied where the whole-G kernels serve the shape, else two-op")
    ap.add_argument("--tied", action="store_true", help="the same as --backward tied")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="before the warmup, copy x once (B*N*H*D*4 bytes read and written): "
                         "a kernel of known traffic that calibrates rocprofv3's FETCH_SIZE / "
                         "WRITE_SIZE counters")
    a = ap.parse_args()
    model = a.workload in MODEL_WORKLOADS
    a.steps = (5 if model else 50) if a.steps is None else a.steps
    a.warmup = (2 if model else 5) if a.warmup is None else a.warmup
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU: every GPU box of this build has one, and the "
              "slice/deslice path is measured on one GPU's share (N=%d requested)" % a.gpus,
              file=sys.stderr)
        sys.exit(2)

    import flashslice_amd.kernels  # noqa: F401  -- registers torch.ops.flashslice
    from flashslice_amd.kernels import _hip

    if a.workload in MODEL_WORKLOADS:
        return bench_model(a, MODEL_WORKLOADS[a.workload])
    if a.workload == "c1":
        return bench_c1(a)
    if a.workload in LAYER_WORKLOADS:
        return bench_layer(a, LAYER_WORKLOADS[a.workload])
    if a.workload in RAGGED_WORKLOADS:
        torch.cuda.set_device(0)
        return bench_ragged(a, RAGGED_WORKLOADS[a.workload])
    B, N, H, D, DV, G, layout, order, desc = WORKLOADS[a.workload]
    if a.dot == "bf16":
        desc = desc.replace("fp32 ieee", "bf16 inputs and dots")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inputs = list(make_inputs(B, N, H, D, DV, G, layout, dev))
    dot = DOTS[a.dot]
    if a.dot == "bf16":  # reference bench/parity_ops.py:134-136: activations and W in bf16
        for i in (0, 1, 2, 3, 5):
            inputs[i] = inputs[i].bfloat16()
    from flashslice_amd.kernels.slice_ops import _use_blocked, _whole_g
    blocked = _use_blocked(D, G, DV, dot)
    whole = _whole_g(D, DV, G)
    if a.tied:
        a.backward = "tied"
    a.tied = a.backward == "tied" or (a.backward == "auto" and whole)

    def ops_of(tied):
        return ((("deslice_fwd", "slice_fwd", "tied_bwd") if order == "deslice-first" else
                 ("slice_fwd", "deslice_fwd", "dtok_pass", "tied_bwd")) if tied else OPS)
    ops_timed = ops_of(a.tied)
    run_step = functools.partial(step_ops, *inputs, order=order, dot=dot, blocked=blocked,
                                 tied=a.tied)
    torch.cuda.synchronize()
    print("[bench] %s; library %s" % (desc, _hip.lib().fs_version().decode()),
          file=sys.stderr, flush=True)

    if a.copy_probe:
        probe = torch.empty_like(inputs[0])
        probe.copy_(inputs[0])
        torch.cuda.synchronize()
        nb = probe.numel() * probe.element_size()
        print("[bench] copy probe: %d bytes read, %d written" % (nb, nb), file=sys.stderr,
              flush=True)
        del probe

    # every event of the measurement, created (and recorded once) before any
    # step: the host work of creating them then leaves no idle gap before the
    # timed steps
    pairs = iter(event_pairs(a.steps * len(ops_timed)))
    evs = [{n: next(pairs) for n in ops_timed} for _ in range(a.steps)]
    bounds = timing_events(a.steps + 1)
    dom_ev = event_pairs(a.steps)
    gc_quiet = quiet_gc()
    gc_quiet.__enter__()

    # determinism: two steps bitwise equal
    r1 = [t.clone() for t in run_step()]
    r2 = run_step()
    deterministic = all(torch.equal(u, v) for u, v in zip(r1, r2))
    del r1, r2

    # peak HBM of one step above the resident inputs
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    res = run_step()
    torch.cuda.synchronize()
    peak_gb = (torch.cuda.max_memory_allocated() - base) / 1e9
    del res

    # the per-op breakdown: K steps with HIP events around every op, after
    # the W warmup steps. Each event is a marker in the stream that the GPU
    # waits on (measured at C2: ~30 us per step for the eight), so the timed
    # steps below carry only those the line needs.
    for _ in range(a.warmup):
        run_step()
    for i in range(a.steps):
        run_step(ev=evs[i])
    torch.cuda.synchronize()
    per_op = {n: sum(e[n][0].elapsed_time(e[n][1]) for e in evs) / a.steps for n in ops_timed}
    dom = max(per_op, key=per_op.get)

    # timed region: K steps; one HIP event at each step boundary and a pair
    # around the dominant kernel (the roofline's launch duration, live)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    bounds[0].record()
    for i in range(a.steps):
        run_step(ev={dom: dom_ev[i]})
        bounds[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dom_ms = sum(e0.elapsed_time(e1) for e0, e1 in dom_ev) / a.steps
    # the other form of the backward where the whole-G kernels serve both
    # (the two backward ops against the merged one): its per-op breakdown,
    # then K steps timed the same way, after W warmup steps
    alt = None
    if whole:
        alt_tied = not a.tied
        alt_ops = ops_of(alt_tied)
        run_alt = functools.partial(step_ops, *inputs, order=order, dot=dot, blocked=blocked,
                                    tied=alt_tied)
        apairs = iter(event_pairs(a.steps * len(alt_ops)))
        aevs = [{n: next(apairs) for n in alt_ops} for _ in range(a.steps)]
        abounds = timing_events(a.steps + 1)
        for _ in range(a.warmup):
            run_alt()
        for i in range(a.steps):
            run_alt(ev=aevs[i])
        abounds[0].record()
        for i in range(a.steps):
            run_alt()
            abounds[i + 1].record()
        torch.cuda.synchronize()
        ams = sorted(abounds[i].elapsed_time(abounds[i + 1]) for i in range(a.steps))
        alt = {"backward": "tied" if alt_tied else "two ops",
               "ms_per_step_median": round(ams[len(ams) // 2], 4),
               "per_op_ms": {n: round(sum(e[n][0].elapsed_time(e[n][1]) for e in aevs)
                                      / a.steps, 4) for n in alt_ops}}
    gc_quiet.__exit__(None, None, None)
    ms_step = 1e3 * wall / a.steps
    in_order = [bounds[i].elapsed_time(bounds[i + 1]) for i in range(a.steps)]
    step_ms = sorted(in_order)
    ms_median = step_ms[len(step_ms) // 2]
    print("[bench] event-timed steps: min %.4f median %.4f max %.4f ms; wall mean %.4f ms; "
          "in order: %s" % (step_ms[0], ms_median, step_ms[-1], 1e3 * wall / a.steps,
                            " ".join("%.3f" % t for t in in_order)),
          file=sys.stderr, flush=True)
    bytes_ = alg_bytes(B, N, H, D, DV, 2 if a.dot == "bf16" else 4)
    flops = alg_flops(B, N, H, D, DV, G)
    if order == "slice-first":
        flops["tied_bwd"] = flops.pop("tied_bwd_sf")
    ach = bytes_[dom] / (dom_ms * 1e-3) / 1e9
    ach_tf = flops[dom] / (dom_ms * 1e-3) / 1e12
    # the step's algorithmic units are the four ops' (the metric's unit),
    # whichever form the backward takes
    total_bytes = sum(bytes_[n] for n in OPS)
    total_flops = sum(flops[n] for n in OPS)
    step_ach = total_bytes / (ms_step * 1e-3) / 1e9
    # counted on fp32 point tensors: a bf16 line has its own file or none
    traffic_name = a.workload + ("-bf16" if a.dot == "bf16" else "") + ("-tied" if a.tied else "")
    traffic = measured_traffic(traffic_name)

    cpu = None
    if not a.no_cpu_baseline:
        v, n_s, thr = cpu_baseline(B, N, H, D, DV, G, layout, order)
        cpu = {"value": round(v / 1e6, 4), "unit": "Mpoints/s", "cores": thr, "kind": "port",
               "sample": "eager PyTorch softmax/einsum oracle (oracle/eager.py), fp32 fwd+bwd "
                         "of the same coupling on %d of the %d points, median of 3 runs, "
                         "torch threads=%d, os.cpu_count()=%d" % (n_s, N, thr, os.cpu_count()),
               "cpu_model": cpu_model()}

    # the same step through the public API and autograd: the two plain ops
    # against the coupling with the merged backward (deslice-first with an
    # MLP between the ops: the deslice -> MLP -> slice chain)
    public = None
    if a.dot == "ieee":
        public = time_public(inputs, order, a.steps, max(2, a.warmup))
        public["step"] = ("slice -> z/(s+eps) -> deslice" if order == "slice-first" else
                          "deslice -> fx = tanh(out) -> slice")
        public["includes"] = "host cost per op call, autograd (the two ops' dx sum)"

    line = {
        "metric": "slice+deslice fwd+bwd Mpoints/s at N=1M,H=8,D=32,G=32 (ms and peak HBM "
                  "alongside)" if a.workload == "c2" else "slice+deslice fwd+bwd Mpoints/s",
        "value": round(B * N / (ms_step * 1e-3) / 1e6, 3),
        "unit": "Mpoints/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        # the median of the K steps' HIP-event times (the reference's bench
        # reports medians, bench_layer.py:27-40); ms_per_step is the wall mean
        "ms_per_step_median": round(ms_median, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if a.dot == "ieee" else "bf16", "data": "synthetic",
        "config": {"workload": desc, "B": B, "N": N, "H": H, "D": D, "DV": DV, "G": G,
                   "weight": layout, "order": order, "dot": a.dot,
                   "ops": "blocked" if blocked else "single-tile",
                   "backward": "tied" if a.tied else "two ops"},
        "roofline": ({"bound": "hbm", "kernel": dom, "achieved": round(ach, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4)}
                     if a.workload == "c2" else
                     {"bound": "mfma", "kernel": dom, "achieved": round(ach_tf, 2),
                      "peak": MFMA_PEAK_TFLOPS[a.dot], "unit": "TFLOP/s",
                      "frac": round(ach_tf / MFMA_PEAK_TFLOPS[a.dot], 4)}),
        "traffic_source": ("profiles/%s_hbm_traffic.txt" % traffic_name) if traffic else None,
        "step_roofline": {"alg_bytes": total_bytes, "achieved_GBs": round(step_ach, 1),
                          "hbm_frac": round(step_ach / HBM_PEAK_GBS, 4),
                          "alg_flops": total_flops,
                          "alg_tflops": round(total_flops / (ms_step * 1e-3) / 1e12, 2)},
        "per_op_ms": {k: round(v, 4) for k, v in per_op.items()},
        "per_op_source": "K steps with HIP events around every op, before the timed steps "
                         "(which carry events only at step boundaries and around the "
                         "dominant kernel)",
        "peak_hbm_gb": round(peak_gb, 3),
        "nxhxg_gb": round(B * N * H * G * 4 / 1e9, 3),
        "deterministic": deterministic,
        "other_backward": alt,
        "public_api": public,
        "cpu_baseline": cpu,
    }
    line["roofline"].update({
        "traffic": traffic.get(dom) if traffic else None,
        "alg_bytes_per_launch": bytes_[dom], "alg_flops_per_launch": flops[dom],
        "ms_per_launch": round(dom_ms, 4)})
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
