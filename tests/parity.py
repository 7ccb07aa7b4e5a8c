"""Shared harness of the GPU parity tests: the HIP path through the public
API and autograd, against the CPU oracle (``oracle/eager.py``).

Gates (reference ``bench/parity_ops.py:51-55, 189-206``):
  * relerr(a, ref) = ||a - ref||_2 / ||ref||_2 in float64;
  * fused vs the float64 oracle within 1.25x of eager fp32's own error
    (+1e-6), or 3x where eager itself sits above 1e-4 (cancellation noise);
    2x for dtau on G-blocked shapes;
  * bf16 dot modes: within 2x of eager-on-bf16-inputs' error (+1e-6);
  * the north-star bound for fp32 ieee: relerr(fused, eager fp32) <= 1e-5
    (+ eager's own error against float64, which a more accurate result may
    sit across from) for every output whose eager error is itself below
    1e-5; outputs whose eager error exceeds it (cancellation sums such as
    dtau and db at large N) are held to the ratio gate;
  * shapes and dtypes of every output and gradient equal the eager ones;
  * two fused runs are bitwise identical.
"""

import math

import torch

import oracle
from flashslice_amd.kernels import (fused_deslice, fused_deslice_slice, fused_slice,
                                    set_dot_mode, set_kernel_mode)


def relerr(a, ref):
    ref = ref.detach().double().cpu()
    a = a.detach().double().cpu()
    n = ref.norm()
    d = (a - ref).norm()
    return (d / n).item() if n > 0 else d.item()


class Case:
    """Leaves of one coupling. ``mode``: gd / hgd leaf weights, or bhgd --
    weight computed from a token stream (non-leaf, non-contiguous)."""

    def __init__(self, B, N, H, D, G, DV=None, mode="hgd", bias=True, Ht=16, seed=7,
                 tau=None):
        self.B, self.N, self.H, self.D, self.G = B, N, H, D, G
        self.DV = D if DV is None else DV
        self.mode, self.bias = mode, bias
        g = torch.Generator().manual_seed(seed)
        r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
        L = {"x": r(B, N, H, D), "fx": r(B, N, H, self.DV), "tok": r(B, H, G, self.DV)}
        L["tau"] = (torch.full((H,), tau) if tau is not None
                    else 0.3 + 0.7 * torch.rand(H, generator=g))
        if mode == "gd":
            L["w"] = r(G, D) / math.sqrt(D)
            if bias:
                L["b"] = 0.1 * r(G)
        elif mode == "hgd":
            L["w"] = r(H, G, D) / math.sqrt(D)
            if bias:
                L["b"] = 0.1 * r(H, G)
        else:
            L["t"] = r(B, G, Ht)
            L["Wk"] = r(Ht, H * D) / (Ht * D) ** 0.25
            if bias:
                L["Wb"] = 0.1 * r(Ht, H)
        self.leaves = L
        self.tm = r(self.DV, self.DV) / math.sqrt(self.DV)
        self.up = {"out": r(B, N, H, self.DV), "z": r(B, H, G, self.DV), "s": r(B, H, G)}

    def build(self, L, amp):
        x, fx, tau, tok = L["x"], L["fx"], L["tau"], L["tok"]
        if self.mode in ("gd", "hgd"):
            w, b = L["w"], L.get("b")
        else:
            B, G, H, D = self.B, self.G, self.H, self.D
            w = (L["t"] @ L["Wk"]).view(B, G, H, D).permute(0, 2, 1, 3)
            b = (L["t"] @ L["Wb"]).permute(0, 2, 1) if self.bias else None
        if amp:  # a 16-bit dtype: x, fx, W, b as the activations of an autocast region
            x, fx, w = x.to(amp), fx.to(amp), w.to(amp)
            b = None if b is None else b.to(amp)
        return x, fx, w, b, tau, tok

    def run(self, dtype, fused, device="cpu", amp=False, order="slice-first", grads=True):
        L = {k: v.detach().to(device=device, dtype=dtype).requires_grad_(grads)
             for k, v in self.leaves.items()}
        x, fx, w, b, tau, tok = self.build(L, amp)
        tm = self.tm.to(device=device, dtype=dtype)
        if fused:
            if order == "slice-first":
                z, s, st = fused_slice(x, fx, w, b, tau, return_stats=True)
                tk = (z / (s + oracle.EPS_TOKEN)[..., None]) @ tm.float()
                out = fused_deslice(x, w, b, tau, tk, stats=st)
            elif order == "tied":  # deslice-first as one op with one backward pass
                out, z, s = fused_deslice_slice(x, fx, w, b, tau, tok.float())
            else:
                out, st = fused_deslice(x, w, b, tau, tok.float(), return_stats=True)
                z, s = fused_slice(x, fx, w, b, tau, stats=st)
        else:
            f32 = (lambda t: None if t is None else (t.float() if amp else t))  # noqa: E731
            out, z, s = oracle.coupling(f32(x), f32(fx), f32(w), f32(b), tau, tm=tm,
                                        tokens=tok,
                                        order="deslice-first" if order == "tied" else order)
        res = {"out": out.detach(), "z_num": z.detach(), "s": s.detach()}
        if grads:
            up = {k: v.to(device) for k, v in self.up.items()}
            loss = oracle.coupling_loss(out.float(), z.float(), s.float(),
                                        up["out"], up["z"], up["s"])
            loss.backward()
            for k, v in L.items():
                if v.grad is not None:
                    res["grad:" + k] = v.grad.detach()
        return res


def check_case(case, order="slice-first", dot="", kernel_mode="auto", gate=1.25,
               blocked=False, grads=True, strict=True, ref_device="cpu", inputs=None):
    """Run ``case`` through the oracle (fp64, fp32) and the HIP path twice;
    return a list of failure strings (empty = pass) and the metrics.
    ``ref_device``: where the oracle's tensors live (the full-size cases
    evaluate the same restatement on the GPU's ATen kernels). ``inputs``:
    None, "bf16" or "fp16" -- the point tensors and W, b in that dtype (the
    bf16 dot levels imply bf16), eager upcasting them to fp32."""
    amp = {"bf16": torch.bfloat16, "fp16": torch.float16}.get(inputs, False)
    if dot in ("bf16", "bf16v"):
        amp = torch.bfloat16
    ref = case.run(torch.float64, fused=False, device=ref_device, order=order, grads=grads)
    ea = case.run(torch.float32, fused=False, device=ref_device, amp=amp, order=order,
                  grads=grads)
    set_kernel_mode(kernel_mode)
    set_dot_mode(dot)
    try:
        fu = case.run(torch.float32, fused=True, device="cuda", amp=amp, order=order, grads=grads)
        fu2 = case.run(torch.float32, fused=True, device="cuda", amp=amp, order=order,
                       grads=grads)
    finally:
        set_dot_mode("")
        set_kernel_mode("auto")
    return compare(ref, ea, fu, fu2, amp=amp, gate=gate, blocked=blocked, strict=strict)


def compare(ref, ea, fu, fu2, amp=False, gate=1.25, blocked=False, strict=True):
    """The gates of the module docstring on result dicts (name -> tensor) of
    the float64 oracle (``ref``), eager fp32 (``ea``) and two runs of the
    HIP path (``fu``, ``fu2``); ``amp``: the 16-bit dtype of the inputs, or
    False. Returns (failures, rows of (name, eager err, fused err,
    fused-vs-eager))."""
    fails, rows = [], []
    for k in ref:
        if k not in fu:
            fails.append("%s missing from the fused run" % k)
            continue
        # with 16-bit activations out (x_mid's dtype) is 16-bit where the
        # fp32-upcast eager run's is fp32
        want_dtype = amp if (amp and k == "out") else ea[k].dtype
        if fu[k].shape != ea[k].shape or fu[k].dtype != want_dtype:
            fails.append("%s: shape/dtype %s %s vs eager %s %s" % (
                k, tuple(fu[k].shape), fu[k].dtype, tuple(ea[k].shape), ea[k].dtype))
        ee, ef, fe = relerr(ea[k], ref[k]), relerr(fu[k], ref[k]), relerr(fu[k], ea[k])
        rows.append((k, ee, ef, fe))
        if ref[k].norm() == 0:
            continue  # identically zero reference (G = 1): reported, not gated
        g = max(gate, 2.0) if (k == "grad:tau" and blocked) else gate
        if amp:
            ok = ef <= 2.0 * ee + 1e-6
        else:
            ok = ef <= g * ee + 1e-6 or (ee > 1e-4 and ef <= 3.0 * ee)
            # fused vs eager within 1e-5, up to eager's own distance from the
            # float64 truth (a result closer to the truth than eager can sit
            # on the other side of it: fe <= ef + ee)
            if strict and ok and ee < 1e-5 and fe > 1e-5 + ee:
                ok = False
        if not ok:
            fails.append("%s: eager %.3e fused %.3e fused-vs-eager %.3e" % (k, ee, ef, fe))
    for k in fu:
        if not torch.equal(fu[k], fu2[k]):
            fails.append("%s: two fused runs differ (not deterministic)" % k)
    return fails, rows
