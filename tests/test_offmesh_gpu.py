"""Off-mesh deslice (reference ROADMAP.md:74-75: "the kernels take a
query-side x_mid with its own N today; add the example and the test").

The slice runs on the mesh points (x_mid, fx_mid: N_mesh rows); the tokens
it forms are deslided onto a different point set, the queries (x_query:
N_query rows, e.g. probe locations or a finer output mesh), through the
same slice projection W, b, tau. Forward and backward through the public
API, held to the CPU oracle with the gates of ``tests/parity.py``; gradients
reach both point sets and the shared parameters.
"""

import math

import pytest
import torch

import oracle
from parity import relerr
from flashslice_amd.kernels import fused_deslice, fused_slice

pytestmark = pytest.mark.gpu


def _run(L, up, dtype, device, fused):
    T = {k: v.detach().to(device=device, dtype=dtype).requires_grad_(True) for k, v in L.items()}
    if fused:
        z, s = fused_slice(T["x"], T["fx"], T["w"], T["b"], T["tau"])
        tok = z / (s + oracle.EPS_TOKEN)[..., None]
        out = fused_deslice(T["xq"], T["w"], T["b"], T["tau"], tok)
    else:
        z, s = oracle.slice_fwd(T["x"], T["fx"], T["w"], T["b"], T["tau"])
        tok = z / (s + oracle.EPS_TOKEN)[..., None]
        out = oracle.deslice_fwd(T["xq"], T["w"], T["b"], T["tau"], tok)
    loss = oracle.coupling_loss(out, z, s, up["out"].to(device), up["z"].to(device),
                                up["s"].to(device))
    loss.backward()
    res = {"out": out.detach(), "z_num": z.detach(), "s": s.detach()}
    res.update({"grad:" + k: v.grad.detach() for k, v in T.items()})
    return res


@pytest.mark.parametrize("n_mesh,n_query,G", [(5000, 1237, 32), (777, 20000, 64), (3000, 1, 32)])
def test_offmesh_deslice(n_mesh, n_query, G):
    g = torch.Generator().manual_seed(11)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    B, H, D = 2, 4, 32
    L = {"x": r(B, n_mesh, H, D), "fx": r(B, n_mesh, H, D), "xq": r(B, n_query, H, D),
         "w": r(H, G, D) / math.sqrt(D), "b": 0.1 * r(H, G),
         "tau": 0.3 + 0.7 * torch.rand(H, generator=g)}
    up = {"out": r(B, n_query, H, D), "z": r(B, H, G, D), "s": r(B, H, G)}
    ref = _run(L, up, torch.float64, "cpu", False)
    ea = _run(L, up, torch.float32, "cpu", False)
    fu = _run(L, up, torch.float32, "cuda", True)
    fails = []
    for k in ref:
        ee, ef, fe = relerr(ea[k], ref[k]), relerr(fu[k], ref[k]), relerr(fu[k], ea[k])
        print("  %-10s eager %.3e  fused %.3e  fused-vs-eager %.3e" % (k, ee, ef, fe))
        assert fu[k].shape == ea[k].shape and fu[k].dtype == ea[k].dtype, k
        ok = ef <= 1.25 * ee + 1e-6 or (ee > 1e-4 and ef <= 3.0 * ee)
        if ok and ee < 1e-5 and fe > 1e-5 + ee:
            ok = False
        if not ok:
            fails.append("%s: eager %.3e fused %.3e fused-vs-eager %.3e" % (k, ee, ef, fe))
    assert not fails, "\n".join(fails)
