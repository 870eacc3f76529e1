"""``kb_estep_vjp_noalloc`` (no work buffer, no device allocation) against ``kb_estep_vjp``, through the C ABI.

The no-allocation entry point runs the same kernels as ``kb_estep_vjp`` with
the library's own device scratch array instead of a caller work buffer, so its
outputs must be bitwise equal.  Two calls in a row, the second with fewer item
rows (the scratch keeps the first call's rows beyond the second call's G),
per dtype; sizes beyond the scratch and a non-NULL work pointer are refused.
"""

import ctypes as ct

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu

MAX_DOUBLES = 65536  # KB_ESTEP_VJP_NOALLOC_MAX (include/kbench_ops.h)


def _tree():
    from kbench.core.kernels import _hip as H

    h = kbtest.problem("3")["static"]["state_helpers"]
    t = lambda k: torch.as_tensor(np.asarray(h[k])).cuda()
    return H.tree_from_parent(t("node_parent"), t("node_child1"), t("node_child2")), int(h["S"]), h


def _case(G, S, h, dt, seed):
    """A forward E step at random E and rates, and random cotangents of its four outputs."""
    from kbench.core.kernels.e_step import e_step_triton_autograd

    g = np.random.default_rng(seed)
    r = lambda lo, hi: torch.as_tensor(g.uniform(lo, hi, size=(G, S)), dtype=dt, device="cuda")
    E, pS, pD, pL, mt = r(-6, -0.2), r(-4, -1), r(-4, -1), r(-4, -1), r(-14, -9)
    col = torch.as_tensor(g.normal(size=S) * 0.3 - np.log2(S), dtype=dt, device="cuda")
    topo = [torch.as_tensor(np.asarray(h[k])).cuda() for k in ("node_parent", "node_child1", "node_child2")]
    with torch.no_grad():
        En, Es1, Es2, Eb = e_step_triton_autograd(E, pS, pD, pL, mt, col, *topo, int(h["max_ancestor_depth"]),
                                                  use_col_weights=True)
    cot = [torch.as_tensor(g.normal(size=(G, S)), dtype=dt, device="cuda") for _ in range(4)]
    return dict(E=E, En=En, Es1=Es1, Es2=Es2, Eb=Eb, pS=pS, pD=pD, pL=pL, col=col, cot=cot)


def _run(entry, tree, c, dt, *, work):
    from kbench.core.kernels import _hip as H

    G, S = c["E"].shape
    outs = [torch.full((G, S), float("nan"), dtype=dt, device="cuda") for _ in range(5)]
    gcol = torch.zeros((S,), dtype=dt, device="cuda")  # the entry points add into it
    io = H.KbEStepVjpIO(
        dtype=H.dtype_code(dt), G=int(G), use_col_weights=1,
        E=H.ptr(c["E"]), E_new=H.ptr(c["En"]), E_s1=H.ptr(c["Es1"]), E_s2=H.ptr(c["Es2"]), Ebar=H.ptr(c["Eb"]),
        log_pS=H.ptr(c["pS"]), log_pD=H.ptr(c["pD"]), log_pL=H.ptr(c["pL"]), col_log_probs=H.ptr(c["col"]),
        g_E_new=H.ptr(c["cot"][0]), g_E_s1=H.ptr(c["cot"][1]), g_E_s2=H.ptr(c["cot"][2]), g_Ebar=H.ptr(c["cot"][3]),
        grad_E=H.ptr(outs[0]), grad_log_pS=H.ptr(outs[1]), grad_log_pD=H.ptr(outs[2]), grad_log_pL=H.ptr(outs[3]),
        grad_max_coupling=H.ptr(outs[4]), grad_col_log_probs=H.ptr(gcol), work=H.ptr(work),
    )
    rc = getattr(H.lib(), entry)(tree.handle, ct.byref(io), H.stream(c["E"].device))
    return rc, outs + [gcol]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_estep_vjp_noalloc_matches_the_allocating_entry_point(dt):
    from kbench.core.kernels import _hip as H

    tree, S, h = _tree()
    print(f"[no-alloc] kb_estep_vjp_noalloc vs kb_estep_vjp, S={S}, dtype={dt}", flush=True)
    for call, G in enumerate((MAX_DOUBLES // S, 3)):  # the full scratch, then a smaller input
        c = _case(G, S, h, dt, seed=100 + call)
        work = torch.empty((G, S), dtype=torch.float64, device="cuda")
        rc_a, ref = _run("kb_estep_vjp", tree, c, dt, work=work)
        H.check(rc_a)
        rc_b, got = _run("kb_estep_vjp_noalloc", tree, c, dt, work=None)
        H.check(rc_b)
        torch.cuda.synchronize()
        names = ("grad_E", "grad_log_pS", "grad_log_pD", "grad_log_pL", "grad_max_coupling", "grad_col")
        for name, a, b in zip(names, ref, got):
            assert bool(torch.isfinite(a).all()), name
            assert torch.equal(a, b), f"call {call} (G={G}): {name} differs"
        print(f"  call {call}: G={G} bitwise equal", flush=True)


def test_estep_vjp_noalloc_refuses_what_it_cannot_hold():
    from kbench.core.kernels import _hip as H

    tree, S, h = _tree()
    too_many = MAX_DOUBLES // S + 1
    c = _case(too_many, S, h, torch.float32, seed=7)
    rc, outs = _run("kb_estep_vjp_noalloc", tree, c, torch.float32, work=None)
    assert rc == -1 and "exceeds" in H.lib().kb_last_error().decode()
    c = _case(2, S, h, torch.float32, seed=8)
    work = torch.empty((2, S), dtype=torch.float64, device="cuda")
    rc, _ = _run("kb_estep_vjp_noalloc", tree, c, torch.float32, work=work)
    assert rc == -1 and "work" in H.lib().kb_last_error().decode()
    torch.cuda.synchronize()
    assert bool(torch.isnan(outs[0]).all())  # nothing was launched for the refused call
