"""The per-call wave loops captured as HIP graphs (``kbench.percall.graph.GraphedSolve``).

The forward and reverse graphs record the wrapper calls of ``SolvePlan``'s eager drivers (the
reference glue's call sequence, kbench/core/inference/forward.py:60-108 and
kbench/api/_implicit_grad.py:195-353), so on the same inputs a replay must give the eager
driver's results bitwise: on these uniform-theta-layout plans the bucket sums run in a fixed
order.  Through them the graphs meet the oracle (loss rel 1e-5, gradients rel 1e-4).

Three points are solved in turn with eager solves and host synchronizations between the
replays, and every replay is checked against the eager solve at its point, with one launch per
sweep and with the sweep chains fused (KBENCH_FUSE_SWEEPS).  Config 3 (per-species theta, the
generated size waves) is checked the same way at two points and timed both ways.
"""

import time

import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu

FUSE = pytest.mark.parametrize("fuse", [False, True], ids=["one_launch_per_sweep", "fused_sweep_chains"])


def _static(name, statewise=None):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    cap = problem_to_captured(kbtest.problem(name, statewise))
    return make_static(cap, "cuda"), cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


def _solve_both(g, plan, th, cw, *, backward=True):
    """(graph results, eager results) at th: loss, pi_wave, pibar_wave[, grad_theta, grad_col]."""
    loss, sv = g.forward(th, cw)
    out = [loss.clone(), sv["pi_wave"].clone(), sv["pibar_wave"].clone()]
    if backward:
        out += [x.clone() for x in g.backward(th, cw, sv)]
    torch.cuda.synchronize()
    eloss, esv = plan.forward(th, cw)
    ref = [eloss, esv["pi_wave"], esv["pibar_wave"]]
    if backward:
        ref += list(plan.backward(th, cw, esv))
    torch.cuda.synchronize()
    return out, ref


NAMES = ("loss", "pi_wave", "pibar_wave", "grad_theta", "grad_col")


@FUSE
@pytest.mark.parametrize("name,statewise,backward", [("tiny", None, True), ("1", None, True), ("1", True, True),
                                                     ("2", None, False)])
def test_graph_replays_equal_the_eager_driver_and_meet_the_oracle(name, statewise, backward, fuse, monkeypatch):
    from kbench.core.kernels import wave_step
    from kbench.percall import plan_of
    from kbench.percall.graph import GraphedSolve

    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", fuse)
    print(f"[percall graph] config={name} statewise={statewise} backward={backward} fuse_sweeps={fuse}", flush=True)
    static, theta, cw = _static(name, statewise)
    plan = plan_of(static)
    g = GraphedSolve(plan, theta, cw)
    for shift in (0.0, 0.25, -0.2):
        got, ref = _solve_both(g, plan, theta + shift, cw, backward=backward)
        same = [torch.equal(a, b) for a, b in zip(got, ref)]
        print(f"  theta+{shift}: loss={float(got[0]):.9g} bitwise equal: {dict(zip(NAMES, same))}", flush=True)
        assert all(same)
        if shift == 0.0:
            _, ref_loss, _ = kbtest.oracle_forward(name, statewise)
            rel = abs(float(got[0]) - ref_loss) / abs(ref_loss)
            print(f"  vs oracle: loss rel={rel:.3e}", flush=True)
            assert rel <= 1e-5
            if backward:
                ref_gt, ref_gc, _ = kbtest.oracle_backward(name, statewise)
                rt = kbtest.norm_rel(got[3].cpu().numpy(), ref_gt)
                rc = kbtest.norm_rel(got[4].cpu().numpy(), ref_gc)
                print(f"  vs oracle: grad_theta rel={rt:.3e} grad_col rel={rc:.3e}", flush=True)
                assert rt <= 1e-4 and rc <= 1e-4


def test_graph_refuses_what_it_cannot_replay():
    from kbench.percall import plan_of
    from kbench.percall.graph import GraphedSolve

    print("[percall graph] refusals", flush=True)
    static, theta, cw = _static("tiny")
    g = GraphedSolve(plan_of(static), theta, cw)
    with pytest.raises(ValueError):
        g.forward(theta.double(), cw)
    w = cw.clone()
    w.view(-1)[0] += 1.0
    with pytest.raises(ValueError):  # uniform at capture, weighted now
        g.forward(theta, w)
    with pytest.raises(RuntimeError):
        g.reverse({})


def test_config3_graph_replays_equal_the_eager_driver():
    """The graphs' outputs (loss, saved rows, the reverse loop's cotangents) equal the eager driver's
    bitwise.  The gradients add the eager E adjoint and theta VJP on both sides, whose torch autograd
    part need not repeat bitwise at this size: they are compared at rel 1e-6, with the spread of two
    eager runs printed beside."""
    from kbench.percall import plan_of
    from kbench.percall.graph import GraphedSolve
    from kbench.percall.solve import root_softmax2

    print("[percall graph] config 3, size waves", flush=True)
    static, theta, cw = _static("3")
    plan = plan_of(static)
    print(f"  waves={len(plan.waves)} rows={plan.C} S={plan.S}", flush=True)
    g = GraphedSolve(plan, theta, cw)
    for shift in (0.0, 0.1):
        th = theta + shift
        loss, sv = g.forward(th, cw)
        got = [loss.clone(), sv["pi_wave"].clone(), sv["pibar_wave"].clone()]
        acc = {k: v.clone() for k, v in vars(g.reverse(sv)).items()}
        gt, gc = (x.clone() for x in g.backward(th, cw, sv))
        torch.cuda.synchronize()
        eloss, esv = plan.forward(th, cw)
        with torch.no_grad():
            seed = -root_softmax2(esv["pi_wave"].index_select(0, plan.roots))
            eacc = vars(plan.reverse_sweep(esv, seed, use_col=g.weighted))
        egt, egc = plan.backward(th, cw, esv)
        egt2, egc2 = plan.backward(th, cw, esv)
        torch.cuda.synchronize()
        same = [torch.equal(a, b) for a, b in zip(got, (eloss, esv["pi_wave"], esv["pibar_wave"]))]
        same_acc = {k: torch.equal(acc[k], eacc[k]) for k in acc}
        print(f"  theta+{shift}: loss={float(got[0]):.9g} loss/pi/pibar equal: {same} cotangents equal: {same_acc}",
              flush=True)
        assert all(same) and all(same_acc.values())
        rt, rc = kbtest.norm_rel_t(gt, egt), kbtest.norm_rel_t(gc, egc)
        print(f"  gradients graph vs eager: theta rel={rt:.3e} col rel={rc:.3e}; eager vs eager: theta "
              f"rel={kbtest.norm_rel_t(egt2, egt):.3e} col rel={kbtest.norm_rel_t(egc2, egc):.3e}", flush=True)
        assert rt <= 1e-6 and rc <= 1e-6

    def clock(run):
        ts = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            run()
            torch.cuda.synchronize()
            ts.append(1e3 * (time.perf_counter() - t0))
        return min(ts)

    def graphed():
        _, sv = g.forward(theta, cw)
        g.backward(theta, cw, sv)

    def eager():
        _, sv = plan.forward(theta, cw)
        plan.backward(theta, cw, sv)

    print(f"  solve: eager per-call {clock(eager):.2f} ms, graph replays {clock(graphed):.2f} ms", flush=True)
