"""``FusedSolver.solve``: a forward and its backward in one call (``kb_solve``).

With an overlap cut, the backward rows of the families whose root lies at or
below the cut run on a second stream, down to the window's lowest level,
while the forward's later levels run; the other rows, the levels below the
window, level 0 and the epilogue follow on the caller's stream.  The
result must be the forward and backward of separate calls: the loss and the
forward's rows bitwise (the forward is the same launches), the active masks
bitwise, the gradients up to the order of the bucket sums (the early rows
add into a second set of workgroup slots); and two solves bitwise equal.
Checked with forced cuts and windows on configs 1 and 2 and on an S = 4095
tree (the large-row kernel's slot offset), against the oracle as well, and
with the default cut and window on config 3 (the bench's workload), where an
overlap is chosen; and captured as one HIP graph, whose replays equal the
eager solve bitwise.
"""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _solvers(p, monkeypatch, cut, low=None):
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    monkeypatch.setenv("KB_OVERLAP_CUT", "-1")
    plain = FusedSolver(static, static.solver_options)
    if cut is None:
        monkeypatch.delenv("KB_OVERLAP_CUT")
    else:
        monkeypatch.setenv("KB_OVERLAP_CUT", str(cut))
    if low is not None:
        monkeypatch.setenv("KB_OVERLAP_LOW", str(low))
    over = FusedSolver(static, static.solver_options)
    return plain, over, theta, cw


def _compare(plain, over, theta, cw):
    loss0, saved0 = plain.run_forward(theta, cw)
    gt0, gc0, info0 = plain.run_backward(theta, cw, saved0, return_info=True)
    loss1, saved1, gt1, gc1, info1 = over.solve(theta, cw, return_info=True)
    loss2, _, gt2, gc2 = over.solve(theta, cw)
    torch.cuda.synchronize()
    assert float(loss1) == float(loss0)
    assert torch.equal(saved1["pi_wave"], saved0["pi_wave"]) and torch.equal(saved1["pibar_wave"], saved0["pibar_wave"])
    assert torch.equal(info1["active_mask"], info0["active_mask"])
    rt = kbtest.norm_rel(gt1.cpu().numpy(), gt0.cpu().numpy())
    rc = kbtest.norm_rel(gc1.cpu().numpy(), gc0.cpu().numpy())
    print(f"  cut={over.overlap_cut} early rows={over.overlap_rows}: grad_theta rel={rt:.2e} grad_col rel={rc:.2e}")
    assert rt <= 1e-6 and rc <= 1e-6
    assert float(loss2) == float(loss1) and torch.equal(gt2, gt1) and torch.equal(gc2, gc1)
    return gt1, gc1


@pytest.mark.parametrize("name,statewise,cut,low", [("1", True, 3, None), ("1", True, 2, None), ("2", None, 4, None),
                                                    ("1", True, 4, 2), ("2", None, 5, 3)])
def test_overlapped_solve_matches_separate_calls_and_oracle(name, statewise, cut, low, monkeypatch):
    print(f"[solve] config={name} statewise={statewise} cut={cut} low={low}", flush=True)
    plain, over, theta, cw = _solvers(kbtest.problem(name, statewise), monkeypatch, cut, low)
    assert over.overlap_cut == cut and over.overlap_rows > 0 and over.overlap_low == (low or 1)
    gt, gc = _compare(plain, over, theta, cw)
    ref_gt, ref_gc, _ = kbtest.oracle_backward(name, statewise)
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  vs oracle: grad_theta rel={rt:.2e} grad_col rel={rc:.2e}")
    assert rt <= 1e-4 and rc <= 1e-4


def test_overlapped_solve_on_a_large_tree(monkeypatch):
    """S = 4095: the large-row backward kernel's early launches use the second slot set."""
    from kbench import synth

    print("[solve] S=4095 cut=6", flush=True)
    cfg = synth.ProblemConfig(2048, 12, n_nni=1, family_leaves_median=21.0, family_leaves_sigma=0.6,
                              family_leaves_max=80, statewise=True, seed=17)
    # the families' roots lie at levels 4, 5, 7, ...: cut 6 takes the first two
    plain, over, theta, cw = _solvers(synth.build_problem(cfg), monkeypatch, 6)
    assert over.S == 4095 and over.overlap_rows > 0
    _compare(plain, over, theta, cw)


def test_default_cut_overlaps_config3_and_not_config1(monkeypatch):
    print("[solve] default cut: config 3 and config 1", flush=True)
    plain, over, theta, cw = _solvers(kbtest.problem("3"), monkeypatch, None)
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    assert over.overlap_cut >= 1 and over.overlap_rows >= n_cu
    _compare(plain, over, theta, cw)
    plain, over, theta, cw = _solvers(kbtest.problem("1", True), monkeypatch, None)
    assert over.overlap_cut == -1 and over.overlap_rows == 0
    loss0, saved0 = plain.run_forward(theta, cw)
    gt0, gc0 = plain.run_backward(theta, cw, saved0)
    loss1, _, gt1, gc1 = over.solve(theta, cw)
    torch.cuda.synchronize()
    assert float(loss1) == float(loss0) and torch.equal(gt1, gt0) and torch.equal(gc1, gc0)


def test_overlapped_solve_replays_from_a_hip_graph(monkeypatch):
    """The one-call solve captured as one HIP graph: the second stream's launches join the capture
    through the fork / join events; every replay, with eager solves between them, equals the eager
    solve bitwise."""
    print("[solve] HIP graph of the one-call solve, config 2 cut 4", flush=True)
    plain, over, theta, cw = _solvers(kbtest.problem("2", None), monkeypatch, 4)
    assert over.overlap_cut == 4 and over.overlap_rows > 0
    loss0, _, gt0, gc0 = over.solve(theta, cw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        loss_g, _, gt_g, gc_g = over.solve(theta, cw, check_solve=False)
    for i in range(3):
        loss_e, _, gt_e, gc_e = over.solve(theta, cw)  # eager work between the replays
        plain.run_backward(theta, cw, plain.run_forward(theta, cw)[1])
        torch.cuda.synchronize()
        gt_g.zero_()
        gc_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        print(f"  replay {i}: loss {float(loss_g):.6f}", flush=True)
        assert float(loss_g) == float(loss0) == float(loss_e)
        assert torch.equal(gt_g, gt0) and torch.equal(gc_g, gc0)
        assert torch.equal(gt_e, gt0) and torch.equal(gc_e, gc0)
    over.backward_stats()  # the E-adjoint solve of the last replay succeeded


def test_solve_refuses_a_backward_that_does_not_read_the_forwards_outputs(monkeypatch):
    """kb_solve checks on the host, before any launch, that the backward io names the forward's outputs."""
    import ctypes as ct

    from kbench import _native as N

    print("[solve] mismatched backward io", flush=True)
    _, over, theta, cw = _solvers(kbtest.problem("1", True), monkeypatch, 3)
    fio, _, saved, keep = over._forward_args(theta, cw, None)
    bio, _, _, _ = over._backward_args(theta, cw, saved, False)
    other = torch.empty_like(saved["pi_wave"])
    bio.pi = N.ptr(other)
    with torch.cuda.device(over.device):
        with pytest.raises(ValueError, match="forward.s outputs"):
            N.check(N.lib().kb_solve(over._plan, ct.byref(fio), ct.byref(bio), N.stream_handle(over.device)))
    del keep
    loss, _, gt, gc = over.solve(theta, cw)  # the plan still works
    torch.cuda.synchronize()
    assert torch.isfinite(gt).all() and torch.isfinite(gc).all() and float(loss) == float(loss)
