"""GPU parity of the native whole-pass driver against the CPU oracle."""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _run_fused_forward(name, statewise=None):
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    loss, saved = solver.run_forward(theta, cw)
    torch.cuda.synchronize()
    return solver, static, theta, cw, loss, saved


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True), ("2", None)])
def test_fused_forward_matches_oracle(name, statewise):
    print(f"[fused-forward] config={name} statewise={statewise}", flush=True)
    solver, static, theta, cw, loss, saved = _run_fused_forward(name, statewise)
    prob, ref_loss, ref = kbtest.oracle_forward(name, statewise)
    stats = solver.forward_stats()
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    print(f"  loss got={float(loss):.9g} ref={ref_loss:.9g} rel={rel:.3e} nE={stats['n_e_iter']}/{ref['n_e_iter']}")
    assert rel <= 1e-5
    for k in ("E", "E_s1", "E_s2", "Ebar"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and ma <= 1e-5
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5)


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True), ("2", None)])
def test_fused_backward_matches_oracle(name, statewise):
    print(f"[fused-backward] config={name} statewise={statewise}", flush=True)
    solver, static, theta, cw, loss, saved = _run_fused_forward(name, statewise)
    gt, gc, info = solver.run_backward(theta, cw, saved, return_info=True)
    stats = solver.backward_stats()
    torch.cuda.synchronize()
    # oracle backward on the oracle's own forward (independent chain)
    ref_gt, ref_gc, ref_info = kbtest.oracle_backward(name, statewise)
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  grad_theta normrel={rt:.3e}  grad_col normrel={rc:.3e}  bicgstab={stats['n_bicgstab']}/{ref_info['n_bicgstab']}")
    mask = info["active_mask"].cpu().numpy().astype(bool)
    ref_mask = np.zeros_like(mask)
    for ws, act in ref_info["masks"]:
        ref_mask[ws:ws + act.shape[0]] = act
    print(f"  active rows got={mask.sum()} ref={ref_mask.sum()} mismatches={(mask != ref_mask).sum()}")
    acc = info["acc"].cpu().numpy()
    names = ["g_pD", "g_pS", "g_E", "g_Ebar", "g_Es1", "g_Es2", "g_mt", "g_col"]
    for j, nm in enumerate(names):
        ref = np.asarray(ref_info["acc"][nm], dtype=np.float64).reshape(-1)
        got = acc[j]
        if ref.size == 1:
            got = np.array([got.sum()])
        print(f"  acc {nm}: normrel={kbtest.norm_rel(got, ref):.3e}")
    assert (mask == ref_mask).all()
    assert rt <= 1e-4 and rc <= 1e-4


@pytest.mark.parametrize("name,statewise", [("1", True), ("2", None)])
def test_row_classes_match_per_row_solve(name, statewise, monkeypatch):
    """Computing each class of identical rows once (default) equals solving every row (KB_DEDUP=0)."""
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    out = []
    for flag in ("1", "0"):
        monkeypatch.setenv("KB_DEDUP", flag)
        solver = FusedSolver(static, static.solver_options)
        loss, saved = solver.run_forward(theta, cw)
        gt, gc, info = solver.run_backward(theta, cw, saved, return_info=True)
        torch.cuda.synchronize()
        out.append((float(loss), saved["pi_wave"].cpu().numpy(), gt.cpu().numpy(), gc.cpu().numpy(),
                    info["active_mask"].cpu().numpy()))
    (l1, pi1, gt1, gc1, m1), (l0, pi0, gt0, gc0, m0) = out
    # forward rows are bitwise equal when a class's splits come in the same order; allow rounding otherwise
    ok, ma, mr = kbtest.compare_inf_safe(pi1, pi0)
    print(f"  loss {l1:.9g} vs {l0:.9g}; pi max_abs={ma:.3e}; grads {kbtest.norm_rel(gt1, gt0):.3e} "
          f"{kbtest.norm_rel(gc1, gc0):.3e}")
    assert ok and (ma <= 1e-4 or mr <= 1e-6)
    assert abs(l1 - l0) <= 1e-6 * abs(l0)
    assert (m1 == m0).all()
    assert kbtest.norm_rel(gt1, gt0) <= 1e-5 and kbtest.norm_rel(gc1, gc0) <= 1e-5


def test_backward_reuses_forward_split_terms_only_when_valid():
    """The backward reuses the forward's stored split terms for that forward's own outputs, and
    recomputes them from pi / pibar otherwise (copies, or outputs of an older forward)."""
    solver, static, theta, cw, loss, saved = _run_fused_forward("1", True)
    g_reuse = solver.run_backward(theta, cw, saved)
    other = dict(saved)
    other["pi_wave"] = saved["pi_wave"].clone()
    other["pibar_wave"] = saved["pibar_wave"].clone()
    g_recompute = solver.run_backward(theta, cw, other)
    _, saved2 = solver.run_forward(theta * 1.01, cw)      # a newer forward on the same plan
    g_old = solver.run_backward(theta, cw, saved)         # must not use the newer split terms
    torch.cuda.synchronize()
    for a, b, c in zip(g_reuse, g_recompute, g_old):
        assert kbtest.norm_rel(a.cpu().numpy(), b.cpu().numpy()) <= 1e-6
        assert kbtest.norm_rel(a.cpu().numpy(), c.cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("name,statewise", [("1", True), ("2", None)])
def test_fused_weighted_columns_match_oracle(name, statewise):
    """Non-uniform column weights: the weighted row kernels and the column branches of the
    E-step and the epilogue against the oracle on the same (float32-rounded) weights."""
    import kbench_oracle as O
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[fused-weighted] config={name} statewise={statewise}", flush=True)
    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    rng = np.random.default_rng(11)
    cw32 = rng.normal(0.0, 0.5, size=int(cap["inputs"]["col_weights"].numel())).astype(np.float32)
    cw = torch.from_numpy(cw32).cuda()
    loss, saved = solver.run_forward(theta, cw)
    gt, gc = solver.run_backward(theta, cw, saved)
    torch.cuda.synchronize()

    prob = O.Problem.from_dict(p)
    th64 = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw64 = cw32.astype(np.float64)
    ref_loss, ref = O.forward(prob, th64, cw64)
    ref_gt, ref_gc, _info, _extra = O.backward(prob, th64, cw64, ref, collect=True)
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    ok, ma, mr = kbtest.compare_inf_safe(saved["pi_wave"].cpu().numpy(), ref["pi_wave"])
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  loss rel={rel:.3e} pi ok={ok} max_abs={ma:.3e} grad_theta={rt:.3e} grad_col={rc:.3e}")
    assert rel <= 1e-5
    assert ok and (ma <= 2e-4 or mr <= 1e-5)
    assert rt <= 1e-4 and rc <= 1e-4


def _big_tree_problem(leaves, families, statewise):
    """Large species tree, few families: the 2048-, 4096- and 8192-position row kernels at an oracle-sized C."""
    from kbench import synth

    cfg = synth.ProblemConfig(leaves, families, n_nni=1, family_leaves_median=21.0, family_leaves_sigma=0.6,
                              family_leaves_max=80, statewise=statewise, seed=17)
    return synth.build_problem(cfg)


@pytest.mark.parametrize("leaves,families,statewise,weighted", [(1024, 6, True, False), (1024, 6, False, True),
                                                                (2048, 4, True, False), (2048, 4, False, True),
                                                                (4096, 3, False, False), (4096, 3, True, True)])
@pytest.mark.parametrize("shapes", ["default", "wide"])
def test_fused_large_trees_match_oracle(leaves, families, statewise, weighted, shapes, monkeypatch):
    """S = 2047, 4095 and 8191: forward rows, loss and gradients against the oracle, with the default
    launch shapes (narrow shapes on these small levels) and with the wide ones forced."""
    import kbench_oracle as O
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    if shapes == "wide":
        monkeypatch.setenv("KB_FWD_WIDE", "3")
        monkeypatch.setenv("KB_BWD_VARIANT", "0")
    print(f"[fused-large] leaves={leaves} statewise={statewise} weighted={weighted} shapes={shapes}", flush=True)
    p = _big_tree_problem(leaves, families, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    n = int(cap["inputs"]["col_weights"].numel())
    cw32 = (np.random.default_rng(5).normal(0.0, 0.5, size=n) if weighted else np.zeros(n)).astype(np.float32)
    cw = torch.from_numpy(cw32).cuda()
    loss, saved = solver.run_forward(theta, cw)
    gt, gc = solver.run_backward(theta, cw, saved)
    torch.cuda.synchronize()

    prob = O.Problem.from_dict(p)
    th64 = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    ref_loss, ref = O.forward(prob, th64, cw32.astype(np.float64))
    ref_gt, ref_gc, _info, _extra = O.backward(prob, th64, cw32.astype(np.float64), ref, collect=True)
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    ok, ma, mr = kbtest.compare_inf_safe(saved["pi_wave"].cpu().numpy(), ref["pi_wave"])
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  S={prob.S} C={prob.C} loss rel={rel:.3e} pi ok={ok} max_abs={ma:.3e} "
          f"grad_theta={rt:.3e} grad_col={rc:.3e}")
    assert rel <= 1e-5
    assert ok and (ma <= 2e-4 or mr <= 1e-5)
    assert rt <= 1e-4 and rc <= 1e-4


@pytest.mark.parametrize("weighted", [False, True])
def test_large_tree_forward_kernels_agree(weighted, monkeypatch):
    """S = 8191: the contiguous-ownership forward on the owner-major tables against the Euler-tour
    kernel (KB_FWD_LARGE=0): same loss and Pi rows to float32 rounding."""
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[fused-large-fwd-ab] weighted={weighted}", flush=True)
    p = _big_tree_problem(4096, 3, True)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    n = int(cap["inputs"]["col_weights"].numel())
    cw32 = (np.random.default_rng(9).normal(0.0, 0.5, size=n) if weighted else np.zeros(n)).astype(np.float32)
    cw = torch.from_numpy(cw32).cuda()
    runs = {}
    for large in ("1", "0"):
        monkeypatch.setenv("KB_FWD_LARGE", large)
        loss, saved = solver.run_forward(theta, cw)
        torch.cuda.synchronize()
        runs[large] = (float(loss), saved["pi_wave"].cpu().numpy(), saved["pibar_wave"].cpu().numpy())
    rel = abs(runs["1"][0] - runs["0"][0]) / abs(runs["0"][0])
    for j, name in ((1, "pi_wave"), (2, "pibar_wave")):
        ok, ma, mr = kbtest.compare_inf_safe(runs["1"][j], runs["0"][j])
        print(f"  {name}: pattern={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5)
    print(f"  loss rel={rel:.3e}")
    assert rel <= 1e-6


@pytest.mark.parametrize("leaves,weighted", [(1024, True), (2048, False), (4096, True)])
def test_large_tree_backward_kernels_agree(leaves, weighted, monkeypatch):
    """S = 2047, 4095 and 8191: the low-register backward row kernel (at S = 2047 its 512-thread shape,
    KB_BWD_LARGE=2) against the general one (KB_BWD_LARGE=0) on the same forward; each run twice is
    bitwise reproducible."""
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[fused-large-ab] leaves={leaves} weighted={weighted}", flush=True)
    p = _big_tree_problem(leaves, 3, True)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    n = int(cap["inputs"]["col_weights"].numel())
    cw32 = (np.random.default_rng(7).normal(0.0, 0.5, size=n) if weighted else np.zeros(n)).astype(np.float32)
    cw = torch.from_numpy(cw32).cuda()
    _, saved = solver.run_forward(theta, cw)
    runs = {}
    on = "2" if leaves <= 1024 else "1"
    for large in (on, "0", on):
        monkeypatch.setenv("KB_BWD_LARGE", large)
        gt, gc = solver.run_backward(theta, cw, saved)
        torch.cuda.synchronize()
        if large in runs:
            assert torch.equal(gt, runs[large][0]) and torch.equal(gc, runs[large][1])
        runs[large] = (gt.clone(), gc.clone())
    rt = kbtest.norm_rel(runs[on][0].cpu().numpy(), runs["0"][0].cpu().numpy())
    rc = kbtest.norm_rel(runs[on][1].cpu().numpy(), runs["0"][1].cpu().numpy())
    print(f"  low-register vs general kernel: grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rt <= 1e-5 and rc <= 1e-5


@pytest.mark.parametrize("statewise", [False, True])
def test_fused_single_leaf_families_match_oracle(statewise):
    """Families of one gene leaf: their root row is a leaf row, so level 0 holds root members (the root
    seed in the level-0 chunk path; two of them share a species, so one class holds two roots)."""
    import kbench_oracle as O
    from kbench import synth
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[fused-single-leaf] statewise={statewise}", flush=True)
    cfg = synth.ProblemConfig(32, 6, n_nni=1, family_leaves_median=4.0, family_leaves_sigma=0.5,
                              family_leaves_max=10, statewise=statewise, seed=23, single_leaf_families=3)
    p = synth.build_problem(cfg)
    roots = np.asarray(p["static"]["wave_layout"]["root_row_ids"])
    w0 = p["static"]["wave_layout"]["wave_metas"][0]
    assert np.sum(roots < int(w0["start"]) + int(w0["W"])) == 3  # three roots among the leaf rows
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    loss, saved = solver.run_forward(theta, cw)
    gt, gc, info = solver.run_backward(theta, cw, saved, return_info=True)
    torch.cuda.synchronize()

    prob = O.Problem.from_dict(p)
    th64 = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw64 = np.asarray(p["inputs"]["col_weights"], dtype=np.float32).astype(np.float64)
    ref_loss, ref = O.forward(prob, th64, cw64)
    ref_gt, ref_gc, _info, extra = O.backward(prob, th64, cw64, ref, collect=True)
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    ok, ma, mr = kbtest.compare_inf_safe(saved["pi_wave"].cpu().numpy(), ref["pi_wave"])
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  S={prob.S} C={prob.C} loss rel={rel:.3e} pi ok={ok} max_abs={ma:.3e} "
          f"grad_theta={rt:.3e} grad_col={rc:.3e}")
    assert rel <= 1e-5
    assert ok and (ma <= 2e-4 or mr <= 1e-5)
    assert rt <= 1e-4 and rc <= 1e-4
    mask = info["active_mask"].cpu().numpy().astype(bool)
    ref_mask = np.zeros_like(mask)
    for ws, act in extra["masks"]:
        ref_mask[ws:ws + len(act)] = act
    assert np.array_equal(mask, ref_mask)


@pytest.mark.parametrize("bad", [-1, "S"])
def test_plan_rejects_leaf_rows_without_a_valid_state(bad):
    """A leaf row's leaf state indexes the state axis: out of range it is refused at plan creation
    (before any kernel could read outside the tables)."""
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem("tiny", None)
    cap = problem_to_captured(p)
    wl = cap["static"]["wave_layout"]
    leaf = wl["leaf_state_index"].clone()
    w0 = wl["wave_metas"][0]
    S = int(cap["static"]["state_helpers"]["S"])
    leaf[int(w0["start"])] = S if bad == "S" else bad
    wl["leaf_state_index"] = leaf
    static = make_static(cap, "cuda")
    with pytest.raises(ValueError, match="leaf state"):
        FusedSolver(static, static.solver_options)


@pytest.mark.parametrize("leaves,weighted", [(1024, True), (2048, False)])
def test_backward_on_a_one_workgroup_grid_matches_oracle(leaves, weighted, monkeypatch):
    """KB_BWD_GRID=1: one persistent workgroup walks every row of each level, so the 1024 x 2
    kernel reloads its LDS chunk of 64 row records and the large-row kernel (S = 4095) keeps one
    bucket slot for a whole level.  Gradients against the oracle and the default grid."""
    import kbench_oracle as O
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[fused-grid1] leaves={leaves} weighted={weighted}", flush=True)
    p = _big_tree_problem(leaves, 16 if leaves == 1024 else 12, True)  # level 1: 130 / 123 rows
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    theta = cap["inputs"]["theta"].cuda()
    n = int(cap["inputs"]["col_weights"].numel())
    cw32 = (np.random.default_rng(11).normal(0.0, 0.5, size=n) if weighted else np.zeros(n)).astype(np.float32)
    cw = torch.from_numpy(cw32).cuda()
    ref = FusedSolver(static, static.solver_options)
    _, saved = ref.run_forward(theta, cw)
    gt0, gc0 = ref.run_backward(theta, cw, saved)
    monkeypatch.setenv("KB_BWD_GRID", "1")
    one = FusedSolver(static, static.solver_options)
    level_rows = one.level_shapes()[0][1:]
    _, saved1 = one.run_forward(theta, cw)
    gt1, gc1 = one.run_backward(theta, cw, saved1)
    torch.cuda.synchronize()
    prob = O.Problem.from_dict(p)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    _, osv = O.forward(prob, th, cw32.astype(np.float64))
    ogt, ogc, _ = O.backward(prob, th, cw32.astype(np.float64), osv)
    rt = kbtest.norm_rel(gt1.cpu().numpy(), ogt)
    rc = kbtest.norm_rel(gc1.cpu().numpy(), ogc)
    dt = kbtest.norm_rel(gt1.cpu().numpy(), gt0.cpu().numpy())
    dc = kbtest.norm_rel(gc1.cpu().numpy(), gc0.cpu().numpy())
    print(f"  rows per split level (max) {int(level_rows.max())}; vs oracle theta={rt:.2e} col={rc:.2e}; "
          f"vs default grid theta={dt:.2e} col={dc:.2e}")
    assert int(level_rows.max()) > 64
    assert rt <= 1e-4 and rc <= 1e-4
    assert dt <= 1e-5 and dc <= 1e-5
