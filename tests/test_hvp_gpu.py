"""GPU parity of the second-order wrappers (kbench.core.kernels.{e_step,wave,dts}_so) and of the
exact / Gauss-Newton HVP call sequences (kbench/newton/hvp.py) against the float64 CPU oracle.

Kernel tests feed the oracle's primal point and random tangents / cotangents
to the HIP wrappers in float64 (tight tolerance) and float32 (rel 1e-4).  The
exact HVP runs the glue on the GPU's own fp32 forward and is compared with
the oracle's HVP at the oracle's forward.  The config-3 checks (the S = 2047
per-species setup of the Newton-CG benchmark, where the oracle is out of
reach) are in test_hvp_config3_gpu.py.
"""

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-9, torch.float32: 1e-4}


def _static(name, statewise=None):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    return static, cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


def _t(x, dt):
    return torch.as_tensor(np.ascontiguousarray(x), dtype=dt, device="cuda")


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all()
    return float(np.abs(got - ref).max()) / max(1.0, float(np.abs(ref).max()))


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("use_col", [False, True])
def test_e_step_backward_so_matches_oracle(dt, use_col):
    print(f"[e-so] dtype={dt} use_col={use_col}", flush=True)
    static, _, _ = _static("1")
    prob, _, _ = kbtest.oracle_forward("1")
    _eso_case(prob, static.state_helpers, dt, use_col)


@pytest.mark.parametrize("use_col", [False, True])
def test_e_step_backward_so_on_long_float32_rows(use_col):
    """S = 8191: float32 rows too long for three float64 LDS rows compute in float32 (1e-4 of the max
    against the float64 oracle); float64 rows of that length stop with the wrappers' ValueError."""
    print(f"[e-so] S=8191 float32 use_col={use_col}", flush=True)
    problem, static, _, _ = _big_tree(4096, True)
    prob = O.Problem.from_dict(problem)
    assert prob.S == 8191
    _eso_case(prob, static.state_helpers, torch.float32, use_col)
    with pytest.raises(ValueError, match="LDS"):
        _eso_case(prob, static.state_helpers, torch.float64, use_col, check=False)


def _eso_case(prob, h, dt, use_col, check=True):
    from kbench.core.kernels.e_step_so import e_step_backward_so

    rng = np.random.default_rng(31)
    S, G, tree = prob.S, 3, prob.tree
    E = np.log2(rng.uniform(0.05, 0.6, (G, S)))
    pS, pD, pL, mt = (rng.uniform(-4, -0.5, (G, S)) for _ in range(4))
    col = rng.uniform(-1, 1, S)
    En, Es1, Es2, Eb = O.e_step(E, pS, pD, pL, mt, col, tree, use_col)
    gN, gB = rng.normal(size=(G, S)), rng.normal(size=(G, S))
    dE, dEn, dEs1, dEs2, dEb, dpS, dpD, dpL = (rng.normal(size=(G, S)) for _ in range(8))
    dEs1 = np.where(np.isfinite(Es1), dEs1, 0.0)
    dEs2 = np.where(np.isfinite(Es2), dEs2, 0.0)
    dEb = np.where(np.isfinite(Eb), dEb, 0.0)
    dcol = rng.normal(size=S)
    ref = None if not check else O.e_step_backward_so(E, En, Es1, Es2, Eb, pS, pD, pL, col, tree, gN, gB, dE, dEn,
                                                        dEs1, dEs2, dEb, dpS, dpD, dpL, dcol, use_col)
    got = e_step_backward_so(*(_t(x, dt) for x in (E, En, Es1, Es2, Eb, pS, pD, pL, col)), h["node_parent"],
                             h["node_child1"], h["node_child2"], int(h["max_ancestor_depth"]), _t(gN, dt), None, None,
                             _t(gB, dt), *(_t(x, dt) for x in (dE, dEn, dEs1, dEs2, dEb, dpS, dpD, dpL, dcol)),
                             use_col_weights=use_col)
    torch.cuda.synchronize()
    if not check:
        return
    for name, g, r in zip(("dE", "dpS", "dpD", "dpL", "dmc", "dcol"), got, ref):
        e = _rel(g.cpu().numpy(), r)
        print(f"  {name}: rel={e:.3e}")
        assert e <= TOL[dt]


def _wave_consts(prob, saved, rng):
    S, G = prob.S, 1
    E = np.asarray(saved["E"])
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    pS, pD, mt = st(saved["log_pS"]), st(saved["log_pD"]), st(saved["max_coupling"])
    consts = O.WaveConsts(mt=mt, DL=1.0 + pD + E, Ebar=np.asarray(saved["Ebar"]), E=E, SL1=pS + saved["E_s2"],
                          SL2=pS + saved["E_s1"], leaf_logp=pS, col=np.zeros(S), use_col_weights=False)
    dc = O.WaveTangentConsts(*(0.3 * rng.normal(size=(G, S)) for _ in range(7)))
    return consts, dc


@pytest.mark.parametrize("name,dt", [("1", torch.float64), ("1", torch.float32), ("big", torch.float32)])
def test_wave_backward_so_matches_oracle(name, dt):
    """Config 1, and S = 8191 ("big") in float32, where the generic kernel's rows are too long for three
    float64 LDS rows and it computes in float32."""
    from kbench.core.kernels.wave_so import wave_backward_so

    print(f"[wave-so] config={name} dtype={dt}", flush=True)
    if name == "big":
        problem, static, _, _ = _big_tree(4096, True)
        prob = O.Problem.from_dict(problem)
        th = np.asarray(problem["inputs"]["theta"], dtype=np.float32).astype(np.float64)
        _, saved = O.forward(prob, th, np.asarray(problem["inputs"]["col_weights"], dtype=np.float64))
    else:
        static, _, _ = _static(name)
        prob, _, saved = kbtest.oracle_forward(name)
    rng = np.random.default_rng(32)
    S, G, C = prob.S, 1, prob.C
    consts, dc = _wave_consts(prob, saved, rng)
    Pi, Pb, rmax = saved["pi_wave"], saved["pibar_wave"], saved["pibar_row_max"]
    fd_dir = lambda X: np.where(np.isfinite(X), rng.normal(size=X.shape), 0.0)
    dPi, dPb = fd_dir(Pi), fd_dir(Pb)
    d_rhs = rng.normal(size=(C, S))
    h = static.state_helpers
    cargs = [_t(x, dt) for x in (consts.mt, consts.DL, dc.dDL, consts.Ebar, dc.dEbar, consts.E, dc.dE, consts.SL1,
                                  dc.dSL1, consts.SL2, dc.dSL2)]
    pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    worst = 0.0
    n_w = len(prob.wave_metas)
    for i in (0, 1, n_w // 2, n_w - 1):
        mo = prob.wave_metas[i]
        ws, W = int(mo["start"]), int(mo["W"])
        rows = np.arange(ws, ws + W)
        split = "sl" in mo
        leaf = None if split else prob.leaf_state[rows]
        dts = d_dts = None
        if split:
            dts = O.dts_forward(Pi, Pb, mo, W, pDp, pSp, prob.item_idx, ws, prob.tree)
            d_dts = fd_dir(dts)
        v = rng.normal(size=(W, S))
        ref = O.wave_backward_so(Pi[rows], dPi[rows], Pb[rows], dPb[rows], v, rmax[rows], prob.item_idx[rows], consts,
                                 dc, prob.tree, leaf_state=leaf, dts_r=dts, d_dts=d_dts, rhs_rows=d_rhs[rows])
        got = wave_backward_so(_t(Pi, dt), _t(dPi, dt), _t(Pb, dt), _t(dPb, dt), _t(v, dt), ws, W, S, _t(rmax, dt),
                               *cargs, None, h["node_child1"], h["node_child2"], h["node_parent"],
                               int(h["max_ancestor_depth"]), None if dts is None else _t(dts, dt),
                               None if d_dts is None else _t(d_dts, dt),
                               leaf_state_idx=static.wave_layout["leaf_state_index"], leaf_logp=_t(consts.leaf_logp, dt),
                               dleaf_logp=_t(dc.dleaf, dt), item_idx=static.rate_item_idx, has_leaf_term=not split,
                               use_col_weights=False, d_rhs=_t(d_rhs, dt))
        torch.cuda.synchronize()
        for g, r in zip(got, ref):
            worst = max(worst, _rel(g.cpu().numpy(), r))
    print(f"  worst rel={worst:.3e}")
    assert worst <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("statewise", [False, True])
def test_dts_backward_so_matches_oracle(dt, statewise):
    from kbench.core.kernels.dts_so import dts_backward_so

    print(f"[dts-so] config=1 statewise={statewise} dtype={dt}", flush=True)
    static, _, _ = _static("1", statewise)
    prob, _, saved = kbtest.oracle_forward("1", statewise)
    rng = np.random.default_rng(33)
    S, G, C = prob.S, 1, prob.C
    consts, dc = _wave_consts(prob, saved, rng)
    Pi, Pb, rmax = saved["pi_wave"], saved["pibar_wave"], saved["pibar_row_max"]
    fd_dir = lambda X: np.where(np.isfinite(X), rng.normal(size=X.shape), 0.0)
    dPi, dPb = fd_dir(Pi), fd_dir(Pb)
    pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    dpD, dpS = rng.normal(size=pDp.shape), rng.normal(size=pSp.shape)
    h = static.state_helpers
    metas_t = static.wave_layout["wave_metas"]
    worst = 0.0
    picks = [i for i, m in enumerate(prob.wave_metas) if "sl" in m]
    for i in picks[:: max(1, len(picks) // 5)]:
        mo, mt_ = prob.wave_metas[i], metas_t[i]
        ws, W = int(mo["start"]), int(mo["W"])
        v = rng.normal(size=(W, S))
        ref = O.dts_backward_so(Pi, dPi, Pb, dPb, v, ws, mo, pDp, pSp, dpD, dpS, consts.mt, dc.dMC, consts.col, rmax,
                                prob.item_idx, prob.tree)
        r_rhs = np.zeros((C, S))
        np.add.at(r_rhs, np.asarray(mo["sl"]), ref["d_rhs_l"])
        np.add.at(r_rhs, np.asarray(mo["sr"]), ref["d_rhs_r"])
        d_rhs = torch.zeros((C, S), dtype=dt, device="cuda")
        g_pD, g_pS = torch.zeros(pDp.shape, dtype=dt, device="cuda"), torch.zeros(pSp.shape, dtype=dt, device="cuda")
        g_mt, g_col = torch.zeros((G, S), dtype=dt, device="cuda"), torch.zeros(S, dtype=dt, device="cuda")
        meta = dict(mt_)
        if mo.get("log_split_probs") is not None:
            meta["log_split_probs"] = _t(np.asarray(mo["log_split_probs"]), dt)
        dts_backward_so(_t(Pi, dt), _t(dPi, dt), _t(Pb, dt), _t(dPb, dt), _t(v, dt), ws, meta, S, _t(pDp, dt),
                        _t(pSp, dt), _t(dpD, dt), _t(dpS, dt), _t(consts.mt, dt), _t(dc.dMC, dt),
                        torch.zeros(S, dtype=dt, device="cuda"), h["node_child1"], h["node_child2"],
                        h["node_parent"], int(h["max_ancestor_depth"]), _t(rmax, dt), static.rate_item_idx, d_rhs,
                        g_pD, g_pS, g_mt, g_col)
        torch.cuda.synchronize()
        red = lambda x, shape: x.sum(axis=0).reshape(shape) if shape[-1] != 1 else np.array(x.sum()).reshape(shape)
        pairs = [(d_rhs, r_rhs), (g_pD, red(ref["d_pD"], pDp.shape)), (g_pS, red(ref["d_pS"], pSp.shape)),
                 (g_mt, ref["d_mt"].sum(axis=0).reshape(1, S)), (g_col, ref["d_col"])]
        for g, r in pairs:
            worst = max(worst, _rel(g.cpu().numpy(), r))
    print(f"  worst rel={worst:.3e}")
    assert worst <= TOL[dt]


@pytest.mark.parametrize("name,statewise,row_classes", [("tiny", None, False), ("tiny", True, False),
                                                         ("1", True, False), ("tiny", None, True),
                                                         ("1", True, True), ("1", None, True)])
def test_exact_hvp_matches_oracle(name, statewise, row_classes):
    from kbench.newton.hvp import HvpPlan
    from kbench.percall.solve import plan_of, run_forward

    print(f"[hvp] config={name} statewise={statewise} row_classes={row_classes}", flush=True)
    static, theta, cw = _static(name, statewise)
    _, sv = run_forward(static, theta, cw)
    hvp = HvpPlan(plan_of(static), theta, cw, sv, row_classes=row_classes)
    u = np.random.default_rng(34).normal(size=tuple(theta.shape))
    Hu = hvp(torch.as_tensor(u, dtype=theta.dtype).cuda().reshape(-1))
    torch.cuda.synchronize()
    prob, _, saved = kbtest.oracle_forward(name, statewise)
    _, _, cache = kbtest.oracle_point_cache(name, statewise)
    th = np.asarray(kbtest.problem(name, statewise)["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    ref = O.hvp_exact(prob, th, saved, u, cache)
    e = _rel(Hu.cpu().numpy(), ref.reshape(-1))
    print(f"  |H u| = {np.abs(ref).max():.4e} rel={e:.3e}")
    assert e <= 1e-3


@pytest.mark.parametrize("leaves", [2048, 4096])
def test_exact_hvp_on_a_large_tree_matches_oracle(leaves):
    """S = 4095 and 8191 (three small families): the class / graph HVP against the oracle's HVP (1e-3 of
    max |H u|), through the kernels' 4- and 8-position shapes; at S = 8191 the E-step second-order,
    E tangent and self-loop contractions compute in float32 (three float64 rows of S exceed the LDS)."""
    from kbench.newton.hvp import HvpPlan
    from kbench.percall.solve import plan_of, run_forward

    print(f"[hvp] large tree leaves={leaves} (S={2 * leaves - 1})", flush=True)
    problem, static, theta, cw = _big_tree(leaves, True)
    _, sv = run_forward(static, theta, cw)
    u = np.random.default_rng(43).normal(size=tuple(theta.shape))
    hvp = HvpPlan(plan_of(static), theta, cw, sv, row_classes=True, graph=True)
    Hu = hvp(torch.as_tensor(u, dtype=theta.dtype).cuda().reshape(-1))
    Hu2 = hvp(torch.as_tensor(u, dtype=theta.dtype).cuda().reshape(-1))
    torch.cuda.synchronize()
    assert torch.equal(Hu, Hu2)
    prob = O.Problem.from_dict(problem)
    th = np.asarray(problem["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw64 = np.asarray(problem["inputs"]["col_weights"], dtype=np.float64)
    _, saved = O.forward(prob, th, cw64)
    _, _, cache = O.build_point_cache(prob, th, cw64, saved)
    ref = O.hvp_exact(prob, th, saved, u, cache)
    e = _rel(Hu.cpu().numpy(), ref.reshape(-1))
    print(f"  |H u| = {np.abs(ref).max():.4e} rel={e:.3e}")
    assert e <= 1e-3


def _big_tree(leaves, statewise):
    """A species tree of 2 * leaves - 1 states with three small families (the epilogue's LDS kernel)."""
    from kbench import synth
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    cfg = synth.ProblemConfig(leaves, 3, n_nni=1, family_leaves_median=21.0, family_leaves_sigma=0.6,
                              family_leaves_max=80, statewise=statewise, seed=17)
    p = synth.build_problem(cfg)
    cap = problem_to_captured(p)
    return p, make_static(cap, "cuda"), cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


@pytest.mark.parametrize("name,statewise", [("1", True), ("1", False), ("big", True)])
def test_e_adjoint_entry_solves_the_e_system(name, statewise):
    """kb_e_adjoint (FusedSolver.e_adjoint) against the oracle's E-step VJP at the same float32 E*:
    w - J_E^T w = q with q = acc_E + VJP(acc_Es1, acc_Es2, acc_Ebar) + q_extra, and the parameter
    cotangents of one E step at (w, acc_Ebar) plus acc's rows (float64, 1e-9 relative).  "big": S = 4095,
    the epilogue's LDS kernel (the register-resident one serves trees of up to 2048 nodes)."""
    from kbench.percall.solve import run_forward
    from kbench.runtime import fused_solver

    print(f"[e adjoint] config={name} statewise={statewise}", flush=True)
    if name == "big":
        problem, static, theta, cw = _big_tree(2048, statewise)
    else:
        problem = kbtest.problem(name, statewise)
        static, theta, cw = _static(name, statewise)
    _, sv = run_forward(static, theta, cw)
    S = int(sv["E"].numel())
    g = np.random.default_rng(39)
    acc = g.normal(size=(8, S)) * 1e-2
    qx = g.normal(size=S) * 1e-2
    w, gout = fused_solver(static).e_adjoint(sv, torch.as_tensor(acc).cuda(), q_extra=torch.as_tensor(qx).cuda())
    torch.cuda.synchronize()
    w, gout = w.cpu().numpy()[None], gout.cpu().numpy()
    prob = O.Problem.from_dict(problem)
    row = lambda k: np.broadcast_to(sv[k].detach().double().cpu().numpy().reshape(-1), (S,))[None].copy()
    E, pS, pD, pL, mt = (row(k) for k in ("E", "log_pS", "log_pD", "log_pL", "max_coupling"))
    col = sv["col_log_probs"].double().cpu().numpy().reshape(S)
    vjp = lambda gn, g1, g2, gb: O.e_step_vjp(E, pS, pD, pL, mt, col, prob.tree, False, gn, g1, g2, gb)
    z = np.zeros((1, S))
    q = acc[2][None] + vjp(z, acc[4][None], acc[5][None], acc[3][None])[0] + qx[None]
    res = w - vjp(w, z, z, z)[0] - q
    rn, qn = float(np.linalg.norm(res)), float(np.linalg.norm(q))
    print(f"  |q|={qn:.3e} residual={rn:.3e}")
    assert rn <= 1e-6 * max(qn, 1.0)  # BiCGSTAB stops at 1e-7 * max(|q|_2, 1) (its own residual)
    _, q0, q1, q3, wbar, gcol = vjp(w, z, z, acc[3][None])
    want = [q0[0] + acc[1], q1[0] + acc[0], q3[0], wbar[0] + acc[6], gcol + acc[7]]
    for i, ref in enumerate(want):
        e = np.abs(gout[i] - ref).max() / max(np.abs(ref).max(), 1e-300)
        print(f"  cotangent {i}: rel={e:.3e}")
        assert e <= 1e-9


def test_e_adjoint_entry_reports_a_failed_solve(monkeypatch):
    """kb_e_adjoint with one BiCGSTAB iteration and an unreachable tolerance: the status words say
    failed, FusedSolver.e_adjoint raises RuntimeError (as the backward does), and check_solve=False
    leaves the status for the caller."""
    from kbench.percall.solve import run_forward
    from kbench.fused import FusedSolver

    static, theta, cw = _static("1", True)
    _, sv = run_forward(static, theta, cw)
    so = dict(static.solver_options.__dict__, bicgstab_max_iter=1, bicgstab_tol=1e-30)
    solver = FusedSolver(static, so)
    S = int(sv["E"].numel())
    acc = torch.as_tensor(np.random.default_rng(42).normal(size=(8, S))).cuda()
    with pytest.raises(RuntimeError, match="BiCGSTAB"):
        solver.e_adjoint(sv, acc)
    solver.e_adjoint(sv, acc, check_solve=False)
    it, failed = (int(x) for x in solver.last_e_status.cpu())
    assert failed == 1 and it == 1


def test_native_tangent_e_adjoint_matches_autograd_bicgstab():
    """The HVP's tangent E side through kb_e_adjoint agrees with BiCGSTAB over autograd E-step products."""
    from kbench.newton.hvp import HvpPlan
    from kbench.percall.solve import plan_of, run_forward

    static, theta, cw = _static("1", True)
    _, sv = run_forward(static, theta, cw)
    plan = plan_of(static)
    u = torch.as_tensor(np.random.default_rng(40).normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda()
    a = HvpPlan(plan, theta, cw, sv, native_e_adjoint=True)(u.reshape(-1))
    b = HvpPlan(plan, theta, cw, sv, native_e_adjoint=False)(u.reshape(-1))
    torch.cuda.synchronize()
    e = kbtest.norm_rel_t(a, b)
    print(f"  native vs autograd E side: rel={e:.3e}")
    assert e <= 1e-4


def test_ggn_hvp_is_symmetric_and_psd():
    from kbench.newton.hvp import ggn_hvp
    from kbench.percall.solve import plan_of, run_forward

    static, theta, cw = _static("1", True)
    _, sv = run_forward(static, theta, cw)
    hvp = ggn_hvp(plan_of(static), theta, cw, sv)
    g = np.random.default_rng(36)
    u1 = torch.as_tensor(g.normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda().reshape(-1)
    u2 = torch.as_tensor(g.normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda().reshape(-1)
    M1, M2 = hvp(u1), hvp(u2)
    torch.cuda.synchronize()
    a, b = float((u2.double() * M1.double()).sum()), float((u1.double() * M2.double()).sum())
    q1 = float((u1.double() * M1.double()).sum())
    print(f"  u2.M u1={a:.6e} u1.M u2={b:.6e} u1.M u1={q1:.6e}")
    assert abs(a - b) <= 1e-3 * max(abs(a), abs(b), 1e-30)
    assert q1 >= -1e-6 * abs(q1)
