"""Pins of the oracle's forward tangents (JVP) by independent checks.

Every tangent function is compared with central finite differences of the
oracle's own primal map (a different code path: the tangents are written
term by term, the primal maps as log-sum-exps), and the composed JVP of the
loss with the oracle's reverse-mode gradient (grad_theta . v), which shares
no code with the tangents.  A dropped term, a swapped child or a missing
ancestor in a tangent fails one of these.
"""

import dataclasses

import numpy as np
import pytest

import kbench_oracle as O
import kbtest


def _tiny(statewise=None):
    p = kbtest.problem("tiny", statewise)
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    return p, prob, theta


def _fd_close(got, fd, rel=1e-6):
    fin = np.isfinite(fd)
    assert fin.any()
    scale = max(1.0, float(np.abs(fd[fin]).max()))
    err = float(np.abs(got[fin] - fd[fin]).max())
    assert err <= rel * scale, (err, scale)


@pytest.mark.parametrize("use_col", [False, True])
def test_e_step_tangent_matches_finite_differences(use_col):
    _, prob, theta = _tiny()
    rng = np.random.default_rng(3)
    S, tree = prob.S, prob.tree
    E = np.log2(rng.uniform(0.05, 0.6, (2, S)))
    pS, pD, pL, mt = (rng.uniform(-4, -0.5, (2, S)) for _ in range(4))
    col = rng.uniform(-1, 1, S)
    dE, dpS, dpD, dpL, dmt = (rng.normal(size=(2, S)) for _ in range(5))
    got = O.e_step_tangent(E, dE, pS, pD, pL, mt, col, dpS, dpD, dpL, dmt, tree, use_col)
    h = 1e-6

    def F(s):
        return O.e_step(E + s * dE, pS + s * dpS, pD + s * dpD, pL + s * dpL, mt + s * dmt, col, tree, use_col)

    fp, fm = F(h), F(-h)
    # e_step returns (E_new, E_s1, E_s2, Ebar); the tangent (dE_new, dE_s1, dE_s2, dEbar)
    for g, a, b in zip(got, fp, fm):
        _fd_close(g, (a - b) / (2 * h))


@pytest.mark.parametrize("statewise", [False, True])
def test_e_tangent_fixed_point_matches_fd_of_the_fixed_point(statewise):
    """dE* along v: tangent fixed point + analytic parameter JVP vs FD of the converged E solve."""
    _, prob, theta = _tiny(statewise)
    rng = np.random.default_rng(4)
    v = rng.normal(size=theta.shape)
    S, tree = prob.S, prob.tree
    G = 1

    def solve(th):
        pS, pD, pL, mt = O.extract_parameters_uniform(th, prob.unnorm_row_max, prob.statewise, prob.itemwise)
        st = [np.broadcast_to(O.as_item_state(np.asarray(x), S, G), (G, S)).copy() for x in (pS, pD, pL, mt)]
        E0 = np.full((G, S), -60.0)
        E, Es1, Es2, Eb, _ = O.e_fixed_point(E0, *st, np.zeros(S), tree, False, max_iter=5000, tol=1e-15)
        return st, (E, Es1, Es2, Eb)

    st, prim = solve(theta)
    d = O.param_jvp_uniform(theta, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
    dst = [np.broadcast_to(O.as_item_state(np.asarray(x), S, G), (G, S)).copy() for x in d]
    got = O.e_tangent_fixed_point(prim[0], *dst, *st, np.zeros(S), tree, max_iter=5000, tol=1e-15,
                                  use_col_weights=False)
    h = 1e-6
    _, pp = solve(theta + h * v)
    _, pm = solve(theta - h * v)
    for g, a, b in zip(got, pp, pm):
        _fd_close(g, (a - b) / (2 * h), rel=1e-6)


def test_param_jvp_matches_finite_differences():
    for statewise in (False, True):
        _, prob, theta = _tiny(statewise)
        v = np.random.default_rng(5).normal(size=theta.shape)
        got = O.param_jvp_uniform(theta, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
        h = 1e-6
        a = O.extract_parameters_uniform(theta + h * v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
        b = O.extract_parameters_uniform(theta - h * v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
        for g, x, y in zip(got, a, b):
            _fd_close(np.broadcast_to(g, np.shape(x)), (np.asarray(x) - np.asarray(y)) / (2 * h), rel=1e-8)


def _saved(prob, theta):
    prob.so.update(pi_iters=120, e_tol=1e-14)
    loss, saved = O.forward(prob, theta, np.zeros(prob.S))
    return loss, saved


def test_dts_tangent_matches_finite_differences():
    _, prob, theta = _tiny(True)
    _, saved = _saved(prob, theta)
    rng = np.random.default_rng(6)
    S, C, tree = prob.S, prob.C, prob.tree
    Pi, Pb = saved["pi_wave"], saved["pibar_wave"]
    dPi = np.where(np.isfinite(Pi), rng.normal(size=Pi.shape), 0.0)
    dPb = np.where(np.isfinite(Pb), rng.normal(size=Pb.shape), 0.0)
    G = 1
    pD = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pS = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    dpD, dpS = rng.normal(size=pD.shape), rng.normal(size=pS.shape)
    metas = [m for m in prob.wave_metas if "sl" in m]
    assert metas
    h = 1e-6
    checked = 0
    for meta in metas[:6]:
        ws, W = int(meta["start"]), int(meta["W"])
        dts = O.dts_forward(Pi, Pb, meta, W, pD, pS, prob.item_idx, ws, tree)
        got = O.dts_tangent(Pi, Pb, dPi, dPb, meta, W, pD, pS, dpD, dpS, dts, prob.item_idx, ws, tree)
        a = O.dts_forward(Pi + h * dPi, Pb + h * dPb, meta, W, pD + h * dpD, pS + h * dpS, prob.item_idx, ws, tree)
        b = O.dts_forward(Pi - h * dPi, Pb - h * dPb, meta, W, pD - h * dpD, pS - h * dpS, prob.item_idx, ws, tree)
        fd = (a - b) / (2 * h)
        assert (got[np.isneginf(dts)] == 0).all()
        _fd_close(got, fd)
        checked += 1
    assert checked > 0


@pytest.mark.parametrize("kind", ["leaf", "split"])
def test_wave_step_tangent_one_sweep_matches_finite_differences(kind):
    _, prob, theta = _tiny()
    _, saved = _saved(prob, theta)
    rng = np.random.default_rng(7)
    S, tree = prob.S, prob.tree
    G = 1
    E = np.asarray(saved["E"])
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    pS, pD, mt = st(saved["log_pS"]), st(saved["log_pD"]), st(saved["max_coupling"])
    consts = O.WaveConsts(mt=mt, DL=1.0 + pD + E, Ebar=np.asarray(saved["Ebar"]), E=E,
                          SL1=pS + saved["E_s2"], SL2=pS + saved["E_s1"], leaf_logp=pS, col=np.zeros(S),
                          use_col_weights=False)
    dc = O.WaveTangentConsts(*(rng.normal(size=(G, S)) for _ in range(7)))
    meta = next(m for m in prob.wave_metas if ("sl" in m) == (kind == "split"))
    ws, W = int(meta["start"]), int(meta["W"])
    rows = np.arange(ws, ws + W)
    items = prob.item_idx[rows]
    Pi = saved["pi_wave"][rows]
    dPi = np.where(np.isfinite(Pi), rng.normal(size=Pi.shape), 0.0)
    leaf = prob.leaf_state[rows] if kind == "leaf" else None
    dts = d_dts = None
    if kind == "split":
        pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
        pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
        dts = O.dts_forward(saved["pi_wave"], saved["pibar_wave"], meta, W, pDp, pSp, prob.item_idx, ws, tree)
        d_dts = np.where(np.isfinite(dts), rng.normal(size=dts.shape), 0.0)
    got, dpibar = O.wave_step_tangent(Pi, dPi, items, consts, dc, tree, leaf_state=leaf, dts_r=dts, d_dts=d_dts,
                                      n_iters=1)
    h = 1e-6

    def F(s):
        c = dataclasses.replace(consts, mt=mt + s * dc.dMC, DL=consts.DL + s * dc.dDL,
                                Ebar=consts.Ebar + s * dc.dEbar, E=E + s * dc.dE, SL1=consts.SL1 + s * dc.dSL1,
                                SL2=consts.SL2 + s * dc.dSL2, leaf_logp=pS + s * dc.dleaf)
        new = O.wave_sweep(Pi + s * dPi, items, c, tree, leaf_state=leaf,
                           dts_r=None if dts is None else dts + s * d_dts)
        pb, _ = O._pibar_from_pi(Pi + s * dPi, c.col, c.mt[items], tree, False)
        return new, pb

    (a, pa), (b, pb) = F(h), F(-h)
    _fd_close(got, (a - b) / (2 * h))
    _fd_close(dpibar, (pa - pb) / (2 * h))


@pytest.mark.parametrize("statewise", [False, True])
def test_jvp_root_scores_matches_finite_differences(statewise):
    """The composed tangent of every Pi / Pibar row vs FD of the converged forward solve."""
    _, prob, theta = _tiny(statewise)
    _, saved = _saved(prob, theta)
    v = np.random.default_rng(8).normal(size=theta.shape)
    roots, dPi, dPb = O.jvp_root_scores(prob, theta, v, saved, self_iters=120, e_tol=1e-14)
    h = 1e-5
    _, sp = O.forward(prob, theta + h * v, np.zeros(prob.S))
    _, sm = O.forward(prob, theta - h * v, np.zeros(prob.S))
    _fd_close(dPi, (sp["pi_wave"] - sm["pi_wave"]) / (2 * h), rel=1e-7)
    _fd_close(dPb, (sp["pibar_wave"] - sm["pibar_wave"]) / (2 * h), rel=1e-7)
    np.testing.assert_array_equal(roots, dPi[prob.root_ids])


def test_jvp_of_the_loss_equals_the_gradient_along_v():
    """Forward-mode and reverse-mode agree: d loss . v from the JVP == grad_theta . v from the adjoint."""
    _, prob, theta = _tiny(True)
    prob.so.update(pi_iters=120, neumann_terms=200, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                   bicgstab_tol=1e-13, e_tol=1e-14)
    cw = np.zeros(prob.S)
    loss, saved = O.forward(prob, theta, cw)
    gt, _, _ = O.backward(prob, theta, cw, saved)
    v = np.random.default_rng(9).normal(size=theta.shape)
    roots, _, _ = O.jvp_root_scores(prob, theta, v, saved, self_iters=120, e_tol=1e-14)
    S, G = prob.S, 1
    d = O.param_jvp_uniform(theta, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    dE = O.e_tangent_fixed_point(np.asarray(saved["E"]), *(st(x) for x in d),
                                 *(st(saved[k]) for k in ("log_pS", "log_pD", "log_pL", "max_coupling")),
                                 np.zeros(S), prob.tree, max_iter=5000, tol=1e-15, use_col_weights=False)[0]
    R, E = saved["root_rows"], saved["E"]
    # the loss is a closed-form function of (root rows, E): differentiate it along (dR, dE) numerically
    h = 1e-6
    dl = (O.nll_from_root_rows(R + h * roots, E + h * dE) - O.nll_from_root_rows(R - h * roots, E - h * dE)) / (2 * h)
    ref = float(np.dot(gt.reshape(-1), v.reshape(-1)))
    assert abs(dl - ref) <= 1e-7 * max(1.0, abs(ref)), (dl, ref)
