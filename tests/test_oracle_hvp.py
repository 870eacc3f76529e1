"""Pins of the oracle's second-order contractions and exact HVP by independent checks.

* each contraction (E-step, self-loop J^T and buckets, split-term backward)
  against central finite differences of the oracle's first-order VJP at a
  fixed cotangent (the contractions are written term by term, the VJPs are
  the backward's own code);
* the head term against finite differences of the parameter VJP;
* the exact HVP against finite differences of the converged gradient, and
  its symmetry u1.H u2 = u2.H u1.
"""

import dataclasses

import numpy as np
import pytest

import kbench_oracle as O
import kbtest


def _fd_close(got, fd, rel=1e-6):
    got = np.asarray(got, dtype=np.float64)
    fd = np.asarray(fd, dtype=np.float64)
    fin = np.isfinite(fd)
    assert fin.any()
    scale = max(1.0, float(np.abs(fd[fin]).max()))
    err = float(np.abs(got[fin] - fd[fin]).max())
    assert err <= rel * scale, (err, scale)


def _converged(statewise=None):
    p = kbtest.problem("tiny", statewise)
    prob = O.Problem.from_dict(p)
    prob.so.update(pi_iters=120, neumann_terms=200, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                   bicgstab_tol=1e-13, e_tol=1e-14)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    loss, saved = O.forward(prob, theta, np.zeros(prob.S))
    return prob, theta, saved


@pytest.mark.parametrize("use_col", [False, True])
def test_e_step_backward_so_matches_fd_of_the_vjp(use_col):
    prob, _, _ = _converged()
    rng = np.random.default_rng(21)
    S, tree, G = prob.S, prob.tree, 2
    E = np.log2(rng.uniform(0.05, 0.6, (G, S)))
    pS, pD, pL, mt = (rng.uniform(-4, -0.5, (G, S)) for _ in range(4))
    col = rng.uniform(-1, 1, S)
    g_new, g_s1, g_s2, g_eb = (rng.normal(size=(G, S)) for _ in range(4))
    dE, dpS, dpD, dpL, dmt = (rng.normal(size=(G, S)) for _ in range(5))
    dcol = rng.normal(size=S)
    En, Es1, Es2, Eb = O.e_step(E, pS, pD, pL, mt, col, tree, use_col)
    # tangents of the saved E-step outputs along the same direction (col enters through use_col)
    h = 1e-6
    fp = O.e_step(E + h * dE, pS + h * dpS, pD + h * dpD, pL + h * dpL, mt + h * dmt, col + h * dcol, tree, use_col)
    fm = O.e_step(E - h * dE, pS - h * dpS, pD - h * dpD, pL - h * dpL, mt - h * dmt, col - h * dcol, tree, use_col)
    dEn, dEs1, dEs2, dEb = (np.where(np.isfinite(a) & np.isfinite(b), (a - b) / (2 * h), 0.0) for a, b in zip(fp, fm))
    got = O.e_step_backward_so(E, En, Es1, Es2, Eb, pS, pD, pL, col, tree, g_new, g_eb, dE, dEn, dEs1, dEs2, dEb,
                               dpS, dpD, dpL, dcol, use_col)

    def V(s):
        return O.e_step_vjp(E + s * dE, pS + s * dpS, pD + s * dpD, pL + s * dpL, mt + s * dmt, col + s * dcol, tree,
                            use_col, g_new, g_s1, g_s2, g_eb)

    a, b = V(h), V(-h)
    # e_step_vjp: (grad_E, grad_pS, grad_pD, grad_pL, grad_mt, grad_col); so: same order
    for k in range(6):
        _fd_close(got[k], (a[k] - b[k]) / (2 * h), rel=2e-6)


def _wave_setup(kind, rng):
    prob, theta, saved = _converged()
    S, G, tree = prob.S, 1, prob.tree
    E = np.asarray(saved["E"])
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    pS, pD, mt = st(saved["log_pS"]), st(saved["log_pD"]), st(saved["max_coupling"])
    consts = O.WaveConsts(mt=mt, DL=1.0 + pD + E, Ebar=np.asarray(saved["Ebar"]), E=E, SL1=pS + saved["E_s2"],
                          SL2=pS + saved["E_s1"], leaf_logp=pS, col=np.zeros(S), use_col_weights=False)
    meta = next(m for m in prob.wave_metas if ("sl" in m) == (kind == "split"))
    return prob, saved, consts, meta, tree


@pytest.mark.parametrize("kind", ["leaf", "split"])
def test_wave_backward_so_matches_fd_of_the_transposed_sweep(kind):
    rng = np.random.default_rng(22)
    prob, saved, consts, meta, tree = _wave_setup(kind, rng)
    S, G = prob.S, 1
    ws, W = int(meta["start"]), int(meta["W"])
    rows = np.arange(ws, ws + W)
    items = prob.item_idx[rows]
    Pi, Pb, rmax = saved["pi_wave"][rows], saved["pibar_wave"][rows], saved["pibar_row_max"][rows]
    v = rng.normal(size=(W, S))
    fd_dir = lambda X: np.where(np.isfinite(X), rng.normal(size=X.shape), 0.0)
    dPi, dPb = fd_dir(Pi), fd_dir(Pb)
    dc = O.WaveTangentConsts(*(0.5 * rng.normal(size=(G, S)) for _ in range(7)))
    leaf = prob.leaf_state[rows] if kind == "leaf" else None
    dts = d_dts = None
    if kind == "split":
        pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
        pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
        dts = O.dts_forward(saved["pi_wave"], saved["pibar_wave"], meta, W, pDp, pSp, prob.item_idx, ws, tree)
        d_dts = fd_dir(dts)
    got = O.wave_backward_so(Pi, dPi, Pb, dPb, v, rmax, items, consts, dc, tree, leaf_state=leaf, dts_r=dts,
                             d_dts=d_dts)

    def F(s):
        c = dataclasses.replace(consts, DL=consts.DL + s * dc.dDL, Ebar=consts.Ebar + s * dc.dEbar,
                                E=consts.E + s * dc.dE, SL1=consts.SL1 + s * dc.dSL1, SL2=consts.SL2 + s * dc.dSL2,
                                leaf_logp=consts.leaf_logp + s * dc.dleaf)
        co = O.self_loop_coeffs(Pi + s * dPi, Pb + s * dPb, rmax, items, c, tree, leaf_state=leaf,
                                dts_r=None if dts is None else dts + s * d_dts)
        alpha = v * co.w_L
        aw = [alpha * ek * co.inv_sum for ek in co.e]
        return [O.apply_JT(v, co, tree), aw[0], aw[1], aw[2], aw[3] + aw[4] + aw[5], aw[3], aw[4]]

    h = 1e-6
    a, b = F(h), F(-h)
    for k in range(7):
        _fd_close(got[k], (a[k] - b[k]) / (2 * h), rel=2e-6)


def test_dts_backward_so_matches_fd_of_the_split_backward():
    rng = np.random.default_rng(23)
    prob, saved, consts, meta, tree = _wave_setup("split", rng)
    S, G = prob.S, 1
    ws, W = int(meta["start"]), int(meta["W"])
    Pi, Pb, rmax = saved["pi_wave"], saved["pibar_wave"], saved["pibar_row_max"]
    fd_dir = lambda X: np.where(np.isfinite(X), rng.normal(size=X.shape), 0.0)
    dPi, dPb = fd_dir(Pi), fd_dir(Pb)
    pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    dpD, dpS = rng.normal(size=pDp.shape), rng.normal(size=pSp.shape)
    mt, dmt = consts.mt, rng.normal(size=consts.mt.shape)
    v = rng.normal(size=(W, S))
    act = np.ones(W, dtype=bool)
    got = O.dts_backward_so(Pi, dPi, Pb, dPb, v, ws, meta, pDp, pSp, dpD, dpS, mt, dmt, consts.col, rmax,
                            prob.item_idx, tree)

    def F(s):
        return O.dts_cross_backward(Pi + s * dPi, Pb + s * dPb, rmax, v, ws, meta, pDp + s * dpD, pSp + s * dpS,
                                    mt + s * dmt, prob.item_idx, tree, act, consts.col, False)

    h = 1e-6
    a, b = F(h), F(-h)
    fd = {k: (a[k] - b[k]) / (2 * h) for k in ("rhs_l", "rhs_r", "g_pD", "g_pS", "col_grad")}
    _fd_close(got["d_rhs_l"], fd["rhs_l"])
    _fd_close(got["d_rhs_r"], fd["rhs_r"])
    _fd_close(got["d_pD"], fd["g_pD"])
    _fd_close(got["d_pS"], fd["g_pS"])
    _fd_close(got["d_mt"], (a["g_mt_l"] + a["g_mt_r"] - b["g_mt_l"] - b["g_mt_r"]) / (2 * h))
    _fd_close(got["d_col"], fd["col_grad"])


@pytest.mark.parametrize("statewise", [False, True])
def test_theta_head_hvp_matches_fd_of_the_parameter_vjp(statewise):
    prob, theta, saved = _converged(statewise)
    rng = np.random.default_rng(24)
    S = prob.S
    G_pS, G_pD, G_pL = (rng.normal(size=np.shape(saved[k])) for k in ("log_pS", "log_pD", "log_pL"))
    G_mt = rng.normal(size=np.shape(saved["max_coupling"]))
    G_col = rng.normal(size=S)
    u = rng.normal(size=theta.shape)
    got = O.theta_head_hvp(prob, theta, u, G_pS, G_pD, G_pL, G_mt)
    h = 1e-6
    cw = np.zeros(S)
    a = O.theta_col_vjp(prob, theta + h * u, cw, False, G_pS, G_pD, G_pL, G_mt, G_col)[0]
    b = O.theta_col_vjp(prob, theta - h * u, cw, False, G_pS, G_pD, G_pL, G_mt, G_col)[0]
    _fd_close(got, (a - b) / (2 * h), rel=1e-8)


@pytest.mark.parametrize("statewise", [False, True])
def test_exact_hvp_matches_fd_of_the_gradient_and_is_symmetric(statewise):
    prob, theta, saved = _converged(statewise)
    cw = np.zeros(prob.S)
    _, _, cache = O.build_point_cache(prob, theta, cw, saved)
    rng = np.random.default_rng(25)
    u1, u2 = rng.normal(size=theta.shape), rng.normal(size=theta.shape)
    H1 = O.hvp_exact(prob, theta, saved, u1, cache, tangent_self_iters=120, e_tol=1e-14)
    H2 = O.hvp_exact(prob, theta, saved, u2, cache, tangent_self_iters=120, e_tol=1e-14)

    def grad(th):
        _, sv = O.forward(prob, th, cw)
        return O.backward(prob, th, cw, sv)[0]

    h = 1e-5
    fd = (grad(theta + h * u1) - grad(theta - h * u1)) / (2 * h)
    _fd_close(H1, fd, rel=1e-7)
    a, b = float(np.sum(u2 * H1)), float(np.sum(u1 * H2))
    assert abs(a - b) <= 1e-9 * max(1.0, abs(a)), (a, b)
