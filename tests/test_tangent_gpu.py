"""GPU parity of the forward-tangent wrappers (kbench.core.kernels.{e_step,dts,wave}_tangent) and of the
forward-tangent call sequence (kbench/newton/hvp.py ``TangentForward``) against the float64 CPU oracle.

Kernel tests feed the oracle's own primal point (Pi*, E*, ...) to the HIP
wrappers, in float64 (tight tolerance: same arithmetic up to summation order)
and in float32 (rel 1e-4 normwise).  The composed JVP runs the glue on the
GPU's own fp32 forward and is compared with the oracle's JVP at the oracle's
forward (rel 1e-4), and at config 3 by size-independent properties:
linearity in v and bitwise determinism.
"""

import functools

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu


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
    assert got.shape == ref.shape
    assert np.isfinite(got).all()
    return float(np.abs(got - ref).max()) / max(1.0, float(np.abs(ref).max()))


TOL = {torch.float64: 1e-9, torch.float32: 1e-4}


@pytest.mark.parametrize("name,dt,statewise", [("1", torch.float64, False), ("1", torch.float32, False),
                                               ("1", torch.float64, True), ("1", torch.float32, True),
                                               ("big", torch.float32, True)])
def test_e_tangent_fixed_point_matches_oracle(name, dt, statewise):
    """Config 1, and S = 8191 ("big") in float32, where the rows are too long for three float64 LDS rows
    and the kernel computes in float32."""
    from kbench.core.kernels.e_step_tangent import e_tangent_fixed_point

    print(f"[e-tangent] config={name} statewise={statewise} dtype={dt}", flush=True)
    static, prob, saved = _wave_fixture(name, statewise, dt)
    S, G = prob.S, 1
    th = _theta(name, statewise, prob)
    v = np.random.default_rng(11).normal(size=th.shape)
    d = O.param_jvp_uniform(th, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    prim = [st(saved[k]) for k in ("log_pS", "log_pD", "log_pL", "max_coupling")]
    ref = O.e_tangent_fixed_point(np.asarray(saved["E"]), *(st(x) for x in d), *prim, np.zeros(S), prob.tree,
                                  max_iter=2000, tol=1e-13, use_col_weights=False)
    h = static.state_helpers
    got = e_tangent_fixed_point(_t(saved["E"], dt), *(_t(st(x), dt) for x in d), *(_t(x, dt) for x in prim),
                                torch.zeros(S, dtype=dt, device="cuda"), h["node_parent"], h["node_child1"],
                                h["node_child2"], int(h["max_ancestor_depth"]), max_iter=2000,
                                tol=1e-13 if dt == torch.float64 else 1e-7, use_col_weights=False)
    torch.cuda.synchronize()
    for name, g, r in zip(("dE", "dE_s1", "dE_s2", "dEbar"), got, ref):
        e = _rel(g.cpu().numpy(), r)
        print(f"  {name}: rel={e:.3e}")
        assert e <= TOL[dt]


def test_e_tangent_float32_long_rows_stop_on_their_rounding_floor():
    """At S = 8191 in float32 the kernel iterates in float32; with the default tol (1e-9, far below
    float32 rounding) it stops on the 9.5e-7 floor well before max_iter, as accurate as at tol 1e-7."""
    from kbench.core.kernels.e_step_tangent import e_tangent_fixed_point

    print("[e-tangent] big float32, default tol: step count", flush=True)
    dt = torch.float32
    static, prob, saved = _wave_fixture("big", True, dt)
    S, G = prob.S, 1
    th = _theta("big", True, prob)
    v = np.random.default_rng(11).normal(size=th.shape)
    d = O.param_jvp_uniform(th, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    prim = [st(saved[k]) for k in ("log_pS", "log_pD", "log_pL", "max_coupling")]
    ref = O.e_tangent_fixed_point(np.asarray(saved["E"]), *(st(x) for x in d), *prim, np.zeros(S), prob.tree,
                                  max_iter=2000, tol=1e-13, use_col_weights=False)
    h = static.state_helpers
    n_iter = torch.zeros(G, dtype=torch.int32, device="cuda")
    got = e_tangent_fixed_point(_t(saved["E"], dt), *(_t(st(x), dt) for x in d), *(_t(x, dt) for x in prim),
                                torch.zeros(S, dtype=dt, device="cuda"), h["node_parent"], h["node_child1"],
                                h["node_child2"], int(h["max_ancestor_depth"]), n_iter_out=n_iter,
                                use_col_weights=False)
    torch.cuda.synchronize()
    steps = int(n_iter[0])
    print(f"  steps={steps} of max_iter=2000")
    assert 1 <= steps < 200
    for name, g, r in zip(("dE", "dE_s1", "dE_s2", "dEbar"), got, ref):
        e = _rel(g.cpu().numpy(), r)
        print(f"  {name}: rel={e:.3e}")
        assert e <= TOL[dt]


def _theta(name, statewise, prob):
    """The fixture's theta as float64 (rounded through float32, as the GPU side holds it)."""
    p = _big_problem(bool(statewise)) if name == "big" else kbtest.problem(name, statewise)
    return np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)


@functools.lru_cache(maxsize=2)
def _big_problem(statewise):
    """A 4096-leaf species tree (S = 8191) with three small families."""
    from kbench import synth

    cfg = synth.ProblemConfig(4096, 3, n_nni=1, family_leaves_median=21.0, family_leaves_sigma=0.6,
                              family_leaves_max=80, statewise=statewise, seed=17)
    return synth.build_problem(cfg)


def _wave_fixture(name, statewise, dt):
    """(static on the GPU, oracle problem, oracle forward intermediates) of one configuration.

    ``name`` "big": a 4096-leaf species tree (S = 8191) with three small families.
    """
    if name == "big":
        from kbench.fused import problem_to_captured
        from kbench.runtime import make_static

        p = _big_problem(bool(statewise))
        static = make_static(problem_to_captured(p), "cuda")
        prob = O.Problem.from_dict(p)
        theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
        _, saved = O.forward(prob, theta, np.asarray(p["inputs"]["col_weights"], dtype=np.float64))
        return static, prob, saved
    static, _, _ = _static(name, statewise)
    prob, _, saved = kbtest.oracle_forward(name, statewise)
    return static, prob, saved


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_dts_tangent_matches_oracle(dt):
    from kbench.core.kernels.dts_tangent import compute_dts_tangent

    print(f"[dts-tangent] config=1 statewise=True dtype={dt}", flush=True)
    static, prob, saved = _wave_fixture("1", True, dt)
    rng = np.random.default_rng(12)
    S, G = prob.S, 1
    Pi, Pb = saved["pi_wave"], saved["pibar_wave"]
    dPi = np.where(np.isfinite(Pi), rng.normal(size=Pi.shape), 0.0)
    dPb = np.where(np.isfinite(Pb), rng.normal(size=Pb.shape), 0.0)
    pD = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pS = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    dpD, dpS = rng.normal(size=pD.shape), rng.normal(size=pS.shape)
    h = static.state_helpers
    metas_t = [m for m in static.wave_layout["wave_metas"] if "sl" in m]
    metas_o = [m for m in prob.wave_metas if "sl" in m]
    worst = 0.0
    for mt_, mo in list(zip(metas_t, metas_o))[:: max(1, len(metas_o) // 8)]:
        ws, W = int(mo["start"]), int(mo["W"])
        dts = O.dts_forward(Pi, Pb, mo, W, pD, pS, prob.item_idx, ws, prob.tree)
        lsp = None if mo.get("log_split_probs") is None else _t(np.asarray(mo["log_split_probs"]), dt)
        ref = O.dts_tangent(Pi, Pb, dPi, dPb, mo, W, pD, pS, dpD, dpS, dts, prob.item_idx, ws, prob.tree)
        got = compute_dts_tangent(_t(Pi, dt), _t(Pb, dt), _t(dPi, dt), _t(dPb, dt), mt_["sl"], mt_["sr"],
                                  h["node_child1"], h["node_child2"], W, mt_["reduce_idx"], _t(pD, dt), _t(pS, dt),
                                  _t(dpD, dt), _t(dpS, dt), _t(dts, dt), static.rate_item_idx,
                                  log_split_probs=lsp, item_offset=ws)
        torch.cuda.synchronize()
        g = got.cpu().numpy()
        assert (g[np.isneginf(dts)] == 0).all()
        worst = max(worst, _rel(g, ref))
    print(f"  worst rel={worst:.3e}")
    assert worst <= TOL[dt]


@pytest.mark.parametrize("name,dt,n_iters", [("1", torch.float64, 1), ("1", torch.float64, 7),
                                             ("1", torch.float32, 1), ("1", torch.float32, 7),
                                             ("big", torch.float32, 7)])
def test_wave_step_tangent_matches_oracle(name, dt, n_iters):
    """Tangent sweeps against the oracle; "big" (S = 8191) runs the float32 preorder kernel at eight
    positions per thread."""
    from kbench.core.kernels.wave_tangent import compute_wave_step_tangent, compute_wave_step_tangent_selfloop

    print(f"[wave-tangent] config={name} dtype={dt} n_iters={n_iters}", flush=True)
    static, prob, saved = _wave_fixture(name, None, dt)
    rng = np.random.default_rng(13)
    S, G, C = prob.S, 1, prob.C
    E = np.asarray(saved["E"])
    st = lambda x: np.broadcast_to(O.as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    pS, pD, mt = st(saved["log_pS"]), st(saved["log_pD"]), st(saved["max_coupling"])
    consts = O.WaveConsts(mt=mt, DL=1.0 + pD + E, Ebar=np.asarray(saved["Ebar"]), E=E, SL1=pS + saved["E_s2"],
                          SL2=pS + saved["E_s1"], leaf_logp=pS, col=np.zeros(S), use_col_weights=False)
    dc = O.WaveTangentConsts(*(0.3 * rng.normal(size=(G, S)) for _ in range(7)))
    Pi = saved["pi_wave"]
    dPi = np.where(np.isfinite(Pi), rng.normal(size=Pi.shape), 0.0)
    h = static.state_helpers
    metas_t = static.wave_layout["wave_metas"]
    Pd, dPd = _t(Pi, dt), _t(dPi, dt)
    cargs = [_t(x, dt) for x in (mt, dc.dMC, consts.DL, dc.dDL, consts.Ebar, dc.dEbar, E, dc.dE, consts.SL1,
                                  dc.dSL1, consts.SL2, dc.dSL2)]
    common = dict(leaf_state_idx=static.wave_layout["leaf_state_index"], leaf_logp=_t(pS, dt),
                  dleaf_logp=_t(dc.dleaf, dt), item_idx=static.rate_item_idx, use_col_weights=False)
    pDp = O.as_item_param(np.asarray(saved["log_pD"]), G, S)
    pSp = O.as_item_param(np.asarray(saved["log_pS"]), G, S)
    worst = worst_b = 0.0
    picks = [0, 1, len(prob.wave_metas) // 2, len(prob.wave_metas) - 1]
    for i in picks:
        mo, mt_ = prob.wave_metas[i], metas_t[i]
        ws, W = int(mo["start"]), int(mo["W"])
        rows = np.arange(ws, ws + W)
        split = "sl" in mo
        leaf = None if split else prob.leaf_state[rows]
        dts = d_dts = None
        if split:
            dts = O.dts_forward(Pi, saved["pibar_wave"], mo, W, pDp, pSp, prob.item_idx, ws, prob.tree)
            d_dts = np.where(np.isfinite(dts), rng.normal(size=dts.shape), 0.0)
        ref, ref_b = O.wave_step_tangent(Pi[rows], dPi[rows], prob.item_idx[rows], consts, dc, prob.tree,
                                         leaf_state=leaf, dts_r=dts, d_dts=d_dts, n_iters=n_iters)
        dts_t = None if dts is None else _t(dts, dt)
        ddts_t = None if d_dts is None else _t(d_dts, dt)
        dpb = torch.zeros((C, S), dtype=dt, device="cuda")
        if n_iters == 1:
            out = torch.zeros((C, S), dtype=dt, device="cuda")
            compute_wave_step_tangent(Pd, dPd, out, ws, W, S, *cargs, None, h["node_child1"], h["node_child2"],
                                      h["node_parent"], int(h["max_ancestor_depth"]), dts_t, ddts_t, dPibar_out=dpb,
                                      has_leaf_term=not split, **common)
        else:
            out = dPd.clone()
            compute_wave_step_tangent_selfloop(Pd, out, ws, W, S, n_iters, *cargs, None, h["node_child1"],
                                               h["node_child2"], h["node_parent"], int(h["max_ancestor_depth"]),
                                               dts_t, ddts_t, dPibar_out=dpb, has_leaf_term=not split, **common)
        torch.cuda.synchronize()
        worst = max(worst, _rel(out[ws:ws + W].cpu().numpy(), ref))
        worst_b = max(worst_b, _rel(dpb[ws:ws + W].cpu().numpy(), ref_b))
    print(f"  dPi worst rel={worst:.3e} dPibar worst rel={worst_b:.3e}")
    assert worst <= TOL[dt] and worst_b <= TOL[dt]


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True)])
def test_jvp_root_scores_matches_oracle(name, statewise):
    from kbench.newton.hvp import TangentForward
    from kbench.percall.solve import plan_of, run_forward

    print(f"[jvp] config={name} statewise={statewise}", flush=True)
    static, theta, cw = _static(name, statewise)
    _, sv = run_forward(static, theta, cw)
    v = torch.as_tensor(np.random.default_rng(14).normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda()
    n_it = int(static.solver_options.pi_iters)
    roots, full = TangentForward(plan_of(static), sv).run(theta, v, sweeps=n_it)
    full = {"dPi": full.dPi, "dPibar": full.dPibar}
    torch.cuda.synchronize()
    prob, _, saved = kbtest.oracle_forward(name, statewise)
    th = np.asarray(kbtest.problem(name, statewise)["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    r_ref, dPi_ref, dPb_ref = O.jvp_root_scores(prob, th, v.cpu().double().numpy(), saved, self_iters=n_it)
    e_r = _rel(roots.cpu().numpy(), r_ref)
    e_pi = _rel(full["dPi"].cpu().numpy(), dPi_ref)
    e_pb = _rel(full["dPibar"].cpu().numpy(), dPb_ref)
    print(f"  roots rel={e_r:.3e} dPi rel={e_pi:.3e} dPibar rel={e_pb:.3e}")
    assert e_r <= 1e-4 and e_pi <= 1e-4 and e_pb <= 1e-4


def test_jvp_root_scores_adaptive_and_unfused_paths_agree():
    """The three self-loop modes of the tangent forward solve the same tangent (config 1)."""
    from kbench.newton.hvp import TangentForward
    from kbench.percall.solve import plan_of, run_forward

    static, theta, cw = _static("1", True)
    _, sv = run_forward(static, theta, cw)
    v = torch.as_tensor(np.random.default_rng(15).normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda()
    tf = TangentForward(plan_of(static), sv)
    a = tf.run(theta, v, sweeps=6)[0]
    b = tf.run(theta, v, sweeps=6, one_call=False)[0]
    c = tf.run(theta, v, sweeps=None, tol=1e-7, max_sweeps=200)[0]
    d = tf.run(theta, v, sweeps=60)[0]
    torch.cuda.synchronize()
    assert _rel(a.cpu().numpy(), b.cpu().numpy()) <= 1e-5
    assert _rel(c.cpu().numpy(), d.cpu().numpy()) <= 1e-4


def test_jvp_root_scores_config3_linear_and_deterministic():
    """Full size (config 3): the JVP is linear in v and bitwise reproducible."""
    from kbench.newton.hvp import TangentForward
    from kbench.percall.solve import plan_of, run_forward

    print("[jvp] config=3", flush=True)
    static, theta, cw = _static("3")
    _, sv = run_forward(static, theta, cw)
    tf = TangentForward(plan_of(static), sv)
    jvp_root_scores = lambda static, theta, v, sv, self_iters: tf.run(theta, v, sweeps=self_iters)[0]
    g = np.random.default_rng(16)
    v1 = torch.as_tensor(g.normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda()
    v2 = torch.as_tensor(g.normal(size=tuple(theta.shape)), dtype=theta.dtype).cuda()
    n_it = int(static.solver_options.pi_iters)
    j1 = jvp_root_scores(static, theta, v1, sv, self_iters=n_it)
    j1b = jvp_root_scores(static, theta, v1, sv, self_iters=n_it)
    j2 = jvp_root_scores(static, theta, v2, sv, self_iters=n_it)
    j12 = jvp_root_scores(static, theta, v1 + 2.0 * v2, sv, self_iters=n_it)
    torch.cuda.synchronize()
    assert torch.equal(j1, j1b)
    assert torch.isfinite(j12).all()
    e = _rel(j12.cpu().numpy(), (j1 + 2.0 * j2).cpu().numpy())
    print(f"  linearity rel={e:.3e}")
    assert e <= 1e-4
