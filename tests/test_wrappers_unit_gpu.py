"""Per-call GPU parity of the first-order wrappers against the float64 CPU oracle.

Each wrapper of ``kbench.core.kernels`` is called once on the oracle's own
primal point (config 1: Pi*, Pibar*, E*, ... of the float64 oracle forward)
and every output of that call is compared with the oracle function that
restates the same reference kernel:

* ``compute_dts_forward`` (pristine dts_fused.py:171-231): ``dts_r`` with and
  without the active-parent mask;
* ``compute_leaf_initial_wave_step`` / ``compute_wave_step``
  (pristine wave_step.py:313-410): one sweep of a leaf wave and of a split
  wave (from the split term, ``input_ws=0``, and from Pi rows), with the final
  Pibar rows and row maxima;
* ``wave_backward_uniform_fused`` (pristine wave_backward.py:1398-1522):
  ``v_k`` on active rows and ``aw0..aw4``, ``aw345`` (zero on inactive rows,
  wave_backward.py:961-966), and the ``grad_col`` increment;
* ``dts_cross_backward_accum_fused`` (pristine wave_backward.py:1980-2190):
  the children's direct adjoint rows added into ``accumulated_rhs``, ``ud``
  and ``A`` of the active parents' sides, ``side_active``, and the
  ``grad_log_pD`` / ``grad_log_pS`` / ``grad_mt`` increments;
* ``uniform_cross_pibar_vjp_tree_from_ud_fused`` (pristine
  wave_backward.py:2330-2446): the in-place subtree sums of ``ud``, the Pibar
  VJP rows added into ``accumulated_rhs`` and the ``grad_col`` increment;
* ``e_step_triton_autograd`` (pristine e_step.py:290-435): one E-step and its
  VJP for every input.

float64 calls use the same arithmetic as the oracle up to summation order
(tolerance 1e-9 of max(1, max|ref|)); float32 calls take the float32-rounded
primal point, with the oracle evaluated at the same rounded values
(tolerance 1e-4).  Inactive rows of ``v_k`` are "don't care" in the reference
(its FIXES.md:56-85) and are not compared.
"""

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-9, torch.float32: 1e-4}
NAME, STATEWISE = "1", True


def _t(x, dt):
    return torch.as_tensor(np.ascontiguousarray(x), dtype=dt, device="cuda")


def _np(t):
    return t.detach().double().cpu().numpy()


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all() and np.isfinite(ref).all()
    if got.size == 0:
        return 0.0
    return float(np.abs(got - ref).max()) / max(1.0, float(np.abs(ref).max()))


def _check_inf_safe(name, got, ref, dt):
    ok, ma, mr = kbtest.compare_inf_safe(got, ref)
    print(f"  {name}: pattern={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
    assert ok, f"{name}: -inf pattern differs"
    assert ma <= TOL[dt] * max(1.0, float(np.abs(ref[np.isfinite(ref)]).max(initial=0.0))), name


class Point:
    """The oracle's forward point, rounded to the call dtype, on the host and the device."""

    def __init__(self, dt):
        self.dt = dt
        self.prob, _, saved = kbtest.oracle_forward(NAME, STATEWISE)
        rnd = (lambda a: np.asarray(a, dtype=np.float64).astype(np.float32).astype(np.float64)) \
            if dt == torch.float32 else (lambda a: np.asarray(a, dtype=np.float64))
        self.h = {k: rnd(v) for k, v in saved.items() if isinstance(v, np.ndarray)}
        p = self.prob
        S, G = p.S, 1
        st = lambda k: np.broadcast_to(O.as_item_state(self.h[k], S, G), (G, S)).copy()
        self.E, self.Ebar, self.Es1, self.Es2 = (st(k) for k in ("E", "Ebar", "E_s1", "E_s2"))
        self.pS, self.pD, self.mt = st("log_pS"), st("log_pD"), st("max_coupling")
        self.col = self.h["col_log_probs"]
        self.consts = {
            "mt": self.mt, "DL": rnd(1.0 + self.pD + self.E), "Ebar": self.Ebar, "E": self.E,
            "SL1": rnd(self.pS + self.Es2), "SL2": rnd(self.pS + self.Es1),
        }
        self.Pi, self.Pb, self.rmax = self.h["pi_wave"], self.h["pibar_wave"], self.h["pibar_row_max"]
        problem = kbtest.problem(NAME, STATEWISE)
        helpers = problem["static"]["state_helpers"]
        self.helpers = {k: torch.as_tensor(np.asarray(v)).cuda() if isinstance(v, np.ndarray) else v
                        for k, v in helpers.items()}
        wl = problem["static"]["wave_layout"]
        self.item_idx = torch.as_tensor(np.asarray(problem["static"]["rate_item_idx"])).cuda()
        self.leaf_idx = torch.as_tensor(np.asarray(wl["leaf_state_index"])).cuda()
        self.metas = wl["wave_metas"]

    def oconsts(self, use_col):
        c = self.consts
        return O.WaveConsts(mt=c["mt"], DL=c["DL"], Ebar=c["Ebar"], E=c["E"], SL1=c["SL1"], SL2=c["SL2"],
                            leaf_logp=self.pS, col=self.col, use_col_weights=use_col)

    def dconsts(self):
        return [_t(self.consts[k], self.dt) for k in ("mt", "DL", "Ebar", "E", "SL1", "SL2")]

    def dmeta(self, m):
        out = {}
        for k, v in m.items():
            out[k] = torch.as_tensor(np.asarray(v)).cuda() if isinstance(v, np.ndarray) else v
        if "log_split_probs" in out and torch.is_tensor(out["log_split_probs"]):
            out["log_split_probs"] = out["log_split_probs"].to(self.dt)
        return out

    def split_waves(self):
        return [m for m in self.metas if "sl" in m]

    def wide_split_waves(self, k=2):
        """The k split waves with the most rows (widest first)."""
        return sorted(self.split_waves(), key=lambda m: -int(m["W"]))[:k]

    def leaf_waves(self):
        return [m for m in self.metas if "sl" not in m]

    def levels(self):
        h = self.helpers
        return dict(compact_level_ptr=h["compact_level_ptr"], compact_level_parents=h["compact_level_parents"],
                    compact_level_child1=h["compact_level_child1"], compact_level_child2=h["compact_level_child2"])


_POINTS = {}


def point(dt):
    if dt not in _POINTS:
        _POINTS[dt] = Point(dt)
    return _POINTS[dt]


def _rhs(W, S, seed, inactive_every=3):
    """Seeded adjoint rows: every third row zero (inactive), one row just below the threshold."""
    g = np.random.default_rng(seed)
    rhs = -np.abs(g.normal(size=(W, S))) * 1e-2
    rhs[::inactive_every] = 0.0
    if W > 1:
        rhs[1] = 0.0
        rhs[1, 0] = -0.5e-6  # below the 1e-6 pruning threshold: inactive
    return rhs


# ---------------------------------------------------------------------- forward
@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_compute_dts_forward_matches_oracle(dt):
    from kbench.core.kernels.dts_fused import compute_dts_forward

    P = point(dt)
    print(f"[unit dts_forward] config={NAME} statewise={STATEWISE} dtype={dt}", flush=True)
    S, G = P.prob.S, 1
    pD_par, pS_par = O.as_item_param(P.h["log_pD"], G, S), O.as_item_param(P.h["log_pS"], G, S)
    Pi_d, Pb_d = _t(P.Pi, dt), _t(P.Pb, dt)
    h = P.helpers
    for m in P.split_waves():
        ws, W = int(m["start"]), int(m["W"])
        dm = P.dmeta(m)
        act = np.ones(W, dtype=bool)
        act[::2] = False
        for mask in (None, act):
            ref = O.dts_forward(P.Pi, P.Pb, m, W, pD_par, pS_par, P.prob.item_idx, ws, P.prob.tree, active=mask)
            got = compute_dts_forward(
                Pi_d, Pb_d, dm["sl"], dm["sr"], h["node_child1"], h["node_child2"], W, dm["reduce_idx"],
                _t(pD_par, dt), _t(pS_par, dt), P.item_idx, log_split_probs=dm.get("log_split_probs"),
                n_eq1=dm.get("n_eq1"), eq1_reduce_idx=dm.get("eq1_reduce_idx"), ge2_ptr=dm.get("ge2_ptr"),
                ge2_parent_ids=dm.get("ge2_parent_ids"), ge2_max_fanout=dm.get("ge2_max_fanout"),
                active_parent_rows=None if mask is None else torch.as_tensor(mask).cuda(), item_offset=ws)
            torch.cuda.synchronize()
            _check_inf_safe(f"wave@{ws} dts_r mask={mask is not None}", _np(got), ref, dt)


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_leaf_init_and_sweeps_match_oracle(dt):
    from kbench.core.kernels.dts_fused import compute_dts_forward
    from kbench.core.kernels.wave_step import compute_leaf_initial_wave_step, compute_wave_step

    P = point(dt)
    print(f"[unit wave_step] config={NAME} statewise={STATEWISE} dtype={dt}", flush=True)
    S, C, G = P.prob.S, P.prob.C, 1
    h = P.helpers
    oc = P.oconsts(False)
    mt, DL, Eb, Ev, SL1, SL2 = P.dconsts()
    col = _t(P.col, dt)
    lp = _t(P.pS, dt)
    common = dict(leaf_state_idx=P.leaf_idx, leaf_logp=lp, item_idx=P.item_idx, use_col_weights=False)
    args = lambda ws, W: (ws, W, S, mt, DL, Eb, Ev, SL1, SL2, col, h["node_child1"], h["node_child2"],
                          h["node_parent"], int(h["max_ancestor_depth"]))

    # leaf wave: leaf initialisation, then one sweep from it with the final Pibar
    m = P.leaf_waves()[0]
    ws, W = int(m["start"]), int(m["W"])
    rows = np.arange(ws, ws + W)
    items = P.prob.item_idx[rows]
    leaf = P.prob.leaf_state[rows]
    buf = torch.full((C, S), float("nan"), dtype=dt, device="cuda")
    compute_leaf_initial_wave_step(buf, ws, W, S, mt, DL, Eb, Ev, SL1, SL2, col, h["node_child1"], h["node_child2"],
                                   h["node_subtree_start"], h["node_subtree_end"], P.leaf_idx, lp, P.item_idx,
                                   use_col_weights=False)
    torch.cuda.synchronize()
    ref0 = O.leaf_initial(leaf, items, oc, P.prob.tree)
    got0 = _np(buf[ws:ws + W])
    _check_inf_safe("leaf init", got0, ref0, dt)
    # the sweep reads the device rows (identical pattern, values within tolerance)
    out = torch.full((C, S), float("nan"), dtype=dt, device="cuda")
    pibar = torch.full((C, S), float("nan"), dtype=dt, device="cuda")
    rmax = torch.full((C,), float("nan"), dtype=dt, device="cuda")
    compute_wave_step(buf, out, pibar, *args(ws, W), None, pibar_row_max=rmax, store_final_pibar=True,
                      has_leaf_term=True, **common)
    torch.cuda.synchronize()
    ref1 = O.wave_sweep(got0, items, oc, P.prob.tree, leaf_state=leaf)
    refb, refm = O._pibar_from_pi(ref1, P.col, P.mt[items], P.prob.tree, False)
    _check_inf_safe("leaf sweep Pi", _np(out[ws:ws + W]), ref1, dt)
    _check_inf_safe("leaf sweep Pibar", _np(pibar[ws:ws + W]), refb, dt)
    _check_inf_safe("leaf sweep row max", _np(rmax[ws:ws + W]), refm, dt)

    # split wave: sweep from the split term (input_ws = 0) and from the Pi rows
    pD_par, pS_par = O.as_item_param(P.h["log_pD"], G, S), O.as_item_param(P.h["log_pS"], G, S)
    m = P.wide_split_waves(1)[0]
    dm = P.dmeta(m)
    ws, W = int(m["start"]), int(m["W"])
    rows = np.arange(ws, ws + W)
    items = P.prob.item_idx[rows]
    dts = O.dts_forward(P.Pi, P.Pb, m, W, pD_par, pS_par, P.prob.item_idx, ws, P.prob.tree)
    dts_d = compute_dts_forward(_t(P.Pi, dt), _t(P.Pb, dt), dm["sl"], dm["sr"], h["node_child1"], h["node_child2"],
                                W, dm["reduce_idx"], _t(pD_par, dt), _t(pS_par, dt), P.item_idx,
                                log_split_probs=dm.get("log_split_probs"), item_offset=ws)
    for from_split in (True, False):
        src = dts_d if from_split else _t(P.Pi, dt)
        src_h = _np(dts_d) if from_split else P.Pi[rows]
        out = torch.full((C, S), float("nan"), dtype=dt, device="cuda")
        pibar = torch.full((C, S), float("nan"), dtype=dt, device="cuda")
        rmax = torch.full((C,), float("nan"), dtype=dt, device="cuda")
        compute_wave_step(src, out, pibar, *args(ws, W), dts_d, pibar_row_max=rmax, store_final_pibar=True,
                          has_leaf_term=False, input_ws=0 if from_split else None, **common)
        torch.cuda.synchronize()
        ref1 = O.wave_sweep(src_h, items, oc, P.prob.tree, dts_r=_np(dts_d))
        refb, refm = O._pibar_from_pi(ref1, P.col, P.mt[items], P.prob.tree, False)
        tag = "from dts" if from_split else "from Pi"
        _check_inf_safe(f"split sweep {tag} Pi", _np(out[ws:ws + W]), ref1, dt)
        _check_inf_safe(f"split sweep {tag} Pibar", _np(pibar[ws:ws + W]), refb, dt)
        _check_inf_safe(f"split sweep {tag} row max", _np(rmax[ws:ws + W]), refm, dt)
    # a sweep without store_final_pibar leaves Pibar and the row maxima alone
    pibar = torch.full((C, S), 7.0, dtype=dt, device="cuda")
    rmax = torch.full((C,), 7.0, dtype=dt, device="cuda")
    out = torch.empty((C, S), dtype=dt, device="cuda")
    compute_wave_step(_t(P.Pi, dt), out, pibar, *args(ws, W), dts_d, pibar_row_max=rmax, store_final_pibar=False,
                      has_leaf_term=False, **common)
    torch.cuda.synchronize()
    assert bool((pibar == 7.0).all()) and bool((rmax == 7.0).all())


# ---------------------------------------------------------------------- backward
def _wave_backward_case(P, dt, m, use_col, neumann_terms=5, solver="neumann", grad_targets=None):
    """(device outputs, oracle outputs, active mask) of one wave_backward_uniform_fused call."""
    from kbench.core.kernels.dts_fused import compute_dts_forward
    from kbench.core.kernels.wave_backward import active_mask_from_rhs_absmax_fused, wave_backward_uniform_fused

    S, G = P.prob.S, 1
    h = P.helpers
    ws, W = int(m["start"]), int(m["W"])
    rows = np.arange(ws, ws + W)
    items = P.prob.item_idx[rows]
    has_splits = "sl" in m
    rhs = _rhs(W, S, seed=100 + ws)
    if dt == torch.float32:
        rhs = rhs.astype(np.float32).astype(np.float64)
    act = O.active_mask(rhs, 1e-6, True)
    act_d = active_mask_from_rhs_absmax_fused(_t(rhs, dt), 1e-6, use_pruning=True)
    assert (act_d.cpu().numpy() == act).all(), "active mask differs"
    pD_par, pS_par = O.as_item_param(P.h["log_pD"], G, S), O.as_item_param(P.h["log_pS"], G, S)
    dts = dts_d = None
    if has_splits:
        dm = P.dmeta(m)
        dts = O.dts_forward(P.Pi, P.Pb, m, W, pD_par, pS_par, P.prob.item_idx, ws, P.prob.tree, active=act)
        dts_d = compute_dts_forward(_t(P.Pi, dt), _t(P.Pb, dt), dm["sl"], dm["sr"], h["node_child1"],
                                    h["node_child2"], W, dm["reduce_idx"], _t(pD_par, dt), _t(pS_par, dt),
                                    P.item_idx, log_split_probs=dm.get("log_split_probs"),
                                    active_parent_rows=act_d, item_offset=ws)
        dts = _np(dts_d)  # same values within tolerance; the oracle continues from the device's
    leaf = None if has_splits else P.prob.leaf_state[rows]
    ref = O.wave_backward_uniform(P.Pi[rows], P.Pb[rows], P.rmax[rows], rhs, items, P.oconsts(use_col),
                                  P.prob.tree, neumann_terms, active=act, leaf_state=leaf, dts_r=dts, solver=solver)
    mt, DL, Eb, Ev, SL1, SL2 = P.dconsts()
    gcol = torch.zeros((S,), dtype=dt, device="cuda")
    got = wave_backward_uniform_fused(
        _t(P.Pi, dt), _t(P.Pb, dt), ws, W, S, dts_d, _t(rhs, dt), mt, DL, Eb, Ev, SL1, SL2, _t(P.col, dt),
        h["node_child1"], h["node_child2"], None, neumann_terms=neumann_terms, leaf_state_idx=P.leaf_idx,
        leaf_logp=_t(P.pS, dt), has_leaf_term=not has_splits, active_mask=act_d, node_parent=h["node_parent"],
        max_ancestor_depth=int(h["max_ancestor_depth"]), pibar_row_max=_t(P.rmax, dt), item_idx=P.item_idx,
        item_indexed_consts=True, grad_col_log_probs=gcol, use_col_weights=use_col, self_loop_solver=solver,
        self_loop_grad_targets=grad_targets, **P.levels())
    torch.cuda.synchronize()
    return [None if x is None else _np(x) for x in got] + [_np(gcol)], list(ref), act


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("use_col", [False, True])
def test_wave_backward_uniform_outputs_match_oracle(dt, use_col):
    P = point(dt)
    print(f"[unit wave_backward] config={NAME} statewise={STATEWISE} dtype={dt} use_col={use_col}", flush=True)
    names = ("v_k", "aw0", "aw1", "aw2", "aw345", "aw3", "aw4", "grad_col")
    for m in (P.leaf_waves()[0], *P.wide_split_waves(2)):
        got, ref, act = _wave_backward_case(P, dt, m, use_col)
        assert act.any() and not act.all()
        for name, g, r in zip(names, got, ref):
            if name == "v_k":
                g, r = g[act], r[act]  # inactive rows of v_k are don't-care
            elif name != "grad_col":
                assert (g[~act] == 0).all(), f"{name}: inactive rows must be zero"
            e = _rel(g, r)
            print(f"  wave@{int(m['start'])} {name}: rel={e:.3e}")
            assert e <= TOL[dt], name


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_wave_backward_gmres_matches_oracle(dt):
    """self_loop_solver="gmres": the wave's GMRES solution (host Krylov loop over HIP J^T applications)
    and every output computed from it, against the oracle's GMRES (pristine wave_backward.py:574-653)."""
    P = point(dt)
    print(f"[unit wave_backward gmres] config={NAME} statewise={STATEWISE} dtype={dt}", flush=True)
    names = ("v_k", "aw0", "aw1", "aw2", "aw345", "aw3", "aw4", "grad_col")
    for m in (P.leaf_waves()[0], *P.wide_split_waves(2)):
        got, ref, act = _wave_backward_case(P, dt, m, True, neumann_terms=6, solver="gmres")
        for name, g, r in zip(names, got, ref):
            if name == "v_k":
                g, r = g[act], r[act]
            elif name != "grad_col":
                assert (g[~act] == 0).all(), f"{name}: inactive rows must be zero"
            e = _rel(g, r)
            print(f"  wave@{int(m['start'])} {name}: rel={e:.3e}")
            assert e <= TOL[dt], name


@pytest.mark.parametrize("vector", [True, False])
def test_self_loop_grad_targets_receive_the_bucket_sums(vector):
    """self_loop_grad_targets: the buckets are added into the caller's accumulators, summed over the
    wave's rows per state (pD / pS per state or in total), and not returned."""
    dt = torch.float64
    P = point(dt)
    S = P.prob.S
    print(f"[unit wave_backward grad targets] param_grad_vector={vector}", flush=True)
    m = P.wide_split_waves(1)[0]
    base, _, _ = _wave_backward_case(P, dt, m, False)
    v, aw0, aw1, aw2, aw345, aw3, aw4, _ = base
    z = lambda n: torch.zeros((n,), dtype=dt, device="cuda")
    tg = [z(S if vector else 1), z(S if vector else 1), z(S), z(S), z(S), z(S), z(S)]
    got, _, _ = _wave_backward_case(P, dt, m, False, grad_targets=(*tg, vector))
    assert all(x is None for x in got[1:7])
    assert _rel(got[0], v) == 0.0
    want = [aw0.sum(0), aw345.sum(0), (aw0 + aw2).sum(0), aw1.sum(0), aw4.sum(0), aw3.sum(0), aw2.sum(0)]
    if not vector:
        want[0], want[1] = want[0].sum(keepdims=True), want[1].sum(keepdims=True)
    for name, t, w in zip(("pD", "pS", "E", "Ebar", "E_s1", "E_s2", "mt"), tg, want):
        e = _rel(_np(t), w)
        print(f"  {name}: rel={e:.3e}")
        assert e <= 1e-12, name


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_split_adjoint_and_pibar_vjp_outputs_match_oracle(dt):
    from kbench.core.kernels.wave_backward import (dts_cross_backward_accum_fused,
                                                   uniform_cross_pibar_vjp_tree_from_ud_fused)

    P = point(dt)
    print(f"[unit dts_cross + pibar_vjp] config={NAME} statewise={STATEWISE} dtype={dt}", flush=True)
    S, C, G = P.prob.S, P.prob.C, 1
    h = P.helpers
    pD_par, pS_par = O.as_item_param(P.h["log_pD"], G, S), O.as_item_param(P.h["log_pS"], G, S)
    for m in P.wide_split_waves(2):
        ws, W = int(m["start"]), int(m["W"])
        dm = P.dmeta(m)
        got_bw, _, act = _wave_backward_case(P, dt, m, use_col=False)
        v = got_bw[0]
        v = np.where(act[:, None], v, 0.0)
        ref = O.dts_cross_backward(P.Pi, P.Pb, P.rmax, v, ws, m, pD_par, pS_par, P.mt, P.prob.item_idx,
                                   P.prob.tree, act, P.col, False)
        sl, sr = np.asarray(m["sl"]), np.asarray(m["sr"])
        n = sl.shape[0]
        on = ref["active_split"]
        base = np.random.default_rng(7).normal(size=(C, S)) * 1e-3
        acc = _t(base, dt)
        gpD = torch.zeros((1, S), dtype=dt, device="cuda")
        gpS = torch.zeros((1, S), dtype=dt, device="cuda")
        gmt = torch.zeros((1, S), dtype=dt, device="cuda")
        ud, A, side_active, _, _ = dts_cross_backward_accum_fused(
            _t(P.Pi, dt), _t(P.Pb, dt), _t(v, dt), ws, dm["sl"], dm["sr"], dm["reduce_idx"],
            dm.get("log_split_probs", dm["sl"].new_zeros((n,), dtype=dt)), _t(pD_par, dt), _t(pS_par, dt),
            h["node_child1"], h["node_child2"], acc, S, active_mask=torch.as_tensor(act).cuda(), merge_s_term=True,
            grad_log_pD=gpD, grad_log_pS=gpS, grad_mt=gmt, accum_param_reductions=True, accum_mt_reduction=True,
            output_pibar_ud=True, output_pibar_side_active=True, pibar_side_threshold=0.0, mt_squeezed=_t(P.mt, dt),
            pibar_row_max=_t(P.rmax, dt), grad_mt_two_stage=True, skip_inactive_pibar_output_zero=True,
            item_idx=P.item_idx)
        torch.cuda.synchronize()
        # children's direct adjoint rows
        want = base.copy()
        np.add.at(want, sl, ref["direct_l"])
        np.add.at(want, sr, ref["direct_r"])
        e = _rel(_np(acc), want)
        print(f"  wave@{ws} accumulated_rhs (direct): rel={e:.3e}")
        assert e <= TOL[dt]
        # u_d staging, row sums and side flags of the active parents' sides
        ud_h, A_h, sa_h = _np(ud), _np(A), side_active.cpu().numpy()
        on2 = np.concatenate([on, on])
        ref_ud = np.concatenate([ref["ud_l"], ref["ud_r"]])
        ref_A = np.concatenate([ref["A_l"], ref["A_r"]])
        for name, g, r in (("ud", ud_h[on2], ref_ud[on2]), ("A", A_h[on2], ref_A[on2])):
            e = _rel(g, r)
            print(f"  wave@{ws} {name}: rel={e:.3e}")
            assert e <= TOL[dt], name
        assert (sa_h[on2] == (np.abs(ref_ud[on2]).max(axis=1) != 0)).all(), "side_active differs"
        # parameter and coupling gradients
        for name, g, r in (("grad_log_pD", _np(gpD)[0], ref["g_pD"].sum(axis=0)),
                           ("grad_log_pS", _np(gpS)[0], ref["g_pS"].sum(axis=0)),
                           ("grad_mt", _np(gmt)[0], ref["g_mt_l"].sum(axis=0) + ref["g_mt_r"].sum(axis=0))):
            e = _rel(g, r)
            print(f"  wave@{ws} {name}: rel={e:.3e}")
            assert e <= TOL[dt], name
        # Pibar VJP of the staged u_d
        acc2 = _t(base, dt)
        gcol = torch.zeros((S,), dtype=dt, device="cuda")
        uniform_cross_pibar_vjp_tree_from_ud_fused(
            _t(P.Pi, dt), _t(P.col, dt), ud, A, dm["sl"], dm["sr"], acc2, S, active_mask=torch.as_tensor(act).cuda(),
            reduce_idx=dm["reduce_idx"], pibar_row_max=_t(P.rmax, dt), skip_zero_sides=True, side_active=side_active,
            grad_col_log_probs=gcol, use_col_weights=False, side_active_threshold=0.0, **P.levels())
        torch.cuda.synchronize()
        want = base.copy()
        np.add.at(want, sl, ref["tree_l"])
        np.add.at(want, sr, ref["tree_r"])
        e = _rel(_np(acc2), want)
        print(f"  wave@{ws} accumulated_rhs (Pibar VJP): rel={e:.3e}")
        assert e <= TOL[dt]
        e = _rel(_np(gcol), ref["col_grad"])
        print(f"  wave@{ws} grad_col: rel={e:.3e}")
        assert e <= TOL[dt]
        live = on2 & sa_h
        ref_sub = np.concatenate([ref["sub_l"], ref["sub_r"]])
        e = _rel(_np(ud)[live], ref_sub[live])
        print(f"  wave@{ws} ud subtree sums (in place): rel={e:.3e}")
        assert e <= TOL[dt]


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
@pytest.mark.parametrize("use_col", [False, True])
def test_e_step_autograd_matches_oracle(dt, use_col):
    from kbench.core.kernels.e_step import e_step_triton_autograd

    P = point(dt)
    print(f"[unit e_step autograd] config={NAME} dtype={dt} use_col={use_col}", flush=True)
    S, G = P.prob.S, 1
    g = np.random.default_rng(3)
    col = P.col + (g.normal(size=S) * 0.3 if use_col else 0.0)
    pL = np.broadcast_to(O.as_item_state(P.h["log_pL"], S, G), (G, S)).copy()
    inputs = [P.E, P.pS, P.pD, pL, P.mt, col]
    if dt == torch.float32:
        inputs = [x.astype(np.float32).astype(np.float64) for x in inputs]
    ref = O.e_step(*inputs, P.prob.tree, use_col)
    cot = [g.normal(size=(G, S)) for _ in range(4)]
    if dt == torch.float32:
        cot = [x.astype(np.float32).astype(np.float64) for x in cot]
    ref_g = O.e_step_vjp(*inputs, P.prob.tree, use_col, *cot)
    h = P.helpers
    xs = [_t(x, dt).requires_grad_(True) for x in inputs]
    out = e_step_triton_autograd(*xs, h["node_parent"], h["node_child1"], h["node_child2"],
                                 int(h["max_ancestor_depth"]), use_col_weights=use_col)
    grads = torch.autograd.grad(out, xs, grad_outputs=[_t(c, dt) for c in cot])
    torch.cuda.synchronize()
    for name, a, b in zip(("E_new", "E_s1", "E_s2", "Ebar"), out, ref):
        _check_inf_safe(name, _np(a), b, dt)
    for name, a, b in zip(("grad_E", "grad_log_pS", "grad_log_pD", "grad_log_pL", "grad_mt", "grad_col"),
                          grads, ref_g):
        e = _rel(_np(a).reshape(np.shape(b)), b)
        print(f"  {name}: rel={e:.3e}")
        assert e <= TOL[dt], name


@pytest.mark.parametrize("n", [1, 64, 300])
@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
def test_rows_sum_accum_adds_float64_column_sums(n, dt):
    """kb_rows_sum_accum: blocks of 1..4 addends and different row counts added into their own
    accumulators, against float64 sums; one addend gives bitwise what kb_rows_sum_into gives."""
    from kbench.core.kernels import _hip as H

    g = torch.Generator(device="cpu").manual_seed(n + 1)
    S = 37
    rows = lambda m: torch.randn((m, S), generator=g, dtype=torch.float64).to(device="cuda", dtype=dt)
    xs = [rows(n) for _ in range(7)] + [rows(2 * n + 5)]
    groups = [(xs[0],), (xs[1], xs[2]), (xs[3], xs[4], xs[5]), (xs[0], xs[2], xs[4], xs[6]), (xs[7],)]
    base = [torch.randn((S,), generator=g, dtype=torch.float64).to(device="cuda", dtype=dt) for _ in groups]
    dst = [b.clone() for b in base]
    H.rows_sum_accum(list(zip(dst, groups)))
    one = base[4].clone()
    H.sum_rows_into(one, xs[7])
    torch.cuda.synchronize()
    assert torch.equal(dst[4], one)
    for d, b, grp in zip(dst, base, groups):
        ref = b.double() + sum(x.double() for x in grp).sum(dim=0)
        err = float((d.double() - ref).abs().max() / ref.abs().max())
        print(f"[rows-sum-accum] n={n} k={len(grp)} dtype={dt} rel={err:.3e}")
        assert err <= (1e-6 if dt == torch.float32 else 1e-13)


@pytest.mark.parametrize("n", [1, 64, 300])
@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
def test_rows_sum_multi_matches_float64_column_sums(n, dt):
    """kb_rows_sum_multi: column sums of single and paired row blocks, against float64 sums, and run
    twice bitwise (fixed order)."""
    from kbench.core.kernels import _hip as H

    g = torch.Generator(device="cpu").manual_seed(n)
    S = 37
    xs = [torch.randn((n, S), generator=g, dtype=torch.float64).to(device="cuda", dtype=dt) for _ in range(7)]
    blocks = [xs[0], (xs[1], xs[2]), xs[3], (xs[4], xs[5]), xs[6]]
    out = H.rows_sum_multi(blocks)
    again = H.rows_sum_multi(blocks)
    torch.cuda.synchronize()
    assert out.shape == (5, S) and out.dtype == dt
    assert torch.equal(out, again)
    ref = torch.stack([(b[0].double() + b[1].double()) if isinstance(b, tuple) else b.double() for b in blocks])
    ref = ref.sum(dim=1)
    err = float((out.double() - ref).abs().max() / ref.abs().max())
    print(f"[rows-sum-multi] n={n} dtype={dt} rel={err:.3e}")
    assert err <= (1e-6 if dt == torch.float32 else 1e-13)
