"""Hessian-vector products of the loss through the per-call wrappers (config 5).

Forward over reverse at a fixed theta, with the wrapper calls of the
reference's newton/forward_tangent.py:99-209 and newton/hvp_exact.py:54-383:

tangent forward (``TangentForward``)
  parameter tangents (a JVP of the rate extraction), ``e_tangent_fixed_point``,
  then per wave in order: ``compute_dts_forward`` + ``compute_dts_tangent``
  (split waves) and the self-loop tangent at Pi* --
  ``compute_wave_step_tangent_selfloop`` for a fixed sweep count in one call,
  the same count as repeated ``compute_wave_step_tangent`` calls, or sweeps
  until max|change| <= tol * max(1, max|dPi|).

tangent reverse (``HvpPlan``), per cached wave in reverse order
  ``compute_dts_tangent`` at the cached split term, ``wave_backward_so`` at the
  cached adjoint (seeded with the tangent adjoint rows, FOLD_RHS), the tangent
  adjoint solve ``wave_backward_uniform_fused`` with the cached mask, the
  bucket sums, then ``dts_cross_backward_accum_fused``,
  ``uniform_cross_pibar_vjp_tree_from_ud_fused`` and ``dts_backward_so``
  (split waves).

E side and head
  ``e_step_backward_so`` contractions at the cached E adjoint, a BiCGSTAB solve
  of the tangent E adjoint, the E-step parameter VJP, and the second
  derivative of the rate extraction by autograd.

The point cache (one backward at theta keeping every wave's adjoint, split
term and mask, the accumulated cotangents and the E adjoint) is built once per
theta by ``SolvePlan.reverse_sweep`` / ``e_adjoint_and_vjp``.

Row classes (``HvpPlan(..., row_classes=True)``): rows with the same inputs
(``synth.row_classes``) have the same forward rows and the same forward
tangents, so the tangent forward runs on one row per class (config 3: 11253
of 33686 rows).  The tangent reverse is linear in the point adjoint v and in
the right-hand sides it propagates, and members of a class whose active flags
agree, and whose children along each split agree in class and flag, share
one adjoint map; so it runs on one row per such class (the classes of
``row_classes`` with the point's active mask), from the members' summed
adjoints and root seeds (fixed-order sums).  On the classes the reverse's
second-order terms, which read the point adjoint and the tangent rows but not
the tangent adjoint, run first as one launch each over all split rows; the
level loop then carries the first-order adjoint only.  The bucket sums, and
through them H u, are those of the row-by-row reverse up to the order of the
sums.

HIP graph (``HvpPlan(..., graph=True)``): for a fixed point the tangent
forward and reverse launch the same kernels on the same buffers for every u,
with no host read in between; they are captured once into a graph and
replayed (the E side, whose BiCGSTAB tests convergence on the host, and the
parameter head run eagerly).  A replay gives bitwise the eager result.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch
from torch.func import jvp

from kbench.core.parameters.extract_parameters import (as_item_param, as_item_state, extract_parameters_uniform,
                                                       extract_parameters_weighted_cols)

from kbench import synth
from kbench.core.kernels import _hip as H

from kbench.percall.krylov import bicgstab
from kbench.percall.solve import LN2, SolvePlan, root_softmax2


def _fold(acc, x, G, S):
    """acc + x for a parameter accumulator ([G, 1] or [G, S]) and an item-state term [G, S].

    With one value per item row the state axis of x is summed (the accumulator is
    counted once, not once per state).
    """
    x = as_item_param(x, G, S)
    if int(acc.shape[-1]) == 1 and int(x.shape[-1]) != 1:
        x = x.sum(dim=-1, keepdim=True)
    return acc + x


class TangentForward:
    """d(Pi)/d(theta) . u through the forward solve, at the saved point of ``plan``.

    ``split_terms`` (optional): the split term of each split wave at the point, keyed by the
    wave's first row, used instead of recomputing it from the saved rows.
    """

    def __init__(self, plan: SolvePlan, saved, split_terms=None):
        self.p = plan
        self.sv = saved
        self.split_terms = split_terms
        S, G = plan.S, int(saved["E"].shape[0])
        item = lambda t: as_item_state(t, S, G)
        E, pS, pD = item(saved["E"]), item(saved["log_pS"]), item(saved["log_pD"])
        self.base = SimpleNamespace(
            mc=item(saved["max_coupling"].squeeze(-1)), dl=1.0 + pD + E, ebar=item(saved["Ebar"]), e=E,
            sl1=pS + item(saved["E_s2"]), sl2=pS + item(saved["E_s1"]), leaf=pS,
            pd_par=as_item_param(saved["log_pD"], G, S), ps_par=as_item_param(saved["log_pS"], G, S))

    def param_tangent(self, theta, u):
        """(dpS, dpD, dpL, dmt): the rate extraction's JVP along u (uniform columns)."""
        st = self.p.static
        urm = self.p.h["unnorm_row_max"].to(device=theta.device, dtype=theta.dtype)
        _, tan = jvp(lambda th: extract_parameters_uniform(th, urm, statewise=st.statewise, itemwise=st.itemwise),
                     (theta,), (u,))
        return tan

    def constants(self, theta, u, e_tol):
        """Tangents of every constant row the sweeps read, plus the raw parameter / E tangents."""
        p, sv = self.p, self.sv
        S, G = p.S, int(sv["E"].shape[0])
        dpS, dpD, dpL, dmt = self.param_tangent(theta, u)
        dE, dEs1, dEs2, dEbar = p.k.e_tangent_fixed_point(
            sv["E"], dpS, dpD, dpL, dmt, sv["log_pS"], sv["log_pD"], sv["log_pL"], sv["max_coupling"],
            sv["col_log_probs"], *p.topo, max_iter=int(p.so.e_max_iter), tol=e_tol, use_col_weights=False)
        item = lambda t: as_item_state(t, S, G)
        de, dps = item(dE), item(dpS)
        return SimpleNamespace(
            dMC=item(dmt.squeeze(-1)), dDL=item(dpD) + de, dEbar=item(dEbar), dE=de, dSL1=dps + item(dEs2),
            dSL2=dps + item(dEs1), dleaf=dps, dpd_par=as_item_param(dpD, G, S), dps_par=as_item_param(dpS, G, S),
            raw=dict(dlog_pS=dpS, dlog_pD=dpD, dlog_pL=dpL, dmax_coupling=dmt, dE=dE, dE_s1=dEs1, dE_s2=dEs2,
                     dEbar=dEbar))

    def interleaved(self, d):
        b = self.base
        return (b.mc, d.dMC, b.dl, d.dDL, b.ebar, d.dEbar, b.e, d.dE, b.sl1, d.dSL1, b.sl2, d.dSL2)

    def run(self, theta, u, *, sweeps=None, one_call=True, tol=None, max_sweeps=200, e_tol=None):
        """-> (root-row tangents, namespace of dPi, dPibar, constant tangents).

        ``sweeps``: a fixed count of tangent sweeps per wave, in one call (``one_call``) or
        one call per sweep; ``None`` sweeps each wave until its largest change is at most
        ``tol * max(1, max|dPi|)`` (``max_sweeps`` at most), then once more storing dPibar.
        """
        p, sv = self.p, self.sv
        dt = sv["pi_wave"].dtype
        tol = (1e-12 if dt == torch.float64 else 1e-6) if tol is None else tol
        e_tol = (1e-12 if dt == torch.float64 else 1e-6) if e_tol is None else e_tol
        d = self.constants(theta, u, e_tol)
        pi, pibar = sv["pi_wave"], sv["pibar_wave"]
        dpi = torch.zeros_like(pi)
        dpibar = torch.zeros_like(pi)
        cst = self.interleaved(d)
        col = sv["col_log_probs"]
        h = p.h
        kw = dict(leaf_state_idx=p.leaf_idx, leaf_logp=self.base.leaf, dleaf_logp=d.dleaf, item_idx=p.item_idx,
                  use_col_weights=False)
        d_dts_of = {}
        for w in p.waves:
            dts = d_dts = None
            if w.split:
                lay = dict(log_split_probs=w.lsp, item_offset=w.ws, **w.extra)
                dts = self.split_terms.get(w.ws) if self.split_terms is not None else None
                if dts is None:
                    dts = p.k.compute_dts_forward(pi, pibar, w.sl, w.sr, h["node_child1"], h["node_child2"], w.W,
                                                  w.reduce_idx, self.base.pd_par, self.base.ps_par,
                                                  item_idx=p.item_idx, **lay)
                d_dts = p.k.compute_dts_tangent(pi, pibar, dpi, dpibar, w.sl, w.sr, h["node_child1"],
                                                h["node_child2"], w.W, w.reduce_idx, self.base.pd_par,
                                                self.base.ps_par, d.dpd_par, d.dps_par, dts, p.item_idx, **lay)
                d_dts_of[w.ws] = d_dts

            def sweep(store):
                p.k.compute_wave_step_tangent(pi, dpi, dpi, w.ws, w.W, p.S, *cst, col, h["node_child1"],
                                              h["node_child2"], p.topo[0], p.topo[3], dts, d_dts,
                                              dPibar_out=dpibar if store else None, has_leaf_term=not w.split, **kw)

            if sweeps is not None and one_call:
                p.k.compute_wave_step_tangent_selfloop(pi, dpi, w.ws, w.W, p.S, max(int(sweeps), 1), *cst, col,
                                                       h["node_child1"], h["node_child2"], p.topo[0], p.topo[3],
                                                       dts, d_dts, dPibar_out=dpibar, has_leaf_term=not w.split,
                                                       **kw)
            elif sweeps is not None:
                for k in range(max(int(sweeps), 1)):
                    sweep(store=k == max(int(sweeps), 1) - 1)
            else:
                prev = dpi.narrow(0, w.ws, w.W).clone()
                for _ in range(int(max_sweeps)):
                    sweep(store=False)
                    cur = dpi.narrow(0, w.ws, w.W)
                    if float((cur - prev).abs().max()) <= tol * max(1.0, float(cur.abs().max())):
                        break
                    prev = cur.clone()
                sweep(store=True)
        return dpi.index_select(0, p.roots), SimpleNamespace(dPi=dpi, dPibar=dpibar, d=d, d_dts=d_dts_of)


def _class_static(static, layout, rep):
    """A static namespace whose rows are the class rows of ``layout`` (tensors on the static's device)."""
    dev = static.rate_item_idx.device

    def conv(x):
        if isinstance(x, np.ndarray):
            return torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        if isinstance(x, dict):
            return {k: conv(v) for k, v in x.items()}
        if isinstance(x, list):
            return [conv(v) for v in x]
        return x

    item = static.rate_item_idx
    if int(item.numel()) > 1:
        item = item.index_select(0, torch.from_numpy(rep).to(dev))
    return SimpleNamespace(wave_layout=conv(layout), state_helpers=static.state_helpers, rate_item_idx=item,
                           itemwise=static.itemwise, statewise=static.statewise,
                           solver_options=static.solver_options, warm_E=None)


def _forward_classes(plan: SolvePlan):
    """(class plan, class_of_row, rep_of_class) of the rows' forward classes, kept on the plan."""
    fc = getattr(plan, "_hvp_forward_classes", None)
    if fc is None:
        st = plan.static
        layout, class_of, rep = synth.row_classes(st.wave_layout, st.rate_item_idx)
        dev = st.rate_item_idx.device
        fc = (SolvePlan(_class_static(st, layout, rep), kernels=plan.k), torch.from_numpy(class_of).to(dev),
              torch.from_numpy(rep).to(dev))
        plan._hvp_forward_classes = fc
    return fc


class _ClassSchedule:
    """The tangent forward and reverse of ``HvpPlan`` on class rows (see the module docstring).

    ``fplan`` / ``fsaved``: the forward classes and their saved rows;
    ``rplan``: the reverse classes (forward classes split by the point's
    active mask); ``cache``: per reverse-class wave, in reverse order,
    (wave, summed point adjoint of the members, split term, active flag);
    ``root_keys``: the reverse class of every family's root row (-1 if the
    root is inactive); ``fc_of_rc``: the forward class of each reverse class.
    """

    def __init__(self, plan: SolvePlan, saved, waves):
        if float(plan.so.pibar_side_threshold) != 0.0:
            raise ValueError("row classes need pibar_side_threshold == 0 (a side rule linear in the adjoint)")
        st = plan.static
        dev = saved["pi_wave"].device
        self.fplan, fc_of_row, frep = _forward_classes(plan)
        self.fsaved = dict(saved, pi_wave=saved["pi_wave"].index_select(0, frep),
                           pibar_wave=saved["pibar_wave"].index_select(0, frep),
                           pibar_row_max=saved["pibar_row_max"].index_select(0, frep))
        active = torch.zeros((plan.C,), dtype=torch.bool, device=dev)
        for w, _, _, mask in waves:
            active[w.ws: w.ws + w.W] = mask
        if bool(active.all()):  # no member dropped: the reverse classes are the forward classes
            rp = self.rplan = self.fplan
            rc_of_row, rrep = fc_of_row, frep
        else:
            layout, rc_of_row, rrep = synth.row_classes(st.wave_layout, st.rate_item_idx, active=active)
            rp = self.rplan = SolvePlan(_class_static(st, layout, rrep), kernels=plan.k)
            rc_of_row = torch.from_numpy(rc_of_row).to(dev)
            rrep = torch.from_numpy(rrep).to(dev)
        self.fc_of_rc = fc_of_row.index_select(0, rrep)
        self.Pi = saved["pi_wave"].index_select(0, rrep)
        self.Pibar = saved["pibar_wave"].index_select(0, rrep)
        self.prm = saved["pibar_row_max"].index_select(0, rrep)
        on = active.index_select(0, rrep)
        none = torch.full_like(rc_of_row, -1)
        V = torch.zeros_like(self.Pi)
        for w, v, _, mask in waves:  # members' adjoints, summed per class in a fixed order
            H.scatter_add_rows(V, v, torch.where(mask, rc_of_row[w.ws: w.ws + w.W], none[: w.W]))
        roots = plan.roots
        self.root_keys = torch.where(active.index_select(0, roots), rc_of_row.index_select(0, roots),
                                     none[: int(roots.numel())])
        c = rp._row_consts(saved["E"], saved["Ebar"], saved["E_s1"], saved["E_s2"], saved["log_pS"],
                           saved["log_pD"], saved["max_coupling"])
        self.cache = []
        for w in reversed(rp.waves):
            mask = on[w.ws: w.ws + w.W].contiguous()
            dts = rp._dts(w, self.Pi, self.Pibar, c, active=mask) if w.split else None
            self.cache.append((w, V[w.ws: w.ws + w.W], dts, mask))
        # every split row as one wave (the class layout is level ordered: the leaf level first, then
        # the split levels, contiguous), for the second-order terms that need no level order
        fwd = self.cache[::-1]
        # with no row pruned the reverse classes are the forward ones: the tangent forward reads
        # these split terms, and the reverse the forward's split-term tangents
        self.split_terms = ({w.ws: dts for w, _, dts, _ in fwd if w.split} if rp is self.fplan else None)
        self.leaf = [(w, v) for w, v, _, _ in fwd if not w.split]
        sw = [(w, dts) for w, _, dts, _ in fwd if w.split]
        self.split_all = None
        if sw:
            ws1 = sw[0][0].ws
            if any(a.ws + a.W != b_.ws for (a, _), (b_, _) in zip(sw, sw[1:])) or sw[-1][0].ws + sw[-1][0].W != rp.C:
                raise ValueError("the class layout's split waves are not contiguous")
            if any(w.leaf_term for w, _ in sw):
                raise ValueError("a split wave of the class layout carries the leaf term")
            dt = self.Pi.dtype
            lsp = torch.cat([w.lsp.reshape(-1).to(dt) if w.lsp is not None else
                             torch.zeros((int(w.sl.numel()),), dtype=dt, device=dev) for w, _ in sw])
            sl, sr = torch.cat([w.sl for w, _ in sw]), torch.cat([w.sr for w, _ in sw])
            red = torch.cat([w.reduce_idx + (w.ws - ws1) for w, _ in sw])
            self.split_all = SimpleNamespace(
                ws=ws1, W=rp.C - ws1, sl=sl, sr=sr, reduce_idx=red, lsp=lsp, v=V[ws1:],
                dts=torch.cat([dts for _, dts in sw]),
                meta={"start": ws1, "W": rp.C - ws1, "sl": sl, "sr": sr, "reduce_idx": red, "log_split_probs": lsp})


class _EGraph:
    """One E step at (E*, parameters) kept as an autograd graph: its transposed products."""

    def __init__(self, plan: SolvePlan, saved):
        self.p = plan
        S, G = plan.S, int(saved["E"].shape[0])
        item = lambda t: as_item_state(t, S, G)
        self.E = saved["E"].detach()
        self.params = [item(saved["log_pS"]), item(saved["log_pD"]), item(saved["log_pL"]),
                       item(saved["max_coupling"].squeeze(-1)), saved["col_log_probs"].contiguous()]
        self.E_var = self.E.clone().requires_grad_(True)
        with torch.enable_grad():
            self.out = plan.k.e_step_triton_autograd(self.E_var, *self.params, *plan.topo, use_col_weights=False)

    def _grad(self, outs, cots):
        with torch.enable_grad():
            (g,) = torch.autograd.grad(outs, self.E_var, grad_outputs=cots, retain_graph=True)
        return g

    def jt(self, w):
        """J_E^T w (the E-step map's transpose at E*)."""
        return self._grad(self.out[0], w.contiguous())

    def aux_t(self, g_s1, g_s2, g_ebar):
        """Transposed derivative of (E_s1, E_s2, Ebar) with respect to E."""
        return self._grad(self.out[1:], (g_s1, g_s2, g_ebar))

    def params_t(self, g_new, g_ebar):
        """Cotangents of (pS, pD, pL, mt, col) from those of (E_new, Ebar) at fixed E*."""
        xs = [x.detach().clone().requires_grad_(True) for x in self.params]
        with torch.enable_grad():
            En, _, _, Eb = self.p.k.e_step_triton_autograd(self.E, *xs, *self.p.topo, use_col_weights=False)
            gs = torch.autograd.grad((En, Eb), xs, grad_outputs=(g_new, g_ebar), allow_unused=True)
        return [torch.zeros_like(x) if g is None else g for g, x in zip(gs, xs)]


class HvpPlan:
    """H u of the summed loss at theta (uniform column weights), through the wrappers."""

    def __init__(self, plan: SolvePlan, theta, col_weights, saved, *, tangent_sweeps=None, row_classes=False,
                 graph=False, native_e_adjoint=None):
        if graph and plan.so.self_loop_solver != "neumann":
            raise ValueError("a captured HVP needs the Neumann self-loop solver (GMRES reads its residuals on the host)")
        self.p, self.sv = plan, saved
        self.graph, self._graph = bool(graph), None
        # the tangent E adjoint in one launch (kb_e_adjoint) for one float32 item row; else
        # BiCGSTAB over autograd E-step products
        self.native_e = (native_e_adjoint if native_e_adjoint is not None else
                         (saved["E"].dtype == torch.float32 and int(saved["E"].shape[0]) == 1
                          and int(saved["E"].numel()) == plan.S))
        self.theta, self.cw = theta, col_weights
        self.sweeps = int(plan.so.pi_iters if tangent_sweeps is None else tangent_sweeps)
        S = plan.S
        self.G = G = int(saved["E"].shape[0])
        # point cache: one backward with every wave's adjoint kept
        self.waves = []
        with torch.no_grad():
            seed = -root_softmax2(saved["pi_wave"].index_select(0, plan.roots))
            self.acc = plan.reverse_sweep(saved, seed, use_col=False, cache=self.waves)
        e_out = {}
        self.grad = plan.e_adjoint_and_vjp(theta, col_weights, saved, self.acc, use_col=False, out=e_out)
        self.wE = e_out["wE"]
        self.q = root_softmax2(saved["pi_wave"].index_select(0, plan.roots))
        self.cls = _ClassSchedule(plan, saved, self.waves) if row_classes else None
        self.tan = (TangentForward(plan, saved) if self.cls is None else
                    TangentForward(self.cls.fplan, self.cls.fsaved, split_terms=self.cls.split_terms))
        self.eg = _EGraph(plan, saved)
        a = self.acc
        base = self.eg.params_t(self.wE, a.Ebar)
        self.cot = SimpleNamespace(pS=_fold(a.pS, base[0], G, S), pD=_fold(a.pD, base[1], G, S), pL=base[2],
                                   mt=a.mt + base[3], col=a.col + base[4])
        # the parameter head: theta -> rates, and the first-order gradient kept differentiable
        st = plan.static
        self.th = theta.detach().clone().requires_grad_(True)
        cw = col_weights.detach().clone().requires_grad_(True)
        with torch.enable_grad():
            pS, pD, pL, mt, col = extract_parameters_weighted_cols(self.th, cw, plan.h, statewise=st.statewise,
                                                                   itemwise=st.itemwise, uniform_fast=True)
            self.rates = (as_item_param(pS, G, S), as_item_param(pD, G, S), as_item_state(pL, S, G),
                          as_item_state(mt, S, G), col)
            (self.g1,) = torch.autograd.grad(self._pair(self.cot), self.th, create_graph=True)

    def _pair(self, cot):
        r = self.rates
        return ((r[0] * cot.pS).sum() + (r[1] * cot.pD).sum() + (r[2] * cot.pL).sum() + (r[3] * cot.mt).sum()
                + (r[4] * cot.col).sum())

    def __call__(self, u_flat):
        u = u_flat.reshape(self.theta.shape).to(self.theta.dtype)
        with torch.no_grad():
            dcot = self._replay(u) if self.graph else self._tangent_cotangents(u)
        with torch.enable_grad():
            (hu,) = torch.autograd.grad((self.g1 * u).sum() + self._pair(dcot), self.th, retain_graph=True)
        if self.graph and self.native_e:  # read after the head is queued, so its host work overlaps the replay
            it, failed = (int(x) for x in self._fused().last_e_status.cpu())
            if failed:
                raise RuntimeError(f"E-adjoint BiCGSTAB solve failed after {it} iterations")
        return hu.reshape(-1)

    def _fused(self):
        from kbench.runtime import fused_solver

        return fused_solver(self.p.static)

    def _tangent_cotangents(self, u, *, check_solve=True):
        d, dacc = self._tangent_reverse(u)
        return self._e_side(d, dacc, check_solve=check_solve)

    def _replay(self, u):
        """The tangent forward, reverse and (with the native E adjoint) E side as one HIP graph:
        captured on the first call, after one eager call that creates every cached layout table
        and kernel attribute; replayed after (``__call__`` reads the E adjoint's status once)."""
        if self._graph is None:
            self._u_in = u.clone()
            self._tangent_cotangents(self._u_in)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                if self.native_e:
                    self._graph_out = self._tangent_cotangents(self._u_in, check_solve=False)
                else:
                    self._graph_out = self._tangent_reverse(self._u_in)
            self._graph = g
        self._u_in.copy_(u)
        self._graph.replay()
        if not self.native_e:
            return self._e_side(*self._graph_out)
        return self._graph_out  # the E adjoint's status is read by the caller

    def _class_reverse(self, d, dPi, dPibar, d_rhs, dacc, targets, cst_so, tan_d_dts):
        """The tangent reverse on the reverse classes, in two parts.

        The second-order terms (``compute_dts_tangent``, ``dts_backward_so``,
        ``wave_backward_so``) read the point adjoint v and the tangent rows, not the tangent
        adjoint, so they run first, each as one launch over all split rows (and the leaf
        level): the split terms' contributions go into the children's right-hand sides, the
        self-loop contraction into every row's own.  The level loop then carries only the
        first-order adjoint (Neumann series, split adjoint, Pibar VJP).  The right-hand side
        a level's solve reads is the same sum as in the level-by-level order.
        """
        k = self.cls
        p, sv, b = k.rplan, self.sv, self.tan.base
        S, G, h, so = p.S, self.G, p.h, p.so
        Pi, Pibar, prm, col = k.Pi, k.Pibar, k.prm, sv["col_log_probs"]
        c1, c2 = h["node_child1"], h["node_child2"]
        sa = k.split_all
        parts = [(w.ws, w.W, v, None, None, w.leaf_term) for w, v in k.leaf]
        if sa is not None:
            if k.split_terms is not None:  # the tangent forward's, on the same rows
                d_dts = torch.cat([tan_d_dts[w.ws] for w in p.waves if w.split])
            else:
                d_dts = p.k.compute_dts_tangent(Pi, Pibar, dPi, dPibar, sa.sl, sa.sr, c1, c2, sa.W, sa.reduce_idx,
                                                b.pd_par, b.ps_par, d.dpd_par, d.dps_par, sa.dts, p.item_idx,
                                                log_split_probs=sa.lsp, item_offset=sa.ws)
            p.k.dts_backward_so(
                Pi, dPi, Pibar, dPibar, sa.v, sa.ws, sa.meta, S, b.pd_par, b.ps_par, d.dpd_par, d.dps_par, b.mc,
                d.dMC, col, c1, c2, p.topo[0], p.topo[3], prm, p.item_idx, d_rhs, dacc.pD, dacc.pS, dacc.mt,
                dacc.col, use_col_weights=False, **p.levels)
            parts.append((sa.ws, sa.W, sa.v, sa.dts, d_dts, False))
        for ws, W, v, dts, d_dts, leaf_term in parts:
            seed, *so_aw = p.k.wave_backward_so(
                Pi, dPi, Pibar, dPibar, v, ws, W, S, prm, *cst_so, col, c1, c2, p.topo[0], p.topo[3], dts, d_dts,
                leaf_state_idx=p.leaf_idx, leaf_logp=b.leaf, dleaf_logp=d.dleaf, item_idx=p.item_idx,
                has_leaf_term=leaf_term, use_col_weights=False, d_rhs=d_rhs)
            d_rhs.narrow(0, ws, W).copy_(seed)
            p._fold_buckets(so_aw, targets, SimpleNamespace(ws=ws, W=W), G)
        for w, _, dts, mask in k.cache:
            dv, *lin_aw = p.k.wave_backward_uniform_fused(
                Pi, Pibar, w.ws, w.W, S, dts, d_rhs.narrow(0, w.ws, w.W), b.mc, b.dl, b.ebar, b.e, b.sl1, b.sl2, col,
                c1, c2, None, neumann_terms=int(so.neumann_terms), leaf_state_idx=p.leaf_idx, leaf_logp=b.leaf,
                has_leaf_term=w.leaf_term, active_mask=mask, node_parent=p.topo[0], max_ancestor_depth=p.topo[3],
                pibar_row_max=prm, item_idx=p.item_idx, item_indexed_consts=True, grad_col_log_probs=dacc.col,
                use_col_weights=False, self_loop_solver=so.self_loop_solver, **p.levels)
            p._fold_buckets(lin_aw, targets, w, G)
            if w.split:
                self._split_adjoint(p, w, dv, mask, d_rhs, dacc, Pi, Pibar, prm, col)
        return dacc

    def _split_adjoint(self, p, w, dv, mask, d_rhs, dacc, Pi, Pibar, prm, col):
        """The split wave's cross adjoint and Pibar VJP of the tangent adjoint dv into the children."""
        b, h, so, S = self.tan.base, p.h, p.so, p.S
        lsp = w.lsp if w.lsp is not None else w.sl.new_zeros((int(w.sl.numel()),), dtype=Pi.dtype)
        ud, A, side_on, _, _ = p.k.dts_cross_backward_accum_fused(
            Pi, Pibar, dv, w.ws, w.sl, w.sr, w.reduce_idx, lsp, b.pd_par, b.ps_par, h["node_child1"],
            h["node_child2"], d_rhs, S, active_mask=mask, merge_s_term=True, grad_log_pD=dacc.pD,
            grad_log_pS=dacc.pS, grad_mt=dacc.mt, accum_param_reductions=True, accum_mt_reduction=True,
            output_pibar_ud=True, output_pibar_side_active=True,
            pibar_side_threshold=so.pibar_side_threshold, mt_squeezed=b.mc, pibar_row_max=prm,
            grad_mt_two_stage=bool(dacc.mt.ndim == 2 and int(dacc.mt.shape[0]) == 1),
            grad_mt_two_stage_tile_splits=128, skip_inactive_pibar_output_zero=True, item_idx=p.item_idx)
        p.k.uniform_cross_pibar_vjp_tree_from_ud_fused(
            Pi, col, ud, A, w.sl, w.sr, d_rhs, S, active_mask=mask, reduce_idx=w.reduce_idx,
            pibar_row_max=prm, skip_zero_sides=True, side_active=side_on, grad_col_log_probs=dacc.col,
            use_col_weights=False, side_active_threshold=so.pibar_side_threshold, **p.levels)

    def _tangent_reverse(self, u):
        """(constant tangents, tangent cotangents accumulated over the waves) along u."""
        sv, a = self.sv, self.acc
        S, G = self.p.S, self.G
        t_root, tf = self.tan.run(self.theta, u, sweeps=self.sweeps)
        d = tf.d
        col = sv["col_log_probs"]
        b = self.tan.base
        # tangent of the root seed -softmax2(root): -ln2 q (t - <q, t>)
        q = self.q
        seed = -LN2 * q * (t_root - (q * t_root).sum(dim=-1, keepdim=True))
        k = self.cls
        if k is None:
            p, waves = self.p, self.waves
            Pi, Pibar, prm = sv["pi_wave"], sv["pibar_wave"], sv["pibar_row_max"]
            dPi, dPibar = tf.dPi, tf.dPibar
            d_rhs = torch.zeros((p.C, S), dtype=Pi.dtype, device=Pi.device)
            d_rhs.index_copy_(0, p.roots, seed)
        else:
            p, waves = k.rplan, k.cache
            Pi, Pibar, prm = k.Pi, k.Pibar, k.prm
            dPi, dPibar = tf.dPi.index_select(0, k.fc_of_rc), tf.dPibar.index_select(0, k.fc_of_rc)
            d_rhs = torch.zeros((p.C, S), dtype=Pi.dtype, device=Pi.device)
            H.scatter_add_rows(d_rhs, seed, k.root_keys, static=(k.root_keys,))
        h = p.h
        dacc = SimpleNamespace(pD=torch.zeros_like(a.pD), pS=torch.zeros_like(a.pS), mt=torch.zeros_like(a.mt),
                               col=torch.zeros_like(a.col), E=torch.zeros_like(a.E), Ebar=torch.zeros_like(a.E),
                               Es1=torch.zeros_like(a.E), Es2=torch.zeros_like(a.E))
        targets = ((dacc.pD, (0,)), (dacc.pS, (3,)), (dacc.E, (0, 2)), (dacc.Ebar, (1,)), (dacc.Es1, (5,)),
                   (dacc.Es2, (4,)), (dacc.mt, (2,)))
        cst_so = (b.mc,) + self.tan.interleaved(d)[2:]  # the contraction takes mt without its tangent
        if k is not None:
            return d, self._class_reverse(d, dPi, dPibar, d_rhs, dacc, targets, cst_so, tf.d_dts)
        so = p.so
        for w, v, dts, mask in waves:
            d_dts = None
            if w.split:
                d_dts = p.k.compute_dts_tangent(Pi, Pibar, dPi, dPibar, w.sl, w.sr, h["node_child1"],
                                                h["node_child2"], w.W, w.reduce_idx, b.pd_par, b.ps_par, d.dpd_par,
                                                d.dps_par, dts, p.item_idx, log_split_probs=w.lsp, item_offset=w.ws)
            seed, *so_aw = p.k.wave_backward_so(
                Pi, dPi, Pibar, dPibar, v, w.ws, w.W, S, prm, *cst_so, col, h["node_child1"], h["node_child2"],
                p.topo[0], p.topo[3], dts, d_dts, leaf_state_idx=p.leaf_idx, leaf_logp=b.leaf, dleaf_logp=d.dleaf,
                item_idx=p.item_idx, has_leaf_term=w.leaf_term, use_col_weights=False, d_rhs=d_rhs)
            dv, *lin_aw = p.k.wave_backward_uniform_fused(
                Pi, Pibar, w.ws, w.W, S, dts, seed, b.mc, b.dl, b.ebar, b.e, b.sl1, b.sl2, col, h["node_child1"],
                h["node_child2"], None, neumann_terms=int(so.neumann_terms), leaf_state_idx=p.leaf_idx,
                leaf_logp=b.leaf, has_leaf_term=w.leaf_term, active_mask=mask, node_parent=p.topo[0],
                max_ancestor_depth=p.topo[3], pibar_row_max=prm, item_idx=p.item_idx, item_indexed_consts=True,
                grad_col_log_probs=dacc.col, use_col_weights=False, self_loop_solver=so.self_loop_solver,
                **p.levels)
            p._fold_buckets(list(zip(so_aw, lin_aw)), targets, w, G)
            if w.split:
                self._split_adjoint(p, w, dv, mask, d_rhs, dacc, Pi, Pibar, prm, col)
                p.k.dts_backward_so(
                    Pi, dPi, Pibar, dPibar, v, w.ws, w.meta, S, b.pd_par, b.ps_par, d.dpd_par, d.dps_par, b.mc,
                    d.dMC, col, h["node_child1"], h["node_child2"], p.topo[0], p.topo[3], prm, p.item_idx, d_rhs,
                    dacc.pD, dacc.pS, dacc.mt, dacc.col, use_col_weights=False, **p.levels)
        return d, dacc

    def _e_side(self, d, dacc, *, check_solve=True):
        """Tangent E adjoint and the tangent parameter cotangents."""
        p, sv, a, eg = self.p, self.sv, self.acc, self.eg
        S, G = p.S, self.G
        E = eg.E
        raw = d.raw
        item = lambda t: as_item_state(t, S, G)
        point = (E, E, sv["E_s1"], sv["E_s2"], sv["Ebar"], *eg.params[:3], eg.params[4], *p.topo)
        along = (item(raw["dE"]), item(raw["dE"]), item(raw["dE_s1"]), item(raw["dE_s2"]), item(raw["dEbar"]),
                 item(raw["dlog_pS"]), item(raw["dlog_pD"]), item(raw["dlog_pL"]), None)
        zero = torch.zeros_like(E)
        so2 = lambda g_new, g_s1, g_s2, g_ebar: p.k.e_step_backward_so(*point, g_new, g_s1, g_s2, g_ebar, *along,
                                                                       use_col_weights=False)
        # the loss's log2(1 - mean 2^E) term: its E gradient and that gradient's tangent
        dE = along[0]
        e2 = torch.exp2(E)
        survive = (1.0 - e2.mean(dim=-1, keepdim=True)).clamp_min(torch.finfo(E.dtype).tiny)
        per_row = 1.0 if G == p.n_fam else float(p.n_fam)
        d_survive = -LN2 * (e2 * dE).mean(dim=-1, keepdim=True)
        d_norm_grad = per_row * (e2 * d_survive / (S * survive * survive) - LN2 * e2 * dE / (S * survive))
        so_p = so2(self.wE, zero, zero, a.Ebar)
        extra = so2(zero, a.Es1, a.Es2, a.Ebar)[0] + d_norm_grad + so2(self.wE, zero, zero, zero)[0]
        if self.native_e:
            # q = dacc.E + (Es1, Es2, Ebar cotangents pulled back to E) + extra, solved and pulled back
            # to the rates by the backward epilogue's float64 BiCGSTAB in one launch
            z = torch.zeros((S,), dtype=torch.float64, device=E.device)
            acc8 = torch.stack([z, z, dacc.E.reshape(S).double(), dacc.Ebar.reshape(S).double(),
                                dacc.Es1.reshape(S).double(), dacc.Es2.reshape(S).double(), z, z])
            _, gs = self._fused().e_adjoint(self.sv, acc8, q_extra=extra.reshape(S), check_solve=check_solve)
            gs = gs.to(E.dtype)
            lin = [gs[0].view_as(E), gs[1].view_as(E), gs[2].view_as(E), gs[3].view_as(E), gs[4]]
        else:
            rhs = dacc.E + eg.aux_t(dacc.Es1, dacc.Es2, dacc.Ebar) + extra
            dwE = bicgstab(lambda x: x - eg.jt(x.view_as(E)).reshape(-1), rhs.reshape(-1),
                           max_iter=int(p.so.bicgstab_max_iter), tol=float(p.so.bicgstab_tol),
                           breakdown_tol=float(p.so.bicgstab_breakdown_tol)).view_as(E)
            lin = eg.params_t(dwE, dacc.Ebar)
        return SimpleNamespace(pS=_fold(dacc.pS, lin[0] + so_p[1], G, S), pD=_fold(dacc.pD, lin[1] + so_p[2], G, S),
                               pL=lin[2] + so_p[3], mt=dacc.mt + lin[3] + so_p[4], col=dacc.col + lin[4] + so_p[5])


def ggn_hvp(plan: SolvePlan, theta, col_weights, saved, *, tol=None, max_sweeps=200, neumann_terms=None,
            use_pruning=None, bicgstab_tol=None):
    """v -> J^T B J v, the Gauss-Newton product with B_f = ln2 (diag q_f - q_f q_f^T) per family.

    J = d(root rows)/d(theta) by ``TangentForward`` (sweeping each wave to convergence);
    J^T by the backward's reverse sweep from a root-row cotangent, without the loss's
    normaliser term.  ``neumann_terms`` / ``use_pruning`` / ``bicgstab_tol`` override
    the solver options of that reverse sweep and its E adjoint.
    """
    tan = TangentForward(plan, saved)
    q = root_softmax2(saved["pi_wave"].index_select(0, plan.roots))

    def hvp(v_flat):
        v = v_flat.reshape(theta.shape).to(theta.dtype)
        with torch.no_grad():
            t, _ = tan.run(theta, v, tol=tol, max_sweeps=max_sweeps)
            cot = LN2 * q * (t - (q * t).sum(dim=-1, keepdim=True))
            acc = plan.reverse_sweep(saved, cot, use_col=False, neumann_terms=neumann_terms, use_pruning=use_pruning)
        g, _ = plan.e_adjoint_and_vjp(theta, col_weights, saved, acc, use_col=False, with_norm=False,
                                      bicgstab_tol=bicgstab_tol)
        return g.reshape(-1)

    return hvp


# ---------------------------------------------------------------------------- entry points
def _require_uniform_columns(col_weights):
    from kbench.percall.solve import uniform_columns

    if not uniform_columns(col_weights):
        raise ValueError("the Hessian-vector products take uniform column weights (use_col_weights=False), "
                         "as the reference's newton path does")


def make_exact_hvp(static, theta, col_weights, sv, *, cache=None, tangent_self_iters=None, row_classes=True,
                   graph=None):
    """``hvp(u_flat) -> H u``: the exact Hessian of the summed loss at theta, analytically
    (reference newton/hvp_exact.py:66-383, same arguments).

    ``sv`` holds the forward intermediates at theta (``kbench.runtime.run_forward`` or the
    per-call ``kbench.percall.run_forward``; the same names on both).  ``cache`` is an
    earlier return value of this function at the same point, whose point cache (one
    backward keeping every adjoint, the E adjoint, the class schedule) is reused.
    ``tangent_self_iters``, the tangent forward's sweeps per wave, resolves as in the
    reference: this argument, then ``NEWTON_TANGENT_SELF_ITERS``, then
    ``solver_options.pi_iters``.  ``row_classes`` runs the tangent pass on one row per
    class of identical rows (same result up to the order of sums); ``graph`` replays that
    pass as one HIP graph (default: with the Neumann self-loop solver, which reads
    nothing back on the host).
    """
    import os

    if cache is not None:
        if not isinstance(cache, HvpPlan):
            raise TypeError("cache must be a value returned by make_exact_hvp")
        return cache
    _require_uniform_columns(col_weights)
    from kbench.percall.solve import plan_of

    plan = plan_of(static)
    if tangent_self_iters is None:
        env = os.environ.get("NEWTON_TANGENT_SELF_ITERS")
        tangent_self_iters = int(env) if env else int(plan.so.pi_iters)
    if graph is None:
        graph = plan.so.self_loop_solver == "neumann" and theta.device.type == "cuda"
    return HvpPlan(plan, theta, col_weights, sv, tangent_sweeps=int(tangent_self_iters), row_classes=bool(row_classes),
                   graph=bool(graph))


def make_ggn_hvp(static, theta, col_weights, sv, *, self_tol=None, self_max_iter=200, vjp_neumann_terms=None,
                 vjp_use_pruning=None, vjp_bicgstab_tol=None):
    """``hvp(v_flat) -> M v``: the Gauss-Newton (Fisher) product at theta, positive semi-definite
    (reference newton/ggn.py:280-303, same arguments).

    The tangent forward sweeps each wave until max|change| <= ``self_tol`` * max(1, max|dPi|)
    (default 1e-6 for float32 rows, 1e-12 for float64), at most ``self_max_iter`` sweeps; the ``vjp_*``
    arguments override the solver options of the reverse sweep and its E adjoint.
    """
    _require_uniform_columns(col_weights)
    from kbench.percall.solve import plan_of

    return ggn_hvp(plan_of(static), theta, col_weights, sv, tol=self_tol, max_sweeps=int(self_max_iter),
                   neumann_terms=vjp_neumann_terms, use_pruning=vjp_use_pruning, bicgstab_tol=vjp_bicgstab_tol)


__all__ = ["TangentForward", "HvpPlan", "ggn_hvp", "make_exact_hvp", "make_ggn_hvp"]
