"""Forward + backward solve through the per-call wrappers, in the reference glue's call sequence.

``SolvePlan(static)`` compiles the static layout once: every wave becomes a
``_Wave`` record holding its row range and its split layout already on the
device, in the form the wrappers take.  ``forward`` / ``backward`` then walk
those records and call the wrappers.

Wrapper calls, per pass (reference lines are those of the frozen glue these
calls stand in for):

forward (kbench/core/inference/solver.py:16-96, forward.py:8-117)
  1. rate parameters (extract_parameters_uniform, or _weighted_cols when the
     column weights differ: one host read), ``e_fixed_point_triton`` from
     ``e_init``;
  2. per wave in order: ``compute_dts_forward`` (split waves), then sweeps
     1 .. pi_iters-1 alternating between the ``pi`` and ``pibar`` buffers
     (odd sweeps write ``pi``); sweep 0 is the leaf initialisation on leaf
     waves (into ``pibar``) and is skipped on split waves, whose sweep 1
     reads the split term (``input_ws=0``); the last sweep stores Pibar and
     the row maxima;
  3. loss: sum over families of -(LSE2(root row) - log2 S - log2(1 - mean 2^E)).

backward (kbench/api/_implicit_grad.py:97-475)
  1. seed the root rows' adjoint with -softmax2(root row);
  2. per wave in reverse: ``active_mask_from_rhs_absmax_fused``,
     ``compute_dts_forward`` with the inactive parents masked (split waves),
     ``wave_backward_uniform_fused``, the bucket sums into the parameter
     cotangents, then ``dts_cross_backward_accum_fused`` and
     ``uniform_cross_pibar_vjp_tree_from_ud_fused`` (split waves);
  3. E adjoint: BiCGSTAB on (I - J_E^T) w = q_E with ``e_step_triton_autograd``
     (failure raises RuntimeError), then the theta / column VJP through the
     parameter extraction and one E step.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from kbench.api.solver_options import SolverOptions
from kbench.core.parameters.extract_parameters import (as_item_param, as_item_state, extract_parameters_uniform,
                                                       extract_parameters_weighted_cols)

from kbench.core.kernels import _hip as H

from . import kernels as K
from .krylov import bicgstab

SAVED = ("E", "E_s1", "E_s2", "Ebar", "root_rows", "pi_wave", "pibar_wave", "pibar_row_max", "log_pS", "log_pD",
         "log_pL", "max_coupling", "col_log_probs")
LN2 = math.log(2.0)
_SPLIT_KW = ("n_eq1", "eq1_reduce_idx", "ge2_ptr", "ge2_parent_ids", "ge2_max_fanout")


@dataclass
class _Wave:
    ws: int
    W: int
    sl: torch.Tensor | None = None
    sr: torch.Tensor | None = None
    reduce_idx: torch.Tensor | None = None
    lsp: torch.Tensor | None = None      # log_split_probs as stored (None: absent)
    extra: dict | None = None            # the optional eq1 / ge2 layout fields
    leaf_term: bool = True               # phase 1 (leaf) rows add the leaf observation term
    meta: dict | None = None             # the wave's layout dict (dts_backward_so takes it whole)

    @property
    def split(self) -> bool:
        return self.sl is not None


def uniform_columns(col_weights: torch.Tensor) -> bool:
    """Every column weight equal (one host read)."""
    w = col_weights.detach().reshape(-1)
    return bool((w == w[0]).all().item())


def root_softmax2(root_rows: torch.Tensor) -> torch.Tensor:
    """2^(x - LSE2(x)) per row; 0 where x is -inf and for rows that are all -inf."""
    lse = torch.logsumexp(root_rows * LN2, dim=-1, keepdim=True) / LN2
    live = torch.isfinite(root_rows) & torch.isfinite(lse)
    return torch.where(live, torch.exp2(torch.where(live, root_rows - lse, torch.zeros_like(root_rows))),
                       torch.zeros_like(root_rows))


def family_nll(root_rows: torch.Tensor, E: torch.Tensor) -> torch.Tensor:
    """Summed -(LSE2(root) - log2 S - log2(1 - mean_s 2^E)) over the families."""
    S = int(root_rows.shape[-1])
    lse = torch.logsumexp(root_rows * LN2, dim=-1) / LN2
    survive = (1.0 - torch.exp2(E).mean(dim=-1)).clamp_min(torch.finfo(E.dtype).tiny)
    return (math.log2(S) + torch.log2(survive) - lse).sum()


class SolvePlan:
    """One static problem compiled for the per-call path (see the module docstring)."""

    def __init__(self, static, *, kernels=None):
        self.k = kernels if kernels is not None else K.real()
        self.static = static
        so = static.solver_options
        self.so = so if isinstance(so, SolverOptions) else SolverOptions(**dict(so))
        self.so.validate()
        self.h = h = static.state_helpers
        wl = static.wave_layout
        self.S = int(h["S"])
        self.C = int(wl["leaf_state_index"].numel())
        self.roots = wl["root_row_ids"]
        self.n_fam = int(self.roots.numel())
        self.item_idx = static.rate_item_idx
        self.leaf_idx = wl["leaf_state_index"]
        self.G = self.n_fam if static.itemwise else 1
        self.topo = (h["node_parent"], h["node_child1"], h["node_child2"], int(h["max_ancestor_depth"]))
        self.levels = {k: h[k] for k in ("compact_level_ptr", "compact_level_parents", "compact_level_child1",
                                         "compact_level_child2")}
        self.waves = []
        for m in wl["wave_metas"]:
            w = _Wave(int(m["start"]), int(m["W"]))
            if "sl" in m:
                w.sl, w.sr, w.reduce_idx = m["sl"], m["sr"], m["reduce_idx"]
                w.lsp = m.get("log_split_probs")
                w.extra = {k: m.get(k) for k in _SPLIT_KW}
                w.meta = m
            w.leaf_term = int(m.get("phase", 2 if w.split else 1)) == 1
            self.waves.append(w)

    # ------------------------------------------------------------------ shared
    def _parameters(self, theta, col_weights, weighted=None):
        """(pS, pD, pL, mt, col, weighted) of theta, as the forward extracts them (``weighted``, when
        given, is the caller's reading of the column weights: no host read here)."""
        if weighted is None:
            weighted = not uniform_columns(col_weights)
        st = self.static
        if weighted:
            pS, pD, pL, mt, col = extract_parameters_weighted_cols(
                theta.detach(), col_weights.detach(), self.h, statewise=st.statewise, itemwise=st.itemwise)
        else:
            urm = self.h["unnorm_row_max"].to(device=theta.device, dtype=theta.dtype)
            pS, pD, pL, mt = extract_parameters_uniform(theta.detach(), urm, statewise=st.statewise,
                                                        itemwise=st.itemwise)
            col = theta.new_full((self.S,), -math.log2(self.S))
        return pS, pD, pL, mt, col, weighted

    def _row_consts(self, E, Ebar, Es1, Es2, pS, pD, mt):
        """The [G, S] constant rows of the sweep and its adjoint (forward.py:37-58)."""
        S, G = self.S, int(E.shape[0])
        item = lambda t: as_item_state(t, S, G)
        E_i, pS_i = item(E), item(pS)
        return SimpleNamespace(
            mt=item(mt.squeeze(-1)), DL=1.0 + item(pD) + E_i, Ebar=item(Ebar), E=E_i,
            SL1=pS_i + item(Es2), SL2=pS_i + item(Es1), leaf=pS_i,
            pD_par=as_item_param(pD, G, S), pS_par=as_item_param(pS, G, S))

    def _dts(self, w, Pi, Pibar, c, *, active=None):
        return self.k.compute_dts_forward(
            Pi, Pibar, w.sl, w.sr, self.h["node_child1"], self.h["node_child2"], w.W, w.reduce_idx, c.pD_par,
            c.pS_par, item_idx=self.item_idx, log_split_probs=w.lsp, active_parent_rows=active, item_offset=w.ws,
            **w.extra)

    # ------------------------------------------------------------------ forward
    def forward(self, theta, col_weights, *, pi_iters=None):
        """theta -> (loss, saved) with the saved tensors named as the reference's run_forward returns them."""
        with torch.no_grad():
            return self._forward(theta, col_weights, int(self.so.pi_iters if pi_iters is None else pi_iters))

    def _forward(self, theta, col_weights, P, weighted=None):
        if P < 2 or P % 2:
            raise ValueError("pi_iters must be an even integer at least 2")
        so, S, C, G = self.so, self.S, self.C, self.G
        pS, pD, pL, mt, col, weighted = self._parameters(theta, col_weights, weighted)
        E0 = theta.new_full((G, S), float(so.e_init))
        E, Es1, Es2, Ebar = self.k.e_fixed_point_triton(
            E0, log_pS=pS, log_pD=pD, log_pL=pL, max_coupling=mt, col_log_probs=col, use_col_weights=weighted,
            node_parent=self.topo[0], node_child1=self.topo[1], node_child2=self.topo[2],
            max_ancestor_depth=self.topo[3], max_iter=so.e_max_iter, tol=so.e_tol)
        c = self._row_consts(E, Ebar, Es1, Es2, pS, pD, mt)
        bufs = {"pi": torch.empty((C, S), dtype=theta.dtype, device=theta.device),
                "pibar": torch.empty((C, S), dtype=theta.dtype, device=theta.device)}
        row_max = torch.empty((C,), dtype=theta.dtype, device=theta.device)
        h = self.h
        consts = (c.mt, c.DL, c.Ebar, c.E, c.SL1, c.SL2, col)
        for w in self.waves:
            dts = self._dts(w, bufs["pi"], bufs["pibar"], c) if w.split else None
            if not w.split:
                self.k.compute_leaf_initial_wave_step(
                    bufs["pibar"], w.ws, w.W, S, *consts, h["node_child1"], h["node_child2"],
                    h["node_subtree_start"], h["node_subtree_end"], self.leaf_idx, c.leaf, item_idx=self.item_idx,
                    use_col_weights=weighted)
            for k in range(1, P):
                dst = "pi" if k % 2 else "pibar"
                from_dts = w.split and k == 1
                src = dts if from_dts else bufs["pibar" if k % 2 else "pi"]
                self.k.compute_wave_step(
                    src, bufs[dst], bufs["pibar"], w.ws, w.W, S, *consts, h["node_child1"], h["node_child2"],
                    self.topo[0], self.topo[3], dts, leaf_state_idx=self.leaf_idx, leaf_logp=c.leaf,
                    item_idx=self.item_idx, pibar_row_max=row_max, store_final_pibar=k == P - 1,
                    has_leaf_term=not w.split, input_ws=0 if from_dts else None, use_col_weights=weighted)
        pi, pibar = bufs["pi"], bufs["pibar"]
        root_rows = pi.index_select(0, self.roots)
        loss = family_nll(root_rows, E)
        saved = dict(zip(SAVED, (E, Es1, Es2, Ebar, root_rows, pi, pibar, row_max, pS, pD, pL, mt, col)))
        return loss, saved

    # ------------------------------------------------------------------ backward
    def backward(self, theta, col_weights, saved):
        """(saved forward tensors) -> (grad_theta, grad_col)."""
        with torch.no_grad():
            use_col = not uniform_columns(col_weights)
            root_pi = saved["pi_wave"].index_select(0, self.roots)
            acc = self.reverse_sweep(saved, -root_softmax2(root_pi), use_col=use_col)
        return self.e_adjoint_and_vjp(theta, col_weights, saved, acc, use_col=use_col)

    def reverse_sweep(self, saved, seed, *, use_col, neumann_terms=None, use_pruning=None, cache=None):
        """Adjoint over the waves in reverse from the root-row seed -> the parameter cotangents.

        With ``cache`` (a list), every wave appends (wave, adjoint v with inactive rows zeroed,
        split term, active mask): what the exact HVP reuses at a fixed point.
        """
        so, S, C = self.so, self.S, self.C
        nt = int(so.neumann_terms if neumann_terms is None else neumann_terms)
        prune = bool(so.use_adjoint_pruning if use_pruning is None else use_pruning)
        thr, side_thr = float(so.adjoint_pruning_threshold), float(so.pibar_side_threshold)
        Pi, Pibar, rmax = saved["pi_wave"], saved["pibar_wave"], saved["pibar_row_max"]
        col = saved["col_log_probs"]
        c = self._row_consts(saved["E"], saved["Ebar"], saved["E_s1"], saved["E_s2"], saved["log_pS"],
                             saved["log_pD"], saved["max_coupling"])
        G = int(saved["E"].shape[0])
        rhs = torch.zeros((C, S), dtype=Pi.dtype, device=Pi.device)
        rhs.index_copy_(0, self.roots, seed.to(Pi.dtype))
        acc = SimpleNamespace(
            pD=torch.zeros_like(c.pD_par), pS=torch.zeros_like(c.pS_par), mt=torch.zeros_like(c.mt),
            col=torch.zeros((S,), dtype=Pi.dtype, device=Pi.device),
            E=torch.zeros_like(saved["E"]), Ebar=torch.zeros_like(saved["E"]), Es1=torch.zeros_like(saved["E"]),
            Es2=torch.zeros_like(saved["E"]))
        # bucket k of the adjoint goes to these cotangents (_implicit_grad.py:289-296)
        # (aw = [aw0, aw1, aw2, aw345, aw3, aw4])
        targets = ((acc.pD, (0,)), (acc.pS, (3,)), (acc.E, (0, 2)), (acc.Ebar, (1,)), (acc.Es1, (5,)),
                   (acc.Es2, (4,)), (acc.mt, (2,)))
        h = self.h
        for w in reversed(self.waves):
            rows = rhs.narrow(0, w.ws, w.W)
            active = self.k.active_mask_from_rhs_absmax_fused(rows, thr, use_pruning=prune).contiguous()
            dts = self._dts(w, Pi, Pibar, c, active=active) if w.split else None
            v, *aw = self.k.wave_backward_uniform_fused(
                Pi, Pibar, w.ws, w.W, S, dts, rows, c.mt, c.DL, c.Ebar, c.E, c.SL1, c.SL2, col,
                h["node_child1"], h["node_child2"], None, neumann_terms=nt, leaf_state_idx=self.leaf_idx,
                leaf_logp=c.leaf, has_leaf_term=w.leaf_term, active_mask=active, node_parent=self.topo[0],
                max_ancestor_depth=self.topo[3], pibar_row_max=rmax, item_idx=self.item_idx,
                item_indexed_consts=True, grad_col_log_probs=acc.col, use_col_weights=use_col,
                self_loop_solver=so.self_loop_solver, **self.levels)
            self._fold_buckets(aw, targets, w, G)
            if cache is not None:
                on = active.reshape(w.W, -1).any(dim=1, keepdim=True)
                cache.append((w, torch.where(on, v, torch.zeros_like(v)), dts, active))
            if w.split:
                lsp = w.lsp if w.lsp is not None else w.sl.new_zeros((int(w.sl.numel()),), dtype=Pi.dtype)
                ud, A, side_on, _, _ = self.k.dts_cross_backward_accum_fused(
                    Pi, Pibar, v, w.ws, w.sl, w.sr, w.reduce_idx, lsp, c.pD_par, c.pS_par, h["node_child1"],
                    h["node_child2"], rhs, S, active_mask=active, merge_s_term=True, grad_log_pD=acc.pD,
                    grad_log_pS=acc.pS, grad_mt=acc.mt, accum_param_reductions=True, accum_mt_reduction=True,
                    output_pibar_ud=True, output_pibar_side_active=True, pibar_side_threshold=side_thr,
                    mt_squeezed=c.mt, pibar_row_max=rmax,
                    grad_mt_two_stage=bool(acc.mt.ndim == 2 and int(acc.mt.shape[0]) == 1),
                    grad_mt_two_stage_tile_splits=128, skip_inactive_pibar_output_zero=True, item_idx=self.item_idx)
                self.k.uniform_cross_pibar_vjp_tree_from_ud_fused(
                    Pi, col, ud, A, w.sl, w.sr, rhs, S, active_mask=active, reduce_idx=w.reduce_idx,
                    pibar_row_max=rmax, skip_zero_sides=True, side_active=side_on, grad_col_log_probs=acc.col,
                    use_col_weights=use_col, side_active_threshold=side_thr, **self.levels)
        return acc

    def _fold_buckets(self, aw, targets, w, G):
        """Add the wave's per-element contributions (aw0, aw1, aw2, aw345, aw3, aw4) into the cotangents.

        An entry of ``aw`` may be a pair of tensors whose sum is the contribution.
        """
        if G == 1:
            # every target's column sums added in one launch; [G, 1] targets (one value per
            # item row) and targets of another dtype go through a state row first
            S = int((aw[0][0] if isinstance(aw[0], (tuple, list)) else aw[0]).shape[1])
            blocks, later = [], []
            for acc, ks in targets:
                add = tuple(x for k in ks for x in (aw[k] if isinstance(aw[k], (tuple, list)) else (aw[k],)))
                if acc.numel() == S and acc.is_contiguous() and acc.dtype == add[0].dtype:
                    blocks.append((acc.view(-1), add))
                else:
                    tmp = torch.zeros((S,), dtype=add[0].dtype, device=add[0].device)
                    blocks.append((tmp, add))
                    later.append((acc, tmp))
            H.rows_sum_accum(blocks)
            for acc, s in later:
                if acc.ndim == 2 and int(acc.shape[1]) == 1:
                    acc[0, 0] += s.sum()
                else:
                    acc.view(-1, acc.shape[-1])[0] += s.to(acc.dtype)
            return
        aw = [x[0] + x[1] if isinstance(x, (tuple, list)) else x for x in aw]
        items = self.item_idx[w.ws: w.ws + w.W]
        for acc, ks in targets:
            contrib = aw[ks[0]] if len(ks) == 1 else aw[ks[0]] + aw[ks[1]]
            if acc.ndim == 2 and int(acc.shape[1]) == 1:
                acc[:, 0].index_add_(0, items, contrib.sum(dim=1))
            elif acc.ndim == 1:
                acc.index_add_(0, items, contrib.sum(dim=1))
            else:
                acc.index_add_(0, items, contrib)

    def e_adjoint_and_vjp(self, theta, col_weights, saved, acc, *, use_col, with_norm=True, bicgstab_tol=None,
                          out=None):
        """E adjoint by BiCGSTAB on (I - J_E^T) w = q_E, then d/d(theta, col_weights).

        ``with_norm`` includes the loss's log2(1 - mean 2^E) term in q_E (off for a
        root-score cotangent); ``out`` (a dict) receives q_E and the E adjoint.
        """
        so = self.so
        E = saved["E"].detach()
        prm = tuple(saved[k] for k in ("log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs"))
        E_var = E.clone().requires_grad_(True)
        with torch.enable_grad():
            E_new, Es1_n, Es2_n, Ebar_n = self.k.e_step_triton_autograd(E_var, *prm, *self.topo,
                                                                        use_col_weights=use_col)
            # d/dE of everything the accumulated cotangents multiply, besides E itself
            head = (Es1_n * acc.Es1).sum() + (Es2_n * acc.Es2).sum() + (Ebar_n * acc.Ebar).sum()
            if with_norm:
                survive = (1.0 - torch.exp2(E_var).mean(dim=-1)).clamp_min(torch.finfo(E.dtype).tiny)
                per_row = 1.0 if int(E.shape[0]) == self.n_fam else float(self.n_fam)
                head = head + per_row * torch.log2(survive).sum()
            (aux,) = torch.autograd.grad(head, E_var, retain_graph=True)
        q = (acc.E + aux).reshape(-1)

        def op(x):  # (I - J_E^T) x
            with torch.enable_grad():
                (jt,) = torch.autograd.grad(E_new, E_var, grad_outputs=x.view_as(E).contiguous(), retain_graph=True)
            return x - jt.reshape(-1)

        wE = bicgstab(op, q, max_iter=int(so.bicgstab_max_iter),
                      tol=float(so.bicgstab_tol if bicgstab_tol is None else bicgstab_tol),
                      breakdown_tol=float(so.bicgstab_breakdown_tol)).view_as(E)
        if out is not None:
            out.update(q_E=q.view_as(E), wE=wE, aux=aux)
        return self.theta_vjp(theta, col_weights, E, wE, acc, use_col=use_col)

    def theta_vjp(self, theta, col_weights, E, wE, acc, *, use_col):
        """Pull the parameter cotangents and the E adjoint back to (theta, col_weights)."""
        S, G = self.S, int(E.shape[0])
        st = self.static
        th = theta.detach().clone().requires_grad_(True)
        cw = col_weights.detach().clone().requires_grad_(True)
        with torch.enable_grad():
            pS, pD, pL, mt, col = extract_parameters_weighted_cols(th, cw, self.h, statewise=st.statewise,
                                                                   itemwise=st.itemwise, uniform_fast=not use_col)
            E_p, _, _, Ebar_p = self.k.e_step_triton_autograd(E, pS, pD, pL, mt, col, *self.topo,
                                                              use_col_weights=use_col)
            total = ((as_item_param(pS, G, S) * acc.pS).sum() + (as_item_param(pD, G, S) * acc.pD).sum()
                     + (mt * acc.mt).sum() + (col * acc.col).sum() + (E_p * wE).sum() + (Ebar_p * acc.Ebar).sum())
            g_theta, g_col = torch.autograd.grad(total, (th, cw))
        return g_theta, g_col


def plan_of(static) -> SolvePlan:
    """The plan of ``static``, kept as an attribute of the static object."""
    p = getattr(static, "_dropin_plan", None)
    if p is None:
        p = SolvePlan(static)
        static._dropin_plan = p
    return p


def run_forward(static, theta, col_weights):
    """The reference's ``run_forward(static, theta, col_weights) -> (loss, saved)`` on the per-call path."""
    return plan_of(static).forward(theta, col_weights)


def run_backward(static, theta, col_weights, saved):
    """The reference's ``run_backward(static, theta, col_weights, saved) -> (grad_theta, grad_col)``."""
    return plan_of(static).backward(theta, col_weights, saved)
