"""CPU oracle for the log-space solver path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy float64, what the reference's pristine Triton
kernels and its frozen Python glue compute.  It is the checker for the HIP
product and nothing else: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path never
calls it (the package raises if its HIP library is missing).

Every function cites the reference file:line it follows.  Reference paths are
relative to the reference repository root; "pristine" means
``experiments/pristine_kernels``.

Conventions (identical to the reference):
* every quantity is in log2 space; ``-inf`` is an exact zero probability;
* ``lse2(x...) = log2(sum 2^x)`` with the maximum subtracted first and a
  ``-inf``-safe maximum (``m_safe = 0`` when every term is ``-inf``);
* "ancestors of s" means ancestors-or-self (the reference's chase starts at s).

Pinning (see tests/test_oracle_*.py): closed forms on one- and three-node
trees, brute-force non-ancestor sums, brute-force split enumeration, dense
Jacobian Neumann series, torch autograd of the E-step and of the parameter
extraction, and float64 finite differences of the converged loss.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

NEG_INF = -np.inf
LN2 = 0.6931471805599453


# ----------------------------------------------------------------------------
# small helpers
# ----------------------------------------------------------------------------

def _safe(m):
    """``m`` with -inf replaced by 0 (the reference's ``m_safe``)."""
    return np.where(np.isneginf(m), 0.0, m)


def lse2_terms(*terms):
    """Elementwise LSE2 over equally shaped term arrays.

    Mirrors the reference's ``m = max(t...); m_safe; log2(sum exp2(t - m_safe)) + m``
    (pristine wave_step.py:177-192; dts_fused.py:59-62; e_step.py:83-91).
    """
    m = terms[0]
    for t in terms[1:]:
        m = np.maximum(m, t)
    ms = _safe(m)
    total = np.zeros_like(m)
    for t in terms:
        total = total + np.exp2(t - ms)
    with np.errstate(divide="ignore"):
        return np.log2(total) + m


def logsumexp2(x, axis=-1, keepdims=False):
    """Reference kbench/core/inference/logspace.py:11-16."""
    row_max = np.max(x, axis=axis, keepdims=True)
    rms = np.where(np.isneginf(row_max), 0.0, row_max)
    total = np.exp2(x - rms).sum(axis=axis, keepdims=True)
    with np.errstate(divide="ignore"):
        res = np.where(total > 0, np.log2(np.where(total > 0, total, 1.0)), NEG_INF) + row_max
    return res if keepdims else np.squeeze(res, axis=axis)


@dataclass
class Tree:
    """Species-tree tables derived from ``state_helpers``."""

    S: int
    parent: np.ndarray
    c1: np.ndarray
    c2: np.ndarray
    max_depth: int
    sub_start: np.ndarray
    sub_end: np.ndarray
    level_ptr: np.ndarray
    level_par: np.ndarray
    level_c1: np.ndarray
    level_c2: np.ndarray
    anc: np.ndarray          # [S, max_depth] ancestor-or-self chain, -1 padded

    @staticmethod
    def from_helpers(h: dict) -> "Tree":
        S = int(h["S"])
        parent = np.asarray(h["node_parent"], dtype=np.int64)
        D = max(1, int(h["max_ancestor_depth"]))
        anc = np.full((S, D), -1, dtype=np.int64)
        cur = np.arange(S, dtype=np.int64)
        for k in range(D):
            valid = (cur >= 0) & (cur < S)
            anc[:, k] = np.where(valid, cur, -1)
            nxt = parent[np.clip(cur, 0, S - 1)]
            cur = np.where(valid, nxt, -1)
        return Tree(
            S=S,
            parent=parent,
            c1=np.asarray(h["node_child1"], dtype=np.int64),
            c2=np.asarray(h["node_child2"], dtype=np.int64),
            max_depth=D,
            sub_start=np.asarray(h["node_subtree_start"], dtype=np.int64),
            sub_end=np.asarray(h["node_subtree_end"], dtype=np.int64),
            level_ptr=np.asarray(h["compact_level_ptr"], dtype=np.int64),
            level_par=np.asarray(h["compact_level_parents"], dtype=np.int64),
            level_c1=np.asarray(h["compact_level_child1"], dtype=np.int64),
            level_c2=np.asarray(h["compact_level_child2"], dtype=np.int64),
            anc=anc,
        )

    def ancestor_sum(self, X):
        """``sum_{a in anc(s)} X[..., a]`` by the reference's bounded chase.

        Pristine e_step.py:52-62, wave_step.py:68-87 (``MAX_ANCESTOR_DEPTH`` steps).
        """
        out = np.zeros_like(X)
        for k in range(self.max_depth):
            a = self.anc[:, k]
            valid = a >= 0
            out = out + np.where(valid, X[..., np.where(valid, a, 0)], 0.0)
        return out

    def subtree_sum(self, U):
        """Bottom-up subtree sums over compact levels, deepest level first.

        Pristine wave_backward.py:479-512 (jt), 700-733 (col grad), 2287-2306 (tree VJP).
        """
        V = U.copy()
        S = self.S
        for lv in range(self.level_ptr.shape[0] - 1):
            sl = slice(int(self.level_ptr[lv]), int(self.level_ptr[lv + 1]))
            p = self.level_par[sl]
            a = self.level_c1[sl]
            b = self.level_c2[sl]
            add = np.where(a < S, V[..., np.minimum(a, S - 1)], 0.0) + np.where(b < S, V[..., np.minimum(b, S - 1)], 0.0)
            V[..., p] = V[..., p] + add
        return V

    def child_gather(self, X, which):
        """``X[..., c[s]]`` with ``-inf`` where the child is the ``>= S`` sentinel."""
        c = self.c1 if which == 1 else self.c2
        valid = (c >= 0) & (c < self.S)
        return np.where(valid, X[..., np.where(valid, c, 0)], NEG_INF)


# ----------------------------------------------------------------------------
# parameters (reference kbench/core/parameters/extract_parameters.py)
# ----------------------------------------------------------------------------

def log2_softmax(logits):
    """``log_softmax(x * ln2) / ln2`` along the last axis (extract_parameters.py:26-28)."""
    m = np.max(logits, axis=-1, keepdims=True)
    return logits - (m + np.log2(np.exp2(logits - m).sum(axis=-1, keepdims=True)))


def extract_parameters_uniform(theta, unnorm_row_max, statewise=False, itemwise=False):
    """Reference extract_parameters.py:25-34."""
    theta = np.asarray(theta, dtype=np.float64)
    logits = np.concatenate([np.zeros(theta.shape[:-1] + (1,)), theta], axis=-1)
    res = log2_softmax(logits)
    pT = res[..., 3]
    if statewise and not itemwise:
        mt = pT + unnorm_row_max
    else:
        mt = pT[..., None] + unnorm_row_max
    return res[..., 0], res[..., 1], res[..., 2], mt


def col_log_probs_from_weights(col_weights):
    """Reference extract_parameters.py:37-38 (natural-log softmax, then /ln2)."""
    w = np.asarray(col_weights, dtype=np.float64)
    m = w.max()
    return (w - (m + np.log(np.exp(w - m).sum()))) / LN2


def col_valid_log_normalizer(col_log_probs, tree: Tree):
    """Reference extract_parameters.py:41-65."""
    p = np.exp2(col_log_probs)
    mass = tree.ancestor_sum(p)
    valid = 1.0 - mass
    with np.errstate(divide="ignore"):
        return np.where(valid > 0.0, -np.log2(np.maximum(valid, np.finfo(np.float64).tiny)), NEG_INF)


def extract_parameters_weighted_cols(theta, col_weights, tree: Tree, statewise=False, itemwise=False,
                                     uniform_fast=False):
    """Reference extract_parameters.py:68-93."""
    theta = np.asarray(theta, dtype=np.float64)
    logits = np.concatenate([np.zeros(theta.shape[:-1] + (1,)), theta], axis=-1)
    res = log2_softmax(logits)
    pT = res[..., 3]
    cl = col_log_probs_from_weights(col_weights)
    cn = col_valid_log_normalizer(cl, tree)
    mt = pT + cn if (statewise and not itemwise) else pT[..., None] + cn
    if uniform_fast:
        mt = mt - math.log2(tree.S)
    return res[..., 0], res[..., 1], res[..., 2], mt, cl


def as_item_param(t, item_rows, S=None):
    """Reference extract_parameters.py:8-15."""
    t = np.asarray(t, dtype=np.float64)
    if t.ndim == 0:
        return np.broadcast_to(t.reshape(1, 1), (item_rows, 1)).copy()
    if t.ndim == 1:
        if S is not None and item_rows == 1 and t.size == S:
            return t.reshape(1, S).copy()
        return t.reshape(item_rows, 1).copy()
    return t.copy()


def as_item_state(t, S, item_rows):
    """Reference extract_parameters.py:18-22."""
    p = as_item_param(t, item_rows, S)
    if p.shape[1] == S:
        return p
    return np.broadcast_to(p, (item_rows, S)).copy()


# ----------------------------------------------------------------------------
# E-step (reference pristine e_step.py)
# ----------------------------------------------------------------------------

def e_step(E, pS, pD, pL, mt, col, tree: Tree, use_col_weights: bool):
    """One E-step update for every item row; returns (E_new, E_s1, E_s2, Ebar).

    Pristine e_step.py:12-99.  All parameters are ``[G, S]``; ``col`` is ``[S]``.
    """
    wE = E + col if use_col_weights else E
    row_max = wE.max(axis=1, keepdims=True)
    rms = _safe(row_max)
    row_sum = np.exp2(wE - rms).sum(axis=1, keepdims=True)
    anc = tree.ancestor_sum(np.exp2(wE - rms))
    E_s1 = tree.child_gather(E, 1)
    E_s2 = tree.child_gather(E, 2)
    denom = row_sum - anc
    with np.errstate(divide="ignore", invalid="ignore"):
        Ebar = np.where(denom > 0.0, np.log2(np.where(denom > 0, denom, 1.0)) + row_max + mt, NEG_INF)
    E_new = lse2_terms(pS + E_s1 + E_s2, pD + 2.0 * E, E + Ebar, pL)
    return E_new, E_s1, E_s2, Ebar


def e_fixed_point(E0, pS, pD, pL, mt, col, tree: Tree, use_col_weights: bool, max_iter=2000, tol=1e-8):
    """Reference pristine e_step.py:438-501 (host loop with the max-diff stop)."""
    max_iter = int(max_iter)
    tol = float(tol)
    if max_iter < 1:
        raise ValueError("max_iter must be at least 1")
    if tol <= 0.0:
        raise ValueError("tol must be positive")
    E_a = np.array(E0, dtype=np.float64, copy=True)
    n_iter = 0
    for _ in range(max_iter):
        E_b, _, _, _ = e_step(E_a, pS, pD, pL, mt, col, tree, use_col_weights)
        n_iter += 1
        max_diff = float(np.max(np.abs(E_b - E_a)))
        E_a = E_b
        if max_diff < tol:
            break
    _, E_s1, E_s2, Ebar = e_step(E_a, pS, pD, pL, mt, col, tree, use_col_weights)
    return E_a, E_s1, E_s2, Ebar, n_iter


def e_step_vjp(E, pS, pD, pL, mt, col, tree: Tree, use_col_weights, g_new, g_s1, g_s2, g_ebar):
    """VJP of :func:`e_step` -- pristine e_step.py:102-241 (prepare + finalize).

    Returns grads w.r.t. (E, pS, pD, pL, mt, col); the ``col`` gradient is the
    one the reference kernel emits regardless of ``use_col_weights``.
    """
    E_new, E_s1, E_s2, Ebar = e_step(E, pS, pD, pL, mt, col, tree, use_col_weights)
    wE = E + col if use_col_weights else E
    row_max = wE.max(axis=1, keepdims=True)
    rms = _safe(row_max)
    r = np.exp2(wE - rms)
    row_sum = r.sum(axis=1, keepdims=True)
    t0 = pS + E_s1 + E_s2
    t1 = pD + 2.0 * E
    t2 = E + Ebar
    t3 = pL
    q0 = g_new * np.exp2(t0 - E_new)
    q1 = g_new * np.exp2(t1 - E_new)
    q2 = g_new * np.exp2(t2 - E_new)
    q3 = g_new * np.exp2(t3 - E_new)
    q0 = np.nan_to_num(q0, nan=0.0)
    q1 = np.nan_to_num(q1, nan=0.0)
    q2 = np.nan_to_num(q2, nan=0.0)
    q3 = np.nan_to_num(q3, nan=0.0)
    wbar = q2 + g_ebar
    grad_E = 2.0 * q1 + q2
    S = tree.S
    for c, g_out in ((tree.c1, g_s1), (tree.c2, g_s2)):
        valid = (c >= 0) & (c < S)
        idx = np.nonzero(valid)[0]
        np.add.at(grad_E, (slice(None), c[idx]), (q0 + g_out)[:, idx])
    anc = tree.ancestor_sum(r)
    denom = row_sum - anc
    with np.errstate(divide="ignore", invalid="ignore"):
        u = np.where(denom > 0.0, wbar / np.where(denom > 0, denom, 1.0), 0.0)
    total_u = u.sum(axis=1, keepdims=True)
    excluded = tree.subtree_sum(u)
    pibar_vjp = r * (total_u - excluded)
    grad_E = grad_E + pibar_vjp
    grad_col = pibar_vjp.sum(axis=0)
    return grad_E, q0, q1, q3, wbar, grad_col


# ----------------------------------------------------------------------------
# forward wave kernels
# ----------------------------------------------------------------------------

def _pibar_from_pi(Pi, col, mt, tree: Tree, use_col_weights):
    """Pibar plus row stats of a block of rows (pristine wave_step.py:15-89, 205-220)."""
    wPi = Pi + col if use_col_weights else Pi
    row_max = wPi.max(axis=1, keepdims=True)
    rms = _safe(row_max)
    X = np.exp2(wPi - rms)
    row_sum = X.sum(axis=1, keepdims=True)
    anc = tree.ancestor_sum(X)
    denom = row_sum - anc
    with np.errstate(divide="ignore", invalid="ignore"):
        pibar = np.where(denom > 0.0, np.log2(np.where(denom > 0, denom, 1.0)) + row_max + mt, NEG_INF)
    return pibar, row_max[:, 0]


@dataclass
class WaveConsts:
    """Per-item constants ``[G, S]`` the wave kernels read (forward.py:37-58)."""

    mt: np.ndarray
    DL: np.ndarray
    Ebar: np.ndarray
    E: np.ndarray
    SL1: np.ndarray
    SL2: np.ndarray
    leaf_logp: np.ndarray   # pS per item [G, S]
    col: np.ndarray         # [S]
    use_col_weights: bool


def wave_sweep(Pi_in, rows_item, consts: WaveConsts, tree: Tree, *, leaf_state=None, dts_r=None):
    """One sweep of the self-loop map for a block of rows.

    Pristine wave_step.py:92-203 (``_wave_step_kernel``).  ``rows_item`` is the
    item index of every row; ``leaf_state`` (leaf waves) adds the leaf term;
    ``dts_r`` (split waves) adds the split term.
    """
    mt = consts.mt[rows_item]
    pibar, _ = _pibar_from_pi(Pi_in, consts.col, mt, tree, consts.use_col_weights)
    t0 = consts.DL[rows_item] + Pi_in
    t1 = Pi_in + consts.Ebar[rows_item]
    t2 = pibar + consts.E[rows_item]
    t3 = consts.SL1[rows_item] + tree.child_gather(Pi_in, 1)
    t4 = consts.SL2[rows_item] + tree.child_gather(Pi_in, 2)
    terms = [t0, t1, t2, t3, t4]
    if leaf_state is not None:
        S = tree.S
        hit = np.arange(S)[None, :] == leaf_state[:, None]
        terms.append(np.where(hit, consts.leaf_logp[rows_item], NEG_INF))
    if dts_r is not None:
        terms.append(dts_r)
    return lse2_terms(*terms)


def leaf_initial(leaf_state, rows_item, consts: WaveConsts, tree: Tree):
    """Pristine wave_step.py:223-310 (``_leaf_initial_wave_step_kernel``)."""
    S = tree.S
    s = np.arange(S)[None, :]
    ls = leaf_state[:, None]
    leaf_start = tree.sub_start[leaf_state][:, None]
    leaf_end = tree.sub_end[leaf_state][:, None]
    descendant = (tree.sub_start[None, :] >= leaf_start) & (tree.sub_start[None, :] < leaf_end)
    hit = s == ls
    leaf_col = consts.col[leaf_state][:, None] if consts.use_col_weights else 0.0
    pS = consts.leaf_logp[rows_item]
    leaf_obs = pS[np.arange(leaf_state.shape[0]), leaf_state][:, None]
    pi_w = np.where(hit, leaf_obs, NEG_INF)
    pibar_w = np.where(~descendant, consts.mt[rows_item] + leaf_col + leaf_obs, NEG_INF)
    pi_s1 = np.where(tree.c1[None, :] == ls, leaf_obs, NEG_INF)
    pi_s2 = np.where(tree.c2[None, :] == ls, leaf_obs, NEG_INF)
    return lse2_terms(
        consts.DL[rows_item] + pi_w,
        pi_w + consts.Ebar[rows_item],
        pibar_w + consts.E[rows_item],
        consts.SL1[rows_item] + pi_s1,
        consts.SL2[rows_item] + pi_s2,
        np.where(hit, pS, NEG_INF),
    )


def _rate_rows(param, items, S):
    """``_load_rate`` addressing (dts_fused.py:11-15): ``[1|G, 1|S]`` -> per-row ``[n, S]``."""
    p = np.asarray(param, dtype=np.float64)
    if p.ndim == 0:
        p = p.reshape(1, 1)
    rows = p[0:1] if p.shape[0] == 1 else p[items]
    return np.broadcast_to(rows, (items.shape[0], S))


def dts_split_terms(Pi, Pibar, l, r, pD_rows, pS_rows, lsp, tree: Tree):
    """The five split terms (+lsp) of dts_fused.py:54-58 for splits ``(l, r)``."""
    Pl, Pr = Pi[l], Pi[r]
    d0 = lsp[:, None] + pD_rows + Pl + Pr
    d1 = lsp[:, None] + Pl + Pibar[r]
    d2 = lsp[:, None] + Pr + Pibar[l]
    d3 = lsp[:, None] + pS_rows + tree.child_gather(Pl, 1) + tree.child_gather(Pr, 2)
    d4 = lsp[:, None] + pS_rows + tree.child_gather(Pr, 1) + tree.child_gather(Pl, 2)
    return d0, d1, d2, d3, d4


def dts_forward(Pi, Pibar, meta, W, pD_param, pS_param, item_idx, ws, tree: Tree, active=None):
    """``dts_r[W, S]``: LSE over each parent's splits and terms (dts_fused.py:171-231)."""
    S = tree.S
    out = np.full((W, S), NEG_INF)
    sl = np.asarray(meta["sl"])
    N = sl.shape[0]
    if N == 0:
        return out
    sr = np.asarray(meta["sr"])
    red = np.asarray(meta["reduce_idx"])
    lsp = np.asarray(meta.get("log_split_probs", np.zeros(N)), dtype=np.float64).reshape(N)
    items = np.asarray(item_idx)[ws + red]
    d = dts_split_terms(Pi, Pibar, sl, sr, _rate_rows(pD_param, items, S), _rate_rows(pS_param, items, S), lsp, tree)
    per_split = lse2_terms(*d)
    for w in np.unique(red):
        sel = np.nonzero(red == w)[0]
        out[w] = lse2_terms(*[per_split[i] for i in sel])
    if active is not None:
        out[~np.asarray(active, dtype=bool)] = NEG_INF
    return out


# ----------------------------------------------------------------------------
# forward driver (reference kbench/core/inference/{solver,forward}.py)
# ----------------------------------------------------------------------------

@dataclass
class Problem:
    """Numpy view of a generated problem (``kbench.synth.build_problem``)."""

    tree: Tree
    wave_metas: list
    leaf_state: np.ndarray
    root_ids: np.ndarray
    item_idx: np.ndarray       # rate_item_idx (row -> parameter row)
    C: int
    S: int
    statewise: bool
    itemwise: bool
    unnorm_row_max: np.ndarray
    so: dict

    @staticmethod
    def from_dict(p: dict) -> "Problem":
        st = p["static"]
        wl = st["wave_layout"]
        so = {
            "e_init": -1.0, "e_max_iter": 2000, "e_tol": 1e-8, "pi_iters": 6, "neumann_terms": 3,
            "self_loop_solver": "neumann", "bicgstab_max_iter": 500, "bicgstab_tol": 1e-7,
            "bicgstab_breakdown_tol": 1e-30, "adjoint_pruning_threshold": 1e-6,
            "use_adjoint_pruning": True, "pibar_side_threshold": 0.0,
        }
        so.update(p["meta"]["solver_options"])
        return Problem(
            tree=Tree.from_helpers(st["state_helpers"]),
            wave_metas=wl["wave_metas"],
            leaf_state=np.asarray(wl["leaf_state_index"], dtype=np.int64),
            root_ids=np.asarray(wl["root_row_ids"], dtype=np.int64),
            item_idx=np.asarray(st["rate_item_idx"], dtype=np.int64),
            C=int(np.asarray(wl["leaf_state_index"]).shape[0]),
            S=int(st["state_helpers"]["S"]),
            statewise=bool(st["statewise"]),
            itemwise=bool(st["itemwise"]),
            unnorm_row_max=np.asarray(st["state_helpers"]["unnorm_row_max"], dtype=np.float64),
            so=so,
        )


def forward(prob: Problem, theta, col_weights, *, pi_iters=None, return_residual=False):
    """``run_forward``: reference kbench/runtime.py:63-75 -> solver.py:16-96 -> forward.py:8-117.

    Returns ``(loss, saved)`` with the reference's saved-tensor names
    (runtime.py:29-32) plus ``n_e_iter``.
    """
    S, C = prob.S, prob.C
    tree = prob.tree
    cw = np.asarray(col_weights, dtype=np.float64).reshape(-1)
    use_col = not bool(np.all(cw == cw[0]))
    if use_col:
        pS, pD, pL, mt, col = extract_parameters_weighted_cols(theta, cw, tree, prob.statewise, prob.itemwise)
    else:
        pS, pD, pL, mt = extract_parameters_uniform(theta, prob.unnorm_row_max, prob.statewise, prob.itemwise)
        col = np.full(S, -math.log2(S))
    G = int(prob.root_ids.shape[0]) if prob.itemwise else 1
    E0 = np.full((G, S), float(prob.so["e_init"]))
    pS_i, pD_i, pL_i, mt_i = (as_item_state(x, S, G) for x in (pS, pD, pL, mt))
    E, E_s1, E_s2, Ebar, n_e = e_fixed_point(E0, pS_i, pD_i, pL_i, mt_i, col, tree, use_col,
                                             prob.so["e_max_iter"], prob.so["e_tol"])
    P = int(prob.so["pi_iters"] if pi_iters is None else pi_iters)
    if P < 2 or P % 2:
        raise ValueError("pi_iters must be an even integer at least 2")
    consts = WaveConsts(
        mt=mt_i, DL=1.0 + pD_i + E, Ebar=Ebar, E=E, SL1=pS_i + E_s2, SL2=pS_i + E_s1,
        leaf_logp=pS_i, col=col, use_col_weights=use_col,
    )
    pD_param = as_item_param(pD, G, S)
    pS_param = as_item_param(pS, G, S)
    pi = np.full((C, S), np.nan)
    pibar = np.full((C, S), np.nan)
    row_max = np.full(C, np.nan)
    residual = np.zeros(C)
    for meta in prob.wave_metas:
        ws, W = int(meta["start"]), int(meta["W"])
        rows = np.arange(ws, ws + W)
        items = prob.item_idx[rows]
        if "sl" in meta:
            dts_r = dts_forward(pi, pibar, meta, W, pD_param, pS_param, prob.item_idx, ws, tree)
            cur = dts_r
            leaf = None
        else:
            dts_r = None
            leaf = prob.leaf_state[rows]
            cur = leaf_initial(leaf, items, consts, tree)
        prev = cur
        for _ in range(1, P):
            prev = cur
            cur = wave_sweep(cur, items, consts, tree, leaf_state=leaf, dts_r=dts_r)
        pi[rows] = cur
        pb, rmax = _pibar_from_pi(cur, col, mt_i[items], tree, use_col)
        pibar[rows] = pb
        row_max[rows] = rmax
        if return_residual:
            fin = np.isfinite(cur) & np.isfinite(prev)
            residual[rows] = np.where(fin, np.abs(cur - prev), 0.0).max(axis=1)
    root_rows = pi[prob.root_ids]
    loss = nll_from_root_rows(root_rows, E)
    saved = {
        "E": E, "E_s1": E_s1, "E_s2": E_s2, "Ebar": Ebar, "root_rows": root_rows,
        "pi_wave": pi, "pibar_wave": pibar, "pibar_row_max": row_max,
        "log_pS": pS, "log_pD": pD, "log_pL": pL, "max_coupling": mt, "col_log_probs": col,
        "n_e_iter": n_e, "use_col_weights": use_col,
    }
    if return_residual:
        saved["pi_residual"] = residual
    return loss, saved


def nll_vector_from_root_rows(root_rows, E):
    """Reference solver.py:132-139."""
    norm = np.maximum(1.0 - np.exp2(E).mean(axis=-1), np.finfo(np.float64).tiny)
    return -(logsumexp2(root_rows, axis=-1) - math.log2(root_rows.shape[-1]) - np.log2(norm))


def nll_from_root_rows(root_rows, E):
    """Reference solver.py:141-142."""
    return float(np.sum(nll_vector_from_root_rows(root_rows, E)))


# ----------------------------------------------------------------------------
# backward pieces (reference pristine wave_backward.py)
# ----------------------------------------------------------------------------

def active_mask(rhs, threshold, use_pruning=True):
    """Pristine wave_backward.py:138-201: ``max|rhs| >= thr`` (``>`` when pruning is off)."""
    row_max = np.max(np.abs(rhs), axis=1) if rhs.shape[1] else np.zeros(rhs.shape[0])
    row_max = np.maximum(row_max, 0.0)
    return row_max > threshold if not use_pruning else row_max >= threshold


@dataclass
class SelfLoopCoeffs:
    diag: np.ndarray
    pcoef: np.ndarray
    p_prime: np.ndarray
    sl1w: np.ndarray
    sl2w: np.ndarray
    w_L: np.ndarray
    e: list
    inv_sum: np.ndarray


def self_loop_coeffs(Pi_s, Pibar_s, row_max, items, consts: WaveConsts, tree: Tree, *, leaf_state=None,
                     dts_r=None):
    """J^T coefficients at Pi* (pristine wave_backward.py:203-416, precompute kernel)."""
    rms = _safe(row_max)[:, None]
    wPi = Pi_s + consts.col if consts.use_col_weights else Pi_s
    p_prime = np.exp2(wPi - rms)
    row_sum = p_prime.sum(axis=1, keepdims=True)
    t0 = consts.DL[items] + Pi_s
    t1 = Pi_s + consts.Ebar[items]
    t2 = Pibar_s + consts.E[items]
    t3 = consts.SL1[items] + tree.child_gather(Pi_s, 1)
    t4 = consts.SL2[items] + tree.child_gather(Pi_s, 2)
    if leaf_state is not None:
        hit = np.arange(tree.S)[None, :] == leaf_state[:, None]
        t5 = np.where(hit, consts.leaf_logp[items], NEG_INF)
    else:
        t5 = np.full_like(Pi_s, NEG_INF)
    m = np.maximum.reduce([t0, t1, t2, t3, t4, t5])
    ms = _safe(m)
    e = [np.exp2(t - ms) for t in (t0, t1, t2, t3, t4, t5)]
    s = e[0] + e[1] + e[2] + e[3] + e[4] + e[5]
    with np.errstate(divide="ignore", invalid="ignore"):
        inv_sum = np.where(s > 0.0, 1.0 / np.where(s > 0, s, 1.0), 0.0)
        if dts_r is not None:
            dts_l = np.log2(s) + m
            pm = np.maximum(dts_l, dts_r)
            pms = _safe(pm)
            pi_new = np.log2(np.exp2(dts_l - pms) + np.exp2(dts_r - pms)) + pm
            w_L = np.where(np.isneginf(dts_l), 0.0, np.exp2(dts_l - pi_new))
        else:
            w_L = np.ones_like(Pi_s)
    anc = tree.ancestor_sum(p_prime)
    denom = row_sum - anc
    with np.errstate(divide="ignore"):
        inv_denom = np.where(denom > 0.0, 1.0 / np.where(denom > 0, denom, 1.0), 0.0)
    return SelfLoopCoeffs(
        diag=w_L * (e[0] + e[1]) * inv_sum,
        pcoef=w_L * e[2] * inv_sum * inv_denom,
        p_prime=p_prime,
        sl1w=w_L * e[3] * inv_sum,
        sl2w=w_L * e[4] * inv_sum,
        w_L=w_L, e=e, inv_sum=inv_sum,
    )


def apply_JT(term, co: SelfLoopCoeffs, tree: Tree):
    """One J^T application (pristine wave_backward.py:419-570, child-edge form)."""
    S = tree.S
    u = term * co.pcoef
    A = u.sum(axis=1, keepdims=True)
    corr = tree.subtree_sum(u)
    base = term * co.diag + co.p_prime * (A - corr)
    # edge weight into column s from its parent p: sl1w[p] if s == c1[p] else sl2w[p]
    edge = np.zeros_like(term)
    par = tree.parent
    for which, w in ((tree.c1, co.sl1w), (tree.c2, co.sl2w)):
        valid = (which >= 0) & (which < S)
        idx = np.nonzero(valid)[0]
        edge[:, which[idx]] = w[:, idx]
    pv = (par >= 0) & (par < S)
    parent_term = np.where(pv[None, :], term[:, np.where(pv, par, 0)], 0.0)
    return base + parent_term * np.where(pv[None, :], edge, 0.0)


def gmres_fixed(apply_a, b, max_iter):
    """Fixed-iteration unrestarted GMRES (pristine wave_backward.py:574-653).

    ``b`` is flattened into one vector (a whole wave), the Arnoldi basis is
    orthogonalised by classical Gram-Schmidt with one reorthogonalisation, the
    iteration stops early when the new basis norm falls to eps * max(|b|, 1),
    and the solution is the basis combination of the least-squares solution of
    the Hessenberg system against |b| e1.  max_iter < 1 or b = 0 give 0.
    """
    shape = b.shape
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    m = int(max_iter)
    if m < 1:
        return np.zeros(shape)
    bn = float(np.linalg.norm(b))
    if bn == 0.0:
        return np.zeros(shape)
    Q = np.zeros((m + 1, b.size))
    H = np.zeros((m + 1, m))
    Q[0] = b / bn
    tol = np.finfo(np.float64).eps * max(bn, 1.0)
    k = m
    for j in range(m):
        w = np.asarray(apply_a(Q[j].reshape(shape)), dtype=np.float64).reshape(-1)
        c = Q[: j + 1] @ w
        w = w - Q[: j + 1].T @ c
        c2 = Q[: j + 1] @ w
        w = w - Q[: j + 1].T @ c2
        H[: j + 1, j] = c + c2
        h = float(np.linalg.norm(w))
        H[j + 1, j] = h
        if h <= tol:
            k = j + 1
            break
        if j + 1 < m:
            Q[j + 1] = w / max(h, np.finfo(np.float64).tiny)
    e1 = np.zeros(k + 1)
    e1[0] = bn
    y = np.linalg.lstsq(H[: k + 1, :k], e1, rcond=None)[0]
    return (Q[:k].T @ y).reshape(shape)


def wave_backward_uniform(Pi_s, Pibar_s, row_max, rhs, items, consts, tree, neumann_terms, *, active,
                          leaf_state=None, dts_r=None, solver="neumann"):
    """``wave_backward_uniform_fused`` (pristine wave_backward.py:969-1395).

    ``solver="neumann"``: v = sum_{n <= N} (J^T)^n rhs; ``"gmres"``: v solves
    (I - J^T) v = rhs over the wave's active rows by ``gmres_fixed`` with
    N = ``neumann_terms`` iterations (pristine wave_backward.py:1136-1188).
    Returns ``(v_k, aw0, aw1, aw2, aw345, aw3, aw4, col_grad)``; inactive rows
    of every output are zero (``v_k`` inactive rows are "don't care" in the reference).
    """
    co = self_loop_coeffs(Pi_s, Pibar_s, row_max, items, consts, tree, leaf_state=leaf_state, dts_r=dts_r)
    act = np.asarray(active, dtype=bool)[:, None]
    v = np.where(act, rhs, 0.0)
    if solver == "gmres":
        v = gmres_fixed(lambda x: np.where(act, x - apply_JT(x, co, tree), 0.0), v, neumann_terms)
    elif solver != "neumann":
        raise ValueError(f"unsupported self-loop solver {solver!r}")
    term = v.copy()
    for _ in range(int(neumann_terms) if solver == "neumann" else 0):
        term = np.where(act, apply_JT(term, co, tree), 0.0)
        v = v + term
    u = v * co.pcoef
    A = u.sum(axis=1, keepdims=True)
    corr = tree.subtree_sum(u)
    col_grad = np.where(act, co.p_prime * (A - corr), 0.0).sum(axis=0)
    alpha = v * co.w_L
    aw = [np.where(act, alpha * ek * co.inv_sum, 0.0) for ek in co.e]
    aw345 = aw[3] + aw[4] + aw[5]
    return v, aw[0], aw[1], aw[2], aw345, aw[3], aw[4], col_grad


def dts_cross_backward(Pi_s, Pibar_s, row_max, v, ws, meta, pD_param, pS_param, mt_item, item_idx, tree,
                       active, col, use_col_weights, side_thr=0.0):
    """``dts_cross_backward_accum_fused`` + ``uniform_cross_pibar_vjp_tree_from_ud_fused``.

    Pristine wave_backward.py:1529-1945 (cross accumulation, merged S term) and
    2229-2327 (Pibar VJP through the subtree sums).  Returns per-split-side
    contributions to the children's adjoint rows and parameter gradients.

    ``side_thr`` is the glue's ``pibar_side_threshold`` (_implicit_grad.py:300-353):
    above 0 a split side takes part in the Pibar VJP only when the abs-sum of its
    staged u_d over the states exceeds it (pristine wave_backward.py:1777-1779,
    1877-1884; the tree kernel returns early for an inactive side, 2263-2266).
    At 0 the sides whose u_d is all zero are skipped, which changes nothing: their
    A and subtree sums are 0.
    """
    S = tree.S
    sl = np.asarray(meta["sl"])
    sr = np.asarray(meta["sr"])
    red = np.asarray(meta["reduce_idx"])
    N = sl.shape[0]
    lsp = np.asarray(meta.get("log_split_probs", np.zeros(N)), dtype=np.float64).reshape(N)
    act = np.asarray(active, dtype=bool)[red]
    items = np.asarray(item_idx)[ws + red]
    d = dts_split_terms(Pi_s, Pibar_s, sl, sr, _rate_rows(pD_param, items, S), _rate_rows(pS_param, items, S),
                        np.zeros(N), tree)
    Pp = Pi_s[ws + red]
    pv = ~np.isneginf(Pp)
    w = [np.where(pv, np.exp2(lsp[:, None] + dk - np.where(pv, Pp, 0.0)), 0.0) for dk in d]
    vk = v[red]
    vd = [np.where(act[:, None], vk * wk, 0.0) for wk in w]
    # direct Pi adjoints into the child rows (merged S term, wave_backward.py:1741-1853)
    rhs_l = vd[0] + vd[1]
    rhs_r = vd[0] + vd[2]
    for cidx, (tl_, tr_) in ((tree.c1, (vd[3], vd[4])), (tree.c2, (vd[4], vd[3]))):
        valid = (cidx >= 0) & (cidx < S)
        idx = np.nonzero(valid)[0]
        rhs_l[:, cidx[idx]] += tl_[:, idx]
        rhs_r[:, cidx[idx]] += tr_[:, idx]
    # Pibar u_d staging (wave_backward.py:1751-1776)
    mt_l = mt_item[np.asarray(item_idx)[sl]]
    mt_r = mt_item[np.asarray(item_idx)[sr]]
    pbl, pbr = Pibar_s[sl], Pibar_s[sr]
    inv_l = np.where(np.isneginf(pbl), 0.0, np.exp2(row_max[sl][:, None] + mt_l - np.where(np.isneginf(pbl), 0.0, pbl)))
    inv_r = np.where(np.isneginf(pbr), 0.0, np.exp2(row_max[sr][:, None] + mt_r - np.where(np.isneginf(pbr), 0.0, pbr)))
    ud_l = vd[2] * inv_l
    ud_r = vd[1] * inv_r
    direct_l, direct_r = rhs_l.copy(), rhs_r.copy()
    # tree VJP (wave_backward.py:2287-2327)
    col_grad = np.zeros(S)
    sums = {}
    for side, child, ud, acc in (("l", sl, ud_l, rhs_l), ("r", sr, ud_r, rhs_r)):
        A = ud.sum(axis=1, keepdims=True)
        sub = tree.subtree_sum(ud)
        wPi = Pi_s[child] + col if use_col_weights else Pi_s[child]
        pp = np.exp2(wPi - _safe(row_max[child])[:, None])
        on = act if side_thr <= 0.0 else act & (np.abs(ud).sum(axis=1) > side_thr)
        sums["side_on_" + side] = on
        contrib = np.where(on[:, None], pp * (A - sub), 0.0)
        acc += contrib
        col_grad += contrib.sum(axis=0)
        sums["A_" + side], sums["sub_" + side], sums["tree_" + side] = A[:, 0], sub, contrib
    # the direct_* rows (before the Pibar VJP), A_*, sub_* (subtree sums of u_d) and
    # tree_* (the Pibar VJP rows) are the intermediate outputs of the two reference
    # kernels: dts_cross_backward_accum_fused and uniform_cross_pibar_vjp_tree_from_ud_fused
    return {
        "rhs_l": rhs_l, "rhs_r": rhs_r, "g_pD": vd[0], "g_pS": vd[3] + vd[4],
        "g_mt_l": vd[2], "g_mt_r": vd[1], "col_grad": col_grad,
        "ud_l": ud_l, "ud_r": ud_r, "direct_l": direct_l, "direct_r": direct_r, "active_split": act, **sums,
    }


# ----------------------------------------------------------------------------
# backward driver (reference kbench/api/_implicit_grad.py)
# ----------------------------------------------------------------------------

def bicgstab(Av, b, max_iter=500, tol=1e-7, breakdown_tol=1e-30):
    """Reference _implicit_grad.py:28-94 (same control flow and stopping rules)."""
    x = np.zeros_like(b)
    r = b - Av(x)
    bnorm = max(float(np.linalg.norm(b)), 1.0)
    rel_res = float(np.linalg.norm(r)) / bnorm
    if rel_res <= tol:
        return x, 0
    r_hat = r.copy()
    rho_old = alpha = omega = 1.0
    v = np.zeros_like(b)
    p = np.zeros_like(b)
    k = 0
    for k in range(1, int(max_iter) + 1):
        rho = float(r_hat @ r)
        if abs(rho) <= breakdown_tol:
            break
        beta = (rho / rho_old) * (alpha / omega)
        p = r + beta * (p - omega * v)
        v = Av(p)
        denom = float(r_hat @ v)
        if abs(denom) <= breakdown_tol:
            break
        alpha = rho / denom
        s = r - alpha * v
        if float(np.linalg.norm(s)) / bnorm <= tol:
            return x + alpha * p, k
        t = Av(s)
        tt = float(t @ t)
        if abs(tt) <= breakdown_tol:
            break
        omega = float(t @ s) / tt
        x = x + alpha * p + omega * s
        r = s - omega * t
        rel_res = float(np.linalg.norm(r)) / bnorm
        if rel_res <= tol:
            return x, k
        if abs(omega) <= breakdown_tol:
            break
        rho_old = rho
    raise RuntimeError(f"E-adjoint BiCGSTAB solve failed after {k} iterations (relative residual {rel_res:.3e})")


def backward(prob: Problem, theta, col_weights, saved, *, collect=False, cache=None):
    """``run_backward``: reference kbench/runtime.py:77-115 -> _implicit_grad.py:97-475.

    With ``cache`` (a dict) the per-wave adjoints, split terms and masks, the accumulated
    cotangents and the E adjoint are stored for the exact HVP (newton/ggn.py:41-210 with
    ``cache``, newton/hvp_exact.py:37-44).
    """
    so = prob.so
    tree = prob.tree
    S, C = prob.S, prob.C
    cw = np.asarray(col_weights, dtype=np.float64).reshape(-1)
    use_col = not bool(np.all(cw == cw[0]))
    Pi_s = saved["pi_wave"]
    Pibar_s = saved["pibar_wave"]
    row_max = saved["pibar_row_max"]
    E = saved["E"]
    G = E.shape[0]
    E_i, Ebar_i, pS_i, pD_i, mt_i = (as_item_state(x, S, G) for x in
                                     (E, saved["Ebar"], saved["log_pS"], saved["log_pD"], saved["max_coupling"]))
    pD_param = as_item_param(saved["log_pD"], G, S)
    pS_param = as_item_param(saved["log_pS"], G, S)
    col = np.asarray(saved["col_log_probs"], dtype=np.float64)
    consts = WaveConsts(mt=mt_i, DL=1.0 + pD_i + E_i, Ebar=Ebar_i, E=E_i,
                        SL1=pS_i + as_item_state(saved["E_s2"], S, G), SL2=pS_i + as_item_state(saved["E_s1"], S, G),
                        leaf_logp=pS_i, col=col, use_col_weights=use_col)
    acc_rhs = np.zeros((C, S))
    g_pD = np.zeros_like(pD_param)
    g_pS = np.zeros_like(pS_param)
    g_mt = np.zeros_like(mt_i)
    g_col = np.zeros(S)
    g_E = np.zeros_like(E)
    g_Ebar = np.zeros_like(E)
    g_Es1 = np.zeros_like(E)
    g_Es2 = np.zeros_like(E)
    root_Pi = Pi_s[prob.root_ids]
    lse = logsumexp2(root_Pi, axis=-1, keepdims=True)
    fin = ~np.isneginf(root_Pi)
    acc_rhs[prob.root_ids] = -np.where(fin, np.exp2(np.where(fin, root_Pi, 0.0) - np.where(fin, lse, 0.0)), 0.0)

    def scatter(acc, contrib):
        # _implicit_grad.py:159-175 with item_rows == 1
        if acc.shape[1] == 1:
            acc[0, 0] += contrib.sum()
        else:
            acc[0] += contrib.sum(axis=0)

    if G != 1:
        raise NotImplementedError("oracle backward covers item_rows == 1 (itemwise=False)")
    masks = []
    side_bounds = []  # per split wave: abs-sums of the staged u_d, left sides then right sides
    thr = float(so["adjoint_pruning_threshold"])
    prune = bool(so["use_adjoint_pruning"])
    N_terms = int(so["neumann_terms"])
    side_thr = float(so.get("pibar_side_threshold", 0.0))
    solver = str(so["self_loop_solver"]).strip().lower()
    if solver not in ("neumann", "gmres"):
        raise ValueError(f"unsupported self-loop solver {solver!r}")
    for meta in reversed(prob.wave_metas):
        ws, W = int(meta["start"]), int(meta["W"])
        rows = np.arange(ws, ws + W)
        items = prob.item_idx[rows]
        rhs = acc_rhs[rows]
        act = active_mask(rhs, thr, prune)
        masks.append((ws, act))
        has_splits = "sl" in meta
        dts_r = (dts_forward(Pi_s, Pibar_s, meta, W, pD_param, pS_param, prob.item_idx, ws, tree, active=act)
                 if has_splits else None)
        leaf = None if has_splits else prob.leaf_state[rows]
        v, aw0, aw1, aw2, aw345, aw3, aw4, cg = wave_backward_uniform(
            Pi_s[rows], Pibar_s[rows], row_max[rows], rhs, items, consts, tree, N_terms,
            active=act, leaf_state=leaf, dts_r=dts_r, solver=solver)
        g_col += cg
        if cache is not None:
            cache.setdefault("waves", []).append(dict(
                ws=ws, W=W, v=np.where(act[:, None], v, 0.0), dts_r=dts_r, active=act, leaf=leaf, meta=meta))
        scatter(g_pD, aw0)
        scatter(g_pS, aw345)
        scatter(g_E, aw0 + aw2)
        scatter(g_Ebar, aw1)
        scatter(g_Es1, aw4)
        scatter(g_Es2, aw3)
        scatter(g_mt, aw2)
        if has_splits:
            out = dts_cross_backward(Pi_s, Pibar_s, row_max, v, ws, meta, pD_param, pS_param, mt_i,
                                     prob.item_idx, tree, act, col, use_col, side_thr=side_thr)
            side_bounds.append(np.concatenate([np.abs(out["ud_l"]).sum(axis=1), np.abs(out["ud_r"]).sum(axis=1)]))
            np.add.at(acc_rhs, np.asarray(meta["sl"]), out["rhs_l"])
            np.add.at(acc_rhs, np.asarray(meta["sr"]), out["rhs_r"])
            scatter(g_pD, out["g_pD"])
            scatter(g_pS, out["g_pS"])
            g_mt[0] += out["g_mt_l"].sum(axis=0) + out["g_mt_r"].sum(axis=0)
            g_col += out["col_grad"]
    grads = e_adjoint_and_theta_vjp(prob, theta, cw, use_col, saved, g_E, g_Ebar, g_Es1, g_Es2, g_pD, g_pS,
                                    g_mt, g_col)
    if cache is not None:
        cache["accum"] = {"g_E": g_E, "g_Ebar": g_Ebar, "g_Es1": g_Es1, "g_Es2": g_Es2, "g_pD": g_pD,
                          "g_pS": g_pS, "g_mt": g_mt, "g_col": g_col}
        cache["wE"] = grads[2]["wE"]
    if collect:
        acc = {"g_E": g_E, "g_Ebar": g_Ebar, "g_Es1": g_Es1, "g_Es2": g_Es2, "g_pD": g_pD, "g_pS": g_pS,
               "g_mt": g_mt, "g_col": g_col}
        grads = grads + ({"masks": masks, "side_bounds": side_bounds, "acc": acc},)
    return grads


def theta_col_vjp(prob: Problem, theta, cw, use_col, G_pS, G_pD, G_pL, G_mt, G_col):
    """VJP of ``extract_parameters_weighted_cols(uniform_fast=not use_col)`` (extract_parameters.py:68-93).

    ``G_*`` are cotangents of (log_pS, log_pD, log_pL, max_coupling, col_log_probs)
    in the shapes that function returns.
    """
    tree = prob.tree
    theta = np.asarray(theta, dtype=np.float64)
    logits = np.concatenate([np.zeros(theta.shape[:-1] + (1,)), theta], axis=-1)
    res = log2_softmax(logits)
    p = np.exp2(res)                                   # softmax of logits*ln2
    G_pT = G_mt if (prob.statewise and not prob.itemwise) else G_mt.sum(axis=-1)
    Gk = np.stack([G_pS, G_pD, G_pL, G_pT], axis=-1)   # d/d result[..., k]
    tot = Gk.sum(axis=-1, keepdims=True)
    grad_logits = Gk - p * tot                          # log2-softmax VJP
    grad_theta = grad_logits[..., 1:]
    # col_norm part of max_coupling
    cl = col_log_probs_from_weights(cw)
    pc = np.exp2(cl)
    mass = tree.ancestor_sum(pc)
    valid = 1.0 - mass
    G_cn = G_mt if G_mt.ndim == 1 else G_mt.sum(axis=0)
    tiny = np.finfo(np.float64).tiny
    u = np.where(valid >= tiny, G_cn / np.where(valid > 0, valid, 1.0), 0.0)
    u = np.where(valid > 0.0, u, 0.0)
    G_cl = G_col + pc * tree.subtree_sum(u)
    q = np.exp(cw - cw.max())
    q = q / q.sum()
    grad_col = (G_cl - q * G_cl.sum()) / LN2
    return grad_theta, grad_col


def e_adjoint_and_theta_vjp(prob: Problem, theta, cw, use_col, saved, g_E, g_Ebar, g_Es1, g_Es2, g_pD, g_pS,
                            g_mt, g_col):
    """Reference _implicit_grad.py:373-475 (E adjoint by BiCGSTAB, then the theta/col VJP)."""
    so = prob.so
    tree = prob.tree
    S = prob.S
    E = saved["E"]
    G = E.shape[0]
    n_fam = int(prob.root_ids.shape[0])
    pS_i, pD_i, pL_i, mt_i = (as_item_state(x, S, G) for x in
                              (saved["log_pS"], saved["log_pD"], saved["log_pL"], saved["max_coupling"]))
    col = np.asarray(saved["col_log_probs"], dtype=np.float64)
    zero = np.zeros_like(E)
    # aux_to_e: d/dE [direct_obj + <E_s1,gEs1> + <E_s2,gEs2> + <Ebar,gEbar>]
    mean = np.exp2(E).mean(axis=-1, keepdims=True)
    norm = 1.0 - mean
    tiny = np.finfo(np.float64).tiny
    scale = n_fam if G != n_fam else 1
    d_direct = np.where(norm >= tiny, -scale * np.exp2(E) / (S * np.where(norm > 0, norm, 1.0)), 0.0)
    gE_aux, _, _, _, _, _ = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, use_col, zero, g_Es1, g_Es2, g_Ebar)
    q_E = g_E + gE_aux + d_direct

    def AG(w_flat):
        wE = w_flat.reshape(E.shape)
        gE, _, _, _, _, _ = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, use_col, wE, zero, zero, zero)
        return (wE - gE).reshape(-1)

    w_flat, n_bicg = bicgstab(AG, q_E.reshape(-1), so["bicgstab_max_iter"], so["bicgstab_tol"],
                              so["bicgstab_breakdown_tol"])
    wE = w_flat.reshape(E.shape)
    # param cotangents: param_loss + E-step(E*, params) with grads (wE on E_new, g_Ebar on Ebar)
    _, q0, q1, q3, wbar, gcol_e = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, use_col, wE, zero, zero, g_Ebar)
    G_all = _fold_cotangents(saved, S, G, q0, q1, q3, wbar, gcol_e, g_pD, g_pS, g_mt, g_col)
    grad_theta, grad_col = theta_col_vjp(prob, theta, cw, use_col, *G_all)
    return grad_theta, grad_col, {"n_bicgstab": n_bicg, "wE": wE, "q_E": q_E}


def _fold_state(gstate, raw, S, G):
    """Gradient w.r.t. an un-expanded parameter from its [G, S] item-state gradient (as_item_state
    is a broadcast)."""
    raw = np.asarray(raw)
    if raw.ndim == 0:
        return gstate.sum()
    if raw.ndim == 1 and raw.size == S and G == 1:
        return gstate.reshape(S)
    return gstate.reshape(raw.shape) if gstate.size == raw.size else gstate.sum(axis=-1).reshape(raw.shape)


def _fold_param(gparam, raw):
    """Gradient w.r.t. an un-expanded parameter from its as_item_param-shaped gradient."""
    raw = np.asarray(raw)
    if raw.ndim == 0:
        return gparam.sum()
    return gparam.reshape(raw.shape) if gparam.size == raw.size else gparam.sum(axis=-1).reshape(raw.shape)


def _fold_cotangents(saved, S, G, e_pS, e_pD, e_pL, e_mt, e_col, g_pD, g_pS, g_mt, g_col):
    """Cotangents of (log_pS, log_pD, log_pL, max_coupling, col_log_probs) in the shapes the
    parameter extraction returns: E-step head terms (item-state) plus the sweep accumulators
    (reference _implicit_grad.py:440-469; newton/hvp_exact.py:163-168, 354-358)."""
    G_pS = _fold_state(e_pS, saved["log_pS"], S, G) + _fold_param(g_pS, saved["log_pS"])
    G_pD = _fold_state(e_pD, saved["log_pD"], S, G) + _fold_param(g_pD, saved["log_pD"])
    G_pL = _fold_state(e_pL, saved["log_pL"], S, G)
    mt_raw = np.asarray(saved["max_coupling"])
    G_mt = _fold_state(e_mt, mt_raw, S, G) + _fold_state(g_mt, mt_raw, S, G)
    G_col = g_col + e_col
    return G_pS, G_pD, G_pL, G_mt, G_col


# ----------------------------------------------------------------------------
# forward tangents (JVP) of the forward maps: reference
# kbench/core/kernels/{e_step_tangent,dts_tangent,wave_tangent}.py and the glue
# newton/forward_tangent.py
# ----------------------------------------------------------------------------

def _child_tangent(tree: Tree, X, which):
    """``X[..., c[s]]`` with 0 where the child is the ``>= S`` sentinel (tangent gathers)."""
    c = tree.c1 if which == 1 else tree.c2
    valid = (c >= 0) & (c < tree.S)
    return np.where(valid, X[..., np.where(valid, c, 0)], 0.0)


def param_jvp_uniform(theta, v, unnorm_row_max, statewise=False, itemwise=False):
    """Tangent of :func:`extract_parameters_uniform` along ``v`` (newton/forward_tangent.py:29-41).

    The rates are a base-2 log-softmax of [0, theta], so d log2 p_k = dl_k - sum_j p_j dl_j
    with dl = [0, v]; max_coupling = log2 p_T + unnorm_row_max has the tangent of log2 p_T.
    """
    th = np.asarray(theta, dtype=np.float64)
    dv = np.asarray(v, dtype=np.float64)
    logits = np.concatenate([np.zeros(th.shape[:-1] + (1,)), th], axis=-1)
    dlog = np.concatenate([np.zeros(dv.shape[:-1] + (1,)), dv], axis=-1)
    p = np.exp2(log2_softmax(logits))
    d = dlog - (p * dlog).sum(axis=-1, keepdims=True)
    urm = np.asarray(unnorm_row_max, dtype=np.float64)
    if statewise and not itemwise:
        dmt = d[..., 3] + 0.0 * urm
    else:
        dmt = d[..., 3][..., None] + 0.0 * urm
    return d[..., 0], d[..., 1], d[..., 2], dmt


def e_step_tangent(E, dE, pS, pD, pL, mt, col, dpS, dpD, dpL, dmt, tree: Tree, use_col_weights: bool):
    """Tangent of one E-step at E along (dE, dparams) (e_step_tangent.py:27-125).

    Returns (dE_new, dE_s1, dE_s2, dEbar); dE_new = sum_k w_k dt_k with the softmax weights of the
    four E-step terms, dEbar = (dRS - dAS) / denom + dmt.
    """
    wE = E + col if use_col_weights else E
    row_max = wE.max(axis=1, keepdims=True)
    rms = _safe(row_max)
    r = np.exp2(wE - rms)
    row_sum = r.sum(axis=1, keepdims=True)
    dRS = (r * dE).sum(axis=1, keepdims=True)
    anc = tree.ancestor_sum(r)
    dAS = tree.ancestor_sum(r * dE)
    E_s1, E_s2 = tree.child_gather(E, 1), tree.child_gather(E, 2)
    dE_s1, dE_s2 = _child_tangent(tree, dE, 1), _child_tangent(tree, dE, 2)
    denom = row_sum - anc
    pos = denom > 0.0
    sd = np.where(pos, denom, 1.0)
    Ebar = np.where(pos, np.log2(sd) + row_max + mt, NEG_INF)
    dEbar = np.where(pos, (dRS - dAS) / sd + dmt, 0.0)
    t = [pS + E_s1 + E_s2, pD + 2.0 * E, E + Ebar, pL]
    dt = [dpS + dE_s1 + dE_s2, dpD + 2.0 * dE, dE + dEbar, dpL]
    m = np.maximum.reduce(t)
    ms = _safe(m)
    e = [np.exp2(tk - ms) for tk in t]
    total = e[0] + e[1] + e[2] + e[3]
    E_new = np.log2(np.where(total > 0, total, 1.0)) + m
    inv = np.where(total > 0.0, 1.0 / np.where(total > 0, total, 1.0), 0.0)
    dE_new = sum(ek * inv * dtk for ek, dtk in zip(e, dt))
    dE_new = np.where(np.isneginf(E_new) | (total <= 0), 0.0, dE_new)
    return dE_new, dE_s1, dE_s2, dEbar


def e_tangent_fixed_point(E_star, dpS, dpD, dpL, dmt, pS, pD, pL, mt, col, tree: Tree, *, max_iter=2000,
                          tol=1e-9, use_col_weights=True, dE0=None):
    """Richardson solve of (I - J_E^EE) dE* = J_E^Ep dp at frozen E* (e_step_tangent.py:174-208).

    Stops when max|dE_new - dE| <= tol * max(1, max|dE_new|).
    """
    G, S = E_star.shape
    st = lambda x: np.broadcast_to(as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S))
    args = tuple(st(x) for x in (pS, pD, pL, mt))
    dargs = tuple(st(x) for x in (dpS, dpD, dpL, dmt))
    dE = np.zeros_like(E_star) if dE0 is None else np.array(dE0, dtype=np.float64)
    for _ in range(int(max_iter)):
        nxt = e_step_tangent(E_star, dE, *args, col, *dargs, tree, use_col_weights)[0]
        diff = float(np.abs(nxt - dE).max())
        dE = nxt
        if diff <= tol * max(1.0, float(np.abs(dE).max())):
            break
    _, dE_s1, dE_s2, dEbar = e_step_tangent(E_star, dE, *args, col, *dargs, tree, use_col_weights)
    return dE, dE_s1, dE_s2, dEbar


def dts_tangent(Pi, Pibar, dPi, dPibar, meta, W, pD_param, pS_param, dpD_param, dpS_param, dts_r, item_idx, ws,
                tree: Tree):
    """Tangent of :func:`dts_forward` (dts_tangent.py:25-122): sum over a row's splits of
    sum_k 2^(t_k - dts_r) dt_k; 0 where dts_r is -inf."""
    S = tree.S
    out = np.zeros((W, S))
    sl = np.asarray(meta["sl"])
    N = sl.shape[0]
    if N == 0:
        return out
    sr = np.asarray(meta["sr"])
    red = np.asarray(meta["reduce_idx"])
    lsp = np.asarray(meta.get("log_split_probs", np.zeros(N)), dtype=np.float64).reshape(N)
    items = np.asarray(item_idx)[ws + red]
    pD, pS = _rate_rows(pD_param, items, S), _rate_rows(pS_param, items, S)
    dpD, dpS = _rate_rows(dpD_param, items, S), _rate_rows(dpS_param, items, S)
    t = dts_split_terms(Pi, Pibar, sl, sr, pD, pS, lsp, tree)
    dPl, dPr = dPi[sl], dPi[sr]
    dt = [dpD + dPl + dPr, dPl + dPibar[sr], dPr + dPibar[sl],
          dpS + _child_tangent(tree, dPl, 1) + _child_tangent(tree, dPr, 2),
          dpS + _child_tangent(tree, dPr, 1) + _child_tangent(tree, dPl, 2)]
    base = dts_r[red]
    live = ~np.isneginf(base)
    with np.errstate(invalid="ignore", over="ignore"):
        contrib = sum(np.exp2(tk - np.where(live, base, 0.0)) * dtk for tk, dtk in zip(t, dt))
    contrib = np.where(live, np.nan_to_num(contrib, nan=0.0, posinf=0.0, neginf=0.0), 0.0)
    np.add.at(out, red, contrib)
    return out


@dataclass
class WaveTangentConsts:
    """Tangents of the wave constants (newton/forward_tangent.py:58-91), [G, S] each."""

    dDL: np.ndarray
    dEbar: np.ndarray
    dE: np.ndarray
    dSL1: np.ndarray
    dSL2: np.ndarray
    dMC: np.ndarray
    dleaf: np.ndarray


def wave_step_tangent(Pi_in, dPi_in, rows_item, consts: WaveConsts, dc: WaveTangentConsts, tree: Tree, *,
                      leaf_state=None, dts_r=None, d_dts=None, n_iters=1):
    """``n_iters`` tangent applications of the sweep at the frozen rows ``Pi_in``
    (wave_tangent.py:38-171 one step; 174-343 the fused self-loop).

    Returns (dPi after n_iters, dPibar of the last iteration's input tangent).
    """
    S = tree.S
    wPi = Pi_in + consts.col if consts.use_col_weights else Pi_in
    row_max = wPi.max(axis=1, keepdims=True)
    rms = _safe(row_max)
    r = np.exp2(wPi - rms)
    row_sum = r.sum(axis=1, keepdims=True)
    anc = tree.ancestor_sum(r)
    mt = consts.mt[rows_item]
    denom = row_sum - anc
    pos = denom > 0.0
    sd = np.where(pos, denom, 1.0)
    pibar = np.where(pos, np.log2(sd) + row_max + mt, NEG_INF)
    t = [consts.DL[rows_item] + Pi_in, Pi_in + consts.Ebar[rows_item], pibar + consts.E[rows_item],
         consts.SL1[rows_item] + tree.child_gather(Pi_in, 1), consts.SL2[rows_item] + tree.child_gather(Pi_in, 2)]
    if leaf_state is not None:
        hit = np.arange(S)[None, :] == np.asarray(leaf_state)[:, None]
        t5 = np.where(hit, consts.leaf_logp[rows_item], NEG_INF)
        dt5 = np.where(hit, dc.dleaf[rows_item], 0.0)
    else:
        t5 = np.full_like(Pi_in, NEG_INF)
        dt5 = np.zeros_like(Pi_in)
    terms = t + [t5]
    if dts_r is not None:
        terms.append(dts_r)
    m = np.maximum.reduce(terms)
    ms = _safe(m)
    e = [np.exp2(tk - ms) for tk in terms]
    total = sum(e)
    result = np.log2(np.where(total > 0, total, 1.0)) + m
    inv = np.where(total > 0.0, 1.0 / np.where(total > 0, total, 1.0), 0.0)
    valid = ~np.isneginf(result) & (total > 0)
    dpi = np.array(dPi_in, dtype=np.float64)
    dpibar = np.zeros_like(dpi)
    for _ in range(max(int(n_iters), 1)):
        dRS = (r * dpi).sum(axis=1, keepdims=True)
        dAS = tree.ancestor_sum(r * dpi)
        dpibar = np.where(pos, (dRS - dAS) / sd + dc.dMC[rows_item], 0.0)
        dt = [dc.dDL[rows_item] + dpi, dpi + dc.dEbar[rows_item], dpibar + dc.dE[rows_item],
              dc.dSL1[rows_item] + _child_tangent(tree, dpi, 1), dc.dSL2[rows_item] + _child_tangent(tree, dpi, 2),
              dt5]
        num = sum(ek * dtk for ek, dtk in zip(e[:6], dt))
        if dts_r is not None:
            num = num + e[6] * d_dts
        dpi = np.where(valid, num * inv, 0.0)
    return dpi, dpibar


def jvp_root_scores(prob: Problem, theta, v, saved, *, self_iters=None, e_tol=1e-12, return_full=False):
    """d(root rows of Pi)/dtheta . v (newton/forward_tangent.py:102-209), uniform column weights.

    Runs the E tangent fixed point, then per wave the split-term tangent and ``self_iters``
    tangent sweeps at the saved Pi* (default: pi_iters).  Returns (roots [n_fam, S], dPi, dPibar),
    plus a dict of the parameter / E tangents and the sweep's tangent constants with
    ``return_full``.
    """
    S, C, tree = prob.S, prob.C, prob.tree
    G = int(prob.root_ids.shape[0]) if prob.itemwise else 1
    n_it = int(prob.so["pi_iters"]) if self_iters is None else int(self_iters)
    dpS, dpD, dpL, dmt = param_jvp_uniform(theta, v, prob.unnorm_row_max, prob.statewise, prob.itemwise)
    st = lambda x: np.broadcast_to(as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    E = np.asarray(saved["E"], dtype=np.float64)
    pS, pD, pL, mt = (st(saved[k]) for k in ("log_pS", "log_pD", "log_pL", "max_coupling"))
    col = np.asarray(saved["col_log_probs"], dtype=np.float64)
    dE, dE_s1, dE_s2, dEbar = e_tangent_fixed_point(E, dpS, dpD, dpL, dmt, pS, pD, pL, mt, col, tree,
                                                    max_iter=int(prob.so["e_max_iter"]), tol=e_tol,
                                                    use_col_weights=False)
    consts = WaveConsts(mt=mt, DL=1.0 + pD + E, Ebar=np.asarray(saved["Ebar"], dtype=np.float64), E=E,
                        SL1=pS + np.asarray(saved["E_s2"], dtype=np.float64),
                        SL2=pS + np.asarray(saved["E_s1"], dtype=np.float64), leaf_logp=pS, col=col,
                        use_col_weights=False)
    dps_i, dpd_i = st(dpS), st(dpD)
    dc = WaveTangentConsts(dDL=dpd_i + dE, dEbar=dEbar, dE=dE, dSL1=dps_i + dE_s2, dSL2=dps_i + dE_s1, dMC=st(dmt),
                           dleaf=dps_i)
    pD_param, pS_param = as_item_param(np.asarray(saved["log_pD"]), G, S), as_item_param(np.asarray(saved["log_pS"]), G, S)
    dpD_param, dpS_param = as_item_param(dpD, G, S), as_item_param(dpS, G, S)
    Pi = np.asarray(saved["pi_wave"], dtype=np.float64)
    Pb = np.asarray(saved["pibar_wave"], dtype=np.float64)
    dPi = np.zeros((C, S))
    dPb = np.zeros((C, S))
    for meta in prob.wave_metas:
        ws, W = int(meta["start"]), int(meta["W"])
        rows = np.arange(ws, ws + W)
        items = prob.item_idx[rows]
        if "sl" in meta:
            dts_r = dts_forward(Pi, Pb, meta, W, pD_param, pS_param, prob.item_idx, ws, tree)
            d_dts = dts_tangent(Pi, Pb, dPi, dPb, meta, W, pD_param, pS_param, dpD_param, dpS_param, dts_r,
                                prob.item_idx, ws, tree)
            leaf = None
        else:
            dts_r = d_dts = None
            leaf = prob.leaf_state[rows]
        dPi[rows], dPb[rows] = wave_step_tangent(Pi[rows], dPi[rows], items, consts, dc, tree, leaf_state=leaf,
                                                 dts_r=dts_r, d_dts=d_dts, n_iters=n_it)
    if return_full:
        full = dict(dpS=dpS, dpD=dpD, dpL=dpL, dmt=dmt, dE=dE, dE_s1=dE_s1, dE_s2=dE_s2, dEbar=dEbar, dc=dc,
                    consts=consts, dpD_param=dpD_param, dpS_param=dpS_param, pD_param=pD_param, pS_param=pS_param)
        return dPi[prob.root_ids], dPi, dPb, full
    return dPi[prob.root_ids], dPi, dPb


# ----------------------------------------------------------------------------
# second-order contractions and the exact HVP: reference
# kbench/core/kernels/{e_step_so,wave_so,dts_so}.py and newton/{ggn,hvp_exact}.py
# ----------------------------------------------------------------------------

def e_step_backward_so(E, E_new, E_s1, E_s2, Ebar, pS, pD, pL, col, tree: Tree, g_new, g_ebar, dE, dE_new, dE_s1,
                       dE_s2, dEbar, dpS, dpD, dpL, dcol=None, use_col_weights=False):
    """Tangent of the E-step VJP at fixed cotangents (e_step_so.py:30-220).

    Returns (d_grad_E, d_grad_pS, d_grad_pD, d_grad_pL, d_grad_mc, d_grad_col).  With the term
    weights q_k = g_new 2^(t_k - E_new):  dq_k = ln2 q_k (dt_k - dE_new); the Pibar part
    r (tot - excl) with u = (q2 + g_ebar) / denom differentiates with the row max frozen.
    The g_s1 / g_s2 cotangents enter the VJP linearly and drop out.
    """
    t = [pS + E_s1 + E_s2, pD + 2.0 * E, E + Ebar, pL]
    dt = [dpS + dE_s1 + dE_s2, dpD + 2.0 * dE, dE + dEbar, dpL]
    with np.errstate(invalid="ignore", over="ignore"):
        q = [np.nan_to_num(g_new * np.exp2(tk - E_new), nan=0.0) for tk in t]
    dq = [np.where(qk != 0.0, LN2 * qk * (dtk - dE_new), 0.0) for qk, dtk in zip(q, dt)]
    d_gE = 2.0 * dq[1] + dq[2]
    S = tree.S
    for c in (tree.c1, tree.c2):
        valid = (c >= 0) & (c < S)
        idx = np.nonzero(valid)[0]
        np.add.at(d_gE, (slice(None), c[idx]), dq[0][:, idx])
    wE = E + col if use_col_weights else E
    dcol_ = np.zeros_like(col) if dcol is None else dcol
    dwE = dE + dcol_ if use_col_weights else dE
    rms = _safe(wE.max(axis=1, keepdims=True))
    r = np.exp2(wE - rms)
    dr = LN2 * r * dwE
    denom = r.sum(axis=1, keepdims=True) - tree.ancestor_sum(r)
    ddenom = dr.sum(axis=1, keepdims=True) - tree.ancestor_sum(dr)
    pos = denom > 0.0
    sd = np.where(pos, denom, 1.0)
    u = np.where(pos, (q[2] + g_ebar) / sd, 0.0)
    du = np.where(pos, (dq[2] - u * ddenom) / sd, 0.0)
    d_pv = (dr * (u.sum(axis=1, keepdims=True) - tree.subtree_sum(u))
            + r * (du.sum(axis=1, keepdims=True) - tree.subtree_sum(du)))
    return d_gE + d_pv, dq[0], dq[1], dq[3], dq[2], d_pv.sum(axis=0)


def wave_backward_so(Pi, dPi, Pibar, dPibar, v, row_max, items, consts: WaveConsts, dc: WaveTangentConsts,
                     tree: Tree, *, leaf_state=None, dts_r=None, d_dts=None, rhs_rows=None):
    """Tangent of one self-loop J^T application and of the parameter buckets at fixed adjoint v
    (wave_so.py:37-293), the saved row max frozen.

    Returns (d_Av (+ rhs_rows when given), d_aw0, d_aw1, d_aw2, d_aw345, d_aw3, d_aw4).
    """
    S = tree.S
    rms = _safe(row_max)[:, None]
    wPi = Pi + consts.col if consts.use_col_weights else Pi
    pp = np.exp2(wPi - rms)
    dpp = LN2 * pp * dPi
    denom = pp.sum(axis=1, keepdims=True) - tree.ancestor_sum(pp)
    ddenom = dpp.sum(axis=1, keepdims=True) - tree.ancestor_sum(dpp)
    pos = denom > 0.0
    inv_den = np.where(pos, 1.0 / np.where(pos, denom, 1.0), 0.0)
    t = [consts.DL[items] + Pi, Pi + consts.Ebar[items], Pibar + consts.E[items],
         consts.SL1[items] + tree.child_gather(Pi, 1), consts.SL2[items] + tree.child_gather(Pi, 2)]
    dt = [dc.dDL[items] + dPi, dPi + dc.dEbar[items], dPibar + dc.dE[items],
          dc.dSL1[items] + _child_tangent(tree, dPi, 1), dc.dSL2[items] + _child_tangent(tree, dPi, 2)]
    if leaf_state is not None:
        hit = np.arange(S)[None, :] == np.asarray(leaf_state)[:, None]
        t.append(np.where(hit, consts.leaf_logp[items], NEG_INF))
        dt.append(np.where(hit, dc.dleaf[items], 0.0))
    else:
        t.append(np.full_like(Pi, NEG_INF))
        dt.append(np.zeros_like(Pi))
    m = np.maximum.reduce(t)
    ms = _safe(m)
    e = [np.exp2(tk - ms) for tk in t]
    tot = sum(e)
    inv = np.where(tot > 0.0, 1.0 / np.where(tot > 0, tot, 1.0), 0.0)
    w = [ek * inv for ek in e]
    dlse = sum(wk * np.where(wk != 0.0, dtk, 0.0) for wk, dtk in zip(w, dt))
    dw = [np.where(wk != 0.0, LN2 * wk * (dtk - dlse), 0.0) for wk, dtk in zip(w, dt)]
    if dts_r is not None:
        with np.errstate(divide="ignore"):
            dts_l = np.where(tot > 0.0, np.log2(np.where(tot > 0, tot, 1.0)) + m, NEG_INF)
        pm = np.maximum(dts_l, dts_r)
        pms = _safe(pm)
        pi_new = np.log2(np.exp2(dts_l - pms) + np.exp2(dts_r - pms)) + pm
        wL = np.where(np.isneginf(dts_l), 0.0, np.exp2(dts_l - np.where(np.isneginf(dts_l), 0.0, pi_new)))
        both = ~np.isneginf(dts_r) & ~np.isneginf(dts_l)
        dwL = np.where(both, LN2 * wL * (1.0 - wL) * (dlse - np.where(both, d_dts, 0.0)), 0.0)
    else:
        wL = np.ones_like(Pi)
        dwL = np.zeros_like(Pi)
    da = [v * (dwL * wk + wL * dwk) for wk, dwk in zip(w, dw)]
    pc = wL * w[2] * inv_den
    dpc = (dwL * w[2] + wL * dw[2]) * inv_den - pc * inv_den * ddenom
    u, du = v * pc, v * dpc
    A, dA = u.sum(axis=1, keepdims=True), du.sum(axis=1, keepdims=True)
    out = (v * (dwL * (w[0] + w[1]) + wL * (dw[0] + dw[1])) + dpp * (A - tree.subtree_sum(u))
           + pp * (dA - tree.subtree_sum(du)))
    if rhs_rows is not None:
        out = out + rhs_rows
    for c, k in ((tree.c1, 3), (tree.c2, 4)):
        valid = (c >= 0) & (c < S)
        idx = np.nonzero(valid)[0]
        np.add.at(out, (slice(None), c[idx]), (v * (dwL * w[k] + wL * dw[k]))[:, idx])
    return out, da[0], da[1], da[2], da[3] + da[4] + da[5], da[3], da[4]


def dts_backward_so(Pi, dPi, Pibar, dPibar, v, ws, meta, pD_param, pS_param, dpD_param, dpS_param, mt_item,
                    dmt_item, col, row_max, item_idx, tree: Tree, use_col_weights=False):
    """Tangent of the split-term backward and its Pibar tree VJP at fixed adjoint v (dts_so.py:29-303),
    the saved row maxes frozen (the parent Pi normaliser is not).

    Returns a dict: d_rhs_l / d_rhs_r [N, S] (into the child rows sl / sr), d_pD / d_pS / d_mt
    [N, S] (per split, in the parent's item row) and d_col [S].
    """
    S = tree.S
    sl, sr = np.asarray(meta["sl"]), np.asarray(meta["sr"])
    red = np.asarray(meta["reduce_idx"])
    N = sl.shape[0]
    lsp = np.asarray(meta.get("log_split_probs", np.zeros(N)), dtype=np.float64).reshape(N)
    items = np.asarray(item_idx)[int(meta["start"]) + red]
    pD, pS = _rate_rows(pD_param, items, S), _rate_rows(pS_param, items, S)
    dpD, dpS = _rate_rows(dpD_param, items, S), _rate_rows(dpS_param, items, S)
    d = dts_split_terms(Pi, Pibar, sl, sr, pD, pS, np.zeros(N), tree)
    dPl, dPr = dPi[sl], dPi[sr]
    dd = [dpD + dPl + dPr, dPl + dPibar[sr], dPr + dPibar[sl],
          dpS + _child_tangent(tree, dPl, 1) + _child_tangent(tree, dPr, 2),
          dpS + _child_tangent(tree, dPr, 1) + _child_tangent(tree, dPl, 2)]
    prow = int(ws) + red
    Pp, dPp = Pi[prow], dPi[prow]
    fin = ~np.isneginf(Pp)
    w = [np.where(fin, np.exp2(lsp[:, None] + dk - np.where(fin, Pp, 0.0)), 0.0) for dk in d]
    vk = v[red]
    vd = [vk * wk for wk in w]
    dvd = [np.where(wk != 0.0, vk * LN2 * wk * (ddk - dPp), 0.0) for wk, ddk in zip(w, dd)]
    rl = dvd[0] + dvd[1]
    rr = dvd[0] + dvd[2]
    for c, (a_l, a_r) in ((tree.c1, (dvd[3], dvd[4])), (tree.c2, (dvd[4], dvd[3]))):
        valid = (c >= 0) & (c < S)
        idx = np.nonzero(valid)[0]
        np.add.at(rl, (slice(None), c[idx]), a_l[:, idx])
        np.add.at(rr, (slice(None), c[idx]), a_r[:, idx])
    mt, dmt = mt_item[items], dmt_item[items]
    d_col = np.zeros(S)
    for child, vdk, dvdk, acc in ((sl, vd[2], dvd[2], rl), (sr, vd[1], dvd[1], rr)):
        pb, dpb = Pibar[child], dPibar[child]
        ok = ~np.isneginf(pb)
        f = np.where(ok, np.exp2(row_max[child][:, None] + mt - np.where(ok, pb, 0.0)), 0.0)
        ud = vdk * f
        dud = dvdk * f + np.where(f != 0.0, vdk * LN2 * f * (dmt - dpb), 0.0)
        A, dA = ud.sum(axis=1, keepdims=True), dud.sum(axis=1, keepdims=True)
        pc = Pi[child]
        wpc = pc + col if use_col_weights else pc
        okc = ~np.isneginf(pc)
        pp = np.where(okc, np.exp2(np.where(okc, wpc, 0.0) - _safe(row_max[child])[:, None]), 0.0)
        contrib = LN2 * pp * dPi[child] * (A - tree.subtree_sum(ud)) + pp * (dA - tree.subtree_sum(dud))
        acc += contrib
        d_col += contrib.sum(axis=0)
    return {"d_rhs_l": rl, "d_rhs_r": rr, "d_pD": dvd[0], "d_pS": dvd[3] + dvd[4], "d_mt": dvd[1] + dvd[2],
            "d_col": d_col}


def theta_head_hvp(prob: Problem, theta, u, G_pS, G_pD, G_pL, G_mt):
    """Second derivative of the parameter extraction contracted with fixed cotangents, along u:
    d/dtheta [theta_col_vjp(theta; G)] . u (newton/hvp_exact.py:153-185, the head term).

    The rates are a base-2 log-softmax of [0, theta]: the VJP is G_k - p_k sum(G); its tangent
    is -dp_k sum(G) with dp = ln2 p (dl - sum p dl), dl = [0, u].  The column normaliser of
    max_coupling does not depend on theta.
    """
    th = np.asarray(theta, dtype=np.float64)
    uu = np.asarray(u, dtype=np.float64).reshape(th.shape)
    logits = np.concatenate([np.zeros(th.shape[:-1] + (1,)), th], axis=-1)
    dl = np.concatenate([np.zeros(uu.shape[:-1] + (1,)), uu], axis=-1)
    p = np.exp2(log2_softmax(logits))
    dp = LN2 * p * (dl - (p * dl).sum(axis=-1, keepdims=True))
    G_pT = G_mt if (prob.statewise and not prob.itemwise) else G_mt.sum(axis=-1)
    tot = (np.stack([G_pS, G_pD, G_pL, G_pT], axis=-1)).sum(axis=-1, keepdims=True)
    return (-dp * tot)[..., 1:]


def build_point_cache(prob: Problem, theta, col_weights, saved):
    """Backward once with the per-wave adjoints cached (newton/hvp_exact.py:37-44)."""
    cache = {}
    gt, gc, _ = backward(prob, theta, col_weights, saved, cache=cache)
    return gt, gc, cache


def hvp_exact(prob: Problem, theta, saved, u, cache, *, tangent_self_iters=None, e_tol=1e-12):
    """Exact Hessian-vector product of the loss at theta (newton/hvp_exact.py:54-383),
    forward-over-reverse at the cached point, uniform column weights, item_rows == 1.

    One tangent forward sweep (``jvp_root_scores``), then in reversed wave order: the
    second-order contraction at the cached adjoint, the tangent adjoint solve with the same
    operator and mask, the split-term backward of the tangent adjoint and its own second-order
    contraction; then the E side (contractions, tangent E-adjoint by BiCGSTAB) and the
    parameter head (linear in the tangent cotangents, plus the head's Hessian term).
    """
    so = prob.so
    tree = prob.tree
    S, C = prob.S, prob.C
    G = saved["E"].shape[0]
    if G != 1:
        raise NotImplementedError("oracle HVP covers item_rows == 1")
    n_it = int(so["pi_iters"]) if tangent_self_iters is None else int(tangent_self_iters)
    uu = np.asarray(u, dtype=np.float64).reshape(np.shape(theta))
    roots_t, dPi, dPb, full = jvp_root_scores(prob, theta, uu, saved, self_iters=n_it, e_tol=e_tol,
                                              return_full=True)
    dc, consts = full["dc"], full["consts"]
    Pi, Pb, rmax = saved["pi_wave"], saved["pibar_wave"], saved["pibar_row_max"]
    acc = cache["accum"]
    wE = cache["wE"]
    st = lambda x: np.broadcast_to(as_item_state(np.asarray(x, dtype=np.float64), S, G), (G, S)).copy()
    pD_param, pS_param = full["pD_param"], full["pS_param"]
    # root seed tangent: -q is the loss seed, d(-q) = -ln2 q (t - <q, t>)
    R = Pi[prob.root_ids]
    fin = ~np.isneginf(R)
    q = np.where(fin, np.exp2(np.where(fin, R, 0.0) - logsumexp2(R, axis=-1, keepdims=True)), 0.0)
    d_rhs = np.zeros((C, S))
    d_rhs[prob.root_ids] = -LN2 * q * (roots_t - (q * roots_t).sum(axis=-1, keepdims=True))
    d_gpD, d_gpS = np.zeros_like(acc["g_pD"]), np.zeros_like(acc["g_pS"])
    d_gE, d_gEbar, d_gEs1, d_gEs2 = (np.zeros((G, S)) for _ in range(4))
    d_gmt, d_gcol = np.zeros_like(acc["g_mt"]), np.zeros(S)

    def scatter(a, contrib):
        if a.shape[1] == 1:
            a[0, 0] += contrib.sum()
        else:
            a[0] += contrib.sum(axis=0)

    N_terms = int(so["neumann_terms"])
    for wave in cache["waves"]:
        ws, W, meta = wave["ws"], wave["W"], wave["meta"]
        rows = np.arange(ws, ws + W)
        items = prob.item_idx[rows]
        dts_r, act, leaf, v_k = wave["dts_r"], wave["active"], wave["leaf"], wave["v"]
        d_dts = None
        if dts_r is not None:
            d_dts = dts_tangent(Pi, Pb, dPi, dPb, meta, W, pD_param, pS_param, full["dpD_param"],
                                full["dpS_param"], dts_r, prob.item_idx, ws, tree)
        c_out = wave_backward_so(Pi[rows], dPi[rows], Pb[rows], dPb[rows], v_k, rmax[rows], items, consts, dc, tree,
                                 leaf_state=leaf, dts_r=dts_r, d_dts=d_dts, rhs_rows=d_rhs[rows])
        dv, *l_aw, cg = wave_backward_uniform(Pi[rows], Pb[rows], rmax[rows], c_out[0], items, consts, tree, N_terms,
                                              active=act, leaf_state=leaf, dts_r=dts_r)
        d_gcol += cg
        aw0, aw1, aw2, aw345, aw3, aw4 = (c + l for c, l in zip(c_out[1:], l_aw))
        scatter(d_gpD, aw0)
        scatter(d_gpS, aw345)
        scatter(d_gE, aw0 + aw2)
        scatter(d_gEbar, aw1)
        scatter(d_gEs1, aw4)
        scatter(d_gEs2, aw3)
        scatter(d_gmt, aw2)
        if dts_r is not None:
            out = dts_cross_backward(Pi, Pb, rmax, dv, ws, meta, pD_param, pS_param, consts.mt, prob.item_idx, tree,
                                     act, consts.col, False)
            np.add.at(d_rhs, np.asarray(meta["sl"]), out["rhs_l"])
            np.add.at(d_rhs, np.asarray(meta["sr"]), out["rhs_r"])
            scatter(d_gpD, out["g_pD"])
            scatter(d_gpS, out["g_pS"])
            d_gmt[0] += out["g_mt_l"].sum(axis=0) + out["g_mt_r"].sum(axis=0)
            d_gcol += out["col_grad"]
            so2 = dts_backward_so(Pi, dPi, Pb, dPb, v_k, ws, meta, pD_param, pS_param, full["dpD_param"],
                                  full["dpS_param"], consts.mt, dc.dMC, consts.col, rmax, prob.item_idx, tree)
            np.add.at(d_rhs, np.asarray(meta["sl"]), so2["d_rhs_l"])
            np.add.at(d_rhs, np.asarray(meta["sr"]), so2["d_rhs_r"])
            scatter(d_gpD, so2["d_pD"])
            scatter(d_gpS, so2["d_pS"])
            d_gmt[0] += so2["d_mt"].sum(axis=0)
            d_gcol += so2["d_col"]
    # ---- E side
    E = saved["E"]
    pS_i, pD_i, pL_i, mt_i = (st(saved[k]) for k in ("log_pS", "log_pD", "log_pL", "max_coupling"))
    col = np.asarray(saved["col_log_probs"], dtype=np.float64)
    zero = np.zeros_like(E)
    dE, dEs1, dEs2, dEbar = full["dE"], full["dE_s1"], full["dE_s2"], full["dEbar"]
    dx = (dE, dE, dEs1, dEs2, dEbar, st(full["dpS"]), st(full["dpD"]), st(full["dpL"]))
    x = (E, E, saved["E_s1"], saved["E_s2"], saved["Ebar"], pS_i, pD_i, pL_i, col, tree)
    aux_lin = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, False, zero, d_gEs1, d_gEs2, d_gEbar)[0]
    so_aux = e_step_backward_so(*x, zero, acc["g_Ebar"], *dx)
    n_fam = int(prob.root_ids.shape[0])
    fam = 1.0 if G == n_fam else float(n_fam)
    e2E = np.exp2(E)
    norm = np.maximum(1.0 - e2E.mean(axis=-1, keepdims=True), np.finfo(np.float64).tiny)
    dnorm = -LN2 * (e2E * dE).mean(axis=-1, keepdims=True)
    dg_norm = fam * (-LN2 * e2E * dE / (S * norm) + e2E * dnorm / (S * norm * norm))
    dq_E = d_gE + aux_lin + so_aux[0] + dg_norm
    so_w = e_step_backward_so(*x, wE, zero, *dx)
    rhs_E = dq_E + so_w[0]

    def AG(w_flat):
        w = w_flat.reshape(E.shape)
        return (w - e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, False, w, zero, zero, zero)[0]).reshape(-1)

    dwE_flat, _ = bicgstab(AG, rhs_E.reshape(-1), so["bicgstab_max_iter"], so["bicgstab_tol"],
                           so["bicgstab_breakdown_tol"])
    dwE = dwE_flat.reshape(E.shape)
    lin = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, False, dwE, zero, zero, d_gEbar)
    so_p = e_step_backward_so(*x, wE, acc["g_Ebar"], *dx)
    d_cot = _fold_cotangents(saved, S, G, lin[1] + so_p[1], lin[2] + so_p[2], lin[3] + so_p[3], lin[4] + so_p[4],
                             lin[5] + so_p[5], d_gpD, d_gpS, d_gmt, d_gcol)
    base = e_step_vjp(E, pS_i, pD_i, pL_i, mt_i, col, tree, False, wE, zero, zero, acc["g_Ebar"])
    cot = _fold_cotangents(saved, S, G, base[1], base[2], base[3], base[4], base[5], acc["g_pD"], acc["g_pS"],
                           acc["g_mt"], acc["g_col"])
    cw = np.zeros(S)
    lin_theta, _ = theta_col_vjp(prob, theta, cw, False, *d_cot)
    return lin_theta + theta_head_hvp(prob, theta, uu, *cot[:4])
