"""Pins of the CPU oracle (oracle/kbench_oracle.py) by independent checks.

The reference ships no golden vectors for this path, so every oracle function
is checked against something that does not restate its own formula:

* closed forms (one-node E fixed point, loss of a constant root row);
* brute force in scalar Python on small trees (ancestor / subtree sums, the
  "all non-ancestors" Pibar sum, the E-step on a three-node tree, the split
  enumeration of the DTS term);
* structural identities (leaf initialisation == one general sweep from the
  one-hot leaf row; col-weight shift invariance of the loss);
* derivatives: the analytic J^T of the sweep and the E-step VJP against
  central finite differences of the oracle's own forward maps, the Neumann
  series against a dense-Jacobian series, and the converged gradient of the
  loss against float64 finite differences.

A plausible mistake in the oracle (a dropped term, a swapped child, a wrong
ancestor set, a sign) fails at least one of these.
"""

import dataclasses
import math

import numpy as np
import pytest

import kbench_oracle as O
import kbtest
from kbench import synth


# ----------------------------------------------------------------- helpers
def _helpers_from_parent(parent, c1, c2):
    """state_helpers dict of a small tree (compact levels bottom-up, preorder subtree ranges)."""
    S = len(parent)
    parent = np.asarray(parent)
    kids = {s: [c for c in (c1[s], c2[s]) if 0 <= c < S] for s in range(S)}
    root = int(np.nonzero(parent < 0)[0][0])
    order, stack = [], [root]
    while stack:
        n = stack.pop()
        order.append(n)
        stack.extend(reversed(kids[n]))
    pos = {n: i for i, n in enumerate(order)}
    size = {}
    for n in reversed(order):
        size[n] = 1 + sum(size[c] for c in kids[n])
    depth = {root: 0}
    for n in order:
        for c in kids[n]:
            depth[c] = depth[n] + 1
    internal = [n for n in range(S) if kids[n]]
    by_depth = sorted(internal, key=lambda n: -depth[n])
    levels, ptr = [], [0]
    for d in sorted({depth[n] for n in internal}, reverse=True):
        lv = [n for n in by_depth if depth[n] == d]
        levels.extend(lv)
        ptr.append(len(levels))
    return {
        "S": S, "node_parent": parent.astype(np.int64),
        "node_child1": np.asarray([c if 0 <= c < S else S for c in c1], np.int64),
        "node_child2": np.asarray([c if 0 <= c < S else S for c in c2], np.int64),
        "max_ancestor_depth": 1 + max(depth.values()),
        "node_subtree_start": np.asarray([pos[n] for n in range(S)], np.int64),
        "node_subtree_end": np.asarray([pos[n] + size[n] for n in range(S)], np.int64),
        "compact_level_ptr": np.asarray(ptr, np.int64),
        "compact_level_parents": np.asarray(levels, np.int64),
        "compact_level_child1": np.asarray([c1[n] for n in levels], np.int64),
        "compact_level_child2": np.asarray([c2[n] for n in levels], np.int64),
        "unnorm_row_max": np.zeros(S, np.float32),
    }


def _random_tree(n_leaves, seed):
    p = synth.build_problem(dataclasses.replace(synth.config("tiny"), n_species_leaves=n_leaves, seed=seed))
    return O.Tree.from_helpers(p["static"]["state_helpers"])


def _ancestors(tree, s):
    out = []
    while 0 <= s < tree.S:
        out.append(s)
        s = int(tree.parent[s])
    return out


def _consts(prob, saved):
    S, G = prob.S, 1
    st = lambda x: O.as_item_state(np.asarray(x, dtype=np.float64), S, G)
    E, pS, pD = st(saved["E"]), st(saved["log_pS"]), st(saved["log_pD"])
    return O.WaveConsts(mt=st(saved["max_coupling"]), DL=1.0 + pD + E, Ebar=st(saved["Ebar"]), E=E,
                        SL1=pS + st(saved["E_s2"]), SL2=pS + st(saved["E_s1"]), leaf_logp=pS,
                        col=np.asarray(saved["col_log_probs"], dtype=np.float64),
                        use_col_weights=bool(saved["use_col_weights"]))


def _weighted_tiny():
    """tiny config with non-uniform column weights (exercises the weighted path)."""
    p = kbtest.problem("tiny")
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    cw = np.linspace(-0.7, 0.9, prob.S)
    return p, prob, theta, cw


# ----------------------------------------------------------------- closed forms
def test_e_fixed_point_one_node_closed_form():
    """S = 1: Ebar = -inf, no children, so e = 2^pD e^2 + 2^pL; E = log2 of the smaller root."""
    tree = O.Tree.from_helpers(_helpers_from_parent([-1], [1], [1]))
    pS, pD, pL = np.array([[-0.4]]), np.array([[-2.5]]), np.array([[-1.7]])
    mt, col = np.array([[-1.0]]), np.array([0.0])
    E, Es1, Es2, Eb, _ = O.e_fixed_point(np.array([[-1.0]]), pS, pD, pL, mt, col, tree, False, tol=1e-14)
    a, b = 2.0 ** pD[0, 0], 2.0 ** pL[0, 0]
    e_star = (1.0 - math.sqrt(1.0 - 4.0 * a * b)) / (2.0 * a)
    assert abs(E[0, 0] - math.log2(e_star)) < 1e-12
    assert np.isneginf(Eb[0, 0]) and np.isneginf(Es1[0, 0]) and np.isneginf(Es2[0, 0])


def test_loss_of_constant_root_row():
    """LSE of a constant row c is c + log2 S, so nll = -(c - log2(1 - mean 2^E))."""
    S, c = 9, -3.25
    E = np.full((1, S), -2.0)
    got = O.nll_vector_from_root_rows(np.full((2, S), c), E)
    ref = -(c - math.log2(1.0 - 2.0 ** -2.0))
    assert np.allclose(got, ref, rtol=0, atol=1e-12)


# ----------------------------------------------------------------- brute force on small trees
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_ancestor_and_subtree_sums_brute_force(seed):
    tree = _random_tree(9, seed)
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(3, tree.S))
    anc = tree.ancestor_sum(X)
    sub = tree.subtree_sum(X)
    for s in range(tree.S):
        a = _ancestors(tree, s)
        assert np.allclose(anc[:, s], X[:, a].sum(axis=1), atol=1e-12)
        d = [j for j in range(tree.S) if s in _ancestors(tree, j)]
        assert np.allclose(sub[:, s], X[:, d].sum(axis=1), atol=1e-12)


@pytest.mark.parametrize("weighted", [False, True])
def test_pibar_is_the_non_ancestor_sum(weighted):
    tree = _random_tree(8, 4)
    rng = np.random.default_rng(7)
    Pi = rng.normal(size=(2, tree.S)) * 3 - 5
    Pi[0, 3] = -np.inf
    col = rng.normal(size=tree.S) * 0.5
    mt = rng.normal(size=(2, tree.S))
    got, rmax = O._pibar_from_pi(Pi, col, mt, tree, weighted)
    for r in range(2):
        w = Pi[r] + (col if weighted else 0.0)
        assert rmax[r] == np.max(w)
        for s in range(tree.S):
            keep = [j for j in range(tree.S) if j not in _ancestors(tree, s)]
            tot = sum(2.0 ** w[j] for j in keep)
            ref = math.log2(tot) + mt[r, s] if tot > 0 else -np.inf
            assert (np.isneginf(ref) and np.isneginf(got[r, s])) or abs(got[r, s] - ref) < 1e-11


def test_e_step_three_node_tree_scalar_loop():
    """One E-step on root 2 with leaves 0, 1, per-state parameters, by scalar loops."""
    helpers = _helpers_from_parent([2, 2, -1], [3, 3, 0], [3, 3, 1])
    tree = O.Tree.from_helpers(helpers)
    rng = np.random.default_rng(11)
    E = rng.uniform(-3, -0.5, size=(1, 3))
    pS, pD, pL, mt = (rng.uniform(-4, -0.5, size=(1, 3)) for _ in range(4))
    col = rng.uniform(-1.2, -0.8, size=3)
    anc = {0: {0, 2}, 1: {1, 2}, 2: {2}}
    kids = {0: None, 1: None, 2: (0, 1)}
    for weighted in (False, True):
        En, Es1, Es2, Eb = O.e_step(E, pS, pD, pL, mt, col, tree, weighted)
        for s in range(3):
            w = [E[0, j] + (col[j] if weighted else 0.0) for j in range(3)]
            tot = sum(2.0 ** w[j] for j in range(3) if j not in anc[s])
            ebar = math.log2(tot) + mt[0, s] if tot > 0 else -math.inf
            terms = [pD[0, s] + 2 * E[0, s], E[0, s] + ebar, pL[0, s]]
            if kids[s]:
                a, b = kids[s]
                terms.append(pS[0, s] + E[0, a] + E[0, b])
                assert Es1[0, s] == E[0, a] and Es2[0, s] == E[0, b]
            ref = math.log2(sum(2.0 ** t for t in terms if t != -math.inf))
            assert abs(En[0, s] - ref) < 1e-12
            assert (math.isinf(ebar) and np.isneginf(Eb[0, s])) or abs(Eb[0, s] - ebar) < 1e-12


def test_dts_split_enumeration_scalar_loop():
    """The DTS term of every split row by explicit enumeration of splits and states."""
    p = kbtest.problem("tiny")
    prob, _, saved = kbtest.oracle_forward("tiny")
    Pi, Pb = saved["pi_wave"], saved["pibar_wave"]
    tree = prob.tree
    S = tree.S
    pD = float(np.asarray(saved["log_pD"]).reshape(-1)[0])
    pS = float(np.asarray(saved["log_pS"]).reshape(-1)[0])
    lse = lambda ts: (lambda m: m + math.log2(sum(2.0 ** (t - m) for t in ts)) if m != -math.inf else -math.inf)(
        max(ts))
    for meta in prob.wave_metas:
        if "sl" not in meta:
            continue
        ws, W = int(meta["start"]), int(meta["W"])
        got = O.dts_forward(Pi, Pb, meta, W, np.array(pD), np.array(pS), prob.item_idx, ws, tree)
        sl, sr, red = (np.asarray(meta[k]) for k in ("sl", "sr", "reduce_idx"))
        lsp = np.asarray(meta.get("log_split_probs", np.zeros(len(sl)))).reshape(-1)
        for w in range(W):
            for s in range(S):
                c1, c2 = int(tree.c1[s]), int(tree.c2[s])
                ch = lambda row, c: Pi[row, c] if 0 <= c < S else -math.inf
                terms = []
                for i in np.nonzero(red == w)[0]:
                    l, r = int(sl[i]), int(sr[i])
                    terms += [lsp[i] + pD + Pi[l, s] + Pi[r, s], lsp[i] + Pi[l, s] + Pb[r, s],
                              lsp[i] + Pi[r, s] + Pb[l, s], lsp[i] + pS + ch(l, c1) + ch(r, c2),
                              lsp[i] + pS + ch(r, c1) + ch(l, c2)]
                ref = lse(terms) if terms else -math.inf
                g = got[w, s]
                assert (math.isinf(ref) and np.isneginf(g)) or abs(g - ref) < 1e-10


# ----------------------------------------------------------------- structural identities
def test_leaf_initial_is_one_sweep_from_the_one_hot_row():
    """Leaf init == the general sweep applied to Pi0 = one-hot(leaf) (its Pibar included)."""
    for weighted in (False, True):
        if weighted:
            p, prob, theta, cw = _weighted_tiny()
            _, saved = O.forward(prob, theta, cw)
        else:
            prob, _, saved = kbtest.oracle_forward("tiny")
        co = _consts(prob, saved)
        tree = prob.tree
        leaves = np.nonzero(tree.c1 >= tree.S)[0]
        items = np.zeros(len(leaves), dtype=np.int64)
        Pi0 = np.full((len(leaves), tree.S), -np.inf)
        Pi0[np.arange(len(leaves)), leaves] = co.leaf_logp[0, leaves]
        a = O.leaf_initial(leaves, items, co, tree)
        b = O.wave_sweep(Pi0, items, co, tree, leaf_state=leaves)
        ok, ma, _ = kbtest.compare_inf_safe(a, b)
        assert ok and ma < 1e-12


def test_loss_invariant_to_col_weight_shift():
    p, prob, theta, cw = _weighted_tiny()
    l0, _ = O.forward(prob, theta, cw)
    l1, _ = O.forward(prob, theta, cw + 3.5)
    assert abs(l0 - l1) < 1e-9 * abs(l0)


def test_active_mask_threshold_rule():
    rhs = np.array([[0.0, 1e-6], [-1e-6, 0.0], [0.0, 0.0], [5e-7, -2e-6]])
    assert O.active_mask(rhs, 1e-6, use_pruning=True).tolist() == [True, True, False, True]
    assert O.active_mask(rhs, 1e-6, use_pruning=False).tolist() == [False, False, False, True]


# ----------------------------------------------------------------- derivatives
def _sweep_rows(prob, saved, weighted_rows):
    """(rows, items, leaf_state or None, dts_r or None) for one leaf and one split row of the tiny problem."""
    out = []
    Pi, Pb = saved["pi_wave"], saved["pibar_wave"]
    pD = np.asarray(saved["log_pD"], dtype=np.float64)
    pS = np.asarray(saved["log_pS"], dtype=np.float64)
    for meta in prob.wave_metas:
        ws, W = int(meta["start"]), int(meta["W"])
        rows = np.arange(ws, ws + W)
        items = prob.item_idx[rows]
        if "sl" in meta:
            dts = O.dts_forward(Pi, Pb, meta, W, O.as_item_param(pD, 1, prob.S), O.as_item_param(pS, 1, prob.S),
                                prob.item_idx, ws, prob.tree)
            out.append((rows, items, None, dts))
        else:
            out.append((rows, items, prob.leaf_state[rows], None))
    return out[:weighted_rows]


@pytest.mark.parametrize("weighted", [False, True])
def test_apply_JT_matches_finite_difference_jacobian(weighted):
    if weighted:
        p, prob, theta, cw = _weighted_tiny()
        _, saved = O.forward(prob, theta, cw)
    else:
        prob, _, saved = kbtest.oracle_forward("tiny")
    co = _consts(prob, saved)
    tree = prob.tree
    rng = np.random.default_rng(3)
    h = 1e-6
    for rows, items, leaf, dts in _sweep_rows(prob, saved, 3):
        for k in range(min(3, len(rows))):
            Pi = saved["pi_wave"][rows[k]][None, :].copy()
            it = items[k:k + 1]
            ls = None if leaf is None else leaf[k:k + 1]
            dr = None if dts is None else dts[k:k + 1]
            f = lambda x: O.wave_sweep(x, it, co, tree, leaf_state=ls, dts_r=dr)[0]
            Pb, rmax = O._pibar_from_pi(Pi, co.col, co.mt[it], tree, co.use_col_weights)
            cf = O.self_loop_coeffs(Pi, Pb, rmax, it, co, tree, leaf_state=ls, dts_r=dr)
            finite = np.isfinite(Pi[0])
            J = np.zeros((tree.S, tree.S))
            for j in np.nonzero(finite)[0]:
                xp, xm = Pi.copy(), Pi.copy()
                xp[0, j] += h
                xm[0, j] -= h
                J[:, j] = (f(xp) - f(xm)) / (2 * h)
            term = rng.normal(size=(1, tree.S))
            term[0, ~finite] = 0.0
            got = O.apply_JT(term, cf, tree)[0][finite]
            ref = (J.T @ term[0])[finite]
            assert np.allclose(got, ref, rtol=1e-6, atol=1e-8 * max(1.0, np.abs(ref).max()))


def test_neumann_series_matches_dense_jacobian_series():
    prob, _, saved = kbtest.oracle_forward("tiny")
    co = _consts(prob, saved)
    tree = prob.tree
    h = 1e-6
    rng = np.random.default_rng(9)
    rows, items, leaf, dts = _sweep_rows(prob, saved, 2)[1]  # a split wave
    Pi = saved["pi_wave"][rows]
    Pb, rmax = O._pibar_from_pi(Pi, co.col, co.mt[items], tree, co.use_col_weights)
    rhs = rng.normal(size=Pi.shape)
    rhs[~np.isfinite(Pi)] = 0.0
    n_terms = 4
    v, *_ = O.wave_backward_uniform(Pi, Pb, rmax, rhs, items, co, tree, n_terms,
                                    active=np.ones(len(rows), dtype=bool), dts_r=dts)
    for k in range(len(rows)):
        x0 = Pi[k:k + 1]
        f = lambda x: O.wave_sweep(x, items[k:k + 1], co, tree, dts_r=dts[k:k + 1])[0]
        J = np.zeros((tree.S, tree.S))
        for j in np.nonzero(np.isfinite(x0[0]))[0]:
            xp, xm = x0.copy(), x0.copy()
            xp[0, j] += h
            xm[0, j] -= h
            J[:, j] = (f(xp) - f(xm)) / (2 * h)
        ref, t = rhs[k].copy(), rhs[k].copy()
        for _ in range(n_terms):
            t = J.T @ t
            ref += t
        fin = np.isfinite(x0[0])
        assert np.allclose(v[k][fin], ref[fin], rtol=1e-5, atol=1e-8 * np.abs(ref).max())


def test_e_step_vjp_matches_finite_differences():
    p, prob, theta, cw = _weighted_tiny()
    _, saved = O.forward(prob, theta, cw)
    tree = prob.tree
    S = tree.S
    rng = np.random.default_rng(21)
    E = np.asarray(saved["E"], dtype=np.float64) + rng.normal(scale=0.05, size=(1, S))
    st = lambda x: O.as_item_state(np.asarray(x, dtype=np.float64), S, 1).copy()
    args = [E, st(saved["log_pS"]), st(saved["log_pD"]), st(saved["log_pL"]), st(saved["max_coupling"]),
            np.asarray(saved["col_log_probs"], dtype=np.float64).copy()]
    g = [rng.normal(size=(1, S)) for _ in range(4)]

    def L(a):
        outs = O.e_step(*a, tree, True)
        return sum(float((gi * np.where(np.isfinite(o), o, 0.0)).sum()) for gi, o in zip(g, outs))

    grads = O.e_step_vjp(*args, tree, True, *g)   # (E, pS, pD, pL, mt, col)
    h = 1e-6
    for which, grad in zip((0, 1, 2, 3, 4, 5), grads):
        flat = args[which].reshape(-1)
        gg = np.asarray(grad).reshape(-1)
        for j in range(flat.size):
            ap = [a.copy() for a in args]
            am = [a.copy() for a in args]
            ap[which].reshape(-1)[j] += h
            am[which].reshape(-1)[j] -= h
            fd = (L(ap) - L(am)) / (2 * h)
            assert abs(gg[j] - fd) <= 1e-6 * max(1.0, abs(fd)), (which, j, gg[j], fd)


@pytest.mark.parametrize("weighted", [False, True])
def test_converged_gradient_matches_finite_differences(weighted):
    """grad_theta / grad_col of the converged solve vs central differences of the loss."""
    p = kbtest.problem("tiny")
    prob = O.Problem.from_dict(p)
    prob.so.update(pi_iters=120, neumann_terms=200, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                   bicgstab_tol=1e-13, e_tol=1e-14)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    cw = np.linspace(-0.7, 0.9, prob.S) if weighted else np.zeros(prob.S)
    loss, saved = O.forward(prob, theta, cw)
    gt, gc, _ = O.backward(prob, theta, cw, saved)
    h = 1e-5
    fd = np.zeros_like(theta)
    for idx in np.ndindex(theta.shape):
        tp, tm = theta.copy(), theta.copy()
        tp[idx] += h
        tm[idx] -= h
        fd[idx] = (O.forward(prob, tp, cw)[0] - O.forward(prob, tm, cw)[0]) / (2 * h)
    assert np.abs(gt - fd).max() <= 1e-6 * np.abs(fd).max()
    if weighted:
        fdc = np.zeros_like(cw)
        for j in range(cw.size):
            cp, cm = cw.copy(), cw.copy()
            cp[j] += h
            cm[j] -= h
            fdc[j] = (O.forward(prob, theta, cp)[0] - O.forward(prob, theta, cm)[0]) / (2 * h)
        assert np.abs(gc - fdc).max() <= 1e-6 * np.abs(fdc).max()


def test_converged_gradient_with_single_leaf_families():
    """Families of one gene leaf (root row = leaf row): grad_theta of the converged solve vs central
    differences of the loss."""
    from kbench import synth

    cfg = synth.ProblemConfig(8, 3, n_nni=1, family_leaves_median=3.0, family_leaves_sigma=0.3,
                              family_leaves_max=5, seed=11, single_leaf_families=2)
    p = synth.build_problem(cfg)
    roots = np.asarray(p["static"]["wave_layout"]["root_row_ids"])
    w0 = p["static"]["wave_layout"]["wave_metas"][0]
    assert np.sum(roots < int(w0["start"]) + int(w0["W"])) == 2
    prob = O.Problem.from_dict(p)
    prob.so.update(pi_iters=120, neumann_terms=200, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                   bicgstab_tol=1e-13, e_tol=1e-14)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    cw = np.zeros(prob.S)
    loss, saved = O.forward(prob, theta, cw)
    gt, _gc, _ = O.backward(prob, theta, cw, saved)
    h = 1e-5
    fd = np.zeros_like(theta)
    for idx in np.ndindex(theta.shape):
        tp, tm = theta.copy(), theta.copy()
        tp[idx] += h
        tm[idx] -= h
        fd[idx] = (O.forward(prob, tp, cw)[0] - O.forward(prob, tm, cw)[0]) / (2 * h)
    assert np.abs(gt - fd).max() <= 1e-6 * np.abs(fd).max()
