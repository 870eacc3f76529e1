"""Seeded synthetic problem generator for the log-space solver path.

The reference ships no fixtures (its ``fixtures/`` and ``data/`` are git-ignored,
reference .gitignore:1-6); its frozen glue only consumes a ``static`` namespace
(reference kbench/runtime.py:47-60).  This module builds that contract from a
seed so every test and benchmark input is reproducible:

* a Yule species tree with ``L`` leaves, i.e. ``S = 2L-1`` state columns;
* gene families simulated along it by duplication / transfer / loss with
  per-unit-branch-length rates (transfers go to a uniformly chosen contemporary
  branch);
* every simulated tree plus ``n_nni`` random NNI-perturbed variants, expanded
  into conditional clades and splits with
  ``log_split_probs = log2(freq(split) / freq(clade))``;
* rows (one per distinct clade) grouped into waves by clade size, each wave a
  contiguous row range, chunked to at most ``max_wave_rows`` rows.

Fields and their meaning follow the reference's readers:
``wave_layout`` (reference kbench/core/inference/forward.py:29-117,
kbench/core/kernels/dts_fused.py:171-231), ``state_helpers``
(reference experiments/pristine_kernels/wave_step.py:157-173, 259-263;
e_step.py:52-62; wave_backward.py:479-512) and ``unnorm_row_max``
(reference kbench/core/parameters/extract_parameters.py:25-34, 87-93: the
uniform forward and the ``uniform_fast`` backward agree only when
``unnorm_row_max[s] = -log2(S - |ancestors-or-self(s)|)``).
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass, field

import numpy as np

MAX_WAVE_ROWS = 8192


# ----------------------------------------------------------------------------
# species tree
# ----------------------------------------------------------------------------

@dataclass
class SpeciesTree:
    """Binary rooted ultrametric tree; leaves are 0..L-1, root is S-1.

    Internal node ids are larger than their children's, so id order is a
    topological (children-first) order.
    """

    L: int
    parent: np.ndarray          # [S] int64, -1 at the root
    child1: np.ndarray          # [S] int64, S for "no child"
    child2: np.ndarray          # [S] int64, S for "no child"
    time: np.ndarray            # [S] float64 node time (root = 0, leaves = height)
    depth: np.ndarray = field(default=None)      # [S] edges from the root
    pre: np.ndarray = field(default=None)        # [S] preorder index
    size: np.ndarray = field(default=None)       # [S] nodes in subtree
    n_leaves_below: np.ndarray = field(default=None)

    @property
    def S(self) -> int:
        return int(self.parent.shape[0])

    @property
    def root(self) -> int:
        return self.S - 1


def yule_tree(L: int, rng: np.random.Generator) -> SpeciesTree:
    """Pure-birth (rate 1 per lineage) tree grown until it has ``L`` lineages."""
    if L < 1:
        raise ValueError("L must be >= 1")
    S = 2 * L - 1
    # lineage = (parent internal node creation index or -1, start time)
    created_parent: list[int] = []    # per internal creation index: parent creation index
    created_time: list[float] = []
    created_children: list[list[tuple[str, int]]] = []
    t = 0.0
    if L == 1:
        parent = np.array([-1], dtype=np.int64)
        c = np.array([S], dtype=np.int64)
        return _finish_tree(SpeciesTree(1, parent, c.copy(), c.copy(), np.zeros(1)))
    created_parent.append(-1)
    created_time.append(0.0)
    created_children.append([])
    active = [0, 0]  # lineages hanging below creation index 0
    while len(active) < L:
        t += rng.exponential(1.0 / len(active))
        i = int(rng.integers(len(active)))
        par = active.pop(i)
        idx = len(created_time)
        created_parent.append(par)
        created_time.append(t)
        created_children.append([])
        created_children[par].append(("i", idx))
        active.extend([idx, idx])
    t_end = t + rng.exponential(1.0 / len(active))
    # leaves get ids 0..L-1 in the order of the active list
    leaf_parent = list(active)
    for leaf_id, par in enumerate(leaf_parent):
        created_children[par].append(("l", leaf_id))
    n_int = len(created_time)
    assert n_int == L - 1
    # internal creation index k -> node id L + (n_int - 1 - k); root (k=0) -> S-1
    def int_id(k: int) -> int:
        return L + (n_int - 1 - k)

    parent = np.full(S, -1, dtype=np.int64)
    child1 = np.full(S, S, dtype=np.int64)
    child2 = np.full(S, S, dtype=np.int64)
    time = np.zeros(S, dtype=np.float64)
    for k in range(n_int):
        nid = int_id(k)
        time[nid] = created_time[k]
        kids = []
        for kind, v in created_children[k]:
            kids.append(int_id(v) if kind == "i" else v)
        assert len(kids) == 2
        child1[nid], child2[nid] = kids
        for kid in kids:
            parent[kid] = nid
    time[:L] = t_end
    return _finish_tree(SpeciesTree(L, parent, child1, child2, time))


def _finish_tree(tree: SpeciesTree) -> SpeciesTree:
    S = tree.S
    depth = np.zeros(S, dtype=np.int64)
    for v in range(S - 2, -1, -1):  # parents have larger ids
        depth[v] = depth[tree.parent[v]] + 1
    pre = np.zeros(S, dtype=np.int64)
    size = np.ones(S, dtype=np.int64)
    nlb = np.zeros(S, dtype=np.int64)
    nlb[: tree.L] = 1
    for v in range(S):  # children before parents
        for c in (tree.child1[v], tree.child2[v]):
            if c < S:
                size[v] += size[c]
                nlb[v] += nlb[c]
    order = 0
    stack = [S - 1]
    while stack:
        v = stack.pop()
        pre[v] = order
        order += 1
        for c in (tree.child2[v], tree.child1[v]):
            if c < S:
                stack.append(c)
    tree.depth, tree.pre, tree.size, tree.n_leaves_below = depth, pre, size, nlb
    return tree


def state_helpers_from_tree(tree: SpeciesTree) -> dict:
    """The ``state_helpers`` dict the glue passes to every kernel wrapper."""
    S = tree.S
    anc_count = tree.depth + 1  # ancestors-or-self
    with np.errstate(divide="ignore"):
        unnorm_row_max = -np.log2((S - anc_count).astype(np.float64))
    internal = np.nonzero(tree.child1 < S)[0]
    # internal nodes grouped by depth, deepest level first (bottom-up order)
    levels = sorted(set(int(d) for d in tree.depth[internal]), reverse=True)
    ptr = [0]
    parents, c1s, c2s = [], [], []
    for d in levels:
        nodes = np.sort(internal[tree.depth[internal] == d])
        parents.extend(nodes.tolist())
        c1s.extend(tree.child1[nodes].tolist())
        c2s.extend(tree.child2[nodes].tolist())
        ptr.append(len(parents))
    return {
        "S": S,
        "node_parent": tree.parent.copy(),
        "node_child1": tree.child1.copy(),
        "node_child2": tree.child2.copy(),
        "max_ancestor_depth": int(anc_count.max()),
        "node_subtree_start": tree.pre.copy(),
        "node_subtree_end": (tree.pre + tree.size).astype(np.int64),
        "compact_level_ptr": np.asarray(ptr, dtype=np.int64),
        "compact_level_parents": np.asarray(parents, dtype=np.int64),
        "compact_level_child1": np.asarray(c1s, dtype=np.int64),
        "compact_level_child2": np.asarray(c2s, dtype=np.int64),
        "unnorm_row_max": unnorm_row_max,
    }


# ----------------------------------------------------------------------------
# DTL gene-family simulation
# ----------------------------------------------------------------------------

class _GeneNode:
    __slots__ = ("kids", "species")

    def __init__(self, kids=None, species=-1):
        self.kids = kids
        self.species = species


def _join(a, b):
    if a is None:
        return b
    if b is None:
        return a
    return _GeneNode(kids=(a, b))


def simulate_family(tree: SpeciesTree, origin: int, rates: tuple[float, float, float],
                    rng: np.random.Generator, max_nodes: int = 200000):
    """Simulate one gene lineage starting on the branch above species ``origin``.

    Returns the gene tree root (``_GeneNode``) or ``None`` if every copy was lost.
    """
    d, tr, l = rates
    total = d + tr + l
    S = tree.S
    t_par = np.where(tree.parent >= 0, tree.time[np.maximum(tree.parent, 0)], -np.inf)
    budget = [max_nodes]

    def contemporaries(t: float, exclude: int) -> np.ndarray:
        alive = (t_par < t) & (tree.time >= t)
        alive[exclude] = False
        return np.nonzero(alive)[0]

    def sim(branch: int, t: float):
        budget[0] -= 1
        if budget[0] < 0:
            raise RuntimeError("family simulation exceeded node budget")
        while True:
            dt = rng.exponential(1.0 / total) if total > 0 else math.inf
            if t + dt >= tree.time[branch]:
                if tree.child1[branch] >= S:
                    return _GeneNode(species=int(branch))
                return _join(sim(int(tree.child1[branch]), float(tree.time[branch])),
                             sim(int(tree.child2[branch]), float(tree.time[branch])))
            t += dt
            u = rng.random() * total
            if u < d:
                return _join(sim(branch, t), sim(branch, t))
            if u < d + tr:
                cands = contemporaries(t, branch)
                if cands.size == 0:
                    continue
                recip = int(cands[rng.integers(cands.size)])
                return _join(sim(branch, t), sim(recip, t))
            return None

    if tree.parent[origin] < 0:
        start = float(tree.time[origin])
    else:
        start = 0.5 * (float(tree.time[tree.parent[origin]]) + float(tree.time[origin]))
    return sim(int(origin), start)


def _gene_tree_arrays(root: _GeneNode):
    """Flatten a gene tree: leaf species list and internal nodes as (left, right) node ids.

    Leaves get ids 0..k-1 (gene leaf index), internal nodes k..2k-2, root last.
    """
    leaves: list[_GeneNode] = []
    order: list[_GeneNode] = []
    stack = [(root, False)]
    while stack:
        node, done = stack.pop()
        if node.kids is None:
            leaves.append(node)
            continue
        if done:
            order.append(node)
        else:
            stack.append((node, True))
            stack.append((node.kids[1], False))
            stack.append((node.kids[0], False))
    ids = {id(n): i for i, n in enumerate(leaves)}
    k = len(leaves)
    for j, n in enumerate(order):
        ids[id(n)] = k + j
    kids = np.array([[ids[id(n.kids[0])], ids[id(n.kids[1])]] for n in order], dtype=np.int64).reshape(-1, 2)
    species = np.array([n.species for n in leaves], dtype=np.int64)
    return species, kids


def _clades_and_splits(k: int, kids: np.ndarray):
    """Clade bitmasks of a gene tree (``kids[j]`` are the children of node k+j)."""
    n_int = kids.shape[0]
    mask = [1 << i for i in range(k)] + [0] * n_int
    # children-first order by iterative DFS from the root (NNI moves break id order)
    order = []
    stack = [(k + n_int - 1, False)]
    while stack:
        v, done = stack.pop()
        if v < k:
            continue
        if done:
            order.append(v)
        else:
            stack.append((v, True))
            stack.append((int(kids[v - k, 0]), False))
            stack.append((int(kids[v - k, 1]), False))
    splits = []
    for v in order:
        a, b = int(kids[v - k, 0]), int(kids[v - k, 1])
        mask[v] = mask[a] | mask[b]
        lo, hi = (mask[a], mask[b]) if mask[a] < mask[b] else (mask[b], mask[a])
        splits.append((mask[v], lo, hi))
    return mask, splits


def _nni(k: int, kids: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    """One random NNI on a rooted binary tree: swap a grandchild with its uncle."""
    n_int = kids.shape[0]
    if n_int < 2:
        return kids.copy()
    par = np.full(k + n_int, -1, dtype=np.int64)
    for j in range(n_int):
        par[kids[j, 0]] = k + j
        par[kids[j, 1]] = k + j
    root = k + n_int - 1
    cand = [k + j for j in range(n_int) if k + j != root]
    v = cand[int(rng.integers(len(cand)))]
    u = int(par[v])
    new = kids.copy()
    urow = u - k
    vrow = v - k
    w_pos = 0 if new[urow, 1] == v else 1          # position of the sibling w in u
    a_pos = int(rng.integers(2))                   # which child of v moves up
    w = int(new[urow, w_pos])
    a = int(new[vrow, a_pos])
    new[urow, w_pos] = a
    new[vrow, a_pos] = w
    return new


# ----------------------------------------------------------------------------
# layout assembly
# ----------------------------------------------------------------------------

@dataclass
class ProblemConfig:
    """Knobs of one synthetic problem (see the five configs in BASELINE terms)."""

    n_species_leaves: int
    n_families: int
    n_nni: int = 0
    rates: tuple[float, float, float] = (0.1, 0.1, 0.2)
    family_leaves_median: float = 10.0
    family_leaves_sigma: float = 0.6
    family_leaves_max: int = 2000
    statewise: bool = False
    seed: int = 0
    max_wave_rows: int = MAX_WAVE_ROWS
    solver_options: dict = field(default_factory=dict)
    # families of one gene leaf (their root row is a leaf row), appended after
    # the simulated ones from a separate random stream
    single_leaf_families: int = 0
    # one parameter row per family (item): theta [n_families, 3], every clade
    # row reads its family's rates (rate_item_idx = the row's family); global
    # rates only, as the reference's extraction defines no per-item per-state
    # layout
    itemwise: bool = False


def build_problem(cfg: ProblemConfig) -> dict:
    """Generate a whole problem: ``{"meta", "static", "inputs"}`` with numpy arrays.

    ``static`` mirrors what the reference's ``make_static`` receives
    (reference kbench/runtime.py:47-60): ``wave_layout``, ``state_helpers``,
    ``rate_item_idx``, ``itemwise``, ``statewise``.
    """
    if cfg.itemwise and cfg.statewise:
        raise ValueError("itemwise problems take one global rate row per item (statewise=False)")
    rng = np.random.default_rng(cfg.seed)
    tree = yule_tree(cfg.n_species_leaves, rng)
    S = tree.S
    helpers = state_helpers_from_tree(tree)

    families = []
    tries = 0
    while len(families) < cfg.n_families:
        tries += 1
        if tries > 200 * cfg.n_families + 1000:
            raise RuntimeError("could not simulate enough families")
        target = float(np.exp(np.log(cfg.family_leaves_median) + cfg.family_leaves_sigma * rng.standard_normal()))
        target = min(max(target, 2.0), float(cfg.family_leaves_max))
        nlb = tree.n_leaves_below
        near = np.nonzero((nlb >= target / 1.5) & (nlb <= target * 1.5))[0]
        if near.size == 0:
            near = np.array([int(np.argmin(np.abs(nlb - target)))])
        origin = int(near[rng.integers(near.size)])
        try:
            g = simulate_family(tree, origin, cfg.rates, rng)
        except RuntimeError:
            continue
        if g is None or g.kids is None:
            continue
        species, kids = _gene_tree_arrays(g)
        k = species.shape[0]
        if k < 2 or k > cfg.family_leaves_max:
            continue
        trees = [kids]
        for _ in range(cfg.n_nni):
            trees.append(_nni(k, kids, rng))
        families.append((species, trees))

    if cfg.single_leaf_families > 0:
        rng1 = np.random.default_rng(cfg.seed + 7919)
        n_sp = cfg.n_species_leaves
        leaf_species = np.nonzero(tree.n_leaves_below == 1)[0] if hasattr(tree, "n_leaves_below") else np.arange(n_sp)
        for _ in range(cfg.single_leaf_families):
            sp = int(leaf_species[rng1.integers(leaf_species.size)])
            families.append((np.array([sp], dtype=np.int64), [np.zeros((0, 2), dtype=np.int64)] * (1 + cfg.n_nni)))

    # clades / splits per family
    fam_rows = []   # per family: list of (size, mask) sorted
    fam_splits = []  # per family: dict parent_mask -> list of (lo, hi, log2 prob)
    for species, trees in families:
        k = species.shape[0]
        clade_freq: dict[int, int] = {}
        split_freq: dict[tuple[int, int, int], int] = {}
        for kids in trees:
            mask, splits = _clades_and_splits(k, kids)
            for m in set(mask):
                clade_freq[m] = clade_freq.get(m, 0) + 1
            for sp in splits:
                split_freq[sp] = split_freq.get(sp, 0) + 1
        by_parent: dict[int, list] = {}
        for (pm, lo, hi), f in sorted(split_freq.items()):
            by_parent.setdefault(pm, []).append((lo, hi, math.log2(f / clade_freq[pm])))
        fam_rows.append(sorted(clade_freq.keys(), key=lambda m: (bin(m).count("1"), m)))
        fam_splits.append(by_parent)

    # global row order: by clade size, then family, then mask
    entries = []
    for f, rows in enumerate(fam_rows):
        for m in rows:
            entries.append((bin(m).count("1"), f, m))
    entries.sort()
    C = len(entries)
    row_of = {(f, m): i for i, (_, f, m) in enumerate(entries)}
    item_idx = np.array([f for (_, f, _) in entries], dtype=np.int64)
    leaf_state = np.full(C, -1, dtype=np.int64)
    for i, (sz, f, m) in enumerate(entries):
        if sz == 1:
            leaf_state[i] = families[f][0][m.bit_length() - 1]
    n_fam = len(families)
    root_row_ids = np.array([row_of[(f, (1 << families[f][0].shape[0]) - 1)] for f in range(n_fam)],
                            dtype=np.int64)

    wave_metas = []
    start = 0
    while start < C:
        size = entries[start][0]
        end = start
        while end < C and entries[end][0] == size and end - start < cfg.max_wave_rows:
            end += 1
        W = end - start
        meta = {"start": start, "W": W}
        if size > 1:
            eq1, ge2 = [], []
            for w in range(W):
                _, f, m = entries[start + w]
                sp = fam_splits[f][m]
                rows = [(row_of[(f, lo)], row_of[(f, hi)], lp) for lo, hi, lp in sp]
                (eq1 if len(rows) == 1 else ge2).append((w, rows))
            sl, sr, red, lsp = [], [], [], []
            for w, rows in eq1:
                for a, b, lp in rows:
                    sl.append(a); sr.append(b); red.append(w); lsp.append(lp)
            n_eq1 = len(sl)
            ge2_ptr = [0]
            ge2_parent = []
            for w, rows in ge2:
                for a, b, lp in rows:
                    sl.append(a); sr.append(b); red.append(w); lsp.append(lp)
                ge2_ptr.append(len(sl) - n_eq1)
                ge2_parent.append(w)
            meta.update({
                "sl": np.asarray(sl, dtype=np.int64),
                "sr": np.asarray(sr, dtype=np.int64),
                "reduce_idx": np.asarray(red, dtype=np.int64),
                "log_split_probs": np.asarray(lsp, dtype=np.float64),
                "n_eq1": n_eq1,
                "eq1_reduce_idx": np.asarray(red[:n_eq1], dtype=np.int64),
                "ge2_ptr": np.asarray(ge2_ptr, dtype=np.int64),
                "ge2_parent_ids": np.asarray(ge2_parent, dtype=np.int64),
                "ge2_max_fanout": int(max([p1 - p0 for p0, p1 in zip(ge2_ptr[:-1], ge2_ptr[1:])], default=0)),
            })
        wave_metas.append(meta)
        start = end

    wave_layout = {
        "leaf_state_index": leaf_state,
        "root_row_ids": root_row_ids,
        "item_idx": item_idx,
        "wave_metas": wave_metas,
    }
    theta_shape = (n_fam, 3) if cfg.itemwise else ((S, 3) if cfg.statewise else (3,))
    theta = rng.uniform(-3.0, -1.0, size=theta_shape)
    col_weights = np.zeros(S, dtype=np.float64)
    so = {"pi_iters": 16, "neumann_terms": 16, "e_tol": 1e-8}
    so.update(cfg.solver_options)
    return {
        "meta": {"S": S, "C": C, "n_items": n_fam, "solver_options": so},
        "static": {
            "wave_layout": wave_layout,
            "state_helpers": helpers,
            "rate_item_idx": item_idx.copy() if cfg.itemwise else np.zeros(C, dtype=np.int64),
            "itemwise": bool(cfg.itemwise),
            "statewise": bool(cfg.statewise),
        },
        "inputs": {"theta": theta, "col_weights": col_weights},
        "tree": tree,
    }


# ----------------------------------------------------------------------------
# named configurations
# ----------------------------------------------------------------------------

def config(name: str | int) -> ProblemConfig:
    """The five BASELINE configurations (plus ``tiny`` for brute-force tests)."""
    key = str(name)
    if key in ("1", "config1"):
        return ProblemConfig(64, 20, n_nni=0, family_leaves_median=11.0, family_leaves_sigma=0.5,
                             family_leaves_max=40, seed=1)
    if key in ("2", "config2"):
        return ProblemConfig(256, 100, n_nni=3, family_leaves_median=14.0, family_leaves_sigma=0.5,
                             family_leaves_max=120, seed=2, solver_options={"e_tol": 1e-6})
    if key in ("3", "config3", "5", "config5"):
        return ProblemConfig(1024, 500, n_nni=3, family_leaves_median=21.0, family_leaves_sigma=0.9,
                             family_leaves_max=320, statewise=True, seed=3)
    if key in ("4", "config4"):
        return ProblemConfig(4096, 3000, n_nni=3, family_leaves_median=30.0, family_leaves_sigma=1.0,
                             family_leaves_max=2000, statewise=True, seed=4)
    if key == "tiny":
        return ProblemConfig(4, 3, n_nni=1, family_leaves_median=3.0, family_leaves_sigma=0.3,
                             family_leaves_max=5, seed=7, solver_options={"pi_iters": 4, "neumann_terms": 3})
    raise KeyError(f"unknown config {name!r}")


def layout_digest(problem: dict) -> str:
    """SHA-256 over every array of the static layout (pins generator determinism)."""
    h = hashlib.sha256()

    def feed(name, v):
        h.update(name.encode())
        if isinstance(v, np.ndarray):
            h.update(str(v.dtype).encode())
            h.update(np.ascontiguousarray(v).tobytes())
        else:
            h.update(repr(v).encode())

    st = problem["static"]
    for k in sorted(st["state_helpers"]):
        feed("sh/" + k, st["state_helpers"][k])
    wl = st["wave_layout"]
    for k in ("leaf_state_index", "root_row_ids", "item_idx"):
        feed("wl/" + k, wl[k])
    for i, m in enumerate(wl["wave_metas"]):
        for k in sorted(m):
            feed(f"w{i}/{k}", m[k])
    feed("theta", np.asarray(problem["inputs"]["theta"]))
    return h.hexdigest()


def summary(problem: dict) -> dict:
    wl = problem["static"]["wave_layout"]
    n_splits = sum(int(m["sl"].shape[0]) for m in wl["wave_metas"] if "sl" in m)
    return {
        "S": problem["meta"]["S"],
        "C": problem["meta"]["C"],
        "n_families": problem["meta"]["n_items"],
        "n_waves": len(wl["wave_metas"]),
        "n_splits": n_splits,
        "max_wave_rows": max(m["W"] for m in wl["wave_metas"]),
        "max_ancestor_depth": problem["static"]["state_helpers"]["max_ancestor_depth"],
    }


def family_subset(problem: dict, families) -> dict:
    """The problem restricted to ``families`` (family ids, in order): same tree, theta and options.

    Rows of other families are dropped and the kept rows renumbered in their
    order; waves keep their order and lose their dropped rows (empty waves
    vanish); every kept parent keeps all of its splits, so the eq1-first /
    ge2-grouped split order survives and its offsets are recomputed.  Rows of
    different families never interact, so a solve over the subset is the
    solve of those families alone (the loss and gradients of a whole problem
    are the sums over a partition of its families).
    """
    if problem["static"]["itemwise"]:
        raise ValueError("family_subset takes problems with one parameter row (itemwise=False)")
    fams = [int(f) for f in families]
    wl = problem["static"]["wave_layout"]
    item = np.asarray(wl["item_idx"])
    pos = {f: i for i, f in enumerate(fams)}
    keep = np.isin(item, np.asarray(fams, dtype=item.dtype))
    new_id = np.cumsum(keep) - 1  # new row id of a kept row
    metas = []
    for m in wl["wave_metas"]:
        s0, W = int(m["start"]), int(m["W"])
        kw = keep[s0:s0 + W]
        if not kw.any():
            continue
        local = np.cumsum(kw) - 1  # new wave-local index of a kept row
        meta = {"start": int(new_id[s0:s0 + W][kw][0]), "W": int(kw.sum())}
        if "sl" in m:
            red = np.asarray(m["reduce_idx"])
            on = kw[red]
            n_eq1 = int(m["n_eq1"])
            ge2_ptr = np.asarray(m["ge2_ptr"])
            ge2_parent = np.asarray(m["ge2_parent_ids"])
            new_ptr, new_parent = [0], []
            for g in range(ge2_parent.shape[0]):
                if kw[ge2_parent[g]]:
                    new_ptr.append(new_ptr[-1] + int(ge2_ptr[g + 1] - ge2_ptr[g]))
                    new_parent.append(int(local[ge2_parent[g]]))
            sel_red = local[red[on]]
            n_eq1_new = int(on[:n_eq1].sum())
            meta.update({
                "sl": new_id[np.asarray(m["sl"])[on]].astype(np.int64),
                "sr": new_id[np.asarray(m["sr"])[on]].astype(np.int64),
                "reduce_idx": sel_red.astype(np.int64),
                "log_split_probs": np.asarray(m["log_split_probs"])[on],
                "n_eq1": n_eq1_new,
                "eq1_reduce_idx": sel_red[:n_eq1_new].astype(np.int64),
                "ge2_ptr": np.asarray(new_ptr, dtype=np.int64),
                "ge2_parent_ids": np.asarray(new_parent, dtype=np.int64),
                "ge2_max_fanout": int(max(np.diff(new_ptr), default=0)),
            })
        metas.append(meta)
    roots = np.asarray(wl["root_row_ids"])
    st = problem["static"]
    C = int(keep.sum())
    out = {
        "meta": dict(problem["meta"], C=C, n_items=len(fams)),
        "static": {
            "wave_layout": {
                "leaf_state_index": np.asarray(wl["leaf_state_index"])[keep],
                "root_row_ids": new_id[roots[fams]].astype(np.int64),
                "item_idx": np.asarray([pos[int(f)] for f in item[keep]], dtype=np.int64),
                "wave_metas": metas,
            },
            "state_helpers": st["state_helpers"],
            "rate_item_idx": np.zeros(C, dtype=np.int64),
            "itemwise": st["itemwise"],
            "statewise": st["statewise"],
        },
        "inputs": problem["inputs"],
    }
    if "tree" in problem:
        out["tree"] = problem["tree"]
    return out


def _host(x):
    """A layout field as a numpy array (device tensors are copied to the host)."""
    if hasattr(x, "detach"):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def _splits_by_parent(wl: dict, C: int) -> list:
    """Row -> [(child l, child r, split log-probability)] in stored split order."""
    splits_of = [[] for _ in range(C)]
    for m in wl["wave_metas"]:
        if "sl" not in m:
            continue
        s0 = int(m["start"])
        sl, sr, red = _host(m["sl"]), _host(m["sr"]), _host(m["reduce_idx"])
        lsp = m.get("log_split_probs")
        lsp = np.zeros(len(sl)) if lsp is None else _host(lsp).reshape(-1)
        for a, b, w, p in zip(sl, sr, red, lsp):
            splits_of[s0 + int(w)].append((int(a), int(b), float(p)))
    return splits_of


def _level_metas(level: np.ndarray, splits: list, cap: int, lsp_dtype=np.float64) -> list:
    """Wave metas of rows already numbered by level: one wave per level (chunked to ``cap`` rows).

    ``splits[r]`` lists row r's splits with children in the same numbering; a
    level-0 wave has no split fields, every other wave lists its parents'
    splits, parents with one split first (``eq1``), then the others (``ge2``).
    """
    C = int(level.shape[0])
    metas = []
    start = 0
    while start < C:
        lv = level[start]
        end = start
        while end < C and level[end] == lv and end - start < cap:
            end += 1
        W = end - start
        meta = {"start": start, "W": W}
        if lv > 0:
            eq1, ge2 = [], []
            for w in range(W):
                sp = splits[start + w]
                (eq1 if len(sp) == 1 else ge2).append((w, sp))
            sl, sr, red, lsp = [], [], [], []
            for w, sp in eq1:
                for a, b, p in sp:
                    sl.append(a); sr.append(b); red.append(w); lsp.append(p)
            n_eq1 = len(sl)
            ge2_ptr, ge2_parent = [0], []
            for w, sp in ge2:
                for a, b, p in sp:
                    sl.append(a); sr.append(b); red.append(w); lsp.append(p)
                ge2_ptr.append(len(sl) - n_eq1)
                ge2_parent.append(w)
            meta.update({
                "sl": np.asarray(sl, dtype=np.int64),
                "sr": np.asarray(sr, dtype=np.int64),
                "reduce_idx": np.asarray(red, dtype=np.int64),
                "log_split_probs": np.asarray(lsp, dtype=lsp_dtype),
                "n_eq1": n_eq1,
                "eq1_reduce_idx": np.asarray(red[:n_eq1], dtype=np.int64),
                "ge2_ptr": np.asarray(ge2_ptr, dtype=np.int64),
                "ge2_parent_ids": np.asarray(ge2_parent, dtype=np.int64),
                "ge2_max_fanout": int(max(np.diff(ge2_ptr), default=0)),
            })
        metas.append(meta)
        start = end
    return metas


def level_waves(problem: dict, max_wave_rows: int | None = None) -> tuple[dict, np.ndarray]:
    """The same problem with its rows regrouped into one wave per clade-DAG level -> (problem, new_of_old).

    A row's level is 0 without splits, else one more than the highest level
    among its splits' children.  Rows are renumbered by (level, old row id);
    each level becomes one wave (chunked to ``max_wave_rows`` if given), in
    increasing level.  Every row keeps its splits (eq1 parents first, then the
    ge2 parents, each parent's splits in their old order), its leaf state, its
    item and root status.  Since a row of the truncated forward and of its
    adjoint depends only on its own children, which lie on lower levels, every
    row's result is the same as under the size waves (summation order across
    parents aside); only the number of waves (wrapper calls and launches per
    solve) changes: 144 -> 19 at config 3.  ``new_of_old[r]`` is the new id
    of old row r (row-indexed outputs map back with ``out[new_of_old]``).
    """
    wl = problem["static"]["wave_layout"]
    C = int(np.asarray(wl["leaf_state_index"]).shape[0])
    splits_of = _splits_by_parent(wl, C)
    level = np.zeros(C, dtype=np.int64)
    for m in wl["wave_metas"]:  # waves are in dependency order: children first
        s0, W = int(m["start"]), int(m["W"])
        for r in range(s0, s0 + W):
            if splits_of[r]:
                level[r] = 1 + max(max(level[a], level[b]) for a, b, _ in splits_of[r])
    order = np.lexsort((np.arange(C), level))  # new -> old
    new_of_old = np.empty(C, dtype=np.int64)
    new_of_old[order] = np.arange(C)
    cap = int(max_wave_rows) if max_wave_rows else C
    splits_new = [[(int(new_of_old[a]), int(new_of_old[b]), p) for a, b, p in splits_of[int(o)]] for o in order]
    metas = _level_metas(level[order], splits_new, cap)
    st = problem["static"]
    out = {
        "meta": dict(problem["meta"]),
        "static": {
            "wave_layout": {
                "leaf_state_index": np.asarray(wl["leaf_state_index"])[order],
                "root_row_ids": new_of_old[np.asarray(wl["root_row_ids"])].astype(np.int64),
                "item_idx": np.asarray(wl["item_idx"])[order],
                "wave_metas": metas,
            },
            "state_helpers": st["state_helpers"],
            "rate_item_idx": np.asarray(st["rate_item_idx"])[order],
            "itemwise": st["itemwise"],
            "statewise": st["statewise"],
        },
        "inputs": problem["inputs"],
    }
    if "tree" in problem:
        out["tree"] = problem["tree"]
    return out, new_of_old


def row_classes(wave_layout: dict, rate_item_idx, active=None) -> tuple[dict, np.ndarray, np.ndarray]:
    """Rows that compute the same values, one row per class -> (class layout, class_of_row, rep_of_class).

    Two rows share a class when they have the same parameter row
    (``rate_item_idx``) and the same wave kind (split or leaf wave, and its
    ``phase``), and either both are leaf-wave rows with the same leaf state, or
    both are split rows whose splits, as (class of one child, class of the
    other, split log-probability) with the two children unordered, form the
    same multiset.  By induction from the leaves, rows of one class have the
    same truncated forward rows (Pi, Pibar, row maxima, split term) and the
    same forward tangents: the only differences are the order in which a
    row's splits are merged.  With ``active`` (one flag per row, e.g. the
    backward's active mask at a point), the flag is part of the key as well,
    so that every member of a class has the same flag and so do the children
    of every member along each split: the adjoint maps of all members of a
    class are then one linear map, applied to each member's own right-hand
    side.

    The class layout is a wave layout whose rows are the classes: class c is
    row c, numbered by (level, first member); one wave per level as
    ``level_waves`` builds them; each class row has the leaf state and the
    splits (children mapped to their classes, in the representative's order)
    of its representative, the first member in row order of the layout's
    waves.  ``root_row_ids`` maps every family's root row to its class (two
    families with equal root rows share one).
    """
    wl = wave_layout
    leaf = _host(wl["leaf_state_index"]).astype(np.int64)
    C = int(leaf.shape[0])
    item = _host(rate_item_idx).astype(np.int64).reshape(-1)
    if item.shape[0] == 1 and C != 1:
        item = np.broadcast_to(item, (C,))
    act = None if active is None else _host(active).astype(bool).reshape(-1)
    splits_of = _splits_by_parent(wl, C)
    cls = np.full(C, -1, dtype=np.int64)
    ids: dict = {}
    reps, level = [], []
    for m in wl["wave_metas"]:  # children first
        s0, W = int(m["start"]), int(m["W"])
        split_wave = "sl" in m
        phase = m.get("phase")
        phase = None if phase is None else int(phase)
        for r in range(s0, s0 + W):
            flag = True if act is None else bool(act[r])
            if split_wave:
                body = tuple(sorted((min(cls[a], cls[b]), max(cls[a], cls[b]), p) for a, b, p in splits_of[r]))
            else:
                body = int(leaf[r])
            key = (split_wave, phase, int(item[r]), flag, body)
            c = ids.get(key)
            if c is None:
                c = ids[key] = len(reps)
                reps.append(r)
                level.append(1 + max(max(level[cls[a]], level[cls[b]]) for a, b, _ in splits_of[r])
                             if split_wave and splits_of[r] else 0)
            cls[r] = c
    if (cls < 0).any():
        raise ValueError("the wave layout does not cover every row")
    reps = np.asarray(reps, dtype=np.int64)
    level = np.asarray(level, dtype=np.int64)
    Cc = int(reps.shape[0])
    order = np.lexsort((reps, level))  # new class id -> old class id
    new_of = np.empty(Cc, dtype=np.int64)
    new_of[order] = np.arange(Cc)
    rep = reps[order]
    lsp_dtype = np.float64
    for m in wl["wave_metas"]:
        if "sl" in m and m.get("log_split_probs") is not None:
            lsp_dtype = _host(m["log_split_probs"]).dtype
            break
    splits_new = [[(int(new_of[cls[a]]), int(new_of[cls[b]]), p) for a, b, p in splits_of[int(r)]] for r in rep]
    layout = {
        "leaf_state_index": leaf[rep],
        "root_row_ids": new_of[cls[_host(wl["root_row_ids"]).astype(np.int64)]],
        "item_idx": _host(wl["item_idx"])[rep],
        "wave_metas": _level_metas(level[order], splits_new, Cc, lsp_dtype),
    }
    return layout, new_of[cls], rep
