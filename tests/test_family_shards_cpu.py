"""Family shards of a problem: the layout subset is exact, and a solve is the sum over a partition.

Rows of different families never interact (every split's children belong to
its parent's family), so the loss and the gradients of a whole problem are the
sums of those of its family shards -- the decomposition the CPU baseline uses
across host cores and a multi-GPU run would use across GPUs.  Pinned here with
the float64 oracle.
"""

import numpy as np
import pytest

import kbench_oracle as O
import kbtest
from kbench import synth


def test_subset_of_every_family_is_the_problem():
    p = kbtest.problem("1")
    q = synth.family_subset(p, range(p["meta"]["n_items"]))
    assert synth.layout_digest(q) == synth.layout_digest(p)


def _solve(p):
    prob = O.Problem.from_dict(p)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    loss, saved = O.forward(prob, th, cw)
    gt, gc, _ = O.backward(prob, th, cw, saved)
    return loss, gt, gc


@pytest.mark.parametrize("name,statewise", [("1", None), ("1", True)])
def test_solve_is_the_sum_over_family_shards(name, statewise):
    p = kbtest.problem(name, statewise)
    # the E adjoint is a linear solve: additive over shards once solved tightly
    so = dict(p["meta"]["solver_options"], bicgstab_tol=1e-14)
    p = dict(p, meta=dict(p["meta"], solver_options=so))
    n = p["meta"]["n_items"]
    shards = [list(range(0, n, 3)), list(range(1, n, 3)), list(range(2, n, 3))]
    parts = [_solve(synth.family_subset(p, fams)) for fams in shards]
    loss, gt, gc = _solve(p)
    assert abs(sum(x[0] for x in parts) - loss) <= 1e-10 * abs(loss)
    for i, full in ((1, gt), (2, gc)):
        tot = sum(x[i] for x in parts)
        assert np.abs(tot - full).max() <= 1e-9 * np.abs(full).max()
    for fams in shards:  # the shard layouts are well formed: splits point to earlier waves of kept rows
        wl = synth.family_subset(p, fams)["static"]["wave_layout"]
        for m in wl["wave_metas"]:
            if "sl" in m:
                assert (np.asarray(m["sl"]) < m["start"]).all() and (np.asarray(m["sr"]) < m["start"]).all()
                assert int(m["n_eq1"]) == len(m["eq1_reduce_idx"]) and m["ge2_ptr"][-1] == len(m["sl"]) - m["n_eq1"]
