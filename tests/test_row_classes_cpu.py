"""``synth.row_classes``: rows with the same inputs merged into one row per class.

The class layout is pinned by the oracle: solving it gives, for every row of
the original layout, the row of its class (the same truncated forward up to
the order in which a row's splits are merged), and the loss of the class
layout's distinct families.  With an active mask the classes refine the
unmasked ones so that members share their flag and, split by split, their
children's classes.
"""

import numpy as np
import pytest

import kbench_oracle as O
from kbench import synth
import kbtest


def _class_problem(p, layout, rep):
    st = p["static"]
    q = dict(p)
    q["static"] = dict(st, wave_layout=layout, rate_item_idx=np.asarray(st["rate_item_idx"])[rep])
    q["meta"] = dict(p["meta"], C=int(rep.shape[0]))
    return q


@pytest.mark.parametrize("name,levels", [("tiny", False), ("1", False), ("1", True), ("2", True)])
def test_class_rows_are_the_member_rows(name, levels):
    p = kbtest.problem(name)
    if levels:
        p, _ = synth.level_waves(p)
    st = p["static"]
    layout, class_of, rep = synth.row_classes(st["wave_layout"], st["rate_item_idx"])
    C = class_of.shape[0]
    assert rep.shape[0] < C  # identical leaf rows at least
    assert np.array_equal(class_of[rep], np.arange(rep.shape[0]))  # a representative is in its own class
    q = _class_problem(p, layout, rep)
    A, B = O.Problem.from_dict(p), O.Problem.from_dict(q)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.zeros(A.S)
    _, sa = O.forward(A, th, cw)
    _, sb = O.forward(B, th, cw)
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        a, b = sa[k], sb[k][class_of]
        fin = np.isfinite(a)
        assert np.array_equal(fin, np.isfinite(b)), k
        assert np.abs(a[fin] - b[fin]).max() <= 1e-12 * max(1.0, np.abs(a[fin]).max()), k


def test_class_layout_is_one_wave_per_level_over_classes():
    p, _ = synth.level_waves(kbtest.problem("1"))
    st = p["static"]
    wl = st["wave_layout"]
    layout, class_of, rep = synth.row_classes(wl, st["rate_item_idx"])
    leaf = np.asarray(wl["leaf_state_index"])
    # members share their leaf state; class ids grow with the level
    assert np.array_equal(leaf, np.asarray(layout["leaf_state_index"])[class_of])
    metas = layout["wave_metas"]
    wave_of = np.empty(rep.shape[0], dtype=np.int64)
    for i, m in enumerate(metas):
        wave_of[int(m["start"]):int(m["start"]) + int(m["W"])] = i
        if "sl" in m:
            children = np.concatenate([m["sl"], m["sr"]])
            assert (wave_of[children] < i).all()
    assert np.array_equal(np.asarray(layout["root_row_ids"]), class_of[np.asarray(wl["root_row_ids"])])


def test_masked_classes_refine_and_agree_along_splits():
    p, _ = synth.level_waves(kbtest.problem("1"))
    st = p["static"]
    wl = st["wave_layout"]
    C = int(np.asarray(wl["leaf_state_index"]).shape[0])
    g = np.random.default_rng(3)
    active = g.random(C) < 0.8
    _, plain, _ = synth.row_classes(wl, st["rate_item_idx"])
    layout, cls, rep = synth.row_classes(wl, st["rate_item_idx"], active=active)
    assert rep.shape[0] > plain.max() + 1  # the mask splits some classes
    for c in range(rep.shape[0]):
        members = np.flatnonzero(cls == c)
        assert len(set(plain[members].tolist())) == 1  # a refinement of the unmasked classes
        assert len(set(active[members].tolist())) == 1  # one flag per class
    # members' splits, as unordered child-class pairs, are the representative's
    splits = {}
    for m in wl["wave_metas"]:
        if "sl" in m:
            for a, b, w in zip(m["sl"], m["sr"], m["reduce_idx"]):
                splits.setdefault(int(m["start"]) + int(w), []).append(tuple(sorted((cls[a], cls[b]))))
    for r, sp in splits.items():
        assert sorted(sp) == sorted(splits[int(rep[cls[r]])])
