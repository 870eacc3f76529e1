"""The generator's item-row problems and the oracle's forward on them (CPU).

* ``ProblemConfig(itemwise=True)`` keeps the layout of the one-row problem (same tree, families,
  rows and splits) and adds theta [n_families, 3] with ``rate_item_idx`` = each row's family;
  per-state item rows and family subsets of item-row problems are refused;
* with every family given the same rates the oracle's item-row forward is bitwise the one-row
  forward (the loss is a sum of per-family terms, each reading its own E row), and with different
  rates the loss moves.
"""

import dataclasses

import numpy as np
import pytest

import kbench_oracle as O


def _pair():
    from kbench import synth

    g = synth.build_problem(synth.config("1"))
    i = synth.build_problem(dataclasses.replace(synth.config("1"), itemwise=True))
    return g, i


def test_item_rows_keep_the_layout_and_index_the_families():
    g, i = _pair()
    wg, wi = g["static"]["wave_layout"], i["static"]["wave_layout"]
    for k in ("leaf_state_index", "root_row_ids", "item_idx"):
        assert np.array_equal(wg[k], wi[k])
    assert len(wg["wave_metas"]) == len(wi["wave_metas"])
    assert i["static"]["itemwise"] and not g["static"]["itemwise"]
    n = int(i["meta"]["n_items"])
    assert i["inputs"]["theta"].shape == (n, 3)
    assert np.array_equal(i["static"]["rate_item_idx"], wi["item_idx"])
    assert np.array_equal(np.asarray(wi["item_idx"])[wi["root_row_ids"]], np.arange(n))


def test_item_rows_refuse_per_state_rates_and_family_subsets():
    from kbench import synth

    with pytest.raises(ValueError):
        synth.build_problem(dataclasses.replace(synth.config("tiny"), itemwise=True, statewise=True))
    _, i = _pair()
    with pytest.raises(ValueError):
        synth.family_subset(i, [0, 1])


def test_oracle_item_row_forward_reduces_to_the_one_row_forward():
    g, i = _pair()
    n = int(i["meta"]["n_items"])
    cw = g["inputs"]["col_weights"]
    lg, sg = O.forward(O.Problem.from_dict(g), g["inputs"]["theta"], cw)
    prob = O.Problem.from_dict(i)
    li, si = O.forward(prob, np.broadcast_to(g["inputs"]["theta"], (n, 3)).copy(), cw)
    assert li == lg
    assert si["E"].shape == (n, g["static"]["state_helpers"]["S"])
    assert np.array_equal(si["E"], np.broadcast_to(sg["E"], si["E"].shape))
    assert np.array_equal(si["pi_wave"], sg["pi_wave"], equal_nan=True)
    l2, _ = O.forward(prob, i["inputs"]["theta"], cw)
    assert abs(l2 - lg) > 1e-3 * abs(lg)
