"""Host-side logic: generator invariants, the DTS layout contract, parameter extraction, memory gate."""

import math

import numpy as np
import pytest
import torch

from kbench import synth
from kbench.core.kernels._dts_layout_contract import (DtsBackwardLayoutCode, DtsForwardAddressMode,
                                                      dts_backward_param_layout, dts_forward_param_layout)
from kbench.core.memory_policy import proposal0_memory_gate, proposal0_wave_scratch_bytes
from kbench.core.parameters import extract_parameters as X
import kbtest


# ------------------------------------------------------------- generator
@pytest.mark.parametrize("name", ["tiny", "1", "2"])
def test_wave_layout_invariants(name):
    p = kbtest.problem(name)
    wl, sh = p["static"]["wave_layout"], p["static"]["state_helpers"]
    S, C = int(sh["S"]), int(np.asarray(wl["leaf_state_index"]).shape[0])
    starts = [int(m["start"]) for m in wl["wave_metas"]]
    sizes = [int(m["W"]) for m in wl["wave_metas"]]
    # waves tile [0, C) in order and respect the reference's wave size cap
    assert starts[0] == 0 and all(a + w == b for a, w, b in zip(starts, sizes, starts[1:]))
    assert starts[-1] + sizes[-1] == C
    wave_of = np.repeat(np.arange(len(sizes)), sizes)
    leaf = np.asarray(wl["leaf_state_index"])
    for k, m in enumerate(wl["wave_metas"]):
        rows = slice(starts[k], starts[k] + sizes[k])
        if "sl" not in m:
            # leaf waves: every row is a species leaf
            assert ((leaf[rows] >= 0) & (leaf[rows] < S)).all()
            assert (np.asarray(sh["node_child1"])[leaf[rows]] >= S).all()
            continue
        sl, sr, red = (np.asarray(m[x]) for x in ("sl", "sr", "reduce_idx"))
        # children lie in earlier waves, every row of a split wave has a split
        assert (wave_of[sl] < k).all() and (wave_of[sr] < k).all()
        assert set(np.unique(red)) == set(range(sizes[k]))
        # eq1 splits first, then the ge2 CSR (reference dts_fused.py:171-231 metadata)
        n_eq1 = int(m["n_eq1"])
        counts = np.bincount(red, minlength=sizes[k])
        assert (counts[np.asarray(m["eq1_reduce_idx"])] == 1).all() and n_eq1 == int((counts == 1).sum())
        ptr, ids = np.asarray(m["ge2_ptr"]), np.asarray(m["ge2_parent_ids"])
        assert ptr[0] == 0 and ptr[-1] == len(sl) - n_eq1
        assert (counts[ids] == np.diff(ptr)).all() and (counts[ids] >= 2).all()
        lsp = np.asarray(m["log_split_probs"]).reshape(-1)
        assert (lsp <= 1e-12).all()
        # split probabilities of each parent sum to one
        tot = np.zeros(sizes[k])
        np.add.at(tot, red, np.exp2(lsp))
        assert np.allclose(tot, 1.0)
    roots = np.asarray(wl["root_row_ids"])
    assert len(roots) == p["meta"]["n_items"] and len(np.unique(roots)) == len(roots)


def test_generator_is_deterministic():
    a = synth.layout_digest(synth.build_problem(synth.config("2")))
    b = synth.layout_digest(synth.build_problem(synth.config("2")))
    assert a == b


def test_config3_shape():
    s = synth.summary(kbtest.problem("3"))
    assert s["S"] == 2047 and 30000 <= s["C"] <= 36000 and s["n_families"] == 500


def test_state_helpers_consistency():
    sh = kbtest.problem("1")["static"]["state_helpers"]
    S = int(sh["S"])
    par, c1, c2 = (np.asarray(sh[k]) for k in ("node_parent", "node_child1", "node_child2"))
    for s in range(S):
        for c in (c1[s], c2[s]):
            if c < S:
                assert par[c] == s
    st, en = np.asarray(sh["node_subtree_start"]), np.asarray(sh["node_subtree_end"])
    # subtree ranges nest: a child's range lies inside its parent's
    for s in range(S):
        if par[s] >= 0:
            assert st[par[s]] < st[s] and en[s] <= en[par[s]]
    # unnorm_row_max = -log2(number of non-ancestors), -inf never (root has S-1)
    depth = np.zeros(S, int)
    for s in range(S):
        a = s
        while par[a] >= 0:
            a = par[a]
            depth[s] += 1
    with np.errstate(divide="ignore"):
        ref = -np.log2((S - depth - 1).astype(float))
    assert np.allclose(np.asarray(sh["unnorm_row_max"]), ref)


# ------------------------------------------------------------- DTS layout contract
def test_backward_layout_codes():
    S = 5
    f = lambda shape, item=True: dts_backward_param_layout(shape, S=S, item_indexed=item)
    assert f(()).code == DtsBackwardLayoutCode.SHARED_SCALAR
    assert f((1, 1)).code == DtsBackwardLayoutCode.SHARED_SCALAR
    assert f((3,)).code == DtsBackwardLayoutCode.ITEM_SCALAR
    assert f((5,)).code == DtsBackwardLayoutCode.ITEM_SCALAR and f((5,)).ambiguous_1d_item_state
    assert f((5,), item=False).code == DtsBackwardLayoutCode.SHARED_STATE
    assert f((3, 1)).code == DtsBackwardLayoutCode.ITEM_SCALAR
    assert f((1, 5)).code == DtsBackwardLayoutCode.ITEM_STATE
    assert f((3, 5)).code == DtsBackwardLayoutCode.ITEM_STATE
    for bad in ((3, 4), (2, 2, 2)):
        with pytest.raises(ValueError):
            f(bad)
    with pytest.raises(ValueError):
        f((3,), item=False)


def test_forward_layout_modes():
    S = 5
    t = torch.zeros(4, S)
    lay = dts_forward_param_layout(t, S=S, item_indexed=True)
    assert lay.mode == DtsForwardAddressMode.ITEM_INDEXED and lay.row_stride == S and lay.state_stride == 1
    assert dts_forward_param_layout((1, S), S=S, item_indexed=True).row_stride == 0
    assert dts_forward_param_layout((S,), S=S, item_indexed=True).intent == "shared_state"
    assert dts_forward_param_layout((3,), S=S, item_indexed=True).intent == "item_scalar"
    assert dts_forward_param_layout((), S=S, item_indexed=False).mode == DtsForwardAddressMode.SHARED_STATE
    with pytest.raises(ValueError):
        dts_forward_param_layout((3,), S=S, item_indexed=False)
    with pytest.raises(ValueError):
        dts_forward_param_layout((2,), S=0, item_indexed=True)


# ------------------------------------------------------------- parameter extraction
def test_log2_rates_are_a_distribution():
    th = torch.tensor([[-2.0, -1.5, -2.5], [0.3, -4.0, 1.0]], dtype=torch.float64)
    pS, pD, pL, mt = X.extract_parameters_uniform(th, torch.zeros(2, dtype=torch.float64), statewise=True)
    tot = torch.exp2(pS) + torch.exp2(pD) + torch.exp2(pL) + torch.exp2(mt)
    assert torch.allclose(tot, torch.ones_like(tot))
    # softmax over [0, theta] in base 2: p_k / p_S = 2^theta_k
    assert torch.allclose(pD - pS, th[:, 0]) and torch.allclose(pL - pS, th[:, 1])


def test_col_valid_log_normalizer_brute_force():
    sh = kbtest.problem("tiny")["static"]["state_helpers"]
    S = int(sh["S"])
    par = np.asarray(sh["node_parent"])
    cw = torch.linspace(-1, 1, S, dtype=torch.float64)
    col = X.col_log_probs_from_weights(cw)
    got = X.col_valid_log_normalizer(col, torch.as_tensor(par), int(sh["max_ancestor_depth"])).numpy()
    p = np.exp(cw.numpy()) / np.exp(cw.numpy()).sum()
    for s in range(S):
        mass, a = 0.0, s
        while a >= 0:
            mass += p[a]
            a = par[a]
        assert abs(got[s] - (-math.log2(1.0 - mass))) < 1e-12


def test_as_item_shapes():
    S = 4
    assert X.as_item_param(torch.tensor(1.0), 3, S).shape == (3, 1)
    assert X.as_item_param(torch.zeros(S), 1, S).shape == (1, S)
    assert X.as_item_param(torch.zeros(3), 3, S).shape == (3, 1)
    assert X.as_item_state(torch.tensor(2.0), S, 3).shape == (3, S)
    assert X.as_item_state(torch.zeros(S), S, 1).shape == (1, S)


def test_weighted_extraction_gradients_match_finite_differences():
    """The glue differentiates the extraction with autograd; check it against FD in float64."""
    sh = {k: torch.as_tensor(v) if isinstance(v, np.ndarray) else v
          for k, v in kbtest.problem("tiny")["static"]["state_helpers"].items()}
    S = int(sh["S"])
    th = torch.tensor([-2.0, -1.0, -2.5], dtype=torch.float64, requires_grad=True)
    cw = torch.linspace(-0.5, 0.5, S, dtype=torch.float64, requires_grad=True)
    g = torch.linspace(1.0, 2.0, S, dtype=torch.float64)

    def obj(t, c):
        pS, pD, pL, mt, col = X.extract_parameters_weighted_cols(t, c, sh, statewise=False)
        return pS * 1.3 + pD * 0.7 - pL + (mt * g).sum() + (col * g.flip(0)).sum()

    gt, gc = torch.autograd.grad(obj(th, cw), (th, cw))
    h = 1e-6
    for j in range(3):
        e = torch.zeros(3, dtype=torch.float64)
        e[j] = h
        fd = (obj(th + e, cw) - obj(th - e, cw)) / (2 * h)
        assert abs(float((gt[j] - fd).detach())) < 1e-7
    for j in range(S):
        e = torch.zeros(S, dtype=torch.float64)
        e[j] = h
        fd = (obj(th, cw + e) - obj(th, cw - e)) / (2 * h)
        assert abs(float((gc[j] - fd).detach())) < 1e-7


# ------------------------------------------------------------- memory gate
def test_memory_gate_without_device():
    ok, need, budget = proposal0_memory_gate(100, 2047, torch.float32)
    assert need == proposal0_wave_scratch_bytes(100, 2047, torch.float32) == 100 * 2047 * 10 * 4
    if not torch.cuda.is_available():
        assert ok and budget is None
    with pytest.raises(ValueError):
        proposal0_memory_gate(-1, 4, torch.float32)
    with pytest.raises(ValueError):
        proposal0_memory_gate(1, 0, torch.float32)
