"""GPU parity of the drop-in wrappers (kbench.core.kernels.*) driven in the reference glue's call sequence.

``kbench.percall.run_forward`` / ``run_backward`` call the
HIP-backed wrappers with the reference glue's sequence and arguments.  Checked
against the float64 CPU oracle (loss rel 1e-5, gradients rel 1e-4, active masks
exact), for determinism, and against the native whole-pass driver
(``kbench.runtime``).
"""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _static(name, statewise=None):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    return static, cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


FUSE = pytest.mark.parametrize("fuse", [False, True], ids=["one_launch_per_sweep", "fused_sweep_chains"])


@FUSE
@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True), ("2", None)])
def test_glue_forward_matches_oracle(name, statewise, fuse, monkeypatch):
    """With one launch per sweep and with each wave's sweep chain in one launch (KBENCH_FUSE_SWEEPS)."""
    from kbench.core.kernels import wave_step
    from kbench.percall import run_forward

    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", fuse)
    print(f"[glue-forward] config={name} statewise={statewise} fuse_sweeps={fuse}", flush=True)
    static, theta, cw = _static(name, statewise)
    loss, saved = run_forward(static, theta, cw)
    torch.cuda.synchronize()
    _, ref_loss, ref = kbtest.oracle_forward(name, statewise)
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    print(f"  loss got={float(loss):.9g} ref={ref_loss:.9g} rel={rel:.3e}")
    assert rel <= 1e-5
    for k in ("E", "E_s1", "E_s2", "Ebar"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e}")
        assert ok and ma <= 1e-5
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5)


@FUSE
@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True)])
def test_glue_backward_matches_oracle(name, statewise, fuse, monkeypatch):
    """The backward at the per-call forward's point, that forward run both ways (KBENCH_FUSE_SWEEPS)."""
    from kbench.core.kernels import wave_step
    from kbench.percall import run_backward, run_forward

    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", fuse)
    print(f"[glue-backward] config={name} statewise={statewise} fuse_sweeps={fuse}", flush=True)
    static, theta, cw = _static(name, statewise)
    loss, saved = run_forward(static, theta, cw)
    gt, gc = run_backward(static, theta, cw, saved)
    torch.cuda.synchronize()
    ref_gt, ref_gc, _ = kbtest.oracle_backward(name, statewise)
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    print(f"  grad_theta normrel={rt:.3e} grad_col normrel={rc:.3e}")
    assert rt <= 1e-4 and rc <= 1e-4


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", True)])
def test_glue_backward_with_gmres_matches_oracle(name, statewise):
    """self_loop_solver="gmres" through the per-call path against the oracle's GMRES backward."""
    import dataclasses

    import kbench_oracle as O
    from kbench.percall import run_backward, run_forward
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    print(f"[glue-backward gmres] config={name} statewise={statewise}", flush=True)
    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    cap["meta"] = dict(cap["meta"], solver_options=dict(cap["meta"]["solver_options"], self_loop_solver="gmres"))
    static = make_static(cap, "cuda")
    assert static.solver_options.self_loop_solver == "gmres"
    theta, cw = cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()
    loss, saved = run_forward(static, theta, cw)
    gt, gc = run_backward(static, theta, cw, saved)
    torch.cuda.synchronize()
    prob = O.Problem.from_dict(p)
    prob.so.update(self_loop_solver="gmres")
    th64 = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw64 = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    _, ref = O.forward(prob, th64, cw64)
    ref_gt, ref_gc, _ = O.backward(prob, th64, cw64, ref)
    neu = kbtest.oracle_backward(name, statewise)[0]
    rt = kbtest.norm_rel(gt.cpu().numpy(), ref_gt)
    rc = kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    dn = kbtest.norm_rel(ref_gt, neu)
    print(f"  grad_theta normrel={rt:.3e} grad_col normrel={rc:.3e} (gmres vs neumann oracle: {dn:.3e})")
    assert rt <= 1e-4 and rc <= 1e-4


def test_level_waves_give_the_same_per_call_solve_and_hvp():
    """Rows regrouped into one wave per dependency level (synth.level_waves): the per-call forward gives
    bitwise the same rows, the gradients and an exact HVP agree with the size-wave layout."""
    from kbench.percall import run_backward, run_forward
    from kbench.newton.hvp import HvpPlan
    from kbench.percall.solve import plan_of
    from kbench import synth
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    print("[level waves] config=1 statewise per-call solve + exact HVP", flush=True)
    p = kbtest.problem("1", True)
    q, new_of_old = synth.level_waves(p)
    out = []
    for prob in (p, q):
        cap = problem_to_captured(prob)
        static = make_static(cap, "cuda")
        theta, cw = cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()
        loss, saved = run_forward(static, theta, cw)
        gt, gc = run_backward(static, theta, cw, saved)
        u = torch.linspace(-1.0, 1.0, theta.numel(), dtype=theta.dtype, device="cuda")
        hv = HvpPlan(plan_of(static), theta, cw, saved)(u)
        torch.cuda.synchronize()
        out.append((loss, saved, gt, gc, hv, len(prob["static"]["wave_layout"]["wave_metas"])))
    (la, sa, ga, gca, ha, na), (lb, sb, gb, gcb, hb, nb) = out
    idx = torch.as_tensor(new_of_old, device="cuda")
    print(f"  waves {na} -> {nb}; loss {float(la):.9g} vs {float(lb):.9g}")
    assert float(la) == float(lb)
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        assert torch.equal(sa[k], sb[k].index_select(0, idx)), k
    rt, rc, rh = kbtest.norm_rel_t(gb, ga), kbtest.norm_rel_t(gcb, gca), kbtest.norm_rel_t(hb, ha)
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e} hvp rel={rh:.3e}")
    assert rt <= 1e-6 and rc <= 1e-6 and rh <= 1e-5


def test_glue_backward_is_deterministic():
    from kbench.percall import run_backward, run_forward

    static, theta, cw = _static("1", True)
    loss, saved = run_forward(static, theta, cw)
    a = run_backward(static, theta, cw, saved)
    b = run_backward(static, theta, cw, saved)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_glue_matches_fused_driver_config2():
    """The per-wrapper path and the whole-pass driver solve the same problem (forward, config 2)."""
    from kbench.percall import run_forward
    from kbench.runtime import run_forward as run_forward_fused

    static, theta, cw = _static("2")
    l1, s1 = run_forward(static, theta, cw)
    l2, s2 = run_forward_fused(static, theta, cw)
    torch.cuda.synchronize()
    rel = abs(float(l1) - float(l2)) / abs(float(l2))
    ok, ma, mr = kbtest.compare_inf_safe(s1["pi_wave"].cpu().numpy(), s2["pi_wave"].cpu().numpy())
    print(f"  loss rel={rel:.3e} pi ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
    assert rel <= 1e-5 and ok and (ma <= 2e-4 or mr <= 1e-5)


def test_active_mask_bit_exact():
    """max|rhs| >= thr (> without pruning), including rows exactly at the threshold."""
    from kbench.core.kernels.wave_backward import active_mask_from_rhs_absmax_fused

    g = torch.Generator().manual_seed(5)
    W, S = 257, 300
    thr = np.float32(1e-6)
    rhs = (torch.rand((W, S), generator=g) * 2e-6 - 1e-6).float()
    rhs[0].zero_()
    rhs[1, 7] = float(thr)            # exactly at the threshold
    rhs[2, 9] = -float(thr)
    rhs[3, 11] = float(np.nextafter(thr, np.float32(0)))
    ref_abs = np.abs(rhs.numpy()).max(axis=1)
    for dt in (torch.float32, torch.float64, torch.bfloat16):
        x = rhs.to(dt).cuda()
        xa = np.abs(x.float().cpu().numpy().astype(np.float64) if dt == torch.bfloat16
                    else x.cpu().numpy().astype(np.float64)).max(axis=1)
        for pruning in (True, False):
            got = active_mask_from_rhs_absmax_fused(x, float(thr), use_pruning=pruning).cpu().numpy()
            ref = xa >= float(thr) if pruning else xa > float(thr)
            assert (got == ref).all(), (dt, pruning)
    assert (ref_abs >= thr)[1] and (ref_abs >= thr)[2] and not (ref_abs >= thr)[3]


def test_wave_step_in_place_matches_out_of_place():
    """Pi_out may alias Pi_in and Pibar (the glue's even sweeps write into the Pibar buffer)."""
    from kbench.core.kernels.wave_step import compute_wave_step
    from kbench.percall import run_forward

    static, theta, cw = _static("1", True)
    loss, saved = run_forward(static, theta, cw)
    pi, pibar = saved["pi_wave"], saved["pibar_wave"]
    h = static.state_helpers
    S = int(h["S"])
    meta = [m for m in static.wave_layout["wave_metas"] if "sl" not in m][0]
    ws, W = int(meta["start"]), int(meta["W"])
    G = 1
    E = saved["E"]
    consts = [x.expand(G, S).contiguous() for x in (saved["max_coupling"].reshape(1, -1),
                                                     1.0 + saved["log_pD"].reshape(1, -1) + E,
                                                     saved["Ebar"], E,
                                                     saved["log_pS"].reshape(1, -1) + saved["E_s2"],
                                                     saved["log_pS"].reshape(1, -1) + saved["E_s1"])]
    common = dict(leaf_state_idx=static.wave_layout["leaf_state_index"],
                  leaf_logp=saved["log_pS"].reshape(1, -1).expand(G, S).contiguous(),
                  item_idx=static.rate_item_idx, store_final_pibar=True, has_leaf_term=True,
                  use_col_weights=False)
    args = (ws, W, S, *consts, saved["col_log_probs"], h["node_child1"], h["node_child2"], h["node_parent"],
            int(h["max_ancestor_depth"]))
    out_a, pb_a, rm_a = pi.clone(), pibar.clone(), saved["pibar_row_max"].clone()
    compute_wave_step(pi.clone(), out_a, pb_a, *args, None, pibar_row_max=rm_a, **common)
    alias, rm_b = pi.clone(), saved["pibar_row_max"].clone()
    compute_wave_step(alias, alias, alias, *args, None, pibar_row_max=rm_b, **common)
    torch.cuda.synchronize()
    sl = slice(ws, ws + W)
    # with Pi_out is Pibar the final Pibar overwrites the new Pi rows, as in the reference
    assert torch.equal(alias[sl], pb_a[sl])
    assert torch.equal(rm_a[sl], rm_b[sl])


def test_glue_config3_forward_matches_fused():
    """Full-size drop-in check: config 3 forward through the wrappers equals the whole-pass driver."""
    from kbench.percall import run_forward
    from kbench.runtime import run_forward as run_forward_fused

    print("[glue-forward] config=3", flush=True)
    static, theta, cw = _static("3")
    l1, s1 = run_forward(static, theta, cw)
    l2, s2 = run_forward_fused(static, theta, cw)
    torch.cuda.synchronize()
    rel = abs(float(l1) - float(l2)) / abs(float(l2))
    ok, ma, mr = kbtest.compare_inf_safe(s1["pi_wave"].cpu().numpy(), s2["pi_wave"].cpu().numpy())
    print(f"  loss rel={rel:.3e} pi ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
    assert rel <= 1e-5 and ok


@pytest.mark.parametrize("name", ["1", "3"])
def test_fused_sweep_chains_match_one_launch_per_sweep(name, monkeypatch):
    """KBENCH_FUSE_SWEEPS: a wave's chained sweeps run as one launch (the linear-space preorder-ownership kernel
    for float rows) and agree with one launch per sweep to float32 rounding: same -inf pattern, loss 1e-6, rows
    2e-4 absolute or 1e-5 relative."""
    from kbench import percall as dropin
    from kbench.core.kernels import wave_step

    print(f"[fuse-sweeps] config={name}", flush=True)
    static, theta, cw = _static(name, True if name == "1" else None)
    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", False)
    la, sa = dropin.run_forward(static, theta, cw)
    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", True)
    lb, sb = dropin.run_forward(static, theta, cw)
    torch.cuda.synchronize()
    assert wave_step._chain is None  # every chain ended with its final call
    rel = abs(float(la) - float(lb)) / abs(float(la))
    print(f"  loss one-per-sweep={float(la):.9g} chained={float(lb):.9g} rel={rel:.3e}")
    assert rel <= 1e-6
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe(sb[k].cpu().numpy(), sa[k].cpu().numpy())
        print(f"  {k}: pattern={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5), k


def test_held_sweeps_run_before_other_work(monkeypatch):
    """A chain broken before its final call (an explicit flush, another wrapper) still yields every sweep.

    The rows agree with one launch per sweep to float32 rounding.
    """
    from kbench.percall.solve import plan_of
    from kbench.core.kernels import _hip as H
    from kbench.core.kernels import wave_step
    from kbench.core.kernels.wave_backward import active_mask_from_rhs_absmax_fused

    static, theta, cw = _static("1", True)
    plan = plan_of(static)
    _, sv = plan.forward(theta, cw)
    c = plan._row_consts(sv["E"], sv["Ebar"], sv["E_s1"], sv["E_s2"], sv["log_pS"], sv["log_pD"],
                         sv["max_coupling"])
    w = next(w for w in plan.waves if not w.split)
    h = static.state_helpers
    C, S = sv["pi_wave"].shape
    args = (w.ws, w.W, S, c.mt, c.DL, c.Ebar, c.E, c.SL1, c.SL2, sv["col_log_probs"], h["node_child1"],
            h["node_child2"], h["node_parent"], int(h["max_ancestor_depth"]), None)
    kw = dict(leaf_state_idx=plan.leaf_idx, leaf_logp=c.leaf, item_idx=plan.item_idx,
              pibar_row_max=sv["pibar_row_max"].clone(), has_leaf_term=True, use_col_weights=False)

    def three_sweeps(broken_by):
        a, b = sv["pi_wave"].clone(), torch.empty_like(sv["pi_wave"])
        bufs = [a, b, a]
        for i in range(3):
            wave_step.compute_wave_step(bufs[i], bufs[i + 1] if i < 2 else b, b, *args, **kw)
        if broken_by == "flush":
            H.flush()
        elif broken_by == "wrapper":
            active_mask_from_rhs_absmax_fused(a, 1e-6)
        return a.clone(), b.clone()

    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", False)
    ref = three_sweeps(None)
    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", True)
    for how in ("flush", "wrapper"):
        got = three_sweeps(how)
        torch.cuda.synchronize()
        assert wave_step._chain is None
        rows = slice(w.ws, w.ws + w.W)
        # the last sweep's output rows; a held chain of several sweeps runs in
        # linear space at preorder positions, with its sums added in another order
        ok, ma, mr = kbtest.compare_inf_safe(got[1][rows].cpu().numpy(), ref[1][rows].cpu().numpy())
        assert ok and (ma <= 2e-4 or mr <= 1e-5), (how, ma, mr)
