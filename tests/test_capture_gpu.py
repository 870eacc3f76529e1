"""Capture / replay of the HIP wrappers during a per-call solve (config 1).

Up to four calls of every wrapper (distinct waves) are recorded while the
per-call driver runs a forward and a backward; each recorded call is then
replayed in isolation and must reproduce its recorded outputs.  The HIP
wrappers sum in a fixed order, so the measured noise floor must be zero and
the replay bitwise equal; the only outputs the wrappers may leave unwritten
are the staged u_d rows (and their sums) of inactive parents.
"""

import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def test_capture_and_replay_every_wrapper(tmp_path):
    from kbench import percall as dropin
    from kbench import capture as cap
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    print("[capture] config=1 statewise per-call solve", flush=True)
    c0 = problem_to_captured(kbtest.problem("1", True))
    static = make_static(c0, "cuda")
    theta, cw = c0["inputs"]["theta"].cuda(), c0["inputs"]["col_weights"].cuda()
    with cap.Capture(per_wrapper=4) as c:
        loss, saved = dropin.run_forward(static, theta, cw)
        dropin.run_backward(static, theta, cw, saved)
    wrappers = {r["wrapper"] for r in c.records}
    print(f"  {len(c.records)} records, pool {len(c.pool)} storages: {sorted(wrappers)}", flush=True)
    assert wrappers == set(cap.WRAPPERS)
    path = tmp_path / "capture.pt"
    c.save(path)
    records, pool = cap.Capture.load(path)
    cap.measure_noise(records, pool)
    masked = [(r["wrapper"], p) for r in records for p in r["valid"]]
    print(f"  masked outputs: {sorted(set(masked))}", flush=True)
    for r in records:
        assert r["noise"] == {}, (r["wrapper"], r["noise"])
        verdicts = cap.replay(r, pool, rtol=0.0, atol=0.0)
        bad = [v for v in verdicts if not v["ok"]]
        assert verdicts and not bad, (r["wrapper"], r["key"], bad)
    # only the staged u_d rows and their sums of inactive parents may stay unwritten
    # (skip_inactive_pibar_output_zero, reference wave_backward.py:1980-2190)
    allowed = {("dts_cross_backward_accum_fused", "[2][0]"), ("dts_cross_backward_accum_fused", "[2][1]")}
    assert set(masked) <= allowed, set(masked) - allowed


def test_recorded_calls_match_the_oracle_on_their_own_inputs():
    """The gate with an independent reference side: every recorded call of a per-call solve is run
    again through the float64 oracle (tests/oracle_wrappers.py) on the call's own recorded inputs, and
    its outputs are compared with the call's recorded HIP outputs (reference capture/capture.py:164-210,
    bench/kernels.py:54-94).  Tolerance 1e-4 relative, or 1e-4 of the output's largest magnitude;
    masks and flags bitwise.  Don't-care regions are those of the reference: unwritten outputs (found
    by the poison runs) and the rows of ``v_k`` whose row is inactive (its FIXES.md:56-85)."""
    import kbench_oracle as O
    from kbench import capture as cap
    from kbench import percall as dropin
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static
    from oracle_wrappers import OracleWrappers

    print("[capture vs oracle] config=1 statewise", flush=True)
    prob = kbtest.problem("1", True)
    c0 = problem_to_captured(prob)
    static = make_static(c0, "cuda")
    theta, cw = c0["inputs"]["theta"].cuda(), c0["inputs"]["col_weights"].cuda()
    with cap.Capture(per_wrapper=4) as c:
        loss, saved = dropin.run_forward(static, theta, cw)
        dropin.run_backward(static, theta, cw, saved)
    cap.measure_noise(c.records, c.pool)
    ow = OracleWrappers(O.Problem.from_dict(prob).tree)
    checked = {}
    for r in c.records:
        dont_care = {}
        if r["wrapper"] == "wave_backward_uniform_fused":
            _, kw = cap.rebuild(r["pre"], c.pool, "cpu")
            act = kw["active_mask"].to(torch.bool)
            post = dict(cap.named_tensors(cap.rebuild(r["post"], c.pool, "cpu")))
            dont_care["[2][0]"] = ~act[:, None].expand_as(post["[2][0]"])
        verdicts = cap.replay(r, c.pool, fn=ow.fn(r["wrapper"]), rtol=1e-4, atol=1e-4, scale_atol=True,
                              dont_care=dont_care)
        worst = max((v["max_rel"] for v in verdicts), default=0.0)
        bad = [v for v in verdicts if not v["ok"]]
        print(f"  {r['wrapper']} key={r['key']}: {len(verdicts)} outputs, worst max_rel={worst:.2e}"
              + (f"  FAILED {bad}" if bad else ""), flush=True)
        assert verdicts and not bad, (r["wrapper"], r["key"], bad)
        checked[r["wrapper"]] = checked.get(r["wrapper"], 0) + 1
    assert set(checked) == set(cap.WRAPPERS), set(cap.WRAPPERS) - set(checked)
