"""Config 5 at its size: the exact HVP on the config-3 problem (S = 2047, C = 33686, per-species theta).

At this size the float64 oracle HVP is out of reach, so the product's HVP
(``kbench.newton.make_exact_hvp``: tangent forward and reverse on one row per
class of identical rows, replayed as one HIP graph; reference
newton/hvp_exact.py:66-383) is checked through what the mathematics fixes,
on two seeded unit directions u1, u2:

* it equals the row-by-row HVP (every row computed, no graph) to rel 1e-4
  of max |H u|: the two differ only in the order of sums;
* symmetry: |u2 . H u1 - u1 . H u2| <= 1e-3 max(|u2 . H u1|, |u1 . H u2|);
* linearity: H(a u1 + b u2) = a H u1 + b H u2 to rel 1e-4;
* replays of the captured graph are bitwise equal;
* central differences along u1 of float64 gradients (the per-call path in
  float64, step 1e-3) agree with H u1 to 5e-3 of max |H u1|.  Float32
  gradients cannot serve here: their rounding over 33686 rows, divided by
  any step small enough for the O(h^2) term, is several percent of H u.

The rows are grouped one wave per dependency level (``synth.level_waves``,
the bench's layout; the same HVP, pinned on configs 1 and S = 4095 / 8191
against the oracle in test_hvp_gpu.py); one more HVP on the generated size
waves agrees with it to rel 1e-4.
"""

import functools

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=None)
def _setup():
    from kbench import synth
    from kbench.fused import problem_to_captured
    from kbench.percall.solve import run_forward
    from kbench.runtime import make_static

    problem = kbtest.problem("3")
    assert problem["static"]["statewise"]
    cap = problem_to_captured(synth.level_waves(problem)[0])
    static = make_static(cap, "cuda")
    theta, cw = cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()
    _, sv = run_forward(static, theta, cw)
    g = np.random.default_rng(2047)
    us = []
    for _ in range(2):
        u = g.normal(size=int(theta.numel()))
        us.append(torch.as_tensor(u / np.linalg.norm(u), dtype=theta.dtype, device="cuda"))
    return problem, static, theta, cw, sv, us


@functools.lru_cache(maxsize=None)
def _fast():
    from kbench.newton.hvp import make_exact_hvp

    _, static, theta, cw, sv, us = _setup()
    hvp = make_exact_hvp(static, theta, cw, sv)
    assert hvp.graph and hvp.cls is not None
    return hvp, [hvp(u).clone() for u in us]


def _rel(a, b):
    return float((a.double() - b.double()).abs().max()) / float(b.double().abs().max())


def test_config3_class_graph_hvp_equals_the_row_by_row_hvp():
    from kbench.newton.hvp import make_exact_hvp

    print("[hvp config3] class/graph vs row by row", flush=True)
    _, static, theta, cw, sv, us = _setup()
    _, fast = _fast()
    rows = make_exact_hvp(static, theta, cw, sv, row_classes=False, graph=False)
    for i, u in enumerate(us):
        ref = rows(u)
        torch.cuda.synchronize()
        e = _rel(fast[i], ref)
        print(f"  u{i + 1}: |H u|={float(ref.abs().max()):.4e} rel={e:.3e}", flush=True)
        assert e <= 1e-4


def test_config3_hvp_is_symmetric_linear_and_replays_bitwise():
    print("[hvp config3] symmetry, linearity, replays", flush=True)
    *_, us = _setup()
    hvp, (h1, h2) = _fast()
    a = float((us[1].double() * h1.double()).sum())
    b = float((us[0].double() * h2.double()).sum())
    print(f"  u2.Hu1={a:.8e} u1.Hu2={b:.8e}", flush=True)
    assert abs(a - b) <= 1e-3 * max(abs(a), abs(b))
    alpha, beta = 0.75, -1.5
    hl = hvp(alpha * us[0] + beta * us[1])
    e = _rel(hl, alpha * h1.double() + beta * h2.double())
    print(f"  linearity rel={e:.3e}", flush=True)
    assert e <= 1e-4
    for _ in range(2):
        again = hvp(us[0])
        torch.cuda.synchronize()
        assert torch.equal(again, h1)


def test_config3_hvp_agrees_with_central_differences_of_float64_gradients():
    from kbench.percall.solve import plan_of

    print("[hvp config3] vs central differences of float64 per-call gradients", flush=True)
    _, static, theta, cw, sv, us = _setup()
    _, (h1, _) = _fast()
    plan = plan_of(static)
    u = us[0].double().reshape(theta.shape)
    x0 = theta.double()
    cw64 = cw.double()

    def grad(x):
        _, s = plan.forward(x, cw64)
        g, _ = plan.backward(x, cw64, s)
        return g.reshape(-1)

    def D(h):
        return (grad(x0 + h * u) - grad(x0 - h * u)) / (2.0 * h)

    d1, d2 = D(1e-3), D(2e-3)
    torch.cuda.synchronize()
    e1, e2 = _rel(d1, h1), _rel(d2, h1)
    print(f"  |H u1|={float(h1.abs().max()):.4e} FD(1e-3) rel={e1:.3e} FD(2e-3) rel={e2:.3e} "
          f"FD steps differ by {_rel(d1, d2):.3e}", flush=True)
    assert e1 <= 5e-3


def test_config3_hvp_on_the_size_waves_equals_the_level_waves():
    from kbench.fused import problem_to_captured
    from kbench.newton.hvp import make_exact_hvp
    from kbench.percall.solve import run_forward
    from kbench.runtime import make_static

    print("[hvp config3] size waves vs level waves", flush=True)
    problem, _, theta, cw, _, us = _setup()
    _, (h1, _) = _fast()
    static = make_static(problem_to_captured(problem), "cuda")
    _, sv = run_forward(static, theta, cw)
    hs = make_exact_hvp(static, theta, cw, sv)(us[0])
    torch.cuda.synchronize()
    e = _rel(hs, h1)
    print(f"  rel={e:.3e}", flush=True)
    assert e <= 1e-4
