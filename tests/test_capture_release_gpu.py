"""Native handles dropped while a HIP graph capture is underway are destroyed after it.

Destroying a plan or a tree handle frees device memory, and a free during a
capture invalidates the capture.  The garbage collector can drop the last
reference to such a handle at any allocation (torch no longer collects before
a capture), so ``kbench._native.release`` holds the destruction back until
no capture is underway.  Here a whole-pass plan and a tree handle sit in
reference cycles, are collected inside a capture, and the capture must still
end and replay correctly; the held-back handles are destroyed at the next
library call outside the capture.
"""

import gc

import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def test_handles_collected_inside_a_capture_are_destroyed_after_it():
    from kbench import _native as N
    from kbench.core.kernels import _hip as H
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print("[capture release] config=tiny", flush=True)
    cap = problem_to_captured(kbtest.problem("tiny", False))
    static = make_static(cap, "cuda")
    gc.collect()
    gc.disable()
    try:
        solver = FusedSolver(static, static.solver_options)
        solver.cycle = solver  # only the cyclic collector frees it
        S = 9
        par = torch.tensor([-1, 0, 0, 1, 1, 2, 2, 3, 3], dtype=torch.long)
        c1 = torch.tensor([1, 3, 5, 7, 9, 9, 9, 9, 9], dtype=torch.long)
        c2 = torch.tensor([2, 4, 6, 8, 9, 9, 9, 9, 9], dtype=torch.long)
        tree = H._create(S, par, c1, c2)
        holder = [tree]
        holder.append(holder)
        del solver, tree, holder

        x = torch.arange(1024, device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = x * 2.0
            freed = gc.collect()
            z = y + 1.0
        assert freed > 0
        held = len(N._held_back)
        assert held >= 2, f"expected the plan and the tree to wait for the capture's end, {held} held back"
        x.copy_(torch.full_like(x, 3.0))
        g.replay()
        torch.cuda.synchronize()
        assert bool(torch.all(z == 7.0))
        N.lib()  # outside the capture: the held-back handles are destroyed now
        assert not N._held_back
    finally:
        gc.enable()
