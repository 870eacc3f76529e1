"""The per-call wave loops captured as HIP graphs: the glue's call sequence launched once per pass.

The reference's glue launches the solve wave by wave (its
kbench/core/inference/forward.py:60-108 issues one ``compute_wave_step`` per
sweep; kbench/api/_implicit_grad.py:195-353 issues the mask, split term,
adjoint, seven bucket sums, split adjoint and Pibar VJP per wave), thousands
of launches per solve.  ``GraphedSolve`` keeps that call sequence -- the
``SolvePlan`` drivers, calling the same wrappers with the same arguments in
the same order -- and records it once:

* forward graph: parameters, E fixed point, per-wave split terms and sweeps,
  loss (``SolvePlan._forward``);
* reverse graph: root seed and the per-wave reverse sweep
  (``SolvePlan.reverse_sweep``).

Each is run once eagerly first (every layout table and kernel attribute the
wrappers cache on first use is built outside the capture), then captured
under ``torch.cuda.graph`` and replayed from then on.  The E adjoint
(BiCGSTAB, whose stopping test reads the host each iteration) and the theta /
column VJP run eagerly after the reverse replay, as in ``SolvePlan.backward``.

Contract:

* inputs are copied into the graphs' own buffers; ``forward`` returns the
  forward graph's outputs (loss and the saved tensors), which the next
  ``forward`` replay overwrites -- clone what must outlive it;
* ``backward`` reads the forward graph's saved tensors; saved tensors from
  elsewhere are copied into them first;
* the column weights' branch (uniform or weighted, one host read) is fixed at
  capture; a call on the other branch raises ``ValueError``, as do changed
  shapes, dtypes or devices;
* GMRES self-loop solves read the host per iteration and cannot be captured:
  ``self_loop_solver="gmres"`` raises ``NotImplementedError``.
"""

from __future__ import annotations

import torch

from .solve import SAVED, SolvePlan, root_softmax2, uniform_columns

__all__ = ["GraphedSolve"]


class GraphedSolve:
    """Forward and reverse wave loops of ``plan`` as two replayable HIP graphs."""

    def __init__(self, plan: SolvePlan, theta: torch.Tensor, col_weights: torch.Tensor):
        if plan.so.self_loop_solver != "neumann":
            raise NotImplementedError("GraphedSolve: the GMRES self-loop solve reads the host per iteration "
                                      "and cannot be captured; use SolvePlan")
        if theta.device.type != "cuda":
            raise ValueError("GraphedSolve needs device tensors")
        self.p = plan
        self.P = int(plan.so.pi_iters)
        self.weighted = not uniform_columns(col_weights)
        self.theta = theta.detach().clone()
        self.cw = col_weights.detach().clone()
        self._fg = self._rg = None
        self._fout = self._racc = None

    def _take(self, theta, col_weights):
        for name, a, b in (("theta", theta, self.theta), ("col_weights", col_weights, self.cw)):
            if a.shape != b.shape or a.dtype != b.dtype or a.device != b.device:
                raise ValueError(f"GraphedSolve: {name} is {tuple(a.shape)} {a.dtype} on {a.device}; the graphs "
                                 f"were captured for {tuple(b.shape)} {b.dtype} on {b.device}")
        if (not uniform_columns(col_weights)) != self.weighted:
            raise ValueError("GraphedSolve: the column weights switched between uniform and weighted since capture")
        self.theta.copy_(theta.detach())
        self.cw.copy_(col_weights.detach())

    def _forward_body(self):
        return self.p._forward(self.theta, self.cw, self.P, weighted=self.weighted)

    def _reverse_body(self):
        sv = self._fout[1]
        seed = -root_softmax2(sv["pi_wave"].index_select(0, self.p.roots))
        return self.p.reverse_sweep(sv, seed, use_col=self.weighted)

    @staticmethod
    def _capture(body):
        with torch.no_grad():
            body()  # eager: builds what the wrappers cache on first use
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(g):
            out = body()
        return g, out

    def forward(self, theta, col_weights):
        """(loss, saved) as ``SolvePlan.forward`` returns them, from one graph replay."""
        self._take(theta, col_weights)
        if self._fg is None:
            self._fg, self._fout = self._capture(self._forward_body)
        self._fg.replay()
        return self._fout

    def reverse(self, saved):
        """The reverse wave loop's parameter cotangents (``SolvePlan.reverse_sweep`` from the root seed)."""
        if self._fout is None:
            raise RuntimeError("GraphedSolve.reverse before the first forward")
        sv = self._fout[1]
        for k in SAVED:
            if saved[k] is not sv[k]:
                sv[k].copy_(saved[k])
        if self._rg is None:
            self._rg, self._racc = self._capture(self._reverse_body)
        self._rg.replay()
        return self._racc

    def backward(self, theta, col_weights, saved):
        """(grad_theta, grad_col): the reverse graph, then the E adjoint and theta VJP eagerly."""
        self._take(theta, col_weights)
        acc = self.reverse(saved)
        return self.p.e_adjoint_and_vjp(self.theta, self.cw, self._fout[1], acc, use_col=self.weighted)
