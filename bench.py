#!/usr/bin/env python
"""Benchmark of the log-space solver path on one MI355X.

Workload: Yule species tree with 1024 leaves (S = 2047 state
columns), 500 DTL-simulated families with 3 NNI variants each (C = 33686 clade
rows in 144 size-waves), per-species theta, fp32, pi_iters = 16,
neumann_terms = 16.  A step is one whole solve: forward (E-step fixed point,
every row's sweeps, loss) plus backward (adjoint over every row, E adjoint,
theta / column VJP), run through the native whole-pass driver with every
input already in HBM.  Rows with identical inputs (row classes) are computed
once in the forward; the line states how many rows that is and also times the
solve with every row computed (``KB_DEDUP=0``).  The backward stops each row's
Neumann series at its first term whose entries are all at most 2^-24 of the
row's largest right-hand-side entry (``FusedSolver.neumann_rtol``); ``neumann``
gives the terms per row and times the same solve summing all 16 terms.

Prints ONE JSON line.  ``value`` is ms per solve (fwd + bwd, HIP events),
lower is better, each solve one ``kb_solve`` call (``FusedSolver.solve``):
the backward rows of the families that end at low dependency levels run on a
second stream beside the forward's later, narrow levels.  ``two_calls``,
``fwd_ms`` and ``bwd_ms`` time the same solves as ``run_forward`` then
``run_backward``, the reference's split.

* ``roofline``: the dominant row kernel's algorithmic HBM bytes per launch
  (S*4 bytes per row: the backward reads Pi*, Pibar* and the adjoint of every
  row and four child rows plus two adjoint rows per split) over its launch
  durations, measured with HIP events on the launch stream in a second timed
  pass; ``traffic`` and the VALU / LDS figures come from the committed
  rocprofv3 counter summaries of this command (profiles/).
* ``cpu_baseline``: the float64 CPU oracle on the box's host cores, computed
  before the GPU is touched: a bounded sample of the config-3 families packed
  by rows into one shard per worker process (the loss and gradients of a
  problem are sums over its family shards), scaled by rows to a full solve;
  beside it, config 1 (BASELINE's CPU case) solved in full the same way.
* ``per_call``: the same solve through the builder's call-sequence drivers
  (``kbench.percall``: the per-call wrappers in the reference glue's order,
  wave buckets folded by native fixed-order row sums): one launch per sweep
  and per wave as the reference launches them (the pristine-structure proxy),
  the same with each wave's sweep chain collapsed into one launch
  (``KBENCH_FUSE_SWEEPS``), and the driver alone (every wrapper a no-op), all
  three over the forward and the per-wave reverse sweep, with the glue's E
  adjoint timed apart; and the whole-solve ratio of the first to ``value``
  (the speedup against the pristine-structure proxy on the same GPU;
  ``vs_baseline`` stays null, no published number exists for this metric).
* ``config5``: BASELINE config 5 on the same problem: the 50 exact
  Hessian-vector products of one Newton-CG step (``kbench.newton.make_exact_hvp``),
  timed as one block, with the roofline of its largest kernel.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kernel-bench_amd"))

HBM_PEAK_GBS = 8000.0
# quarter-rate transcendentals (v_exp_f32 / v_log_f32 / v_rcp_f32): 16 lanes per CU per clock,
# 256 CUs at 2.4 GHz
TRANS_PEAK_PER_S = 256 * 16 * 2.4e9
def _profile_file(kind: str, config: str):
    """The committed rocprofv3 summary (``traffic`` or ``sq_counters``) of one configuration."""
    return ROOT / "profiles" / f"{kind}_config{config}.json"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-workers", type=int, default=0,
                    help="worker processes of the CPU baseline (default: the host cores, at most 16)")
    ap.add_argument("--cpu-families-per-worker", type=int, default=2)
    ap.add_argument("--no-per-call", action="store_true", help="skip the per-call (drop-in) timings")
    ap.add_argument("--no-dedup-off", action="store_true", help="skip the KB_DEDUP=0 timing")
    ap.add_argument("--no-config5", action="store_true", help="skip the config-5 Hessian-vector product timing")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--hvp-layout", choices=("both", "levels"), default="both",
                    help="--workload hvp: time the size waves and the level waves, or the level waves only")
    ap.add_argument("--hvp-variants", choices=("all", "fast"), default="all",
                    help="--workload hvp: also time the row-by-row and the uncaptured class HVPs (all), or only "
                         "the class HVP replayed as a graph (fast)")
    ap.add_argument("--workload", choices=("solve", "glue", "hvp"), default="solve",
                    help="solve: whole-pass driver (the metric); glue: only the per-call drop-in timings; "
                         "hvp: exact Hessian-vector products of the config-5 Newton-CG setup")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 plain copy kernels of MIB MiB (read + write), the reference point "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters to HBM bytes")
    return ap.parse_args()


def log(args, msg):
    if args.verbose:
        print(msg, file=sys.stderr, flush=True)


def calibrate_copy(mib: int) -> None:
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads and writes n * 4 bytes
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "kernel": "elementwise mul by 1", "launches": 5,
                      "bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4}))


# ---------------------------------------------------------------------- CPU baseline
def _oracle_solve(sub: dict) -> tuple:
    """Oracle forward + backward of one family shard (runs in a worker process, one thread)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import kbench_oracle as O

    with threadpool_limits(1):
        t0 = time.perf_counter()
        prob = O.Problem.from_dict(sub)
        th = np.asarray(sub["inputs"]["theta"], dtype=np.float64)
        cw = np.asarray(sub["inputs"]["col_weights"], dtype=np.float64)
        loss, saved = O.forward(prob, th, cw)
        gt, gc, _ = O.backward(prob, th, cw, saved)
        return loss, gt, gc, time.perf_counter() - t0


def _sharded_oracle(problem: dict, families, workers: int) -> dict:
    """Wall time of the oracle over ``families`` split into ``workers`` family shards."""
    import multiprocessing as mp

    from kbench import synth

    import numpy as np

    fams = list(families)
    # greedy packing by rows, largest family first, onto the least loaded shard
    fam_rows = np.bincount(np.asarray(problem["static"]["wave_layout"]["item_idx"]))
    shards, load = [[] for _ in range(workers)], [0] * workers
    for f in sorted(fams, key=lambda f: -int(fam_rows[f])):
        i = load.index(min(load))
        shards[i].append(f)
        load[i] += int(fam_rows[f])
    subs = [synth.family_subset(problem, sorted(s)) for s in shards if s]
    rows = sum(int(s["meta"]["C"]) for s in subs)
    # fork before the process touches the GPU (main() calls this first)
    with mp.get_context("fork").Pool(len(subs)) as pool:
        t0 = time.perf_counter()
        parts = pool.map(_oracle_solve, subs)
        wall = time.perf_counter() - t0
    return {"wall_s": wall, "rows": rows, "families": len(fams), "shards": len(subs),
            "loss": float(sum(p[0] for p in parts)), "busiest_shard_s": max(p[3] for p in parts),
            "cpu_s": sum(p[3] for p in parts)}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args, problem: dict) -> dict:
    """The CPU path on this host's cores (see the module docstring)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    from kbench import synth

    avail = len(os.sched_getaffinity(0))
    workers = args.cpu_workers or min(16, avail)
    C = int(problem["meta"]["C"])
    sample = _sharded_oracle(problem, range(min(int(problem["meta"]["n_items"]),
                                                 workers * args.cpu_families_per_worker)), workers)
    # a full solve's 500 families pack evenly onto the workers: its time is the
    # sample's CPU seconds per row times C rows over the workers
    value = sample["cpu_s"] * 1e3 * C / sample["rows"] / workers
    p1 = synth.build_problem(synth.config("1"))
    full1 = _sharded_oracle(p1, range(int(p1["meta"]["n_items"])), workers)
    return {
        "value": round(value, 1),
        "unit": f"ms per config-{args.config} solve (fwd+bwd) on {workers} cores, scaled by rows from the sample",
        "cores": workers,
        "kind": "port",
        "sample": (f"float64 numpy oracle (one thread per process), the first {sample['families']} of the "
                   f"config-{args.config} families packed by rows into {sample['shards']} shards on {workers} worker "
                   f"processes: {sample['rows']} of {C} rows, {sample['cpu_s']:.1f} worker CPU-s "
                   f"({sample['wall_s']:.2f} s wall, busiest shard {sample['busiest_shard_s']:.2f} s); "
                   f"value = CPU-s per row x {C} rows / {workers} workers"),
        "host": {"affinity_cores": avail, "workers": workers, "cpu": _cpu_model()},
        "config1_full": {"ms": round(full1["wall_s"] * 1e3, 1), "rows": full1["rows"],
                         "families": full1["families"], "workers": full1["shards"],
                         "note": "BASELINE config 1 (S=127, fp64 oracle) solved in full, fwd+bwd, wall time"},
    }


# ---------------------------------------------------------------------- per-call (drop-in) path
def _time_host(step, warmup: int, steps: int) -> float:
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ts = []
    for _ in range(steps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        step()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t) * 1e3)
    return statistics.median(ts)


def per_call_timings(static, theta, cw, steps: int = 5, static_levels=None) -> dict:
    """ms per solve through the builder's per-call drivers (``kbench.percall``: the wrappers called in the
    reference glue's call sequence, with the wave buckets folded by the library's fixed-order row sums).

    Four timings of the same scope, the forward plus the backward's per-wave reverse sweep, so that
    they compare: one launch per sweep (the pristine-structure proxy), each wave's sweep chain in one
    launch (``KBENCH_FUSE_SWEEPS``), that fused-chain call sequence captured once as two HIP graphs
    and replayed (``kbench.percall.graph.GraphedSolve``), and the same driver with every wrapper
    replaced by a no-op (its Python, torch glue and host syncs alone).  The glue's E adjoint and theta VJP, which follow the
    reverse sweep and do not depend on the wave launches (a BiCGSTAB over E-step products whose
    iteration count depends on the cotangents, so a no-op run would not repeat it), are timed apart;
    the whole solve is the sum.  With ``static_levels`` (the same problem regrouped by
    ``synth.level_waves``) the timings are repeated on one wave per dependency level.
    """
    import torch

    from kbench.core.kernels import wave_step
    from kbench.percall.graph import GraphedSolve
    from kbench.percall.kernels import noop
    from kbench.percall.solve import SolvePlan, root_softmax2

    def waves(p):
        def step():
            _, sv = p.forward(theta, cw)
            with torch.no_grad():
                p.reverse_sweep(sv, -root_softmax2(sv["pi_wave"].index_select(0, p.roots)), use_col=False)
        return step

    def e_side(p):
        _, sv = p.forward(theta, cw)
        with torch.no_grad():
            acc = p.reverse_sweep(sv, -root_softmax2(sv["pi_wave"].index_select(0, p.roots)), use_col=False)
        return lambda: p.e_adjoint_and_vjp(theta, cw, sv, acc, use_col=False)

    def three(st):
        plan = SolvePlan(st)
        floor_plan = SolvePlan(st, kernels=noop())
        old = wave_step.FUSE_SWEEPS
        try:
            wave_step.FUSE_SWEEPS = False
            per_launch = _time_host(waves(plan), 2, steps)
            wave_step.FUSE_SWEEPS = True
            fused = _time_host(waves(plan), 2, steps)
            gs = GraphedSolve(plan, theta, cw)  # captured in the first warm-up call, chains fused

            def graphed():
                _, sv = gs.forward(theta, cw)
                gs.reverse(sv)

            graph_ms = _time_host(graphed, 2, steps)
            del gs
        finally:
            wave_step.FUSE_SWEEPS = old
        torch.cuda.empty_cache()
        floor = _time_host(waves(floor_plan), 2, steps)
        e_ms = _time_host(e_side(plan), 2, steps)
        return {"ms_one_launch_per_sweep": round(per_launch, 3), "ms_sweep_chains_fused": round(fused, 3),
                "ms_graph_replay": round(graph_ms, 3),
                "ms_glue_floor": round(floor, 3), "ms_e_adjoint_and_theta_vjp": round(e_ms, 3),
                "ms_solve_one_launch_per_sweep": round(per_launch + e_ms, 3),
                "ms_solve_sweep_chains_fused": round(fused + e_ms, 3),
                "ms_solve_graph_replay": round(graph_ms + e_ms, 3)}

    out = three(static)
    out["note"] = (
        "host wall time (median of %d) through the builder's call-sequence driver (kbench.percall: the "
        "per-call wrappers in the reference glue's order, wave buckets folded by native fixed-order row sums, "
        "where the frozen glue calls _scatter_accum per bucket): ms_one_launch_per_sweep / "
        "ms_sweep_chains_fused / ms_glue_floor time the forward plus the per-wave reverse sweep with one "
        "launch per sweep and wave (the pristine-structure proxy), with each wave's sweep chain in one launch "
        "(KBENCH_FUSE_SWEEPS=1), and with every wrapper a no-op (same driver code and calls); ms_graph_replay "
        "times the same fused-chain call sequence captured once as two HIP graphs (kbench.percall.graph: "
        "forward and reverse wave loops) and replayed; the glue's E adjoint and theta VJP "
        "(ms_e_adjoint_and_theta_vjp) are timed apart and added in ms_solve_*" % steps)
    if static_levels is not None:
        lv = three(static_levels)
        lv["n_waves"] = len(static_levels.wave_layout["wave_metas"])
        lv["note"] = ("the same timings with the rows regrouped into one wave per dependency level "
                      "(synth.level_waves: same rows, same per-row results, fewer waves, so fewer wrapper calls)")
        out["level_waves"] = lv
    return out


def _unit_directions(theta, n: int, seed: int = 0):
    """``n`` seeded Gaussian directions of theta's size, each normalised to unit length (config 5)."""
    import numpy as np
    import torch

    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        u = g.normal(size=int(theta.numel()))
        out.append(torch.as_tensor(u / np.linalg.norm(u), dtype=theta.dtype, device=theta.device))
    return out


def _tangent_sweep_launches(hvp, u):
    """HIP-event time and algorithmic bytes of every tangent-sweep launch (``wave_tan_pre_kernel``, one per
    level: the HVP's largest kernel) in one eager HVP of ``hvp`` -> (ms list, bytes list).

    The wrapper is looked up by the drivers on every call, so it is replaced for this one HVP; events go
    on torch's current stream, where the wrappers launch.  Bytes per launch: 4*S per row for Pi*, the
    incoming dPi and the outgoing dPi and dPibar rows, plus the split term and its tangent on split rows
    (the constant rows are one [1, S] row each, shared by the launch).
    """
    import inspect

    import torch

    from kbench.core.kernels import wave_tangent as WT

    orig = WT.compute_wave_step_tangent_selfloop
    sig = inspect.signature(orig)
    rec = []

    def timed(*a, **k):
        b = sig.bind(*a, **k)
        W, S = int(b.arguments["W"]), int(b.arguments["S"])
        split = b.arguments.get("DTS_reduced") is not None
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        orig(*a, **k)
        e1.record()
        rec.append((e0, e1, 4.0 * S * W * (6 if split else 4)))

    WT.compute_wave_step_tangent_selfloop = timed
    try:
        with torch.no_grad():
            hvp._tangent_cotangents(u.reshape(hvp.theta.shape).to(hvp.theta.dtype))
        torch.cuda.synchronize()
    finally:
        WT.compute_wave_step_tangent_selfloop = orig
    return [a.elapsed_time(b) for a, b, _ in rec], [x for _, _, x in rec]


def config5_timing(static_levels, theta, cw, warmup: int = 3, n_hvp: int = 50) -> dict:
    """BASELINE config 5 on the config-3 problem: one Newton-CG step's 50 exact HVPs along seeded unit
    Gaussian directions, timed as one block (host wall, synchronised at both ends), through
    ``kbench.newton.make_exact_hvp`` (row classes, one HIP graph per point) on the level waves."""
    import statistics as st

    import torch

    from kbench.newton.hvp import make_exact_hvp
    from kbench.percall.solve import run_forward

    us = _unit_directions(theta, n_hvp + warmup, seed=5)
    _, sv = run_forward(static_levels, theta, cw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hvp = make_exact_hvp(static_levels, theta, cw, sv)
    hvp(us[0])  # the first call captures the graph
    torch.cuda.synchronize()
    cache_ms = (time.perf_counter() - t0) * 1e3
    for u in us[1:warmup]:
        hvp(u)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for u in us[warmup:]:
        hvp(u)
    torch.cuda.synchronize()
    block_ms = (time.perf_counter() - t0) * 1e3
    dur, byt = _tangent_sweep_launches(hvp, us[0])
    avg_ms, avg_b = st.mean(dur), st.mean(byt)
    achieved = avg_b / (avg_ms * 1e-3) / 1e9
    del hvp
    # a Newton step moves theta: the next point's forward, point cache and first (captured) HVP, with
    # the process's one-off set-up (layouts, plans, first launches) already done
    theta2 = theta + 1e-3 * us[0].reshape(theta.shape)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _, sv2 = run_forward(static_levels, theta2, cw)
    hvp2 = make_exact_hvp(static_levels, theta2, cw, sv2)
    hvp2(us[1])
    torch.cuda.synchronize()
    point_ms = (time.perf_counter() - t0) * 1e3
    del hvp2, sv2
    return {
        "ms_per_hvp": round(block_ms / n_hvp, 4),
        "ms_per_newton_cg_step_50_hvps": round(block_ms * 50.0 / n_hvp, 2),
        "point_cache_ms": round(cache_ms, 2),
        "ms_new_point": round(point_ms, 2),
        "ms_per_newton_cg_step_with_new_point": round(point_ms + block_ms * 50.0 / n_hvp, 2),
        "roofline": {"bound": "hbm", "kernel": "wave_tan_pre_kernel", "achieved": round(achieved, 3),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6),
                     "launches": len(dur), "launch_unit": "one tangent-sweep launch per dependency level",
                     "avg_launch_ms": round(avg_ms, 5), "algorithmic_bytes_per_launch": round(avg_b, 1),
                     "kernel_ms_per_hvp": round(sum(dur), 4)},
        "note": (f"{n_hvp} exact HVPs (seeded unit Gaussian directions) after {warmup} warm-up HVPs, timed as "
                 "one block; make_exact_hvp on the level waves: tangent forward and reverse on one row per class "
                 "of identical rows, replayed as one HIP graph; point_cache_ms = the point cache, the class "
                 "schedule and the first (captured) HVP, including the process's one-off set-up; ms_new_point = the "
                 "same at the next point (theta moved by 1e-3 along a unit direction: per-call forward, point "
                 "cache, class schedule, first HVP), which a Newton-CG step pays once besides its 50 HVPs; the "
                 "kernel roofline from HIP events around each tangent-sweep launch of one eager HVP"),
    }


def bench_hvp(args, static, theta, cw, summ, static_levels) -> None:
    """Exact Hessian-vector products (config 5) through the per-call wrappers, on the size waves and on
    one wave per dependency level (``synth.level_waves``; the same HVP, fewer wrapper calls)."""
    import torch

    from kbench.newton.hvp import make_exact_hvp
    from kbench.percall.solve import run_forward

    us = _unit_directions(theta, 4)

    def timed(st, row_classes=False, graph=False):
        _, sv = run_forward(st, theta, cw)
        t0 = time.perf_counter()
        hvp = make_exact_hvp(st, theta, cw, sv, row_classes=row_classes, graph=graph)
        torch.cuda.synchronize()
        cache_ms = (time.perf_counter() - t0) * 1e3
        k = [0]

        def step():
            k[0] += 1
            hvp(us[k[0] % len(us)])

        return _time_host(step, args.warmup, args.steps), cache_ms

    ms_size = cache_size = None
    if args.hvp_layout == "both":
        ms_size, cache_size = timed(static)
    ms_rows = cache_rows = ms_eager = None
    if args.hvp_variants == "all":
        ms_rows, cache_rows = timed(static_levels)
        ms_eager, _ = timed(static_levels, row_classes=True)
    ms, cache_ms = timed(static_levels, row_classes=True, graph=True)
    print(json.dumps({
        "metric": "exact Hessian-vector product ms (config 5: per-species theta, forward tangent + tangent adjoint)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic",
        "config": {"workload": (f"config{args.config} exact HVP through the per-call wrappers, rows in one wave per "
                                f"dependency level ({len(static_levels.wave_layout['wave_metas'])} waves), tangent "
                                "forward and reverse on one row per class of identical rows, replayed as one HIP "
                                "graph"),
                   "S": summ["S"], "C": summ["C"], "point_cache_ms": round(cache_ms, 3)},
        "ms_per_newton_cg_step_50_hvps": round(50 * ms, 2),
        "row_by_row": None if ms_rows is None else {"ms": round(ms_rows, 4), "point_cache_ms": round(cache_rows, 3)},
        "row_classes_without_graph_ms": None if ms_eager is None else round(ms_eager, 4),
        "size_waves": None if ms_size is None else {"n_waves": summ["n_waves"], "ms": round(ms_size, 4),
                                                    "point_cache_ms": round(cache_size, 3)},
    }))


# ---------------------------------------------------------------------- the solve metric
def _counters(kernel_symbol: str, config: str):
    """VALU / LDS figures of the committed rocprofv3 SQ-counter summary for ``kernel_symbol``."""
    f = _profile_file("sq_counters", config)
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get("kernels", {})
    hits = {k: v for k, v in rec.items() if kernel_symbol in k}
    return hits or None


def _traffic(kernel_symbol: str, config: str):
    f = _profile_file("traffic", config)
    if not f.exists():
        return None
    # HBM bytes per dispatch from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this command,
    # scaled by a copy kernel of known size; a kernel launched in several shapes: the
    # dispatch-weighted mean over them
    rec = json.loads(f.read_text()).get("kernels", {})
    hits = [v for k, v in rec.items() if kernel_symbol in k]
    n = sum(float(v["dispatches"]) for v in hits)
    return round(sum(float(v["traffic"]) * float(v["dispatches"]) for v in hits) / n, 1) if n else None


def _timed_solve_calls(solver, theta, cw, steps: int):
    """HIP-event times of ``steps`` one-call solves (``FusedSolver.solve``: the forward and its backward
    in one ``kb_solve``, early families' backward rows beside the forward's later levels) and the host
    wall time per solve; a failed E-adjoint solve raises."""
    import torch

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    for a, b in ev:
        a.record()
        loss = solver.solve(theta, cw, check_solve=False)[0]
        b.record()
        solver.backward_stats()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t_wall) * 1e3 / steps
    return [a.elapsed_time(b) for a, b in ev], wall, loss


def _timed_solves(solver, theta, cw, steps: int):
    """HIP-event times (total, fwd, bwd) of ``steps`` solves as two calls (``run_forward``, then
    ``run_backward``); a failed E-adjoint solve raises."""
    import torch

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    for a, m, b in ev:
        a.record()
        loss, saved = solver.run_forward(theta, cw)
        m.record()
        solver.run_backward(theta, cw, saved, check_solve=False)
        b.record()
        solver.backward_stats()  # raises RuntimeError if the E-adjoint BiCGSTAB failed
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t_wall) * 1e3 / steps
    return ([a.elapsed_time(b) for a, _, b in ev], [a.elapsed_time(m) for a, m, _ in ev],
            [m.elapsed_time(b) for _, m, b in ev], wall, loss)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only (--gpus {args.gpus} requested); this build has no "
              "multi-GPU path: families would shard across GPUs with one all-reduce of O(S) gradient "
              "accumulators, which is not implemented here.", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    from kbench import synth

    t0 = time.time()
    problem = synth.build_problem(synth.config(args.config))
    summ = synth.summary(problem)
    # the CPU baseline forks its workers before anything touches the GPU
    cpu = None if (args.no_cpu_baseline or args.workload != "solve") else cpu_baseline(args, problem)
    log(args, f"[bench] problem + cpu baseline {time.time() - t0:.1f}s {summ}")

    import numpy as np
    import torch

    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cap = problem_to_captured(problem)
    static = make_static(cap, dev)
    theta = cap["inputs"]["theta"].to(dev)
    cw = cap["inputs"]["col_weights"].to(dev)
    static_levels = None
    if args.workload != "solve" or not args.no_per_call or not args.no_config5:
        static_levels = make_static(problem_to_captured(synth.level_waves(problem)[0]), dev)
    if args.workload == "hvp":
        return bench_hvp(args, static, theta, cw, summ, static_levels)
    if args.workload == "glue":
        print(json.dumps({"config": f"config{args.config}",
                          **per_call_timings(static, theta, cw, args.steps, static_levels)}))
        return
    solver = FusedSolver(static, static.solver_options)
    for i in range(args.warmup):
        _timed_solve_calls(solver, theta, cw, 1)
        _timed_solves(solver, theta, cw, 1)
        log(args, f"[bench] warmup {i + 1}/{args.warmup}")
    fstats = solver.forward_stats()

    # ---- timed region 1: whole solves in one call each (value)
    tot, wall, loss = _timed_solve_calls(solver, theta, cw, args.steps)
    ms = statistics.mean(tot)
    bstats = solver.backward_stats()
    # ---- the same solves as two calls (the reference's run_forward / run_backward split)
    tot2, fwd, bwd, wall2, loss2 = _timed_solves(solver, theta, cw, args.steps)
    if float(loss2) != float(loss):
        raise RuntimeError(f"one-call and two-call solves disagree on the loss: {float(loss)} vs {float(loss2)}")
    log(args, f"[bench] timed {args.steps} steps: {ms:.3f} ms/solve in one call (overlap cut {solver.overlap_cut}, "
              f"{solver.overlap_rows} early rows); two calls {statistics.mean(tot2):.3f} (fwd "
              f"{statistics.mean(fwd):.3f}, bwd {statistics.mean(bwd):.3f}), wall {wall:.3f}")

    # ---- timed region 2: per-launch HIP events around every row-kernel launch (roofline), on two-call
    # solves (one launch per level and pass on one stream); the process's forwards number
    # 2 W + 2 K + 1 .. 2 W + 3 K here (W warmup iterations of one one-call and one two-call solve,
    # then K of each timed), the window of a kernel trace that matches these launches
    prof_forwards = [2 * args.warmup + 2 * args.steps + 1, 2 * args.warmup + 3 * args.steps]
    solver.profile(True)
    fw_ms, bw_ms = [], []
    for _ in range(args.steps):
        _, saved = solver.run_forward(theta, cw)
        solver.run_backward(theta, cw, saved)
        fw_ms.append(solver.level_launch_ms("forward"))
        bw_ms.append(solver.level_launch_ms("backward"))
    solver.profile(False)
    fw = np.mean(np.stack(fw_ms), axis=0)
    bw = np.mean(np.stack(bw_ms), axis=0)
    W, Nw = solver.level_shapes()
    B = 4.0 * solver.S
    fwd_bytes = B * (2 * W + 4 * Nw)
    bwd_bytes = B * (3 * W + 8 * Nw)
    # transcendental instructions per position: backward row 8 for the J^T coefficients (six exp2,
    # two reciprocals) and 1 for p', per split 9 (five split shares, two Pibar factors, two p');
    # forward (linear-space sweeps) 2 per row for the row's leaf / merge terms, 6 per split
    # (five exp2 and the merge's log2)
    fwd_trans = solver.S * (2.0 * W + 6.0 * Nw)
    bwd_trans = solver.S * (9.0 * W + 9.0 * Nw)
    trans = {"fwd_row_kernel": fwd_trans, "bwd_row_kernel": bwd_trans}
    kernels = {"fwd_row_kernel": (fw, fwd_bytes), "bwd_row_kernel": (bw, bwd_bytes)}
    dom = max(kernels, key=lambda k: kernels[k][0].sum())
    dur, byt = kernels[dom]
    # rows of more than 2048 states run the backward's low-register kernel
    sym = "bwd_row_large_kernel" if dom == "bwd_row_kernel" and solver.S > 2048 else dom
    avg_ms = float(dur.mean())
    avg_bytes = float(byt.mean())
    achieved = avg_bytes / (avg_ms * 1e-3) / 1e9
    counters = _counters(sym, args.config)
    trans_rate = float(trans[dom].mean()) / (avg_ms * 1e-3)
    valu = None
    if counters:
        nd = sum(float(c["dispatches"]) for c in counters.values())
        valu = sum(float(c["valu_active_frac"]) * float(c["dispatches"]) for c in counters.values()) / nd
    roofs = {"hbm": achieved / HBM_PEAK_GBS, "transcendental": trans_rate / TRANS_PEAK_PER_S}
    if valu is not None:
        roofs["valu_issue"] = valu
    nearest = max(roofs, key=roofs.get)
    limiter = (f"{nearest} ({roofs[nearest]:.2f} of its peak)" if roofs[nearest] >= 0.5 else
               f"latency: no roof above half of its peak (HBM {roofs['hbm']:.2f}, transcendental "
               f"{roofs['transcendental']:.2f}" + (f", VALU active {valu:.2f} of wave cycles" if valu is not None
                                                   else "") + "); the time goes to barriers, LDS and memory latency")
    roofline = {
        # the line's roofs are HBM or MFMA; the row kernels issue no MFMA, so the memory roof is the one
        # quoted, and `limiter` says which of the measured roofs (HBM, transcendental, VALU issue) is nearest
        "bound": "hbm",
        "kernel": sym,
        "achieved": round(achieved, 3),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 6),
        "traffic": _traffic(sym, args.config),
        "launches": int(len(dur)),
        "launch_unit": "one launch per clade-DAG dependency level",
        "events_over_forwards": prof_forwards,
        "avg_launch_ms": round(avg_ms, 5),
        "algorithmic_bytes_per_launch": round(avg_bytes, 1),
        "kernel_ms_per_solve": {k: round(float(v[0].sum()), 4) for k, v in kernels.items()},
        "compute": {"transcendental_ops_per_launch": round(float(trans[dom].mean()), 1),
                    "achieved_per_s": round(trans_rate, 1), "peak_per_s": TRANS_PEAK_PER_S,
                    "frac": round(trans_rate / TRANS_PEAK_PER_S, 6),
                    "valu_active_frac": None if valu is None else round(valu, 4),
                    "note": ("no dense contraction, so no MFMA roof: the compute side is the quarter-rate "
                             "transcendental unit (algorithmic count per position from the kernel's formulas) "
                             "and VALU issue (SQ counters of the committed profile, dispatch-weighted)")},
        "limiter": limiter,
        "counters": counters,
    }
    whole_bytes = float(fwd_bytes.sum() + bwd_bytes.sum())

    # ---- the same solve with every row computed (row classes off)
    dedup_off = None
    if not args.no_dedup_off:
        old = os.environ.get("KB_DEDUP")
        os.environ["KB_DEDUP"] = "0"
        try:
            flat = FusedSolver(static, static.solver_options)
        finally:
            if old is None:
                os.environ.pop("KB_DEDUP")
            else:
                os.environ["KB_DEDUP"] = old
        _timed_solve_calls(flat, theta, cw, 2)
        _timed_solves(flat, theta, cw, 1)
        t_one = _timed_solve_calls(flat, theta, cw, max(3, args.steps // 2))[0]
        t_all, f_all, b_all, _, _ = _timed_solves(flat, theta, cw, max(3, args.steps // 2))
        dedup_off = {"ms": round(statistics.mean(t_one), 4), "ms_two_calls": round(statistics.mean(t_all), 4),
                     "fwd_ms": round(statistics.mean(f_all), 4), "bwd_ms": round(statistics.mean(b_all), 4)}
        del flat
    # ---- the Neumann series: terms per solved row at the solver's early stop, and the same solve
    # with every term summed (the reference's series, neumann_rtol = 0)
    _, saved_n = solver.run_forward(theta, cw)
    terms = solver.run_backward(theta, cw, saved_n, return_info=True)[2]["neumann_terms"].cpu().numpy()
    terms = terms[terms != 255]
    neumann = {"neumann_terms": int(solver.so["neumann_terms"]), "rtol": solver.neumann_rtol,
               "terms_mean": round(float(terms.mean()), 3), "terms_max": int(terms.max()),
               "note": ("each row's series stops at its first term whose entries are all at most rtol times the "
                        "row's largest right-hand-side entry (the term included); ms_full_series times the same "
                        "solve summing every term")}
    if not args.no_dedup_off:
        full = FusedSolver(static, static.solver_options, neumann_rtol=0.0)
        _timed_solve_calls(full, theta, cw, 2)
        _timed_solves(full, theta, cw, 1)
        t_one = _timed_solve_calls(full, theta, cw, max(3, args.steps // 2))[0]
        t_all, f_all, b_all, _, _ = _timed_solves(full, theta, cw, max(3, args.steps // 2))
        neumann.update(ms_full_series=round(statistics.mean(t_one), 4),
                       ms_two_calls_full_series=round(statistics.mean(t_all), 4),
                       bwd_ms_full_series=round(statistics.mean(b_all), 4))
        del full
    per_call = None if args.no_per_call else per_call_timings(static, theta, cw, static_levels=static_levels)
    if per_call is not None:
        # the whole-pass solve against the pristine-structure proxy on the same GPU
        per_call["speedup_vs_pristine_structure_proxy"] = round(per_call["ms_solve_one_launch_per_sweep"] / ms, 2)
    config5 = None
    if not args.no_config5 and not solver.statewise:
        config5 = {"skipped": "config 5 asks for per-species theta"}
    elif not args.no_config5:
        config5 = config5_timing(static_levels, theta, cw)

    out = {
        "metric": "fwd+bwd ms per solve at S=1024,C=32k; achieved HBM GB/s vs roofline",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded Yule tree + DTL families + NNI variants; random theta in [-3,-1])",
        "config": {
            "workload": (f"config{args.config}: fwd+bwd solve, S={summ['S']} columns ({(summ['S'] + 1) // 2} "
                         f"leaves), C={summ['C']} rows, {summ['n_waves']} waves, {summ['n_splits']} splits, "
                         f"per-species theta, pi_iters=16, neumann_terms=16 (early stop at rtol {solver.neumann_rtol:.3g}, "
                         f"{neumann['terms_mean']:.2f} terms per row on average); row classes: the forward computes "
                         f"{solver.n_forward_rows} of {summ['C']} rows (identical rows written from one "
                         f"computation), the backward solves {solver.n_backward_rows}; one call per solve, "
                         f"{solver.overlap_rows} backward rows beside the forward's levels above {solver.overlap_cut}"),
            "S_leaves": (summ["S"] + 1) // 2,
            "S_columns": summ["S"],
            "C": summ["C"],
            "n_waves": summ["n_waves"],
            "n_splits": summ["n_splits"],
            "n_families": summ["n_families"],
            "forward_rows_computed": solver.n_forward_rows,
            "backward_rows_solved": solver.n_backward_rows,
        },
        "overlap": {"cut": solver.overlap_cut, "early_rows": solver.overlap_rows,
                    "note": ("value times one kb_solve call per solve: the backward rows of the families whose "
                             "root lies at or below dependency level `cut` run on a second stream beside the "
                             "forward's later levels (-1: no overlap, the two passes in order); two_calls times "
                             "run_forward then run_backward, the reference's split, with fwd_ms / bwd_ms")},
        "two_calls": {"ms": round(statistics.mean(tot2), 4), "median_ms": round(statistics.median(tot2), 4),
                      "host_wall_ms_per_step": round(wall2, 4)},
        "fwd_ms": round(statistics.mean(fwd), 4),
        "bwd_ms": round(statistics.mean(bwd), 4),
        "median_ms": round(statistics.median(tot), 4),
        "min_ms": round(min(tot), 4),
        "host_wall_ms_per_step": round(wall, 4),
        "dedup_off": dedup_off,
        "neumann": neumann,
        "hbm_gbps_whole_solve": round(whole_bytes / (ms * 1e-3) / 1e9, 3),
        "e_step_iters": fstats["n_e_iter"],
        "bicgstab_iters": bstats["n_bicgstab"],
        "loss": float(loss),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_call": per_call,
        "config5": config5,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
