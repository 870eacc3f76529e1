#!/usr/bin/env python
"""Benchmark of the log-space solver path on one MI355X.

Workload: Yule species tree with 1024 leaves (S = 2047 state
columns), 500 DTL-simulated families with 3 NNI variants each (C ~ 33.7k clade
rows in size-waves), per-species theta, fp32, pi_iters = 16, neumann_terms = 16.
A step is one whole solve: forward (E-step fixed point, all waves, loss) plus
backward (adjoint over all waves, E adjoint, theta / column VJP), run through
the native whole-pass driver with every input already in HBM.

Prints ONE JSON line (rank 0).  ``value`` is ms per solve (fwd + bwd), lower is
better.  ``roofline`` reports the dominant wave kernel: algorithmic HBM bytes
per launch (S*4 bytes per row: forward writes Pi and Pibar and reads four child
rows per split; backward reads Pi*, Pibar* and the adjoint per row and four
child rows plus two adjoint rows per split) divided by its launch durations,
measured with HIP events on the launch stream in a second timed pass.
``cpu_baseline`` times the float64 CPU oracle on a bounded sample of the same
workload (the config-3 species tree with its first 20 families) and scales it
by row count to one full solve.
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
TRAFFIC_FILE = ROOT / "profiles" / "traffic_config3.json"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-families", type=int, default=20)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--workload", choices=("solve", "glue", "hvp"), default="solve",
                    help="solve: whole-pass driver (the metric); glue: the same solve through the per-wrapper "
                         "drop-in path; hvp: exact Hessian-vector products of the config-5 Newton-CG setup")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 plain copy kernels of MIB MiB (read + write), the reference point "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters to HBM bytes")
    return ap.parse_args()


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


def log(args, msg):
    if args.verbose:
        print(msg, file=sys.stderr, flush=True)


def cpu_baseline(args, full_rows: int) -> dict:
    """Oracle fwd+bwd on the config's tree with its first families, scaled by rows."""
    import dataclasses

    os.environ.setdefault("OMP_NUM_THREADS", "1")
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np

    import kbench_oracle as O
    from kbench import synth

    cfg = dataclasses.replace(synth.config(args.config), n_families=args.cpu_sample_families)
    p = synth.build_problem(cfg)
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    t0 = time.perf_counter()
    _, saved = O.forward(prob, theta, cw)
    O.backward(prob, theta, cw, saved)
    dt = time.perf_counter() - t0
    rows = int(p["meta"]["C"])
    return {
        "value": dt * 1e3 * full_rows / rows,
        "unit": "ms per solve (fwd+bwd, scaled by rows)",
        "cores": 1,
        "kind": "port",
        "sample": (f"float64 numpy oracle, config-{args.config} species tree with its first "
                   f"{args.cpu_sample_families} families ({rows} of {full_rows} rows), fwd+bwd "
                   f"{dt:.2f} s on 1 host core, scaled by {full_rows}/{rows}"),
    }


def bench_other(args, static, theta, cw, summ) -> None:
    """Secondary workloads (not the metric): the per-wrapper solve and the exact HVP."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "tests"))  # the call-sequence drivers of the per-call wrappers
    from dropin.solve import plan_of, run_backward, run_forward

    cfg = {"S_columns": summ["S"], "C": summ["C"], "n_waves": summ["n_waves"], "n_splits": summ["n_splits"]}
    if args.workload == "glue":
        def step():
            loss, sv = run_forward(static, theta, cw)
            run_backward(static, theta, cw, sv)
            return loss

        metric = "fwd+bwd ms per solve through the per-wrapper drop-in path (reference glue call sequence)"
    else:
        from dropin.hvp import HvpPlan

        loss, sv = run_forward(static, theta, cw)
        t0 = time.perf_counter()
        hvp = HvpPlan(plan_of(static), theta, cw, sv)
        torch.cuda.synchronize()
        cfg["point_cache_ms"] = round((time.perf_counter() - t0) * 1e3, 3)
        g = np.random.default_rng(0)
        us = [torch.as_tensor(g.normal(size=tuple(theta.shape)), dtype=theta.dtype, device=theta.device).reshape(-1)
              for _ in range(4)]
        k = [0]

        def step():
            k[0] += 1
            return hvp(us[k[0] % len(us)])

        metric = "exact Hessian-vector product ms (config 5: per-species theta, forward tangent + tangent adjoint)"
    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(args, f"[bench] warmup {i + 1}/{args.warmup}")
    times = []
    for i in range(args.steps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t) * 1e3)
        log(args, f"[bench] step {i + 1}/{args.steps}: {times[-1]:.3f} ms")
    ms = statistics.mean(times)
    out = {"metric": metric, "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": dict(workload=f"config{args.config} {args.workload}", **cfg),
           "median_ms": round(statistics.median(times), 4), "min_ms": round(min(times), 4)}
    if args.workload == "hvp":
        out["ms_per_newton_cg_step_50_hvps"] = round(50 * ms, 2)
    print(json.dumps(out))


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
    import numpy as np
    import torch

    from kbench import synth
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    t0 = time.time()
    problem = synth.build_problem(synth.config(args.config))
    summ = synth.summary(problem)
    cap = problem_to_captured(problem)
    static = make_static(cap, dev)
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].to(dev)
    cw = cap["inputs"]["col_weights"].to(dev)
    log(args, f"[bench] setup {time.time() - t0:.1f}s {summ}")
    if args.workload != "solve":
        return bench_other(args, static, theta, cw, summ)

    def step():
        loss, saved = solver.run_forward(theta, cw)
        gt, gc = solver.run_backward(theta, cw, saved)
        return loss, gt, gc

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(args, f"[bench] warmup {i + 1}/{args.warmup}")
    fstats = solver.forward_stats()
    bstats = solver.backward_stats()

    # ---- timed region 1: whole solves (value)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t_wall = time.perf_counter()
    for i in range(args.steps):
        a, m, b = ev[i]
        a.record()
        loss, saved = solver.run_forward(theta, cw)
        m.record()
        gt, gc = solver.run_backward(theta, cw, saved)
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t_wall) * 1e3 / args.steps
    tot = [a.elapsed_time(b) for a, _, b in ev]
    fwd = [a.elapsed_time(m) for a, m, _ in ev]
    bwd = [m.elapsed_time(b) for _, m, b in ev]
    ms = statistics.mean(tot)
    log(args, f"[bench] timed {args.steps} steps: {ms:.3f} ms/solve (fwd {statistics.mean(fwd):.3f}, "
              f"bwd {statistics.mean(bwd):.3f}), wall {wall:.3f}")
    bstats = solver.backward_stats()

    # ---- timed region 2: per-launch HIP events around every wave kernel (roofline)
    solver.profile(True)
    fw_ms, bw_ms = [], []
    for i in range(args.steps):
        loss, saved = solver.run_forward(theta, cw)
        gt, gc = solver.run_backward(theta, cw, saved)
        fw_ms.append(solver.level_launch_ms("forward"))
        bw_ms.append(solver.level_launch_ms("backward"))
    solver.profile(False)
    fw = np.mean(np.stack(fw_ms), axis=0)
    bw = np.mean(np.stack(bw_ms), axis=0)
    W, Nw = solver.level_shapes()
    B = 4.0 * solver.S
    fwd_bytes = B * (2 * W + 4 * Nw)
    bwd_bytes = B * (3 * W + 8 * Nw)
    kernels = {
        "fwd_wave_kernel": (fw, fwd_bytes),
        "bwd_wave_kernel": (bw, bwd_bytes),
    }
    symbol = {"fwd_wave_kernel": "fwd_row_kernel", "bwd_wave_kernel": "bwd_row_kernel"}
    dom = max(kernels, key=lambda k: kernels[k][0].sum())
    dur, byt = kernels[dom]
    avg_ms = float(dur.mean())
    avg_bytes = float(byt.mean())
    achieved = avg_bytes / (avg_ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists() and args.config == "3":
        # HBM bytes per dispatch from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this
        # command, scaled by a copy kernel of known size (kbench.rocprof_summary)
        rec = json.loads(TRAFFIC_FILE.read_text()).get("kernels", {})
        # (a kernel launched in several shapes: dispatch-weighted mean over them)
        hits = [v for k, v in rec.items() if symbol[dom] in k]
        n = sum(float(v["dispatches"]) for v in hits)
        traffic = round(sum(float(v["traffic"]) * float(v["dispatches"]) for v in hits) / n, 1) if n else None
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 3),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 6),
        "traffic": traffic,
        "launches": int(len(dur)),
        "launch_unit": "one launch per clade-DAG dependency level",
        "avg_launch_ms": round(avg_ms, 5),
        "algorithmic_bytes_per_launch": round(avg_bytes, 1),
        "kernel_ms_per_solve": {k: round(float(v[0].sum()), 4) for k, v in kernels.items()},
    }
    whole_bytes = float(fwd_bytes.sum() + bwd_bytes.sum())

    cpu = None if args.no_cpu_baseline else cpu_baseline(args, int(summ["C"]))
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
            "workload": f"config{args.config}: fwd+bwd solve, S={summ['S']} columns "
                        f"({(summ['S'] + 1) // 2} leaves), C={summ['C']} rows, {summ['n_waves']} waves, "
                        f"{summ['n_splits']} splits, per-species theta, pi_iters=16, neumann_terms=16",
            "S_leaves": (summ["S"] + 1) // 2,
            "S_columns": summ["S"],
            "C": summ["C"],
            "n_waves": summ["n_waves"],
            "n_splits": summ["n_splits"],
            "n_families": summ["n_families"],
        },
        "fwd_ms": round(statistics.mean(fwd), 4),
        "bwd_ms": round(statistics.mean(bwd), 4),
        "median_ms": round(statistics.median(tot), 4),
        "min_ms": round(min(tot), 4),
        "host_wall_ms_per_step": round(wall, 4),
        "hbm_gbps_whole_solve": round(whole_bytes / (ms * 1e-3) / 1e9, 3),
        "e_step_iters": fstats["n_e_iter"],
        "bicgstab_iters": bstats["n_bicgstab"],
        "loss": float(loss),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
