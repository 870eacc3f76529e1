"""Summaries of rocprofv3 CSV output for the solver's kernels.

Two sub-commands, both reading the CSV files rocprofv3 writes with
``--output-format csv``:

``stats DIR``
    Per-kernel table from ``DIR/*_kernel_stats.csv`` (calls, average and total
    duration, share of GPU time), as Markdown.  With ``--window K:FIRST:LAST``
    the table is computed from ``DIR/*_kernel_trace.csv`` instead, over the
    dispatches from the FIRST-th dispatch of the kernel whose name contains K
    (counted from 1) up to, not including, its (LAST+1)-th: e.g. the solves
    of one timed pass of a benchmark, counted by a kernel that runs once per
    solve.

``sq CSV [--json] [--window K:FIRST:LAST]``
    Per-kernel SQ counters of one ``--pmc`` run divided by ``SQ_WAVES``; with
    ``--json`` also the fractions of wave cycles spent issuing VALU
    (``SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES``) and waiting on LDS
    (``SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES``), both counters in the same
    (quad-cycle) units.

``traffic --fetch F --write W --cal-fetch CF --cal-write CW [--window K:FIRST:LAST]``
    HBM bytes per dispatch of each solver kernel from two ``--pmc`` runs
    (``FETCH_SIZE``, then ``WRITE_SIZE``; both in KiB per dispatch), each scaled
    by what the same counter reads for a plain copy kernel of known size
    (``bench.py --calibrate-copy``).  Prints JSON: per kernel the average
    fetched and written bytes per dispatch and their sum (``traffic``).

    python -m kbench.rocprof_summary traffic --fetch pmc_fetch/run_counter_collection.csv ...
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
from collections import defaultdict


def _short(name: str) -> str:
    name = re.sub(r"\(.*$", "", name)
    name = re.sub(r"^void ", "", name)
    return name


def kernel_stats(path: str) -> list[dict]:
    files = glob.glob(os.path.join(path, "*kernel_stats.csv")) if os.path.isdir(path) else [path]
    if not files:
        raise FileNotFoundError(f"no *kernel_stats.csv under {path}")
    out = []
    with open(files[0], newline="") as fh:
        for r in csv.DictReader(fh):
            out.append({
                "kernel": r["Name"],
                "calls": int(r["Calls"]),
                "total_ms": float(r["TotalDurationNs"]) / 1e6,
                "avg_us": float(r["AverageNs"]) / 1e3,
                "min_us": float(r["MinNs"]) / 1e3,
                "max_us": float(r["MaxNs"]) / 1e3,
                "pct": float(r["Percentage"]),
            })
    return out


def _window(rows, window: str | None):
    """The rows of the dispatches inside ``window`` = "K:FIRST:LAST", in dispatch order: from the
    FIRST-th dispatch of the kernel whose name contains K (from 1) up to, not including, its
    (LAST+1)-th.  Without a window, every row."""
    if not window:
        return list(rows)
    marker, a, b = window.rsplit(":", 2)
    first, last = int(a), int(b)
    seen, inside, out, prev = 0, False, [], None
    for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
        if marker in r["Kernel_Name"] and r["Dispatch_Id"] != prev:
            seen += 1
            inside = first <= seen <= last
        prev = r["Dispatch_Id"]
        if inside:
            out.append(r)
    if seen < last:
        raise ValueError(f"{marker!r} dispatched {seen} times, fewer than {last}")
    return out


def window_stats(path: str, window: str) -> list[dict]:
    """Per-kernel statistics of the dispatches inside ``window`` (see ``stats``)."""
    files = glob.glob(os.path.join(path, "*kernel_trace.csv")) if os.path.isdir(path) else [path]
    if not files:
        raise FileNotFoundError(f"no *kernel_trace.csv under {path}")
    with open(files[0], newline="") as fh:
        rows = _window(csv.DictReader(fh), window)
    dur = defaultdict(list)
    for r in rows:
        dur[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in dur.values())
    out = [{"kernel": k, "calls": len(v), "total_ms": sum(v) / 1e3, "avg_us": sum(v) / len(v), "min_us": min(v),
            "max_us": max(v), "pct": 100.0 * sum(v) / total} for k, v in dur.items()]
    return sorted(out, key=lambda r: -r["total_ms"])


def stats_markdown(path: str, top: int = 20, window: str | None = None) -> str:
    if window:
        rows = window_stats(path, window)
    else:
        rows = kernel_stats(path)
    lines = ["| kernel | calls | avg us | min us | max us | total ms | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        lines.append(f"| `{_short(r['kernel'])[:90]}` | {r['calls']} | {r['avg_us']:.1f} | {r['min_us']:.1f} | "
                     f"{r['max_us']:.1f} | {r['total_ms']:.2f} | {r['pct']:.2f} |")
    return "\n".join(lines)


def _counter_means(path: str, counter: str, window: str | None = None) -> dict[str, tuple[int, float]]:
    acc = defaultdict(list)
    with open(path, newline="") as fh:
        for r in _window(csv.DictReader(fh), window):
            if r["Counter_Name"] == counter:
                acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: (len(v), sum(v) / len(v)) for k, v in acc.items()}


def _calibration(path: str, counter: str, expected_bytes: float) -> float:
    """bytes per counter unit, from the largest dispatch of the copy run."""
    best = 0.0
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] == counter:
                best = max(best, float(r["Counter_Value"]))
    if best <= 0:
        raise ValueError(f"{path}: no {counter} reading for the copy kernel")
    return expected_bytes / best


def traffic(fetch: str, write: str, cal_fetch: str, cal_write: str, cal_bytes: float, prefix: str = "kb::",
            window: str | None = None) -> dict:
    f_scale = _calibration(cal_fetch, "FETCH_SIZE", cal_bytes)
    w_scale = _calibration(cal_write, "WRITE_SIZE", cal_bytes)
    fm = _counter_means(fetch, "FETCH_SIZE", window)
    wm = _counter_means(write, "WRITE_SIZE", window)
    out = {"calibration": {"copy_bytes": cal_bytes, "fetch_bytes_per_unit": f_scale,
                           "write_bytes_per_unit": w_scale}, "kernels": {}}
    for name in sorted(set(fm) | set(wm)):
        if prefix and prefix not in name:
            continue
        n_f, f = fm.get(name, (0, 0.0))
        n_w, w = wm.get(name, (0, 0.0))
        out["kernels"][_short(name)] = {
            "dispatches": max(n_f, n_w),
            "fetch_bytes": f * f_scale,
            "write_bytes": w * w_scale,
            "traffic": f * f_scale + w * w_scale,
        }
    return out


def _sq_totals(path: str, prefix: str, window: str | None = None):
    tot = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(set)
    with open(path, newline="") as fh:
        for r in _window(csv.DictReader(fh), window):
            if prefix and prefix not in r["Kernel_Name"]:
                continue
            k = _short(r["Kernel_Name"])
            tot[k][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[k].add(r["Dispatch_Id"])
    return tot, disp


def sq_json(path: str, prefix: str = "kb::", window: str | None = None) -> dict:
    """Per-kernel SQ counters per wave and the VALU-issue / LDS-wait fractions of wave cycles."""
    tot, disp = _sq_totals(path, prefix, window)
    out = {}
    for k, v in tot.items():
        w = v.get("SQ_WAVES", 0.0)
        cyc = v.get("SQ_WAVE_CYCLES", 0.0)
        rec = {"dispatches": len(disp[k]), "waves": w}
        rec.update({f"{c}_per_wave": v[c] / w for c in v if c != "SQ_WAVES" and w})
        if cyc:
            if "SQ_ACTIVE_INST_VALU" in v:
                rec["valu_active_frac"] = v["SQ_ACTIVE_INST_VALU"] / cyc
            if "SQ_WAIT_INST_LDS" in v:
                rec["lds_wait_frac"] = v["SQ_WAIT_INST_LDS"] / cyc
        out[k] = rec
    return {"source": "rocprofv3 --pmc SQ counters", "kernels": out}


def sq_markdown(path: str, prefix: str = "kb::", window: str | None = None) -> str:
    """Per-kernel SQ counter totals of one ``--pmc`` run, normalised per wave."""
    tot, disp = _sq_totals(path, prefix, window)
    names = sorted({c for v in tot.values() for c in v})
    per_wave = [c for c in names if c != "SQ_WAVES"]
    head = "| kernel | dispatches | waves | " + " | ".join(f"{c} / wave" for c in per_wave) + " |"
    lines = [head, "|---|" + "---:|" * (2 + len(per_wave))]
    for k, v in sorted(tot.items(), key=lambda kv: -kv[1].get("SQ_INSTS_VALU", 0.0)):
        w = v.get("SQ_WAVES", 0.0)
        cells = [f"{v[c] / w:.0f}" if w else "-" for c in per_wave]
        lines.append(f"| `{k[:60]}` | {len(disp[k])} | {w:.0f} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("dir")
    a.add_argument("--top", type=int, default=20)
    a.add_argument("--window", help="KERNEL:FIRST:LAST, from the kernel trace (see the module docstring)")
    b = sub.add_parser("traffic")
    b.add_argument("--fetch", required=True)
    b.add_argument("--write", required=True)
    b.add_argument("--cal-fetch", required=True)
    b.add_argument("--cal-write", required=True)
    b.add_argument("--cal-mib", type=float, default=512.0)
    b.add_argument("--window", help="KERNEL:FIRST:LAST over the fetch and write runs")
    c = sub.add_parser("sq")
    c.add_argument("csv")
    c.add_argument("--json", action="store_true")
    c.add_argument("--window", help="KERNEL:FIRST:LAST")
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(stats_markdown(args.dir, args.top, args.window))
    elif args.cmd == "sq":
        print(json.dumps(sq_json(args.csv, window=args.window), indent=1) if args.json
              else sq_markdown(args.csv, window=args.window))
    else:
        print(json.dumps(traffic(args.fetch, args.write, args.cal_fetch, args.cal_write, args.cal_mib * (1 << 20),
                                 window=args.window), indent=1))


if __name__ == "__main__":
    main()
