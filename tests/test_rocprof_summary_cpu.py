"""``kbench.rocprof_summary``: per-kernel statistics over a window of dispatches.

A kernel trace and a counter file written by hand (rocprofv3's CSV columns)
with three "solves", each one marker dispatch followed by two row-kernel
dispatches, the middle solve's on two streams out of start-time order.  The
window ``marker:2:2`` must hold exactly the second solve's dispatches, by
dispatch order; without a window every dispatch counts.
"""

import csv

import pytest

from kbench import rocprof_summary as R

TRACE_COLS = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
COUNTER_COLS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]

# (dispatch id, kernel, start ns, end ns)
DISPATCHES = [
    (1, "kb::estep_pre_kernel<1024, 2>(...)", 0, 1000),
    (2, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 1000, 3000),
    (3, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 3000, 7000),
    (4, "kb::estep_pre_kernel<1024, 2>(...)", 10000, 11000),
    (5, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 13000, 23000),  # second stream: starts after 6
    (6, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 12000, 32000),
    (7, "kb::estep_pre_kernel<1024, 2>(...)", 40000, 41000),
    (8, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 41000, 42000),
    (9, "kb::bwd_row_kernel<1024, 2, false, true>(...)", 42000, 43000),
]


def _write(tmp_path):
    d = tmp_path / "trace"
    d.mkdir()
    with open(d / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_ALL)
        w.writerow(TRACE_COLS)
        for i, k, a, b in DISPATCHES:
            w.writerow(["KERNEL_DISPATCH", i, k, a, b])
    counters = tmp_path / "run_counter_collection.csv"
    with open(counters, "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_ALL)
        w.writerow(COUNTER_COLS)
        for i, k, a, b in DISPATCHES:
            w.writerow([i, k, "FETCH_SIZE", float(i)])
    return d, counters


def test_window_holds_the_second_solve(tmp_path):
    d, _ = _write(tmp_path)
    rows = {r["kernel"]: r for r in R.window_stats(str(d), "estep_pre:2:2")}
    bwd = rows["kb::bwd_row_kernel<1024, 2, false, true>(...)"]
    assert bwd["calls"] == 2
    assert bwd["avg_us"] == pytest.approx((10.0 + 20.0) / 2)
    assert bwd["min_us"] == pytest.approx(10.0) and bwd["max_us"] == pytest.approx(20.0)
    assert rows["kb::estep_pre_kernel<1024, 2>(...)"]["calls"] == 1
    assert sum(r["pct"] for r in rows.values()) == pytest.approx(100.0)
    both = {r["kernel"]: r for r in R.window_stats(str(d), "estep_pre:1:3")}
    assert both["kb::bwd_row_kernel<1024, 2, false, true>(...)"]["calls"] == 6
    with pytest.raises(ValueError):
        R.window_stats(str(d), "estep_pre:2:4")


def test_counter_means_over_a_window(tmp_path):
    _, counters = _write(tmp_path)
    name = "kb::bwd_row_kernel<1024, 2, false, true>(...)"
    assert R._counter_means(str(counters), "FETCH_SIZE", "estep_pre:2:2")[name] == (2, 5.5)
    assert R._counter_means(str(counters), "FETCH_SIZE")[name] == (6, (2 + 3 + 5 + 6 + 8 + 9) / 6)
    assert R._counter_means(str(counters), "FETCH_SIZE", "estep_pre:3:3")[name] == (2, 8.5)
