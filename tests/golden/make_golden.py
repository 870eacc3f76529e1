"""Write the golden fixtures of the CPU test suite (run from the repository root).

    python tests/golden/make_golden.py

The reference holds no golden vectors for this path (its fixtures/ and data/
directories are git-ignored and absent), so the fixtures here are regression
anchors produced by this repository's own generator and float64 oracle, whose
correctness is pinned separately (tests/test_oracle_pins.py).  Each fixture
records, for one generated problem: the generator's layout digest, the
problem summary, and the oracle's loss, E and gradients.
"""

from __future__ import annotations

import dataclasses
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "kernel-bench_amd"), str(ROOT / "oracle")]

import kbench_oracle as O  # noqa: E402
from kbench import synth  # noqa: E402

CASES = {
    "tiny": ("tiny", None),
    "config1": ("1", None),
    "config1_statewise": ("1", True),
}


def make(name: str, statewise):
    cfg = synth.config(name)
    if statewise is not None:
        cfg = dataclasses.replace(cfg, statewise=statewise)
    p = synth.build_problem(cfg)
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    loss, saved = O.forward(prob, theta, cw)
    gt, gc, info = O.backward(prob, theta, cw, saved)
    return p, {
        "loss": np.float64(loss), "E": np.asarray(saved["E"], np.float64),
        "root_rows": np.asarray(saved["root_rows"], np.float64),
        "grad_theta": np.asarray(gt, np.float64), "grad_col": np.asarray(gc, np.float64),
        "n_e_iter": np.int64(saved["n_e_iter"]), "n_bicgstab": np.int64(info["n_bicgstab"]),
    }


def main():
    out = Path(__file__).resolve().parent
    index = {}
    for key, (name, statewise) in CASES.items():
        p, arrays = make(name, statewise)
        np.savez_compressed(out / f"{key}.npz", **arrays)
        index[key] = {"config": name, "statewise": statewise, "digest": synth.layout_digest(p),
                      "summary": synth.summary(p), "loss": float(arrays["loss"])}
        print(key, index[key]["summary"], f"loss={index[key]['loss']:.12g}")
    (out / "index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
