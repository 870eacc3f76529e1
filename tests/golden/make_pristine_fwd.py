"""Write the reference's own forward outputs on config 1 as fixtures (run in the build container only).

The truncated forward schedule -- pi_iters - 1 sweeps per wave, leaf waves
from the leaf initialisation, split waves from their split term -- has no
closed form to pin it, so this script runs the reference itself: its frozen
glue (kbench/runtime.py:63-75 -> core/inference/solver.py, forward.py) over
its pristine Triton kernels (experiments/pristine_kernels/*.py, registered
under the kernel module names the glue imports), interpreted on the CPU
(TRITON_INTERPRET=1), on the problems this
repository generates.  It needs /root/reference and triton; the GPU box has
neither and only reads the fixtures.

Fixtures (tests/golden/pristine_fwd_<case>.npz): the problem's layout digest
and theta, pi_iters, and the reference's loss, E, E_s1, E_s2, Ebar, pi_wave,
pibar_wave and pibar_row_max.  Cases: config 1 with global theta at
pi_iters 16 and 4, config 1 with per-species theta at 16; config 2 (S = 511,
multi-split rows, e_tol 1e-6) at pi_iters 16, whose fixture keeps every row
maximum, the root rows of pi_wave and a seeded sample of 192 other rows of
pi_wave and pibar_wave (``rows``), to stay small.

    python tests/golden/make_pristine_fwd.py [case ...]

Python's bytecode cache is off, so the run writes nothing into the reference
tree.
"""

from __future__ import annotations

import importlib.util
import os
import sys
from pathlib import Path

sys.dont_write_bytecode = True  # nothing written under /root/reference

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REFERENCE = Path("/root/reference")

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402


def _load(name: str, path: Path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


# this repository's generator, loaded by path (its package name clashes with the reference's)
synth = _load("kb_synth_generator", REPO / "kernel-bench_amd" / "kbench" / "synth.py")


def _captured(problem: dict, pi_iters: int):
    import torch

    def conv(x):
        if isinstance(x, np.ndarray):
            return torch.from_numpy(x.astype(np.float32) if x.dtype == np.float64 else x)
        if isinstance(x, dict):
            return {k: conv(v) for k, v in x.items()}
        if isinstance(x, list):
            return [conv(v) for v in x]
        return x

    st = problem["static"]
    so = dict(problem["meta"]["solver_options"], pi_iters=int(pi_iters))
    return {
        "meta": dict(problem["meta"], solver_options=so),
        "static": {k: conv(st[k]) for k in ("wave_layout", "state_helpers", "rate_item_idx")}
        | {"itemwise": st["itemwise"], "statewise": st["statewise"]},
        "inputs": {k: conv(v) for k, v in problem["inputs"].items()},
    }


def main():
    import dataclasses

    sys.path.insert(0, str(REFERENCE))
    pristine = REFERENCE / "experiments" / "pristine_kernels"
    import kbench.core.kernels  # noqa: F401  (the reference's package, for the module names)

    # the whole pristine set (the glue's runtime module imports the backward too)
    for mod in ("_dts_layout_contract", "e_step", "dts_fused", "wave_step", "wave_backward"):
        _load(f"kbench.core.kernels.{mod}", pristine / f"{mod}.py")
    from kbench.runtime import make_static, run_forward

    cases = {"config1": ("1", None, 16), "config1_pi4": ("1", None, 4), "config1_statewise": ("1", True, 16),
             "config2": ("2", None, 16)}
    chosen = sys.argv[1:] or list(cases)
    for name in chosen:
        cfg_name, statewise, pi_iters = cases[name]
        cfg = synth.config(cfg_name)
        if statewise is not None:
            cfg = dataclasses.replace(cfg, statewise=statewise)
        problem = synth.build_problem(cfg)
        cap = _captured(problem, pi_iters)
        static = make_static(cap, "cpu")
        loss, saved = run_forward(static, cap["inputs"]["theta"], cap["inputs"]["col_weights"])
        out = {k: saved[k].detach().cpu().numpy() for k in ("E", "E_s1", "E_s2", "Ebar", "pi_wave", "pibar_wave",
                                                            "pibar_row_max")}
        if cfg_name != "1":
            C = int(out["pi_wave"].shape[0])
            roots = np.asarray(problem["static"]["wave_layout"]["root_row_ids"], dtype=np.int64)
            rest = np.setdiff1d(np.arange(C), roots)
            rows = np.sort(np.concatenate([roots, np.random.default_rng(2).choice(rest, 192, replace=False)]))
            out["rows"] = rows
            out["pi_wave"] = out["pi_wave"][rows]
            out["pibar_wave"] = out["pibar_wave"][rows]
        np.savez_compressed(HERE / f"pristine_fwd_{name}.npz", digest=np.array(synth.layout_digest(problem)),
                            theta=np.asarray(cap["inputs"]["theta"].numpy()), pi_iters=np.array(pi_iters),
                            loss=np.array(float(loss)), **out)
        print(f"{name}: pi_iters={pi_iters} loss={float(loss):.7f}", flush=True)


if __name__ == "__main__":
    main()
