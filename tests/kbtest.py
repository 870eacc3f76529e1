"""Helpers shared by the tests: cached problems, oracle runs and inf-safe comparison."""

from __future__ import annotations

import functools

import numpy as np

from kbench import synth


@functools.lru_cache(maxsize=None)
def problem(name: str, statewise: bool | None = None) -> dict:
    import dataclasses

    cfg = synth.config(name)
    if statewise is not None:
        cfg = dataclasses.replace(cfg, statewise=statewise)
    return synth.build_problem(cfg)


@functools.lru_cache(maxsize=None)
def oracle_forward(name: str, statewise: bool | None = None):
    import kbench_oracle as O

    p = problem(name, statewise)
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    loss, saved = O.forward(prob, theta, cw)
    return prob, loss, saved


@functools.lru_cache(maxsize=None)
def oracle_backward(name: str, statewise: bool | None = None):
    import kbench_oracle as O

    p = problem(name, statewise)
    prob, loss, saved = oracle_forward(name, statewise)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    gt, gc, info, extra = O.backward(prob, theta, cw, saved, collect=True)
    info = dict(info)
    info.update(extra)
    return gt, gc, info


def compare_inf_safe(got, ref):
    """(ok_pattern, max_abs, max_rel) over positions that are not equal (incl. matching +-inf).

    Same agreement rule as the reference's golden gate (bench/_common.py:80-120):
    exact equality (so matching -inf) or both NaN agree; a disagreement
    involving a non-finite value is a pattern failure.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    agree = (got == ref) | (np.isnan(got) & np.isnan(ref))
    dis = ~agree
    if not dis.any():
        return True, 0.0, 0.0
    g, r = got[dis], ref[dis]
    if not (np.isfinite(g).all() and np.isfinite(r).all()):
        return False, float("inf"), float("inf")
    d = np.abs(g - r)
    return True, float(d.max()), float((d / np.maximum(np.abs(r), 1e-12)).max())


def norm_rel(got, ref):
    """max|got - ref| / max|ref| (normwise relative error)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = max(float(np.abs(ref).max()), 1e-300)
    return float(np.abs(got - ref).max()) / den


@functools.lru_cache(maxsize=None)
def oracle_point_cache(name: str, statewise: bool | None = None):
    """Oracle backward at the generated theta with the per-wave adjoint cache of the exact HVP."""
    import kbench_oracle as O

    p = problem(name, statewise)
    prob, loss, saved = oracle_forward(name, statewise)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    return O.build_point_cache(prob, theta, cw, saved)


def compare_inf_safe_t(got, ref, chunk_rows: int = 2048):
    """Device-side ``compare_inf_safe`` for large tensors, in row chunks (float64 differences).

    Returns (ok_pattern, max_abs, max_rel) with the same agreement rule.
    """
    import torch

    g_all = got.reshape(got.shape[0], -1) if got.ndim > 1 else got.reshape(-1, 1)
    r_all = ref.reshape(ref.shape[0], -1) if ref.ndim > 1 else ref.reshape(-1, 1)
    assert g_all.shape == r_all.shape, (tuple(got.shape), tuple(ref.shape))
    ma = mr = 0.0
    for i in range(0, g_all.shape[0], chunk_rows):
        g = g_all[i:i + chunk_rows].double()
        r = r_all[i:i + chunk_rows].double()
        dis = ~((g == r) | (torch.isnan(g) & torch.isnan(r)))
        if not bool(dis.any()):
            continue
        gd, rd = g[dis], r[dis]
        if not (bool(torch.isfinite(gd).all()) and bool(torch.isfinite(rd).all())):
            return False, float("inf"), float("inf")
        d = (gd - rd).abs()
        ma = max(ma, float(d.max()))
        mr = max(mr, float((d / rd.abs().clamp_min(1e-12)).max()))
    return True, ma, mr


def norm_rel_t(got, ref) -> float:
    """Device-side ``norm_rel``."""
    den = max(float(ref.double().abs().max()), 1e-300)
    return float((got.double() - ref.double()).abs().max()) / den
