"""Scratch-memory gate of the per-wave backward (reference kbench/core/memory_policy.py:1-81).

``proposal0_memory_gate(W, S, dtype)`` answers whether a wave's [W, S]
scratch (ten tensors, as the reference counts) fits the device budget:
min(total * fraction, free - reserve), with the fraction and reserve taken
from GPUREC_MEMORY_POLICY_FRACTION / GPUREC_MEMORY_POLICY_RESERVE_GIB
(defaults 0.85 and 1 GiB).  Same names, arguments and errors as the
reference.
"""

from __future__ import annotations

import os
from numbers import Integral, Real

import torch

GIB = 1024 ** 3


def _as_int(name: str, value) -> int:
    if isinstance(value, bool):
        raise ValueError(f"{name} must be an integer")
    if isinstance(value, Integral):
        return int(value)
    if isinstance(value, Real) and float(value).is_integer():
        return int(value)
    raise ValueError(f"{name} must be an integer")


def _nonnegative_int(name: str, value) -> int:
    v = _as_int(name, value)
    if v < 0:
        raise ValueError(f"{name} must be non-negative")
    return v


def _positive_int(name: str, value) -> int:
    v = _as_int(name, value)
    if v <= 0:
        raise ValueError(f"{name} must be positive")
    return v


def dtype_nbytes(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def cuda_memory_budget_bytes(device=None, *, default_fraction: float = 0.85, default_reserve_gib: float = 1.0):
    """Usable device bytes, or None without a device."""
    if not torch.cuda.is_available():
        return None
    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, torch.device):
        idx = device.index if device.index is not None else torch.cuda.current_device()
    else:
        idx = int(device)
    free_b, total_b = torch.cuda.mem_get_info(idx)
    frac = float(os.environ.get("GPUREC_MEMORY_POLICY_FRACTION", str(default_fraction)))
    reserve = int(float(os.environ.get("GPUREC_MEMORY_POLICY_RESERVE_GIB", str(default_reserve_gib))) * GIB)
    return max(0, min(int(total_b * frac), max(0, int(free_b) - reserve)))


def proposal0_wave_scratch_bytes(W, S, dtype, *, scratch_tensors: int = 10) -> int:
    return (_nonnegative_int("W", W) * _positive_int("S", S) * _nonnegative_int("scratch_tensors", scratch_tensors)
            * dtype_nbytes(dtype))


def proposal0_memory_gate(W, S, dtype, *, device=None, already_live_bytes: int = 0):
    """(fits, required bytes, budget bytes or None)."""
    required = _nonnegative_int("already_live_bytes", already_live_bytes) + proposal0_wave_scratch_bytes(W, S, dtype)
    budget = cuda_memory_budget_bytes(device)
    if budget is None:
        return True, required, budget
    return required <= budget, required, budget
