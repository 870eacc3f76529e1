"""Base-2 log-space helpers of the glue (reference kbench/core/inference/logspace.py:1-16)."""

from __future__ import annotations

import torch

_NEG_INF = float("-inf")


def safe_log2(x: torch.Tensor) -> torch.Tensor:
    """log2(x) for x > 0, -inf elsewhere (no NaN for x <= 0)."""
    pos = x > 0
    return torch.where(pos, torch.log2(torch.where(pos, x, torch.ones_like(x))), torch.full_like(x, _NEG_INF))


def logsumexp2(x: torch.Tensor, dim: int, keepdim: bool = False) -> torch.Tensor:
    """log2 sum 2^x along ``dim``; all -inf gives -inf."""
    m = x.max(dim=dim, keepdim=True).values
    ms = torch.where(m == _NEG_INF, torch.zeros_like(m), m)
    out = safe_log2(torch.exp2(x - ms).sum(dim=dim, keepdim=True)) + m
    return out if keepdim else out.squeeze(dim)
