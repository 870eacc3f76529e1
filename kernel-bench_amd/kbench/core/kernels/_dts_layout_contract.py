"""Parameter-layout classification of the split (DTS) wrappers.

Same public API and codes as the reference kbench/core/kernels/_dts_layout_contract.py
(enums, frozen dataclasses, ``dts_forward_param_layout``,
``dts_backward_param_layout``), since callers compare the codes.  Host-only
logic: it classifies a tensor or shape, the wrappers normalise the tensors.

Precedence (the reference's, kept deliberately):
* forward, item-indexed: a 1-d tensor of length S is a shared state vector,
  any other 1-d tensor holds one scalar per item;
* backward, item-indexed: any 1-d tensor with more than one element holds one
  scalar per item, so a bare [G] with G == S is ambiguous (flagged).
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum
from numbers import Integral
from typing import Any, Sequence


class DtsForwardAddressMode(IntEnum):
    SHARED_STATE = 0
    ITEM_INDEXED = 4


class DtsBackwardLayoutCode(IntEnum):
    SHARED_SCALAR = 0
    SHARED_STATE = 1
    ITEM_SCALAR = 2
    ITEM_STATE = 3


@dataclass(frozen=True)
class DtsForwardParamLayout:
    mode: DtsForwardAddressMode
    row_stride: int
    state_stride: int
    intent: str
    ambiguous_1d_item_state: bool = False


@dataclass(frozen=True)
class DtsBackwardParamLayout:
    code: DtsBackwardLayoutCode
    intent: str
    ambiguous_1d_item_state: bool = False


def _count(name: str, value) -> int:
    if isinstance(value, bool) or not isinstance(value, Integral):
        raise ValueError(f"{name} must be a positive integer")
    v = int(value)
    if v <= 0:
        raise ValueError(f"{name} must be positive")
    return v


def _shape(value_or_shape: Any) -> tuple[int, ...]:
    raw = getattr(value_or_shape, "shape", value_or_shape)
    if isinstance(raw, (str, bytes)):
        raise ValueError("DTS parameter shape must be a sequence of dimensions")
    try:
        dims = tuple(raw)
    except TypeError as exc:
        raise ValueError("DTS parameter shape must be a sequence of dimensions") from exc
    out = []
    for d in dims:
        if isinstance(d, bool) or not isinstance(d, Integral):
            raise ValueError("DTS parameter shape dimensions must be integers")
        if int(d) < 0:
            raise ValueError("DTS parameter shape dimensions must be non-negative")
        out.append(int(d))
    return tuple(out)


def _strides(value_or_shape: Any, shape: tuple[int, ...], strides: Sequence[int] | None) -> tuple[int, ...]:
    raw = strides
    method = getattr(value_or_shape, "stride", None)
    if raw is None and callable(method):
        raw = method()
    if raw is None:
        out, acc = [], 1
        for d in reversed(shape):
            out.append(acc)
            acc *= max(1, d)
        return tuple(reversed(out))
    try:
        vals = tuple(raw)
    except TypeError as exc:
        raise ValueError("DTS parameter strides must be a sequence of integers") from exc
    if len(vals) != len(shape):
        raise ValueError("DTS parameter strides must match shape rank")
    for v in vals:
        if isinstance(v, bool) or not isinstance(v, Integral):
            raise ValueError("DTS parameter strides must be integers")
    return tuple(int(v) for v in vals)


def _numel(shape: tuple[int, ...]) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


def dts_forward_param_layout(value_or_shape: Any, *, S: int, item_indexed: bool,
                             strides: Sequence[int] | None = None) -> DtsForwardParamLayout:
    """Forward addressing of a DTS parameter (reference _dts_layout_contract.py:59-139)."""
    n_states = _count("S", S)
    shape = _shape(value_or_shape)
    st = _strides(value_or_shape, shape, strides)
    if item_indexed:
        mode = DtsForwardAddressMode.ITEM_INDEXED
        if len(shape) == 0:
            return DtsForwardParamLayout(mode, 0, 0, "shared_scalar")
        if len(shape) == 1:
            if _numel(shape) == n_states:
                return DtsForwardParamLayout(mode, 0, st[0], "shared_state", ambiguous_1d_item_state=True)
            return DtsForwardParamLayout(mode, st[0], 0, "item_scalar")
        if len(shape) == 2:
            if shape[1] == 1:
                return DtsForwardParamLayout(mode, st[0], 0, "item_scalar")
            if shape[1] == n_states:
                return DtsForwardParamLayout(mode, 0 if shape[0] == 1 else st[0], st[1], "item_state")
        raise ValueError("item-indexed DTS parameters must be scalar, [S], [G], [G, 1], "
                         f"or [G, S]; got shape {shape} with S={n_states}")
    if len(shape) == 0:
        return DtsForwardParamLayout(DtsForwardAddressMode.SHARED_STATE, 0, 1, "shared_scalar_expanded_to_state")
    if len(shape) == 1 and _numel(shape) == n_states:
        return DtsForwardParamLayout(DtsForwardAddressMode.SHARED_STATE, 0, 1, "shared_state")
    raise ValueError(f"DTS parameters must be scalar or [S] without item indexing; got shape {shape} with "
                     f"S={n_states}")


def dts_backward_param_layout(value_or_shape: Any, *, S: int, item_indexed: bool) -> DtsBackwardParamLayout:
    """Backward layout code of a DTS parameter or gradient (reference _dts_layout_contract.py:142-188)."""
    n_states = _count("S", S)
    shape = _shape(value_or_shape)
    if _numel(shape) == 1:
        return DtsBackwardParamLayout(DtsBackwardLayoutCode.SHARED_SCALAR, "shared_scalar")
    if item_indexed and len(shape) == 1:
        return DtsBackwardParamLayout(DtsBackwardLayoutCode.ITEM_SCALAR, "item_scalar",
                                      ambiguous_1d_item_state=shape[0] == n_states)
    if len(shape) == 1 and shape[0] == n_states:
        return DtsBackwardParamLayout(DtsBackwardLayoutCode.SHARED_STATE, "shared_state")
    if item_indexed and len(shape) == 2:
        if shape[1] == 1:
            return DtsBackwardParamLayout(DtsBackwardLayoutCode.ITEM_SCALAR, "item_scalar")
        if shape[1] == n_states:
            return DtsBackwardParamLayout(DtsBackwardLayoutCode.ITEM_STATE, "item_state")
    raise ValueError(f"DTS parameters must be scalar, [S], [G], [G, 1], or [G, S]; got shape {shape} with "
                     f"S={n_states}")


__all__ = [
    "DtsBackwardLayoutCode",
    "DtsBackwardParamLayout",
    "DtsForwardAddressMode",
    "DtsForwardParamLayout",
    "dts_backward_param_layout",
    "dts_forward_param_layout",
]
