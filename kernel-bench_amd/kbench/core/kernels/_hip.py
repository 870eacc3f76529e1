"""Plumbing shared by the HIP-backed wrappers of ``kbench.core.kernels``.

* dtype codes and argument checks (the reference raises RuntimeError for an
  unsupported dtype or device and ValueError for layouts);
* species-tree handles (``kb_tree``), built once per set of topology tensors
  and cached with a strong reference to those tensors, so a cached handle can
  never be matched by a different tensor reusing the same memory;
* fixed-order row accumulation (``kb_rows_scatter_add``, ``kb_rows_sum_into``),
  which replaces the reference's atomic adds;
* version counters: a kernel that writes a caller's tensor through a raw
  pointer is invisible to torch, so every wrapper bumps the version of each
  tensor it writes in place (``wrote``), as torch's own in-place ops do.  A
  cache keyed on a tensor's version (the whole-pass driver's reuse of a
  forward's split terms, ``static_cached``) then sees the change.

There is no CPU path: every launcher raises if the HIP library is missing.
"""

from __future__ import annotations

import ctypes as ct
from collections import OrderedDict

import torch

from ... import _native as N
from ..._native_ops import (KB_BF16, KB_F32, KB_F64, KbDtsCrossIO, KbDtsIO, KbDtsSoIO, KbDtsTanIO, KbEStepIO,
                            KbEStepSoIO, KbEStepVjpIO, KbETanIO, KbLeafInitIO, KbPibarVjpIO, KbWaveBwdIO, KbWaveSoIO,
                            KbWaveStepIO, KbWaveTanIO)

__all__ = [
    "KB_BF16", "KB_F32", "KB_F64", "KbDtsCrossIO", "KbDtsIO", "KbEStepIO", "KbEStepVjpIO", "KbLeafInitIO",
    "KbPibarVjpIO", "KbWaveBwdIO", "KbWaveStepIO", "KbETanIO", "KbDtsTanIO", "KbWaveTanIO", "KbEStepSoIO",
    "KbWaveSoIO", "KbDtsSoIO",
    "lib", "check", "ptr", "stream", "dtype_code", "defer", "flush", "require_device", "f", "i64", "tree_from_parent",
    "tree_from_levels", "scatter_add_rows", "sum_rows_into", "rows_sum_accum", "static_cached", "wrote",
]

check = N.check
ptr = N.ptr

# a callable that launches work held back by a wrapper (the chained sweeps of
# compute_wave_step under KBENCH_FUSE_SWEEPS), or None
_deferred = None


def defer(run) -> None:
    """Register held-back work; it runs before the next launch of any wrapper."""
    global _deferred
    _deferred = run


def flush() -> None:
    """Launch any held-back work now (the wrappers do this before their own launches)."""
    global _deferred
    run, _deferred = _deferred, None
    if run is not None:
        run()


def lib():
    """The HIP library, after launching any held-back work (stream order is kept)."""
    if _deferred is not None:
        flush()
    return N.lib()


def stream(device) -> int:
    return N.stream_handle(device)


def dtype_code(dtype) -> int:
    if dtype == torch.float32:
        return KB_F32
    if dtype == torch.float64:
        return KB_F64
    raise RuntimeError(f"the HIP kernels support float32 and float64 tensors only, got {dtype}")


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} requires a HIP device tensor, got {t.device}")


def f(t, dtype, device):
    """t as a contiguous ``dtype`` tensor on ``device`` (None stays None).

    Tensors that already qualify are returned as they are without a dispatch
    (the per-sweep wrappers call this for every constant on every launch).
    """
    if t is None:
        return None
    if not torch.is_tensor(t):
        t = torch.as_tensor(t)
    elif t.dtype is dtype and t.device == device and t.is_contiguous():
        return t
    return t.to(device=device, dtype=dtype).contiguous()


def wrote(*ts) -> None:
    """Bump the version counter of every tensor a kernel has written in place (None skipped).

    Inference-mode tensors carry no version counter and are skipped.
    """
    for t in ts:
        if t is not None and not t.is_inference():
            torch.autograd.graph.increment_version(t)


def i64(t, device):
    if t is None:
        return None
    if t.dtype is torch.long and t.device == device and t.is_contiguous():
        return t
    return t.to(device=device, dtype=torch.long).contiguous()


# ---------------------------------------------------------------- tree handles
_TREES: "OrderedDict[tuple, tuple]" = OrderedDict()
_TREE_CACHE_SIZE = 32


class _Tree:
    def __init__(self, handle: ct.c_void_p, S: int):
        self.handle = handle
        self.S = S

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            if self.handle:
                N.release("kb_tree_destroy", self.handle)  # held back while a graph capture is underway
        except Exception:
            pass


def _key(*ts):
    # addresses are unique across devices in one process (unified addressing)
    return tuple((t.data_ptr(), t.shape, t._version) for t in ts)


def _create(S: int, parent, c1, c2) -> _Tree:
    par = torch.as_tensor(parent, dtype=torch.long).contiguous()
    a = torch.as_tensor(c1, dtype=torch.long).contiguous()
    b = torch.as_tensor(c2, dtype=torch.long).contiguous()
    h = ct.c_void_p()
    P = ct.POINTER(ct.c_int64)
    check(lib().kb_tree_create(int(S), ct.cast(par.data_ptr(), P), ct.cast(a.data_ptr(), P),
                               ct.cast(b.data_ptr(), P), ct.byref(h)))
    return _Tree(h, int(S))


def _cached(key, keep, build):
    hit = _TREES.get(key)
    if hit is not None:
        _TREES.move_to_end(key)
        return hit[0]
    tree = build()
    _TREES[key] = (tree, keep)
    while len(_TREES) > _TREE_CACHE_SIZE:
        _TREES.popitem(last=False)
    return tree


def tree_from_parent(node_parent, node_child1, node_child2) -> _Tree:
    """Tree handle from state_helpers node_parent / node_child1 / node_child2."""
    S = int(node_parent.numel())
    key = ("parent", S) + _key(node_parent, node_child1, node_child2)
    return _cached(key, (node_parent, node_child1, node_child2),
                   lambda: _create(S, node_parent.detach().cpu(), node_child1.detach().cpu(),
                                   node_child2.detach().cpu()))


def tree_from_levels(S, level_ptr, level_parents, level_child1, level_child2) -> _Tree:
    """Tree handle from the compact_level_* tables (parent with its two children per entry)."""
    S = int(S)
    key = ("levels", S) + _key(level_ptr, level_parents, level_child1, level_child2)

    def build():
        p = level_parents.detach().cpu().long()
        a = level_child1.detach().cpu().long()
        b = level_child2.detach().cpu().long()
        parent = torch.full((S,), -1, dtype=torch.long)
        c1 = torch.full((S,), S, dtype=torch.long)
        c2 = torch.full((S,), S, dtype=torch.long)
        ok_a = (a >= 0) & (a < S) & (p >= 0) & (p < S)
        ok_b = (b >= 0) & (b < S) & (p >= 0) & (p < S)
        parent[a[ok_a]] = p[ok_a]
        parent[b[ok_b]] = p[ok_b]
        c1[p[ok_a]] = a[ok_a]
        c2[p[ok_b]] = b[ok_b]
        return _create(S, parent, c1, c2)

    return _cached(key, (level_ptr, level_parents, level_child1, level_child2), build)


# ------------------------------------------------------ static-layout cache
_STATIC: "OrderedDict[tuple, tuple]" = OrderedDict()
_STATIC_CACHE_SIZE = 8192


def static_cached(tag, tensors, build):
    """``build()`` memoised on the identity of layout tensors that do not change between calls
    (wave metadata, topology) and on any plain values among ``tensors``.  The entry keeps strong
    references to the tensors, so their memory cannot be reused by another tensor while the entry
    lives; an in-place change bumps their version and misses."""
    key = (tag,) + tuple(_key(t)[0] if torch.is_tensor(t) else t for t in tensors)
    hit = _STATIC.get(key)
    if hit is not None:
        _STATIC.move_to_end(key)
        return hit[0]
    val = build()
    _STATIC[key] = (val, tuple(t for t in tensors if torch.is_tensor(t)))
    while len(_STATIC) > _STATIC_CACHE_SIZE:
        _STATIC.popitem(last=False)
    return val


# ------------------------------------------------------ fixed-order accumulation
def _sorted_keys(keys, device):
    keys_sorted, order = torch.sort(keys.to(device=device, dtype=torch.long).reshape(-1), stable=True)
    return keys_sorted, order.to(torch.int32)


def scatter_add_rows(dst: torch.Tensor, src: torch.Tensor, keys, *, row_stride=None, static=None) -> None:
    """dst[keys[r]] += src[r] for every row r, summed per key in increasing r.

    ``dst`` rows are ``row_stride`` elements apart (default: dst.shape[-1]);
    row_stride 0 adds every row into the single row ``dst`` (all keys must be 0).
    Negative keys are skipped.  With ``static`` (a tuple of layout tensors that determine
    ``keys``), ``keys`` may be a callable and its sort is cached on their identity.
    """
    n = int(src.shape[0])
    if n == 0:
        return
    S = int(src.shape[1])
    if static is not None:
        keys_sorted, order32 = static_cached(("scatter_keys", str(src.device)), static,
                                             lambda: _sorted_keys(keys() if callable(keys) else keys, src.device))
    else:
        keys_sorted, order32 = _sorted_keys(keys, src.device)
    stride = int(dst.shape[-1]) if row_stride is None else int(row_stride)
    check(lib().kb_rows_scatter_add(dtype_code(src.dtype), S, n, ptr(src), ptr(order32), ptr(keys_sorted),
                                    ptr(dst), stride, stream(src.device)))
    wrote(dst)


def rows_sum_multi(blocks) -> torch.Tensor:
    """[m, S] column sums of up to 8 [n, S] row blocks, in row order with float64 partial sums.

    Each entry of ``blocks`` is a tensor or a pair of tensors (summed elementwise in the
    reduction); all share n, S, dtype and device.
    """
    import ctypes as ct

    pairs = [b if isinstance(b, (tuple, list)) else (b, None) for b in blocks]
    first = pairs[0][0]
    n, S = int(first.shape[0]), int(first.shape[1])
    m = len(pairs)
    if not 1 <= m <= 8:
        raise ValueError(f"rows_sum_multi takes 1..8 blocks, got {m}")
    for x, y in pairs:
        for t in (x,) if y is None else (x, y):
            _check_rows(t, n, S, first, "rows_sum_multi")
    out = torch.empty((m, S), device=first.device, dtype=first.dtype)
    chunks = (n + 63) // 64
    work = torch.empty((m * chunks * S if chunks > 1 else 1,), device=first.device, dtype=torch.float64)
    a = (ct.c_void_p * m)(*[ptr(x) for x, _ in pairs])
    b = (ct.c_void_p * m)(*[ptr(y) if y is not None else None for _, y in pairs])
    check(lib().kb_rows_sum_multi(dtype_code(first.dtype), S, n, m, a, b, ptr(out), ptr(work), stream(first.device)))
    return out


def rows_sum_accum(blocks) -> None:
    """dst += column sums of row blocks, all in one launch (two above 64 rows).

    ``blocks``: up to 8 pairs (dst, addends): dst a contiguous [S] tensor (distinct
    per block), addends a [n, S] tensor or a tuple of up to 4 of them whose sum is
    the block's rows; rows summed in order in float64, as ``sum_rows_into`` does.
    """
    import ctypes as ct

    blocks = [(d, a if isinstance(a, (tuple, list)) else (a,)) for d, a in blocks]
    m = len(blocks)
    if m == 0:
        return
    if m > 8:
        raise ValueError(f"rows_sum_accum takes at most 8 blocks, got {m}")
    first = blocks[0][1][0]
    S = int(first.shape[1])
    n = [int(a[0].shape[0]) for _, a in blocks]
    for (d, a), nb in zip(blocks, n):
        if not 1 <= len(a) <= 4:
            raise ValueError(f"rows_sum_accum takes 1..4 addends per block, got {len(a)}")
        for t in a:
            _check_rows(t, nb, S, first, "rows_sum_accum")
        if (not torch.is_tensor(d) or d.dtype != first.dtype or d.device != first.device or not d.is_contiguous()
                or d.numel() != S):
            raise ValueError("rows_sum_accum: every accumulator must be a contiguous tensor of S elements with the "
                             "addends' dtype and device")
    chunks = max((x + 63) // 64 for x in n)
    work = torch.empty((m * chunks * S if chunks > 1 else 1,), device=first.device, dtype=torch.float64)
    addends = []
    for _, a in blocks:
        addends += [ptr(x) for x in a] + [None] * (4 - len(a))
    check(lib().kb_rows_sum_accum(
        dtype_code(first.dtype), S, m, (ct.c_int64 * m)(*n), (ct.c_int32 * m)(*[len(a) for _, a in blocks]),
        (ct.c_void_p * (4 * m))(*addends), (ct.c_void_p * m)(*[ptr(d) for d, _ in blocks]), ptr(work),
        stream(first.device)))
    wrote(*[d for d, _ in blocks])


def _check_rows(t, n, S, first, what):
    """``t`` is a contiguous [n, S] tensor with ``first``'s dtype and device (the C entry points take raw
    pointers and cannot check what they read)."""
    if (not torch.is_tensor(t) or t.ndim != 2 or int(t.shape[0]) != n or int(t.shape[1]) != S
            or t.dtype != first.dtype or t.device != first.device or not t.is_contiguous()):
        raise ValueError(f"{what}: every addend must be a contiguous [{n}, {S}] tensor of dtype {first.dtype} "
                         f"on {first.device}")


def sum_rows_into(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst += src.sum(0), in row order with float64 partial sums."""
    n = int(src.shape[0])
    if n == 0:
        return
    S = int(src.shape[1])
    work = torch.empty(((n + 63) // 64) * S, device=src.device, dtype=torch.float64)
    check(lib().kb_rows_sum_into(dtype_code(src.dtype), S, n, ptr(src), ptr(dst), ptr(work), stream(src.device)))
    wrote(dst)
