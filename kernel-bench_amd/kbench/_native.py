"""ctypes binding of ``libkbench_hip.so`` (the C ABI in include/kbench_hip.h).

The library is built in-tree by ``kernel-bench_amd/csrc/build.py`` and lives
next to this file.  There is no fallback: if the library is missing or fails
to load, every entry point of this package raises.
"""

from __future__ import annotations

import ctypes as ct
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkbench_hip.so"
ABI_VERSION = 4

_lib = None
_load_error: str | None = None


class NativeLibraryMissing(RuntimeError):
    """The HIP library is not built or cannot be loaded."""


class KbError(RuntimeError):
    """A C-ABI call returned an error code."""


i32 = ct.c_int32
i64 = ct.c_int64
f64 = ct.c_double
vp = ct.c_void_p
P_i64 = ct.POINTER(ct.c_int64)
P_i32 = ct.POINTER(ct.c_int32)
P_f32 = ct.POINTER(ct.c_float)
P_f64 = ct.POINTER(ct.c_double)


class KbLayout(ct.Structure):
    _fields_ = [
        ("S", i32), ("C", i32), ("n_fam", i32), ("n_waves", i32),
        ("node_parent", P_i64), ("node_child1", P_i64), ("node_child2", P_i64),
        ("node_subtree_start", P_i64), ("node_subtree_end", P_i64),
        ("unnorm_row_max", P_f32),
        ("leaf_state_index", P_i64), ("rate_item_idx", P_i64), ("root_row_ids", P_i64),
        ("wave_start", P_i64), ("wave_size", P_i64), ("wave_has_splits", P_i32),
        ("n_splits", i64),
        ("split_parent", P_i64), ("split_left", P_i64), ("split_right", P_i64),
        ("split_log_prob", P_f64),
    ]


class KbForwardIO(ct.Structure):
    _fields_ = [
        ("theta", vp), ("statewise", i32), ("col_weights", vp), ("use_col_weights", i32),
        ("e_init", f64), ("e_max_iter", i32), ("e_tol", f64), ("pi_iters", i32),
        ("E", vp), ("E_s1", vp), ("E_s2", vp), ("Ebar", vp),
        ("log_pS", vp), ("log_pD", vp), ("log_pL", vp),
        ("max_coupling", vp), ("col_log_probs", vp),
        ("pi", vp), ("pibar", vp), ("pibar_row_max", vp), ("loss", vp),
    ]


class KbBackwardIO(ct.Structure):
    _fields_ = [
        ("theta", vp), ("statewise", i32), ("col_weights", vp), ("use_col_weights", i32),
        ("neumann_terms", i32), ("pruning_threshold", f64), ("use_pruning", i32),
        ("bicgstab_max_iter", i32), ("bicgstab_tol", f64), ("bicgstab_breakdown_tol", f64),
        ("E", vp), ("E_s1", vp), ("E_s2", vp), ("Ebar", vp),
        ("log_pS", vp), ("log_pD", vp), ("log_pL", vp), ("max_coupling", vp), ("col_log_probs", vp),
        ("pi", vp), ("pibar", vp), ("pibar_row_max", vp),
        ("grad_theta", vp), ("grad_col", vp),
        ("active_mask", vp), ("acc_out", vp), ("forward_token", i64),
        ("neumann_rtol", f64), ("neumann_terms_out", vp),
    ]


class KbEAdjointIO(ct.Structure):
    _fields_ = [
        ("statewise", i32), ("use_col_weights", i32), ("with_norm", i32), ("bicgstab_max_iter", i32),
        ("bicgstab_tol", f64), ("bicgstab_breakdown_tol", f64),
        ("E", vp), ("log_pS", vp), ("log_pD", vp), ("log_pL", vp), ("max_coupling", vp), ("col_log_probs", vp),
        ("acc", vp), ("q_extra", vp), ("w_out", vp), ("g_out", vp), ("work", vp), ("status", vp),
    ]


E_ADJOINT_WORK_VECTORS = 16


def _declare(lib):
    lib.kb_last_error.restype = ct.c_char_p
    lib.kb_abi_version.restype = ct.c_int
    lib.kb_plan_create.argtypes = [ct.POINTER(KbLayout), ct.POINTER(vp)]
    lib.kb_plan_create.restype = ct.c_int
    lib.kb_plan_destroy.argtypes = [vp]
    lib.kb_plan_destroy.restype = None
    lib.kb_plan_info.argtypes = [vp, P_i32, ct.c_int]
    lib.kb_plan_info.restype = ct.c_int
    lib.kb_forward.argtypes = [vp, ct.POINTER(KbForwardIO), vp]
    lib.kb_forward.restype = ct.c_int
    lib.kb_forward_stats.argtypes = [vp, P_i32, P_f64, vp]
    lib.kb_forward_stats.restype = ct.c_int
    if hasattr(lib, "kb_backward"):
        lib.kb_backward.argtypes = [vp, ct.POINTER(KbBackwardIO), vp]
        lib.kb_backward.restype = ct.c_int
    lib.kb_solve.argtypes = [vp, ct.POINTER(KbForwardIO), ct.POINTER(KbBackwardIO), vp]
    lib.kb_solve.restype = ct.c_int
    lib.kb_profile_enable.argtypes = [vp, ct.c_int]
    lib.kb_profile_enable.restype = ct.c_int
    lib.kb_profile_read.argtypes = [vp, ct.c_int, P_f32, ct.c_int]
    lib.kb_profile_read.restype = ct.c_int
    lib.kb_forward_token.argtypes = [vp]
    lib.kb_forward_token.restype = ct.c_int64
    if hasattr(lib, "kb_e_adjoint"):
        lib.kb_e_adjoint.argtypes = [vp, ct.POINTER(KbEAdjointIO), vp]
        lib.kb_e_adjoint.restype = ct.c_int
    if hasattr(lib, "kb_backward_stats"):
        lib.kb_backward_stats.argtypes = [vp, P_i32, vp]
        lib.kb_backward_stats.restype = ct.c_int
    from . import _native_ops  # declares the per-wrapper entry points
    _native_ops.declare(lib)


# Native handles (plans, trees) whose destruction waits for the end of a HIP
# graph capture.  Destroying one frees device memory, and a free while a
# capture is underway invalidates that capture; the garbage collector can drop
# the last reference to a handle at any point, captures included.
_held_back: list = []


def _capture_underway() -> bool:
    import torch

    try:
        return bool(torch.cuda.is_initialized() and torch.cuda.is_current_stream_capturing())
    except Exception:  # pragma: no cover - interpreter shutdown order
        return False


def release(destroy: str, handle) -> None:
    """Call the library's ``destroy`` entry point on ``handle`` now, or once no capture is underway."""
    _held_back.append((destroy, handle))
    if not _capture_underway():
        release_held_back()


def release_held_back() -> None:
    """Destroy every handle held back by ``release`` (call outside graph captures)."""
    while _held_back and _lib is not None:  # a handle exists only once the library is loaded
        name, h = _held_back.pop()
        getattr(_lib, name)(h)


def lib():
    """Load (once) and return the HIP library; raise if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        if _held_back and not _capture_underway():
            release_held_back()
        return _lib
    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built; run `python kernel-bench_amd/csrc/build.py` "
            "(or __graft_entry__.build()) first"
        )
    try:
        handle = ct.CDLL(str(LIB_PATH), mode=os.RTLD_LOCAL if hasattr(os, "RTLD_LOCAL") else 0)
    except OSError as exc:  # pragma: no cover - depends on the host
        _load_error = str(exc)
        raise NativeLibraryMissing(f"cannot load {LIB_PATH}: {exc}") from exc
    if handle.kb_abi_version() != ABI_VERSION:
        raise NativeLibraryMissing(f"{LIB_PATH} ABI {handle.kb_abi_version()} != {ABI_VERSION}; rebuild")
    _declare(handle)
    _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().kb_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg)
        raise KbError(f"libkbench_hip error {rc}: {msg}")


def ptr(t) -> int:
    """Device (or host) address of a tensor, or 0 for None."""
    return 0 if t is None else int(t.data_ptr())


def stream_handle(device=None) -> int:
    """The raw ``hipStream_t`` of torch's current stream on ``device`` (default: the current device).

    Read through torch's raw-stream accessor (one C call, no Stream object):
    the per-call wrappers ask for it on every launch.
    """
    import torch

    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, torch.device):
        idx = device.index if device.index is not None else torch.cuda.current_device()
    else:
        idx = int(device)
    return int(torch._C._cuda_getCurrentRawStream(idx))
