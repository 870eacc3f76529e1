"""The C-ABI library loads and exports every entry point declared in include/*.h.

No compute call here (there is no GPU in the CPU suite); host-only entry
points (ABI version, LDS limits, error text) are called.  The product path has
no CPU fallback: wrappers refuse host tensors and a missing library raises.
"""

import re
from pathlib import Path

import pytest
import torch

from kbench import _native as N

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(kb_[a-z_0-9]+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = _declared()
    for must in ("kb_plan_create", "kb_forward", "kb_backward", "kb_tree_create", "kb_wave_step",
                 "kb_dts_forward", "kb_wave_backward", "kb_dts_cross_backward", "kb_pibar_vjp", "kb_estep",
                 "kb_estep_vjp", "kb_active_mask", "kb_leaf_init", "kb_rows_scatter_add", "kb_rows_sum_into",
                 "kb_rows_sum_multi"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_host_only_entry_points():
    lib = N.lib()
    assert lib.kb_abi_version() == N.ABI_VERSION
    assert lib.kb_ops_max_states(0) == 8192
    assert 4096 <= lib.kb_ops_max_states(1) < 8192
    assert isinstance(lib.kb_last_error(), bytes)
    # argument checks that precede any device call
    assert lib.kb_rows_sum_multi(0, 4, 2, 9, None, None, None, None, None) != 0
    assert b"at most 8" in lib.kb_last_error()
    import ctypes as ct

    n, k = (ct.c_int64 * 2)(3, 3), (ct.c_int32 * 2)(1, 5)
    a, d = (ct.c_void_p * 8)(*([16] * 8)), (ct.c_void_p * 2)(32, 64)
    assert lib.kb_rows_sum_accum(0, 4, 9, n, k, a, d, None, None) != 0
    assert b"at most 8" in lib.kb_last_error()
    assert lib.kb_rows_sum_accum(0, 4, 2, n, k, a, d, None, None) != 0
    assert b"addends" in lib.kb_last_error()
    k[1] = 1
    d[1] = 32
    assert lib.kb_rows_sum_accum(0, 4, 2, n, k, a, d, None, None) != 0
    assert b"share an accumulator" in lib.kb_last_error()


def test_wrappers_refuse_host_tensors():
    from kbench.core.kernels.wave_backward import active_mask_from_rhs_absmax_fused
    from kbench.core.kernels.e_step import e_fixed_point_triton

    with pytest.raises(ValueError):
        active_mask_from_rhs_absmax_fused(torch.zeros(2, 3), 1e-6)
    E = torch.zeros(1, 3)
    with pytest.raises(RuntimeError):
        e_fixed_point_triton(E, E, E, E, E, torch.zeros(3), torch.tensor([2, 2, -1]), torch.tensor([3, 3, 0]),
                             torch.tensor([3, 3, 1]), 2)


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setattr(N, "LIB_PATH", tmp_path / "libkbench_hip.so")
    with pytest.raises(N.NativeLibraryMissing):
        N.lib()
