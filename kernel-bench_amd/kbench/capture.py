"""Capture and replay of per-call wrapper calls: a per-kernel parity gate.

Semantics follow the reference's harness (reference kbench/_capture_io.py:25-103,
capture/capture.py:81-210, bench/kernels.py:54-94, bench/_common.py:80-120):

* a capture records, for up to ``per_wrapper`` calls of each wrapper with
  distinct integer arguments (ws, W, S, ...), the state before the call
  (arguments) and after it (arguments, which the wrappers mutate in place,
  and the return value);
* arguments that share memory in the original call share it again on replay
  (``Pi_out is Pibar``, a wave's rows viewed out of a [C, S] buffer);
* outputs the wrapper never writes are "don't care": each recorded call is
  run twice with every ``torch.empty`` / ``torch.empty_like`` float tensor
  pre-filled with a different poison value, and positions that keep the
  poison are masked out of the comparison; among written positions the
  run-to-run difference is the wrapper's own noise floor (zero for the HIP
  wrappers, which sum in a fixed order);
* replay rebuilds the inputs on the device, calls the wrapper and compares
  every output with the recorded one, -inf/NaN-safe, passing when
  max_abs <= max(atol, margin * noise_abs) or max_rel <= max(rtol, margin * noise_rel).

Design: a snapshot stores whole *storages* as raw bytes, each byte image
once (a storage whose bytes equal its previous snapshot reuses it; the HIP
wrappers write through raw pointers, so torch's version counters cannot tell);
a tensor argument is (storage group, storage snapshot, dtype, offset, shape,
stride).  Replay allocates one device storage
per group and rebuilds every tensor as a view of it, so views and aliases
come back exactly.  Records are plain dicts, lists, numbers, strings and
tensors: ``save`` / ``load`` round-trip through ``torch.save`` and
``torch.load(weights_only=True)``.
"""

from __future__ import annotations

import importlib
from contextlib import contextmanager

import torch
from torch.overrides import TorchFunctionMode

# the per-call wrappers of kbench.core.kernels a capture interposes on
WRAPPERS = {
    "compute_leaf_initial_wave_step": "kbench.core.kernels.wave_step",
    "compute_wave_step": "kbench.core.kernels.wave_step",
    "compute_dts_forward": "kbench.core.kernels.dts_fused",
    "e_fixed_point_triton": "kbench.core.kernels.e_step",
    "active_mask_from_rhs_absmax_fused": "kbench.core.kernels.wave_backward",
    "wave_backward_uniform_fused": "kbench.core.kernels.wave_backward",
    "dts_cross_backward_accum_fused": "kbench.core.kernels.wave_backward",
    "uniform_cross_pibar_vjp_tree_from_ud_fused": "kbench.core.kernels.wave_backward",
}

POISON = (3.0e30, -3.0e30)   # the two fills of the unwritten-output detection
POISON_GAP = 1.0e15          # a run-to-run difference above this is an unwritten position
NOISE_MARGIN = 4.0


def _dtype_name(dt: torch.dtype) -> str:
    return str(dt).replace("torch.", "")


def _dtype(name: str) -> torch.dtype:
    return getattr(torch, name)


class _Snapshot:
    """Storage snapshots of one capture, as CPU bytes; unchanged bytes reuse the previous snapshot."""

    def __init__(self, pool: list):
        self.pool = pool
        self.last = {}  # (address, bytes) of a storage -> index of its latest snapshot

    def storage(self, t: torch.Tensor) -> int:
        st = t.untyped_storage()
        key = (st.data_ptr(), st.nbytes())
        raw = torch.empty(0, dtype=torch.uint8, device=t.device).set_(st).detach().cpu().clone()
        idx = self.last.get(key)
        if idx is None or not torch.equal(self.pool[idx], raw):
            self.pool.append(raw)
            idx = self.last[key] = len(self.pool) - 1
        return idx

    def struct(self, obj, groups: dict):
        """``obj`` with every tensor replaced by its description (groups: storage -> group id, per call)."""
        if torch.is_tensor(obj):
            ptr = obj.untyped_storage().data_ptr()
            g = groups.setdefault(ptr, len(groups))
            return {"tensor": [g, self.storage(obj), _dtype_name(obj.dtype), int(obj.storage_offset()),
                               list(obj.shape), list(obj.stride())]}
        if isinstance(obj, dict):
            return {"dict": {k: self.struct(v, groups) for k, v in obj.items()}}
        if isinstance(obj, (list, tuple)):
            return {"list" if isinstance(obj, list) else "tuple": [self.struct(v, groups) for v in obj]}
        return {"value": obj}


def rebuild(desc, pool, device):
    """Tensors of a described structure on ``device``: one fresh storage per group, views as recorded."""
    stores = {}

    def conv(d):
        if "tensor" in d:
            g, idx, dt, off, shape, stride = d["tensor"]
            if g not in stores:
                stores[g] = pool[idx].to(device, copy=True).untyped_storage()  # never the pool's own bytes
            return torch.empty(0, dtype=_dtype(dt), device=device).set_(stores[g], off, shape, stride)
        if "dict" in d:
            return {k: conv(v) for k, v in d["dict"].items()}
        if "list" in d:
            return [conv(v) for v in d["list"]]
        if "tuple" in d:
            return tuple(conv(v) for v in d["tuple"])
        return d["value"]

    return conv(desc)


def named_tensors(obj, prefix="", out=None):
    """[(path, tensor)] of every tensor leaf, in a fixed order."""
    out = [] if out is None else out
    if torch.is_tensor(obj):
        out.append((prefix, obj))
    elif isinstance(obj, dict):
        for k, v in obj.items():
            named_tensors(v, f"{prefix}.{k}", out)
    elif isinstance(obj, (list, tuple)):
        for i, v in enumerate(obj):
            named_tensors(v, f"{prefix}[{i}]", out)
    return out


def _int_key(args, kwargs):
    return [v for v in list(args) + list(kwargs.values()) if isinstance(v, int) and not isinstance(v, bool)]


class Capture:
    """Context manager that records wrapper calls (see the module docstring).

    ``wrappers`` maps wrapper name -> module path (default ``WRAPPERS``); the
    module attribute is replaced while the context is open, so callers that
    resolve the wrapper from its module at call time are recorded.
    """

    def __init__(self, per_wrapper: int = 4, wrappers: dict | None = None):
        self.per_wrapper = int(per_wrapper)
        self.wrappers = dict(WRAPPERS if wrappers is None else wrappers)
        self.records: list[dict] = []
        self.pool: list[torch.Tensor] = []
        self._restore = []

    def _shim(self, name, module):
        original = getattr(module, name)
        seen = []
        snap = _Snapshot(self.pool)

        def recorded(*args, **kwargs):
            key = _int_key(args, kwargs)
            take = len(seen) < self.per_wrapper and key not in seen
            if not take:
                return original(*args, **kwargs)
            _settle()
            groups = {}
            pre = snap.struct([list(args), dict(kwargs)], groups)
            ret = original(*args, **kwargs)
            _settle()
            post = snap.struct([list(args), dict(kwargs), ret], dict(groups))
            seen.append(key)
            self.records.append({"wrapper": name, "module": module.__name__, "key": key, "pre": pre, "post": post})
            return ret

        setattr(module, name, recorded)
        self._restore.append((module, name, original))

    def __enter__(self):
        for name, mod in self.wrappers.items():
            self._shim(name, importlib.import_module(mod))
        return self

    def __exit__(self, *exc):
        for module, name, original in reversed(self._restore):
            setattr(module, name, original)
        self._restore.clear()
        return False

    def save(self, path) -> None:
        torch.save({"records": self.records, "pool": self.pool}, path)

    @staticmethod
    def load(path) -> tuple[list, list]:
        d = torch.load(path, map_location="cpu", weights_only=True)
        return d["records"], d["pool"]


class _PoisonEmpty(TorchFunctionMode):
    """Fill every floating-point ``torch.empty`` / ``empty_like`` result with ``value``."""

    def __init__(self, value: float):
        super().__init__()
        self.value = value

    def __torch_function__(self, func, types, args=(), kwargs=None):
        out = func(*args, **(kwargs or {}))
        if func in (torch.empty, torch.empty_like) and torch.is_tensor(out) and out.is_floating_point():
            out.fill_(self.value)
        return out


def _settle():
    """Run work a wrapper held back (KBENCH_FUSE_SWEEPS chains) and wait for the device."""
    from kbench.core.kernels import _hip

    _hip.flush()
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def _wrapper_fn(rec):
    return getattr(importlib.import_module(rec["module"]), rec["wrapper"])


def _run(rec, pool, device, fn=None, poison=None):
    args, kwargs = rebuild(rec["pre"], pool, device)
    fn = fn or _wrapper_fn(rec)
    if poison is None:
        ret = fn(*args, **kwargs)
        _settle()
    else:
        with _PoisonEmpty(poison):
            ret = fn(*args, **kwargs)
            _settle()
    return named_tensors([args, kwargs, ret])


def measure_noise(records, pool, device="cuda") -> None:
    """Add ``valid`` (paths -> bool masks of written positions, only where some are unwritten) and
    ``noise`` (paths -> [max_abs, max_rel] run-to-run difference at written positions) to every record."""
    for rec in records:
        a, b = (dict(_run(rec, pool, device, poison=p)) for p in POISON)
        valid, noise = {}, {}
        for path, x in a.items():
            y = b.get(path)
            if y is None or x.shape != y.shape or not x.is_floating_point():
                continue
            x64, y64 = x.detach().double().cpu(), y.detach().double().cpu()
            diff = (x64 - y64).abs()
            unwritten = (~torch.isfinite(diff) & ~(torch.isnan(x64) & torch.isnan(y64))) | (diff > POISON_GAP)
            unwritten &= ~(x64 == y64)
            if bool(unwritten.any()):
                valid[path] = ~unwritten
            off = ~(x64 == y64) & ~(torch.isnan(x64) & torch.isnan(y64)) & ~unwritten
            if bool(off.any()):
                d = diff[off]
                noise[path] = [float(d.max()), float((d / y64[off].abs().clamp_min(1e-12)).max())]
        rec["valid"], rec["noise"] = valid, noise


def compare(got, ref, *, rtol, atol, noise_abs=0.0, noise_rel=0.0, margin=NOISE_MARGIN) -> dict:
    """-inf / NaN-safe comparison with a noise-widened tolerance (reference bench/_common.py:80-120)."""
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    if g.shape != r.shape:
        return {"ok": False, "max_abs": float("inf"), "max_rel": float("inf"), "reason": "shape"}
    off = ~((g == r) | (torch.isnan(g) & torch.isnan(r)))
    if not bool(off.any()):
        return {"ok": True, "max_abs": 0.0, "max_rel": 0.0, "reason": ""}
    d = (g[off] - r[off]).abs()
    if not bool(torch.isfinite(d).all()):
        return {"ok": False, "max_abs": float("inf"), "max_rel": float("inf"), "reason": "non-finite mismatch"}
    ma = float(d.max())
    mr = float((d / r[off].abs().clamp_min(1e-12)).max())
    ok = ma <= max(atol, margin * noise_abs) or mr <= max(rtol, margin * noise_rel)
    return {"ok": ok, "max_abs": ma, "max_rel": mr, "reason": "" if ok else "tolerance"}


def replay(rec, pool, *, device="cuda", fn=None, rtol=2e-3, atol=2e-3, scale_atol=False,
           dont_care=None) -> list[dict]:
    """Re-run one recorded call and compare every output with the recorded post-call state.

    ``fn`` replaces the recorded wrapper (another implementation with the same signature: the gate
    then compares it with the recorded outputs).  ``scale_atol`` measures ``atol`` against each
    output's largest finite magnitude (at least 1).  ``dont_care`` maps an output path to a boolean
    mask of positions to leave out (the caller's don't-care regions, beside the unwritten ones that
    ``measure_noise`` finds).
    """
    got = _run(rec, pool, device, fn=fn)
    want = dict(named_tensors(rebuild(rec["post"], pool, "cpu")))
    out = []
    valid, noise = rec.get("valid", {}), rec.get("noise", {})
    dont_care = dont_care or {}
    for path, t in got:
        if path not in want or not torch.is_tensor(want[path]):
            continue
        g, r = t.detach().cpu(), want[path]
        m = valid.get(path)
        if path in dont_care:
            keep = ~dont_care[path].to(torch.bool).cpu()
            m = keep if m is None else (m & keep)
        if m is not None:
            g, r = g[m], r[m]
        if not g.is_floating_point():
            v = {"ok": bool(torch.equal(g, r)), "max_abs": 0.0, "max_rel": 0.0, "reason": "exact"}
        else:
            na, nr = noise.get(path, (0.0, 0.0))
            a_eff = atol
            if scale_atol:
                fin = r.double()[torch.isfinite(r.double())]
                a_eff = atol * max(1.0, float(fin.abs().max()) if fin.numel() else 1.0)
            v = compare(g, r, rtol=rtol, atol=a_eff, noise_abs=na, noise_rel=nr)
        v["path"] = path
        out.append(v)
    return out


@contextmanager
def recording(per_wrapper: int = 4, wrappers: dict | None = None):
    """``with recording() as cap: ...`` -- shorthand for ``Capture``."""
    cap = Capture(per_wrapper, wrappers)
    with cap:
        yield cap
