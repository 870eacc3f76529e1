"""Capture / replay mechanics on the CPU, with a stand-in wrapper module.

The stand-in has the traits of the real wrappers: it writes rows of an output
it receives as a view of a larger buffer, mutates an argument that aliases
another, allocates a return tensor with ``torch.empty`` and leaves some of it
unwritten.  The capture must rebuild views and aliases exactly, mask the
unwritten positions, find no noise in a deterministic function, survive a
``weights_only`` save / load, and its replay gate must fail an injected error
(also on a single element) while ignoring changes at unwritten positions (the
reference's negative tests, its docs/FIXES.md:81-85 and 121-135).
"""

import sys
import types

import pytest
import torch

from kbench import capture as cap

MOD = "kbtest_fake_wrappers"


def _step(x, out, acc, *, ws, W, scale=2.0):
    """out[ws:ws+W] = scale * x[ws:ws+W]; acc += out rows; returns rows with odd columns unwritten."""
    rows = x[ws:ws + W] * scale
    out[ws:ws + W] = rows
    acc += rows.sum(dim=0)
    ret = torch.empty((W, x.shape[1]))
    ret[:, ::2] = rows[:, ::2] + 1.0
    return ret


@pytest.fixture()
def fake_module():
    m = types.ModuleType(MOD)
    m.step = _step
    sys.modules[MOD] = m
    yield m
    sys.modules.pop(MOD, None)


def _drive(m, x, buf, acc):
    for ws in (0, 2, 4):
        m.step(x, buf, acc, ws=ws, W=2)
    m.step(x, buf, acc, ws=0, W=2)  # same integer key: not recorded again


def test_capture_replay_round_trip(fake_module, tmp_path):
    x = torch.arange(48, dtype=torch.float32).reshape(6, 8)
    buf = torch.zeros(6, 8)
    acc = buf[5]  # aliases the output buffer (its last row)
    with cap.Capture(per_wrapper=3, wrappers={"step": MOD}) as c:
        _drive(fake_module, x, buf, acc)
    assert [r["key"] for r in c.records] == [[0, 2], [2, 2], [4, 2]]
    path = tmp_path / "cap.pt"
    c.save(path)
    records, pool = cap.Capture.load(path)
    # the alias survives the rebuild: acc is a view of the output buffer
    args, kwargs = cap.rebuild(records[1]["pre"], pool, "cpu")
    assert args[2].untyped_storage().data_ptr() == args[1].untyped_storage().data_ptr()
    assert args[2].storage_offset() == 5 * 8
    cap.measure_noise(records, pool, device="cpu")
    for r in records:
        assert r["noise"] == {}                       # deterministic: no run-to-run difference
        mask = r["valid"]["[2]"]                      # the return value's odd columns are unwritten
        assert mask[:, ::2].all() and not mask[:, 1::2].any()
        verdicts = cap.replay(r, pool, device="cpu")
        assert verdicts and all(v["ok"] for v in verdicts), verdicts


def test_replay_gate_fails_an_injected_error_and_ignores_unwritten_positions(fake_module):
    x = torch.randn(6, 8)
    buf = torch.zeros(6, 8)
    with cap.Capture(per_wrapper=3, wrappers={"step": MOD}) as c:
        _drive(fake_module, x, buf, buf[5])
    cap.measure_noise(c.records, c.pool, device="cpu")
    rec = c.records[1]

    def off_by_one_element(*a, **k):
        ret = _step(*a, **k)
        a[1][k["ws"], 3] += 1e-2  # one element of the written rows
        return ret

    def scribbles_on_unwritten(*a, **k):
        ret = _step(*a, **k)
        ret[:, 1::2] = 123.0
        return ret

    bad = cap.replay(rec, c.pool, device="cpu", fn=off_by_one_element, rtol=1e-6, atol=1e-6)
    assert not all(v["ok"] for v in bad)
    fine = cap.replay(rec, c.pool, device="cpu", fn=scribbles_on_unwritten, rtol=1e-6, atol=1e-6)
    assert all(v["ok"] for v in fine)


def test_compare_is_inf_safe():
    ninf = float("-inf")
    a = torch.tensor([ninf, 1.0, float("nan")])
    assert cap.compare(a, a.clone(), rtol=0, atol=0)["ok"]
    assert not cap.compare(torch.tensor([ninf, 1.0]), torch.tensor([0.0, 1.0]), rtol=1, atol=1)["ok"]
    assert cap.compare(torch.tensor([1.0]), torch.tensor([1.1]), rtol=0, atol=0, noise_abs=0.03)["ok"]
