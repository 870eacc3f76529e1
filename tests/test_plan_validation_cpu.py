"""Plan creation refuses malformed layouts before any device work (CPU: the C ABI is called directly).

``kb_plan_create`` validates the host layout before its first HIP call, so a
refused layout returns KB_ERR_ARG (-1) here without a GPU.  Each case corrupts
one field of the tiny problem's layout: int64 values are range-checked before
they are narrowed (a value that would wrap into range is refused), and every
row must lie in exactly one wave.
"""

import ctypes as ct

import pytest

import kbtest


def _arrays():
    from kbench.fused import layout_arrays, problem_to_captured
    from kbench.runtime import make_static

    static = make_static(problem_to_captured(kbtest.problem("tiny", None)), "cpu")
    return layout_arrays(static)


def _create(arrays):
    from kbench import _native as N
    from kbench.fused import kb_layout

    lib = N.lib()
    L = kb_layout(arrays)
    handle = ct.c_void_p()
    rc = lib.kb_plan_create(ct.byref(L), ct.byref(handle))
    return rc, lib.kb_last_error().decode()


def _first_leaf_row(a):
    w = int(next(i for i, h in enumerate(a["wave_has_splits"]) if not h))
    return int(a["wave_start"][w])


def _corrupt_leaf_state(a, value):
    a["leaf_state_index"][_first_leaf_row(a)] = value


def _corrupt_wave_overlap(a):
    a["wave_size"][0] += 1  # the first row of wave 1 is claimed by wave 0 too


def _corrupt_wave_gap(a):
    a["wave_size"][-1] -= 1  # the last row is in no wave


CASES = {
    "leaf state = S": (lambda a: _corrupt_leaf_state(a, a["S"]), "leaf state"),
    "leaf state wraps to 1 as int32": (lambda a: _corrupt_leaf_state(a, 2 ** 32 + 1), "leaf state"),
    "leaf state < -1": (lambda a: _corrupt_leaf_state(a, -2), "leaf state"),
    "root row wraps to 0 as int32": (lambda a: a["root_row_ids"].__setitem__(0, 2 ** 32), "root_row_ids"),
    "item index wraps to 0 as int32": (lambda a: a["rate_item_idx"].__setitem__(0, 2 ** 32), "rate_item_idx"),
    "overlapping waves": (_corrupt_wave_overlap, "lies in waves"),
    "row in no wave": (_corrupt_wave_gap, "lies in no wave"),
}


@pytest.mark.parametrize("case", list(CASES))
def test_plan_create_refuses(case):
    corrupt, message = CASES[case]
    a = _arrays()
    corrupt(a)
    rc, msg = _create(a)
    print(f"  {case}: rc={rc} '{msg}'")
    assert rc == -1 and message in msg
