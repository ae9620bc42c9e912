"""Lever emulator pinned on hand-derived cases of the reference's weave
semantics (lib/SchedWeave.cpp, lib/SchedWorkQueue.cpp), plus the fail-safe
edges a host can force (null tables, num_tasks 0, order_size mismatch, OOB
and duplicate entries, flags gate, W vs tasks)."""
import random
from collections import Counter

import pytest

import levers


def test_remap_static_cases():
    order = [3, 2, 1, 0] + list(range(4, 16))
    assert [levers.remap_static(p, 4, order, None, 16) for p in range(4)] == [3, 2, 1, 0]
    assert [levers.remap_static(p, 4, None, None, 16) for p in range(4)] == [0, 1, 2, 3]
    # out-of-grid entry and negative entry fall back to pid
    bad = [9, -1, 1, 0]
    assert [levers.remap_static(p, 4, bad, None, 16) for p in range(4)] == [0, 1, 1, 0]
    # pid >= max_tasks: no table lookup
    assert levers.remap_static(5, 8, [7] * 8, None, 4) == 5
    # order_size gate: unchecked (0), matching (4), stale (6) -> identity
    assert [levers.remap_static(p, 4, order, {"order_size": 0}, 16) for p in range(4)] == [3, 2, 1, 0]
    assert [levers.remap_static(p, 4, order, {"order_size": 4}, 16) for p in range(4)] == [3, 2, 1, 0]
    assert [levers.remap_static(p, 4, order, {"order_size": 6}, 16) for p in range(4)] == [0, 1, 2, 3]


def test_remap_wq_bounded_by_num_tasks():
    order = [5, 1, 0, 2, 3, 4]
    c = {"num_tasks": 4, "order_size": 0}
    # entry 5 >= num_tasks 4 -> raw
    assert [levers.remap_wq(r, 4, order, c, 16) for r in range(4)] == [0, 1, 0, 2]
    assert [levers.remap_wq(r, 4, order, {"order_size": 5}, 16) for r in range(4)] == [0, 1, 2, 3]


def test_policy_predicate():
    rows = {0: (0.7, 0, 0), 1: (0.5, 0, 0), 2: (0.0, 0, 1), 3: (9.0, 0, 2)}
    c = {"lambda_bw": 0.5, "rows": rows}
    # score = q - 0.5 - 0.1 > 0  <=>  q > 0.6
    assert levers.policy(0, c, 16, H=0.1) == (True, False)
    assert levers.policy(1, c, 16, H=0.1) == (False, False)
    assert levers.policy(2, c, 16, H=0.1) == (True, False)   # hint urgent
    assert levers.policy(3, c, 16, H=0.1) == (False, True)   # hint polite
    assert levers.policy(0, None, 16) == (False, False)
    assert levers.policy(20, c, 16) == (False, False)        # task >= max
    # neutral plane: lambda 0, q 0 -> score -H < 0 -> stock
    assert levers.policy(5, {"rows": {}}, 16) == (False, False)


def test_budget():
    c = {"rows": {0: (0.0, 0, 0), 1: (0.0, 7, 0)}}
    assert levers.budget(0, c, 16) == levers.NOCAP
    assert levers.budget(1, c, 16) == 7
    assert levers.budget(1, None, 16) == levers.NOCAP
    assert levers.budget(40, c, 16) == levers.NOCAP


@pytest.mark.parametrize("ntasks", [1, 7, 64])
@pytest.mark.parametrize("W", [1, 3, 16, 64, 70])
@pytest.mark.parametrize("pi", ["identity", "reversed", "random"])
def test_work_queue_runs_every_task_exactly_once(ntasks, W, pi):
    if pi == "identity":
        order = list(range(ntasks))
    elif pi == "reversed":
        order = list(range(ntasks))[::-1]
    else:
        order = list(range(ntasks))
        random.Random(ntasks * W).shuffle(order)
    c = {"num_tasks": ntasks}
    for seed in range(3):
        ex, rows = levers.run_launch(ntasks=ntasks, grid=W, wq=True, order=order, ctrl=c,
                                     seed=seed)
        assert Counter(ex) == Counter(range(ntasks))
        assert Counter(rows) == Counter(range(ntasks))


def test_work_queue_disarm_switches_to_static():
    order = list(range(8))[::-1]
    # num_tasks == 0 -> stock path over the launched grid, pi still live
    ex, _ = levers.run_launch(ntasks=8, grid=8, wq=True, order=order, ctrl={"num_tasks": 0})
    assert ex == order
    # no queue -> stock path
    ex, _ = levers.run_launch(ntasks=8, grid=8, wq=True, order=order, ctrl={"num_tasks": 8},
                              queue=False)
    assert ex == order
    # stock path with W < tasks serves only W tasks (the host must launch the full grid)
    ex, _ = levers.run_launch(ntasks=8, grid=3, wq=True, ctrl={"num_tasks": 0})
    assert ex == [0, 1, 2]


def test_duplicate_entries_with_unchecked_size_break_exactly_once_and_stamp_fixes_it():
    dup = [0, 0, 2, 3]
    ex, _ = levers.run_launch(ntasks=4, grid=4, wq=False, order=dup, ctrl={"order_size": 0})
    assert Counter(ex) == Counter([0, 0, 2, 3])
    ex, _ = levers.run_launch(ntasks=4, grid=4, wq=False, order=dup, ctrl={"order_size": 5})
    assert ex == [0, 1, 2, 3]


def test_timer_gate():
    _, rows = levers.run_launch(ntasks=5, grid=5, wq=False, ctrl={"flags": 1})
    assert rows == []
    _, rows = levers.run_launch(ntasks=5, grid=5, wq=False, ctrl={"flags": 0}, max_tasks=3)
    assert sorted(rows) == [0, 1, 2]


def test_ctrl_bytes_layout():
    import struct
    b = levers.ctrl_bytes({"num_tasks": 9, "lambda_bw": 0.5, "flags": 1, "order_size": 4,
                           "rows": {2: (0.25, 300, 2)}}, 8)
    assert len(b) == 32 + 64
    assert struct.unpack_from("<I", b, 4)[0] == 9
    assert struct.unpack_from("<f", b, 8)[0] == 0.5
    assert struct.unpack_from("<I", b, 24)[0] == 1
    assert struct.unpack_from("<I", b, 28)[0] == 4
    assert struct.unpack_from("<fHB", b, 32 + 16) == (0.25, 300, 2)
