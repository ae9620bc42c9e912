"""Lever emulator -- TEST INFRASTRUCTURE ONLY (imported by tests/ alone).

A CPU restatement of the decisions the reference weave makes for each lever,
so the tests can predict exactly which tasks a launch executes and which
timer rows it writes, and check the GPU against that prediction:

  remap_static   lib/SchedWeave.cpp:444-526   pi on the static grid
  remap_wq       lib/SchedWorkQueue.cpp:305-343  pi inside the claim loop
  policy         lib/SchedWeave.cpp:532-581   urgent / polite flags
  budget         lib/SchedWeave.cpp:585-614   shed budget (tau)
  run_launch     lib/SchedWorkQueue.cpp:345-448 + SchedWeave.cpp:979-1049
                 the tasks each workgroup executes and the timer rows hit

Tables are plain Python: order (list of int32 or None), ctrl (dict with
num_tasks, lambda_bw, flags, order_size, rows: {task: (q, tau, hint)}) or None.
"""
from __future__ import annotations

import random
import struct

NOCAP = 0xFFFFFFFF
U32 = 0xFFFFFFFF


def _u32(x: int) -> int:
    return x & U32


def remap_static(pid, nctaid, order, ctrl, max_tasks):
    if order is None or pid >= max_tasks:
        return pid
    mapped = _u32(order[pid])
    size_ok = True
    if ctrl is not None:
        osz = ctrl.get("order_size", 0)
        size_ok = osz == 0 or osz == nctaid
    return mapped if (mapped < nctaid and size_ok) else pid


def remap_wq(raw, num_tasks, order, ctrl, max_tasks):
    if order is None or raw >= max_tasks:
        return raw
    mapped = _u32(order[raw])
    osz = ctrl.get("order_size", 0)
    ok = mapped < num_tasks and (osz == 0 or osz == num_tasks)
    return mapped if ok else raw


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def policy(task, ctrl, max_tasks, dT=1.0, dR=1.0, H=0.25):
    """(urgent, polite), computed in float32 like the kernel."""
    if ctrl is None or task >= max_tasks:
        return False, False
    q, tau, hint = ctrl.get("rows", {}).get(task, (0.0, 0, 0))
    lam = ctrl.get("lambda_bw", 0.0)
    score = _f32(_f32(_f32(_f32(q) * _f32(dT)) - _f32(_f32(lam) * _f32(dR))) - _f32(H))
    urgent = hint == 1 or (hint == 0 and score > 0.0)
    return urgent, hint == 2


def budget(task, ctrl, max_tasks):
    if ctrl is None or task >= max_tasks:
        return NOCAP
    tau = ctrl.get("rows", {}).get(task, (0.0, 0, 0))[1]
    return tau if tau else NOCAP


def run_launch(*, ntasks, grid, wq, order=None, ctrl=None, queue=True,
               max_tasks=4096, queue_start=None, seed=0):
    """Simulate one launch. Returns (executed, timer_rows):
    executed: list of task ids in the order the bodies ran (claim order is
    randomised with `seed` to cover interleavings; the set/multiset is what
    the invariants speak about); timer_rows: multiset of rows incremented.
    Tasks >= ntasks are skipped by the body (bounds guard)."""
    executed = []
    timer_off = ctrl is not None and (ctrl.get("flags", 0) & 1)
    timer_on = not timer_off

    def body(task):
        if task >= ntasks:
            return
        executed.append(task)

    if not wq:
        for pid in range(grid):
            body(remap_static(pid, grid, order, ctrl, max_tasks))
    else:
        armed = queue and ctrl is not None
        nt = ctrl.get("num_tasks", 0) if armed else 0
        if nt == 0:
            for pid in range(grid):
                body(remap_static(pid, grid, order, ctrl, max_tasks))
        else:
            counter = grid if queue_start is None else queue_start
            rng = random.Random(seed)
            live = [pid for pid in range(grid) if pid < nt]
            raw = {pid: pid for pid in live}
            while live:
                pid = rng.choice(live)
                body(remap_wq(raw[pid], nt, order, ctrl, max_tasks))
                t = counter
                counter += 1
                if t >= nt:
                    live.remove(pid)
                else:
                    raw[pid] = t
    rows = [t for t in executed if t < max_tasks] if timer_on else []
    return executed, rows


def ctrl_bytes(ctrl, max_tasks):
    """Serialise a ctrl dict into SchedCtrl bytes (header + max_tasks rows)."""
    buf = bytearray(32 + 8 * max_tasks)
    struct.pack_into("<II4fII", buf, 0, ctrl.get("generation", 0), ctrl.get("num_tasks", 0),
                     ctrl.get("lambda_bw", 0.0), 0.0, 0.0, 0.0, ctrl.get("flags", 0),
                     ctrl.get("order_size", 0))
    for task, (q, tau, hint) in ctrl.get("rows", {}).items():
        if task < max_tasks:
            struct.pack_into("<fHBB", buf, 32 + 8 * task, q, tau, hint, 0)
    return bytes(buf)
