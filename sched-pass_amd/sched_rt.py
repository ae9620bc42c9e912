"""sched_rt.py -- the per-step scheduling control plane on torch-ROCm, with the
API of reference python/sched_rt.py:287-609 (SchedPlane).

The reference keeps its tables in a fixed-VA host mapping registered with the
driver (so a JIT-compiled kernel can bake the addresses). The kernels here take
the table addresses as launch arguments instead, so the tables live in device
memory: one 1 MiB device arena with the reference's offsets (ORDER 0x0,
CTRL 0x40000, TIMER 0x80000, QUEUE 0xC0000). Consequences:
  * setters write a host mirror; push() copies it to the device in stream
    order (rows first, the generation word last, as the reference does);
  * the timer rows are device memory already (what the reference measured
    for the observation channel: device atomics are ~free, host-mapped ones
    cost +26.5%); read_timer() is a device-to-host copy on a side stream;
  * clear_timer() is a fill kernel, so it is safe inside captured graphs.
Out of scope on purpose (they exist for the reference's clang-JIT cache or
inspect NVIDIA binaries): bake_env, arm_process_env, compute_bake_env,
_weave_tag, the fixed-VA guarantee, r_for_cached_so.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import torch

from sched_abi import (CTRL_FLAGS_OFF, CTRL_LAMBDA_OFF, CTRL_NUM_TASKS_OFF,
                       CTRL_ORDER_SIZE_OFF, CTRL_ROWS_OFF, FLAG_TIMER_OFF,
                       HINT_AUTO, HINT_POLITE, HINT_URGENT, ROW_SIZE, last_error,
                       load_library)
from sched_pd import desc_order, upload_into

__all__ = ["SchedPlane", "SchedArenaError", "HINT_AUTO", "HINT_URGENT",
           "HINT_POLITE", "FLAG_TIMER_OFF", "MANIFEST", "LEVER_ARMING"]

# Arena layout (reference python/sched_rt.py:84-89).
ORDER_OFF = 0x00000
CTRL_OFF = 0x40000
TIMER_OFF = 0x80000
QUEUE_OFF = 0xC0000
ARENA_BYTES = 0x100000
MAX_TASKS_LIMIT = 16384

# Lever manifest in the row shape of reference python/sched_rt.py:72-79 (the
# mirror of include/sched/SchedManifest.h:76-105): name, effect, min_sm, compile
# knob, disable sense, cache tag; list order = the order the kernels apply the
# levers in (the claim loop, then the remap, the budget, the stream's policy,
# the timer's commit). The last four fields belong to the reference's
# compile-time weave and do not apply here: every lever runs on gfx950
# (min_sm 0), none is compiled in or out (knob None, disable False) and there
# is no JIT cache (tag ""); each is armed per launch by its table. The
# reference's sixth row, "pdl" (programmatic dependent launch, sm90), has no
# counterpart on a HIP stream and is not listed.
MANIFEST = [
    ("workqueue", "acquire", 0, None, False, ""),
    ("pi", "E1/permute", 0, None, False, ""),
    ("shed", "E2/budget", 0, None, False, ""),
    ("policy", "E0/hint", 0, None, False, ""),
    ("timer", "O/observe", 0, None, False, ""),
]

# How each lever is armed here: the tables it reads and the switch.
LEVER_ARMING = {
    "workqueue": ("ctrl,queue", "launch with workers=W and num_tasks > 0"),
    "pi": ("order,ctrl", "order table (identity by default), order_size in {0, N}"),
    "shed": ("ctrl", "row tau > 0"),
    "policy": ("ctrl", "row hint, or q*dT - lambda_bw*dR - H > 0"),
    "timer": ("timer,ctrl", "timer table, flags bit0 clear"),
}


class SchedArenaError(RuntimeError):
    """The device arena could not be created, or its tables not bound."""


# The plane last bound to the library's __sched_* slots (bind_launcher),
# held so that its tables outlive the launches that read them there.
_BOUND = None


class SchedPlane:
    """Per-step scheduling tables for the decode kernels (one per device)."""

    def __init__(self, max_tasks: int = 4096, device: str = "cuda"):
        if max_tasks > MAX_TASKS_LIMIT:
            raise ValueError(f"a plane holds at most {MAX_TASKS_LIMIT} rows per table "
                             f"(asked for {max_tasks}): each table sits in a 256 KiB "
                             "slot of the arena")
        self.N = int(max_tasks)
        self.dev = torch.device(device)
        try:
            self.arena = torch.zeros(ARENA_BYTES, dtype=torch.uint8, device=self.dev)
        except RuntimeError as e:
            raise SchedArenaError(f"arena allocation failed: {e}") from e
        self._order_arena = self.arena[ORDER_OFF:ORDER_OFF + 4 * self.N].view(torch.int32)
        self.ctrl_bytes = CTRL_ROWS_OFF + ROW_SIZE * self.N
        self._ctrl_dev = self.arena[CTRL_OFF:CTRL_OFF + self.ctrl_bytes]
        self._timer_arena = self.arena[TIMER_OFF:TIMER_OFF + 8 * self.N].view(torch.int64)
        self._queue = self.arena[QUEUE_OFF:QUEUE_OFF + 4].view(torch.int32)
        self._ctrl_host = bytearray(self.ctrl_bytes)
        self._rows_end = self.ctrl_bytes  # mirror bytes push() must copy (rows written)
        self._generation = 0
        self._pushed_hdr = None    # header body (bytes 4 .. rows) last published
        self._timer_dev = None      # separate device row buffer (use_device_timer)
        self._timer_stream = None
        self._order_dev = None      # separate device order table (use_device_order)
        self.reset_order()
        self.push()

    # -- table addresses for the launcher ------------------------------------
    def _order_view(self) -> torch.Tensor:
        return self._order_dev if self._order_dev is not None else self._order_arena

    def _timer_view(self) -> torch.Tensor:
        return self._timer_dev if self._timer_dev is not None else self._timer_arena

    def tables(self) -> dict:
        return {"order": self._order_view().data_ptr(),
                "ctrl": self._ctrl_dev.data_ptr(),
                "timer": self._timer_view().data_ptr(),
                "queue": self._queue.data_ptr()}

    # -- the slot-reading launchers ---------------------------------------------
    def bind_launcher(self) -> None:
        """Put this plane's tables into the library's __sched_* slots, so the
        launchers that read their levers from the slots -- the reference's
        launch_paged_softmax (python/kernels/paged_softmax.cu:47-54), and
        paged_decode(..., rt_tables=True) -- run with this plane's pi, rows,
        timer and queue, its max_tasks rows bounding the task ids that get
        levers. The reference reaches the same by baking the plane's
        addresses into a JIT build (bake_env, python/sched_rt.py:489-555).
        What the plane pushes afterwards takes effect at the next launch;
        use_device_timer / use_device_order re-bind the moved table. One
        plane is bound per process (the slots are the library's); another
        plane's bind_launcher, unbind_launcher, or the C runtime's
        sched_rt_init / sched_rt_disarm end the binding. The module holds
        the bound plane, so its tables outlive every launch that reads them
        from the slots."""
        global _BOUND
        with torch.cuda.device(self.dev):
            t = self.tables()
            lib = load_library()
            if not lib.sched_rt_bind_tables(ctypes.c_void_p(t["order"]),
                                            ctypes.c_void_p(t["ctrl"]),
                                            ctypes.c_void_p(t["timer"]),
                                            ctypes.c_void_p(t["queue"]), self.N):
                raise SchedArenaError(f"binding the plane's tables failed: {last_error()}")
        _BOUND = self

    def unbind_launcher(self) -> None:
        """Null the slots if they hold this plane's tables (the slot-reading
        launchers then run stock)."""
        global _BOUND
        if self.bound:
            with torch.cuda.device(self.dev):
                if not load_library().sched_rt_disarm():
                    raise SchedArenaError(f"unbinding failed: {last_error()}")
        if _BOUND is self:
            _BOUND = None

    @property
    def bound(self) -> bool:
        """True while the slots hold this plane's tables (read back from the
        device: synchronous)."""
        if _BOUND is not self:
            return False
        slots = (ctypes.c_uint64 * 4)()
        with torch.cuda.device(self.dev):
            if not load_library().sched_rt_slots(slots):
                raise SchedArenaError(f"reading the slots failed: {last_error()}")
        t = self.tables()
        return list(slots) == [t["order"], t["ctrl"], t["timer"], t["queue"]]

    @property
    def num_tasks(self) -> int:
        return struct.unpack_from("<I", self._ctrl_host, CTRL_NUM_TASKS_OFF)[0]

    def use_device_timer(self) -> None:
        """Move the observation rows to their own device buffer, read back on
        a side stream (reference python/sched_rt.py:319-331)."""
        if self._timer_dev is None:
            was_bound = self.bound
            self._timer_dev = torch.zeros(self.N, dtype=torch.int64, device=self.dev)
            self._timer_stream = torch.cuda.Stream(device=self.dev)
            if was_bound:
                self.bind_launcher()

    def use_device_order(self) -> None:
        """Kernel-resident order table in its own device tensor, installable
        device-to-device without a host sync (python/sched_rt.py:333-347).
        Starts as identity."""
        if self._order_dev is None:
            was_bound = self.bound
            self._order_dev = torch.arange(self.N, dtype=torch.int32, device=self.dev)
            if was_bound:
                self.bind_launcher()

    # -- pi (python/sched_rt.py:365-395) ---------------------------------------
    def set_order(self, tasks) -> None:
        """tasks[i] = the task the i-th claim / workgroup serves (a prefix;
        the tail keeps its current entries)."""
        t = torch.as_tensor(tasks, dtype=torch.int32)
        n = min(t.numel(), self.N)
        if t.is_cuda:
            self._order_view()[:n].copy_(t[:n])
        else:
            upload_into(self._order_view()[:n], t[:n])   # queued, not waited for

    def reset_order(self) -> None:
        self.set_order(torch.arange(self.N, dtype=torch.int32))

    def set_order_size(self, n: int) -> None:
        struct.pack_into("<I", self._ctrl_host, CTRL_ORDER_SIZE_OFF, int(n))

    def install_order(self, tasks, n: int) -> None:
        """Table first, validity stamp second (published by the next push).
        A permutation of more than max_tasks work items cannot be installed:
        the items past the table would keep their own ids while the table
        maps others onto them (duplicated and missing work)."""
        if int(n) > self.N:
            raise ValueError(f"order for {n} work items exceeds the plane's {self.N} rows")
        self.set_order(tasks)
        self.set_order_size(n)

    # -- ctrl mirror (python/sched_rt.py:397-443) -------------------------------
    def set_lambda(self, bw=0.0, l2=0.0, smem=0.0, comp=0.0) -> None:
        struct.pack_into("<4f", self._ctrl_host, CTRL_LAMBDA_OFF,
                         float(bw), float(l2), float(smem), float(comp))

    def set_num_tasks(self, n: int) -> None:
        """Also the per-step work-queue switch: 0 = stock static path."""
        struct.pack_into("<I", self._ctrl_host, CTRL_NUM_TASKS_OFF, int(n))

    def set_timer_enabled(self, on: bool) -> None:
        (flags,) = struct.unpack_from("<I", self._ctrl_host, CTRL_FLAGS_OFF)
        flags = (flags & ~FLAG_TIMER_OFF) | (0 if on else FLAG_TIMER_OFF)
        struct.pack_into("<I", self._ctrl_host, CTRL_FLAGS_OFF, flags)

    def set_row(self, i: int, q: float = 0.0, tau: int = 0, hint: int = HINT_AUTO) -> None:
        if not 0 <= i < self.N:
            raise IndexError(f"row {i} outside [0, {self.N})")
        struct.pack_into("<fHBB", self._ctrl_host, CTRL_ROWS_OFF + ROW_SIZE * i,
                         float(q), int(tau) & 0xFFFF, int(hint) & 0xFF, 0)
        self._rows_end = max(self._rows_end, CTRL_ROWS_OFF + ROW_SIZE * (i + 1))

    def set_rows(self, q=None, tau=None, hint=None, n: int | None = None) -> None:
        """Vectorised set_row over rows [0, n)."""
        import numpy as np
        n = self.N if n is None else int(n)
        rows = np.zeros(n, dtype=[("q", "<f4"), ("tau", "<u2"), ("hint", "u1"), ("pad", "u1")])
        if q is not None:
            rows["q"] = np.asarray(torch.as_tensor(q, dtype=torch.float32).cpu())[:n]
        if tau is not None:
            rows["tau"] = np.asarray(torch.as_tensor(tau, dtype=torch.int64).cpu())[:n] & 0xFFFF
        if hint is not None:
            rows["hint"] = np.asarray(torch.as_tensor(hint, dtype=torch.int64).cpu())[:n] & 0xFF
        self._ctrl_host[CTRL_ROWS_OFF:CTRL_ROWS_OFF + ROW_SIZE * n] = rows.tobytes()
        self._rows_end = max(self._rows_end, CTRL_ROWS_OFF + ROW_SIZE * n)

    def push(self) -> None:
        """Publish the mirror (generation++): rows and header body first, the
        generation word last, in stream order. Nothing is queued when no row
        was written since the last push and the header body holds the bytes
        last published (the kernels only read the block)."""
        hdr = bytes(self._ctrl_host[4:CTRL_ROWS_OFF])
        if self._rows_end == 0 and hdr == self._pushed_hdr:
            return
        self._pushed_hdr = hdr
        self._generation += 1
        struct.pack_into("<I", self._ctrl_host, 0, self._generation)
        # the header plus the rows written since the last push (rows past
        # them hold the same bytes on both sides)
        end = max(CTRL_ROWS_OFF, self._rows_end)
        self._rows_end = 0
        host = torch.frombuffer(bytearray(self._ctrl_host[:end]), dtype=torch.uint8)
        # pinned staging: the copies are queued, not waited for
        upload_into(self._ctrl_dev[4:end], host[4:])
        upload_into(self._ctrl_dev[:4], host[:4])

    # -- timer (python/sched_rt.py:446-462) -------------------------------------
    def clear_timer(self) -> None:
        self._timer_view().zero_()

    def read_timer(self) -> torch.Tensor:
        """Per-task cycles as an int64 CPU tensor. The caller guarantees the
        writing launches are complete (after a sync or an event)."""
        t = self._timer_view()
        if self._timer_stream is not None:
            with torch.cuda.stream(self._timer_stream):
                out = t.to("cpu", non_blocking=True)
            self._timer_stream.synchronize()
            return out
        return t.cpu()

    def read_timer_async(self):
        """(rows, event): a device-to-host copy of the per-task cycles into a
        pinned int64 buffer, queued on the timer stream (use_device_timer) or
        the current one; the rows are valid once event.query() is true. The
        buffer is reused by the next call: read it first. The caller
        guarantees the writing launches are complete."""
        t = self._timer_view()
        if getattr(self, "_timer_host", None) is None or self._timer_host.numel() != t.numel():
            self._timer_host = torch.empty(t.numel(), dtype=torch.int64, pin_memory=True)
        s = self._timer_stream or torch.cuda.current_stream(self.dev)
        with torch.cuda.stream(s):
            self._timer_host.copy_(t, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(s)
        return self._timer_host, ev

    # -- work queue (python/sched_rt.py:464-471) --------------------------------
    def reset_queue(self, workers: int) -> None:
        self._queue.fill_(int(workers))
        self._queue_w = int(workers)

    def prime_queue(self, workers: int) -> None:
        """Prime the ticket counter for a launch of `workers` workers unless it
        already holds that value: a launch that took its last ticket leaves the
        counter at its own worker count, so only a change of W needs a write
        (a stream-ordered fill, safe in captured graphs)."""
        if getattr(self, "_queue_w", None) != int(workers):
            self.reset_queue(workers)

    # -- resident-prefix sizing (python/sched_rt.py:478-487) --------------------
    def sm_count(self) -> int:
        return torch.cuda.get_device_properties(self.dev).multi_processor_count

    def r_from_occupancy(self, blocks_per_sm: int) -> int:
        return int(blocks_per_sm) * self.sm_count()

    # -- pi builders (python/sched_rt.py:557-609) --------------------------------
    @staticmethod
    def _grouped_lpt(c, block: int) -> torch.Tensor:
        """Tiles grouped `block` at a time by index (tile i in group i //
        block); groups served in descending summed cost, tiles of a group in
        ascending index. block <= 1, or a batch of at most one group, is plain
        longest-first. Every sort is stable: ties keep ascending index."""
        cost = np.asarray(torch.as_tensor(c).float().flatten(), np.float64)
        n = cost.size
        if block <= 1 or n <= block:
            return torch.from_numpy(desc_order(cost).astype(np.int32))
        group = np.arange(n) // block
        group_cost = np.bincount(group, weights=cost)
        rank = np.empty(group_cost.size, np.int64)
        rank[desc_order(group_cost)] = np.arange(group_cost.size)
        # primary key: the group's rank; secondary: the tile index (a stable
        # ascending sort by rank)
        order = desc_order(-rank[group].astype(np.float64))
        return torch.from_numpy(order.astype(np.int32))

    @staticmethod
    def region_order(cost, R: int, block: int | None = None) -> torch.Tensor:
        """pi for a launch of R resident workers over n tiles. n <= R: every
        tile starts at once, so tiles are grouped for locality (grouped
        longest-first, block 16 by default). n > R: the R tiles that start
        first alternate the heaviest ceil(R/2) (heaviest first) with the
        lightest floor(R/2) (lightest first), so heavy work starts early
        and light work frees workers to claim more; the remaining tiles
        follow heaviest first."""
        c = np.asarray(torch.as_tensor(cost).float().flatten(), np.float64)
        n = c.size
        if R <= 0 or n <= int(R):
            return SchedPlane._grouped_lpt(torch.from_numpy(c), 16 if block is None else block)
        R = int(R)
        by_cost = desc_order(c)
        n_heavy = (R + 1) // 2
        n_light = R - n_heavy
        heavy, middle, light = np.split(by_cost, [n_heavy, n - n_light])
        first = np.empty(R, np.int64)
        first[0::2] = heavy
        first[1::2] = light[::-1]
        return torch.from_numpy(np.concatenate([first, middle]).astype(np.int32))
