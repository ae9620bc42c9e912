"""serving.py -- the per-step control loop around a decode step, for any
serving engine (reference python/sched_sglang_plugin.py:148-342, whose
on_batch_begin / on_batch_end / _consume_probe are bound to SGLang's batch
objects; here the engine passes request ids and KV lengths).

Per step, as in the reference:
  on_batch_begin(rids, kv_lens) -> launch arguments for sched_pd.paged_decode
    * advance the last probe's readout, never waiting for the device: once
      the GPU has passed the probe step (event query) its timer rows' copy to
      pinned host memory is queued; once that copy is done (event query) the
      rows are folded into the controller;
    * cadence gate: re-plan every `plan_every` steps, on probe steps, and
      whenever the step's split plan has a different number of work items
      than the installed order or armed queue covers (a request crossed a
      tile boundary: an order of the wrong size would fall back to identity
      in the kernel, a queue would be disarmed); in between the installed
      tables stay;
    * bind work items to requests (one per (request, kv-head) task, or the
      split-KV tiles of plan_tiles);
    * predict per-request cost, spread it over the work items;
    * regime gate: ticket queue armed (W = resident workgroups) when the
      batch has more items than resident slots, a heavy tail
      (max/mean > clc_imbalance) and uncertain predictions
      (> clc_resid); one wave (items <= R): any live order retired, stock
      grid; otherwise the LPT order over items (in groups of lpt_block,
      per item by default), stock grid. Tables are installed at once:
      every write is a copy on the current stream, ordered behind the
      previous step's kernels (the reference plugin writes host-mapped
      tables and waits for the GPU to go idle first). Call the hooks with
      the decode's stream current;
    * hints when the batch's KV exceeds the L2: long requests polite, short
      ones urgent, q = predicted cost;
    * push; clear the timer on probe steps.
  on_batch_end()
    * record the step's completion event; on a probe step keep (event,
      binding) pending and switch the timer off for the following steps;
    * enforcing, host work for the next step while this one is queued on the
      device: advance the probe readout, and when the next step will
      re-plan, compute its decision (cost, regime, plan, order) for the
      batch a decode step predicts (the same requests, one token longer).
      on_batch_begin installs it if the batch and the controller's version
      match, else decides afresh: the same tables either way, but the heavy
      host work no longer sits between a step's start and its launch.
Observing only, a step without a probe launches without the lever tables,
and the plane's timer flag stays on, so the hooks publish the plane once
and then only when the batch's task count or order changes.

begin() / end() wrap the two hooks for an engine loop: a failure is counted,
logged once per site, and that step runs the stock decode. A batch larger
than the plane's tables raises (loudly) instead of being truncated.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from sched_controller import SchedControlPlane
from sched_rt import HINT_POLITE, HINT_URGENT, SchedPlane


@dataclass
class HookConfig:
    """Knobs of the reference plugin's _STATE (python/sched_sglang_plugin.py:
    36-106), with the same defaults."""
    plan_every: int = 8          # re-plan cadence (steps)
    timer_every: int = 8         # probe cadence (steps)
    clc: str = "auto"            # ticket-queue arming: off | on | auto
    clc_resid: float = 0.75      # auto: arm above this prediction uncertainty
    clc_imbalance: float = 3.0   # auto: and above this max/mean item cost
    resident: int = 0            # R, workgroups resident at once (0 = unknown)
    observe_only: bool = False   # bind and measure, never change the schedule
    kv_bytes_per_token: int = 0  # 0 = no hints
    l2_bytes: int = 0            # hint threshold (0 = the device's L2 size)
    page_size: int = 16
    tile_pages: int = 0          # split-KV tile (pages); 0 = one item per task
    # Tile size of the plan under the LPT order (0 = tile_pages). With the
    # heaviest items first the last items are short anyway, and fewer,
    # larger items cost less start-up: on 256 requests (lognormal contexts)
    # the enforcing loop's decode ran 371 us over 128-page tiles, 350 us
    # over 192 and 359 us over 256, while the stock (identity) order wants
    # the smaller tiles (410 / 419 / 423 us).
    lpt_tile_pages: int = 0
    policy: str = "lpt"
    # Group size of the LPT order in the queued regime (the reference's
    # SCHED_LPT_BLOCK, default 16 there for locality between neighbouring
    # tiles). 1 = plain per-item longest-first: on MI355X no workgroup reuses
    # another's data, and on 256 requests over 3352 tiles of 128 pages
    # (lognormal contexts) the static grid ran 401.7 us in list order,
    # 392.2 us with groups of 16 and 341.9 us with per-item LPT.
    lpt_block: int = 1


class ServingHooks:
    """Owns the controller and drives one SchedPlane through the steps."""

    def __init__(self, plane: SchedPlane, num_kv_heads: int, config: HookConfig | None = None,
                 controller: SchedControlPlane | None = None, event_factory=None):
        self.plane = plane
        self.hkv = int(num_kv_heads)
        self.cfg = config or HookConfig()
        self.ctl = controller or SchedControlPlane(policy=self.cfg.policy)
        self._event = event_factory or (lambda: torch.cuda.Event())
        self.step = 0
        self.timer_armed = False
        self.pending = None      # (event, binding, rows) of an unread probe step
        self.inflight = None     # completion event of the last step
        self.binding = None      # (rids, kv_lens, nitems) of the last plan
        self.order_n = None      # items of the live order, None = identity
        self.armed_n = None      # items the armed ticket queue covers
        self.launch = {"plane": plane, "workers": 0, "tiles": None, "tile_pages": 0}
        self.plan_tp = self.cfg.tile_pages   # tile size of the live plan
        if plane.dev.type == "cuda":
            # probe rows read back on a side stream: the readout waits for the
            # probe step only, not for the kernels queued after it
            plane.use_device_timer()
        self.last_batch = None   # (rids, kv_lens) of the last step, enforcing
        self.ahead = None        # a re-plan computed after the last launch
        self.probes_folded = 0
        self.hook_errors = 0
        self._err_sites = set()

    # -- helpers ---------------------------------------------------------------
    def _items(self, kv_lens, tile_pages=None):
        """(tiles or None, item -> request index, pages per item) of the
        plan over tiles of `tile_pages` pages (default: the live plan's)."""
        n = len(kv_lens)
        ps = self.cfg.page_size
        tp = self.plan_tp if tile_pages is None else tile_pages
        pages = -(-np.asarray(kv_lens, np.int64) // ps)
        if tp > 0:
            import sched_pd
            # built on the host (reading a device plan back would wait for
            # the previous step's kernels); the decode uploads it with its
            # other per-step arrays
            tiles = sched_pd.plan_tiles_host(kv_lens, ps, tp, self.hkv)
            req = tiles[:, 0] // self.hkv
            first = tiles[:, 1] * tp
            item_pages = np.clip(pages[req] - first, 0, tp)
            return tiles, req, item_pages
        req = np.repeat(np.arange(n), self.hkv)
        return None, req, pages[req]

    def _count(self, kv_lens, tile_pages) -> int:
        """Work items of the plan over tiles of `tile_pages` pages (without
        building it)."""
        n = len(kv_lens)
        if tile_pages <= 0:
            return n * self.hkv
        pages = -(-np.asarray(kv_lens, np.int64) // self.cfg.page_size)
        return int(np.maximum(1, -(-pages // tile_pages)).sum()) * self.hkv

    def _consume_probe(self) -> None:
        """Fold the pending probe's timer rows (per task) into per-request
        cost (python/sched_sglang_plugin.py:345-377), never waiting for the
        device: once the probe step's event has fired, the rows' copy to the
        host is queued; once that copy's event has fired, they are folded."""
        if self.pending is None:
            return
        ev, b, rows = self.pending
        if not ev.query():
            return
        if rows is None and self.plane.dev.type == "cuda":
            rows, ev2 = self.plane.read_timer_async()
            self.pending = (ev2, b, rows)
            return
        self.pending = None
        rids, kv_list = b[0], b[1]
        n = len(rids)
        cyc = (rows if rows is not None else torch.as_tensor(self.plane.read_timer()))
        cyc = cyc.to(torch.int64).numpy()
        m = min(n * self.hkv, cyc.size)
        per_task = np.zeros(n * self.hkv, np.int64)   # task = request * hkv + head
        per_task[:m] = cyc[:m]
        self.ctl.observe(rids, kv_list, per_task.reshape(n, self.hkv).sum(1).tolist())
        self.probes_folded += 1

    # -- the hooks ---------------------------------------------------------------
    def on_batch_begin(self, rids, kv_lens) -> dict:
        """Tables for this step; returns the launch arguments to pass to
        sched_pd.paged_decode or PagedKvCache.decode / decode_step (plane,
        workers, tiles as a host int32 array, tile_pages)."""
        cfg, p = self.cfg, self.plane
        step = self.step
        self.step += 1
        if not cfg.observe_only:
            self.last_batch = (tuple(rids), np.array(kv_lens, np.int64))
        self._consume_probe()
        probe = step % cfg.timer_every == 0 and self.pending is None
        live = self.armed_n if self.launch["workers"] else self.order_n
        if step % cfg.plan_every != 0 and not probe and \
                (live is None or live == self._count(kv_lens, self.plan_tp)):
            # off cadence, and the installed tables still cover the engine's
            # per-step plan (from host lengths, at the live plan's tile size)
            self.timer_armed = False
            tiles = None
            if self.plan_tp > 0:
                import sched_pd
                tiles = sched_pd.plan_tiles_host(kv_lens, cfg.page_size, self.plan_tp,
                                                 self.hkv)
            self.launch = dict(self.launch, tiles=tiles)
            return self._observed(self.launch)
        # re-plan: the regime is decided over the configured tiles
        kv_list = kv_lens.tolist() if isinstance(kv_lens, np.ndarray) else \
            [int(x) for x in kv_lens]
        rids = list(rids)
        n = len(rids)
        tp = cfg.tile_pages
        nitems = self._count(kv_list, tp)
        if max(nitems, n * self.hkv) > p.N:
            # never truncate a batch to the tables (python/sched_sglang_plugin.py:
            # 99-118): a larger plane is the fix
            raise RuntimeError(f"batch of {nitems} work items / {n * self.hkv} tasks exceeds "
                               f"the plane's max_tasks {p.N}")

        # observing, the plane is bound on probe steps only, so its timer
        # flag stays on and a re-plan publishes nothing new
        p.set_timer_enabled(probe or cfg.observe_only)
        self.timer_armed = probe
        workers = 0
        plan = None          # (tiles, cost per item) of the plan the launch takes
        if not cfg.observe_only:
            d = self._take_ahead(rids, kv_lens)
            if d is None:
                d = self._decide(rids, kv_list, nitems)
            workers, plan, nitems = self._apply(d, kv_list)
        else:
            self._retire_order()
            p.set_num_tasks(0)
            self.plan_tp = tp
        p.push()
        if probe:
            p.clear_timer()
        self.binding = (rids, kv_list, nitems)
        if plan is not None:
            tiles = plan[0]
        else:
            tiles = self._items(kv_list, self.plan_tp)[0]
        self.launch = {"plane": p, "workers": workers, "tiles": tiles,
                       "tile_pages": self.plan_tp if tiles is not None else 0}
        return self._observed(self.launch)

    def _decide(self, rids, kv_list, nitems) -> dict:
        """The enforcing re-plan for a batch, without writing any table:
        predicted cost per request spread over the work items by pages, the
        regime, the plan the launch takes and its order. `nitems` counts the
        items over the configured tiles."""
        cfg, p = self.cfg, self.plane
        tp = cfg.tile_pages
        cost_req = self.ctl.predict(rids, kv_list)
        req_pages = np.maximum(-(-np.asarray(kv_list, np.int64) // cfg.page_size), 1)

        def costed(tile_pages):
            tiles, item_req, item_pages = self._items(kv_list, tile_pages)
            return tiles, torch.as_tensor(
                cost_req[item_req] * item_pages / req_pages[item_req], dtype=torch.float32)

        R = cfg.resident
        arm = cfg.clc == "on"
        plan = None
        if cfg.clc == "auto" and R > 0 and nitems > R and \
                self.ctl.uncertainty(rids, kv_list) > cfg.clc_resid:
            plan = costed(tp)
            cost_item = plan[1]
            imbalance = float(cost_item.max() / max(float(cost_item.mean()), 1e-6))
            arm = imbalance > cfg.clc_imbalance
        d = {"cost_req": cost_req, "nitems": nitems}
        if arm:
            plan = plan or costed(tp)
            d.update(regime="queue", plan=plan, plan_tp=tp,
                     order=SchedPlane.region_order(plan[1], R),
                     workers=R if R > 0 else 2 * p.sm_count())
        elif R > 0 and nitems <= R:
            d.update(regime="one_wave", plan=None, plan_tp=tp)
        else:
            # the LPT order, over its own (larger) tiles when configured
            plan_tp = (cfg.lpt_tile_pages or tp) if tp > 0 else 0
            if plan is None or plan_tp != tp:
                plan = costed(plan_tp)
            d.update(regime="lpt", plan=plan, plan_tp=plan_tp, nitems=plan[1].numel(),
                     order=SchedPlane.region_order(plan[1], 0, block=cfg.lpt_block))
        return d

    def _apply(self, d: dict, kv_list) -> tuple:
        """Install a _decide() result in the plane (tables, item count, hints);
        returns (workers, plan, work items)."""
        p = self.plane
        nitems = d["nitems"]
        workers = 0
        if d["regime"] == "queue":
            p.install_order(d["order"], nitems)
            self.order_n = nitems
            p.set_num_tasks(nitems)
            self.armed_n = nitems
            workers = d["workers"]
        elif d["regime"] == "one_wave":
            self._retire_order()
            p.set_num_tasks(0)
        else:
            p.install_order(d["order"], nitems)
            self.order_n = nitems
            p.set_num_tasks(0)
        self.plan_tp = d["plan_tp"]
        self._hints(kv_list, d["cost_req"])
        return workers, d["plan"], nitems

    def _plan_ahead(self) -> None:
        """Enforcing, after a step's launch: if the next step will re-plan (by
        cadence, or because its item count changes), compute its decision now
        for the batch a decode step predicts (the same requests, each one
        token longer), while the device still has this step queued; the
        next on_batch_begin uses it only if the batch and the controller's
        state (its version, which every fold of measurements advances) are
        those it was computed for."""
        self.ahead = None
        last = self.last_batch
        if self.cfg.observe_only or last is None:
            return
        rids, kv = last
        kv_next = kv + 1
        nxt = self.step
        live = self.armed_n if self.launch["workers"] else self.order_n
        due = nxt % self.cfg.plan_every == 0 or nxt % self.cfg.timer_every == 0
        if not due and (live is None or live == self._count(kv_next, self.plan_tp)):
            return
        kv_list = kv_next.tolist()
        nitems = self._count(kv_list, self.cfg.tile_pages)
        if max(nitems, len(rids) * self.hkv) > self.plane.N:
            return       # on_batch_begin raises for this batch
        d = self._decide(list(rids), kv_list, nitems)
        self.ahead = (nxt, rids, kv_next, self.ctl.version, d)

    def _take_ahead(self, rids, kv_lens):
        """The decision _plan_ahead computed for this step, if it was computed
        for this batch and no probe was folded since; else None."""
        a, self.ahead = self.ahead, None
        if a is None or a[0] != self.step - 1 or a[3] != self.ctl.version:
            return None
        if tuple(rids) != a[1]:
            return None
        kv = np.asarray(kv_lens, np.int64)
        if kv.shape != a[2].shape or not np.array_equal(kv, a[2]):
            return None
        return a[4]

    def _observed(self, launch: dict) -> dict:
        """Observing, a step without a probe has nothing to measure and no
        schedule to change: it launches without the lever tables (the same
        bits, without the per-item pi and policy-row reads)."""
        if self.cfg.observe_only and not self.timer_armed:
            return dict(launch, plane=None, workers=0)
        return launch

    def on_batch_end(self) -> None:
        """After the step's launches (python/sched_sglang_plugin.py:311-342):
        no synchronize; the completion event gates the next table writes and
        the probe readout."""
        ev = self._event()
        ev.record()
        self.inflight = ev
        # host work while this step is queued on the device: an earlier
        # probe's readout first (this step's probe, if any, is pending next)
        self._consume_probe()
        if self.timer_armed:
            self.pending = (ev, self.binding, None)
            if not self.cfg.observe_only:
                # enforcing, the next steps launch with the plane: timer off
                self.plane.set_timer_enabled(False)
                self.plane.push()
        self._plan_ahead()

    # -- engine-facing wrappers: a hook never takes the serving loop down --------
    STOCK = {"plane": None, "workers": 0, "tiles": None, "tile_pages": 0}

    def begin(self, rids, kv_lens) -> dict:
        """on_batch_begin for an engine loop: an exception is counted and
        logged (first per site), and the step runs the stock decode (no
        levers) instead (python/sched_sglang_plugin.py:594-606, 648-662)."""
        try:
            return self.on_batch_begin(rids, kv_lens)
        except Exception as e:  # noqa: BLE001 -- any failure degrades to stock
            self._hook_error("begin", e)
            return dict(self.STOCK)

    def end(self) -> None:
        try:
            self.on_batch_end()
        except Exception as e:  # noqa: BLE001
            self._hook_error("end", e)

    def _hook_error(self, where: str, exc: Exception) -> None:
        self.hook_errors += 1
        if where not in self._err_sites:
            self._err_sites.add(where)
            print(f"[sched-serving] {where} hook error (control plane degraded; serving "
                  f"continues with the stock decode): {exc!r}", flush=True)

    # -- pieces ----------------------------------------------------------------
    def _retire_order(self) -> None:
        if self.order_n is not None:
            self.plane.reset_order()
            self.plane.set_order_size(0)
            self.order_n = None

    def _hints(self, kv_list, cost_req) -> None:
        """Residency hints when the batch's KV exceeds the L2 (reference
        python/sched_sglang_plugin.py:290-301). Rows are per task: the
        kernels read policy rows by task, not by split item."""
        bpt = self.cfg.kv_bytes_per_token
        if not bpt or not kv_list:
            return
        l2 = self.cfg.l2_bytes or torch.cuda.get_device_properties(self.plane.dev).L2_cache_size
        if float(sum(kv_list)) * bpt <= l2:
            return
        thr = float(np.median(cost_req))
        ntask = len(kv_list) * self.hkv
        if ntask > self.plane.N:
            return
        task_req = np.repeat(np.arange(len(kv_list)), self.hkv)
        long_ = cost_req[task_req] >= thr
        self.plane.set_rows(q=cost_req[task_req].astype(np.float32),
                            hint=np.where(long_, HINT_POLITE, HINT_URGENT), n=ntask)

    def stats(self) -> str:
        """One status line (python/sched_sglang_plugin.py:302-309)."""
        b = self.binding
        u = self.ctl.uncertainty(b[0], b[1]) if b and b[0] else 0.0
        return (f"[sched-serving] step={self.step} items={b[2] if b else 0} "
                f"R={self.cfg.resident} probes={self.probes_folded} uncert={u:.2f} "
                f"hook_errors={self.hook_errors} "
                f"mode={'observe' if self.cfg.observe_only else 'enforce'}")
