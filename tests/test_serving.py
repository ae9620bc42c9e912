"""The engine-agnostic serving hooks on the CPU (a SchedPlane in host memory,
events faked): cadence, probes, the timer fold, each regime of the gate and
the hints, against the reference plugin's rules
(python/sched_sglang_plugin.py:148-377)."""
import struct

import numpy as np
import torch

import sched_abi as abi
from sched_rt import HINT_POLITE, HINT_URGENT, SchedPlane
from serving import HookConfig, ServingHooks


class Ev:
    def __init__(self, done=True):
        self.done = done

    def record(self):
        pass

    def query(self):
        return self.done


def plane(n=256):
    return SchedPlane(max_tasks=n, device="cpu")


def ctrl_u32(p, off):
    return struct.unpack_from("<I", bytes(p._ctrl_dev[:64].numpy()), off)[0]


def order(p, n):
    return p._order_view()[:n].tolist()


def test_cadence_gate_and_probe_timer():
    p = plane()
    h = ServingHooks(p, 2, HookConfig(plan_every=4, timer_every=4), event_factory=Ev)
    rids, kv = [10, 11, 12], [100, 900, 300]
    gen0 = p._generation
    h.on_batch_begin(rids, kv)               # step 0: plan + probe
    assert h.timer_armed and p._generation == gen0 + 1
    assert ctrl_u32(p, abi.CTRL_FLAGS_OFF) & abi.FLAG_TIMER_OFF == 0
    h.on_batch_end()                         # probe pending, timer off pushed
    assert h.pending is not None
    assert ctrl_u32(p, abi.CTRL_FLAGS_OFF) & abi.FLAG_TIMER_OFF
    g = p._generation
    for _ in range(3):                       # steps 1..3: off cadence, no writes
        h.on_batch_begin(rids, kv)
        h.on_batch_end()
        assert not h.timer_armed
    assert p._generation == g


def test_probe_fold_is_per_request_sum_over_kv_heads():
    p = plane()
    h = ServingHooks(p, 2, HookConfig(plan_every=1, timer_every=1), event_factory=Ev)
    rids, kv = [7, 8], [64, 512]
    h.on_batch_begin(rids, kv)
    p._timer_view()[:4] = torch.tensor([10, 20, 300, 400])   # tasks (r, h)
    h.on_batch_end()
    seen = {}
    h.ctl.observe = lambda r, k, c: seen.update(r=r, k=k, c=c)
    h.on_batch_begin(rids, kv)
    assert seen == {"r": [7, 8], "k": [64, 512], "c": [30, 700]}
    assert h.probes_folded == 1


def test_probe_waits_for_its_event():
    p = plane()
    ev = Ev(done=False)
    h = ServingHooks(p, 1, HookConfig(plan_every=1, timer_every=1), event_factory=lambda: ev)
    h.on_batch_begin([1], [16])
    h.on_batch_end()
    h.on_batch_begin([1], [16])              # GPU not done: stays pending
    assert h.pending is not None and h.probes_folded == 0
    ev.done = True
    h.on_batch_begin([1], [16])
    assert h.probes_folded == 1


def test_one_wave_retires_order_and_stays_static():
    p = plane()
    h = ServingHooks(p, 2, HookConfig(plan_every=1, timer_every=100, resident=64),
                     event_factory=Ev)
    h.order_n = 6
    p.set_order(torch.tensor([5, 4, 3, 2, 1, 0]))
    p.set_order_size(6)
    launch = h.on_batch_begin([1, 2, 3], [10, 20, 30])
    assert launch["workers"] == 0 and h.order_n is None
    assert order(p, 6) == list(range(6)) and ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 0
    assert ctrl_u32(p, abi.CTRL_NUM_TASKS_OFF) == 0


def test_queued_regime_installs_lpt_with_a_step_in_flight():
    # the order is a stream-ordered copy behind the previous step's kernels:
    # installed at once, without waiting for the GPU to go idle
    p = plane()
    ev = Ev(done=False)
    h = ServingHooks(p, 1, HookConfig(plan_every=1, timer_every=100, resident=2, clc="off"),
                     event_factory=lambda: ev)
    kv = [16, 4096, 512, 64]
    h.on_batch_end()                         # a step in flight
    h.on_batch_begin([0, 1, 2, 3], kv)
    assert h.order_n == 4
    assert order(p, 4) == SchedPlane.region_order(torch.tensor(kv, dtype=torch.float32),
                                                  0, block=1).tolist()
    assert ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 4


def test_queued_regime_lpt_group_size():
    # per-item longest-first by default; the reference's grouped form with
    # lpt_block = 16
    kv = [int(x) for x in np.random.default_rng(3).integers(16, 4096, 40)]
    for block in (1, 16):
        p = plane()
        h = ServingHooks(p, 1, HookConfig(plan_every=1, timer_every=100, resident=2, clc="off",
                                          lpt_block=block), event_factory=lambda: Ev(done=True))
        h.on_batch_begin(list(range(40)), kv)
        want = SchedPlane.region_order(torch.tensor(kv, dtype=torch.float32), 0, block=block)
        assert order(p, 40) == want.tolist(), block
    assert SchedPlane.region_order(torch.tensor(kv, dtype=torch.float32), 0, block=1).tolist() \
        != SchedPlane.region_order(torch.tensor(kv, dtype=torch.float32), 0, block=16).tolist()


def test_auto_arms_the_queue_only_for_an_uncertain_heavy_tail():
    kv_tail = [16] * 31 + [16384]
    kv_flat = [1024] * 32
    for kv, expect in ((kv_tail, True), (kv_flat, False)):
        p = plane()
        h = ServingHooks(p, 1, HookConfig(plan_every=1, timer_every=100, resident=8),
                         event_factory=Ev)
        launch = h.on_batch_begin(list(range(32)), kv)   # cold estimator: uncertainty 1.0
        assert (launch["workers"] == 8) == expect
        assert (ctrl_u32(p, abi.CTRL_NUM_TASKS_OFF) == 32) == expect
        if expect:
            ref = SchedPlane.region_order(torch.tensor(kv, dtype=torch.float32), 8)
            assert order(p, 32) == ref.tolist()


def test_observe_only_never_orders_or_arms():
    p = plane()
    h = ServingHooks(p, 1, HookConfig(plan_every=1, timer_every=1, resident=2, clc="on",
                                      observe_only=True), event_factory=Ev)
    launch = h.on_batch_begin([0, 1, 2, 3], [16, 4096, 512, 64])
    assert launch["workers"] == 0 and h.order_n is None and h.timer_armed


def test_hints_when_kv_exceeds_l2():
    p = plane()
    h = ServingHooks(p, 2, HookConfig(plan_every=1, timer_every=100, resident=64,
                                      kv_bytes_per_token=4096, l2_bytes=1 << 20),
                     event_factory=Ev)
    h.on_batch_begin([0, 1, 2], [4096, 16, 1024])   # 21 MB > 1 MB
    rows = np.frombuffer(bytes(p._ctrl_host[abi.CTRL_ROWS_OFF:abi.CTRL_ROWS_OFF + 6 * 8]),
                         dtype=np.dtype([("q", "<f4"), ("tau", "<u2"), ("hint", "u1"),
                                         ("pad", "u1")]))
    assert list(rows["hint"]) == [HINT_POLITE] * 2 + [HINT_URGENT] * 2 + [HINT_POLITE] * 2
    assert rows["q"][0] > rows["q"][4] > rows["q"][2]


def test_split_items_spread_cost_by_pages():
    p = plane()
    h = ServingHooks(p, 2, HookConfig(plan_every=1, timer_every=100, resident=2, clc="off",
                                      tile_pages=4), event_factory=Ev)
    launch = h.on_batch_begin([0, 1], [16 * 10, 16])   # 3 + 1 chunks per task
    assert launch["tiles"].shape[0] == 2 * 3 + 2 * 1 and launch["tile_pages"] == 4
    assert h.order_n == 8
    o = order(p, 8)
    assert sorted(o) == list(range(8))


def test_off_cadence_replans_when_the_item_count_changes():
    # a request crossing a tile boundary between re-plans: the armed queue
    # (and the order) are rebuilt for the new item count, not disarmed
    p = plane()
    h = ServingHooks(p, 1, HookConfig(plan_every=4, timer_every=100, resident=2, clc="on",
                                      tile_pages=1), event_factory=Ev)
    first = h.on_batch_begin([0, 1, 2], [32, 32, 32])           # 2 one-page chunks each
    assert first["workers"] == 2 and first["tiles"].shape[0] == 6
    g = p._generation
    same = h.on_batch_begin([0, 1, 2], [32, 32, 32])
    assert same["workers"] == 2 and p._generation == g         # still matches: no writes
    grown = h.on_batch_begin([0, 1, 2], [33, 32, 32])           # 3 chunks for r0
    assert grown["tiles"].shape[0] == 7 and grown["workers"] == 2
    assert ctrl_u32(p, abi.CTRL_NUM_TASKS_OFF) == 7 and h.armed_n == 7
    assert ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 7
    assert sorted(order(p, 7)) == list(range(7))


def test_off_cadence_lpt_order_follows_the_item_count():
    p = plane()
    h = ServingHooks(p, 1, HookConfig(plan_every=8, timer_every=100, resident=2, clc="off",
                                      tile_pages=1), event_factory=Ev)
    h.on_batch_begin([0, 1, 2], [32, 16, 48])                   # 2 + 1 + 3 items
    assert h.order_n == 6 and ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 6
    h.on_batch_begin([0, 1, 2], [32, 17, 48])                   # r1 grows to 2 chunks
    assert h.order_n == 7 and ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 7
    assert sorted(order(p, 7)) == list(range(7))


def test_oversized_batch_raises_and_begin_degrades_to_stock(capsys):
    p = plane(8)
    h = ServingHooks(p, 2, HookConfig(plan_every=1, timer_every=1), event_factory=Ev)
    import pytest
    with pytest.raises(RuntimeError, match="max_tasks"):
        h.on_batch_begin([0, 1, 2, 3, 4], [16] * 5)          # 10 tasks > 8 rows
    launch = h.begin([0, 1, 2, 3, 4], [16] * 5)
    assert launch == ServingHooks.STOCK and h.hook_errors == 1
    h.begin([0, 1, 2, 3, 4], [16] * 5)
    assert h.hook_errors == 2
    out = capsys.readouterr().out
    assert out.count("begin hook error") == 1                 # first per site only
    assert "hook_errors=2" in h.stats()
    assert h.begin([0, 1], [16, 32])["plane"] is p            # recovers on a valid batch


def test_lpt_regime_plans_over_its_own_tile_size():
    p = plane()
    h = ServingHooks(p, 1, HookConfig(plan_every=4, timer_every=100, resident=2, clc="off",
                                      tile_pages=1, lpt_tile_pages=2), event_factory=Ev)
    kv = [64, 16, 48]                                   # 4 + 1 + 3 pages
    launch = h.on_batch_begin([0, 1, 2], kv)            # LPT regime: 2-page tiles
    assert launch["tile_pages"] == 2 and launch["tiles"].shape[0] == 2 + 1 + 2
    assert h.order_n == 5 and ctrl_u32(p, abi.CTRL_ORDER_SIZE_OFF) == 5
    assert sorted(order(p, 5)) == list(range(5))
    off = h.on_batch_begin([0, 1, 2], kv)               # off cadence: same plan size
    assert off["tile_pages"] == 2 and off["tiles"].shape[0] == 5
    grown = h.on_batch_begin([0, 1, 2], [64, 40, 48])   # r1 to 3 pages: re-plan at 2
    assert grown["tile_pages"] == 2 and grown["tiles"].shape[0] == 6 and h.order_n == 6
    # the queue regime keeps the configured tiles
    q = ServingHooks(plane(), 1, HookConfig(plan_every=1, timer_every=100, resident=2,
                                            clc="on", tile_pages=1, lpt_tile_pages=2),
                     event_factory=Ev)
    armed = q.on_batch_begin([0, 1, 2], kv)
    assert armed["workers"] == 2 and armed["tile_pages"] == 1 and armed["tiles"].shape[0] == 8


def test_observing_binds_the_plane_only_on_probe_steps():
    p = plane()
    h = ServingHooks(p, 1, HookConfig(plan_every=2, timer_every=4, observe_only=True),
                     event_factory=Ev)
    planes = []
    for step in range(8):
        launch = h.on_batch_begin([0, 1], [100, 300])
        planes.append(launch["plane"] is p)
        assert launch["workers"] == 0
        h.on_batch_end()
    # probes at steps 0 and 4 (each read back before the next); the rest
    # run without the tables
    assert planes == [True, False, False, False, True, False, False, False]


def test_push_without_changes_publishes_nothing():
    p = plane()
    p.set_num_tasks(5)
    p.push()
    g = p._generation
    p.push()
    p.set_num_tasks(5)                        # the same bytes
    p.push()
    assert p._generation == g
    p.set_row(3, q=1.0)                       # a row written
    p.push()
    assert p._generation == g + 1
    p.set_timer_enabled(False)                # a header change
    p.push()
    assert p._generation == g + 2
    assert ctrl_u32(p, abi.CTRL_NUM_TASKS_OFF) == 5
    assert ctrl_u32(p, abi.CTRL_FLAGS_OFF) & abi.FLAG_TIMER_OFF
    assert struct.unpack_from("<fHBB", bytes(p._ctrl_dev.numpy()),
                              abi.CTRL_ROWS_OFF + 3 * abi.ROW_SIZE)[0] == 1.0


def test_observing_publishes_the_plane_once():
    """Observing binds the plane on probe steps only, with the timer on; the
    plane is published on the first step and not again while the batch keeps
    its shape."""
    p = plane()
    h = ServingHooks(p, 2, HookConfig(observe_only=True, plan_every=4, timer_every=4),
                     event_factory=Ev)
    rids, kv = [10, 11, 12], [100, 900, 300]
    gens, bound = [], []
    for _ in range(13):
        launch = h.on_batch_begin(rids, kv)
        bound.append(launch["plane"] is p)
        assert bound[-1] == h.timer_armed
        h.on_batch_end()
        gens.append(p._generation)
    assert gens == [gens[0]] * len(gens)
    assert sum(bound) >= 2 and h.probes_folded >= 1
    assert ctrl_u32(p, abi.CTRL_FLAGS_OFF) & abi.FLAG_TIMER_OFF == 0


def _run_steps(h, p, rids, kv0, steps, timer_fill=None):
    """Decode-style steps (each request one token longer per step); returns
    per step the launch and the plane's published bytes."""
    got = []
    kv = np.asarray(kv0, np.int64)
    for i in range(steps):
        launch = h.on_batch_begin(rids, kv + i)
        if timer_fill is not None and h.timer_armed:
            n = len(rids)
            p._timer_view()[:n] = torch.as_tensor(timer_fill(kv + i))
        h.on_batch_end()
        got.append((launch["workers"], launch["tile_pages"],
                    None if launch["tiles"] is None else launch["tiles"].tolist(),
                    bytes(p._ctrl_dev.numpy()[:4096]), p._order_view()[:4096].tolist()))
    return got


def _hooks(cfg, fresh):
    p = plane(4096)
    h = ServingHooks(p, 1, cfg, event_factory=Ev)
    if fresh:
        h._plan_ahead = lambda: None          # every re-plan decided at begin
    return p, h


def test_plan_ahead_installs_the_tables_a_fresh_re_plan_would():
    rng = np.random.default_rng(11)
    rids = list(range(48))
    kv0 = rng.integers(16, 3000, 48)
    fill = lambda kv: (kv * 7 + 1000).tolist()        # noqa: E731  measured cost per request
    for cfg in (HookConfig(plan_every=4, timer_every=4, resident=16, tile_pages=8,
                           lpt_tile_pages=12),
                HookConfig(plan_every=4, timer_every=8, resident=16, clc="on", tile_pages=8),
                HookConfig(plan_every=3, timer_every=5, resident=512, tile_pages=8)):
        runs = []
        for fresh in (False, True):
            p, h = _hooks(cfg, fresh)
            where = []                        # "begin" / "end" per decision made
            decide, begin = h._decide, h.on_batch_begin
            inside = [False]

            def spy(*a, _d=decide, _w=where, _i=inside):
                _w.append("begin" if _i[0] else "end")
                return _d(*a)

            def begin_spy(*a, _b=begin, _i=inside):
                _i[0] = True
                try:
                    return _b(*a)
                finally:
                    _i[0] = False
            h._decide, h.on_batch_begin = spy, begin_spy
            runs.append((_run_steps(h, p, rids, kv0, 17, fill), where))
        (ahead, where_ahead), (fresh, where_fresh) = runs
        assert ahead == fresh, cfg
        assert where_fresh.count("begin") > 1 and "end" not in where_fresh
        # ahead: re-plans decided at the previous step's end, except the
        # first step and those whose decision a probe's fold (a new fit)
        # made stale
        assert where_ahead[0] == "begin" and where_ahead.count("end") > 1, where_ahead
        assert where_ahead.count("begin") < where_fresh.count("begin"), where_ahead


def test_plan_ahead_is_dropped_when_the_batch_or_the_fit_differs():
    cfg = HookConfig(plan_every=2, timer_every=100, resident=4, clc="off", tile_pages=4)
    p, h = _hooks(cfg, False)
    rids, kv = [0, 1, 2, 3, 4, 5], np.array([100, 900, 300, 64, 2000, 40])
    h.on_batch_begin(rids, kv)
    h.on_batch_end()
    h.on_batch_begin(rids, kv + 1)            # off cadence
    h.on_batch_end()
    assert h.ahead is not None                # the next step re-plans
    # a batch that is not the predicted one (a request grew by two tokens)
    other = kv + 2
    other[1] += 60
    launch = h.on_batch_begin(rids, other)
    p2, h2 = _hooks(cfg, True)
    h2.on_batch_begin(rids, kv)
    h2.on_batch_end()
    h2.on_batch_begin(rids, kv + 1)
    h2.on_batch_end()
    want = h2.on_batch_begin(rids, other)
    assert launch["tiles"].tolist() == want["tiles"].tolist()
    assert order(p, h.order_n) == order(p2, h2.order_n)
    h.on_batch_end()
    h.on_batch_begin(rids, other + 1)
    h.on_batch_end()
    assert h.ahead is not None
    ver = h.ctl.version
    h.ctl.observe(rids, (other + 2).tolist(), [5000, 1, 1, 1, 1, 1])  # the fit moved
    assert h.ctl.version == ver + 1
    seen = []
    decide = h._decide
    h._decide = lambda *a: seen.append(1) or decide(*a)
    h.on_batch_begin(rids, other + 2)
    assert seen == [1]                        # decided afresh at begin
