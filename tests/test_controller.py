"""The closed-loop controller (CPU): the reference's own smoke checks
(python/sched_controller.py:180-215), known-answer fits, every policy, the
dead-band, and the fold from per-task timer rows to per-request cost."""
import random

import numpy as np
import pytest

from sched_controller import (CostModel, SchedControlPlane, task_costs_per_request,
                              task_order_from_requests)


class FakePlane:
    def __init__(self):
        self.o, self.n, self.pushes = None, None, 0

    def set_order(self, o):
        self.o = list(o)

    def set_num_tasks(self, n):
        self.n = n

    def push(self):
        self.pushes += 1


def test_reference_smoke():
    random.seed(0)
    ctl = SchedControlPlane(policy="lpt")
    plane = FakePlane()
    alpha_true, beta_true = 7.5, 120.0
    rids = list(range(64))
    lens = [random.choice([64, 512]) for _ in rids]
    for _ in range(20):
        cyc = [alpha_true * ln + beta_true + random.gauss(0, 5) for ln in lens]
        ctl.step(plane, rids, lens, cycles=cyc)
    a, b = ctl.coefficients()
    assert abs(a - alpha_true) / alpha_true < 0.05
    oracle = sorted(range(len(lens)), key=lambda i: -lens[i])
    got = ctl.order(rids, lens)
    assert [lens[i] for i in got] == [lens[i] for i in oracle]
    before = ctl.order(rids, lens)
    lens2 = list(lens)
    lens2[0] += 1
    assert ctl.order(rids, lens2) == before
    assert plane.n == 64 and plane.pushes == 20 and sorted(plane.o) == rids


def test_fit_known_answers():
    f = CostModel()
    assert f.coefficients() == (1.0, 0.0)
    f.add([2.0], [10.0])
    assert f.coefficients() == (5.0, 0.0)     # one point: proportional
    f.add([2.0], [14.0])
    assert f.coefficients() == (6.0, 0.0)     # all x equal: proportional
    g = CostModel()
    for x in (1.0, 2.0, 3.0, 10.0):
        g.add([x], [3.0 * x + 4.0])
    a, b = g.coefficients()
    assert abs(a - 3.0) < 1e-12 and abs(b - 4.0) < 1e-12
    # a whole step at once gives the same fit as one sample at a time
    h = CostModel()
    h.add([1.0, 2.0, 3.0, 10.0], [7.0, 10.0, 13.0, 34.0])
    assert np.allclose(h.coefficients(), (3.0, 4.0), rtol=0, atol=1e-12)
    # least squares on noisy data: numpy's lstsq on the same samples
    rng = np.random.default_rng(0)
    x = rng.uniform(16, 32768, 500)
    y = 7.5 * x + 120 + rng.normal(0, 50, 500)
    m = CostModel()
    m.add(x, y)
    want = np.linalg.lstsq(np.stack([x, np.ones_like(x)], 1), y, rcond=None)[0]
    assert np.allclose(m.coefficients(), want, rtol=1e-9)


def test_forgetting_tracks_a_drifting_cost():
    # cost per token doubles half way: the forgetting fit follows, the plain
    # least-squares fit averages the two regimes
    plain, fading = CostModel(), CostModel(forget=0.5)
    x = np.array([100.0, 1000.0, 5000.0])
    for step in range(40):
        slope = 2.0 if step < 20 else 4.0
        for m in (plain, fading):
            m.add(x, slope * x + 10.0)
    assert abs(fading.coefficients()[0] - 4.0) < 1e-4   # old regime weighs 0.5**20
    assert 2.5 < plain.coefficients()[0] < 3.5
    with pytest.raises(ValueError):
        CostModel(forget=0.0)


def test_step_estimate_does_not_depend_on_listing_order():
    rng = np.random.default_rng(1)
    rids = list(range(32))
    lens = rng.integers(16, 4096, 32)
    cyc = 3.0 * lens + 50 + rng.normal(0, 20, 32)
    a, b = SchedControlPlane(), SchedControlPlane()
    a.observe(rids, lens, cyc)
    perm = rng.permutation(32)
    b.observe([rids[i] for i in perm], lens[perm], cyc[perm])
    assert np.allclose(a.predict(rids, lens), b.predict(rids, lens), rtol=1e-12)


def test_policies_and_errors():
    ctl = SchedControlPlane(policy="srpt", deadband=0.0)
    for _ in range(3):
        ctl.observe([0, 1, 2], [100, 10, 50], [1000, 100, 500])
    assert ctl.order([0, 1, 2], [100, 10, 50]) == [1, 2, 0]
    ctl.policy = "lpt"
    ctl.clear_published()
    assert ctl.order([0, 1, 2], [100, 10, 50]) == [0, 2, 1]
    ctl.policy = "edf"
    ctl.clear_published()
    # slack = deadline - elapsed - t_hat
    assert ctl.order([0, 1, 2], [100, 10, 50], deadlines=[5000, 150, 1000],
                     elapsed=[0, 0, 0]) == [1, 2, 0]
    with pytest.raises(ValueError):
        SchedControlPlane(policy="edf").order([0], [1])
    with pytest.raises(ValueError):
        SchedControlPlane(policy="fifo").order([0], [1])


def test_deadband_srpt_republishes_only_real_gains():
    ctl = SchedControlPlane(policy="srpt", deadband=0.05)
    for _ in range(3):
        ctl.observe([0, 1], [10, 20], [10, 20])
    first = ctl.order([0, 1], [10, 20])
    assert first == [0, 1]
    # a real reversal of the costs is a large gain: republished
    assert ctl.order([0, 1], [30, 5]) == [1, 0]
    # a negligible change keeps the published order
    assert ctl.order([0, 1], [29, 6]) == [1, 0]


def test_lpt_deadband_keeps_the_first_published_order():
    # the reference's gain is old minus new total completion time; LPT
    # maximises it, so a changed LPT ranking is never republished
    ctl = SchedControlPlane(policy="lpt")
    for _ in range(3):
        ctl.observe([0, 1], [10, 20], [10, 20])
    assert ctl.order([0, 1], [10, 20]) == [1, 0]
    assert ctl.order([0, 1], [30, 5]) == [1, 0]


def test_uncertainty_and_gamma():
    ctl = SchedControlPlane()
    assert ctl.uncertainty([], []) == 1.0
    ctl.observe([0, 1], [10, 20], [10.0, 20.0])
    u = ctl.uncertainty([0, 1, 7], [10, 20, 30])
    assert u > 0  # request 7 was never observed: its whole prediction is doubt
    ctl.observe_step(100.0, 150.0)
    assert abs(ctl.gamma - (0.75 + 0.25 * 1.5)) < 1e-12
    ctl.observe_step(0.0, 5.0)  # ignored
    assert abs(ctl.gamma - 1.125) < 1e-12
    assert ctl.predict_one(-1e9) == 0.0


def test_fold_and_expand():
    rows = [1, 2, 3, 4, 5, 6]
    assert task_costs_per_request(rows, 3, 2) == [3.0, 7.0, 11.0]
    assert task_order_from_requests([2, 0], 2) == [4, 5, 0, 1]


def test_request_plane_expands_to_tasks():
    from sched_controller import RequestPlane
    inner = FakePlane()
    ctl = SchedControlPlane(policy="lpt")
    ctl.step(RequestPlane(inner, 4), [10, 11, 12], [5, 50, 20], cycles=[5, 50, 20])
    assert inner.o == [4, 5, 6, 7, 8, 9, 10, 11, 0, 1, 2, 3]
    assert inner.n == 12 and inner.pushes == 1
