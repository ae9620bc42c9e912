"""The pi builders of the plane (reference python/sched_rt.py:557-609),
against hand-derived orders: grouped longest-first and the resident-region
order. Both must be permutations; ties keep ascending index."""
import numpy as np
import torch

from sched_rt import SchedPlane


def L(t):
    return [int(x) for x in t]


def test_grouped_lpt_known_orders():
    # groups of 2: {0,1} = 2, {2,3} = 10, {4} = 2 -> group 1, then 0, then 2
    assert L(SchedPlane._grouped_lpt(torch.tensor([1., 1., 5., 5., 2.]), 2)) == [2, 3, 0, 1, 4]
    # inside a group the index order stays, whatever the costs
    assert L(SchedPlane._grouped_lpt(torch.tensor([1., 9., 0., 0.]), 2)) == [0, 1, 2, 3]
    # block 1 (and a batch of one group) is plain longest-first, ties by index
    c = torch.tensor([3., 7., 3., 9., 7.])
    assert L(SchedPlane._grouped_lpt(c, 1)) == [3, 1, 4, 0, 2]
    assert L(SchedPlane._grouped_lpt(c, 8)) == [3, 1, 4, 0, 2]


def test_region_order_known_orders():
    c = torch.tensor([9., 1., 8., 2., 7., 3., 6., 4., 5.])
    # R = 4: heaviest two (0, 2) on even slots, lightest two lightest-first
    # (1, 3) on odd slots, then the rest heaviest first
    assert L(SchedPlane.region_order(c, 4)) == [0, 1, 2, 3, 4, 6, 8, 7, 5]
    # R = 3: two heavy, one light
    assert L(SchedPlane.region_order(c, 3)) == [0, 1, 2, 4, 6, 8, 7, 5, 3]
    # n <= R: grouped longest-first (one group of 16 -> plain longest-first)
    assert L(SchedPlane.region_order(c, 9)) == [0, 2, 4, 6, 8, 7, 5, 3, 1]
    assert L(SchedPlane.region_order(c, 0)) == [0, 2, 4, 6, 8, 7, 5, 3, 1]


def test_builders_are_permutations():
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.integers(1, 200))
        c = torch.tensor(rng.integers(0, 5, n).astype(np.float32))
        for o in (SchedPlane._grouped_lpt(c, int(rng.integers(0, 20))),
                  SchedPlane.region_order(c, int(rng.integers(0, 250)))):
            assert o.dtype == torch.int32
            assert sorted(L(o)) == list(range(n))


def test_desc_order_is_the_stable_descending_sort():
    """The packed-key sort against numpy's stable sort of -cost, on what the
    builders see (float32 costs, page counts with many ties) and the cases
    the packing must get right: signed zeros tie, infinities order, and
    inputs that float32 cannot hold exactly (or NaN) take the plain sort."""
    import sched_pd
    rng = np.random.default_rng(1)
    cases = [rng.random(3352).astype(np.float32), rng.integers(0, 129, 3352).astype(np.float64),
             np.array([]), np.array([5.0]), np.array([0.0, -0.0, 0.0, -0.0, 1.0, -1.0]),
             np.array([np.inf, -np.inf, 3.0, np.inf, -1.0, -np.inf]), rng.random(100),
             np.array([1.0, np.nan, 2.0, np.nan]), rng.standard_normal(5000).astype(np.float32),
             np.array([1e-45, 0.0, -1e-45, 3.4e38, -3.4e38], np.float32)]
    for c in cases:
        got = sched_pd.desc_order(c)
        assert got.dtype == np.int64
        assert np.array_equal(got, np.argsort(-np.asarray(c, np.float64), kind="stable")), c


def test_plan_tiles_host_reuses_the_last_plan_safely():
    import sched_pd
    lens = np.array([1, 300, 2047, 2048, 2049, 5000])
    a = sched_pd.plan_tiles_host(lens, 16, 128, 2)
    a[:] = -1                                       # a copy: the cache is untouched
    b = sched_pd.plan_tiles_host(lens + 1, 16, 128, 2)   # same chunk counts
    per_req = [1, 1, 1, 2, 2, 3]                    # chunks of 128 pages after +1 token
    assert b.shape == (2 * sum(per_req), 2)
    assert b[:, 0].tolist() == [t for t in range(12) for _ in range(per_req[t // 2])]
    c = sched_pd.plan_tiles_host(lens + 100, 16, 128, 2)  # request 2 crosses a boundary
    assert c.shape[0] == b.shape[0] + 2
    d = sched_pd.plan_tiles_host(lens + 100, 16, 64, 2)   # other tile size: rebuilt
    assert d.shape[0] > c.shape[0]
    e = sched_pd.plan_tiles_host(lens + 100, 16, 128, 1)  # other head count: rebuilt
    assert e.shape[0] == c.shape[0] // 2
