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
