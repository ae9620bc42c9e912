"""The closed loop on the GPU: timer rows from a work-queue decode feed the
controller, whose order goes back to the plane for the next launch. Every
launch must give the same bits, and the fitted cost model must rank the
longest requests first."""
import numpy as np
import pytest
import torch

import sched_pd
import workloads
from sched_controller import RequestPlane, SchedControlPlane, task_costs_per_request
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def test_timer_to_controller_to_plane_loop():
    rng = np.random.default_rng(5)
    R, hkv = 32, 8
    ctx = rng.integers(16, 4096, R)
    ctx[3] = 12000                      # one straggler
    b = workloads.make_batch(ctx, num_q_heads=32, num_kv_heads=hkv, head_dim=128,
                             kv_dtype=torch.bfloat16, q_dtype=torch.bfloat16, seed=5,
                             device="cuda")
    n = R * hkv
    plane = SchedPlane(max_tasks=n)
    ctl = SchedControlPlane(policy="lpt")
    view = RequestPlane(plane, hkv)
    W = 64
    plane.set_num_tasks(n)
    plane.push()
    plane.reset_queue(W)
    base = None
    rids = list(range(R))
    for step in range(4):
        plane.clear_timer()
        out = torch.empty(R, 32, 128, dtype=torch.float32, device="cuda")
        sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                              out=out, plane=plane, workers=W)
        torch.cuda.synchronize()
        if base is None:
            base = out.clone()
        assert torch.equal(out, base), f"step {step}"
        rows = plane.read_timer()[:n].cpu().numpy()
        assert (rows > 0).all()
        cost = task_costs_per_request(rows, R, hkv)
        order = ctl.step(view, rids, ctx.tolist(), cycles=cost)
    alpha, _ = ctl.coefficients()
    assert alpha > 0
    assert order[0] == 3                 # the straggler goes first
    top = set(order[:R // 4])
    longest = set(np.argsort(-ctx)[:R // 4].tolist())
    assert len(top & longest) >= R // 4 - 2
