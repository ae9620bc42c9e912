"""A SchedPlane driving the reference's launcher: the plane's tables bound
into the library's __sched_* slots (SchedPlane.bind_launcher), then
launch_paged_softmax called as reference test/py/test_dynamic_loop.py:145-190
calls its woven build, step for step, on that fixture's own inputs."""
import ctypes

import numpy as np
import pytest
import torch

from sched_rt import SchedPlane
from test_gpu_runtime import SD, Fixture, close, fixture_dynamic_loop

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(schedlib):
    torch.cuda.init()
    yield schedlib
    schedlib.sched_rt_disarm()


def slots(lib):
    s = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slots(s)
    return list(s)


def test_dynamic_loop_through_bound_plane(lib):
    f = Fixture(fixture_dynamic_loop)
    nseq = f.nseq
    # stock: nothing in the slots
    lib.sched_rt_disarm()
    golden = f.launch(lib)
    assert close(golden.cpu(), f.reference()), "stock kernel vs the CPU reference"

    plane = SchedPlane(max_tasks=nseq, device="cuda")
    plane.bind_launcher()
    t = plane.tables()
    assert slots(lib) == [t["order"], t["ctrl"], t["timer"], t["queue"]]
    assert plane.bound

    # neutral tables: bit-exact, one timer row per request
    plane.set_num_tasks(nseq)
    plane.push()
    plane.clear_timer()
    assert torch.equal(f.launch(lib), golden), "bound plane, neutral tables == stock"
    cyc = plane.read_timer()
    assert int((cyc > 0).sum()) == nseq, "one timer row per request"

    # the timer sees the straggler
    longs = [r for r in range(nseq) if r % 8 == 0]
    shorts = [r for r in range(nseq) if r % 8]
    long_c, short_c = cyc[longs].double().mean(), cyc[shorts].double().mean()
    assert long_c > 2 * short_c, f"long {long_c:.0f} vs short {short_c:.0f} cycles"

    # pi reprogrammed from the plane: reversed, then LPT from the cycles
    plane.set_order(torch.arange(nseq - 1, -1, -1))
    assert torch.equal(f.launch(lib), golden), "reversed pi bit-exact"
    order = torch.argsort(cyc, descending=True).to(torch.int32)
    plane.set_order(order)
    assert torch.equal(f.launch(lib), golden), "LPT pi from measured cycles bit-exact"

    # shed: tau 8 on every row = the truncated reference (first 8 tokens of
    # every page, the woven loop's counter)
    plane.reset_order()
    plane.set_rows(tau=[8] * nseq, n=nseq)
    plane.push()
    shed = f.launch(lib)
    assert not torch.equal(shed, golden) and torch.isfinite(shed).all()
    assert close(shed.cpu(), f.reference(tau=8)), "shed vs the truncated reference"
    plane.set_rows(tau=[0] * nseq, n=nseq)
    plane.push()
    assert torch.equal(f.launch(lib), golden)

    # the timer gate from the plane's flags
    plane.set_timer_enabled(False)
    plane.push()
    plane.clear_timer()
    assert torch.equal(f.launch(lib), golden)
    assert int((plane.read_timer() > 0).sum()) == 0
    plane.set_timer_enabled(True)
    plane.push()

    # unbind: stock again, slots null
    plane.unbind_launcher()
    assert not plane.bound and not any(slots(lib))
    assert torch.equal(f.launch(lib), golden)


def test_bound_rows_bound_the_levers(lib):
    """Task ids at or past the plane's max_tasks get no levers: a 32-row plane
    over the 64-request fixture times requests 0..31 only, and its reversed
    pi entries for workgroups 0..31 are taken only where they name a task
    below the grid size (all of them here); outputs stay bit-exact."""
    f = Fixture(fixture_dynamic_loop)
    lib.sched_rt_disarm()
    golden = f.launch(lib)
    plane = SchedPlane(max_tasks=32, device="cuda")
    plane.bind_launcher()
    plane.clear_timer()
    plane.set_order(torch.arange(31, -1, -1))
    assert torch.equal(f.launch(lib), golden)
    rows = plane.read_timer()
    assert int((rows > 0).sum()) == 32
    plane.unbind_launcher()


def test_moved_tables_rebind(lib):
    """use_device_timer / use_device_order move a table out of the arena; a
    bound plane re-binds, and the launches write the moved rows."""
    f = Fixture(fixture_dynamic_loop)
    lib.sched_rt_disarm()
    golden = f.launch(lib)
    plane = SchedPlane(max_tasks=f.nseq, device="cuda")
    plane.bind_launcher()
    plane.use_device_timer()
    plane.use_device_order()
    t = plane.tables()
    assert slots(lib) == [t["order"], t["ctrl"], t["timer"], t["queue"]]
    plane.clear_timer()
    plane.set_order(torch.arange(f.nseq - 1, -1, -1))
    assert torch.equal(f.launch(lib), golden)
    assert int((plane.read_timer() > 0).sum()) == f.nseq
    plane.unbind_launcher()


def test_runtime_init_takes_the_slots_back(lib):
    """sched_rt_init after a bind puts the runtime's own tables back (and the
    plane reports itself unbound); disarm nulls them."""
    f = Fixture(fixture_dynamic_loop)
    plane = SchedPlane(max_tasks=f.nseq, device="cuda")
    plane.bind_launcher()
    assert lib.sched_rt_init()
    assert not plane.bound
    own = slots(lib)
    assert all(own) and own[0] != plane.tables()["order"]
    golden = f.launch(lib)
    assert lib.sched_rt_disarm()
    assert torch.equal(f.launch(lib), golden)


def test_eight_thousand_tasks_through_the_launcher(lib):
    """8192 requests (twice the C runtime's 4096 rows) through
    launch_paged_softmax with a bound 8192-row plane: every request gets a
    timer row, and LPT from them is bit-exact against identity."""
    nseq, pt, nl, ns = 8192, 32, 24, 3
    g = torch.Generator().manual_seed(0)
    is_long = torch.rand(nseq, generator=g) < 0.1
    nbl = torch.where(is_long, nl, ns).to(torch.int32)
    starts = torch.cumsum(nbl, 0) - nbl
    bt = torch.zeros(nseq, nl, dtype=torch.int32)
    for r in range(nseq):
        bt[r, :nbl[r]] = torch.arange(int(starts[r]), int(starts[r]) + int(nbl[r]))
    npages = int(nbl.sum())
    kv = torch.randn(npages * pt * 2 * SD + 4096, device="cuda")
    q = torch.randn(nseq, SD, device="cuda")
    out = torch.zeros(nseq, SD, device="cuda")
    btd, nbld = bt.cuda(), nbl.cuda()

    def run():
        lib.launch_paged_softmax(kv.data_ptr(), btd.data_ptr(), nbld.data_ptr(), q.data_ptr(),
                                 out.data_ptr(), nseq, nl, pt,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return out.clone()

    lib.sched_rt_disarm()
    golden = run()
    plane = SchedPlane(max_tasks=nseq, device="cuda")
    plane.bind_launcher()
    plane.clear_timer()
    assert torch.equal(run(), golden)
    cyc = plane.read_timer()
    assert int((cyc > 0).sum()) == nseq
    order = np.argsort(-cyc.numpy(), kind="stable").astype(np.int32)
    # the rows rank long requests above short ones: a long request's row
    # exceeds a short one's with probability near 1 (rank-sum statistic).
    # A row is the task's wall time, so a short task's includes the
    # contention of the long ones beside it and the top-|long| rows are not
    # exactly the long requests (0.85-0.9 of them; 0.985-0.995 here).
    c, lg = cyc.numpy().astype(np.float64), is_long.numpy()
    ranks = c.argsort(kind="stable").argsort() + 1.0
    nlong, nshort = int(lg.sum()), int((~lg).sum())
    assert (ranks[lg].sum() - nlong * (nlong + 1) / 2) / (nlong * nshort) > 0.95
    plane.install_order(order, nseq)
    plane.push()
    assert torch.equal(run(), golden)
    plane.unbind_launcher()
