"""Split-KV work items in ranged rows (task, chunk | nchunks << 16, p0, p1):
chunk sizes that differ within a launch and within a task. A ranged plan
with the pair plan's ranges gives the pair plan's bits; a tail plan (small
chunks at the end of the claim order) matches the oracle and is bitwise the
same under every pi and ticket-queue schedule; ranges past a shorter context
add nothing; a plan that does not reach the context flags its tasks stale
and leaves every arrival counter zero."""
import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
import sched_pd
import workloads
from parity import TOL_BF16, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu

CTX = [1, 16, 17, 300, 2048, 5000, 0, 777, 4100]


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def batch(ctx, kv=torch.bfloat16, hq=32, hkv=8, seed=0, v_layout="dmajor"):
    b = workloads.make_batch(np.asarray(ctx), num_q_heads=hq, num_kv_heads=hkv, head_dim=128,
                             kv_dtype=kv, q_dtype=torch.bfloat16, seed=seed, device="cuda")
    if v_layout == "tokmajor":           # V as [pages, Hkv, page, d], same values
        b["v_pool"] = b["v_pool"].permute(0, 1, 3, 2).contiguous()
    return b


def run(b, mode=abi.SOFTMAX, **kw):
    torch.cuda.synchronize()
    rows = b["q"].shape[1] if mode == abi.SOFTMAX else b["v_pool"].shape[1]
    out = torch.full((b["ctx_lens"].numel(), rows, 128), float("nan"), device="cuda")
    sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                          out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], mode=mode, **kw)
    torch.cuda.synchronize()
    return out


def ref(b, plane=None, **kw):
    ctrl = bytes(plane._ctrl_host) if plane is not None else None
    return oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                         k_scale=b["k_scale"], v_scale=b["v_scale"], ctrl=ctrl,
                         max_tasks=plane.N if plane is not None else 4096, **kw)


def same(a, b):
    return bool(torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0))) and \
        bool(torch.equal(torch.isnan(a), torch.isnan(b)))


def check(out, r):
    got = out.cpu().numpy()
    fin = np.isfinite(r)
    assert np.array_equal(np.isnan(got), ~fin)        # the empty request is 0/0
    e = par_err(got[fin], r[fin])
    assert e <= TOL_BF16, e
    return e


@pytest.mark.parametrize("kvt,layout,flags", [
    (torch.bfloat16, "dmajor", 0), (torch.bfloat16, "tokmajor", 0),
    (torch.float8_e4m3fn, "dmajor", 0), (torch.bfloat16, "dmajor", abi.FLAG_FORCE_VALU)])
def test_ranged_rows_with_pair_ranges_give_the_pair_bits(kvt, layout, flags):
    b = batch(CTX, kv=kvt, seed=3, v_layout=layout)
    tp = 16
    pairs = sched_pd.plan_tiles_host(CTX, 16, tp, 8)
    ranged = sched_pd.plan_ranges_host(CTX, 16, 8, tile_pages=tp, tail_frac=0.0)
    o_pair = run(b, tiles=pairs, tile_pages=tp, flags=flags, v_layout=layout)
    o_rng = run(b, tiles=ranged, flags=flags, v_layout=layout)
    assert same(o_pair, o_rng)
    check(o_rng, ref(b, v_layout=layout))


@pytest.mark.parametrize("kvt", [torch.bfloat16, torch.float8_e4m3fn])
def test_tail_plan_parity_and_schedule_invariance(kvt):
    b = batch(CTX, kv=kvt, seed=5)
    ntask = len(CTX) * 8
    rng = np.random.default_rng(7)
    urgency = rng.uniform(0, 1, ntask)
    order = np.argsort(-urgency, kind="stable")
    tiles = sched_pd.plan_ranges_host(CTX, 16, 8, task_order=order, tile_pages=32,
                                      tail_pages=5, tail_frac=0.4)
    sizes = tiles[:, 3] - tiles[:, 2]
    assert sizes.max() == 32 and ((sizes > 0) & (sizes < 32)).any()  # both sizes in the plan
    n = tiles.shape[0]
    out = run(b, tiles=tiles)
    print(f"tail plan {kvt}: {n} items, err {check(out, ref(b)):.3g}")
    plane = SchedPlane(max_tasks=max(n, ntask))
    pi = sched_pd.tile_order_by_task_key(torch.from_numpy(tiles), urgency)
    plane.install_order(pi, n)
    plane.set_num_tasks(n)
    plane.push()
    assert same(run(b, plane=plane, tiles=tiles), out)
    for W in (7, 300, n + 5):
        plane.reset_queue(W)
        plane.clear_timer()
        assert same(run(b, plane=plane, tiles=tiles, workers=W), out)
        assert (plane.read_timer()[:ntask].numpy() > 0).all()
    ws = sched_pd.workspace_for(0, "cuda")
    assert int(ws[:sched_pd.WS_COUNTERS_OFF + 4 * ntask].view(torch.int32).abs().sum()) == 0


def test_ranges_past_a_shorter_context_add_nothing():
    """A plan for longer contexts: request 1's last chunks lie past its
    context (they read nothing and merge empty partials); the result is the
    oracle's, and no task is stale."""
    old_ctx, new_ctx = [100, 3000, 1000], [100, 700, 1000]
    b = batch(new_ctx, seed=11)
    plan = sched_pd.plan_ranges_host(old_ctx, 16, 8, tile_pages=16, tail_pages=4,
                                     tail_frac=0.5)
    ws = sched_pd.workspace_for(0, "cuda")
    sched_pd.stale_plan_count(ws, reset=True)
    for flags in (0, abi.FLAG_FORCE_VALU):
        check(run(b, tiles=plan, flags=flags), ref(b))
    assert sched_pd.stale_plan_count(ws) == 0


@pytest.mark.parametrize("flags,workers", [(0, 0), (abi.FLAG_FORCE_VALU, 0), (0, 37)])
def test_stale_ranged_plan_is_flagged_and_leaves_counters_clean(flags, workers):
    """Request 1 grew past its last range (a multi-chunk task), request 2 past
    its single chunk: both are stale (NaN rows, counted, counters untouched);
    request 0 is right. A fresh plan on the same workspace is right
    everywhere."""
    old_ctx, new_ctx = [100, 3000, 200], [100, 3100, 260]
    b = batch(new_ctx, seed=13)
    hkv = 8
    stale = sched_pd.plan_ranges_host(old_ctx, 16, hkv, tile_pages=64, tail_pages=16,
                                      tail_frac=0.3)
    assert (stale[stale[:, 0] == 16, 1] >> 16 == 1).all()          # request 2: one chunk
    fresh = sched_pd.plan_ranges_host(new_ctx, 16, hkv, tile_pages=64, tail_pages=16,
                                      tail_frac=0.3)
    n = max(stale.shape[0], fresh.shape[0])
    plane = SchedPlane(max_tasks=n)
    r = ref(b)
    ws = sched_pd.workspace_for(0, "cuda")
    sched_pd.stale_plan_count(ws, reset=True)
    for plan in (stale, fresh):
        plane.set_num_tasks(plan.shape[0] if workers else 0)
        plane.push()
        if workers:
            plane.reset_queue(workers)
        got = run(b, plane=plane, tiles=plan, flags=flags, workers=workers).cpu().numpy()
        if plan is stale:
            assert np.isnan(got[1:]).all()
            assert par_err(got[0], r[0]) <= TOL_BF16
            assert sched_pd.stale_plan_count(ws, reset=True) == 2 * hkv
        else:
            assert par_err(got, r) <= TOL_BF16
            assert sched_pd.stale_plan_count(ws) == 0
        counters = ws[sched_pd.WS_COUNTERS_OFF:sched_pd.WS_COUNTERS_OFF + 4 * len(new_ctx) * hkv]
        assert int(counters.view(torch.int32).abs().sum()) == 0


def test_ranged_rows_with_shed_and_linear():
    ctx = [40, 3000, 1000, 4096]
    b = batch(ctx, seed=17)
    ntask = len(ctx) * 8
    tiles = sched_pd.plan_ranges_host(ctx, 16, 8, task_order=np.arange(ntask)[::-1],
                                      tile_pages=32, tail_pages=7, tail_frac=0.5)
    plane = SchedPlane(max_tasks=max(tiles.shape[0], ntask))
    tau = np.random.default_rng(19).integers(0, 3000, size=ntask)
    plane.set_rows(tau=tau, n=ntask)
    plane.push()
    for flags in (0, abi.FLAG_FORCE_VALU):
        o = run(b, plane=plane, tiles=tiles, flags=flags)
        assert par_err(o.cpu(), ref(b, plane)) <= TOL_BF16
    w = torch.randn(4096, device="cuda")
    o = run(b, plane=plane, tiles=tiles, mode=abi.LINEAR, lin_w=w)
    assert par_err(o.cpu(), ref(b, plane, mode=abi.LINEAR, lin_w=w.cpu().numpy())) <= TOL_BF16


def test_malformed_host_plan_is_refused_before_launch():
    b = batch([300, 40], seed=23)
    plan = sched_pd.plan_ranges_host([300, 40], 16, 8, tile_pages=4, tail_frac=0.0)
    plan[1, 2] += 1                                                  # gap in task 0's ranges
    with pytest.raises(ValueError):
        run(b, tiles=plan)


def test_host_plan_on_a_side_stream():
    """paged_decode(stream=side) with a host plan: the plan's upload, the
    workspace and the launch all go to the side stream, so the result equals
    the current stream's while that stream is kept busy."""
    b = batch(CTX, seed=29)
    tiles = sched_pd.plan_ranges_host(CTX, 16, 8, tile_pages=24, tail_pages=5, tail_frac=0.5)
    want = run(b, tiles=tiles)
    side = torch.cuda.Stream()
    busy = torch.randn(2048, 2048, device="cuda")
    for _ in range(3):
        out = torch.full_like(want, float("nan"))
        side.wait_stream(torch.cuda.current_stream())
        for _ in range(3):
            busy = busy @ busy / 64.0
        sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                              out=out, tiles=tiles, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert same(out, want)
