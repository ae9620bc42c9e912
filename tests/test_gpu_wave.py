"""The one-wave-per-item kernel (1..3 q-heads per kv-head, token-major rows)
against the oracle, and its levers bitwise: pi, the ticket queue (W above and
below the task count), the timer rows, both shed scopes with skip and load +
mask, windows of 64 pages, page sizes that are not powers of two, the
reference fixture's [token][K|V] pages, split-KV work items (pair and graded
plans, stale plans), and the general VALU and MFMA kernels on the same
inputs."""
import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
import sched_pd
import workloads
from parity import TOL_BF16, TOL_F32, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu

CTX = [1, 15, 16, 17, 33, 100, 511, 1025, 5000, 0]


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def batch(kv, d, ps, heads=4, ctx=CTX, seed=0, q_dtype=torch.float32):
    # fp32 Q: the MFMA kernel (which takes 16-bit Q with d 128) does not apply
    b = workloads.make_batch(np.asarray(ctx), num_q_heads=heads, num_kv_heads=heads,
                             head_dim=d, page_size=ps, kv_dtype=kv, q_dtype=q_dtype, seed=seed,
                             device="cuda")
    b["v_pool"] = b["v_pool"].permute(0, 1, 3, 2).contiguous()   # token-major V
    return b


def run(b, plane=None, flags=0, default=False, **kw):
    # the MFMA kernel is kept out unless `default`, so the one-wave kernel
    # runs wherever it applies (the MFMA kernel takes 16-bit d-128 caches on
    # power-of-two pages by default)
    R, H, d = b["q"].shape
    out = torch.full((R, H, d), float("nan"), device="cuda")
    args = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                               out=out, v_layout="tokmajor", plane=plane,
                               flags=flags | (0 if default else abi.FLAG_NO_MFMA), **kw)
    sched_pd.launch(args)
    torch.cuda.synchronize()
    return out, sched_pd.kernel_kind(args)


def ref(b, plane=None, **kw):
    ctrl = bytes(plane._ctrl_host) if plane is not None else None
    return oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                         v_layout="tokmajor", ctrl=ctrl,
                         max_tasks=plane.N if plane is not None else 4096, **kw)


def same(a, b):
    return bool(torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0))) and \
        bool(torch.equal(torch.isnan(a), torch.isnan(b)))


@pytest.mark.parametrize("kv,d", [(torch.float32, 32), (torch.float32, 64), (torch.float32, 128),
                                  (torch.bfloat16, 64), (torch.bfloat16, 128),
                                  (torch.float16, 64), (torch.float16, 128)])
@pytest.mark.parametrize("ps", [16, 32, 48])
def test_wave_kernel_parity_and_levers(kv, d, ps):
    b = batch(kv, d, ps, seed=d + ps)
    tol = TOL_F32 if kv == torch.float32 else TOL_BF16
    out, kind = run(b)
    assert kind == "wave"
    r = ref(b)
    assert par_err(out.cpu(), r, f"wave {kv} d{d} p{ps}") <= tol
    assert torch.isnan(out[-1]).all()          # an empty context gives the reference's 0/0
    gen, _ = run(b, flags=abi.FLAG_NO_WAVE)
    assert par_err(gen.cpu(), r) <= tol
    n = len(CTX) * 4
    plane = SchedPlane(max_tasks=n)
    plane.set_order(torch.arange(n - 1, -1, -1, dtype=torch.int32))
    plane.push()
    plane.clear_timer()
    o, _ = run(b, plane=plane)
    assert same(o, out)
    rows = plane.read_timer()[:n].numpy()
    assert (rows > 0).all()
    for W in (5, 2 * sched_pd.cu_count(), n + 3):
        plane.set_num_tasks(n)
        plane.push()
        o, _ = run(b, plane=plane, workers=W)
        assert same(o, out), W


@pytest.mark.parametrize("scope", [abi.TAU_PREFIX, abi.TAU_PER_PAGE])
@pytest.mark.parametrize("ps", [16, 32])
def test_wave_kernel_shed(scope, ps):
    b = batch(torch.float32, 64, ps, seed=3)
    n = len(CTX) * 4
    rng = np.random.default_rng(ps)
    plane = SchedPlane(max_tasks=n)
    ctx = np.repeat(np.asarray(CTX), 4)
    tau = (rng.integers(1, np.maximum(ctx, 1) + 1) if scope == abi.TAU_PREFIX
           else rng.integers(1, ps + 1, n))
    tau[::5] = 0
    plane.set_rows(tau=tau, n=n)
    plane.push()
    out, kind = run(b, plane=plane, tau_scope=scope)
    assert kind == "wave"
    assert par_err(out.cpu(), ref(b, plane, tau_scope=scope), f"shed {scope}") <= TOL_F32
    o, _ = run(b, plane=plane, tau_scope=scope, flags=abi.FLAG_SHED_LOADS)
    assert same(o, out)


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float16])
def test_wave_kernel_16bit_q_at_d64(kv):
    b = batch(kv, 64, 16, seed=11, q_dtype=kv)
    out, kind = run(b)
    assert kind == "wave"
    assert par_err(out.cpu(), ref(b), f"wave {kv} q d64") <= TOL_BF16


def test_wave_kernel_on_the_fixture_layout():
    """The reference JIT kernel's layout: fp32 d 32, [token][K|V] pages of 32
    tokens, one head, ctx counted in pages; pages packed per request."""
    SD, PT = 32, 32
    rng = np.random.default_rng(9)
    nbl = rng.integers(1, 30, 300).astype(np.int32)
    npages = int(nbl.sum())
    bt = np.zeros((nbl.size, int(nbl.max())), np.int32)
    at = 0
    perm = rng.permutation(npages).astype(np.int32)
    for r, k in enumerate(nbl):
        bt[r, :k] = perm[at:at + k]
        at += k
    kv = torch.randn(npages, 1, PT, 2 * SD, device="cuda")
    q = torch.randn(nbl.size, 1, SD, device="cuda")
    out = torch.zeros(nbl.size, 1, SD, device="cuda")
    bt_t, nbl_t = torch.from_numpy(bt).cuda(), torch.from_numpy(nbl).cuda()
    args = sched_pd.build_args(q, kv[..., :SD], kv[..., SD:], bt_t, nbl_t, out=out,
                               v_layout="tokmajor", sm_scale=0.125,
                               tau_scope=abi.TAU_PER_PAGE, flags=abi.FLAG_CTX_IN_PAGES)
    assert sched_pd.kernel_kind(args) == "wave"
    sched_pd.launch(args)
    torch.cuda.synchronize()
    r = oracle.decode(q, kv[..., :SD], kv[..., SD:], bt_t, nbl_t, v_layout="tokmajor",
                      sm_scale=0.125, tau_scope=abi.TAU_PER_PAGE, ctx_in_pages=True)
    assert par_err(out.cpu(), r, "fixture layout") <= TOL_F32


def test_wave_static_positions_over_several_rounds():
    """A static launch larger than the resident workgroups: positions run
    wave-major within each round of resident workgroups (so consecutive pi
    entries land in different workgroups), every task exactly once (its
    timer row set), outputs bitwise against the stock launch under identity,
    reversed and random pi, including a last round that is partial."""
    res = sched_pd.occupancy(sched_pd.build_args(
        torch.zeros(4, 1, 32, device="cuda"), torch.zeros(1, 1, 16, 32, device="cuda"),
        torch.zeros(1, 1, 16, 32, device="cuda"), torch.zeros(4, 1, dtype=torch.int32,
                                                              device="cuda"),
        torch.ones(4, dtype=torch.int32, device="cuda"), out=torch.zeros(4, 1, 32, device="cuda"),
        v_layout="tokmajor")) * sched_pd.cu_count()
    n = min(16383, 2 * res + 7)
    rng = np.random.default_rng(4)
    ctx = rng.integers(1, 40, n)
    b = batch(torch.float32, 32, 16, heads=1, ctx=ctx, seed=5)
    out, kind = run(b)
    assert kind == "wave"
    print(f"resident items {res}, tasks {n}")
    r = ref(b)
    assert par_err(out.cpu(), r, "wave rounds") <= TOL_F32
    plane = SchedPlane(max_tasks=n)
    for name, order in (("identity", np.arange(n)), ("reversed", np.arange(n)[::-1]),
                        ("random", rng.permutation(n))):
        plane.set_order(torch.from_numpy(order.astype(np.int32).copy()))
        plane.push()
        plane.clear_timer()
        o, _ = run(b, plane=plane)
        assert same(o, out), name
        rows = plane.read_timer()[:n].numpy()
        assert (rows > 0).all(), name


def batch_g(kv, d, ps, G, heads=4, ctx=CTX, seed=0, q_dtype=torch.float32):
    b = workloads.make_batch(np.asarray(ctx), num_q_heads=G * heads, num_kv_heads=heads,
                             head_dim=d, page_size=ps, kv_dtype=kv, q_dtype=q_dtype, seed=seed,
                             device="cuda")
    b["v_pool"] = b["v_pool"].permute(0, 1, 3, 2).contiguous()   # token-major V
    return b


@pytest.mark.parametrize("G", [2, 3])
@pytest.mark.parametrize("kv,d,qd", [(torch.float32, 32, torch.float32),
                                     (torch.float32, 128, torch.float32),
                                     (torch.bfloat16, 128, torch.bfloat16),
                                     (torch.bfloat16, 64, torch.float32),
                                     (torch.float16, 128, torch.float16)])
@pytest.mark.parametrize("ps", [16, 32])
def test_wave_kernel_groups_parity_and_levers(G, kv, d, qd, ps):
    """2 and 3 q-heads per kv-head on the one-wave kernel (below the MFMA
    kernel's 4): the oracle, pi and the queue bitwise, one timer row per
    task, and the MFMA kernel where it applies within the tolerance."""
    b = batch_g(kv, d, ps, G, seed=G * d + ps, q_dtype=qd)
    tol = TOL_F32 if kv == torch.float32 else TOL_BF16
    nm = abi.FLAG_NO_MFMA          # the MFMA kernel is the default where it applies
    out, kind = run(b, flags=nm)
    assert kind == "wave"
    r = ref(b)
    assert par_err(out.cpu(), r, f"wave G{G} {kv} d{d} p{ps}") <= tol
    n = len(CTX) * 4
    plane = SchedPlane(max_tasks=n)
    plane.set_order(torch.arange(n - 1, -1, -1, dtype=torch.int32))
    plane.push()
    plane.clear_timer()
    o, _ = run(b, plane=plane, flags=nm)
    assert same(o, out)
    assert (plane.read_timer()[:n].numpy() > 0).all()
    plane.set_num_tasks(n)
    plane.push()
    o, _ = run(b, plane=plane, workers=7, flags=nm)
    assert same(o, out)
    if kv != torch.float32 and d == 128 and qd == kv:
        m, k2 = run(b, default=True)
        assert k2 == "mfma"
        assert par_err(m.cpu(), r) <= tol


@pytest.mark.parametrize("G", [1, 3])
@pytest.mark.parametrize("ranged", [False, True])
def test_wave_kernel_split_items(G, ranged):
    """Split-KV work items on the one-wave kernel: a pair plan or a graded
    ranged plan, static grid, pi (reversed over items) and the ticket queue
    bitwise equal; the oracle; every task's timer row; counters left zero."""
    ctx = [1, 15, 300, 2049, 5000, 64, 0, 777]
    b = batch_g(torch.bfloat16, 128, 16, G, heads=2, ctx=ctx, seed=21 + G, q_dtype=torch.float32)
    if ranged:
        tiles = sched_pd.plan_graded_host(ctx, 16, 2, sizes=((0.0, 40), (0.5, 12), (0.9, 4)))
        kw = dict(tiles=tiles)
    else:
        tiles = sched_pd.plan_tiles_host(ctx, 16, 24, 2)
        kw = dict(tiles=tiles, tile_pages=24)
    nt = tiles.shape[0]
    ntask = len(ctx) * 2
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.clear_timer()
    out, kind = run(b, plane=plane, **kw)
    assert kind == "wave"
    assert par_err(out.cpu(), ref(b), f"split G{G} ranged={ranged}") <= TOL_BF16
    assert (plane.read_timer()[:ntask].numpy()[np.repeat(np.asarray(ctx), 2) > 0] > 0).all()
    plane.install_order(torch.arange(nt - 1, -1, -1, dtype=torch.int32), nt)
    plane.push()
    o, _ = run(b, plane=plane, **kw)
    assert same(o, out)
    plane.set_num_tasks(nt)
    plane.push()
    for W in (3, 64, nt + 5):
        o, _ = run(b, plane=plane, workers=W, **kw)
        assert same(o, out), W
    ws = sched_pd.workspace_for(0, "cuda")
    assert int(ws[sched_pd.WS_COUNTERS_OFF:sched_pd.WS_COUNTERS_OFF + 4 * ntask]
               .view(torch.int32).abs().sum()) == 0


def test_wave_kernel_split_items_stale_plan_and_shed():
    """A plan built for shorter contexts: the grown tasks' rows NaN and
    counted, the others right; then prefix budgets over a budget-aware
    graded plan against the oracle."""
    old_ctx, new_ctx = [100, 900, 40], [100, 1300, 40]
    b = batch_g(torch.float32, 64, 16, 2, heads=2, ctx=new_ctx, seed=31)
    fresh, _ = run(b, tiles=sched_pd.plan_tiles_host(new_ctx, 16, 8, 2), tile_pages=8)
    assert par_err(fresh.cpu(), ref(b)) <= TOL_F32
    ws = sched_pd.workspace_for(0, "cuda")        # the one the launches use
    sched_pd.stale_plan_count(ws, reset=True)
    tiles = sched_pd.plan_tiles_host(old_ctx, 16, 8, 2)
    out, kind = run(b, tiles=tiles, tile_pages=8)
    assert kind == "wave"
    got = out.cpu().numpy()
    assert np.isnan(got[1]).all()
    r = ref(b)
    assert par_err(got[[0, 2]], np.asarray(r)[[0, 2]]) <= TOL_F32
    assert sched_pd.stale_plan_count(ws, reset=True) == 2
    ntask = 6
    tau = np.array([0, 50, 700, 3, 0, 17])
    plane = SchedPlane(max_tasks=64)
    plane.set_rows(tau=tau, n=ntask)
    plane.push()
    gtiles = sched_pd.plan_graded_host(new_ctx, 16, 2, sizes=((0.0, 16), (0.7, 4)), tau=tau)
    o, _ = run(b, plane=plane, tiles=gtiles)
    assert par_err(o.cpu(), ref(b, plane), "split shed") <= TOL_F32
