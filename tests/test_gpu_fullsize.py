"""The measured workloads at their full sizes: the Llama-3-8B uniform step
(64 x 2048, 4 GiB pool), the heterogeneous batch (256 requests, lognormal
ctx up to 32k), the shed sweep (128 requests, tau ~ U[ctx/4, ctx]) and the
Qwen2-7B fp8 batch (512 requests). Size-independent properties on the whole
batch (schedule invariance, finiteness), and oracle parity on a sample of
requests that always includes the longest one: the sampled requests' pages
are gathered into a compact pool so the oracle reads megabytes, not the
whole pool."""
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

# par_err <= TOL_BF16: mixed form and per-row norm-relative error (tests/parity.py)


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib




def sample(ctx, k, seed):
    """k request indices: the longest, the shortest and k-2 random others."""
    ctx = np.asarray(ctx)
    rng = np.random.default_rng(seed)
    pick = {int(np.argmax(ctx)), int(np.argmin(ctx))}
    for r in rng.permutation(ctx.size):
        if len(pick) >= k:
            break
        pick.add(int(r))
    return np.array(sorted(pick))


def compact(b, idx):
    """The sampled requests with their pages copied into a fresh pool (page
    ids renumbered): same KV, same scales, a pool of only those pages."""
    ps = b["page_size"]
    ctx = b["ctx_lens"].cpu().numpy()[idx].astype(np.int64)
    bt = b["block_table"].cpu().numpy()[idx]
    npg = (ctx + ps - 1) // ps
    used = np.concatenate([bt[i, :npg[i]] for i in range(idx.size)]).astype(np.int64)
    uniq, inv = np.unique(used, return_inverse=True)
    nbt = np.zeros((idx.size, max(int(npg.max()), 1)), np.int32)
    at = 0
    for i in range(idx.size):
        nbt[i, :npg[i]] = inv[at:at + npg[i]]
        at += npg[i]
    sel = torch.from_numpy(uniq).cuda()
    out = {"q": b["q"][torch.from_numpy(idx).cuda()].contiguous(),
           "k_pool": b["k_pool"][sel].contiguous(), "v_pool": b["v_pool"][sel].contiguous(),
           "block_table": torch.from_numpy(nbt).cuda(),
           "ctx_lens": torch.from_numpy(ctx.astype(np.int32)).cuda(), "page_size": ps,
           "k_scale": None, "v_scale": None}
    if b["k_scale"] is not None:
        out["k_scale"] = b["k_scale"][sel].contiguous()
        out["v_scale"] = b["v_scale"][sel].contiguous()
    return out


def decode(b, **kw):
    R = b["ctx_lens"].numel()
    rows = b["v_pool"].shape[1] if kw.get("mode", abi.SOFTMAX) == abi.LINEAR else b["q"].shape[1]
    out = torch.full((R, rows, 128), float("nan"), dtype=torch.float32, device="cuda")
    sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                          out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], **kw)
    torch.cuda.synchronize()
    return out


def oracle_of(c, plane=None, **kw):
    ctrl = None
    if plane is not None:
        ctrl = bytes(plane._ctrl_host)
    return oracle.decode(c["q"], c["k_pool"], c["v_pool"], c["block_table"], c["ctx_lens"],
                         k_scale=c["k_scale"], v_scale=c["v_scale"], ctrl=ctrl,
                         max_tasks=plane.N if plane is not None else 4096, **kw)


def check_sample(b, out, idx, hkv, tau=None, **kw):
    """Oracle parity of out[idx] on the compacted sample; tau per task of the
    whole batch (prefix budget) or None; kw: the oracle's mode arguments."""
    c = compact(b, idx)
    plane = None
    if tau is not None:
        plane = SchedPlane(max_tasks=idx.size * hkv, device="cpu")
        plane.set_rows(tau=np.asarray(tau).reshape(-1, hkv)[idx].reshape(-1), n=idx.size * hkv)
    r = oracle_of(c, plane, **kw)
    e = par_err(out[torch.from_numpy(idx).cuda()].cpu(), r)
    print(f"sample {idx.tolist()} ctx {c['ctx_lens'].cpu().tolist()} err {e:.3g}", flush=True)
    assert e <= TOL_BF16


def test_llama3_8b_uniform_full_size():
    """The bench step itself: 64 x 2048 bf16 over the 65,536-page pool. pi
    reversed under the ticket queue gives the static grid's bits; sampled
    requests match the oracle."""
    print("case llama3_8b_uniform", flush=True)
    b = workloads.workload("llama3_8b_uniform", seed=0)
    ntask = 64 * 8
    base = decode(b)
    assert torch.isfinite(base).all()
    plane = SchedPlane(max_tasks=ntask)
    plane.set_order(torch.arange(ntask - 1, -1, -1, dtype=torch.int32))
    plane.set_num_tasks(ntask)
    plane.push()
    W = 2 * sched_pd.cu_count()
    plane.reset_queue(W)
    assert torch.equal(decode(b, plane=plane, workers=W), base)
    check_sample(b, base, sample(b["ctx_lens"].cpu().numpy(), 6, 1), 8)


def test_hetero_batch_full_size():
    """256 requests, lognormal ctx (max ~26k): split tiles under the queue
    with pi by urgency and pi longest-first give the same bits as the static
    grid over the same tiles; the unsplit static grid agrees within the bf16
    tolerance; sampled requests (the longest included) match the oracle."""
    print("case llama3_8b_hetero", flush=True)
    b = workloads.workload("llama3_8b_hetero", seed=0)
    ctx = b["ctx_lens"].cpu().numpy()
    ntask, tp = 256 * 8, 128
    W = 2 * sched_pd.cu_count()
    tiles = sched_pd.plan_tiles(ctx, 16, tp, 8)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.set_num_tasks(0)
    plane.push()
    static_tiles = decode(b, plane=plane, tiles=tiles, tile_pages=tp)
    assert torch.isfinite(static_tiles).all()
    for order in (sched_pd.tile_order_by_task_key(tiles, b["urgency"]),
                  sched_pd.tile_order_lpt(sched_pd.tile_pages_loaded(tiles, ctx, 16, tp, 8))):
        plane.install_order(order, nt)
        plane.set_num_tasks(nt)
        plane.push()
        plane.reset_queue(W)
        assert torch.equal(decode(b, plane=plane, workers=W, tiles=tiles, tile_pages=tp),
                           static_tiles)
    unsplit = decode(b)
    assert par_err(unsplit.cpu(), static_tiles.cpu()) <= TOL_BF16
    check_sample(b, static_tiles, sample(ctx, 5, 2), 8)
    # a ranged plan with short chunks for the tasks claimed last (pi by
    # urgency): the queue gives the static grid's bits over the same plan
    rt = sched_pd.plan_ranges_host(ctx, 16, 8, task_order=np.argsort(-b["urgency"],
                                                                    kind="stable"),
                                   tile_pages=160, tail_pages=64, tail_frac=0.1)
    nr = rt.shape[0]
    rplane = SchedPlane(max_tasks=max(nr, ntask))
    rplane.set_num_tasks(0)
    rplane.push()
    ranged_static = decode(b, plane=rplane, tiles=rt)
    rplane.install_order(sched_pd.tile_order_by_task_key(rt, b["urgency"]), nr)
    rplane.set_num_tasks(nr)
    rplane.push()
    rplane.reset_queue(W)
    assert torch.equal(decode(b, plane=rplane, workers=W, tiles=rt), ranged_static)
    assert par_err(ranged_static.cpu(), static_tiles.cpu()) <= TOL_BF16
    check_sample(b, ranged_static, sample(ctx, 5, 5), 8)


@pytest.mark.parametrize("mode", [abi.SOFTMAX, abi.LINEAR])
def test_shed_full_size(mode):
    """128 requests, tau ~ U[ctx/4, ctx] per task (prefix budget), policy
    armed (q ~ U(0,1), lambda_bw 0.5, H 0.1, urgent ring 4 pages), both shed
    variants: online softmax (masked score -inf) and the linear contraction
    (masked value 0). Skipping the pages past tau gives the bits of loading and
    masking them, under the queue with pi longest-first over 256-page tiles;
    sampled requests (the longest included) match the truncated oracle."""
    print(f"case llama3_8b_shed mode {mode}", flush=True)
    b = workloads.workload("llama3_8b_shed", seed=0)
    ctx = b["ctx_lens"].cpu().numpy()
    ntask, tp = 128 * 8, 256
    W = 2 * sched_pd.cu_count()
    tiles = sched_pd.plan_tiles(ctx, 16, tp, 8)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.set_lambda(0.5)
    plane.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    pages = sched_pd.tile_pages_loaded(tiles, ctx, 16, tp, 8, tau=b["tau"])
    plane.install_order(sched_pd.tile_order_lpt(pages), nt)
    plane.set_num_tasks(nt)
    plane.push()
    plane.reset_queue(W)
    kw = dict(plane=plane, workers=W, tiles=tiles, tile_pages=tp, policy=(1.0, 1.0, 0.1),
              pf_dist=4)
    okw = {}
    if mode == abi.LINEAR:
        w = torch.randn(8192, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3))
        kw.update(mode=abi.LINEAR, lin_w=w)
        okw = dict(mode=abi.LINEAR, lin_w=w.cpu().numpy())
    skip = decode(b, **kw)
    assert torch.isfinite(skip).all()
    assert torch.equal(decode(b, flags=abi.FLAG_SHED_LOADS, **kw), skip)
    # the policy priced out (no task urgent) gives the same bits
    plane.set_lambda(1000.0)
    plane.push()
    assert torch.equal(decode(b, **kw), skip)
    check_sample(b, skip, sample(ctx, 5, 3), 8, tau=b["tau"], **okw)
    # a ranged plan cut from the pages each task reads (pi by urgency, short
    # chunks for the tasks claimed last): loading and masking the shed
    # tokens gives the bits of skipping them; sampled requests match
    rt = sched_pd.plan_ranges_host(ctx, 16, 8, task_order=np.argsort(-b["urgency"],
                                                                    kind="stable"),
                                   tile_pages=160, tail_pages=64, tail_frac=0.1,
                                   tau=b["tau"][:ntask])
    nr = rt.shape[0]
    rplane = SchedPlane(max_tasks=max(nr, ntask))
    rplane.set_lambda(0.5)
    rplane.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    rplane.install_order(sched_pd.tile_order_by_task_key(rt, b["urgency"]), nr)
    rplane.set_num_tasks(nr)
    rplane.push()
    rplane.reset_queue(W)
    rkw = dict(kw, plane=rplane, tiles=rt)
    del rkw["tile_pages"]
    rskip = decode(b, **rkw)
    assert torch.isfinite(rskip).all()
    assert torch.equal(decode(b, flags=abi.FLAG_SHED_LOADS, **rkw), rskip)
    assert par_err(rskip.cpu(), skip.cpu()) <= TOL_BF16
    check_sample(b, rskip, sample(ctx, 5, 6), 8, tau=b["tau"], **okw)


def test_qwen2_fp8_full_size():
    """512 requests, fp8 KV with per-(page, head) scales: the queue over
    256-page tiles with the timer on agrees with the static unsplit grid
    within the tolerance, every task's timer row is set, and sampled
    requests match the oracle on the dequantised KV."""
    print("case qwen2_7b_fp8", flush=True)
    b = workloads.workload("qwen2_7b_fp8", seed=0)
    ctx = b["ctx_lens"].cpu().numpy()
    ntask, tp = 512 * 4, 256
    W = 2 * sched_pd.cu_count()
    tiles = sched_pd.plan_tiles(ctx, 16, tp, 4)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.set_num_tasks(nt)
    plane.push()
    plane.reset_queue(W)
    plane.clear_timer()
    wq = decode(b, plane=plane, workers=W, tiles=tiles, tile_pages=tp)
    assert torch.isfinite(wq).all()
    cyc = plane.read_timer()[:ntask].numpy()
    assert np.all(cyc > 0)
    static = decode(b)
    assert par_err(static.cpu(), wq.cpu()) <= TOL_BF16
    check_sample(b, wq, sample(ctx, 6, 4), 4)
    # the queue over a ranged plan (320-page chunks, 128-page ones for the
    # last tenth of the pages)
    rt = sched_pd.plan_ranges_host(ctx, 16, 4, tile_pages=320, tail_pages=128, tail_frac=0.1)
    nr = rt.shape[0]
    rplane = SchedPlane(max_tasks=max(nr, ntask))
    rplane.set_num_tasks(nr)
    rplane.push()
    rplane.reset_queue(W)
    rq = decode(b, plane=rplane, workers=W, tiles=rt)
    assert torch.isfinite(rq).all()
    assert par_err(static.cpu(), rq.cpu()) <= TOL_BF16
    check_sample(b, rq, sample(ctx, 6, 7), 4)
