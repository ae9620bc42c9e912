"""The fused append + decode step (sched_paged_decode_append through
PagedKvCache.decode_step) against the writer followed by the decode on a
second cache with the same contents: pools and outputs bitwise equal, over a
multi-step loop with tokens that open new pages, for bf16, fp16 and fp8
caches (fp8: the pages' scales grown and their earlier codes re-encoded as
the writer does, over steps of growing magnitude), 16- and 64-token pages, 1
and 4 q-heads per kv-head, fp32 and 16-bit source rows, with split tiles,
the ticket queue and pi; and the oracle on the result. Caches the fused
path does not take (d-major V) fall back to the two launches with the same
result; a direct fused launch on them is refused."""
import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
import sched_pd
from kv_cache import PagedKvCache, build_append_args, paired_scales
from parity import TOL_BF16, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu

HKV, D = 2, 128


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def make_pair(dtype, ps, lens, v_layout="tokmajor", seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    R = len(lens)
    npages = int(sum(-(-(n + 8) // ps) for n in lens)) + R + 4
    caches = [PagedKvCache(npages, HKV, D, ps, dtype=dtype, v_layout=v_layout) for _ in range(2)]
    T = int(sum(lens))
    src = torch.float32 if dtype == torch.float8_e4m3fn else dtype
    k = (torch.randn(T, HKV, D, device="cuda", generator=g) / D ** 0.5).to(src)
    v = (torch.randn(T, HKV, D, device="cuda", generator=g) / D ** 0.5).to(src)
    for c in caches:
        for r in range(R):
            c.add_request(r)
        c.append(list(range(R)), k, v, list(lens))
    return caches, g


def same(a, b):
    return bool(torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8)))


FP8 = torch.float8_e4m3fn


def qdtype(dtype):
    return torch.bfloat16 if dtype == FP8 else dtype


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, FP8])
@pytest.mark.parametrize("ps", [16, 64])
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("src32", [False, True])
def test_fused_step_equals_append_then_decode(dtype, ps, G, src32):
    # lengths just below, at and past page boundaries, so steps open pages
    lens = [1, 15, 16, 17, 31, 47, 63, 64, 65, 100, 127, 200]
    (fa, sep), g = make_pair(dtype, ps, lens, seed=ps + G)
    R = len(lens)
    rids = list(range(R))
    q = (torch.randn(R, HKV * G, D, device="cuda", generator=g) / D ** 0.5).to(qdtype(dtype))
    for step in range(5):
        st = torch.float32 if src32 else qdtype(dtype)
        # fp8: magnitudes grow step by step, so most pages' scales regrow
        amp = 2.0 ** step if dtype == FP8 else 1.0
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) * amp / D ** 0.5).to(st)
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) * amp / D ** 0.5).to(st)
        # fp32 output: the oracle check below then measures the kernel, not
        # the output's rounding (bf16 alone rounds by up to 2^-9 relative)
        o_fused = fa.decode_step(q, rids, k1, v1, out_dtype=torch.float32)
        sep.append(rids, k1, v1)
        o_sep = sep.decode(q, rids, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert same(o_fused, o_sep), step
        assert same(fa.k_pool, sep.k_pool) and same(fa.v_pool, sep.v_pool), step
        assert [fa.lens[r] for r in rids] == [sep.lens[r] for r in rids]
        if dtype == FP8:
            assert same(fa.k_scale, sep.k_scale) and same(fa.v_scale, sep.v_scale), step
    bt, ctx = fa.block_table(rids)
    ref = oracle.decode(q, fa.k_pool, fa.v_pool, bt, ctx, v_layout="tokmajor",
                        k_scale=fa.k_scale, v_scale=fa.v_scale)
    assert par_err(o_fused.float().cpu(), ref, f"fused {dtype} p{ps} G{G}") <= TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ps", [16, 64])
def test_fused_step_on_the_one_wave_kernel(dtype, ps):
    """One q-head per kv-head with the MFMA kernel kept out, so the one-wave
    kernel streams the step and writes the token: pools and outputs bitwise
    equal to append-then-decode on the same kernel."""
    lens = [1, 15, 16, 17, 31, 47, 63, 64, 65, 100, 127, 200]
    (fa, sep), g = make_pair(dtype, ps, lens, seed=ps + 7)
    R = len(lens)
    rids = list(range(R))
    q = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).to(qdtype(dtype))
    for step in range(4):
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).to(dtype)
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).to(dtype)
        o_fused = fa.decode_step(q, rids, k1, v1, out_dtype=torch.float32,
                                 flags=abi.FLAG_NO_MFMA)
        sep.append(rids, k1, v1)
        o_sep = sep.decode(q, rids, out_dtype=torch.float32, flags=abi.FLAG_NO_MFMA)
        torch.cuda.synchronize()
        assert same(o_fused, o_sep), step
        assert same(fa.k_pool, sep.k_pool) and same(fa.v_pool, sep.v_pool), step
    bt, ctx = fa.block_table(rids)
    assert sched_pd.kernel_kind(sched_pd.build_args(
        q, fa.k_pool, fa.v_pool, bt, ctx, out=torch.empty_like(o_fused), v_layout="tokmajor",
        flags=abi.FLAG_NO_MFMA)) == "wave"
    ref = oracle.decode(q, fa.k_pool, fa.v_pool, bt, ctx, v_layout="tokmajor")
    assert par_err(o_fused.float().cpu(), ref, f"fused wave {dtype} p{ps}") <= TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, FP8])
@pytest.mark.parametrize("ranged", [False, True])
def test_fused_step_with_tiles_queue_and_pi(ranged, dtype):
    lens = [int(x) for x in np.random.default_rng(2).integers(1, 900, 40)]
    (fa, sep), g = make_pair(dtype, 16, lens, seed=3)
    R = len(lens)
    rids = list(range(R))
    q = (torch.randn(R, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    tp = 8
    for step in range(4):
        amp = 2.0 ** step if dtype == FP8 else 1.0
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) * amp / D ** 0.5).bfloat16()
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) * amp / D ** 0.5).bfloat16()
        after = [fa.lens[r] + 1 for r in rids]          # plan from the post-append lengths
        if ranged:     # host rows, chunks of 8 pages and of 3 at the end of pi
            tiles = sched_pd.plan_ranges_host(after, 16, HKV, task_order=np.arange(R * HKV)[::-1],
                                              tile_pages=tp, tail_pages=3, tail_frac=0.5)
        else:
            tiles = sched_pd.plan_tiles(after, 16, tp, HKV)
        nt = tiles.shape[0]
        plane = SchedPlane(max_tasks=max(nt, R * HKV))
        plane.install_order(torch.arange(nt - 1, -1, -1, dtype=torch.int32), nt)
        plane.set_num_tasks(nt)
        plane.push()
        plane.reset_queue(7)
        tkw = dict(tiles=tiles) if ranged else dict(tiles=tiles, tile_pages=tp)
        o_fused = fa.decode_step(q, rids, k1, v1, plane=plane, workers=7, **tkw)
        sep.append(rids, k1, v1)
        o_sep = sep.decode(q, rids, **tkw)
        torch.cuda.synchronize()
        assert same(fa.k_pool, sep.k_pool) and same(fa.v_pool, sep.v_pool), step
        assert same(o_fused, o_sep), step
        if dtype == FP8:
            assert same(fa.k_scale, sep.k_scale) and same(fa.v_scale, sep.v_scale), step


@pytest.mark.parametrize("layout", ["tokmajor", "dmajor"])
def test_steps_on_a_side_stream_match_the_current_stream(layout):
    """decode_step with stream=: the step's uploads, table update, append
    and decode all go to that stream (the fused launch, or the writer then
    the decode for d-major V); pools and outputs equal the same steps on the
    current stream, which is kept busy meanwhile."""
    lens = [int(x) for x in np.random.default_rng(5).integers(1, 600, 24)]
    (a, b), g = make_pair(torch.bfloat16, 16, lens, v_layout=layout, seed=11)
    R = len(lens)
    rids = list(range(R))
    q = (torch.randn(R, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    side = torch.cuda.Stream()
    busy = torch.randn(2048, 2048, device="cuda")
    for step in range(6):
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
        tiles = sched_pd.plan_tiles_host(a.lengths(rids) + 1, 16, 4, HKV)
        o_a = a.decode_step(q, rids, k1, v1, tiles=tiles, tile_pages=4)
        side.wait_stream(torch.cuda.current_stream())
        for _ in range(3):
            busy = busy @ busy / 64.0        # the current stream stays busy
        o_b = b.decode_step(q, rids, k1, v1, tiles=tiles, tile_pages=4, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert same(a.k_pool, b.k_pool) and same(a.v_pool, b.v_pool), (layout, step)
        assert same(o_a, o_b), (layout, step)


def test_caches_without_the_fused_path_fall_back_and_direct_launch_is_refused():
    lens = [5, 16, 40]
    for dtype, layout in ((torch.float8_e4m3fn, "dmajor"), (torch.bfloat16, "dmajor")):
        (fa, sep), g = make_pair(dtype, 16, lens, v_layout=layout, seed=7)
        rids = [0, 1, 2]
        q = (torch.randn(3, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
        k1 = (torch.randn(3, HKV, D, device="cuda", generator=g) / D ** 0.5)
        k1 = k1 if dtype == torch.float8_e4m3fn else k1.bfloat16()
        o = fa.decode_step(q, rids, k1, k1)
        sep.append(rids, k1, k1)
        o2 = sep.decode(q, rids)
        torch.cuda.synchronize()
        assert same(o, o2), (dtype, layout)
        bt, ctx = fa.block_table(rids)
        out = torch.empty(3, HKV * 4, D, dtype=torch.bfloat16, device="cuda")
        args = sched_pd.build_args(q, fa.k_pool, fa.v_pool, bt, ctx, out=out, v_layout=layout,
                                   k_scale=fa.k_scale, v_scale=fa.v_scale)
        app = build_append_args(k1, k1, torch.arange(4, dtype=torch.int32, device="cuda"), ctx,
                                fa.k_pool, fa.v_pool, bt, v_layout=layout, k_scale=fa.k_scale,
                                v_scale=fa.v_scale, max_append=1)
        with pytest.raises(RuntimeError, match="fused append"):
            sched_pd.launch_with_append(args, app)


def test_fused_launch_over_a_csr_page_table():
    """The C entry point with a CSR table (page_indptr + indices), against
    sched_kv_append + sched_paged_decode over copies of the same pools."""
    from kv_cache import append as kv_append
    from kv_cache import ctx_lens_from_last_page_len
    lens = [3, 16, 33, 70, 129]
    (c, _), g = make_pair(torch.bfloat16, 16, lens, seed=11)
    rids = list(range(len(lens)))
    c.reserve(rids, [1] * len(lens))
    for r in rids:
        c.lens[r] += 1                      # room for this step's token
    indptr, idx, last = c.csr(rids)
    ctx = ctx_lens_from_last_page_len(indptr, last, 16).to(torch.int32)
    R = len(lens)
    q = (torch.randn(R, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    app_ptr = torch.arange(R + 1, dtype=torch.int32, device="cuda")
    outs, pools = [], []
    for fused in (True, False):
        kp, vp = c.k_pool.clone(), c.v_pool.clone()
        out = torch.empty(R, HKV * 4, D, dtype=torch.bfloat16, device="cuda")
        args = sched_pd.build_args(q, kp, vp, idx, ctx, out=out, page_indptr=indptr,
                                   v_layout="tokmajor")
        if fused:
            app = build_append_args(k1, v1, app_ptr, ctx, kp, vp, idx, page_indptr=indptr,
                                    v_layout="tokmajor", max_append=1)
            sched_pd.launch_with_append(args, app)
        else:
            kv_append(k1, v1, app_ptr, ctx, kp, vp, idx, page_indptr=indptr,
                      v_layout="tokmajor", max_append=1)
            sched_pd.launch(args)
        torch.cuda.synchronize()
        outs.append(out)
        pools.append((kp, vp))
    assert same(outs[0], outs[1])
    assert same(pools[0][0], pools[1][0]) and same(pools[0][1], pools[1][1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, FP8])
@pytest.mark.parametrize("ranged", [False, True])
def test_fused_launch_with_a_stale_plan_still_writes_the_token(ranged, dtype):
    """A plan built from the lengths before the append, where the new token
    opens a page in a chunk the plan does not hold (64 tokens in 4-page
    chunks of 16-token pages: the 65th token starts chunk 1). The fused
    launch flags those tasks stale (NaN rows, counted), yet writes every
    token: the pools equal the writer's, and the tasks the plan still covers
    equal append-then-decode. Through PagedKvCache.decode_step a host plan
    this stale is refused before anything is written."""
    from kv_cache import append as kv_append
    lens = [64, 10, 128, 40]          # requests 0 and 2 open a page in a new chunk
    (c, _), g = make_pair(dtype, 16, lens, seed=13)
    rids = list(range(len(lens)))
    R, tp = len(lens), 4
    before = c.lengths(rids)
    if ranged:
        plan_h = sched_pd.plan_ranges_host(before, 16, HKV, tile_pages=tp, tail_pages=tp)
    else:
        plan_h = sched_pd.plan_tiles_host(before, 16, tp, HKV)
    q = (torch.randn(R, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    # the cache refuses a stale host plan for its fused step, and is unchanged
    kp0, vp0 = c.k_pool.clone(), c.v_pool.clone()
    tkw = dict(tiles=plan_h) if ranged else dict(tiles=plan_h, tile_pages=tp)
    with pytest.raises(ValueError, match="stale"):
        c.decode_step(q, rids, k1, v1, **tkw)
    assert c.lengths(rids).tolist() == list(before)
    assert same(c.k_pool, kp0) and same(c.v_pool, vp0)
    # the kernel path: one launch with the stale plan, against the writer
    c.reserve(rids, [1] * R)
    for r in rids:
        c.lens[r] += 1
    bt, ctx = c.block_table(rids)
    app_ptr = torch.arange(R + 1, dtype=torch.int32, device="cuda")
    plan = torch.from_numpy(plan_h).cuda()
    outs, pools = [], []
    fp8 = dtype == FP8
    for fused in (True, False):
        kp, vp = c.k_pool.clone(), c.v_pool.clone()
        sc = {}
        if fp8:
            ks, vs = paired_scales(c.k_scale.numel(), "cuda")
            ks.copy_(c.k_scale)
            vs.copy_(c.v_scale)
            sc = dict(k_scale=ks, v_scale=vs)
        out = torch.empty(R, HKV * 4, D, dtype=torch.bfloat16, device="cuda")
        ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
        kw = dict(tiles=plan, workspace=ws) if ranged else \
            dict(tiles=plan, tile_pages=tp, workspace=ws)
        args = sched_pd.build_args(q, kp, vp, bt, ctx, out=out, v_layout="tokmajor", **sc, **kw)
        if fused:
            app = build_append_args(k1, v1, app_ptr, ctx, kp, vp, bt, v_layout="tokmajor",
                                    max_append=1, **sc)
            sched_pd.launch_with_append(args, app)
        else:
            kv_append(k1, v1, app_ptr, ctx, kp, vp, bt, v_layout="tokmajor", max_append=1, **sc)
            sched_pd.launch(args)
        torch.cuda.synchronize()
        outs.append(out)
        pools.append((kp, vp) + ((sc["k_scale"], sc["v_scale"]) if fp8 else ()))
        assert sched_pd.stale_plan_count(ws) == 2 * HKV
        assert int(ws[sched_pd.WS_COUNTERS_OFF:sched_pd.WS_COUNTERS_OFF + 4 * R * HKV]
                   .view(torch.int32).abs().sum()) == 0
    for a_, b_ in zip(pools[0], pools[1]):
        assert same(a_, b_)
    got = outs[0].float()
    assert torch.isnan(got[[0, 2]]).all() and torch.isfinite(got[[1, 3]]).all()
    assert same(outs[0][[1, 3]], outs[1][[1, 3]])
    ref = oracle.decode(q, pools[0][0], pools[0][1], bt, ctx, v_layout="tokmajor",
                        **({"k_scale": pools[0][2], "v_scale": pools[0][3]} if fp8 else {}))
    assert par_err(got[[1, 3]].cpu(), np.asarray(ref)[[1, 3]]) <= TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, FP8])
def test_fused_step_under_a_shed_budget(dtype):
    """Prefix budgets below the new token's position: the token is still
    written (the pages past the budget are not read), and the output equals
    append-then-decode under the same rows."""
    lens = [30, 100, 250, 17]
    (fa, sep), g = make_pair(dtype, 16, lens, seed=17)
    R = len(lens)
    rids = list(range(R))
    q = (torch.randn(R, HKV * 4, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
    plane = SchedPlane(max_tasks=R * HKV)
    plane.set_rows(tau=[5, 8, 40, 300, 16, 0, 1, 2], n=R * HKV)
    plane.push()
    for step in range(3):
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).bfloat16()
        o_fused = fa.decode_step(q, rids, k1, v1, plane=plane)
        sep.append(rids, k1, v1)
        o_sep = sep.decode(q, rids, plane=plane)
        torch.cuda.synchronize()
        assert same(fa.k_pool, sep.k_pool) and same(fa.v_pool, sep.v_pool), step
        assert same(o_fused, o_sep), step
        if dtype == FP8:
            assert same(fa.k_scale, sep.k_scale) and same(fa.v_scale, sep.v_scale), step


@pytest.mark.parametrize("dtype", [torch.bfloat16, FP8])
@pytest.mark.parametrize("G", [1, 4])
def test_fused_step_opens_an_empty_requests_first_page(dtype, G):
    """Requests that hold no token yet (added, nothing appended) take their
    first token in a fused step beside requests that hold many: the same
    pools, scales and outputs as the writer followed by the decode."""
    lens = [0, 40, 0, 17, 300]
    R = len(lens)
    g = torch.Generator(device="cuda").manual_seed(29)
    npages = int(sum(-(-(n + 4) // 16) for n in lens)) + R + 4
    caches = [PagedKvCache(npages, HKV, D, 16, dtype=dtype) for _ in range(2)]
    T = int(sum(lens))
    src = torch.float32 if dtype == FP8 else dtype
    k = (torch.randn(T, HKV, D, device="cuda", generator=g) / D ** 0.5).to(src)
    v = (torch.randn(T, HKV, D, device="cuda", generator=g) / D ** 0.5).to(src)
    for c in caches:
        for r in range(R):
            c.add_request(r)
        c.append(list(range(R)), k, v, list(lens))
    fa, sep = caches
    rids = list(range(R))
    q = (torch.randn(R, HKV * G, D, device="cuda", generator=g) / D ** 0.5).to(qdtype(dtype))
    for step in range(3):
        k1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).to(qdtype(dtype))
        v1 = (torch.randn(R, HKV, D, device="cuda", generator=g) / D ** 0.5).to(qdtype(dtype))
        o_f = fa.decode_step(q, rids, k1, v1, out_dtype=torch.float32)
        sep.append(rids, k1, v1)
        o_s = sep.decode(q, rids, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert same(o_f, o_s), step
        assert same(fa.k_pool, sep.k_pool) and same(fa.v_pool, sep.v_pool), step
        if dtype == FP8:
            assert same(fa.k_scale, sep.k_scale) and same(fa.v_scale, sep.v_scale), step
    assert [fa.lens[r] for r in rids] == [n + 3 for n in lens]
    bt, ctx = fa.block_table(rids)
    ref = oracle.decode(q, fa.k_pool, fa.v_pool, bt, ctx, v_layout="tokmajor",
                        k_scale=fa.k_scale, v_scale=fa.v_scale)
    assert par_err(o_f.cpu(), ref, f"empty requests {dtype} G{G}") <= TOL_BF16
