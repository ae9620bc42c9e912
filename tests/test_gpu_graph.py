"""One serving step captured in a HIP graph: the cache writer appends a
token per request and the decode (ticket queue, pi, timer) reads the cache.
Nothing in the step records a memset (the queue resets itself, split-KV
counters too); the graph is replayed several times with eager work in
between, and every replay matches the eager step bit for bit."""
import numpy as np
import pytest
import torch

import kv_cache
import sched_pd
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


@pytest.mark.parametrize("dtype,tile_pages", [(torch.bfloat16, 0), (torch.bfloat16, 4),
                                              (torch.float8_e4m3fn, 8)])
def test_captured_step_replays_match_eager(dtype, tile_pages):
    rng = np.random.default_rng(11)
    R, hkv, hq, d, ps = 12, 8, 32, 128, 16
    lens = rng.integers(40, 900, R)
    cache = kv_cache.PagedKvCache(1024, hkv, d, ps, dtype=dtype)
    rids = list(range(R))
    for r in rids:
        cache.add_request(r)
    T = int(lens.sum())
    cache.append(rids, (torch.randn(T, hkv, d, device="cuda") / d ** 0.5).bfloat16(),
                 torch.randn(T, hkv, d, device="cuda").bfloat16(), lens.tolist())
    # the step's static inputs: one new token per request at a fixed position
    cache.reserve(rids, [1] * R)
    for r in rids:
        cache.lens[r] += 1
    bt, ctx = cache.block_table(rids)
    app = torch.arange(R + 1, dtype=torch.int32, device="cuda")
    k1 = torch.empty(R, hkv, d, device="cuda", dtype=torch.bfloat16)
    v1 = torch.empty_like(k1)
    q = torch.empty(R, hq, d, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(R, hq, d, device="cuda", dtype=torch.float32)
    tiles = sched_pd.plan_tiles(ctx.cpu(), ps, tile_pages, hkv) if tile_pages else None
    nitems = tiles.shape[0] if tiles is not None else R * hkv
    plane = SchedPlane(max_tasks=max(nitems, R * hkv))
    plane.install_order(torch.randperm(nitems, generator=torch.Generator().manual_seed(2))
                        .to(torch.int32), nitems)
    plane.set_num_tasks(nitems)
    plane.push()
    a_app = kv_cache.build_append_args(k1, v1, app, ctx, cache.k_pool, cache.v_pool, bt,
                                       k_scale=cache.k_scale, v_scale=cache.v_scale,
                                       max_append=1, v_layout=cache.v_layout)
    a_dec = sched_pd.build_args(q, cache.k_pool, cache.v_pool, bt, ctx, out=out,
                                k_scale=cache.k_scale, v_scale=cache.v_scale, plane=plane,
                                workers=48, tiles=tiles, tile_pages=tile_pages,
                                v_layout=cache.v_layout)

    def step(stream):
        kv_cache.launch_append(a_app, stream)
        sched_pd.launch(a_dec, stream)

    def fresh_inputs(seed):
        g = torch.Generator(device="cuda").manual_seed(seed)
        k1.copy_((torch.randn(R, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16())
        v1.copy_(torch.randn(R, hkv, d, device="cuda", generator=g).bfloat16())
        q.copy_((torch.randn(R, hq, d, device="cuda", generator=g) / d ** 0.5).bfloat16())

    side = torch.cuda.Stream()
    fresh_inputs(0)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(side)                     # warm outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step(side)
    torch.cuda.synchronize()
    for rep in range(4):
        print(f"replay {rep} dtype={dtype} tile_pages={tile_pages}", flush=True)
        fresh_inputs(100 + rep)
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        # eager work between replays, then the same step eagerly
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {rep}"
