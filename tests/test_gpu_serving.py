"""A serving loop on the GPU: per step the writer appends one token per
request, the hooks plan the step, the decode runs with the hooks' tables and
launch arguments; every step's output is bit-identical to the stock decode of
the same work-item plan, within the tolerance of the unsplit decode and of the
oracle on the cache's pools, with and without the L2 hints; probe steps feed
the controller."""
import numpy as np
import pytest
import torch

import kv_cache
import oracle
from parity import TOL_BF16, par_err
from sched_rt import SchedPlane
from serving import HookConfig, ServingHooks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


@pytest.mark.parametrize("clc,tile_pages,hints", [("on", 0, False), ("off", 0, False),
                                                  ("auto", 8, False), ("on", 8, True),
                                                  ("off", 0, True)])
def test_serving_loop_keeps_outputs_bit_identical(clc, tile_pages, hints):
    rng = np.random.default_rng(3)
    R, hkv, hq, d, ps = 24, 8, 32, 128, 16
    lens = rng.integers(16, 1500, R)
    lens[5] = 3000
    cache = kv_cache.PagedKvCache(4096, hkv, d, ps, dtype=torch.bfloat16)
    rids = list(range(100, 100 + R))
    for r in rids:
        cache.add_request(r)
    T = int(lens.sum())
    k = (torch.randn(T, hkv, d, device="cuda") / d ** 0.5).bfloat16()
    v = torch.randn(T, hkv, d, device="cuda").bfloat16()
    cache.append(rids, k, v, lens.tolist())
    plane = SchedPlane(max_tasks=4096)
    # hints: an L2 budget far below the batch's KV, so long requests run
    # polite and short ones urgent
    hooks = ServingHooks(plane, hkv, HookConfig(plan_every=2, timer_every=3, resident=64,
                                                clc=clc, tile_pages=tile_pages,
                                                kv_bytes_per_token=hkv * d * 2 * 2 if hints else 0,
                                                l2_bytes=1 << 20))
    for step in range(8):
        print(f"step {step} clc={clc} tile_pages={tile_pages}", flush=True)
        k1 = (torch.randn(R, hkv, d, device="cuda") / d ** 0.5).bfloat16()
        v1 = torch.randn(R, hkv, d, device="cuda").bfloat16()
        cache.append(rids, k1, v1)
        q = (torch.randn(R, hq, d, device="cuda") / d ** 0.5).bfloat16()
        kv_now = [cache.lens[r] for r in rids]
        launch = hooks.on_batch_begin(rids, kv_now)
        out = torch.empty(R, hq, d, dtype=torch.float32, device="cuda")
        cache.decode(q, rids, out=out, **launch)
        hooks.on_batch_end()
        # the stock decode of the same split plan (a split changes the
        # summation order, the levers must not)
        ref = torch.empty_like(out)
        cache.decode(q, rids, out=ref, tiles=launch["tiles"], tile_pages=launch["tile_pages"])
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"step {step}"
        if step % 3 == 0:
            # the hooks-driven step against the oracle on the cache's pools
            bt, ctx = cache.block_table(rids)
            r = oracle.decode(q, cache.k_pool, cache.v_pool, bt, ctx, v_layout=cache.v_layout)
            assert par_err(out.cpu(), r, f"serving step {step}") <= TOL_BF16
        if launch["tiles"] is not None:
            whole = torch.empty_like(out)
            cache.decode(q, rids, out=whole)
            torch.cuda.synchronize()
            # a split changes the summation order (and the running max each
            # partial is scaled against): the tolerance, as against the oracle
            assert par_err(out.cpu(), whole.cpu()) <= TOL_BF16
    torch.cuda.synchronize()
    hooks.on_batch_begin(rids, [cache.lens[r] for r in rids])   # folds the last probe
    assert hooks.probes_folded >= 2
    alpha, _ = hooks.ctl.coefficients()
    assert alpha > 0
