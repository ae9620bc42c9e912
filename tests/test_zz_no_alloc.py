"""The no-allocation entry point (sched_paged_decode_noalloc) against
sched_paged_decode with a workspace: the same kernels over the same split
plan, so the same bits. Two calls in a row, the second over a smaller batch
(the scratch keeps the first call's partials; the counters are cleared per
call), with pi and the ticket queue armed, over pair and ranged plans; a
launch without tiles; and the refusals (a workspace passed in, a plan
beyond the scratch)."""
import ctypes

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


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def _batch(ctx, seed):
    return workloads.make_batch(np.asarray(ctx), num_q_heads=32, num_kv_heads=8, head_dim=128,
                                kv_dtype=torch.bfloat16, q_dtype=torch.bfloat16, seed=seed,
                                device="cuda")


def _args(b, out, plane, tiles, tp, workers):
    return sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                               b["ctx_lens"], out=out, plane=plane, tiles=tiles, tile_pages=tp,
                               workers=workers)


def _noalloc(lib, args):
    a = abi.SchedDecodeArgs.from_buffer_copy(args)
    a.workspace, a.workspace_bytes = None, 0
    s = torch.cuda.current_stream()
    return lib.sched_paged_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(s.cuda_stream))


@pytest.mark.parametrize("workers,ranged", [(0, False), (97, False), (97, True)])
def test_noalloc_matches_the_workspace_entry_point(lib, workers, ranged):
    for step, (ctx, seed) in enumerate((([16, 3000, 9000, 700, 5000, 1, 2048, 4100], 1),
                                        ([600, 33, 1500], 2))):
        print(f"noalloc step {step} workers {workers} ranged {ranged} ctx {ctx}", flush=True)
        b = _batch(ctx, seed)
        tp = 32
        if ranged:     # 32-page chunks, 7-page ones for the later half of the pages
            tiles = sched_pd.plan_ranges_host(ctx, 16, 8, tile_pages=tp, tail_pages=7,
                                              tail_frac=0.5)
        else:
            tiles = sched_pd.plan_tiles(ctx, 16, tp, 8)
        nt = tiles.shape[0]
        plane = SchedPlane(max_tasks=max(nt, len(ctx) * 8))
        plane.install_order(torch.arange(nt - 1, -1, -1, dtype=torch.int32), nt)
        plane.set_num_tasks(nt if workers else 0)
        plane.push()
        want = torch.full((len(ctx), 32, 128), float("nan"), device="cuda")
        got = torch.full_like(want, float("nan"))
        a = _args(b, want, plane, tiles, tp, workers)
        sched_pd.launch(a)
        a2 = _args(b, got, plane, tiles, tp, workers)
        assert _noalloc(lib, a2) == 0, abi.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        r = oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"])
        assert par_err(got.cpu(), r) <= TOL_BF16


def test_noalloc_without_tiles_and_refusals(lib):
    b = _batch([100, 2000], 3)
    want = torch.empty(2, 32, 128, device="cuda")
    got = torch.empty_like(want)
    sched_pd.launch(_args(b, want, None, None, 0, 0))
    assert _noalloc(lib, _args(b, got, None, None, 0, 0)) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    tiles = sched_pd.plan_tiles([100, 2000], 16, 4, 8)
    a = _args(b, got, None, tiles, 4, 0)
    # a workspace passed in is refused
    assert lib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "no workspace" in abi.last_error()
    # a plan beyond the scratch is refused before any launch
    a.workspace, a.workspace_bytes = None, 0
    a.num_tiles = 1 << 22
    assert lib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "scratch" in abi.last_error() or "holds" in abi.last_error()
