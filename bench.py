"""Benchmark: paged-decode KV-read bandwidth and heterogeneous-batch makespan.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-hetero] [--no-cpu]
                    [--sections hetero,shed,fp8,kv,layouts,pi,trace,fixture,serving]

One step = one decode launch over the Llama-3-8B-shaped bf16 GQA batch (Hq 32,
Hkv 8, d 128, page 16, 64 requests x 2048 tokens, levers null). The pool is
1,048,576 tokens (65,536 pages, 4 GiB of KV); eight block tables over disjoint
pages rotate across steps, so each step reads 512 MiB the previous seven did
not touch and the 256 MB MALL cannot serve a repeated working set. Inputs are
resident in HBM before timing starts.

Printed (rank 0, one JSON line): value = KV-read GB/s of the whole job,
roofline of the decode kernel (algorithmic KV bytes / average kernel time:
HIP events on the launch stream around the timed region of back-to-back
launches, divided by the steps; against 8 TB/s), the heterogeneous-batch
makespan of the static grid and the ticket work queue (W = 2 x CU), two
measured read ceilings (contiguous streaming, and random whole pages -- the
decode's own access pattern -- for one step's bytes), and the CPU
baseline (the oracle's fp32 port of the reference CPU loop, OpenMP, on a
bounded sample, timed on this host). Further sections: the shed/policy and
fp8 configurations, the cache writer, V layouts, and the reference's own
evaluations re-run here (pi makespan through the FlashInfer wrapper, the
serving-trace eval, the heterogeneous-batch fixture).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sched-pass_amd"))

HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--no-hetero", action="store_true",
                   help="headline decode only (same as --sections '')")
    p.add_argument("--sections", default="hetero,shed,fp8,kv,layouts,pi,trace,fixture,serving",
                   help="comma list of the extra measurements: hetero, shed, fp8, kv, "
                        "layouts, pi, trace, fixture, serving")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--tables", type=int, default=8)
    return p.parse_args()


def time_launches(fn, steps, stream):
    """Per-launch HIP event pairs on `stream`; returns (mean kernel ms, list)."""
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        fn(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    return sum(ms) / len(ms), ms


def time_region(fn, steps, stream):
    """Mean ms per launch over `steps` back-to-back launches, one HIP event
    pair on `stream` around the whole run."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def read_ceiling_gbs(torch, sched_pd, buf):
    """Achievable streaming-read bandwidth: the library's read probe over
    `buf` (>= 2 GiB, far beyond the 256 MB MALL); min over 3 repeats of 3
    back-to-back launches per event pair."""
    import ctypes
    import sched_abi
    lib = sched_abi.load_library()
    nbytes = buf.numel() * buf.element_size()
    stream = torch.cuda.current_stream()
    s = ctypes.c_void_p(stream.cuda_stream)
    if lib.sched_pd_read_probe(ctypes.c_void_p(buf.data_ptr()), nbytes, None, s):
        raise RuntimeError(sched_abi.last_error())
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(3):
            lib.sched_pd_read_probe(ctypes.c_void_p(buf.data_ptr()), nbytes, None, s)
        e1.record(stream)
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / 3)
    return nbytes / (best * 1e-3) / 1e9


def random_block_ceiling_gbs(torch, buf, nbytes, block, seed=7, launches=5):
    """Read ceiling for the decode's access pattern: `nbytes` of random
    `block`-byte blocks of `buf` (one step's worth of pages, each a page of
    every kv-head), read by the library's block probe. Min over 3 repeats of
    `launches` back-to-back launches per event pair."""
    import ctypes
    import sched_abi
    lib = sched_abi.load_library()
    total = buf.numel() * buf.element_size()
    g = torch.Generator(device=buf.device).manual_seed(seed)
    ids = torch.randperm(total // block, device=buf.device, generator=g)[:nbytes // block]
    ids = ids.to(torch.int32).contiguous()
    stream = torch.cuda.current_stream()
    s = ctypes.c_void_p(stream.cuda_stream)
    call = lambda: lib.sched_pd_read_probe_blocks(ctypes.c_void_p(buf.data_ptr()), total,  # noqa: E731
                                                  ctypes.c_void_p(ids.data_ptr()), ids.numel(),
                                                  block, None, s)
    if call():
        raise RuntimeError(sched_abi.last_error())
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(launches):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / launches)
    return ids.numel() * block / (best * 1e-3) / 1e9


def bench_uniform(args, torch, sched_pd, workloads):
    b = workloads.workload("llama3_8b_uniform", seed=0, n_tables=args.tables)
    out = torch.empty(64, 32, 128, dtype=torch.bfloat16, device="cuda")
    launches = [sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], bt, b["ctx_lens"], out=out)
                for bt in b["block_tables"]]
    kind = sched_pd.kernel_kind(launches[0])
    stream = torch.cuda.current_stream()
    step = lambda i: sched_pd.launch(launches[i % len(launches)], stream)
    # Inputs resident before timing: every table's pages are read once (the
    # pool was allocated just before, and a table's first read pays ~100 us
    # of first-touch cost), then the W warmup steps.
    for bt_args in launches:
        sched_pd.launch(bt_args, stream)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # The timed region opens behind two queued launches (the two tables
    # before the first timed step's, so no table is read twice in a row): the
    # start event fires while the device is busy and the
    # host is already ahead, so the region holds the timed launches back to
    # back and no idle gap before the first one (a launch queued after a
    # synchronize reaches the device tens of microseconds after its event).
    step(-2)
    step(-1)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = ev0.elapsed_time(ev1)
    kern_ms, per = time_launches(step, args.steps, stream)
    kv = b["kv_bytes"]
    ceiling = read_ceiling_gbs(torch, sched_pd, b["k_pool"])
    page_bytes = b["k_pool"][0].numel() * b["k_pool"].element_size()   # one page, all kv-heads
    ceiling_pages = random_block_ceiling_gbs(torch, b["k_pool"], kv, page_bytes)
    return {
        "kv_bytes": kv, "ms_per_step": wall_ms / args.steps,
        "random_page_ceiling_gbs": ceiling_pages, "page_bytes": page_bytes,
        # the timed region holds only this kernel's launches, queued back to
        # back: its event span / steps is the kernel's average duration (the
        # per-launch event pairs below add their own gaps)
        "kernel_ms": wall_ms / args.steps, "kernel_ms_single": kern_ms,
        "read_ceiling_gbs": ceiling,
        "kernel_ms_min": min(per), "kernel": kind, "occupancy": sched_pd.occupancy(launches[0]),
    }


# Split-KV tiles hold 1 MiB of one kv-head's KV: 128 pages of bf16, 256 of
# fp8 (d 128, page 16). Swept: bf16 32..256 pages, fp8 64..512.
TILE_BYTES = 1 << 20


def tile_pages_for(elem_bytes, page=16, head_dim=128):
    return TILE_BYTES // (page * head_dim * 2 * elem_bytes)


TILE_PAGES = tile_pages_for(2)
# Graded plans for queue launches under an order unrelated to cost (identity,
# urgency): chunks of one kv-head's KV of 1.25 MiB, then 0.5 MiB for the pages
# claimed after the first 90% of the step's, then 128 KiB after 98% (bf16:
# 160 / 64 / 16 pages; fp8: 320 / 128 / 32).
GRADED_BYTES = ((0.0, 5 << 18), (0.9, 1 << 19), (0.98, 1 << 17))


def graded_sizes(elem_bytes):
    """The graded plan's (fraction, chunk pages) levels for a KV element size."""
    per_page = 16 * 128 * 2 * elem_bytes
    return tuple((f, nbytes // per_page) for f, nbytes in GRADED_BYTES)


def _makespan_us(torch, sched_pd, a, stream, reps=5, launches=20):
    """Min over `reps` of the mean of `launches` back-to-back launches (HIP
    events on the launch stream), microseconds."""
    for _ in range(3):
        sched_pd.launch(a, stream)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(launches):
            sched_pd.launch(a, stream)
        e1.record(stream)
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / launches)
    return best * 1000.0


def bench_hetero(torch, sched_pd, workloads, SchedPlane, cu, tile_pages=TILE_PAGES):
    """256 requests, lognormal contexts; pi by a uniform-random urgency per
    task. Static grid (one workgroup per task) against the ticket work queue
    with W = 2 x CU persistent workers; the queue claims split-KV tiles of
    `tile_pages` pages. The other two corners are reported as well, the
    queue with LPT from the timer, and pi alone (longest-first by pages over
    the static grid of tiles); and the queue, pi still by urgency, over a
    graded plan whose chunks are cut smaller the later they are claimed (the
    configuration's queue launch, reported as ticket_wq_us)."""
    import numpy as np
    b = workloads.workload("llama3_8b_hetero", seed=0)
    ntask = 256 * 8
    q = b["urgency"]
    W = 2 * cu
    out = torch.empty(256, 32, 128, dtype=torch.bfloat16, device="cuda")
    tiles = sched_pd.plan_tiles(b["ctx_lens"], 16, tile_pages, 8)
    nt = tiles.shape[0]
    if nt > 16384:
        raise ValueError(f"{nt} tiles exceed the 16384-row plane; use larger tiles")
    p_task = SchedPlane(max_tasks=ntask)
    p_task.install_order(np.argsort(-q, kind="stable").astype(np.int32), ntask)
    p_task.set_num_tasks(ntask)
    p_task.push()
    p_tile = SchedPlane(max_tasks=max(nt, ntask))
    p_tile.install_order(sched_pd.tile_order_by_task_key(tiles, q), nt)
    p_tile.set_num_tasks(nt)
    p_tile.push()
    p_task.reset_queue(W)
    p_tile.reset_queue(W)
    common = dict(out=out)
    A = {
        "static_task": sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                           b["ctx_lens"], plane=p_task, workers=0, **common),
        "wq_task": sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                       b["ctx_lens"], plane=p_task, workers=W, **common),
        "static_tiles": sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                            b["ctx_lens"], plane=p_tile, workers=0, tiles=tiles,
                                            tile_pages=tile_pages, **common),
        "wq_tiles": sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                        b["ctx_lens"], plane=p_tile, workers=W, tiles=tiles,
                                        tile_pages=tile_pages, **common),
    }
    stream = torch.cuda.current_stream()
    res = {k: round(_makespan_us(torch, sched_pd, a, stream), 2) for k, a in A.items()}
    # per-task residency of one work-queue step from the timer rows
    p_tile.clear_timer()
    sched_pd.launch(A["wq_tiles"], stream)
    torch.cuda.synchronize()
    cyc = p_tile.read_timer()[:ntask].numpy()
    # closed loop: pi over tiles by the measured per-task cost, longest first,
    # on tiles of twice the size (with the heaviest work first the tail is
    # short items anyway, and fewer items cost less start-up)
    tp2 = 2 * tile_pages
    tiles2 = sched_pd.plan_tiles(b["ctx_lens"], 16, tp2, 8)
    nt2 = tiles2.shape[0]
    p_lpt = SchedPlane(max_tasks=max(nt2, ntask))
    p_lpt.install_order(sched_pd.tile_order_by_task_key(tiles2, cyc.astype(np.float64)), nt2)
    p_lpt.set_num_tasks(nt2)
    p_lpt.push()
    p_lpt.reset_queue(W)
    a_lpt = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                plane=p_lpt, workers=W, tiles=tiles2, tile_pages=tp2, **common)
    res["wq_tiles_lpt_timer"] = round(_makespan_us(torch, sched_pd, a_lpt, stream), 2)
    # pi alone: the static grid over the 128-page tiles ordered longest-first
    # by the pages each reads (known on the host), no queue
    p_st = SchedPlane(max_tasks=max(nt, ntask))
    p_st.install_order(sched_pd.tile_order_lpt(
        sched_pd.tile_pages_loaded(tiles, b["ctx_lens"], 16, tile_pages, 8)), nt)
    p_st.push()
    a_st = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                               plane=p_st, workers=0, tiles=tiles, tile_pages=tile_pages, **common)
    res["static_tiles_lpt_pages"] = round(_makespan_us(torch, sched_pd, a_st, stream), 2)
    # the queue over the graded plan: pi by urgency as above, chunks cut
    # smaller the later they are claimed (the configuration's queue launch)
    ctx = b["ctx_lens"].cpu().numpy()
    sizes = graded_sizes(2)
    gtiles = sched_pd.plan_graded_host(ctx, 16, 8, task_order=np.argsort(-q, kind="stable"),
                                       sizes=sizes)
    ntg = gtiles.shape[0]
    p_grd = SchedPlane(max_tasks=max(ntg, ntask))
    p_grd.install_order(sched_pd.tile_order_by_task_key(torch.from_numpy(gtiles), q), ntg)
    p_grd.set_num_tasks(ntg)
    p_grd.push()
    p_grd.reset_queue(W)
    a_grd = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                plane=p_grd, workers=W, tiles=gtiles, **common)
    res["wq_graded"] = round(_makespan_us(torch, sched_pd, a_grd, stream), 2)
    # the static grid over the same graded plan and pi: the queue's own part
    p_grd_st = SchedPlane(max_tasks=max(ntg, ntask))
    p_grd_st.install_order(sched_pd.tile_order_by_task_key(gtiles, q), ntg)
    p_grd_st.push()
    a_grd_st = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                   b["ctx_lens"], plane=p_grd_st, workers=0, tiles=gtiles,
                                   **common)
    res["static_graded"] = round(_makespan_us(torch, sched_pd, a_grd_st, stream), 2)
    kv = b["kv_bytes"]

    def cut(a, b_):
        return round(100.0 * (res[a] - res[b_]) / res[a], 2)

    return {
        # the configuration's comparison: the queue (over the graded plan)
        # against the static grid of one workgroup per task, both under pi
        # by urgency; then its two parts, the split alone (static grid over
        # the same plan) and the queue alone over that plan and over tasks
        "static_us": res["static_task"], "ticket_wq_us": res["wq_graded"],
        "queue_plus_split_cut_pct": cut("static_task", "wq_graded"),
        "split_cut_pct": cut("static_task", "static_graded"),
        "queue_cut_pct": cut("static_graded", "wq_graded"),
        "queue_over_tasks_cut_pct": cut("static_task", "wq_task"),
        # the same over 128-page pair tiles
        "pair_tiles": {"queue_plus_split_cut_pct": cut("static_task", "wq_tiles"),
                       "split_cut_pct": cut("static_task", "static_tiles"),
                       "queue_cut_pct": cut("static_tiles", "wq_tiles")},
        "graded_vs_pair_tiles_pct": -cut("wq_tiles", "wq_graded"),
        # orders by cost, for reference: LPT from the timer (queue), LPT by
        # pages on the static grid
        "queue_plus_split_plus_lpt_timer_cut_pct": cut("static_task", "wq_tiles_lpt_timer"),
        "split_plus_lpt_static_cut_pct": cut("static_task", "static_tiles_lpt_pages"),
        "graded_tiles": ntg, "graded_sizes": [list(x) for x in sizes],
        "corners_us": res, "workers": W, "tasks": ntask, "tiles": nt, "tile_pages": tile_pages,
        "lpt_tile_pages": tp2,
        "kv_bytes": kv, "wq_kv_gbs": round(kv / (res["wq_graded"] * 1e-6) / 1e9, 1),
        "residency_cycles": {"p50": int(np.percentile(cyc, 50)),
                             "p99": int(np.percentile(cyc, 99)), "max": int(cyc.max())},
    }


def bench_shed(torch, sched_pd, workloads, SchedPlane, cu, tile_pages=TILE_PAGES):
    """128 requests, ctx ~ U{1024..8192}, per-task tau ~ U{ctx/4..ctx}; policy
    armed (q ~ U(0,1), lambda_bw 0.5, H 0.1: urgent tasks keep pf_dist = 4
    pages in flight per wave); the lever's A/B (firing, priced out, all
    urgent, all polite) on the softmax skip launch. Online softmax (score -> -inf) and linear contraction (value -> 0)
    variants; pages past the budget skipped (default) or loaded and masked
    (the reference weave's behaviour). Work queue over split tiles, pi by
    urgency; the softmax skip launch over a graded plan cut from the pages
    each task reads (no empty work items past the budgets), chunks smaller
    the later they are claimed (and the linear skip launch over the same
    plan); then the skip variants with
    pi = longest-first over tiles of twice the size by the pages each reads
    (known on the host from ctx and tau)."""
    import numpy as np
    import sched_abi as abi
    b = workloads.workload("llama3_8b_shed", seed=0)
    R, ntask = 128, 128 * 8
    ctx = b["ctx_lens"].cpu().numpy()
    tiles = sched_pd.plan_tiles(ctx, 16, tile_pages, 8)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.set_lambda(0.5)
    plane.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    plane.install_order(sched_pd.tile_order_by_task_key(tiles, b["urgency"]), nt)
    plane.set_num_tasks(nt)
    plane.push()
    W = 2 * cu
    plane.reset_queue(W)
    stream = torch.cuda.current_stream()
    full = workloads.kv_bytes(ctx, 8, 128, torch.bfloat16)
    kept = workloads.kv_bytes(ctx, 8, 128, torch.bfloat16, tau=b["tau"][::8])
    res = {"tasks": ntask, "tiles": nt, "urgent_frac": round(float((b["urgency"] > 0.6).mean()), 3),
           "kv_bytes_ctx": full, "kv_bytes_kept": kept}
    out = torch.empty(R, 32, 128, dtype=torch.bfloat16, device="cuda")
    lout = torch.empty(R, 8, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.randn(8192, device="cuda")
    for name, kw, o, vb in (
            ("softmax_skip", {}, out, 1.0),
            ("softmax_shed_loads", {"flags": abi.FLAG_SHED_LOADS}, out, 1.0),
            ("linear_skip", {"mode": abi.LINEAR, "lin_w": w}, lout, 0.5)):
        a = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                out=o, plane=plane, workers=W, tiles=tiles, tile_pages=tile_pages,
                                policy=(1.0, 1.0, 0.1), pf_dist=4, **kw)
        us = _makespan_us(torch, sched_pd, a, stream)
        loaded = (full if "loads" in name else kept) * vb
        res[name] = {"us": round(us, 2), "gbs_loaded": round(loaded / us / 1e3, 1),
                     "gbs_ctx_equiv": round(full * vb / us / 1e3, 1)}
    # the policy lever on the softmax skip launch: the config's pricing fires
    # it (q > lambda_bw + H: urgent tasks keep pf_dist = 4 pages in flight per
    # wave instead of 2), against priced out (lambda_bw = 1000: no task
    # urgent), every task urgent and every task polite. Same bits every time.
    # Per class (the tasks the pricing makes urgent, q > 0.6, and the rest):
    # the timer's residency cycles per page read, summed over each task's
    # tiles and over 5 launches of each variant -- what the action changes
    # is how fast a task streams, which the makespan need not show.
    ab = {}
    base = None
    kept_tok = np.repeat(ctx, 8).astype(np.int64)
    tau_t = np.asarray(b["tau"][:ntask], dtype=np.int64)
    kept_tok = np.where(tau_t > 0, np.minimum(kept_tok, tau_t), kept_tok)
    task_pages = (kept_tok + 15) // 16
    urgent = np.asarray(b["urgency"][:ntask]) > 0.6
    for name, lam, hint in (("firing", 0.5, None), ("priced_out", 1000.0, None),
                            ("all_urgent", 0.5, abi.HINT_URGENT),
                            ("all_polite", 0.5, abi.HINT_POLITE)):
        plane.set_lambda(lam)
        plane.set_rows(q=b["urgency"], tau=b["tau"], hint=np.full(ntask, 0 if hint is None else hint),
                       n=ntask)
        plane.push()
        a = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                b["ctx_lens"], out=out, plane=plane, workers=W, tiles=tiles,
                                tile_pages=tile_pages, policy=(1.0, 1.0, 0.1), pf_dist=4)
        ab[name + "_us"] = round(_makespan_us(torch, sched_pd, a, stream), 2)
        plane.clear_timer()
        for _ in range(5):
            sched_pd.launch(a, stream)
        torch.cuda.synchronize()
        cyc = plane.read_timer()[:ntask].numpy().astype(np.float64) / 5
        for cls, m in (("urgent", urgent), ("other", ~urgent)):
            ab[f"{name}_{cls}_cycles_per_page"] = round(float(cyc[m].sum() / task_pages[m].sum()), 1)
        if base is None:
            base = out.clone()
        elif not torch.equal(out, base):
            raise AssertionError(f"policy {name} changed the output bits")
    plane.set_lambda(0.5)
    plane.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    plane.push()
    ab["bit_exact"] = True
    ab["firing_vs_priced_out_pct"] = round(
        100.0 * (ab["firing_us"] - ab["priced_out_us"]) / ab["priced_out_us"], 2)
    for cls in ("urgent", "other"):
        f_, p_ = ab[f"firing_{cls}_cycles_per_page"], ab[f"priced_out_{cls}_cycles_per_page"]
        ab[f"firing_vs_priced_out_{cls}_cycles_pct"] = round(100.0 * (f_ - p_) / p_, 2)
    res["policy_ab"] = ab
    sizes = graded_sizes(2)
    rtiles = sched_pd.plan_graded_host(ctx, 16, 8, task_order=np.argsort(-b["urgency"],
                                                                          kind="stable"),
                                       sizes=sizes, tau=b["tau"][:ntask])
    ntr = rtiles.shape[0]
    plane_r = SchedPlane(max_tasks=max(ntr, ntask))
    plane_r.set_lambda(0.5)
    plane_r.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    plane_r.install_order(sched_pd.tile_order_by_task_key(torch.from_numpy(rtiles),
                                                          b["urgency"]), ntr)
    plane_r.set_num_tasks(ntr)
    plane_r.push()
    plane_r.reset_queue(W)
    a = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                            out=out, plane=plane_r, workers=W, tiles=rtiles,
                            policy=(1.0, 1.0, 0.1), pf_dist=4)
    us = _makespan_us(torch, sched_pd, a, stream)
    res["softmax_skip_graded"] = {
        "us": round(us, 2), "gbs_loaded": round(kept / us / 1e3, 1),
        "gbs_ctx_equiv": round(full / us / 1e3, 1), "tiles": ntr,
        "graded_sizes": [list(x) for x in sizes],
        "vs_tiles_pct": round(100.0 * (us - res["softmax_skip"]["us"]) / res["softmax_skip"]["us"], 2)}
    sched_pd.launch(a, stream)
    torch.cuda.synchronize()
    if not torch.equal(torch.isfinite(out), torch.ones_like(out, dtype=torch.bool)):
        raise AssertionError("the graded shed launch left non-finite outputs")
    a = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                            out=lout, plane=plane_r, workers=W, tiles=rtiles, mode=abi.LINEAR,
                            lin_w=w, policy=(1.0, 1.0, 0.1), pf_dist=4)
    us = _makespan_us(torch, sched_pd, a, stream)
    res["linear_skip_graded"] = {
        "us": round(us, 2), "gbs_loaded": round(kept * 0.5 / us / 1e3, 1),
        "vs_tiles_pct": round(100.0 * (us - res["linear_skip"]["us"]) / res["linear_skip"]["us"], 2)}
    tp2 = 2 * tile_pages
    tiles2 = sched_pd.plan_tiles(ctx, 16, tp2, 8)
    nt2 = tiles2.shape[0]
    plane2 = SchedPlane(max_tasks=max(nt2, ntask))
    plane2.set_lambda(0.5)
    plane2.set_rows(q=b["urgency"], tau=b["tau"], n=ntask)
    pages = sched_pd.tile_pages_loaded(tiles2, ctx, 16, tp2, 8, tau=b["tau"])
    plane2.install_order(sched_pd.tile_order_lpt(pages), nt2)
    plane2.set_num_tasks(nt2)
    plane2.push()
    plane2.reset_queue(W)
    res["lpt_tile_pages"] = tp2
    for name, kw, o, vb in (("softmax_skip_lpt", {}, out, 1.0),
                            ("linear_skip_lpt", {"mode": abi.LINEAR, "lin_w": w}, lout, 0.5)):
        a = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                out=o, plane=plane2, workers=W, tiles=tiles2, tile_pages=tp2,
                                policy=(1.0, 1.0, 0.1), pf_dist=4, **kw)
        us = _makespan_us(torch, sched_pd, a, stream)
        res[name] = {"us": round(us, 2), "gbs_loaded": round(kept * vb / us / 1e3, 1),
                     "gbs_ctx_equiv": round(full * vb / us / 1e3, 1)}
    return res


def bench_fp8(torch, sched_pd, workloads, SchedPlane, cu, tile_pages=tile_pages_for(1)):
    """Qwen2-7B shape (Hq 28 / Hkv 4), fp8-e4m3fn KV with per-(page, head)
    scales ((K, V) pairs per (page, head)), bf16 Q/out, 512 requests,
    lognormal ctx (median 2048, sigma 1.2, max 16384). The configuration's
    launch: the ticket work queue (identity pi, timer on) over the graded
    plan, chunks cut smaller the later they are claimed; beside it the same
    queue over 256-page pair tiles, the static grid of one workgroup per
    task, the queue with pi over tiles (twice the size) by the timer's
    per-task cycles, longest first, and with pi by the tasks' page counts
    (known before the launch) over tiles three times the size."""
    import numpy as np
    b = workloads.workload("qwen2_7b_fp8", seed=0)
    R, ntask = 512, 512 * 4
    ctx = b["ctx_lens"].cpu().numpy()
    tiles = sched_pd.plan_tiles(ctx, 16, tile_pages, 4)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ntask))
    plane.set_num_tasks(nt)
    plane.push()
    W = 2 * cu
    plane.reset_queue(W)
    out = torch.empty(R, 28, 128, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream()
    a_wq = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                               out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], plane=plane,
                               workers=W, tiles=tiles, tile_pages=tile_pages)
    plane2 = SchedPlane(max_tasks=ntask)
    a_st = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                               out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], plane=plane2)
    us_wq = _makespan_us(torch, sched_pd, a_wq, stream)
    us_st = _makespan_us(torch, sched_pd, a_st, stream)
    plane.clear_timer()
    sched_pd.launch(a_wq, stream)
    torch.cuda.synchronize()
    cyc = plane.read_timer()[:ntask].numpy()
    # closed loop: pi over tiles (twice the size) by the measured per-task
    # cost, longest first
    tp2 = 2 * tile_pages
    tiles2 = sched_pd.plan_tiles(ctx, 16, tp2, 4)
    nt2 = tiles2.shape[0]
    plane3 = SchedPlane(max_tasks=max(nt2, ntask))
    plane3.install_order(sched_pd.tile_order_by_task_key(tiles2, cyc.astype(np.float64)), nt2)
    plane3.set_num_tasks(nt2)
    plane3.push()
    plane3.reset_queue(W)
    a_lpt = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], plane=plane3,
                                workers=W, tiles=tiles2, tile_pages=tp2)
    us_lpt = _makespan_us(torch, sched_pd, a_lpt, stream)
    # open loop: pi by the tasks' page counts, known on the host before the
    # launch (no probe), over 768-page tiles (the best of 256..1024 measured)
    tp3 = 3 * tile_pages
    tiles3 = sched_pd.plan_tiles(ctx, 16, tp3, 4)
    nt3 = tiles3.shape[0]
    plane4 = SchedPlane(max_tasks=max(nt3, ntask))
    task_pages = np.repeat(-(-ctx // 16), 4).astype(np.float64)
    plane4.install_order(sched_pd.tile_order_by_task_key(tiles3, task_pages), nt3)
    plane4.set_num_tasks(nt3)
    plane4.push()
    plane4.reset_queue(W)
    a_len = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], plane=plane4,
                                workers=W, tiles=tiles3, tile_pages=tp3)
    us_len = _makespan_us(torch, sched_pd, a_len, stream)
    sizes = graded_sizes(1)
    rtiles = sched_pd.plan_graded_host(ctx, 16, 4, sizes=sizes)
    ntr = rtiles.shape[0]
    plane5 = SchedPlane(max_tasks=max(ntr, ntask))
    plane5.set_num_tasks(ntr)
    plane5.push()
    plane5.reset_queue(W)
    a_rng = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                                out=out, k_scale=b["k_scale"], v_scale=b["v_scale"], plane=plane5,
                                workers=W, tiles=rtiles)
    us_rng = _makespan_us(torch, sched_pd, a_rng, stream)
    kv = b["kv_bytes"]
    # the configuration's launch (ticket queue, identity pi, timer on) is the
    # queue over the graded plan; the queue over 256-page pair tiles beside it
    return {"kv_bytes": kv, "ticket_wq_us": round(us_rng, 2), "static_task_us": round(us_st, 2),
            "ticket_wq_plan": "graded", "graded_tiles": ntr,
            "graded_sizes": [list(x) for x in sizes],
            "wq_pair_tiles_us": round(us_wq, 2), "gbs_pair_tiles": round(kv / us_wq / 1e3, 1),
            "wq_tiles_lpt_timer_us": round(us_lpt, 2),
            "wq_tiles_lpt_length_us": round(us_len, 2),
            "gbs": round(kv / us_rng / 1e3, 1), "gbs_lpt_timer": round(kv / us_lpt / 1e3, 1),
            "gbs_lpt_length": round(kv / us_len / 1e3, 1), "lpt_length_tile_pages": tp3,
            "tiles": nt, "tile_pages": tile_pages, "lpt_tile_pages": tp2, "workers": W,
            "max_ctx": int(ctx.max()),
            "residency_cycles": {"p50": int(np.percentile(cyc, 50)),
                                 "p99": int(np.percentile(cyc, 99)), "max": int(cyc.max())}}


def bench_kv_append(torch, steps=20):
    """The cache writer (sched_kv_append) on the Llama-3-8B decode shape
    (Hkv 8, d 128, page 16, d-major V), bf16 K/V rows into a bf16 and an fp8
    cache, fp16 rows into an fp16 cache:
      decode_step: one token for each of 64 requests at ragged positions
        (ctx after the append ~ U[1024, 2048]);
      bulk: the whole 64 x 2048-token KV of the uniform batch in one call.
    Bytes per call = source rows read + cache bytes written (+ fp8 scales);
    the d-major V's read-merge of a partial 4-slot group is not counted."""
    import numpy as np
    import kv_cache
    R, T, hkv, d, ps = 64, 2048, 8, 128, 16
    stream = torch.cuda.current_stream()
    g = torch.Generator(device="cuda").manual_seed(5)
    res = {}
    fp8 = torch.float8_e4m3fn
    npg = R * T // ps
    bt = torch.randperm(npg, device="cuda", generator=g).int().view(R, T // ps)
    k_big = torch.randn(R * T, hkv, d, device="cuda", generator=g).bfloat16()
    v_big = torch.randn(R * T, hkv, d, device="cuda", generator=g).bfloat16()
    rng = np.random.default_rng(5)
    ctx_step = torch.from_numpy(rng.integers(1024, 2049, R).astype(np.int32)).cuda()
    k1, v1 = k_big[:R].contiguous(), v_big[:R].contiguous()
    app_step = torch.arange(R + 1, dtype=torch.int32, device="cuda")
    app_bulk = torch.arange(0, R * T + 1, T, dtype=torch.int32, device="cuda")
    ctx_bulk = torch.full((R,), T, dtype=torch.int32, device="cuda")
    for name, dt in (("bf16", torch.bfloat16), ("fp8", fp8), ("fp16", torch.float16)):
        if dt == torch.float16:
            k_big, v_big = k_big.half(), v_big.half()
            k1, v1 = k_big[:R].contiguous(), v_big[:R].contiguous()
        kp = torch.zeros(npg, hkv, ps, d, dtype=dt, device="cuda")
        vp = torch.zeros(npg, hkv, d, ps, dtype=dt, device="cuda")
        ks = vs = None
        if dt == fp8:
            ks = torch.zeros(npg * hkv, device="cuda")
            vs = torch.zeros_like(ks)
        esz = kp.element_size()
        scale_b = 0 if ks is None else 2 * 4
        for label, src_k, src_v, app, ctx, ntok, max_app in (
                ("bulk", k_big, v_big, app_bulk, ctx_bulk, R * T, T),
                ("decode_step", k1, v1, app_step, ctx_step, R, 1)):
            a = kv_cache.build_append_args(src_k, src_v, app, ctx, kp, vp, bt, k_scale=ks,
                                           v_scale=vs, max_append=max_app)
            step = lambda i: kv_cache.launch_append(a, stream)  # noqa: E731
            for i in range(3):
                step(i)
            torch.cuda.synchronize()
            ms = time_region(step, steps, stream)
            _, per = time_launches(step, steps, stream)
            pages_touched = R * hkv * (-(-max_app // ps))
            nbytes = ntok * hkv * d * 2 * (2 + esz) + pages_touched * scale_b
            res[f"{label}_{name}"] = {"us": round(ms * 1e3, 2),
                                      "single_launch_events_min_us": round(min(per) * 1e3, 2),
                                      "bytes": nbytes,
                                      "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                      "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9
                                                             / HBM_PEAK_GBS, 4)}
        del kp, vp, ks, vs
    return res


def profiled_traffic():
    """HBM bytes per decode launch from the committed PMC summary (two
    rocprofv3 --pmc runs, FETCH_SIZE calibrated on the read probe), or None."""
    import re
    path = os.path.join(ROOT, "profiles", "decode_mfma_llama3_8b_uniform_pmc.md")
    try:
        m = re.search(r"^traffic_bytes_per_launch: (\d+)$", open(path).read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def profiled_mfma_busy():
    """MFMA busy % of the C2 decode kernel from the committed counter summary
    (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs), or None."""
    import re
    path = os.path.join(ROOT, "profiles", "decode_mfma_busy.md")
    try:
        m = re.search(r"^mfma_busy_pct_c2: ([0-9.]+)$", open(path).read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def bench_layouts(torch, sched_pd, workloads, tables=4):
    """The uniform step's batch (64 x 2048, bf16, Hq 32 / Hkv 8) with V stored
    token-major: HND pages [P, Hkv, 16, 128] and FlashInfer's NHD cache
    [P, 2, 16, Hkv, 128] read in place; the same values as the d-major
    layout, rotating `tables` block tables. Then a serving step (the writer
    appends one token per request, then the decode) on each 16-token-page V
    layout, and the MFMA against the VALU kernel at 1, 2 and 4 q-heads per
    kv-head."""
    import kv_cache
    import sched_abi as abi
    R, T, hkv, hq, d, ps = 64, 2048, 8, 32, 128, 16
    npg = R * T // ps * tables
    g = torch.Generator(device="cuda").manual_seed(11)
    q = (torch.randn(R, hq, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    ctx = torch.full((R,), T, dtype=torch.int32, device="cuda")
    out = torch.empty(R, hq, d, dtype=torch.bfloat16, device="cuda")
    perm = torch.randperm(npg, device="cuda", generator=g).int()
    bts = [perm[i * (npg // tables):(i + 1) * (npg // tables)].view(R, T // ps).contiguous()
           for i in range(tables)]
    kv_bytes = R * T * hkv * d * 2 * 2
    stream = torch.cuda.current_stream()

    def measure(k_pool, v_pool, layout):
        args = [sched_pd.build_args(q, k_pool, v_pool, bt, ctx, out=out, v_layout=layout)
                for bt in bts]
        f = lambda i: sched_pd.launch(args[i % tables], stream)  # noqa: E731
        for i in range(2 * tables):
            f(i)
        torch.cuda.synchronize()
        ms = min(time_region(f, 20, stream) for _ in range(3))
        return {"us": round(ms * 1e3, 2), "gbs": round(kv_bytes / ms / 1e6, 1),
                "kernel": sched_pd.kernel_kind(args[0])}

    def serving_step(k_pool, v_pool, layout, k_scale=None, v_scale=None):
        # one decode step of a server: append each request's new token
        # (position 2047, the cache writer), then decode all 2048 tokens
        k1 = (torch.randn(R, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
        v1 = (torch.randn(R, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
        app = torch.arange(R + 1, dtype=torch.int32, device="cuda")
        ins = [kv_cache.build_append_args(k1, v1, app, ctx, k_pool, v_pool, bt, v_layout=layout,
                                          k_scale=k_scale, v_scale=v_scale, max_append=1)
               for bt in bts]
        dec = [sched_pd.build_args(q, k_pool, v_pool, bt, ctx, out=out, v_layout=layout,
                                   k_scale=k_scale, v_scale=v_scale) for bt in bts]
        fa = lambda i: kv_cache.launch_append(ins[i % tables], stream)  # noqa: E731
        fd = lambda i: sched_pd.launch(dec[i % tables], stream)  # noqa: E731

        def both(i):
            fa(i)
            fd(i)
        for i in range(2 * tables):
            both(i)
        torch.cuda.synchronize()
        out_ = {}
        for name, f in (("append", fa), ("decode", fd), ("step", both)):
            out_[name + "_us"] = round(min(time_region(f, 20, stream) for _ in range(3)) * 1e3, 2)
        if layout == "tokmajor" and k_pool.dtype in (torch.bfloat16, torch.float16,
                                                     torch.float8_e4m3fn):
            # the same step as one launch (the decode writes the token first;
            # fp8: its page's scale grown as the writer grows it)
            ff = lambda i: sched_pd.launch_with_append(dec[i % tables], ins[i % tables],  # noqa: E731
                                                       stream)
            for i in range(2 * tables):
                ff(i)
            torch.cuda.synchronize()
            out_["fused_step_us"] = round(min(time_region(ff, 20, stream) for _ in range(3)) * 1e3,
                                          2)
        return out_

    res = {}
    kp = (torch.randn(npg, hkv, ps, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    vp = (torch.randn(npg, hkv, ps, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    res["hnd_token_major_v"] = measure(kp, vp, "tokmajor")
    res["hnd_d_major_v"] = measure(kp, vp.view(npg, hkv, d, ps), "dmajor")
    # 16-token pages: the layout a serving step (append + decode) runs faster on
    st = {"token_major_v": serving_step(kp, vp, "tokmajor"),
          "d_major_v": serving_step(kp, vp.view(npg, hkv, d, ps), "dmajor")}
    st["faster"] = min(("token_major_v", "d_major_v"), key=lambda k: st[k]["step_us"])
    st["paged_kv_cache_default"] = kv_cache.PagedKvCache(1, hkv, d, 16, dtype=torch.bfloat16,
                                                         device="cuda").v_layout
    res["serving_step_page16"] = st
    # The kernel by q-heads per kv-head (same KV bytes: Hkv 8, bf16 Q): over
    # token-major V the MFMA kernel against the one-wave kernel (the default
    # for the shapes the MFMA kernel does not take); over d-major V the MFMA
    # kernel against the general VALU kernel
    grp = {}
    for G in (1, 2, 3, 4):
        qg = (torch.randn(R, 8 * G, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
        og = torch.empty(R, 8 * G, d, dtype=torch.bfloat16, device="cuda")
        row = {}
        for name, vpool, layout, flags in (
                ("tokmajor_mfma", vp, "tokmajor", abi.FLAG_NO_WAVE),
                ("tokmajor_wave", vp, "tokmajor", abi.FLAG_NO_MFMA),
                ("dmajor_mfma", vp.view(npg, hkv, d, ps), "dmajor", 0),
                ("dmajor_valu", vp.view(npg, hkv, d, ps), "dmajor", abi.FLAG_FORCE_VALU)):
            args = [sched_pd.build_args(qg, kp, vpool, bt, ctx, out=og, v_layout=layout,
                                        flags=flags) for bt in bts]
            kind = sched_pd.kernel_kind(args[0])
            if name.endswith("wave") and kind != "wave":
                continue                     # G = 4: the one-wave kernel stops at 3
            f = lambda i: sched_pd.launch(args[i % tables], stream)  # noqa: E731
            for i in range(2 * tables):
                f(i)
            torch.cuda.synchronize()
            row[name + "_us"] = round(min(time_region(f, 20, stream) for _ in range(3)) * 1e3, 2)
        for layout, vpool in (("tokmajor", vp), ("dmajor", vp.view(npg, hkv, d, ps))):
            row[layout + "_default"] = sched_pd.kernel_kind(sched_pd.build_args(
                qg, kp, vpool, bts[0], ctx, out=og, v_layout=layout))
        if "tokmajor_wave_us" in row:
            row["wave_vs_mfma_pct"] = round(
                100.0 * (row["tokmajor_wave_us"] - row["tokmajor_mfma_us"]) /
                row["tokmajor_mfma_us"], 2)
        grp[f"G{G}"] = row
    res["kernel_by_group"] = grp
    del kp, vp
    torch.cuda.empty_cache()
    # the same serving step over an fp8 cache (per-(page, head) scales)
    f8 = torch.float8_e4m3fn
    kp8 = torch.randn(npg, hkv, ps, d, device="cuda", generator=g).to(f8)
    vp8 = torch.randn(npg, hkv, ps, d, device="cuda", generator=g).to(f8)
    ks = torch.rand(npg * hkv, device="cuda", generator=g) * 0.09 + 0.01
    vs = torch.rand(npg * hkv, device="cuda", generator=g) * 0.09 + 0.01
    st8 = {"token_major_v": serving_step(kp8, vp8, "tokmajor", ks, vs),
           "d_major_v": serving_step(kp8, vp8.view(npg, hkv, d, ps), "dmajor", ks, vs)}
    st8["faster"] = min(("token_major_v", "d_major_v"), key=lambda k: st8[k]["step_us"])
    st8["paged_kv_cache_default"] = kv_cache.PagedKvCache(1, hkv, d, 16, dtype=f8,
                                                          device="cuda").v_layout
    res["serving_step_page16_fp8"] = st8
    del kp8, vp8, ks, vs
    torch.cuda.empty_cache()
    nhd = (torch.randn(npg, 2, ps, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    kview, vview = kv_cache.nhd_views(nhd)
    res["flashinfer_nhd_in_place"] = measure(kview, vview, "tokmajor")
    del nhd, kview, vview
    torch.cuda.empty_cache()
    res["kv_bytes"] = kv_bytes
    return res


def bench_pi_makespan(torch, sched_pd, batch_sizes=(256, 1024, 4096, 8192)):
    """The reference's isolated pi-makespan evaluation (test/py/
    eval_pi_makespan.py:31-130) through FlashInfer's wrapper calls: Qwen-3B
    GQA decode (Hq 16 / Hkv 2, d 128, page 16), fp16 Q and NHD cache, pages
    per request ~ exp(N(2.6, 1.1)) clipped to [1, 512], static grid; pi
    identity, longest-first and shortest-first by pages (over (request,
    kv-head) tasks). Min over 5 repeats of the mean of 20 launches."""
    import numpy as np
    from flashinfer_compat import BatchDecodeWithPagedKVCacheWrapper
    from sched_rt import SchedPlane
    page, hd, nqo, nkv = 16, 128, 16, 2
    gen = torch.Generator().manual_seed(1)
    stream = torch.cuda.current_stream()
    res = {}
    for bs in batch_sizes:
        pages = torch.exp(torch.normal(2.6, 1.1, (bs,), generator=gen)).clamp(1, 512).to(
            torch.int32)
        npages = int(pages.sum())
        indptr = torch.zeros(bs + 1, dtype=torch.int32)
        indptr[1:] = torch.cumsum(pages, 0)
        indptr = indptr.cuda()
        indices = torch.arange(npages, dtype=torch.int32, device="cuda")
        last = torch.full((bs,), page, dtype=torch.int32, device="cuda")
        q = torch.randn(bs, nqo, hd, dtype=torch.float16, device="cuda")
        kv = torch.randn(npages, 2, page, nkv, hd, dtype=torch.float16, device="cuda")
        ntask = bs * nkv
        plane = SchedPlane(max_tasks=ntask)
        w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD", plane=plane)
        w.plan(indptr, indices, last, nqo, nkv, hd, page, data_type=torch.float16,
               q_data_type=torch.float16)
        out = torch.empty(bs, nqo, hd, dtype=torch.float16, device="cuda")
        args = sched_pd.build_args(q, *w._views(kv), indices, w._plan["ctx"], out=out,
                                   page_indptr=indptr, v_layout="tokmajor", plane=plane)
        cost = np.repeat(pages.numpy().astype(np.float64), nkv)
        orders = {"identity": None,
                  "lpt": np.argsort(-cost, kind="stable").astype(np.int32),
                  "spt": np.argsort(cost, kind="stable").astype(np.int32)}
        row = {}
        for name, order in orders.items():
            if order is None:
                plane.reset_order()
                plane.set_order_size(0)
            else:
                plane.install_order(order, ntask)
            plane.push()
            row[name] = round(_makespan_us(torch, sched_pd, args, stream), 2)
        if bs == batch_sizes[-1]:
            # the residency timer's cost (reference ROADMAP.md:1481-1488):
            # identity order, timer rows off against on (device rows)
            plane.reset_order()
            plane.set_order_size(0)
            for name, on in (("timer_off", False), ("timer_on", True)):
                plane.set_timer_enabled(on)
                plane.push()
                row[name] = round(_makespan_us(torch, sched_pd, args, stream), 2)
            row["timer_cost_pct"] = round(
                100 * (row["timer_on"] - row["timer_off"]) / row["timer_off"], 2)
        row["lpt_vs_identity_pct"] = round(100 * (row["lpt"] - row["identity"]) / row["identity"], 2)
        row["spt_vs_identity_pct"] = round(100 * (row["spt"] - row["identity"]) / row["identity"], 2)
        row["kv_bytes"] = npages * page * nkv * hd * 2 * 2
        row["gbs_lpt"] = round(row["kv_bytes"] / row["lpt"] / 1e3, 1)
        res[str(bs)] = row
        del q, kv, out, plane, w, args
        torch.cuda.empty_cache()
    return res


# Split work items of the serving-trace eval's one-wave steps: 4 pages of 32
# tokens (32 KiB of fp32 K and V), about two of a wave's rings in flight
# (swept 3..12 pages: 4-6 best at 8192 requests, 3-4 at 256).
SPLIT_PAGES = 4


def bench_trace_eval(torch, sched_pd, batch_sizes=(256, 2048, 8192), steps=30):
    """The reference's serving-trace evaluation (test/py/eval_trace.py:36-160,
    published at README.md:95-118): NSEQ requests of one fp32 head (d 32)
    over 32-token [token][K | V] pages -- the JIT launcher's fixture format,
    python/kernels/paged_softmax.cu -- 10% long with 24 pages, the rest 3,
    pages packed in request order; one task per request, static grid.
    Every step is the reference's launcher, launch_paged_softmax, as the
    eval calls it: stock with the library's __sched_* slots empty, the
    policies with a SchedPlane of NSEQ rows bound into them
    (SchedPlane.bind_launcher; 8192 rows at the largest size, twice the C
    runtime's own table). Policies: identity, sorted ascending (longs
    last), LPT from the true lengths, and LPT from the previous step's
    timer rows (closed loop: one identity step fills the rows). Each policy
    runs `steps` steps, each timed alone with events (as the reference
    does); mean and min per policy, outputs bit-exact against identity, and
    the bound launcher bit-exact against the same plane passed in the
    argument block. The regime map repeats identity against the closed loop
    at every batch size. Then the same steps over split work items (a pair
    plan of SPLIT_PAGES pages, static grid, through the argument block):
    stock, identity and LPT over the items from the timer, at every size."""
    import ctypes

    import numpy as np
    import sched_abi as abi
    from sched_rt import SchedPlane
    SD, PT, NS, NL, PAD = 32, 32, 3, 24, 4096
    stream = torch.cuda.current_stream()
    lib = abi.load_library()

    def step_ms(a):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        a()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    res = {"regime_lpt_timer_vs_identity_pct": {}, "regime_split_lpt_timer_vs_identity_pct": {},
           "regime_split_identity_vs_identity_pct": {}, "split_pages": SPLIT_PAGES,
           "step_us": {}}
    for nseq in batch_sizes:
        gen = torch.Generator().manual_seed(0)
        is_long = torch.rand(nseq, generator=gen) < 0.1
        nbl_h = torch.where(is_long, NL, NS).to(torch.int32)
        npages = int(nbl_h.sum())
        bt = torch.zeros(nseq, NL, dtype=torch.int32)
        starts = torch.cumsum(nbl_h, 0) - nbl_h
        for r in range(nseq):
            bt[r, :nbl_h[r]] = torch.arange(int(starts[r]), int(starts[r]) + int(nbl_h[r]),
                                            dtype=torch.int32)
        bt, nbl = bt.cuda(), nbl_h.cuda()
        kv = torch.randn(npages * PT * 2 * SD + PAD, device="cuda")
        pages = kv[:npages * PT * 2 * SD].view(npages, 1, PT, 2 * SD)
        q = torch.randn(nseq, 1, SD, device="cuda")
        out = torch.zeros(nseq, 1, SD, device="cuda")
        common = dict(out=out, v_layout="tokmajor", sm_scale=0.125, tau_scope=abi.TAU_PER_PAGE,
                      flags=abi.FLAG_CTX_IN_PAGES)
        k_view, v_view = pages[..., :SD], pages[..., SD:]
        plane = SchedPlane(max_tasks=nseq)
        plane.set_num_tasks(0)
        plane.set_timer_enabled(True)
        plane.push()
        stock = sched_pd.build_args(q, k_view, v_view, bt, nbl, **common)
        by_args = sched_pd.build_args(q, k_view, v_view, bt, nbl, plane=plane, **common)
        s_ptr = ctypes.c_void_p(stream.cuda_stream)
        launcher = lambda: lib.launch_paged_softmax(  # noqa: E731
            kv.data_ptr(), bt.data_ptr(), nbl.data_ptr(), q.data_ptr(), out.data_ptr(),
            nseq, NL, PT, s_ptr)
        lengths = nbl_h.numpy()
        orders = {"identity": None,
                  "sorted_ascending": np.argsort(lengths, kind="stable").astype(np.int32),
                  "lpt_oracle": np.argsort(-lengths, kind="stable").astype(np.int32),
                  "lpt_timer": "timer"}
        row, golden, exact = {}, None, True
        lib.sched_rt_disarm()
        if nseq == batch_sizes[-1]:
            for _ in range(5):
                launcher()
            t = [step_ms(launcher) for _ in range(steps)]
            row["stock"] = {"mean_us": round(1e3 * float(np.mean(t)), 2),
                            "min_us": round(1e3 * min(t), 2), "kernel": sched_pd.kernel_kind(stock)}
            # the same step on the general VALU kernel (one workgroup per task)
            gen = sched_pd.build_args(q, k_view, v_view, bt, nbl,
                                      **dict(common, flags=common["flags"] | abi.FLAG_NO_WAVE))
            for _ in range(3):
                sched_pd.launch(gen, stream)
            t = [step_ms(lambda: sched_pd.launch(gen, stream)) for _ in range(steps)]
            row["stock_general_kernel"] = {"mean_us": round(1e3 * float(np.mean(t)), 2),
                                           "min_us": round(1e3 * min(t), 2)}
        plane.bind_launcher()
        for _ in range(5):
            launcher()
        # the bound launcher and the argument-block path run the same kernel
        # over the same tables
        launcher()
        torch.cuda.synchronize()
        o_launcher = out.clone()
        sched_pd.launch(by_args, stream)
        torch.cuda.synchronize()
        res.setdefault("launcher_bit_exact_vs_args_path", True)
        res["launcher_bit_exact_vs_args_path"] &= bool(torch.equal(out, o_launcher))
        armed = launcher
        for name, order in orders.items():
            if nseq != batch_sizes[-1] and name not in ("identity", "lpt_timer"):
                continue
            if order is None:
                plane.reset_order()
            elif isinstance(order, str):
                plane.reset_order()
                plane.clear_timer()
                armed()
                torch.cuda.synchronize()
                cyc = plane.read_timer()[:nseq].cpu().numpy()
                order = np.argsort(-cyc, kind="stable").astype(np.int32)
                nlong = int(is_long.sum())
                row["timer_top_are_long_pct"] = round(
                    100.0 * float(is_long.numpy()[order[:nlong]].mean()), 1)
                plane.install_order(order, nseq)
            else:
                plane.install_order(order, nseq)
            plane.push()
            plane.clear_timer()
            t = [step_ms(armed) for _ in range(steps)]
            if nseq == batch_sizes[-1]:
                # per-request residency of this policy's steps (timer rows,
                # averaged over the steps): the tail the order has to hide
                rows_ = plane.read_timer()[:nseq].cpu().numpy() / steps
                row.setdefault("residency_cycles", {})[name] = _residency(rows_, is_long)
            o = out.clone()
            if golden is None:
                golden = o
            else:
                exact = exact and bool(torch.equal(o, golden))
            row[name] = {"mean_us": round(1e3 * float(np.mean(t)), 2),
                         "min_us": round(1e3 * min(t), 2)}
        base = row["identity"]["mean_us"]
        gain = round(100 * (row["lpt_timer"]["mean_us"] - base) / base, 2)
        res["regime_lpt_timer_vs_identity_pct"][str(nseq)] = gain
        res["step_us"][str(nseq)] = {"identity": row["identity"]["mean_us"],
                                     "lpt_timer": row["lpt_timer"]["mean_us"]}
        # the same step over split work items (a pair plan of SPLIT_PAGES
        # pages, static grid; one wave per item), through the argument block:
        # stock (no lever tables), and pi (identity, LPT over the items by
        # the identity step's timer rows) from the plane, bit-exact between
        # them
        plane.unbind_launcher()
        lens_tok = nbl_h.numpy().astype(np.int64) * PT
        tiles = sched_pd.plan_tiles_host(lens_tok, PT, SPLIT_PAGES, 1)
        nti = tiles.shape[0]
        split = {}
        a_split = sched_pd.build_args(q, k_view, v_view, bt, nbl, tiles=tiles,
                                      tile_pages=SPLIT_PAGES, **common)
        for _ in range(3):
            sched_pd.launch(a_split, stream)
        t = [step_ms(lambda: sched_pd.launch(a_split, stream)) for _ in range(steps)]
        split["stock"] = {"mean_us": round(1e3 * float(np.mean(t)), 2),
                          "min_us": round(1e3 * min(t), 2)}
        o_split = out.clone()
        p_items = SchedPlane(max_tasks=max(nti, nseq))
        p_items.set_num_tasks(0)
        p_items.push()
        a_items = sched_pd.build_args(q, k_view, v_view, bt, nbl, tiles=tiles,
                                      tile_pages=SPLIT_PAGES, plane=p_items, **common)
        for name in ("identity", "lpt_timer"):
            if name == "lpt_timer":
                # closed loop: one identity step fills the per-request rows
                p_items.clear_timer()
                sched_pd.launch(a_items, stream)
                torch.cuda.synchronize()
                cyc = p_items.read_timer()[:nseq].cpu().numpy().astype(np.float64)
                p_items.install_order(sched_pd.tile_order_by_task_key(tiles, cyc), nti)
                p_items.push()
            for _ in range(3):
                sched_pd.launch(a_items, stream)
            p_items.clear_timer()
            t = [step_ms(lambda: sched_pd.launch(a_items, stream)) for _ in range(steps)]
            if nseq == batch_sizes[-1]:
                rows_ = p_items.read_timer()[:nseq].cpu().numpy() / steps
                split.setdefault("residency_cycles", {})[name] = _residency(rows_, is_long)
            split[name] = {"mean_us": round(1e3 * float(np.mean(t)), 2),
                           "min_us": round(1e3 * min(t), 2)}
            exact = exact and bool(torch.equal(out, o_split))
        sb = split["identity"]["mean_us"]
        res["regime_split_lpt_timer_vs_identity_pct"][str(nseq)] = round(
            100 * (split["lpt_timer"]["mean_us"] - sb) / sb, 2)
        res["regime_split_identity_vs_identity_pct"][str(nseq)] = round(
            100 * (sb - base) / base, 2)
        split["items"] = nti
        if nseq == batch_sizes[-1]:
            row["split"] = split
        if nseq == batch_sizes[-1]:
            for name in ("sorted_ascending", "lpt_oracle", "lpt_timer"):
                row[name]["vs_identity_pct"] = round(
                    100 * (row[name]["mean_us"] - base) / base, 2)
            st = row["stock"]["mean_us"]
            for name in ("identity", "sorted_ascending", "lpt_oracle", "lpt_timer"):
                row[name]["vs_stock_pct"] = round(100 * (row[name]["mean_us"] - st) / st, 2)
            row["kv_bytes"] = npages * PT * 2 * SD * 4
            for name in ("stock", "stock_general_kernel", "lpt_timer"):
                gbs = row["kv_bytes"] / row[name]["mean_us"] / 1e3
                row[name]["gbs"] = round(gbs, 1)
                row[name]["frac_hbm_peak"] = round(gbs / HBM_PEAK_GBS, 4)
            for name in ("stock", "identity", "lpt_timer"):
                gbs = row["kv_bytes"] / row["split"][name]["mean_us"] / 1e3
                row["split"][name]["gbs"] = round(gbs, 1)
                row["split"][name]["frac_hbm_peak"] = round(gbs / HBM_PEAK_GBS, 4)
            res[str(nseq)] = row
        res.setdefault("bit_exact_vs_identity", True)
        res["bit_exact_vs_identity"] = res["bit_exact_vs_identity"] and exact
        del kv, pages, q, out, plane, stock, armed, by_args, launcher, a_split, a_items, p_items
        torch.cuda.empty_cache()
    return res


def _residency(rows, is_long):
    """Percentiles of per-request residency (timer rows: the cycles a
    request's work items were resident, summed over its items) for the
    short and the long requests of the trace eval."""
    import numpy as np
    rows = np.asarray(rows, np.float64)
    lng = np.asarray(is_long, bool)
    out = {}
    for label, sel in (("short", ~lng), ("long", lng)):
        x = rows[sel]
        out[label] = {"p50": int(np.percentile(x, 50)), "p90": int(np.percentile(x, 90)),
                      "max": int(x.max())}
    return out


def _lcg_uniform(n, seed):
    """n draws of the reference fixtures' generator (s = s*1664525 +
    1013904223 mod 2^32, value ((s >> 8) & 0xffff) / 65536 - 0.5; test/
    hetero_batch.cu:104-108), vectorised: within a block of B steps,
    s_(k+j) = A_j s_k + C_j mod 2^32 with A_j, C_j the j-step affine map."""
    import numpy as np
    a, c, m, B = 1664525, 1013904223, (1 << 32) - 1, 4096
    A = np.empty(B, np.uint64)
    C = np.empty(B, np.uint64)
    x, y = 1, 0
    for j in range(B):           # the (j + 1)-step map
        x, y = (x * a) & m, (y * a + c) & m
        A[j], C[j] = x, y
    out = np.empty(n, np.float32)
    s = seed
    for k in range(0, n, B):
        st = (A * np.uint64(s) + C) & np.uint64(m)
        w = min(B, n - k)
        out[k:k + w] = ((st[:w] >> np.uint64(8)) & np.uint64(0xFFFF)).astype(np.float32) \
            / 65536.0 - 0.5
        s = int(st[B - 1])
    return out


def bench_fixture_hetero(torch, sched_pd, iters=100):
    """The reference's heterogeneous-batch fixture (test/hetero_batch.cu:
    34-330, published at README.md:135-138): the linear contraction over
    fp32 pages of 64 tokens x d 128 (weights indexed by token-in-page), 64
    tasks -- every 8th long with 32 pages, the rest 4 -- on the fixture's own
    LCG inputs (seed 777) and page map. Levers come from the C runtime's
    slots (sched_rt_*), as the fixture arms them: static grid unarmed, then
    the ticket queue with W = 16 workers under identity, longs last, LPT from
    one profiling step's timer rows, LPT + cache hints (longs polite, shorts
    urgent) and longs last + hints; and the LPT order on the static grid
    (claim loop off). Mean of `iters` back-to-back launches each; every
    schedule bit-exact against the static grid."""
    import ctypes
    import numpy as np
    import sched_abi as abi
    lib = abi.load_library()
    NSEQ, D, PT, LONGB, SHORTB, W, PAD = 64, 128, 64, 32, 4, 16, 8192
    npages = NSEQ * LONGB
    n = npages * PT * D + PAD + PT
    vals = _lcg_uniform(n, 777)   # the fixture's generator: kv first, then w
    kv = torch.from_numpy(vals[:npages * PT * D + PAD]).cuda()
    w = torch.from_numpy(vals[npages * PT * D + PAD:]).cuda()
    is_long = np.arange(NSEQ) % 8 == 0
    nbl = torch.from_numpy(np.where(is_long, LONGB, SHORTB).astype(np.int32)).cuda()
    bt = torch.tensor([[(t * LONGB + b * 17 + 5) % npages for b in range(LONGB)]
                       for t in range(NSEQ)], dtype=torch.int32).cuda()
    v_pool = kv[:npages * PT * D].view(npages, 1, PT, D)
    out = torch.zeros(NSEQ, 1, D, device="cuda")
    common = dict(out=out, mode=abi.LINEAR, v_layout="tokmajor", lin_w=w, lin_w_period=PT,
                  flags=abi.FLAG_CTX_IN_PAGES)
    stream = torch.cuda.current_stream()
    static = sched_pd.build_args(None, None, v_pool, bt, nbl, **common)
    queue = sched_pd.build_args(None, None, v_pool, bt, nbl, rt_tables=True, workers=W, **common)
    static_pi = sched_pd.build_args(None, None, v_pool, bt, nbl, rt_tables=True, **common)

    def mean_us(a):
        for _ in range(3):
            sched_pd.launch(a, stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iters):
            sched_pd.launch(a, stream)
        e1.record(stream)
        torch.cuda.synchronize()
        return round(1e3 * e0.elapsed_time(e1) / iters, 2)

    def set_order(tasks):
        order = np.arange(abi.SCHED_MAX_TASKS, dtype=np.int32)
        order[:len(tasks)] = tasks
        assert lib.sched_rt_set_order(order.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                      order.size)

    lib.sched_rt_disarm()
    sched_pd.launch(static, stream)
    torch.cuda.synchronize()
    golden = out.clone()
    res = {"static_us": mean_us(static)}
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(NSEQ)
    assert lib.sched_rt_push_ctrl() and lib.sched_rt_queue_reset(W)
    segregated = np.concatenate([np.flatnonzero(~is_long), np.flatnonzero(is_long)])
    exact = True

    def run(name):
        nonlocal exact
        out.zero_()
        sched_pd.launch(queue, stream)
        torch.cuda.synchronize()
        exact = exact and bool(torch.equal(out, golden))
        res[name + "_us"] = mean_us(queue)

    set_order(np.arange(NSEQ))
    run("identity")
    set_order(segregated)
    run("longs_last")
    lib.sched_rt_timer_clear()
    set_order(np.arange(NSEQ))
    sched_pd.launch(queue, stream)
    torch.cuda.synchronize()
    cyc = np.array([lib.sched_rt_timer(t) for t in range(NSEQ)], np.float64)
    lpt = np.argsort(-cyc, kind="stable").astype(np.int32)
    res["timer_ranks_longs_first"] = bool(is_long[lpt[:8]].all())
    set_order(lpt)
    run("lpt_timer")
    # the same order on the static grid (claim loop off: num_tasks 0)
    lib.sched_rt_set_num_tasks(0)
    assert lib.sched_rt_push_ctrl()
    out.zero_()
    sched_pd.launch(static_pi, stream)
    torch.cuda.synchronize()
    exact = exact and bool(torch.equal(out, golden))
    res["static_lpt_timer_us"] = mean_us(static_pi)
    lib.sched_rt_set_num_tasks(NSEQ)
    assert lib.sched_rt_push_ctrl()
    for t in range(NSEQ):
        lib.sched_rt_set_task(t, 0.0, 0, abi.HINT_POLITE if is_long[t] else abi.HINT_URGENT)
    assert lib.sched_rt_push_ctrl()
    run("lpt_timer_hints")
    set_order(segregated)
    run("longs_last_hints")
    lib.sched_rt_disarm()
    res["bit_exact_vs_static"] = exact
    res["lpt_timer_vs_identity_pct"] = round(
        100 * (res["lpt_timer_us"] - res["identity_us"]) / res["identity_us"], 2)
    res["queue_best_vs_static_pct"] = round(
        100 * (min(res["identity_us"], res["lpt_timer_us"], res["longs_last_us"])
               - res["static_us"]) / res["static_us"], 2)
    res["kv_bytes"] = int(nbl.sum().item()) * PT * D * 4
    return res


def bench_serving(torch, sched_pd, workloads, steps=40, warm=8, reps=3):
    """An engine-style decode loop, the reference's stock / observe / enforce
    A/B of its serving plugin (ROADMAP.md:820-830) without an engine: 256
    requests of the Llama-3-8B shape (bf16, Hq 32 / Hkv 8, page 16) with
    lognormal contexts (median 1024, sigma 1.2); per step the cache writer
    appends one token per request, then the decode runs over 128-page split
    tiles; the step is PagedKvCache.decode_step (the append fused into the
    decode: one launch per step). Modes: stock (the same split plan, no lever
    tables), stock as two launches (the writer, then the decode), the serving
    hooks observing only (bind, probe the timer 1 step in 8, never change the
    schedule), and the hooks enforcing (controller orders, queue arming,
    re-plan every 8 steps; the LPT order over 192-page tiles). Reported per
    mode: wall
    clock per step, GPU time between events around the loop, the host time
    of the plan (stock: the split plan; hooks: begin + end), and the decode
    launches' own GPU time (each step's launch re-run back to back in a
    second pass; for the fused mode the fused launch, which rewrites the
    same token): the last is what the levers change, the plan time is what
    they cost the host. The wall clock is the fastest of `reps` timed runs
    of `steps` steps."""
    import time
    import numpy as np
    import kv_cache
    from sched_rt import SchedPlane
    from serving import HookConfig, ServingHooks
    R, hkv, hq, d, ps, tp = 256, 8, 32, 128, 16, 128
    rng = np.random.default_rng(0)
    lens = workloads.lognormal_ctx(R, 1024, 1.2, 16, 32768, rng)
    grow = (reps + 1) * steps + warm + 1  # tokens one mode appends (each starts over)
    npages = int((-(-(lens + grow) // ps)).sum()) + R
    g = torch.Generator(device="cuda").manual_seed(9)
    cache = kv_cache.PagedKvCache(npages, hkv, d, ps, dtype=torch.bfloat16)
    rids = list(range(R))
    for r in rids:
        cache.add_request(r)
    at = 0
    while at < R:            # prefill in slices (bounded temporaries)
        sl = list(range(at, min(at + 32, R)))
        n = int(lens[sl].sum())
        k = (torch.randn(n, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
        v = (torch.randn(n, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
        cache.append(sl, k, v, lens[sl].tolist())
        at += len(sl)
        del k, v
    q = (torch.randn(R, hq, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    k1 = (torch.randn(R, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    v1 = (torch.randn(R, hkv, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    out = torch.empty(R, hq, d, dtype=torch.bfloat16, device="cuda")
    cu = sched_pd.cu_count()
    bt0, ctx0 = cache.block_table(rids)
    occ = sched_pd.occupancy(sched_pd.build_args(q, cache.k_pool, cache.v_pool, bt0, ctx0,
                                                 out=out, v_layout=cache.v_layout))
    res = {"requests": R, "steps": steps, "tile_pages": tp, "resident": occ * cu}
    stream = torch.cuda.current_stream()
    start = [cache.lens[r] for r in rids]
    for mode in ("stock_two_launches", "stock", "observe", "enforce"):
        cache.truncate(rids, start)       # every mode decodes the same contexts
        hooks = None
        fused = mode != "stock_two_launches"
        if mode in ("observe", "enforce"):
            plane = SchedPlane(max_tasks=16384)
            # the LPT order over 1.5 MiB tiles of one kv-head's KV (192 pages)
            hooks = ServingHooks(plane, hkv, HookConfig(observe_only=mode == "observe",
                                                        tile_pages=tp, lpt_tile_pages=3 * tp // 2,
                                                        resident=occ * cu))

        host = [0.0]
        inflight = []

        def step(ev=None):
            # at most two steps in flight, as an engine that reads a step's
            # sampled tokens one step later keeps (an unbounded run-ahead
            # fills the device queue and stalls in ways no engine sees)
            if len(inflight) >= 2:
                inflight.pop(0).synchronize()
            if not fused:
                cache.append(rids, k1, v1)
            # the plan is built from the lengths the decode will see
            now = cache.lengths(rids) + (1 if fused else 0)
            h0 = time.perf_counter()
            if hooks is None:
                launch = {"tiles": sched_pd.plan_tiles_host(now, ps, tp, hkv), "tile_pages": tp}
            else:
                launch = hooks.on_batch_begin(rids, now)
            host[0] += time.perf_counter() - h0
            if fused:
                cache.decode_step(q, rids, k1, v1, out=out, **launch)
            else:
                cache.decode(q, rids, out=out, **launch)
            h0 = time.perf_counter()
            if hooks is not None:
                hooks.on_batch_end()
            host[0] += time.perf_counter() - h0
            done = torch.cuda.Event()
            done.record(stream)
            inflight.append(done)
            if ev is not None:
                # the step's decode again, 1 + 3 times with the same tables
                # (timer gate already off): the last 3 back to back between
                # the events, so the interval is GPU time, not host time
                bt, ctx = cache.block_table(rids)
                a = sched_pd.build_args(q, cache.k_pool, cache.v_pool, bt, ctx, out=out,
                                        v_layout=cache.v_layout, **launch)
                run = lambda: sched_pd.launch(a)  # noqa: E731
                if fused:
                    # the fused launch rewrites the step's token in place: the
                    # same bytes every time
                    app = kv_cache.build_append_args(
                        k1, v1, torch.arange(R + 1, dtype=torch.int32, device="cuda"), ctx,
                        cache.k_pool, cache.v_pool, bt, v_layout=cache.v_layout, max_append=1)
                    run = lambda: sched_pd.launch_with_append(a, app)  # noqa: E731
                run()
                ev[0].record(stream)
                for _ in range(3):
                    run()
                ev[1].record(stream)
        for _ in range(warm):
            step()
        torch.cuda.synchronize()
        # `reps` timed runs of `steps` steps each, the fastest kept (a host
        # stall of tens of ms, seen once on the box, otherwise sets a run)
        best = None
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            host[0] = 0.0
            t0 = time.perf_counter()
            e0.record(stream)
            for _ in range(steps):
                step()
            e1.record(stream)
            torch.cuda.synchronize()
            run = ((time.perf_counter() - t0) * 1e3 / steps, host[0] * 1e6 / steps,
                   e0.elapsed_time(e1) / steps)
            if best is None or run[0] < best[0]:
                best = run
        wall, plan_us, gpu_ms = best
        # the decode launches alone, per step (a separate pass, so the
        # relaunches do not perturb the wall-clock figure)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        for ev in evs:
            step(ev)
        torch.cuda.synchronize()
        dec = sorted(a.elapsed_time(b) * 1e3 / 3 for a, b in evs)
        res[mode] = {"wall_ms_per_step": round(wall, 3),
                     "gpu_ms_per_step": round(gpu_ms, 3),
                     "tokens_per_s": round(R / (wall * 1e-3), 1),
                     "plan_host_us_per_step": round(plan_us, 1),
                     "decode_us_median": round(dec[len(dec) // 2], 2),
                     "decode_us_mean": round(sum(dec) / len(dec), 2)}
        if hooks is not None:
            res[mode]["probes_folded"] = hooks.probes_folded
            res[mode]["hook_errors"] = hooks.hook_errors
    for mode in ("stock_two_launches", "observe", "enforce"):
        res[mode]["vs_stock_pct"] = round(
            100 * (res[mode]["wall_ms_per_step"] - res["stock"]["wall_ms_per_step"])
            / res["stock"]["wall_ms_per_step"], 2)
        res[mode]["decode_vs_stock_pct"] = round(
            100 * (res[mode]["decode_us_mean"] - res["stock"]["decode_us_mean"])
            / res["stock"]["decode_us_mean"], 2)
    del cache
    torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, workloads):
    """The oracle's fp32 port (the reference CPU loop, OpenMP over tasks) on
    the uniform workload's shape (64 requests x 2048 tokens, a pool of just
    the batch's pages), on all host threads, min of 3 (~10 CPU-seconds);
    plus one thread on 2 of the requests."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    def timed(n_req, threads, reps=3):
        b = workloads.make_batch(np.full(n_req, 2048), num_q_heads=32, num_kv_heads=8, seed=3,
                                 device="cuda")
        host = {k: b[k].cpu() for k in ("q", "k_pool", "v_pool", "block_table", "ctx_lens")}
        del b["k_pool"], b["v_pool"]
        run = lambda: oracle.decode(host["q"], host["k_pool"], host["v_pool"],  # noqa: E731
                                    host["block_table"], host["ctx_lens"],
                                    precision=oracle.F32, threads=threads)
        run()  # warm
        best = float("inf")
        for _ in range(reps):
            t0 = time.perf_counter()
            run()
            best = min(best, time.perf_counter() - t0)
        return b["kv_bytes"], best

    threads = len(os.sched_getaffinity(0))
    kv, best = timed(64, threads)
    kv1, best1 = timed(2, 1)
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(kv / best / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"the whole 64 x 2048-token step (KV {kv >> 20} MiB), fp32 oracle port of "
                      f"the reference CPU loop, {threads} OpenMP threads, min of 3: "
                      f"{best * 1e3:.1f} ms",
            "single_thread_gbs": round(kv1 / best1 / 1e9, 3),
            "single_thread_sample": f"2 of the requests (KV {kv1 >> 20} MiB), 1 thread: "
                                    f"{best1 * 1e3:.1f} ms",
            "cpu_model": cpu}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}); "
              f"the decode path shards by request / kv-head with no exchange between GPUs",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import sched_pd
    import workloads
    from sched_rt import SchedPlane

    torch.cuda.set_device(0)
    cu = sched_pd.cu_count()
    u = bench_uniform(args, torch, sched_pd, workloads)
    gbs = u["kv_bytes"] / (u["ms_per_step"] * 1e-3) / 1e9
    kern_gbs = u["kv_bytes"] / (u["kernel_ms"] * 1e-3) / 1e9
    line = {
        "metric": "paged-decode KV-read GB/s (% HBM peak) + hetero-batch makespan µs",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(u["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1)/sqrt(128) Q/K/V, random page permutation)",
        "config": {"workload": "llama3_8b_uniform", "requests": 64, "ctx": 2048,
                   "q_heads": 32, "kv_heads": 8, "head_dim": 128, "page": 16,
                   "pool_tokens": 1048576, "rotating_tables": args.tables,
                   "levers": "null (stock)", "parallelism": "1 GPU"},
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": f"decode_{u['kernel']}",
                     "kernel_us": round(u["kernel_ms"] * 1e3, 2),
                     "single_launch_events_us": round(u["kernel_ms_single"] * 1e3, 2),
                     "single_launch_events_min_us": round(u["kernel_ms_min"] * 1e3, 2),
                     "bytes_per_launch": u["kv_bytes"], "wg_per_cu": u["occupancy"],
                     "measured_read_ceiling_gbs": round(u["read_ceiling_gbs"], 1),
                     "frac_of_measured_ceiling": round(kern_gbs / u["read_ceiling_gbs"], 4),
                     "measured_random_page_ceiling_gbs": round(u["random_page_ceiling_gbs"], 1),
                     "random_page_bytes": u["page_bytes"],
                     "frac_of_random_page_ceiling": round(kern_gbs / u["random_page_ceiling_gbs"], 4)},
    }
    # counter values are not measured by this run: they are read from the
    # committed rocprofv3 summaries named beside them
    line["roofline"]["traffic"] = profiled_traffic()
    line["roofline"]["traffic_source"] = "profiles/decode_mfma_llama3_8b_uniform_pmc.md"
    line["roofline"]["kernel_trace_source"] = "profiles/decode_mfma_llama3_8b_uniform.md"
    line["roofline"]["mfma_busy_pct"] = profiled_mfma_busy()
    line["roofline"]["mfma_busy_source"] = "profiles/decode_mfma_busy.md"
    sections = set() if args.no_hetero else set(x for x in args.sections.split(",") if x)
    if "hetero" in sections:
        line["hetero_makespan"] = bench_hetero(torch, sched_pd, workloads, SchedPlane, cu)
    if "shed" in sections:
        line["shed_policy"] = bench_shed(torch, sched_pd, workloads, SchedPlane, cu)
    if "fp8" in sections:
        line["fp8_qwen2_7b"] = bench_fp8(torch, sched_pd, workloads, SchedPlane, cu)
    if "pi" in sections:
        line["pi_makespan_flashinfer_shape"] = bench_pi_makespan(torch, sched_pd)
    if "layouts" in sections:
        line["kv_layouts"] = bench_layouts(torch, sched_pd, workloads)
    if "kv" in sections:
        line["kv_append"] = bench_kv_append(torch)
    if "trace" in sections:
        line["trace_eval"] = bench_trace_eval(torch, sched_pd)
    if "fixture" in sections:
        line["fixture_hetero"] = bench_fixture_hetero(torch, sched_pd)
    if "serving" in sections:
        line["serving_loop"] = bench_serving(torch, sched_pd, workloads)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, workloads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
