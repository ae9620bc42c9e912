"""Seeded random decode cases across the launch space against the oracle:
KV type (bf16, fp16, fp8, fp32), head dim, page size, V layout, q-heads per
kv-head, ragged contexts (an empty request included), no plan / pair tiles /
graded ranged rows, per-task prefix budgets. Each case runs twice: with pi
reversed or random and the ticket queue on, and with the identity order on
the static grid; the two are bitwise equal, and the second is held to the
oracle with the same control block."""
import numpy as np
import pytest
import torch

import oracle
import sched_pd
import workloads
from parity import TOL_BF16, TOL_F32, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
KV = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp8": FP8, "fp32": torch.float32}


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    kv = ["bf16", "fp16", "fp8", "fp32"][seed % 4]
    d = int(rng.choice([32, 64, 128])) if kv == "fp32" else int(rng.choice([64, 128]))
    if kv == "fp8":
        d = 128 if rng.uniform() < 0.7 else 64
    ps = int(rng.choice([16, 32, 64]))
    layout = str(rng.choice(["dmajor", "tokmajor"]))
    hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 3, 4, 7]))
    R = int(rng.integers(1, 12))
    ctx = rng.integers(0, 3000, R)
    ctx[rng.uniform(size=R) < 0.15] = 0
    ctx[0] = max(int(ctx[0]), 1)
    plan = str(rng.choice(["none", "pairs", "graded"]))
    return dict(kv=kv, d=d, ps=ps, layout=layout, hkv=hkv, G=G, ctx=ctx.astype(np.int64),
                plan=plan, rng=rng)


@pytest.mark.parametrize("seed", range(40))
def test_random_case_matches_the_oracle_under_every_schedule(seed):
    c = draw(seed)
    kvt = KV[c["kv"]]
    qt = torch.float32 if c["kv"] == "fp32" else torch.float16 if c["kv"] == "fp16" \
        else torch.bfloat16
    hq = c["G"] * c["hkv"]
    print(f"case {seed}: {c['kv']} d{c['d']} page{c['ps']} {c['layout']} Hq{hq} Hkv{c['hkv']} "
          f"plan {c['plan']} ctx {c['ctx'].tolist()}", flush=True)
    b = workloads.make_batch(c["ctx"], num_q_heads=hq, num_kv_heads=c["hkv"], head_dim=c["d"],
                             page_size=c["ps"], kv_dtype=kvt, q_dtype=qt, seed=seed,
                             device="cuda")
    if c["layout"] == "tokmajor":
        b["v_pool"] = b["v_pool"].permute(0, 1, 3, 2).contiguous()
    R, hkv, rng = len(c["ctx"]), c["hkv"], c["rng"]
    ntask = R * hkv
    kw = {}
    if c["plan"] == "pairs":
        tp = int(rng.integers(1, 12))
        kw = dict(tiles=sched_pd.plan_tiles_host(c["ctx"], c["ps"], tp, hkv), tile_pages=tp)
    elif c["plan"] == "graded":
        big = int(rng.integers(2, 24))
        kw = dict(tiles=sched_pd.plan_graded_host(
            c["ctx"], c["ps"], hkv, task_order=rng.permutation(ntask),
            sizes=((0.0, big), (0.6, max(1, big // 3)), (0.9, 1))))
    nitems = kw["tiles"].shape[0] if kw else ntask
    # per-task prefix budgets (0 = none); the plans line up every page
    tau = rng.integers(0, 3000, ntask)
    tau[rng.uniform(size=ntask) < 0.4] = 0
    outs = []
    for schedule in ("shuffled", "identity"):
        plane = SchedPlane(max_tasks=max(nitems, ntask, 64))
        plane.set_rows(tau=tau, n=ntask)
        workers = 0
        if schedule == "shuffled":
            order = np.arange(nitems)[::-1] if seed % 2 else rng.permutation(nitems)
            plane.install_order(torch.from_numpy(order.astype(np.int32)), nitems)
            workers = int(rng.integers(1, 40))
            plane.set_num_tasks(nitems)
        plane.push()
        if workers:
            plane.reset_queue(workers)
        out = torch.full((R, hq, c["d"]), float("nan"), device="cuda")
        sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                              out=out, k_scale=b["k_scale"], v_scale=b["v_scale"],
                              v_layout=c["layout"], plane=plane, workers=workers, **kw)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    a, r = outs
    assert torch.equal(torch.isnan(a), torch.isnan(r)) and \
        torch.equal(torch.nan_to_num(a, nan=3.0), torch.nan_to_num(r, nan=3.0)), "schedule bits"
    ref = oracle.decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"],
                        v_layout=c["layout"], k_scale=b["k_scale"], v_scale=b["v_scale"],
                        ctrl=bytes(plane._ctrl_host), max_tasks=plane.N)
    got = r.numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(got), ~fin)          # empty requests are 0/0
    tol = TOL_F32 if c["kv"] == "fp32" else TOL_BF16
    assert par_err(got[fin], ref[fin], f"case {seed}") <= tol
