"""GPU parity of the decode kernels against the oracle, and bitwise invariance
of every lever that must not change outputs. All launches go through the C ABI
(sched_paged_decode) via sched_pd.build_args/launch."""
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

# par_err <= tol asserts both the mixed form |a-r| <= tol (1 + |r|) and the
# per-row norm-relative error ||a-r|| / ||r|| <= tol (tests/parity.py)




def run(b, plane=None, out_dtype=torch.float32, **kw):
    torch.cuda.synchronize()
    d = b["v_pool"].shape[3 if kw.get("v_layout", "dmajor") == "tokmajor" else 2]
    out = torch.full((b["ctx_lens"].numel(), b["q"].shape[1] if kw.get("mode", 0) == 0
                      else b["v_pool"].shape[1], d), float("nan"),
                     dtype=out_dtype, device="cuda")
    sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], kw.pop("bt", b["block_table"]),
                          b["ctx_lens"], out=out, k_scale=b["k_scale"], v_scale=b["v_scale"],
                          plane=plane, **kw)
    torch.cuda.synchronize()
    return out


def ref(b, plane=None, **kw):
    ctrl = None
    if plane is not None:
        ctrl = bytes(plane._ctrl_host)
    return oracle.decode(b["q"], b["k_pool"], b["v_pool"], kw.pop("bt", b["block_table"]),
                         b["ctx_lens"], k_scale=b["k_scale"], v_scale=b["v_scale"], ctrl=ctrl,
                         max_tasks=plane.N if plane is not None else 4096, **kw)


def batch(ctx, hq=32, hkv=8, d=128, kv=torch.bfloat16, qd=torch.bfloat16, seed=0):
    return workloads.make_batch(np.asarray(ctx), num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                                kv_dtype=kv, q_dtype=qd, seed=seed, device="cuda")


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


# --- parity -------------------------------------------------------------------

def test_mha_fp32_small_parity_tau_and_pi():
    """fp32, 16 requests, MHA 8 heads, d 64, page 16, ctx ~ U[64,512];
    pi identity vs reversed bitwise; tau 0 and tau = ctx/2 vs the oracle."""
    b = workloads.workload("mha_fp32_small", seed=1)
    R, H = 16, 8
    plane = SchedPlane(max_tasks=R * H)
    plane.set_num_tasks(R * H)
    plane.push()
    a = run(b, plane=plane)
    assert sched_pd.kernel_kind(sched_pd.build_args(
        b["q"], b["k_pool"], b["v_pool"], b["block_table"], b["ctx_lens"], out=a)) == "valu"
    e = par_err(a.cpu(), ref(b, plane))
    print(f"fp32 tau=0 err {e:.3g}")
    assert e <= TOL_F32
    plane.set_order(torch.arange(R * H - 1, -1, -1))
    assert torch.equal(run(b, plane=plane), a)
    plane.reset_order()
    ctx = b["ctx_lens"].cpu().numpy()
    plane.set_rows(tau=np.repeat(ctx // 2, H), n=R * H)
    plane.push()
    s = run(b, plane=plane)
    e = par_err(s.cpu(), ref(b, plane))
    print(f"fp32 tau=ctx/2 err {e:.3g}")
    assert e <= TOL_F32
    assert not torch.equal(s, a)
    plane.set_order(torch.arange(R * H - 1, -1, -1))
    assert torch.equal(run(b, plane=plane), s)


@pytest.mark.parametrize("ctx", [[2048] * 4, [1, 15, 16, 17, 33, 100, 511, 5000]])
@pytest.mark.parametrize("force_valu", [False, True])
def test_bf16_gqa_parity(ctx, force_valu):
    b = batch(ctx, seed=len(ctx))
    flags = abi.FLAG_FORCE_VALU if force_valu else 0
    out = run(b, flags=flags)
    args = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                               b["ctx_lens"], out=out, flags=flags)
    assert sched_pd.kernel_kind(args) == ("valu" if force_valu else "mfma")
    e = par_err(out.cpu(), ref(b))
    print(f"bf16 {'valu' if force_valu else 'mfma'} err {e:.3g}")
    assert e <= TOL_BF16
    # a bf16 output is the RNE of the fp32 one, which is held to the oracle
    # above (rounding the output alone costs ~1.3e-3 row-relative)
    o16 = run(b, flags=flags, out_dtype=torch.bfloat16)
    assert torch.equal(o16, out.to(torch.bfloat16))


def token_major(b):
    """The batch with V stored token-major ([P, Hkv, page, d]), same values."""
    c = dict(b)
    c["v_pool"] = b["v_pool"].permute(0, 1, 3, 2).contiguous()
    return c


@pytest.mark.parametrize("kvt", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (28, 4), (64, 4)])
def test_token_major_v_matches_dmajor_bitwise(hq, hkv, kvt):
    """bf16 or fp8 V stored token-major (FlashInfer's HND / NHD rows) takes
    the MFMA kernel with an in-lane operand build and a permuted dim order in
    its accumulators; every output element sums the same products in the
    same order as the d-major kernel, so the bits agree. Then the oracle, the
    VALU kernel on the same layout, and split tiles under the queue with pi
    reversed against the static grid."""
    b = batch([1, 15, 16, 17, 300, 2048, 5000], hq=hq, hkv=hkv, kv=kvt, seed=hq + hkv)
    t = token_major(b)
    d_out = run(b)
    t_out = run(t, v_layout="tokmajor")
    args = sched_pd.build_args(t["q"], t["k_pool"], t["v_pool"], t["block_table"],
                               t["ctx_lens"], out=t_out, v_layout="tokmajor")
    assert sched_pd.kernel_kind(args) == "mfma"
    assert torch.equal(d_out, t_out)
    e = par_err(t_out.cpu(), ref(t, v_layout="tokmajor"))
    print(f"token-major mfma G={hq // hkv} err {e:.3g}")
    assert e <= TOL_BF16
    v = run(t, v_layout="tokmajor", flags=abi.FLAG_FORCE_VALU)
    assert par_err(v.cpu(), ref(t, v_layout="tokmajor")) <= TOL_BF16
    ctx = t["ctx_lens"].cpu().numpy()
    tiles = sched_pd.plan_tiles(ctx, 16, 32, hkv)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ctx.size * hkv))
    plane.set_num_tasks(0)
    plane.push()
    st = run(t, plane=plane, v_layout="tokmajor", tiles=tiles, tile_pages=32)
    plane.set_order(torch.arange(nt - 1, -1, -1, dtype=torch.int32))
    plane.set_num_tasks(nt)
    plane.push()
    plane.reset_queue(2 * sched_pd.cu_count())
    wq = run(t, plane=plane, v_layout="tokmajor", tiles=tiles, tile_pages=32,
             workers=2 * sched_pd.cu_count())
    assert torch.equal(st, wq)
    assert par_err(st.cpu(), ref(t, v_layout="tokmajor")) <= TOL_BF16


@pytest.mark.parametrize("kvt", [torch.bfloat16, torch.float8_e4m3fn])
def test_token_major_v_linear_matches_dmajor_bitwise(kvt):
    b = batch([16, 700, 2048, 3], kv=kvt, seed=9)
    t = token_major(b)
    w = torch.randn(4096, device="cuda")
    d_out = run(b, mode=abi.LINEAR, lin_w=w)
    t_out = run(t, mode=abi.LINEAR, lin_w=w, v_layout="tokmajor")
    assert torch.equal(d_out, t_out)
    e = par_err(t_out.cpu(), ref(t, mode=abi.LINEAR, lin_w=w.cpu().numpy(),
                                   v_layout="tokmajor"))
    assert e <= TOL_BF16


PG_CTX = [1, 15, 16, 17, 33, 100, 511, 5000]


@pytest.mark.parametrize("ps", [32, 64, 256])
@pytest.mark.parametrize("kvt,layout", [(torch.bfloat16, "dmajor"),
                                        (torch.float8_e4m3fn, "dmajor"),
                                        (torch.float8_e4m3fn, "tokmajor"),
                                        (torch.bfloat16, "tokmajor"),
                                        (torch.float16, "tokmajor"),
                                        (torch.float16, "dmajor")])
def test_pages_of_more_than_16_tokens(ps, kvt, layout):
    """Pages of 32..256 tokens run on the MFMA kernel as 16-token blocks
    (block b is sub-block b % m of table entry b / m): oracle parity for
    GQA 4 and 7, and pi reversed under the queue over split tiles (in pages)
    against the static grid over the same tiles. fp16 caches take fp16 Q."""
    for hq, hkv in ((32, 8), (28, 4)):
        b = workloads.make_batch(np.asarray(PG_CTX), num_q_heads=hq, num_kv_heads=hkv,
                                 page_size=ps, kv_dtype=kvt, seed=ps + hq, device="cuda",
                                 q_dtype=torch.float16 if kvt == torch.float16 else
                                 torch.bfloat16)
        if layout == "tokmajor":
            b = token_major(b)
        out = run(b, v_layout=layout)
        args = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                   b["ctx_lens"], out=out, v_layout=layout,
                                   k_scale=b["k_scale"], v_scale=b["v_scale"])
        assert sched_pd.kernel_kind(args) == "mfma"
        e = par_err(out.cpu(), ref(b, v_layout=layout))
        print(f"page {ps} {kvt} {layout} G={hq // hkv} err {e:.3g}", flush=True)
        assert e <= TOL_BF16
    ctx = b["ctx_lens"].cpu().numpy()
    tp = 2
    tiles = sched_pd.plan_tiles(ctx, ps, tp, hkv)
    nt = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(nt, ctx.size * hkv))
    plane.set_num_tasks(0)
    plane.push()
    st = run(b, plane=plane, v_layout=layout, tiles=tiles, tile_pages=tp)
    plane.set_order(torch.arange(nt - 1, -1, -1, dtype=torch.int32))
    plane.set_num_tasks(nt)
    plane.push()
    plane.reset_queue(2 * sched_pd.cu_count())
    wq = run(b, plane=plane, v_layout=layout, tiles=tiles, tile_pages=tp,
             workers=2 * sched_pd.cu_count())
    assert torch.equal(st, wq)
    assert par_err(st.cpu(), ref(b, v_layout=layout)) <= TOL_BF16


@pytest.mark.parametrize("scope", [abi.TAU_PREFIX, abi.TAU_PER_PAGE])
def test_pages_of_32_tokens_shed_and_linear(scope):
    """Shed on 32-token pages: the per-page scope counts the offset in the
    whole page (not the 16-token block); skipping and load + mask agree
    bitwise; the linear contraction over the same pages."""
    rng = np.random.default_rng(8)
    ctx = rng.integers(300, 3000, size=5)
    b = workloads.make_batch(ctx, num_q_heads=32, num_kv_heads=8, page_size=32, seed=12,
                             device="cuda")
    n = ctx.size * 8
    plane = SchedPlane(max_tasks=n)
    if scope == abi.TAU_PREFIX:
        tau = np.repeat([rng.integers(-(-c // 4), c + 1) for c in ctx], 8)
    else:
        tau = rng.integers(1, 33, size=n)   # in-page budgets, both blocks of a page
    plane.set_rows(tau=tau, n=n)
    plane.push()
    s = run(b, plane=plane, tau_scope=scope)
    e = par_err(s.cpu(), ref(b, plane, tau_scope=scope))
    print(f"page 32 shed scope {scope} err {e:.3g}", flush=True)
    assert e <= TOL_BF16
    assert torch.equal(run(b, plane=plane, tau_scope=scope, flags=abi.FLAG_SHED_LOADS), s)
    w = torch.randn(4096, device="cuda")
    lo = run(b, plane=plane, mode=abi.LINEAR, lin_w=w, tau_scope=scope)
    e = par_err(lo.cpu(), ref(b, plane, mode=abi.LINEAR, lin_w=w.cpu().numpy(),
                                tau_scope=scope))
    assert e <= TOL_BF16


@pytest.mark.parametrize("ranged", [False, True])
def test_split_pages_of_32_tokens_under_a_mid_page_budget(ranged):
    """Split tiles over 32-token pages with prefix budgets that end inside a
    page (40 tokens: 2 pages, 3 of their 16-token blocks) and chunks wholly
    past the budget: those chunks read nothing (their block range is empty,
    not reversed), the rest match the oracle, and loading + masking the shed
    tokens gives the same bits."""
    rng = np.random.default_rng(29)
    ctx = np.array([3000, 2000, 700, 90])
    hkv, ps, tp = 8, 32, 2
    b = workloads.make_batch(ctx, num_q_heads=32, num_kv_heads=hkv, page_size=ps, seed=29,
                             device="cuda")
    n = ctx.size * hkv
    tau = rng.integers(1, 1200, size=n)
    tau[::3] = 40
    tau[1::5] = 0                                  # no cap
    if ranged:
        tiles = sched_pd.plan_ranges_host(ctx, ps, hkv, task_order=rng.permutation(n),
                                          tile_pages=tp, tail_pages=1, tail_frac=0.5)
        kw = dict(tiles=tiles)
    else:
        tiles = sched_pd.plan_tiles_host(ctx, ps, tp, hkv)
        kw = dict(tiles=tiles, tile_pages=tp)
    assert (sched_pd.tile_pages_loaded(tiles, ctx, ps, tp, hkv, tau=tau) == 0).any()
    plane = SchedPlane(max_tasks=max(n, tiles.shape[0]))
    plane.set_rows(tau=tau, n=n)
    plane.push()
    s = run(b, plane=plane, **kw)
    e = par_err(s.cpu(), ref(b, plane))
    print(f"split page 32 mid-page budget ranged={ranged} err {e:.3g}", flush=True)
    assert e <= TOL_BF16
    assert torch.equal(run(b, plane=plane, flags=abi.FLAG_SHED_LOADS, **kw), s)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (28, 4), (16, 2), (64, 4)])
def test_fp16_cache_parity(hq, hkv):
    """An fp16 cache with fp16 Q (FlashInfer's dtype in the reference's
    serving tests) runs on the MFMA kernel's fp16 operands: oracle parity,
    fp16 output the RNE of the fp32 one, the VALU kernel on the same inputs,
    and pi reversed under the queue bitwise against the static grid."""
    b = batch([1, 15, 16, 17, 300, 2048, 5000], hq=hq, hkv=hkv, kv=torch.float16,
              qd=torch.float16, seed=hq * hkv)
    out = run(b)
    args = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                               b["ctx_lens"], out=out)
    assert sched_pd.kernel_kind(args) == "mfma"
    r = ref(b)
    e = par_err(out.cpu(), r)
    print(f"fp16 mfma G={hq // hkv} err {e:.3g}", flush=True)
    assert e <= TOL_BF16
    o16 = run(b, out_dtype=torch.float16)
    assert torch.equal(out.to(torch.float16), o16)
    v = run(b, flags=abi.FLAG_FORCE_VALU)
    assert par_err(v.cpu(), r) <= TOL_BF16
    n = b["ctx_lens"].numel() * hkv
    plane = SchedPlane(max_tasks=n)
    plane.set_order(torch.arange(n - 1, -1, -1, dtype=torch.int32))
    plane.set_num_tasks(n)
    plane.push()
    plane.reset_queue(2 * sched_pd.cu_count())
    assert torch.equal(run(b, plane=plane, workers=2 * sched_pd.cu_count()), out)
    t = token_major(b)
    assert torch.equal(run(t, v_layout="tokmajor"), out)


def test_fp16_shapes_off_the_mfma_path():
    """fp16 caches on the VALU kernel against the oracle: 32-token pages with
    the MFMA kernel switched off, and what the MFMA kernel does not take
    (fp32 Q, the linear mode)."""
    b = workloads.make_batch(np.asarray([100, 700, 33]), num_q_heads=32, num_kv_heads=8,
                             page_size=32, kv_dtype=torch.float16, q_dtype=torch.float16,
                             seed=5, device="cuda")
    out = run(b, flags=abi.FLAG_FORCE_VALU)
    assert par_err(out.cpu(), ref(b)) <= TOL_BF16
    b = batch([100, 700, 33], kv=torch.float16, qd=torch.float32, seed=6)
    assert par_err(run(b).cpu(), ref(b)) <= TOL_BF16
    w = torch.randn(4096, device="cuda")
    lo = run(b, mode=abi.LINEAR, lin_w=w)
    assert par_err(lo.cpu(), ref(b, mode=abi.LINEAR, lin_w=w.cpu().numpy())) <= TOL_BF16


def test_bf16_output_is_rne_of_fp32_output():
    b = batch([300, 2048, 17], seed=3)
    f = run(b)
    h = run(b, out_dtype=torch.bfloat16)
    assert torch.equal(f.to(torch.bfloat16), h)


@pytest.mark.parametrize("hq,hkv", [(28, 4), (32, 8), (16, 16), (64, 4)])
def test_fp8_parity(hq, hkv):
    b = batch([16, 700, 2048, 3, 257], hq=hq, hkv=hkv, kv=torch.float8_e4m3fn, seed=hq)
    out = run(b)
    e = par_err(out.cpu(), ref(b))
    print(f"fp8 G={hq // hkv} err {e:.3g}")
    assert e <= TOL_BF16


@pytest.mark.parametrize("scope", [abi.TAU_PREFIX, abi.TAU_PER_PAGE])
@pytest.mark.parametrize("kvt", [torch.bfloat16, torch.float8_e4m3fn])
def test_shed_softmax_matches_truncated_reference(scope, kvt):
    rng = np.random.default_rng(4)
    ctx = rng.integers(1024, 4097, size=6)
    b = batch(ctx, kv=kvt, seed=5)
    n = len(ctx) * 8
    plane = SchedPlane(max_tasks=n)
    if scope == abi.TAU_PREFIX:
        tau = np.repeat([rng.integers(-(-c // 4), c + 1) for c in ctx], 8)
    else:
        tau = rng.integers(1, 17, size=n)
    tau[::7] = 0  # some tasks unshed
    plane.set_rows(tau=tau, n=n)
    plane.push()
    out = run(b, plane=plane, tau_scope=scope)
    e = par_err(out.cpu(), ref(b, plane, tau_scope=scope))
    print(f"shed scope {scope} {kvt} err {e:.3g}")
    assert e <= TOL_BF16
    # loading the shed pages and masking them gives the same bits (MFMA and VALU)
    same = run(b, plane=plane, tau_scope=scope, flags=abi.FLAG_SHED_LOADS)
    assert torch.equal(out, same)
    v = run(b, plane=plane, tau_scope=scope, flags=abi.FLAG_FORCE_VALU)
    assert par_err(v.cpu(), ref(b, plane, tau_scope=scope)) <= TOL_BF16
    assert torch.equal(v, run(b, plane=plane, tau_scope=scope,
                              flags=abi.FLAG_FORCE_VALU | abi.FLAG_SHED_LOADS))


@pytest.mark.parametrize("kvt", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("period", [0, 16])
@pytest.mark.parametrize("force_valu", [False, True])
def test_linear_contraction_and_value_shed(kvt, period, force_valu):
    ctx = [64, 1000, 5, 2048]
    b = batch(ctx, hq=8, hkv=8, d=64 if kvt == torch.float32 else 128, kv=kvt,
              qd=torch.float32 if kvt == torch.float32 else torch.bfloat16, seed=6)
    w = torch.randn(4096, device="cuda")
    n = len(ctx) * 8
    plane = SchedPlane(max_tasks=n)
    tau = np.random.default_rng(7).integers(0, 2048, size=n)
    plane.set_rows(tau=tau, n=n)
    plane.push()
    flags = abi.FLAG_FORCE_VALU if force_valu else 0
    out = run(b, plane=plane, mode=abi.LINEAR, lin_w=w, lin_w_period=period, flags=flags)
    args = sched_pd.build_args(None, None, b["v_pool"], b["block_table"], b["ctx_lens"],
                               out=out, mode=abi.LINEAR, lin_w=w, flags=flags)
    expect = "valu" if (force_valu or kvt == torch.float32) else "mfma"
    assert sched_pd.kernel_kind(args) == expect
    r = ref(b, plane, mode=abi.LINEAR, lin_w=w.cpu().numpy(), lin_w_period=period)
    tol = TOL_F32 if kvt == torch.float32 else TOL_BF16
    e = par_err(out.cpu(), r)
    print(f"linear {kvt} err {e:.3g}")
    assert e <= tol


def test_empty_request_gives_nan_like_the_reference():
    b = batch([0, 64, 0])
    out = run(b)
    assert torch.isnan(out[0]).all() and torch.isnan(out[2]).all()
    assert torch.isfinite(out[1]).all()


def test_csr_page_table():
    b = batch([100, 2048, 33], seed=8)
    ctx = b["ctx_lens"].cpu().numpy()
    npg = (ctx + 15) // 16
    bt = b["block_table"].cpu().numpy()
    indptr = torch.tensor(np.concatenate([[0], np.cumsum(npg)]), dtype=torch.int32, device="cuda")
    flat = torch.tensor(np.concatenate([bt[r, :npg[r]] for r in range(3)]), dtype=torch.int32,
                        device="cuda")
    a = run(b)
    c = run(b, bt=flat, page_indptr=indptr, check_tables=True)
    assert torch.equal(a, c)
    # the host check refuses a table whose reach leaves the pool, before launch
    bad = flat.clone()
    bad[-1] = b["k_pool"].shape[0]
    with pytest.raises(ValueError, match="request 2 has a page id"):
        run(b, bt=bad, page_indptr=indptr, check_tables=True)


# --- levers that must not change a bit ---------------------------------------

def _hetero(seed=9):
    ctx = np.random.default_rng(seed).integers(1, 3000, size=24)
    return batch(ctx, seed=seed)


@pytest.mark.parametrize("pi", ["reversed", "random", "lpt"])
def test_pi_is_bit_invariant(pi):
    b = _hetero()
    n = 24 * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane)
    if pi == "reversed":
        order = torch.arange(n - 1, -1, -1)
    elif pi == "random":
        order = torch.randperm(n)
    else:
        order = SchedPlane._grouped_lpt(torch.repeat_interleave(b["ctx_lens"].cpu(), 8).float(), 1)
    plane.install_order(order, n)
    plane.push()
    assert torch.equal(run(b, plane=plane), base)


@pytest.mark.parametrize("W", [1, 7, 192, 197, 512])
def test_work_queue_is_bit_invariant_and_times_every_task(W):
    b = _hetero(10)
    n = 24 * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane)
    plane.set_num_tasks(n)
    plane.install_order(torch.randperm(n), n)
    plane.push()
    plane.reset_queue(W)
    plane.clear_timer()
    out = run(b, plane=plane, workers=W)
    assert torch.equal(out, base)
    rows = plane.read_timer()[:n]
    assert int((rows > 0).sum()) == n
    # the counter reset itself: a second launch without a host reset is exact too
    plane.clear_timer()
    assert torch.equal(run(b, plane=plane, workers=W), base)
    assert int((plane.read_timer()[:n] > 0).sum()) == n


def test_policy_levers_are_bit_invariant():
    b = _hetero(11)
    n = 24 * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane)
    rng = np.random.default_rng(0)
    plane.set_lambda(0.5)
    plane.set_rows(q=rng.uniform(0, 1, n), hint=rng.integers(0, 3, n), n=n)
    plane.push()
    assert torch.equal(run(b, plane=plane, policy=(1.0, 1.0, 0.1)), base)
    plane.set_rows(hint=np.full(n, abi.HINT_URGENT), n=n)
    plane.push()
    assert torch.equal(run(b, plane=plane), base)
    plane.set_rows(hint=np.full(n, abi.HINT_POLITE), n=n)
    plane.push()
    assert torch.equal(run(b, plane=plane), base)


@pytest.mark.parametrize("kvt,layout,ps", [(torch.bfloat16, "dmajor", 16),
                                           (torch.float8_e4m3fn, "dmajor", 16),
                                           (torch.float8_e4m3fn, "dmajor", 32),
                                           (torch.bfloat16, "tokmajor", 16)])
def test_pf_dist_sets_the_urgent_depth_and_keeps_the_bits(kvt, layout, ps):
    """Every urgent task at each ring depth the kernel serves (pf_dist 0 =
    the deepest): same bits as the stock launch; a depth it does not serve is
    an error, not ignored."""
    ctx = np.array([1, 16, 17, 100, 700, 2048, 4000, 33])
    b = workloads.make_batch(ctx, num_q_heads=32, num_kv_heads=8, page_size=ps, kv_dtype=kvt,
                             seed=21, device="cuda")
    if layout == "tokmajor":
        b = token_major(b)
    n = ctx.size * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane, v_layout=layout)
    args = sched_pd.build_args(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                               b["ctx_lens"], out=base, v_layout=layout)
    lo, hi = sched_pd.prefetch_range(args)
    assert 1 <= lo <= hi
    plane.set_rows(hint=np.full(n, abi.HINT_URGENT), n=n)
    plane.push()
    for pf in [0, *range(lo, hi + 1)]:
        assert torch.equal(run(b, plane=plane, v_layout=layout, pf_dist=pf), base), pf
    with pytest.raises(RuntimeError, match="pf_dist"):
        run(b, plane=plane, v_layout=layout, pf_dist=hi + 1)
    # priced-in urgency (q > lambda_bw + H) takes the same path as the hint
    plane.set_lambda(0.5)
    plane.set_rows(q=np.full(n, 0.9), hint=np.zeros(n, np.int64), n=n)
    plane.push()
    assert torch.equal(run(b, plane=plane, v_layout=layout, pf_dist=lo,
                           policy=(1.0, 1.0, 0.1)), base)


def test_timer_rows_gate_and_cost_ranking():
    ctx = np.array([16] * 16 + [8192] * 2)
    b = batch(ctx, seed=12)
    n = len(ctx) * 8
    plane = SchedPlane(max_tasks=n)
    plane.use_device_timer()
    base = run(b)
    plane.clear_timer()
    assert torch.equal(run(b, plane=plane), base)
    cyc = plane.read_timer()[:n].numpy()
    assert (cyc > 0).all()
    long_c = cyc[16 * 8:].mean()
    short_c = cyc[:16 * 8].mean()
    print(f"timer long {long_c:.0f} short {short_c:.0f}")
    assert long_c > 2 * short_c
    plane.set_timer_enabled(False)
    plane.push()
    plane.clear_timer()
    assert torch.equal(run(b, plane=plane), base)
    assert int((plane.read_timer() != 0).sum()) == 0


def test_remap_edge_cases_follow_the_emulator():
    import levers
    b = _hetero(13)
    n = 24 * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane)
    # out-of-range and negative entries fall back to the workgroup's own id
    order = np.arange(n)
    order[3], order[5] = n + 7, -2
    plane.set_order(torch.tensor(order, dtype=torch.int32))
    assert torch.equal(run(b, plane=plane), base)
    # duplicates under a stale order_size stamp: whole launch takes identity
    dup = np.arange(n)
    dup[10] = 11
    plane.set_order(torch.tensor(dup, dtype=torch.int32))
    plane.set_order_size(n + 1)
    plane.push()
    assert torch.equal(run(b, plane=plane), base)
    # duplicates unchecked (order_size 0): task 10 never runs, 11 runs twice
    plane.set_order_size(0)
    plane.push()
    plane.clear_timer()
    out = run(b, plane=plane)
    ex, rows = levers.run_launch(ntasks=n, grid=n, wq=False, order=list(dup),
                                 ctrl={"order_size": 0}, max_tasks=n)
    missing = sorted(set(range(n)) - set(ex))
    assert missing == [10]
    r, h = divmod(10, 8)
    assert torch.isnan(out[r, h * 4:(h + 1) * 4]).all()
    keep = torch.ones(n, dtype=torch.bool)
    keep[10] = False
    o = out.view(24, 8, 4, 128)[:].reshape(n, 4, 128)
    assert torch.equal(o[keep], base.view(n, 4, 128)[keep])
    t = plane.read_timer()[:n].numpy()
    assert t[10] == 0 and t[11] > 0


def test_num_tasks_zero_takes_the_static_path():
    b = _hetero(14)
    n = 24 * 8
    plane = SchedPlane(max_tasks=n)
    base = run(b, plane=plane)
    plane.set_num_tasks(0)
    plane.set_order(torch.arange(n - 1, -1, -1))
    plane.push()
    plane.clear_timer()
    # workers requested, but num_tasks 0 disarms the claim loop: full grid
    assert torch.equal(run(b, plane=plane, workers=16), base)
    assert int((plane.read_timer()[:n] > 0).sum()) == n


# --- split-KV work items ------------------------------------------------------

SPLIT_CTX = [1, 16, 17, 300, 2048, 5000, 0, 777]


@pytest.mark.parametrize("tp", [1, 3, 16, 64])
@pytest.mark.parametrize("kvt", [torch.bfloat16, torch.float8_e4m3fn])
def test_split_kv_parity_and_schedule_invariance(tp, kvt):
    b = batch(SPLIT_CTX, kv=kvt, seed=tp)
    ntask = len(SPLIT_CTX) * 8
    tiles = sched_pd.plan_tiles(SPLIT_CTX, 16, tp, 8)
    n = tiles.shape[0]
    plane = SchedPlane(max_tasks=max(n, ntask))
    out = run(b, plane=plane, tiles=tiles, tile_pages=tp)
    r = ref(b)
    fin = np.isfinite(r)
    assert np.array_equal(np.isnan(out.cpu().numpy()), ~fin)  # the empty request is 0/0
    e = par_err(out.cpu().numpy()[fin], r[fin])
    print(f"split tp={tp} {kvt} items={n} err {e:.3g}")
    assert e <= TOL_BF16
    # pi over work items
    plane.install_order(torch.arange(n - 1, -1, -1), n)
    plane.push()
    assert _same(run(b, plane=plane, tiles=tiles, tile_pages=tp), out)
    plane.install_order(torch.randperm(n), n)
    plane.set_num_tasks(n)
    plane.push()
    for W in (3, 100, n + 9):
        plane.reset_queue(W)
        plane.clear_timer()
        o = run(b, plane=plane, tiles=tiles, tile_pages=tp, workers=W)
        assert _same(o, out)
        rows = plane.read_timer()[:ntask].numpy()
        assert (rows > 0).all()  # every task's chunks add into its own row
    # relaunch with the same W and no host reset: arrival counters and the
    # ticket counter reset themselves
    q0 = int(plane._queue.item())
    assert q0 == n + 9
    plane._queue_w = n + 9
    assert _same(run(b, plane=plane, tiles=tiles, tile_pages=tp, workers=n + 9), out)
    assert int(plane._queue.item()) == n + 9
    ws = sched_pd.workspace_for(0, "cuda")
    assert int(ws[:sched_pd.WS_COUNTERS_OFF + 4 * ntask].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("flags,workers", [(0, 0), (abi.FLAG_FORCE_VALU, 0), (0, 37)])
def test_stale_split_plan_is_flagged_and_leaves_counters_clean(flags, workers):
    """A plan built for older lengths: request 1 grew past two tile
    boundaries (its tasks are stale: output rows NaN, counted, arrival
    counters untouched), request 2 shrank below one (its extra chunk is
    skipped, the output is right). A fresh plan on the same workspace then
    gives the oracle's result everywhere and leaves every counter zero."""
    old_ctx, new_ctx = [100, 3000, 1000], [100, 3600, 400]
    b = batch(new_ctx, seed=41)
    hkv, tp = 8, 32
    stale_plan = sched_pd.plan_tiles(old_ctx, 16, tp, hkv)
    fresh_plan = sched_pd.plan_tiles(new_ctx, 16, tp, hkv)
    n = max(stale_plan.shape[0], fresh_plan.shape[0], len(new_ctx) * hkv)
    plane = SchedPlane(max_tasks=n)
    r = ref(b)
    ws = sched_pd.workspace_for(0, "cuda")
    sched_pd.stale_plan_count(ws, reset=True)
    for plan in (stale_plan, fresh_plan):
        nt = plan.shape[0]
        plane.set_num_tasks(nt if workers else 0)
        plane.push()
        if workers:
            plane.reset_queue(workers)
        o = run(b, plane=plane, tiles=plan, tile_pages=tp, flags=flags, workers=workers)
        got = o.cpu().numpy()
        if plan is stale_plan:
            assert np.isnan(got[1]).all()
            assert par_err(got[[0, 2]], r[[0, 2]]) <= TOL_BF16
            assert sched_pd.stale_plan_count(ws, reset=True) == hkv
        else:
            assert par_err(got, r) <= TOL_BF16
            assert sched_pd.stale_plan_count(ws) == 0
        counters = ws[sched_pd.WS_COUNTERS_OFF:sched_pd.WS_COUNTERS_OFF + 4 * len(new_ctx) * hkv]
        assert int(counters.view(torch.int32).abs().sum()) == 0


def _same(a, b):
    return bool(torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0))) and \
        bool(torch.equal(torch.isnan(a), torch.isnan(b)))


def test_split_kv_with_shed_valu_and_linear():
    ctx = [40, 3000, 1000, 4096]
    b = batch(ctx, seed=31)
    ntask = len(ctx) * 8
    tiles = sched_pd.plan_tiles(ctx, 16, 32, 8)
    plane = SchedPlane(max_tasks=max(tiles.shape[0], ntask))
    tau = np.random.default_rng(3).integers(0, 3000, size=ntask)
    plane.set_rows(tau=tau, n=ntask)
    plane.push()
    for flags in (0, abi.FLAG_FORCE_VALU):
        o = run(b, plane=plane, tiles=tiles, tile_pages=32, flags=flags)
        assert par_err(o.cpu(), ref(b, plane)) <= TOL_BF16
    w = torch.randn(4096, device="cuda")
    o = run(b, plane=plane, tiles=tiles, tile_pages=32, mode=abi.LINEAR, lin_w=w)
    r = ref(b, plane, mode=abi.LINEAR, lin_w=w.cpu().numpy())
    assert par_err(o.cpu(), r) <= TOL_BF16


def test_split_args_keep_their_workspace_when_the_cache_grows():
    """Arguments built for a small plan, then for one that needs a larger
    workspace (the cache replaces its tensor), then new allocations of the
    old size filled with garbage: relaunching the first arguments still
    writes into their own workspace and gives the oracle's result. A stream
    of its own gives the test a workspace cache entry of its own."""
    small = batch([3000, 40], seed=43)
    big = batch([3000] * 24, seed=44)
    outs = [torch.empty(2, 32, 128, device="cuda"), torch.empty(24, 32, 128, device="cuda")]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    a_small = sched_pd.build_args(small["q"], small["k_pool"], small["v_pool"],
                                  small["block_table"], small["ctx_lens"], out=outs[0],
                                  tiles=sched_pd.plan_tiles_host([3000, 40], 16, 16, 8),
                                  tile_pages=16, stream=s)
    n_small = a_small._ws.numel()
    a_big = sched_pd.build_args(big["q"], big["k_pool"], big["v_pool"], big["block_table"],
                                big["ctx_lens"], out=outs[1],
                                tiles=sched_pd.plan_tiles_host([3000] * 24, 16, 16, 8),
                                tile_pages=16, stream=s)
    assert a_big.workspace != a_small.workspace            # the cache grew
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        junk = [torch.full((n_small,), 0x7F, dtype=torch.uint8, device="cuda") for _ in range(4)]
        for _ in range(2):
            sched_pd.launch(a_small, s)
            sched_pd.launch(a_big, s)
    torch.cuda.synchronize()
    assert par_err(outs[0].cpu(), ref(small)) <= TOL_BF16
    assert par_err(outs[1].cpu(), ref(big)) <= TOL_BF16
    assert int(a_small._ws[:sched_pd.WS_COUNTERS_OFF + 4 * 16].view(torch.int32).abs().sum()) == 0
    del junk


def test_split_workspace_counters_grow_safely():
    small = batch([3000, 40], seed=41)
    big = batch([3000] * 12, seed=42)
    for b in (small, big, small, big):
        ctx = b["ctx_lens"].cpu().numpy()
        tiles = sched_pd.plan_tiles(ctx, 16, 16, 8)
        o = run(b, tiles=tiles, tile_pages=16)
        assert par_err(o.cpu(), ref(b)) <= TOL_BF16
