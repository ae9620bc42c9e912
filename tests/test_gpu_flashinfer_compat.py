"""FlashInfer's batch-decode wrapper calls, as the reference's serving tests
make them (test/py/test_flashinfer_arm.py:40-100), on this library: fp16 Q
and NHD cache, plan() / run(); pi permutes (request, kv-head) tasks with the
output bit-exact, the timer fills a row per task, and the output matches the
oracle. HND and (k, v)-pair caches give the same bits as NHD."""
import numpy as np
import pytest
import torch

import oracle
import sched_pd
from flashinfer_compat import BatchDecodeWithPagedKVCacheWrapper
from parity import TOL_BF16, par_err
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def setup(bs=8, max_pages=8, page=16, nqo=8, nkv=8, hd=128, seed=0):
    torch.manual_seed(seed)
    dev = "cuda"
    kv_indptr = torch.arange(0, bs * max_pages + 1, max_pages, dtype=torch.int32, device=dev)
    kv_indices = torch.arange(bs * max_pages, dtype=torch.int32, device=dev)
    last_len = torch.full((bs,), page, dtype=torch.int32, device=dev)
    q = torch.randn(bs, nqo, hd, dtype=torch.float16, device=dev)
    kv = torch.randn(bs * max_pages, 2, page, nkv, hd, dtype=torch.float16, device=dev)
    return kv_indptr, kv_indices, last_len, q, kv


def test_armed_pi_is_bit_exact_and_the_timer_fills():
    indptr, indices, last, q, kv = setup()
    bs, nqo, nkv, hd, page = 8, 8, 8, 128, 16
    plane = SchedPlane(max_tasks=1024)
    plane.set_num_tasks(plane.N)
    plane.push()
    w = BatchDecodeWithPagedKVCacheWrapper(
        torch.empty(1 << 20, dtype=torch.uint8, device="cuda"), "NHD", plane=plane)
    w.plan(indptr, indices, last, nqo, nkv, hd, page, data_type=torch.float16,
           q_data_type=torch.float16)
    plane.reset_order()
    plane.clear_timer()
    golden = w.run(q, kv).clone()
    torch.cuda.synchronize()
    assert golden.dtype == torch.float16 and golden.shape == (bs, nqo, hd)
    cyc = plane.read_timer()[:bs * nkv]
    assert int((cyc > 0).sum()) == bs * nkv
    # swap adjacent pairs of the first tasks (the reference's permutation)
    order = torch.arange(plane.N, dtype=torch.int32)
    npair = bs - (bs % 2)
    order[:npair] = order[:npair].view(-1, 2).flip(1).reshape(-1)
    plane.set_order(order)
    permuted = w.run(q, kv).clone()
    assert torch.equal(permuted, golden)
    plane.set_order(torch.arange(bs * nkv - 1, -1, -1, dtype=torch.int32))
    assert torch.equal(w.run(q, kv), golden)
    kview, vview = (kv[:, 0].permute(0, 2, 1, 3), kv[:, 1].permute(0, 2, 1, 3))
    ctx = torch.full((bs,), 8 * page, dtype=torch.int32, device="cuda")
    r = np.asarray(oracle.decode(q, kview, vview, indices, ctx, page_indptr=indptr,
                                 v_layout="tokmajor"), np.float64)
    g = golden.float().cpu().double().numpy()
    assert par_err(g, r) <= TOL_BF16


def test_layouts_and_ragged_batch_agree():
    """A ragged batch (partial last pages, an empty request) in NHD, HND and
    (k, v)-pair form: the same bits, and the oracle's values."""
    rng = np.random.default_rng(5)
    bs, page, nqo, nkv, hd = 6, 16, 16, 2, 128
    pages = np.array([3, 1, 0, 7, 2, 5], np.int32)
    P = int(pages.sum()) + 4
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)).cuda()
    indices = torch.from_numpy(rng.permutation(P)[:pages.sum()].astype(np.int32)).cuda()
    last = torch.from_numpy(rng.integers(1, page + 1, bs).astype(np.int32)).cuda()
    q = torch.randn(bs, nqo, hd, dtype=torch.float16, device="cuda")
    nhd = torch.randn(P, 2, page, nkv, hd, dtype=torch.float16, device="cuda")
    hnd = nhd.permute(0, 1, 3, 2, 4).contiguous()
    outs = []
    for layout, cache in (("NHD", nhd), ("HND", hnd), ("NHD", (nhd[:, 0], nhd[:, 1])),
                          ("HND", (hnd[:, 0], hnd[:, 1]))):
        w = BatchDecodeWithPagedKVCacheWrapper(None, layout)
        w.plan(indptr, indices, last, nqo, nkv, hd, page, data_type=torch.float16,
               q_data_type=torch.float16)
        outs.append(w.run(q, cache, out=torch.empty(bs, nqo, hd, device="cuda")))
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o[pages > 0], outs[0][pages > 0])
    from kv_cache import ctx_lens_from_last_page_len, nhd_views
    ctx = ctx_lens_from_last_page_len(indptr, last, page)
    k, v = nhd_views(nhd)
    r = np.asarray(oracle.decode(q, k, v, indices, ctx, page_indptr=indptr,
                                 v_layout="tokmajor"), np.float64)
    g = outs[0].cpu().double().numpy()
    keep = pages > 0
    assert par_err(g[keep], r[keep]) <= TOL_BF16


def test_plan_and_run_reject_what_they_cannot_honour():
    indptr, indices, last, q, kv = setup(bs=2, max_pages=2)
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    with pytest.raises(RuntimeError):
        w.run(q, kv)
    with pytest.raises(ValueError):
        w.plan(indptr, indices, last, 8, 8, 128, 16, pos_encoding_mode="ROPE_LLAMA")
    with pytest.raises(ValueError):
        w.plan(indptr, indices, last, 8, 3, 128, 16)
    w.plan(indptr, indices, last, 8, 8, 128, 16, data_type=torch.bfloat16)
    with pytest.raises(ValueError):
        w.run(q, kv)      # fp16 cache against a bf16 plan


def test_fp8_nhd_cache_with_flashinfer_scales():
    """An fp8 e4m3fn NHD cache with bf16 Q, FlashInfer's per-tensor k_scale /
    v_scale floats: the MFMA kernel on the cache in place (token-major fp8 V)
    against the oracle on the same codes and scales."""
    import kv_cache
    torch.manual_seed(5)
    bs, max_pages, page, nqo, nkv, hd = 6, 9, 16, 16, 4, 128
    pages = torch.tensor([1, 9, 4, 7, 2, 5], dtype=torch.int32)
    indptr = torch.zeros(bs + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(pages, 0)
    npg = int(indptr[-1])
    indptr = indptr.cuda()
    indices = torch.randperm(npg + 3)[:npg].to(torch.int32).cuda()
    last = torch.tensor([16, 3, 9, 16, 1, 12], dtype=torch.int32).cuda()
    kv = torch.randn(npg + 3, 2, page, nkv, hd, device="cuda").to(torch.float8_e4m3fn)
    q = (torch.randn(bs, nqo, hd, device="cuda") / hd ** 0.5).bfloat16()
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    w.plan(indptr, indices, last, nqo, nkv, hd, page, data_type=torch.float8_e4m3fn,
           q_data_type=torch.bfloat16)
    out = w.run(q, kv, k_scale=0.0625, v_scale=0.125)
    torch.cuda.synchronize()
    kview, vview = kv_cache.nhd_views(kv)
    out32 = torch.empty(out.shape, dtype=torch.float32, device="cuda")
    args = sched_pd.build_args(q, kview, vview, indices, w._plan["ctx"],
                               out=out32, page_indptr=indptr,
                               v_layout="tokmajor", k_scale=w._scales(kview, 0.0625, 0.125)[0],
                               v_scale=w._scales(kview, 0.0625, 0.125)[1])
    assert sched_pd.kernel_kind(args) == "mfma"
    sched_pd.launch(args)
    torch.cuda.synchronize()
    # the wrapper's bf16 output is the RNE of the same decode's fp32 output
    assert torch.equal(out, out32.to(out.dtype))
    n = (npg + 3) * nkv
    ref = np.asarray(oracle.decode(q, kview, vview, indices, w._plan["ctx"],
                                   page_indptr=indptr, v_layout="tokmajor",
                                   k_scale=torch.full((n,), 0.0625),
                                   v_scale=torch.full((n,), 0.125)), np.float64)
    assert par_err(out32.cpu(), ref) <= TOL_BF16
