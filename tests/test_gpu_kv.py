"""The KV-cache writer on the GPU: sched_kv_append through the C ABI against
the oracle, bit for bit (pools, scales, error count), the hardware fp8
encoder on every tie, the cache manager's decode loop, and size-independent
readback properties at the full Llama-3-8B decode size."""
import numpy as np
import pytest
import torch

import kv_cache
import oracle
import sched_pd
from parity import TOL_BF16, par_err
from kv_cases import FP8, append_case, random_pool

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def raw(t):
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == FP8:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def run_gpu(c, heads_per_group=0):
    dev = "cuda"
    k_pool, v_pool = c["k_pool"].to(dev), c["v_pool"].to(dev)
    ks = None if c["k_scale"] is None else c["k_scale"].to(dev)
    vs = None if c["v_scale"] is None else c["v_scale"].to(dev)
    errors = torch.zeros(1, dtype=torch.int32, device=dev)
    pind = None if c["pind"] is None else torch.from_numpy(c["pind"]).to(dev)
    torch.cuda.synchronize()
    kv_cache.append(c["k_src"].to(dev), c["v_src"].to(dev), torch.from_numpy(c["app"]).to(dev),
                    torch.from_numpy(c["ctx"].astype(np.int32)).to(dev), k_pool, v_pool,
                    torch.from_numpy(c["table"]).to(dev), page_indptr=pind,
                    v_layout=c["v_layout"], k_scale=ks, v_scale=vs, errors=errors,
                    heads_per_group=heads_per_group)
    torch.cuda.synchronize()
    return (raw(k_pool), raw(v_pool), None if ks is None else ks.cpu().numpy(),
            None if vs is None else vs.cpu().numpy(), int(errors.item()))


def assert_same(got, ref):
    for g, r, what in zip(got, ref, ("k_pool", "v_pool", "k_scale", "v_scale", "errors")):
        if r is None:
            assert g is None, what
        elif what == "errors":
            assert g == r, what
        else:
            assert np.array_equal(g, r), (what, int(np.sum(g != r)))


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32, FP8, torch.float16])
@pytest.mark.parametrize("v_layout", ["dmajor", "tokmajor"])
@pytest.mark.parametrize("csr", [False, True])
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32, torch.float16])
def test_append_is_bit_exact_with_the_oracle(kv, v_layout, csr, src):
    # d = 20 (a multiple of 4, not of 8) runs the 4-element chunk path, the
    # others the 8-element one
    for seed, (hkv, d) in enumerate([(8, 128), (4, 64), (2, 32), (3, 20)]):
        print(f"case kv={kv} v={v_layout} csr={csr} src={src} hkv={hkv} d={d}", flush=True)
        c = append_case(100 + seed, kv, v_layout, csr, hkv=hkv, d=d, src_dtype=src)
        assert_same(run_gpu(c), c["out"])


@pytest.mark.parametrize("kv", [torch.bfloat16, FP8])
@pytest.mark.parametrize("hpw", [1, 2, 4, 8])
def test_every_head_grouping_gives_the_same_bytes(kv, hpw):
    c = append_case(41, kv, "dmajor", hkv=8, d=128, prior=[3, 0, 17, 30, 9], n=[1, 40, 9, 20, 3])
    assert_same(run_gpu(c, heads_per_group=hpw), c["out"])


def test_append_into_partial_pages_regrows_fp8_scales():
    # every request already holds a partial page; the new rows are 16x larger
    c = append_case(7, FP8, "dmajor", prior=[3, 5, 17, 30, 1], n=[1, 4, 9, 20, 15], hkv=8, d=128)
    got = run_gpu(c)
    assert_same(got, c["out"])
    assert np.any(got[2] != c["k_scale"].numpy())


def test_page_size_32_and_64():
    for ps in (32, 64):
        c = append_case(11, FP8, "dmajor", hkv=4, d=128, ps=ps)
        assert_same(run_gpu(c), c["out"])
        c = append_case(12, torch.bfloat16, "tokmajor", hkv=4, d=128, ps=ps, csr=True)
        assert_same(run_gpu(c), c["out"])


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32, FP8, torch.float16])
def test_small_and_odd_page_sizes(kv):
    """Page sizes 8, 12 and 20 (multiples of 4, not of 16) with a d-major V:
    appends of 1 to 3 pages + 1 tokens on top of prior tokens, so first and
    last pages are partial and the 4-slot groups straddle o0 and o1."""
    for seed, ps in enumerate((8, 12, 20)):
        print(f"case kv={kv} ps={ps}", flush=True)
        c = append_case(60 + seed, kv, "dmajor", hkv=4, d=64, ps=ps,
                        prior=[0, 3, ps - 1, 2 * ps + 5, 7], n=[ps, 1, 2, 3 * ps + 1, 29])
        assert_same(run_gpu(c), c["out"])


def test_errors_are_counted_and_nothing_else_is_written():
    rng = np.random.default_rng(9)
    hkv, d, ps = 2, 8, 8
    c = dict(k_src=torch.ones(12, hkv, d, dtype=torch.bfloat16),
             v_src=torch.full((12, hkv, d), 2.0, dtype=torch.bfloat16),
             app=np.array([0, 3, 8, 11, 12], np.int32), ctx=np.array([3, 2, 3, 1]),
             table=np.array([[9, 0], [1, 0], [-1, 0], [2, 0]], np.int32), pind=None,
             k_pool=random_pool((4, hkv, ps, d), torch.bfloat16, rng),
             v_pool=random_pool((4, hkv, d, ps), torch.bfloat16, rng),
             k_scale=None, v_scale=None, v_layout="dmajor", ps=ps)
    c["out"] = oracle.kv_append(c["k_src"], c["v_src"], c["app"], c["ctx"], c["k_pool"],
                                c["v_pool"], c["table"])
    got = run_gpu(c)
    assert got[4] == (3 + 5 + 3) * hkv
    assert_same(got, c["out"])


def test_hardware_fp8_encoder_on_every_tie_and_neighbour():
    """One page whose K amax is exactly 448 (scale 1): the kernel's codes for
    every e4m3 value, every midpoint between neighbours and the floats just
    either side of each midpoint equal torch's RNE cast."""
    vals = oracle.fp8_e4m3_table()
    vals = np.unique(vals[np.isfinite(vals)])
    mids = (vals[:-1] + vals[1:]) / 2
    x = np.concatenate([vals, mids, np.nextafter(mids, np.float32(np.inf)),
                        np.nextafter(mids, np.float32(-np.inf))]).astype(np.float32)
    x = np.concatenate([x, [448.0]])
    d = 128
    T = -(-x.size // d)
    padded = np.zeros(T * d, np.float32)
    padded[:x.size] = x
    ps = 16 * -(-T // 16)
    src = torch.from_numpy(padded.reshape(T, 1, d)).cuda()
    k_pool = torch.zeros(1, 1, ps, d, dtype=FP8, device="cuda")
    v_pool = torch.zeros(1, 1, d, ps, dtype=FP8, device="cuda")
    ks = torch.zeros(1, device="cuda")
    vs = torch.zeros(1, device="cuda")
    kv_cache.append(src, src, torch.tensor([0, T], dtype=torch.int32, device="cuda"),
                    torch.tensor([T], dtype=torch.int32, device="cuda"), k_pool, v_pool,
                    torch.zeros(1, 1, dtype=torch.int32, device="cuda"), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert ks.item() == 1.0
    got = raw(k_pool)[0, 0, :T].reshape(-1)[:x.size]
    ref = torch.from_numpy(x).to(FP8).view(torch.uint8).numpy()
    assert np.array_equal(got, ref), int(np.sum(got != ref))


def _rounding_cases(dtype):
    """fp32 values that pin a round-to-nearest-even conversion: for fp16 every
    finite value, every midpoint between neighbours and the floats either
    side of it, the overflow boundary and fp32 denormals; for bf16 random
    fp32 bit patterns over the whole exponent range (denormals and the
    largest finite values included) whose low 16 bits are an exact tie,
    either side of one, zero or random. Both signs, infinities, no NaN."""
    rng = np.random.default_rng(9)
    if dtype == torch.float16:
        vals = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
        mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
        mids = np.append(mids, np.float32(65520.0))
        x = np.concatenate([vals, mids, np.nextafter(mids, np.float32(np.inf)),
                            np.nextafter(mids, np.float32(-np.inf)), [7e4, 1e30, 1e-40, 1e-45]])
    else:
        hi = rng.integers(0, 1 << 16, 40000, dtype=np.uint32) << 16
        lo = rng.choice(np.array([0x8000, 0x7fff, 0x8001, 0, 0xffff], np.uint32), 40000)
        lo = np.where(rng.random(40000) < 0.2, rng.integers(0, 1 << 16, 40000, dtype=np.uint32), lo)
        x = (hi | lo).astype(np.uint32).view(np.float32)
        x = x[np.isfinite(x)]
        x = np.concatenate([x, np.array([0x7f7f8000, 0x7f7fffff, 0x7f7f7fff, 0x00008000, 0x00018000],
                                        np.uint32).view(np.float32)])
    x = np.concatenate([x, [np.inf, 0.0]]).astype(np.float32)
    return np.concatenate([x, -x])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_hardware_16bit_rounding_on_ties_neighbours_and_extremes(dtype):
    """fp32 rows appended into a bf16 / fp16 cache (K token-major, V d-major,
    16-token pages in order): every stored code equals torch's RNE cast of
    its source value."""
    x = _rounding_cases(dtype)
    d, ps = 128, 16
    T = ps * -(-x.size // (d * ps))
    padded = np.zeros(T * d, np.float32)
    padded[:x.size] = x
    npg = T // ps
    src = torch.from_numpy(padded.reshape(T, 1, d)).cuda()
    k_pool = torch.zeros(npg, 1, ps, d, dtype=dtype, device="cuda")
    v_pool = torch.zeros(npg, 1, d, ps, dtype=dtype, device="cuda")
    table = torch.arange(npg, dtype=torch.int32, device="cuda").view(1, npg)
    print(f"case dtype={dtype} values={x.size} rows={T}", flush=True)
    kv_cache.append(src, src, torch.tensor([0, T], dtype=torch.int32, device="cuda"),
                    torch.tensor([T], dtype=torch.int32, device="cuda"), k_pool, v_pool, table)
    torch.cuda.synchronize()
    ref = torch.from_numpy(padded).to(dtype).view(torch.int16).numpy().view(np.uint16)
    got_k = raw(k_pool).reshape(-1)
    got_v = raw(v_pool.permute(0, 1, 3, 2)).reshape(-1)
    assert np.array_equal(got_k, ref), int(np.sum(got_k != ref))
    assert np.array_equal(got_v, ref), int(np.sum(got_v != ref))


@pytest.mark.parametrize("dtype,ps,layout", [
    (torch.bfloat16, 16, "auto"), (torch.bfloat16, 16, "dmajor"), (FP8, 16, "auto"),
    (FP8, 16, "dmajor"), (torch.float16, 16, "auto"), (torch.float16, 16, "dmajor"),
    (torch.bfloat16, 32, "auto"), (FP8, 32, "auto"), (torch.float16, 32, "auto")])
def test_cache_prefill_then_decode_loop(dtype, ps, layout):
    """PagedKvCache: a prefill append, then 20 one-token appends per request
    (page boundaries crossed), mirrored on the oracle; then a decode step over
    the cache against the oracle decode on the same pools. An fp16 cache is
    fed fp16 rows and decoded with fp16 Q (the reference's FlashInfer serving
    dtype), the others bf16. The default V layout is token-major; d-major on
    request."""
    half = torch.float16 if dtype == torch.float16 else torch.bfloat16
    rng = np.random.default_rng(21)
    hkv, hq, d, R = 8, 32, 128, 6
    cache = kv_cache.PagedKvCache(64 if ps == 16 else 40, hkv, d, ps, dtype=dtype,
                                  v_layout=layout)
    lay = cache.v_layout
    assert lay == ("tokmajor" if layout == "auto" else layout)
    rids = list(range(R))
    for r in rids:
        cache.add_request(r)
    host = [raw(cache.k_pool), raw(cache.v_pool),
            None if cache.k_scale is None else cache.k_scale.cpu().numpy(),
            None if cache.v_scale is None else cache.v_scale.cpu().numpy()]

    def step(counts):
        T = int(sum(counts))
        k = torch.from_numpy(rng.standard_normal((T, hkv, d)).astype(np.float32)).to(half)
        v = torch.from_numpy(rng.standard_normal((T, hkv, d)).astype(np.float32)).to(half)
        cache.append(rids, k.cuda(), v.cuda(), counts)
        bt, ctx = cache.block_table(rids)
        app = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        as_t = (lambda a: torch.from_numpy(a).view(FP8)) if dtype == FP8 else \
               (lambda a: torch.from_numpy(a.view(np.int16)).view(dtype))
        kp, vp, ks, vs, err = oracle.kv_append(k, v, app, ctx.cpu().numpy(), as_t(host[0]),
                                               as_t(host[1]), bt.cpu().numpy(), v_layout=lay,
                                               k_scale=host[2], v_scale=host[3])
        assert err == 0
        host[:] = [kp, vp, ks, vs]

    step(rng.integers(1, 100, R).tolist())
    for _ in range(20):
        step([1] * R)
    torch.cuda.synchronize()
    assert np.array_equal(raw(cache.k_pool), host[0])
    assert np.array_equal(raw(cache.v_pool), host[1])
    if dtype == FP8:
        assert np.array_equal(cache.k_scale.cpu().numpy(), host[2])
        assert np.array_equal(cache.v_scale.cpu().numpy(), host[3])
    q = torch.randn(R, hq, d, dtype=half, device="cuda")
    out = torch.empty(R, hq, d, dtype=torch.float32, device="cuda")
    cache.decode(q, rids, out=out)
    bt, ctx = cache.block_table(rids)
    ref = oracle.decode(q, cache.k_pool, cache.v_pool, bt, ctx, k_scale=cache.k_scale,
                        v_scale=cache.v_scale, v_layout=lay)
    r = np.asarray(ref, np.float64)
    assert par_err(out.cpu(), r, f"cache loop {dtype} page {ps}") <= TOL_BF16
    args = sched_pd.build_args(q, cache.k_pool, cache.v_pool, bt, ctx, out=out, v_layout=lay,
                               k_scale=cache.k_scale, v_scale=cache.v_scale)
    assert sched_pd.kernel_kind(args) == "mfma"


def test_table_update_kernel_writes_exactly_the_updates():
    """sched_kv_table_update against numpy: in-range triples written (the
    last of duplicates is not relied on: none here), out-of-range ones
    ignored, n == 0 a no-op; the table around the updates untouched."""
    import ctypes
    import sched_abi as abi
    lib = abi.load_library()
    rng = np.random.default_rng(4)
    rows, width = 37, 70
    host = rng.integers(-5, 1000, (rows, width)).astype(np.int32)
    tab = torch.from_numpy(host).cuda()
    cells = rng.choice(rows * width, 300, replace=False)
    r, c = (cells // width).astype(np.int32), (cells % width).astype(np.int32)
    v = rng.integers(0, 1 << 30, 300).astype(np.int32)
    r[:5] = [-1, rows, -100, rows + 3, rows + 7]  # out of range: ignored
    c[5:9] = [-2, width, width + 1, 1 << 30]
    upd = torch.from_numpy(np.concatenate([r, c, v])).cuda()
    s = torch.cuda.current_stream()
    ptr = ctypes.c_void_p
    assert lib.sched_kv_table_update(ptr(tab.data_ptr()), rows, width, ptr(upd.data_ptr()), 300,
                                     ptr(s.cuda_stream)) == 0
    assert lib.sched_kv_table_update(ptr(tab.data_ptr()), rows, width, ptr(upd.data_ptr()), 0,
                                     ptr(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    want = host.copy()
    ok = (r >= 0) & (r < rows) & (c >= 0) & (c < width)
    want[r[ok], c[ok]] = v[ok]
    assert ok.sum() == 300 - 9
    assert np.array_equal(tab.cpu().numpy(), want)


def test_incremental_block_table_matches_a_rebuild():
    """Steps of one-token and multi-token appends (pages added every few
    steps, rows of different lengths): after each, the device table the
    cache keeps between steps equals the table rebuilt from its page lists."""
    rng = np.random.default_rng(8)
    cache = kv_cache.PagedKvCache(600, 2, 64, 16, dtype=torch.bfloat16)
    rids = list(range(9))
    for r in rids:
        cache.add_request(r)
    k = torch.zeros(400, 2, 64, dtype=torch.bfloat16, device="cuda")
    cache.append(rids, k[:9 * 20], k[:9 * 20], [20] * 9)
    for step in range(60):
        counts = [1] * 9 if step % 7 else rng.integers(1, 40, 9).tolist()
        cache.append(rids, k[:sum(counts)], k[:sum(counts)], counts)
        bt, ctx = cache.block_table(rids)
        got = bt.cpu().numpy()
        for i, r in enumerate(rids):
            n = len(cache.pages[r])
            assert got[i, :n].tolist() == cache.pages[r], (step, r)
            assert (got[i, n:] == -1).all(), (step, r)
        assert ctx.cpu().tolist() == [cache.lens[r] for r in rids]


def _full_size(dtype):
    """Llama-3-8B decode KV (64 requests x 2048 tokens, Hkv 8, d 128, page 16)
    written by one bulk append into a shuffled pool (fp16 rows into an fp16
    cache, bf16 rows otherwise)."""
    R, T, hkv, d, ps = 64, 2048, 8, 128, 16
    g = torch.Generator(device="cuda").manual_seed(3)
    src = torch.float16 if dtype == torch.float16 else torch.bfloat16
    k = torch.randn(R * T, hkv, d, device="cuda", generator=g).to(src)
    v = torch.randn(R * T, hkv, d, device="cuda", generator=g).to(src)
    npg = R * T // ps
    pages = torch.randperm(npg + 512, device="cuda", generator=g)[:npg].int().view(R, T // ps)
    kp = torch.zeros(npg + 512, hkv, ps, d, dtype=dtype, device="cuda")
    vp = torch.zeros(npg + 512, hkv, d, ps, dtype=dtype, device="cuda")
    ks = vs = None
    if dtype == FP8:
        ks = torch.zeros((npg + 512) * hkv, device="cuda")
        vs = torch.zeros_like(ks)
    app = torch.arange(0, R * T + 1, T, dtype=torch.int32, device="cuda")
    ctx = torch.full((R,), T, dtype=torch.int32, device="cuda")
    errors = torch.zeros(1, dtype=torch.int32, device="cuda")
    kv_cache.append(k, v, app, ctx, kp, vp, pages, k_scale=ks, v_scale=vs, max_append=T,
                    errors=errors)
    torch.cuda.synchronize()
    assert errors.item() == 0
    # gather back into [R*T, hkv, d] through the table
    flat = pages.reshape(-1).long()
    kb = kp[flat].permute(0, 2, 1, 3).reshape(R * T, hkv, d)
    vb = vp[flat].permute(0, 3, 1, 2).reshape(R * T, hkv, d)
    return k, v, kb, vb, flat, ks, vs, hkv, ps


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_full_size_append_reads_back_identically(dtype):
    k, v, kb, vb, *_ = _full_size(dtype)
    assert torch.equal(kb, k) and torch.equal(vb, v)


def test_full_size_fp8_append_scales_and_error_bound():
    k, v, kb, vb, flat, ks, vs, hkv, ps = _full_size(FP8)
    for src, back, sc in ((k, kb, ks), (v, vb, vs)):
        amax = src.float().abs().view(-1, ps, hkv, 128).amax(dim=(1, 3))      # [pages, hkv]
        s = sc.view(-1, hkv)[flat]                                             # [pages, hkv]
        # the least power of two with amax <= 448 s
        assert torch.all(amax <= 448 * s) and torch.all(amax > 224 * s)
        assert torch.all(torch.frexp(s).mantissa == 0.5)
        deq = back.float().view(-1, ps, hkv, 128) * s[:, None, :, None]
        x = src.float().view(-1, ps, hkv, 128)
        bound = x.abs() * 2 ** -4 + s[:, None, :, None] * 2 ** -10
        assert torch.all((deq - x).abs() <= bound)


def test_flashinfer_fp16_nhd_cache_in_place():
    """The reference's FlashInfer serving shape (test/py/eval_pi_makespan.py:
    31-60: fp16 Q and NHD cache, page 16, Hq 16 / Hkv 2, d 128, full last
    pages) decoded in place on the MFMA kernel against the oracle."""
    rng = np.random.default_rng(33)
    P, ps, hkv, hq, d, R = 96, 16, 2, 16, 128, 8
    pages = rng.integers(1, 12, R).astype(np.int32)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)).cuda()
    indices = torch.from_numpy(rng.permutation(P)[:pages.sum()].astype(np.int32)).cuda()
    last = torch.full((R,), ps, dtype=torch.int32, device="cuda")
    ctx = kv_cache.ctx_lens_from_last_page_len(indptr, last, ps)
    kv = torch.randn(P, 2, ps, hkv, d, device="cuda").half()
    q = torch.randn(R, hq, d, device="cuda").half()
    kview, vview = kv_cache.nhd_views(kv)
    out = torch.empty(R, hq, d, dtype=torch.float16, device="cuda")
    args = sched_pd.build_args(q, kview, vview, indices, ctx, out=out, page_indptr=indptr,
                               v_layout="tokmajor")
    assert sched_pd.kernel_kind(args) == "mfma"
    sched_pd.launch(args)
    torch.cuda.synchronize()
    ref = np.asarray(oracle.decode(q, kview, vview, indices, ctx, page_indptr=indptr,
                                   v_layout="tokmajor"), np.float64)
    got = out.float().cpu().double().numpy()
    assert par_err(got, ref) <= TOL_BF16


def test_flashinfer_nhd_cache_decodes_in_place_and_imports():
    """A FlashInfer NHD cache [P, 2, page, Hkv, d] with its CSR table
    (indptr, indices, last_page_len; test/py/eval_pi_makespan.py:46-60) is
    decoded in place (strided views, token-major V) and, imported through the
    writer into the d-major layout, by the MFMA kernel; both match the oracle
    on the same cache."""
    rng = np.random.default_rng(31)
    P, ps, hkv, hq, d = 64, 16, 4, 16, 128
    pages = np.array([3, 1, 7, 2, 9, 5], np.int32)
    R = pages.size
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)).cuda()
    indices = torch.from_numpy(rng.permutation(P)[:pages.sum()].astype(np.int32)).cuda()
    last = torch.from_numpy(rng.integers(1, ps + 1, R).astype(np.int32)).cuda()
    ctx = kv_cache.ctx_lens_from_last_page_len(indptr, last, ps)
    kv = (torch.randn(P, 2, ps, hkv, d, device="cuda") / d ** 0.5).bfloat16()
    q = (torch.randn(R, hq, d, device="cuda") / d ** 0.5).bfloat16()
    kview, vview = kv_cache.nhd_views(kv)
    out = torch.empty(R, hq, d, dtype=torch.float32, device="cuda")
    args = sched_pd.build_args(q, kview, vview, indices, ctx, out=out, page_indptr=indptr,
                               v_layout="tokmajor")
    assert sched_pd.kernel_kind(args) == "mfma"
    sched_pd.launch(args)
    torch.cuda.synchronize()
    ref = np.asarray(oracle.decode(q, kview, vview, indices, ctx, page_indptr=indptr,
                                   v_layout="tokmajor"), np.float64)
    err = lambda o: par_err(o.cpu(), ref, "nhd in place")  # noqa: E731
    assert err(out) <= TOL_BF16
    # import: gather each request's tokens in order and append them
    rows_k, rows_v = [], []
    for r in range(R):
        pg = indices[int(indptr[r]):int(indptr[r + 1])].long()
        n = int(ctx[r])
        rows_k.append(kv[pg, 0].reshape(-1, hkv, d)[:n])
        rows_v.append(kv[pg, 1].reshape(-1, hkv, d)[:n])
    cache = kv_cache.PagedKvCache(P, hkv, d, ps, dtype=torch.bfloat16)
    for r in range(R):
        cache.add_request(r)
    cache.append(list(range(R)), torch.cat(rows_k), torch.cat(rows_v),
                 ctx.cpu().tolist())
    out2 = torch.empty_like(out)
    cache.decode(q, list(range(R)), out=out2)
    torch.cuda.synchronize()
    assert err(out2) <= TOL_BF16
    # same values, same page order per request: the token-major and d-major
    # MFMA paths give the same bits
    assert torch.equal(out, out2)
