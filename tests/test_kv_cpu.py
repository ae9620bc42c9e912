"""The KV-cache writer without a GPU: the oracle's encoders pinned against
torch's own conversions, the power-of-two scale rule against its closed
form, the append restatement against a readback through the page table and
an independent scatter, the ABI mirror, and the host page allocator."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
from kv_cache import OutOfPages, PageAllocator, PagedKvCache, ctx_lens_from_last_page_len
from kv_cases import FP8, append_case, fp8_values, pages_of, random_pool, readback

# --- encoders ------------------------------------------------------------------

def test_fp8_encoder_matches_torch_on_ties_neighbours_and_random():
    vals = np.sort(fp8_values()[np.isfinite(fp8_values())])
    vals = np.unique(vals)
    mids = (vals[:-1] + vals[1:]) / 2                       # exact ties
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf))]).astype(np.float32)
    rng = np.random.default_rng(0)
    rnd = (rng.choice([-1, 1], 60000) * np.exp2(rng.uniform(-14, np.log2(448), 60000)))
    x = np.concatenate([vals, mids, near, rnd]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    ours = oracle.fp8_e4m3_encode(x)
    ref = torch.from_numpy(x).to(FP8).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    # every code decodes and re-encodes to itself
    codes = np.array([c for c in range(256) if c not in (0x7f, 0xff)], np.uint8)
    assert np.array_equal(oracle.fp8_e4m3_encode(fp8_values()[codes]), codes)


def test_fp8_encoder_saturates_and_keeps_nan():
    assert list(oracle.fp8_e4m3_encode([448.0, 449.0, 1e30, -1e30, np.inf])) == \
        [0x7e, 0x7e, 0x7e, 0xfe, 0x7e]
    assert oracle.fp8_e4m3_encode([np.nan])[0] & 0x7f == 0x7f


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(50000).astype(np.float32) * np.exp2(rng.integers(-30, 30, 50000))
    bits = x.view(np.uint32)
    ties = ((bits & ~np.uint32(0xffff)) | np.uint32(0x8000)).view(np.float32)  # exact ties
    x = np.concatenate([x, ties])
    lib = oracle.load()
    ours = np.array([lib.oracle_float_to_bf16(float(v)) for v in x], np.uint16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_rne_matches_numpy_and_torch():
    """binary16 encoding against numpy's and torch's IEEE conversions: every
    representable value, the exact midpoints between neighbours (ties to
    even), one ulp either side of them, the overflow boundary and random
    values across the subnormal and normal range."""
    vals = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = (vals[:-1].astype(np.float64) + vals[1:]) / 2        # exact in fp32
    mids = np.append(mids, 65520.0).astype(np.float32)            # 65504 | inf
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf))])
    rng = np.random.default_rng(2)
    rnd = rng.standard_normal(40000).astype(np.float32) * np.exp2(rng.integers(-28, 17, 40000))
    x = np.concatenate([vals, mids, near, rnd, [7e4, 1e30, np.inf, 1e-30, 0.0]]).astype(np.float32)
    x = np.concatenate([x, -x])
    ours = oracle.f16_encode(x)
    with np.errstate(over="ignore"):
        assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))
    assert np.array_equal(ours, torch.from_numpy(x).half().view(torch.int16).numpy().view(np.uint16))
    # every finite code re-encodes to itself; overflow and NaN
    assert np.array_equal(oracle.f16_encode(vals), np.arange(0, 0x7c00, dtype=np.uint16))
    assert list(oracle.f16_encode([65519.99, 65520.0, -65520.0])) == [0x7bff, 0x7c00, 0xfc00]
    assert oracle.f16_encode([np.nan])[0] & 0x7e00 == 0x7e00


@pytest.mark.parametrize("a", [448.0, 448.0 * 2 ** -20, 449.0, 224.0, 224.5, 1.0, 3e38,
                               1e-40, 2 ** -130, 0.875, 0.8751])
def test_pow2_scale_closed_form(a):
    s = oracle.pow2_scale(a)
    m, e = np.frexp(np.float32(s))
    assert m == 0.5                                   # a power of two
    assert a <= 448 * s                               # covers a
    assert s == 2.0 ** -126 or a > 224 * s            # and is the least such
    assert oracle.pow2_scale(0.0) == 0.0


# --- append restatement ------------------------------------------------------------

@pytest.mark.parametrize("v_layout", ["dmajor", "tokmajor"])
@pytest.mark.parametrize("csr", [False, True])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
def test_oracle_append_reads_back_exactly(v_layout, csr, dt):
    c = append_case(3, dt, v_layout, csr,
                    src_dtype=torch.float16 if dt == torch.float16 else torch.bfloat16)
    assert c["out"][4] == 0
    for r in range(5):
        for i in range(c["n"][r]):
            k, v = readback(c, r, c["prior"][r] + i)
            row = c["app"][r] + i
            assert np.array_equal(k, c["k_src"][row].to(dt).double().numpy())
            assert np.array_equal(v, c["v_src"][row].to(dt).double().numpy())


def test_oracle_append_matches_an_independent_scatter():
    """The position rule restated as FlashInfer's (batch_indices, positions)
    scatter in numpy: every other byte of the pools is left as it was."""
    c = append_case(4, torch.bfloat16, "dmajor")
    kp0 = c["k_pool"].view(torch.int16).numpy().view(np.uint16).copy()
    vp0 = c["v_pool"].view(torch.int16).numpy().view(np.uint16).copy()
    ksrc = c["k_src"].view(torch.int16).numpy().view(np.uint16)
    vsrc = c["v_src"].view(torch.int16).numpy().view(np.uint16)
    ps = c["ps"]
    for r in range(5):
        for i in range(c["n"][r]):
            pos = c["ctx"][r] - c["n"][r] + i
            page, t = pages_of(c, r)[pos // ps], pos % ps
            kp0[page, :, t, :] = ksrc[c["app"][r] + i]
            vp0[page, :, :, t] = vsrc[c["app"][r] + i]
        end = c["ctx"][r]
        if end % ps and c["n"][r]:   # d-major group padding after the last slot
            page = pages_of(c, r)[(end - 1) // ps]
            t1 = end % ps
            vp0[page, :, :, t1:(t1 + 3) & ~3] = 0
    assert np.array_equal(c["out"][0], kp0)
    assert np.array_equal(c["out"][1], vp0)


def test_a_shifted_position_rule_is_caught():
    """Planted mistake, in the oracle's inputs: positions one later than the
    rule (ctx_lens + 1) fail the readback check."""
    c = append_case(3, torch.bfloat16, "dmajor", n=[5, 9, 3, 17, 2], prior=[3, 0, 14, 16, 30])
    bad = dict(c)
    bad["out"] = oracle.kv_append(c["k_src"], c["v_src"], c["app"], c["ctx"] + 1, c["k_pool"],
                                  c["v_pool"], np.pad(c["table"], ((0, 0), (0, 1)),
                                                      constant_values=0))
    bad["table"] = np.pad(c["table"], ((0, 0), (0, 1)), constant_values=0)
    k, _ = readback(bad, 1, 0)
    assert not np.array_equal(k, c["k_src"][c["app"][1]].double().numpy())


def test_oracle_fp8_bulk_append_scales_and_error_bound():
    c = append_case(5, FP8, "dmajor", prior=[0] * 5, n=[16, 33, 7, 64, 1])
    kp, vp, ksc, vsc, err = c["out"]
    assert err == 0
    hkv = 2
    for r in range(5):
        for b, page in enumerate(pages_of(c, r)[:-(-c["ctx"][r] // 16)]):
            lo, hi = b * 16, min(c["ctx"][r], (b + 1) * 16)
            rows = slice(c["app"][r] + lo, c["app"][r] + hi)
            for h in range(hkv):
                for src, sc in ((c["k_src"], ksc), (c["v_src"], vsc)):
                    a = float(src[rows, h].float().abs().max())
                    assert sc[page * hkv + h] == oracle.pow2_scale(a)
    for r in range(5):
        for i in range(c["n"][r]):
            k, v = readback(c, r, i)
            for got, src in ((k, c["k_src"]), (v, c["v_src"])):
                x = src[c["app"][r] + i].double().numpy()
                page = pages_of(c, r)[i // 16]
                s = (ksc if src is c["k_src"] else vsc)[page * hkv:(page + 1) * hkv, None]
                # e4m3: relative half-ulp 2^-4 (normal), absolute 2^-10 * s (subnormal)
                assert np.all(np.abs(got - x) <= np.abs(x) * 2 ** -4 + s * 2 ** -10 + 1e-30)


def test_oracle_fp8_token_by_token_equals_bulk_up_to_subnormal_double_rounding():
    rng = np.random.default_rng(7)
    hkv, d, ps, T = 2, 16, 16, 16
    x = torch.from_numpy((rng.standard_normal((T, hkv, d)) *
                          np.exp2(rng.integers(-6, 6, (T, 1, 1)))).astype(np.float32)).bfloat16()
    y = x * 2
    pool = lambda: torch.zeros(1, hkv, ps, d).to(FP8)       # noqa: E731
    vpool = lambda: torch.zeros(1, hkv, d, ps).to(FP8)      # noqa: E731
    table = np.zeros((1, 1), np.int32)
    bulk = oracle.kv_append(x, y, [0, T], [T], pool(), vpool(), table,
                            k_scale=np.zeros(hkv, np.float32), v_scale=np.zeros(hkv, np.float32))
    kp, vp = pool().view(torch.uint8).numpy(), vpool().view(torch.uint8).numpy()
    ks, vs = np.zeros(hkv, np.float32), np.zeros(hkv, np.float32)
    for t in range(T):
        kp, vp, ks, vs, err = oracle.kv_append(x[t:t + 1], y[t:t + 1], [0, 1], [t + 1],
                                               torch.from_numpy(kp).view(FP8),
                                               torch.from_numpy(vp).view(FP8), table,
                                               k_scale=ks, v_scale=vs)
        assert err == 0
    assert np.array_equal(ks, bulk[2]) and np.array_equal(vs, bulk[3])
    for got, ref in ((kp, bulk[0]), (vp, bulk[1])):
        diff = got != ref
        # only codes that are subnormal in the bulk encoding may differ
        assert np.all(np.abs(fp8_values()[ref[diff]]) < 2 ** -6)
        assert diff.mean() < 0.05


def test_oracle_counts_errors_and_writes_nothing_for_them():
    rng = np.random.default_rng(9)
    hkv, d, ps = 2, 8, 8
    k_pool = random_pool((4, hkv, ps, d), torch.bfloat16, rng)
    v_pool = random_pool((4, hkv, d, ps), torch.bfloat16, rng)
    src = torch.ones(12, hkv, d, dtype=torch.bfloat16)
    # r0: page id 9 outside the pool; r1: n > ctx; r2: table entry -1;
    # r3: a valid single-token append into page 2 slot 0
    table = np.array([[9, 0], [1, 0], [-1, 0], [2, 0]], np.int32)
    app = [0, 3, 8, 11, 12]
    ctx = [3, 2, 3, 1]
    kp, vp, _, _, err = oracle.kv_append(src, src, app, ctx, k_pool, v_pool, table)
    assert err == (3 + 5 + 3) * hkv
    k0 = k_pool.view(torch.int16).numpy().view(np.uint16)
    changed = np.argwhere(kp != k0)
    assert set(changed[:, 0].tolist()) <= {2}
    assert np.all(kp[2, :, 0, :] == 0x3f80)


# --- ABI mirror ------------------------------------------------------------------

def test_kv_struct_layout_matches_c():
    lib = oracle.load()
    buf = (ctypes.c_int64 * 16)()
    n = lib.oracle_kv_args_layout(buf, 16)
    A = abi.SchedKvAppendArgs
    assert list(buf[:n]) == [ctypes.sizeof(A), A.num_pages.offset, A.k_src.offset,
                             A.src_tok_stride.offset, A.append_indptr.offset, A.k_pool.offset,
                             A.k_page_stride.offset, A.v_dim_stride.offset, A.k_scale.offset,
                             A.errors.offset]


def test_kv_default_args_match(schedlib):
    c = abi.SchedKvAppendArgs()
    schedlib.sched_kv_default_args(ctypes.byref(c))
    assert bytes(c) == bytes(abi.default_kv_args())


def kv_fake(**kw):
    a = abi.default_kv_args()
    a.num_requests, a.num_kv_heads, a.head_dim, a.page_size = 2, 8, 128, 16
    a.num_tokens, a.num_pages, a.bt_stride = 2, 64, 4
    a.src_tok_stride, a.src_head_stride = 8 * 128, 128
    a.k_page_stride, a.k_head_stride, a.k_tok_stride = 8 * 16 * 128, 16 * 128, 128
    a.v_page_stride, a.v_head_stride, a.v_tok_stride, a.v_dim_stride = 8 * 16 * 128, 16 * 128, 1, 16
    for i, f in enumerate(("k_src", "v_src", "append_indptr", "ctx_lens", "block_table",
                           "k_pool", "v_pool")):
        setattr(a, f, ctypes.c_void_p(0x10000 * (i + 1)))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(abi_version=7), "abi_version"),
    (dict(src_dtype=abi.FP8_E4M3), "src dtype"),
    (dict(kv_dtype=5), "kv dtype"),
    (dict(head_dim=6), "head_dim"),
    (dict(page_size=300), "page_size"),
    (dict(k_pool=None), "required pointer"),
    (dict(kv_dtype=abi.FP8_E4M3), "k_scale"),
    (dict(bt_stride=0), "bt_stride"),
    (dict(num_pages=0), "num_pages"),
    (dict(v_tok_stride=2, v_dim_stride=16), "d-major"),
    (dict(k_tok_stride=130), "multiples of 4"),
    (dict(k_pool=ctypes.c_void_p(0x10002)), "aligned"),
    (dict(heads_per_group=3), "heads_per_group"),
    (dict(heads_per_group=128), "heads_per_group"),
])
def test_kv_append_rejects_invalid_args(schedlib, kw, msg):
    a = kv_fake(**kw)
    assert schedlib.sched_kv_append(ctypes.byref(a), None) == -1
    assert msg in abi.last_error()


def test_kv_append_with_no_requests_is_a_no_op(schedlib):
    assert schedlib.sched_kv_append(ctypes.byref(kv_fake(num_requests=0)), None) == 0


# --- host bookkeeping ----------------------------------------------------------------

def test_page_allocator():
    a = PageAllocator(8)
    p = a.alloc(3)
    assert list(p) == [0, 1, 2] and a.num_free == 5
    q = a.alloc(5)
    assert sorted(np.concatenate([p, q]).tolist()) == list(range(8))
    with pytest.raises(OutOfPages):
        a.alloc(1)
    a.free(p[1:2])
    assert list(a.alloc(1)) == [1]                  # LIFO reuse
    with pytest.raises(ValueError):
        a.free([1, 1])
    a.free([1])
    with pytest.raises(ValueError):
        a.free([1])                                 # double free
    with pytest.raises(ValueError):
        a.free([8])


def test_cache_bookkeeping_and_tables_on_cpu():
    c = PagedKvCache(10, 2, 8, page_size=4, dtype=torch.bfloat16, device="cpu")
    for rid in "abc":
        c.add_request(rid)
    c.reserve(["a", "b", "c"], [5, 4, 0])
    c.lens.update(a=5, b=4, c=0)
    assert [len(c.pages[r]) for r in "abc"] == [2, 1, 0]
    bt, ctx = c.block_table(["a", "b", "c"])
    assert bt.shape[0] == 3 and bt.shape[1] >= 2 and ctx.tolist() == [5, 4, 0]
    assert bt[0, :2].tolist() == c.pages["a"] and bt[1, 0] == c.pages["b"][0]
    assert (bt[1, 1:] == -1).all() and (bt[2] == -1).all()
    indptr, idx, last = c.csr(["a", "b", "c"])
    assert indptr.tolist() == [0, 2, 3, 3] and last.tolist() == [1, 4, 0]
    assert ctx_lens_from_last_page_len(indptr, last, 4).tolist() == [5, 4, 0]
    with pytest.raises(OutOfPages):
        c.reserve(["c"], [100])
    assert c.allocator.num_free == 7               # all or nothing
    c.release("a")
    assert c.allocator.num_free == 9


def test_block_table_updates_in_place_like_a_rebuild():
    """Steps that add pages to some requests upload only those entries; the
    table then equals one built from scratch. Growing past the width, a new
    request list and a release rebuild it."""
    rng = np.random.default_rng(4)
    c = PagedKvCache(4000, 2, 8, page_size=4, dtype=torch.bfloat16, device="cpu")
    rids = list(range(12))
    for r in rids:
        c.add_request(r)

    def fresh():
        w = max(len(c.pages[r]) for r in rids)
        t = np.full((len(rids), w), -1, np.int32)
        for i, r in enumerate(rids):
            t[i, :len(c.pages[r])] = c.pages[r]
        return t

    c.reserve(rids, rng.integers(1, 40, 12).tolist())
    for r in rids:
        c.lens[r] = 4 * len(c.pages[r])
    bt, _ = c.block_table(rids)
    first = bt
    for step in range(60):
        grow = rng.integers(0, 20, 12)
        c.reserve(rids, grow.tolist())
        for r, g in zip(rids, grow):
            c.lens[r] += int(g)
        bt, ctx = c.block_table(rids)
        want = fresh()
        got = bt.numpy()
        assert np.array_equal(got[:, :want.shape[1]], want), step
        assert (got[:, want.shape[1]:] == -1).all()
        assert ctx.tolist() == [c.lens[r] for r in rids]
    assert bt.shape[1] > first.shape[1]          # outgrew the width once at least
    bt2, _ = c.block_table(rids[::-1])             # another list: rebuilt
    assert np.array_equal(bt2.numpy()[:, :want.shape[1]], want[::-1])
    c.release(rids[0])
    bt3, _ = c.block_table(rids[1:])
    assert np.array_equal(bt3.numpy()[:, :want.shape[1]], want[1:])


def test_cache_append_rolls_back_a_rejected_launch():
    c = PagedKvCache(8, 2, 8, page_size=4, dtype=torch.bfloat16, device="cpu")
    c.add_request("a")
    c.add_request("b")
    rows = torch.zeros(5, 2, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):          # host tensors: the launcher refuses them
        c.append(["a", "b"], rows, rows, [2, 3])
    assert c.lens == {"a": 0, "b": 0} and c.pages == {"a": [], "b": []}
    assert c.allocator.num_free == 8
    with pytest.raises(ValueError):
        c.append(["a", "a"], rows, rows, [2, 3])


def test_cache_v_layout_choice():
    """token-major V by default for every dtype and page size (what a serving
    step of append + decode runs fastest on); d-major on request."""
    fp8 = torch.float8_e4m3fn
    for dt, ps, lay in ((torch.bfloat16, 16, "tokmajor"), (torch.bfloat16, 32, "tokmajor"),
                        (torch.float16, 64, "tokmajor"), (fp8, 16, "tokmajor"),
                        (torch.float32, 32, "tokmajor")):
        c = PagedKvCache(4, 2, 8, page_size=ps, dtype=dt, device="cpu")
        assert c.v_layout == lay
        assert tuple(c.v_pool.shape) == ((4, 2, 8, ps) if lay == "dmajor" else (4, 2, ps, 8))
    c = PagedKvCache(4, 2, 8, page_size=32, dtype=torch.bfloat16, device="cpu", v_layout="dmajor")
    assert tuple(c.v_pool.shape) == (4, 2, 8, 32)
    with pytest.raises(ValueError):
        PagedKvCache(4, 2, 8, page_size=32, device="cpu", v_layout="hnd")


def test_lengths_view_slots_and_failed_append_rollback():
    """cache.lens reads and writes the per-request arrays; released slots are
    reused; an append whose launch is rejected (here: host pools) leaves
    lengths, page lists and the allocator as they were."""
    c = PagedKvCache(64, 2, 8, page_size=4, dtype=torch.bfloat16, device="cpu")
    for rid in ("a", "b", "c"):
        c.add_request(rid)
    c.reserve(["a", "b", "c"], [6, 1, 9])
    c.lens.update(a=6, b=1, c=9)
    assert dict(c.lens) == {"a": 6, "b": 1, "c": 9} and len(c.lens) == 3
    got = c.lengths(["c", "a"])
    assert got.tolist() == [9, 6]
    got[0] = 100                            # a copy
    assert c.lens["c"] == 9
    with pytest.raises(KeyError):
        c.lengths(["a", "zz"])
    with pytest.raises(KeyError):
        c.lens["zz"] = 3
    with pytest.raises(TypeError):
        del c.lens["a"]
    before = ({r: list(p) for r, p in c.pages.items()}, dict(c.lens), c.allocator.num_free)
    k = torch.zeros(3 + 4 + 8, 2, 8, dtype=torch.bfloat16)
    with pytest.raises(Exception):
        c.append(["a", "b", "c"], k, k, [3, 4, 8])
    assert ({r: list(p) for r, p in c.pages.items()}, dict(c.lens),
            c.allocator.num_free) == before
    with pytest.raises(ValueError):
        c.append(["a", "a"], k[:2], k[:2], [1, 1])
    c.release("b")
    c.add_request("d")                      # takes b's slot
    assert c.lens["d"] == 0 and c.pages["d"] == [] and "b" not in c.lens
    c.reserve(["d", "a"], [5, 2])
    c.lens["d"] = 5
    bt, ctx = c.block_table(["d", "a"])
    assert ctx.tolist() == [5, 6] and bt[0, :2].tolist() == c.pages["d"]


def test_truncate_frees_the_pages_past_the_new_lengths():
    c = PagedKvCache(32, 1, 8, page_size=4, dtype=torch.bfloat16, device="cpu")
    for rid in ("a", "b"):
        c.add_request(rid)
    c.reserve(["a", "b"], [10, 3])
    c.lens.update(a=10, b=3)
    free0 = c.allocator.num_free
    pa = list(c.pages["a"])
    c.truncate(["a", "b"], [5, 3])
    assert c.lens["a"] == 5 and c.pages["a"] == pa[:2] and c.lens["b"] == 3
    assert c.allocator.num_free == free0 + 1
    with pytest.raises(ValueError):
        c.truncate(["a"], [6])
    c.truncate(["a"], [0])
    assert c.pages["a"] == [] and c.allocator.num_free == free0 + 3
    bt, ctx = c.block_table(["a", "b"])
    assert ctx.tolist() == [0, 3] and (bt[0] == -1).all()
