"""The C ABI without a GPU: the library loads, exports exactly what
include/*.h declare, the ctypes mirror matches the C layout, and the
host-side argument validation / kernel selection behave (no device calls)."""
import ctypes
import os
import re
import subprocess

import pytest

import oracle
import sched_abi as abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("sched_pd.h", "sched_kv.h")]


def test_every_header_is_listed():
    assert sorted(os.listdir(os.path.join(ROOT, "include"))) == sorted(
        os.path.basename(h) for h in HEADERS)


def header_functions():
    src = "".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*[A-Za-z_][\w \*]*?\b(\w+)\s*\([^;{]*\)\s*;", src, re.M)
    return sorted(set(n for n in names if n not in ("static_assert",)))


def test_header_declares_what_the_mirror_binds():
    assert header_functions() == sorted(abi.SIGNATURES)


def test_library_exports_every_declared_symbol(schedlib):
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [f for f in header_functions() if f not in exported]
    assert not missing, missing
    for f in header_functions():
        assert getattr(schedlib, f) is not None


def test_device_slot_symbols_exist(schedlib):
    # the __sched_* slots live in the device code object; the host side keeps
    # their shadow symbols for hipMemcpyToSymbol.
    out = subprocess.run(["nm", "-C", abi.LIB_PATH], capture_output=True, text=True).stdout
    for s in ("__sched_task_order", "__sched_ctrl", "__sched_timer", "__sched_queue"):
        assert s in out, s


def test_struct_layout_matches_c():
    lib = oracle.load()
    buf = (ctypes.c_int64 * 32)()
    n = lib.oracle_args_layout(buf, 32)
    A = abi.SchedDecodeArgs
    expect = [ctypes.sizeof(A), A.sm_scale.offset, A.lin_w_period.offset, A.q.offset,
              A.k_page_stride.offset, A.v_dim_stride.offset, A.k_scale.offset,
              A.block_table.offset, A.lin_w.offset, A.order.offset, A.queue.offset,
              32 + 8 * abi.SCHED_MAX_TASKS, A.tile_pages.offset, A.tiles.offset,
              A.num_tiles.offset, A.workspace.offset, A.workspace_bytes.offset]
    assert list(buf[:n]) == expect


def test_default_args_match(schedlib):
    c = abi.SchedDecodeArgs()
    schedlib.sched_pd_default_args(ctypes.byref(c))
    p = abi.default_args()
    assert bytes(c) == bytes(p)


def test_plane_constants_mirror_header():
    src = open(HEADERS[0]).read()
    def define(name):
        return int(re.search(rf"#define {name} (\w+)", src).group(1).rstrip("u"), 0)
    assert define("SCHED_MAX_TASKS") == abi.SCHED_MAX_TASKS
    assert define("SCHED_CTRL_ROWS_OFF") == abi.CTRL_ROWS_OFF
    assert define("SCHED_CTRL_FLAGS_OFF") == abi.CTRL_FLAGS_OFF
    assert define("SCHED_CTRL_ORDER_SIZE_OFF") == abi.CTRL_ORDER_SIZE_OFF
    assert define("SCHED_PD_ABI_VERSION") == abi.ABI_VERSION
    assert define("SCHED_PD_FLAG_SHED_LOADS") == abi.FLAG_SHED_LOADS
    assert define("SCHED_PD_TILES_PAIRS") == abi.TILES_PAIRS
    assert define("SCHED_PD_TILES_RANGED") == abi.TILES_RANGED
    import sched_rt
    assert (sched_rt.ORDER_OFF, sched_rt.CTRL_OFF, sched_rt.TIMER_OFF, sched_rt.QUEUE_OFF) == \
        (0, 0x40000, 0x80000, 0xC0000)


def fake_args(**kw):
    """Argument block with fake (never dereferenced) 256-aligned addresses."""
    a = abi.default_args()
    a.mode = abi.SOFTMAX
    a.kv_dtype = a.q_dtype = a.o_dtype = abi.BF16
    a.num_requests, a.num_q_heads, a.num_kv_heads = 4, 32, 8
    a.head_dim, a.page_size, a.bt_stride = 128, 16, 8
    a.k_page_stride, a.k_head_stride, a.k_tok_stride = 8 * 16 * 128, 16 * 128, 128
    a.v_page_stride, a.v_head_stride, a.v_tok_stride, a.v_dim_stride = 8 * 16 * 128, 16 * 128, 1, 16
    for i, f in enumerate(("q", "out", "k_pool", "v_pool", "block_table", "ctx_lens")):
        setattr(a, f, ctypes.c_void_p(0x10000 * (i + 1)))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def kind(lib, a):
    return lib.sched_paged_decode_kernel_kind(ctypes.byref(a))


def test_kernel_selection(schedlib):
    assert kind(schedlib, fake_args()) == 1                               # bf16 GQA -> MFMA
    assert kind(schedlib, fake_args(kv_dtype=abi.FP8_E4M3)) == 1          # fp8 -> MFMA
    assert kind(schedlib, fake_args(flags=abi.FLAG_FORCE_VALU)) == 0
    assert kind(schedlib, fake_args(q_dtype=abi.F32)) == 0                # fp32 Q keeps fp32 scores
    assert kind(schedlib, fake_args(kv_dtype=abi.F32, q_dtype=abi.F32)) == 0
    assert kind(schedlib, fake_args(v_tok_stride=128, v_dim_stride=1)) == 1  # token-major V
    assert kind(schedlib, fake_args(v_tok_stride=1024, v_dim_stride=1)) == 1  # NHD rows, Hkv 8
    assert kind(schedlib, fake_args(v_tok_stride=132, v_dim_stride=1)) == 0  # rows not 16-B aligned
    assert kind(schedlib, fake_args(kv_dtype=abi.FP8_E4M3, v_tok_stride=128,
                                    v_dim_stride=1)) == 1                    # fp8 token-major V
    assert kind(schedlib, fake_args(kv_dtype=abi.FP8_E4M3, v_tok_stride=132,
                                    v_dim_stride=1)) == 0                    # rows not 8-B aligned
    assert kind(schedlib, fake_args(page_size=32, v_dim_stride=32)) == 1  # 2 blocks per page
    assert kind(schedlib, fake_args(page_size=256, v_dim_stride=256)) == 1
    assert kind(schedlib, fake_args(page_size=48, v_dim_stride=48)) == 0  # not a power of two
    assert kind(schedlib, fake_args(page_size=32, v_dim_stride=16)) == 0  # V rows not one page
    assert kind(schedlib, fake_args(num_q_heads=28, num_kv_heads=4)) == 1   # G = 7
    f16 = dict(kv_dtype=abi.F16, q_dtype=abi.F16, o_dtype=abi.F16)
    assert kind(schedlib, fake_args(**f16)) == 1                            # fp16 cache + Q
    assert kind(schedlib, fake_args(v_tok_stride=1024, v_dim_stride=1, **f16)) == 1  # NHD
    assert kind(schedlib, fake_args(kv_dtype=abi.F16, q_dtype=abi.BF16)) == 0
    assert kind(schedlib, fake_args(page_size=32, v_dim_stride=32, **f16)) == 1   # fp16, 32-token pages
    assert kind(schedlib, fake_args(kv_dtype=abi.F16, q_dtype=abi.FP8_E4M3)) == -1
    # 1..3 q-heads per kv-head over token-major rows: the MFMA kernel where it
    # applies, else one wave per work item
    mha = dict(num_q_heads=8, num_kv_heads=8, v_tok_stride=128, v_dim_stride=1)
    assert kind(schedlib, fake_args(**mha)) == 1                             # bf16 d 128: MFMA
    assert kind(schedlib, fake_args(**mha, flags=abi.FLAG_NO_MFMA)) == 2     # -> one wave
    assert kind(schedlib, fake_args(**mha, flags=abi.FLAG_NO_WAVE)) == 1
    assert kind(schedlib, fake_args(**dict(mha, num_q_heads=16))) == 1       # G = 2: MFMA
    assert kind(schedlib, fake_args(**dict(mha, num_q_heads=24))) == 1       # G = 3: MFMA
    assert kind(schedlib, fake_args(**dict(mha, num_q_heads=24), q_dtype=abi.F32)) == 2
    assert kind(schedlib, fake_args(**dict(mha, num_q_heads=32))) == 1       # G = 4: MFMA
    # the one-wave kernel's lane offsets into a 16-token chunk are 32 bits:
    # a chunk's rows spanning 2 GiB or more go to the general kernel
    d64 = dict(mha, head_dim=64)
    assert kind(schedlib, fake_args(**dict(d64, k_tok_stride=1 << 25, v_tok_stride=1 << 25))) == 2
    assert kind(schedlib, fake_args(**dict(d64, k_tok_stride=1 << 26, v_tok_stride=128))) == 0
    assert kind(schedlib, fake_args(**dict(d64, k_tok_stride=128, v_tok_stride=1 << 26))) == 0
    assert kind(schedlib, fake_args(**mha, pf_dist=3)) == 1                  # a prefetch depth
    assert kind(schedlib, fake_args(v_tok_stride=128, v_dim_stride=1,
                                    flags=abi.FLAG_NO_MFMA)) == 0            # G = 4, no MFMA
    assert kind(schedlib, fake_args(**dict(mha, num_q_heads=16),
                                    flags=abi.FLAG_NO_MFMA)) == 2
    assert kind(schedlib, fake_args(**mha, head_dim=64)) == 2                # bf16 d 64
    assert kind(schedlib, fake_args(**mha, q_dtype=abi.F32)) == 2            # fp32 Q
    assert kind(schedlib, fake_args(**mha, page_size=48)) == 2               # page 48
    assert kind(schedlib, fake_args(**mha, kv_dtype=abi.F32, q_dtype=abi.F32)) == 2
    assert kind(schedlib, fake_args(**mha, head_dim=64, flags=abi.FLAG_NO_WAVE)) == 0
    assert kind(schedlib, fake_args(**mha, kv_dtype=abi.F32, q_dtype=abi.F32,
                                    flags=abi.FLAG_NO_WAVE)) == 0
    assert kind(schedlib, fake_args(**mha, kv_dtype=abi.FP8_E4M3)) == 1      # no fp8 wave kernel
    assert kind(schedlib, fake_args(num_q_heads=8, num_kv_heads=8)) == 1      # d-major V: MFMA
    assert kind(schedlib, fake_args(**mha, mode=abi.LINEAR,
                                    lin_w=ctypes.c_void_p(0x80000))) == 1     # linear: not wave
    assert kind(schedlib, fake_args(**mha, tiles=ctypes.c_void_p(0x90000), num_tiles=8,
                                    tile_pages=4, workspace=ctypes.c_void_p(0xA0000),
                                    workspace_bytes=1 << 20,
                                    flags=abi.FLAG_NO_MFMA)) == 2            # split plans too
    assert kind(schedlib, fake_args(num_q_heads=16, num_kv_heads=8)) == 1  # d-major V: MFMA


def prefetch_range(lib, a):
    lo, hi = ctypes.c_uint32(), ctypes.c_uint32()
    rc = lib.sched_paged_decode_prefetch_range(ctypes.byref(a), ctypes.byref(lo), ctypes.byref(hi))
    return rc, lo.value, hi.value


def test_prefetch_range_and_pf_dist_validation(schedlib):
    """pf_dist picks an urgent ring depth the selected kernel compiles, or
    0 for its deepest; anything else is refused before any launch."""
    fp8 = dict(kv_dtype=abi.FP8_E4M3)
    tok = dict(v_tok_stride=128, v_dim_stride=1)
    cases = [(fake_args(), (2, 4)),                                   # bf16 d-major page 16
             (fake_args(**fp8), (4, 6)),                              # fp8 d-major
             (fake_args(page_size=32, v_dim_stride=32, **fp8), (4, 5)),  # fp8 d-major, 32-token pages
             (fake_args(**tok), (2, 3)),                              # bf16 token-major
             (fake_args(**tok, **fp8), (4, 4)),                       # fp8 token-major
             (fake_args(flags=abi.FLAG_FORCE_VALU), (0, 0))]          # VALU: no ring
    for a, want in cases:
        rc, lo, hi = prefetch_range(schedlib, a)
        assert rc == 0 and (lo, hi) == want, (want, lo, hi)
        for pf in range(0, 9):
            a.pf_dist = pf
            ok = pf == 0 or lo <= pf <= hi
            rc = schedlib.sched_paged_decode_kernel_kind(ctypes.byref(a))
            assert (rc >= 0) == ok, (want, pf)
            if not ok:
                assert "pf_dist" in abi.last_error()
        # the range query ignores the block's own pf_dist
        a.pf_dist = 99
        assert prefetch_range(schedlib, a) == (0, lo, hi)


@pytest.mark.parametrize("field,value,msg", [
    ("abi_version", 7, "abi_version"),
    ("num_q_heads", 33, "multiple"),
    ("num_q_heads", 8 * 17, "at most 16"),
    ("head_dim", 96, "head_dim"),
    ("page_size", 8, "page_size"),
    ("tau_scope", 5, "tau_scope"),
    ("kv_dtype", 9, "dtype"),
    ("ctx_lens", None, "required"),
    ("bt_stride", 0, "bt_stride"),
])
def test_invalid_arguments_fail_loudly_without_launching(schedlib, field, value, msg):
    a = fake_args(**{field: value})
    rc = schedlib.sched_paged_decode(ctypes.byref(a), None)
    assert rc != 0
    assert msg in abi.last_error()
    assert kind(schedlib, a) == -1


def test_linear_mode_needs_weights(schedlib):
    a = fake_args(mode=abi.LINEAR)
    assert schedlib.sched_paged_decode(ctypes.byref(a), None) != 0
    assert "lin_w" in abi.last_error()


def test_misaligned_k_pool_rejected_for_valu(schedlib):
    a = fake_args(kv_dtype=abi.F32, q_dtype=abi.F32, k_pool=ctypes.c_void_p(0x10004))
    assert schedlib.sched_paged_decode(ctypes.byref(a), None) != 0
    assert "16-byte" in abi.last_error()


def test_missing_library_is_an_error(tmp_path):
    saved = abi._LIB
    abi._LIB = None
    try:
        with pytest.raises(abi.SchedLibraryError):
            abi.load_library(str(tmp_path / "nope.so"))
    finally:
        abi._LIB = saved


def test_noalloc_refuses_a_workspace_and_oversized_plans_without_the_gpu(schedlib):
    a = fake_args(tiles=ctypes.c_void_p(0x90000), num_tiles=8, tile_pages=4,
                  workspace=ctypes.c_void_p(0xA0000), workspace_bytes=1 << 20)
    assert schedlib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "no workspace" in abi.last_error()
    a.workspace, a.workspace_bytes = None, 0
    a.num_tiles = 1 << 22          # 4M items x 4 heads x 512 B of partials
    assert schedlib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "holds 16777216" in abi.last_error()
    assert schedlib.sched_paged_decode_noalloc(None, None) != 0
    # zero kv-heads with a plan: rejected (not a division by zero in the host)
    a.num_tiles = 8
    a.num_kv_heads = 0
    assert schedlib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "num_kv_heads is 0" in abi.last_error()
    a.num_kv_heads, a.num_q_heads = 4, 6
    assert schedlib.sched_paged_decode_noalloc(ctypes.byref(a), None) != 0
    assert "not a multiple" in abi.last_error()


def test_bind_tables_row_limit_without_the_gpu(schedlib):
    """sched_rt_bind_tables refuses more rows than the plane window holds
    before it touches a slot."""
    assert not schedlib.sched_rt_bind_tables(None, None, None, None,
                                             abi.RT_BIND_MAX_TASKS + 1)
    assert "max_tasks 16385 > 16384" in abi.last_error()


def test_split_arguments_validated(schedlib):
    a = fake_args(tiles=ctypes.c_void_p(0x90000), num_tiles=8, tile_pages=4)
    need = schedlib.sched_paged_decode_workspace_bytes(ctypes.byref(a))
    # stale counter + counters (32 tasks) + (m, l) for 8 items x 4 heads +
    # partials 8 x 4 x 128 f32, regions 256-byte aligned
    assert need == 256 + 256 + 256 + 8 * 4 * 128 * 4
    assert schedlib.sched_paged_decode(ctypes.byref(a), None) != 0
    assert "workspace" in abi.last_error()
    a.workspace, a.workspace_bytes = ctypes.c_void_p(0xA0000), need - 1
    assert schedlib.sched_paged_decode(ctypes.byref(a), None) != 0
    a.tile_pages = 0
    assert schedlib.sched_paged_decode(ctypes.byref(a), None) != 0
    assert "tile_pages" in abi.last_error()


def test_plan_tiles_is_task_major():
    import numpy as np
    import sched_pd
    t = sched_pd.plan_tiles([0, 16, 17, 100], 16, 2, 2, device="cpu").numpy()
    # pages per request: 0, 1, 2, 7 -> chunks 1, 1, 1, 4; two kv-heads each
    assert t[:, 0].tolist() == [0, 1, 2, 3, 4, 5, 6, 6, 6, 6, 7, 7, 7, 7]
    assert t[:, 1].tolist() == [0, 0, 0, 0, 0, 0, 0, 1, 2, 3, 0, 1, 2, 3]
    o = sched_pd.tile_order_by_task_key(torch_tiles(t), np.arange(8.0)).numpy()
    assert o[:4].tolist() == [10, 11, 12, 13] and o[-1] == 0


def test_tile_pages_loaded_and_lpt_order():
    import numpy as np
    import sched_abi as abi
    import sched_pd
    t = sched_pd.plan_tiles([0, 16, 17, 100], 16, 2, 2, device="cpu").numpy()
    # without a budget: 0, 1, 2, 7 pages per request -> chunks of at most 2
    got = sched_pd.tile_pages_loaded(t, [0, 16, 17, 100], 16, 2, 2)
    assert got.tolist() == [0, 0, 1, 1, 2, 2, 2, 2, 2, 1, 2, 2, 2, 1]
    # prefix budget on request 3's tasks (6 and 7): 33 tokens -> 3 pages,
    # 0 (no cap) and 5 tokens -> 1 page; per-page scope reads every page
    tau = np.array([0, 0, 0, 0, 0, 0, 33, 5])
    got = sched_pd.tile_pages_loaded(t, [0, 16, 17, 100], 16, 2, 2, tau=tau)
    assert got[6:].tolist() == [2, 1, 0, 0, 1, 0, 0, 0]
    per_page = sched_pd.tile_pages_loaded(t, [0, 16, 17, 100], 16, 2, 2, tau=tau,
                                          tau_scope=abi.TAU_PER_PAGE)
    assert per_page[6:].tolist() == [2, 2, 2, 1, 2, 2, 2, 1]
    o = sched_pd.tile_order_lpt(got).numpy()
    assert sorted(o.tolist()) == list(range(14))
    assert all(got[o[i]] >= got[o[i + 1]] for i in range(13))
    assert o[:3].tolist() == [4, 5, 6]   # ties keep index order


def _ranged_by_loops(ctx, ps, hkv, order, tp, tail, frac):
    # the ranged plan written out one task at a time, in claim order
    npg = [-(-c // ps) for c in ctx for _ in range(hkv)]
    total, before, size = sum(npg), 0, {}
    for t in order:
        size[t] = tp if before < (1 - frac) * total else tail
        before += npg[t]
    rows = []
    for t in range(len(npg)):
        nch = max(1, -(-npg[t] // size[t]))
        for c in range(nch):
            rows.append([t, c | nch << 16, c * size[t], min((c + 1) * size[t], npg[t])])
    return rows


def test_ranged_plan_rows_and_tail():
    import numpy as np
    import sched_pd
    ctx = [0, 16, 17, 100, 3000, 250]
    pairs = sched_pd.plan_tiles_host(ctx, 16, 4, 2)
    # no tail: the pair plan's chunks with their page ranges spelled out
    r = sched_pd.plan_ranges_host(ctx, 16, 2, tile_pages=4, tail_frac=0.0)
    assert np.array_equal(r[:, 0], pairs[:, 0]) and np.array_equal(r[:, 1] & 0xFFFF, pairs[:, 1])
    npg = np.repeat((np.array(ctx) + 15) // 16, 2)
    nch = np.maximum(1, (npg + 3) // 4)
    assert np.array_equal(r[:, 1] >> 16, nch[r[:, 0]])
    assert np.array_equal(r[:, 2], 4 * pairs[:, 1])
    assert np.array_equal(r[:, 3], np.minimum(4 * pairs[:, 1] + 4, npg[r[:, 0]]))
    rng = np.random.default_rng(5)
    for frac, tp, tail in ((0.0, 4, 1), (0.3, 8, 2), (0.6, 16, 3), (1.0, 5, 2)):
        order = rng.permutation(len(ctx) * 2)
        got = sched_pd.plan_ranges_host(ctx, 16, 2, task_order=order, tile_pages=tp,
                                        tail_pages=tail, tail_frac=frac)
        assert got.tolist() == _ranged_by_loops(ctx, 16, 2, order, tp, tail, frac)
        sched_pd.check_ranged_plan(got)
    # under prefix budgets only the pages read are cut; the last range runs
    # to the context's end
    tau = np.array([0, 0, 5, 5, 40, 0, 1000, 17, 0, 0, 100, 240])
    got = sched_pd.plan_ranges_host(ctx, 16, 2, tile_pages=2, tail_frac=0.0, tau=tau)
    sched_pd.check_ranged_plan(got)
    load = (np.where(tau > 0, np.minimum(np.repeat(ctx, 2), tau), np.repeat(ctx, 2)) + 15) // 16
    for t in range(12):
        rows = got[got[:, 0] == t]
        assert len(rows) == max(1, -(-load[t] // 2))
        assert rows[-1, 3] == npg[t] and (rows[:-1, 3] - rows[:-1, 2] == 2).all()
    read = sched_pd.tile_pages_loaded(got, ctx, 16, 0, 2, tau=tau)
    assert np.bincount(got[:, 0], weights=read, minlength=12).tolist() == load.tolist()
    assert ((read > 0) | (load[got[:, 0]] == 0)).all()            # no empty item
    with pytest.raises(ValueError):
        sched_pd.plan_ranges_host(ctx, 16, 2, task_order=[0, 1])
    with pytest.raises(ValueError):
        sched_pd.plan_ranges_host(ctx, 16, 2, tail_pages=0)


def test_check_ranged_plan_rejects_malformed_lists():
    import numpy as np
    import sched_pd
    good = sched_pd.plan_ranges_host([100, 40], 16, 1, tile_pages=2, tail_frac=0.0)
    # request 0: 7 pages in 4 chunks, request 1: 3 pages in 2 chunks
    assert good.tolist() == [[0, 0 | 4 << 16, 0, 2], [0, 1 | 4 << 16, 2, 4],
                             [0, 2 | 4 << 16, 4, 6], [0, 3 | 4 << 16, 6, 7],
                             [1, 0 | 2 << 16, 0, 2], [1, 1 | 2 << 16, 2, 3]]
    sched_pd.check_ranged_plan(good)
    bad = []
    b = good.copy(); b[[1, 2]] = b[[2, 1]]; bad.append(b)             # chunks out of order
    b = good.copy(); b[2, 2] = 5; bad.append(b)                       # gap in the ranges
    b = good.copy(); b[3, 1] = 3 | 5 << 16; bad.append(b)             # nchunks differ
    bad.append(good[:5].copy())                                       # last task cut short
    b = good.copy(); b[4, 2] = 1; bad.append(b)                       # chunk 0 not from page 0
    b = good.copy(); b[5, 0] = 0; bad.append(b)                       # task changes mid-chunks
    b = good.copy(); b[1, 3] = 1; bad.append(b)                       # p1 < p0
    b = good.copy(); b[4:, 0] = 0; bad.append(b)                      # a task's second group
    for b in bad:
        with pytest.raises(ValueError):
            sched_pd.check_ranged_plan(b)
    with pytest.raises(ValueError):
        sched_pd.check_ranged_plan(np.zeros((0, 4), np.int32))
    # pages read under a prefix budget: task 0 capped at 40 tokens = 3 pages
    got = sched_pd.tile_pages_loaded(good, [100, 40], 16, 0, 1, tau=np.array([40, 0]))
    assert got.tolist() == [2, 1, 0, 0, 2, 1]


def test_ranged_tile_format_validated(schedlib):
    ws = dict(tiles=ctypes.c_void_p(0x90000), num_tiles=8, workspace=ctypes.c_void_p(0xA0000),
              workspace_bytes=1 << 20)
    assert kind(schedlib, fake_args(**ws, tile_format=abi.TILES_RANGED)) == 1  # no tile_pages
    assert kind(schedlib, fake_args(**ws, tile_format=abi.TILES_PAIRS)) == -1
    assert "tile_pages" in abi.last_error()
    assert kind(schedlib, fake_args(**ws, tile_format=2, tile_pages=4)) == -1
    assert "tile_format" in abi.last_error()


def torch_tiles(t):
    import torch
    return torch.from_numpy(t)


def test_copy_to_device_validates_without_the_gpu(schedlib):
    p = ctypes.c_void_p
    assert schedlib.sched_pd_copy_to_device(None, None, 0, None) == 0         # nothing to copy
    assert schedlib.sched_pd_copy_to_device(None, p(0x10000), 64, None) != 0
    assert "NULL" in abi.last_error()
    assert schedlib.sched_pd_copy_to_device(p(0x10000), None, 64, None) != 0
    assert not schedlib.sched_pd_staging_alloc(0)
    assert "sched_pd_staging_alloc" in abi.last_error()
    assert not schedlib.sched_pd_staging_alloc((1 << 32) + 1)


def test_table_update_validates_without_the_gpu(schedlib):
    p = ctypes.c_void_p
    assert schedlib.sched_kv_table_update(None, 4, 8, None, 0, None) == 0     # nothing to do
    assert schedlib.sched_kv_table_update(None, 4, 8, p(0x10000), 3, None) != 0
    assert "sched_kv_table_update" in abi.last_error()
    assert schedlib.sched_kv_table_update(p(0x10000), 4, 0, p(0x20000), 3, None) != 0


def test_block_probe_validates_arguments_without_the_gpu(schedlib):
    buf = ctypes.c_void_p(0x10000)
    ids = (ctypes.c_int32 * 4)(0, 1, 2, 3)
    assert schedlib.sched_pd_read_probe_blocks(buf, 1 << 20, None, 4, 4096, None, None) != 0
    assert "block probe" in abi.last_error()
    assert schedlib.sched_pd_read_probe_blocks(buf, 1 << 20, ids, 4, 4095, None, None) != 0
    assert schedlib.sched_pd_read_probe_blocks(buf, 1 << 20, ids, 0, 4096, None, None) == 0


def test_check_page_table_accepts_reachable_ids_and_names_the_bad_request():
    import torch
    from sched_pd import check_page_table
    bt = torch.tensor([[3, 1, -1], [0, 2, 4]], dtype=torch.int32)
    ctx = torch.tensor([17, 33], dtype=torch.int32)     # 2 and 3 pages of 16
    check_page_table(bt, ctx, 16, 5)                     # -1 past the reach is fine
    with pytest.raises(ValueError, match="request 1 has a page id"):
        check_page_table(bt, ctx, 16, 4)                 # page 4 of a 4-page pool
    with pytest.raises(ValueError, match="request 0 has a page id"):
        check_page_table(bt, torch.tensor([33, 1], dtype=torch.int32), 16, 5)  # reaches -1
    with pytest.raises(ValueError, match="request 1 needs 4 pages"):
        check_page_table(bt, torch.tensor([1, 49], dtype=torch.int32), 16, 5)
    with pytest.raises(ValueError, match="negative"):
        check_page_table(bt, torch.tensor([1, -1], dtype=torch.int32), 16, 5)
    check_page_table(bt, torch.tensor([2, 3], dtype=torch.int32), 16, 5, ctx_in_pages=True)
    # CSR
    ind = torch.tensor([0, 2, 5], dtype=torch.int32)
    flat = torch.tensor([3, 1, 0, 2, 4], dtype=torch.int32)
    check_page_table(flat, ctx, 16, 5, page_indptr=ind)
    with pytest.raises(ValueError, match="request 0 needs 3 pages, its segment has 2"):
        check_page_table(flat, torch.tensor([40, 1], dtype=torch.int32), 16, 5, page_indptr=ind)
    with pytest.raises(ValueError, match="CSR"):
        check_page_table(flat, ctx, 16, 5, page_indptr=torch.tensor([0, 3, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match="CSR"):
        check_page_table(flat, ctx, 16, 5, page_indptr=torch.tensor([0, 2, 6], dtype=torch.int32))


def test_fused_append_refusals_without_the_gpu(schedlib):
    """sched_paged_decode_append checks its two argument blocks on the host
    and names what it does not take (nothing is launched)."""
    a = fake_args(v_tok_stride=128, v_dim_stride=1)          # token-major V
    w = abi.default_kv_args()
    w.num_requests, w.num_kv_heads, w.head_dim, w.page_size = 4, 8, 128, 16
    w.num_tokens, w.bt_stride = 4, 8
    w.src_dtype = w.kv_dtype = abi.BF16
    w.k_src, w.v_src = ctypes.c_void_p(0x70000), ctypes.c_void_p(0x80000)
    for f in ("k_pool", "v_pool", "ctx_lens", "block_table"):
        setattr(w, f, getattr(a, f))
    for f in ("k_page_stride", "k_head_stride", "k_tok_stride", "v_page_stride",
              "v_head_stride", "v_tok_stride", "v_dim_stride"):
        setattr(w, f, getattr(a, f))
    w.src_tok_stride, w.src_head_stride = 8 * 128, 128
    fn = schedlib.sched_paged_decode_append

    def refused(word, **changes):
        saved = {k: getattr(w, k) for k in changes}
        for k, v in changes.items():
            setattr(w, k, v)
        rc = fn(ctypes.byref(a), ctypes.byref(w), None)
        for k, v in saved.items():
            setattr(w, k, v)
        return rc != 0 and word in abi.last_error()

    assert fn(None, ctypes.byref(w), None) != 0
    assert refused("abi_version", abi_version=99)
    assert refused("one token per request", num_tokens=5)
    assert refused("must be the decode's", ctx_lens=ctypes.c_void_p(0x990000))
    assert refused("4-byte aligned", k_src=ctypes.c_void_p(0x70002))
    assert refused("cache dtypes differ", kv_dtype=abi.F16)
    a.kv_dtype = w.kv_dtype = abi.F32
    assert refused("bf16, fp16 or fp8 caches only")
    a.kv_dtype = w.kv_dtype = abi.FP8_E4M3
    assert refused("needs its k_scale / v_scale")                 # no scales
    a.k_scale, a.v_scale = ctypes.c_void_p(0xB0000), ctypes.c_void_p(0xB0004)
    w.k_scale, w.v_scale = ctypes.c_void_p(0xB0000), ctypes.c_void_p(0xC0000)
    assert refused("the same in both")
    w.v_scale = ctypes.c_void_p(0xB0004)
    assert refused("fp32, bf16 or fp16 for an fp8 cache", src_dtype=abi.FP8_E4M3)
    a.k_scale = a.v_scale = w.k_scale = w.v_scale = None
    a.kv_dtype = w.kv_dtype = abi.BF16
    a.v_tok_stride, a.v_dim_stride = 1, 16                  # d-major V
    assert refused("token-major V")


def test_plan_checks_remember_plans_by_content_only():
    """The host checks keep what they established about recent plans keyed
    by the plan's bytes: a plan changed in place after a passing check, or
    an equal-looking plan of another dtype or shape, is checked again."""
    import numpy as np
    import sched_pd
    ctx = [100, 40, 300]
    pairs = sched_pd.plan_tiles_host(ctx, 16, 4, 2)
    sched_pd.check_pair_plan(pairs)
    sched_pd.check_pair_plan(pairs)                       # remembered
    sched_pd.check_plan_covers(pairs, ctx, 16, 2, tile_pages=4)
    pairs[1, 1] = 5                                       # the same array, now malformed
    with pytest.raises(ValueError):
        sched_pd.check_pair_plan(pairs)
    pairs[1, 1] = 1
    sched_pd.check_pair_plan(pairs)
    with pytest.raises(ValueError):                       # coverage: a longer context
        sched_pd.check_plan_covers(pairs, [100, 40, 400], 16, 2, tile_pages=4)
    with pytest.raises(ValueError):                       # the same rows at another tile size
        sched_pd.check_plan_covers(pairs, ctx, 16, 2, tile_pages=2)
    ranged = sched_pd.plan_ranges_host(ctx, 16, 2, tile_pages=3, tail_frac=0.0)
    sched_pd.check_ranged_plan(ranged)
    sched_pd.check_plan_covers(ranged, ctx, 16, 2)
    bad = ranged.copy()
    bad[[1, 2]] = bad[[2, 1]]
    with pytest.raises(ValueError):
        sched_pd.check_ranged_plan(bad)
    ranged[0, 3] = 1                                      # in place: a gap after row 0
    with pytest.raises(ValueError):
        sched_pd.check_ranged_plan(ranged)
    # more distinct plans than remembered: each still checked correctly
    for n in range(1, 12):
        p = sched_pd.plan_tiles_host([16 * n, 40], 16, 2, 1)
        sched_pd.check_pair_plan(p)
        sched_pd.check_plan_covers(p, [16 * n, 40], 16, 1, tile_pages=2)
        with pytest.raises(ValueError):
            sched_pd.check_plan_covers(p, [16 * n + 33, 40], 16, 1, tile_pages=2)


def test_graded_plan_rows_by_position_in_the_claim_order():
    """plan_graded_host against rows derived by hand: 10 + 2 + 20 pages on
    the claim line (32 pages), sizes 8 before the line's middle and 3 after;
    a task crossing the middle is cut there."""
    import numpy as np
    import sched_pd
    ctx = [160, 32, 320]                        # 10, 2, 20 pages of 16 tokens
    got = sched_pd.plan_graded_host(ctx, 16, 1, sizes=((0.0, 8), (0.5, 3)))
    want = [[0, 0 | 2 << 16, 0, 8], [0, 1 | 2 << 16, 8, 10],
            [1, 0 | 1 << 16, 0, 2],
            [2, 0 | 7 << 16, 0, 4], [2, 1 | 7 << 16, 4, 7], [2, 2 | 7 << 16, 7, 10],
            [2, 3 | 7 << 16, 10, 13], [2, 4 | 7 << 16, 13, 16], [2, 5 | 7 << 16, 16, 19],
            [2, 6 | 7 << 16, 19, 20]]
    assert got.tolist() == want
    sched_pd.check_ranged_plan(got)
    sched_pd.check_plan_covers(got, ctx, 16, 1)
    # claimed in reverse: task 2 first (its 20 pages: 16 of them before the
    # middle), then task 1 and task 0 after it
    rev = sched_pd.plan_graded_host(ctx, 16, 1, task_order=[2, 1, 0], sizes=((0.0, 8), (0.5, 3)))
    by_task = {t: rev[rev[:, 0] == t][:, 2:].tolist() for t in range(3)}
    assert by_task[2] == [[0, 8], [8, 16], [16, 19], [19, 20]]
    assert by_task[1] == [[0, 2]]
    assert by_task[0] == [[0, 3], [3, 6], [6, 9], [9, 10]]
    # budgets: task 2 reads 5 pages (70 tokens); only those are lined up,
    # and its last range runs on to the context's last page
    tau = sched_pd.plan_graded_host(ctx, 16, 1, sizes=((0.0, 8), (0.5, 3)),
                                    tau=np.array([0, 0, 70]))
    assert tau[tau[:, 0] == 2][:, 2:].tolist() == [[0, 3], [3, 20]]
    sched_pd.check_plan_covers(tau, ctx, 16, 1)
    # an empty task keeps one empty chunk; heads repeat each request
    empty = sched_pd.plan_graded_host([0, 40], 16, 2, sizes=((0.0, 2),))
    assert empty.tolist() == [[0, 1 << 16, 0, 0], [1, 1 << 16, 0, 0],
                              [2, 0 | 2 << 16, 0, 2], [2, 1 | 2 << 16, 2, 3],
                              [3, 0 | 2 << 16, 0, 2], [3, 1 | 2 << 16, 2, 3]]
    for bad in (((0.1, 8),), ((0.0, 8), (0.0, 4)), ((0.0, 0),), ((0.0, 8), (1.0, 2))):
        with pytest.raises(ValueError):
            sched_pd.plan_graded_host(ctx, 16, 1, sizes=bad)
    with pytest.raises(ValueError):
        sched_pd.plan_graded_host(ctx, 16, 1, task_order=[0, 0, 1])
