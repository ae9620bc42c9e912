"""The C runtime contract (sched_rt_*) and the reference's launcher
(launch_paged_softmax) on the GPU, mode by mode as the reference fixture runs
them (test/paged_decode.cu:282-475 and test/py/test_dynamic_loop.py:118-190),
on the fixtures' own generated inputs."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
import sched_pd
from parity import TOL_F32, par_err

pytestmark = pytest.mark.gpu

SD = 32


def lcg(n, seed):
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = ((s >> 8) & 0xFFFF) / 65536.0 - 0.5
    return out, s


def fixture_paged_decode():
    """test/paged_decode.cu:236-251 with the softmax section's q (:430-432):
    NSEQ 64, 8 pages of 64 tokens, page layout [token][K(32) | V(32)]."""
    nseq, nblocks, pt = 64, 8, 64
    npages = nseq * nblocks
    vals, s = lcg(npages * pt * 2 * SD + nblocks * pt + nseq * SD, 12345)
    kv = vals[:npages * pt * 2 * SD]
    q = vals[npages * pt * 2 * SD + nblocks * pt:].reshape(nseq, 1, SD)
    bt = np.array([(i * 37 + 11) % npages for i in range(nseq * nblocks)], np.int32)
    return kv, bt.reshape(nseq, nblocks), q, np.full(nseq, nblocks, np.int32), pt


def fixture_dynamic_loop():
    """test/py/test_dynamic_loop.py:39-42,103-115: NSEQ 64, PT 32, longs (t%8==0)
    24 pages, shorts 3, torch.Generator seed 1 uniform - 0.5."""
    nseq, pt, nlong, nshort = 64, 32, 24, 3
    npages = nseq * nlong
    g = torch.Generator().manual_seed(1)
    kv = (torch.rand(npages * pt * 2 * SD + 4096, generator=g) - 0.5).numpy()
    q = (torch.rand(nseq * SD, generator=g) - 0.5).numpy().reshape(nseq, 1, SD)
    nbl = np.array([nlong if t % 8 == 0 else nshort for t in range(nseq)], np.int32)
    bt = np.array([[(t * nlong + b * 7 + 3) % npages for b in range(nlong)] for t in range(nseq)],
                  np.int32)
    return kv, bt, q, nbl, pt


class Fixture:
    def __init__(self, make):
        kv, bt, q, nbl, pt = make()
        self.pt, self.nseq = pt, q.shape[0]
        self.kv_h, self.bt_h, self.q_h, self.nbl_h = kv, bt, q, nbl
        self.kv = torch.from_numpy(kv).cuda()
        self.bt = torch.from_numpy(bt).cuda()
        self.q = torch.from_numpy(q.copy()).cuda()
        self.nbl = torch.from_numpy(nbl).cuda()
        self.out = torch.zeros(self.nseq, 1, SD, device="cuda")

    def launch(self, lib):
        self.out.zero_()
        lib.launch_paged_softmax(self.kv.data_ptr(), self.bt.data_ptr(), self.nbl.data_ptr(),
                                 self.q.data_ptr(), self.out.data_ptr(), self.nseq,
                                 self.bt.shape[1], self.pt,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return self.out.clone()

    def reference(self, tau=0):
        npages = self.kv_h.size // (self.pt * 2 * SD)
        pages = self.kv_h[:npages * self.pt * 2 * SD].reshape(npages, 1, self.pt, 2 * SD)
        import levers
        ctrl = levers.ctrl_bytes({"rows": {t: (0.0, tau, 0) for t in range(self.nseq)}}, 4096)
        return oracle.decode(self.q_h, pages[..., :SD], pages[..., SD:], self.bt_h, self.nbl_h,
                             v_layout="tokmajor", sm_scale=0.125, tau_scope=abi.TAU_PER_PAGE,
                             ctrl=ctrl, ctx_in_pages=True)


def close(a, r, tol=TOL_F32):
    """fp32: the mixed form and the per-row norm-relative error within tol."""
    return par_err(a, r) <= tol


def timer_rows(lib, n):
    buf = (ctypes.c_ulonglong * n)()
    assert lib.sched_rt_timer_read(buf, n)
    return np.array(buf[:], np.uint64)


@pytest.fixture(scope="module")
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def test_reference_fixture_modes(lib):
    f = Fixture(fixture_paged_decode)
    lib.sched_rt_disarm()
    # A inert
    golden = f.launch(lib)
    assert close(golden.cpu(), f.reference()), "A inert vs CPU reference"
    # arm
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(f.nseq)
    assert lib.sched_rt_push_ctrl()
    slots = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slots(slots) and all(slots)
    # B identity, neutral policy
    lib.sched_rt_timer_clear()
    assert torch.equal(f.launch(lib), golden)
    assert int((timer_rows(lib, f.nseq) > 0).sum()) == f.nseq
    assert lib.sched_rt_timer(0) > 0
    # C reversed pi
    order = np.arange(4096, dtype=np.int32)
    order[:f.nseq] = np.arange(f.nseq)[::-1]
    assert lib.sched_rt_set_order(order.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), 4096)
    assert torch.equal(f.launch(lib), golden)
    # D aggressive policy (q >> 0, lambda 0)
    lib.sched_rt_set_lambda(0.0, 0.0, 0.0, 0.0)
    for i in range(f.nseq):
        lib.sched_rt_set_task(i, 100.0, 0, 0)
    lib.sched_rt_push_ctrl()
    lib.sched_rt_timer_clear()
    assert torch.equal(f.launch(lib), golden)
    assert int((timer_rows(lib, f.nseq) > 0).sum()) == f.nseq
    # E priced out
    lib.sched_rt_set_lambda(1000.0, 0.0, 0.0, 0.0)
    lib.sched_rt_push_ctrl()
    assert torch.equal(f.launch(lib), golden)
    # G/H shed: tau 0 bit-exact, tau 8 = truncated reference (first 8 tokens of every page)
    for i in range(f.nseq):
        lib.sched_rt_set_task(i, 0.0, 0, 0)
    lib.sched_rt_push_ctrl()
    assert torch.equal(f.launch(lib), golden)
    for i in range(f.nseq):
        lib.sched_rt_set_tau(i, 8)
    lib.sched_rt_push_ctrl()
    shed = f.launch(lib)
    assert not torch.equal(shed, golden) and torch.isfinite(shed).all()
    assert close(shed.cpu(), f.reference(tau=8))
    for i in range(f.nseq):
        lib.sched_rt_set_tau(i, 0)
    lib.sched_rt_push_ctrl()
    # timer gate
    lib.sched_rt_set_timer_enabled(False)
    lib.sched_rt_push_ctrl()
    lib.sched_rt_timer_clear()
    assert torch.equal(f.launch(lib), golden)
    assert int((timer_rows(lib, f.nseq) > 0).sum()) == 0
    lib.sched_rt_set_timer_enabled(True)
    lib.sched_rt_push_ctrl()
    # disarm -> stock, slots null; re-arm reuses the buffers
    assert lib.sched_rt_disarm()
    assert lib.sched_rt_slots(slots) and not any(slots)
    assert torch.equal(f.launch(lib), golden)
    assert lib.sched_rt_init()
    slots2 = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slots(slots2) and all(slots2)
    order = np.arange(4096, dtype=np.int32)
    lib.sched_rt_set_order(order.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), 4096)
    lib.sched_rt_disarm()


def test_dynamic_loop_demo(lib):
    f = Fixture(fixture_dynamic_loop)
    lib.sched_rt_disarm()
    golden = f.launch(lib)
    assert close(golden.cpu(), f.reference())
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(f.nseq)
    lib.sched_rt_push_ctrl()
    lib.sched_rt_timer_clear()
    assert torch.equal(f.launch(lib), golden)
    cyc = timer_rows(lib, f.nseq).astype(np.float64)
    assert int((cyc > 0).sum()) == f.nseq
    longs = [t for t in range(f.nseq) if t % 8 == 0]
    shorts = [t for t in range(f.nseq) if t % 8]
    assert cyc[longs].mean() > 2 * cyc[shorts].mean()
    # LPT from the measured cycles: bit-exact
    order = np.arange(4096, dtype=np.int32)
    order[:f.nseq] = np.argsort(-cyc, kind="stable").astype(np.int32)
    lib.sched_rt_set_order(order.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), 4096)
    assert torch.equal(f.launch(lib), golden)
    # shed on the same kernel: truncated reference
    for i in range(f.nseq):
        lib.sched_rt_set_tau(i, 8)
    lib.sched_rt_push_ctrl()
    assert close(f.launch(lib).cpu(), f.reference(tau=8))
    for i in range(f.nseq):
        lib.sched_rt_set_tau(i, 0)
    lib.sched_rt_push_ctrl()
    lib.sched_rt_set_order(np.arange(4096, dtype=np.int32).ctypes.data_as(
        ctypes.POINTER(ctypes.c_int32)), 4096)
    lib.sched_rt_disarm()


def test_shed_quality_curve(lib):
    """The shed quality contract (test/py/eval_quality.py:30-70) on the
    dynamic-loop fixture: tau = 0 is full attention, every tau in (24, 16, 8,
    4) matches its truncated reference, and the cosine to full attention
    does not rise as the budget shrinks."""
    f = Fixture(fixture_dynamic_loop)
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(f.nseq)
    full = np.asarray(f.reference(tau=0), np.float64).ravel()
    last = None
    try:
        for tau in (0, 24, 16, 8, 4):
            for i in range(f.nseq):
                lib.sched_rt_set_tau(i, tau)
            lib.sched_rt_push_ctrl()
            o = f.launch(lib).cpu().double().numpy()
            assert close(o, f.reference(tau=tau)), f"tau {tau}"
            o = o.ravel()
            cos = float(o @ full / (np.linalg.norm(o) * np.linalg.norm(full)))
            if tau == 0:
                assert cos > 1 - 1e-9
            if last is not None:
                assert cos <= last + 1e-6, f"tau {tau}: cosine {cos} > {last}"
            last = cos
    finally:
        for i in range(f.nseq):
            lib.sched_rt_set_tau(i, 0)
        lib.sched_rt_push_ctrl()
        lib.sched_rt_disarm()


def test_runtime_work_queue_through_rt_tables(lib):
    """Ticket queue armed through the C runtime (flags RT_TABLES)."""
    import sched_pd
    import workloads
    b = workloads.make_batch(np.array([40, 3000, 700, 16, 1, 2048]), num_q_heads=32,
                             num_kv_heads=8, seed=21)
    n = 6 * 8
    ref = sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                b["ctx_lens"], out_dtype=torch.float32)
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(n)
    lib.sched_rt_push_ctrl()
    for W in (5, n, 3 * n):
        assert lib.sched_rt_queue_reset(W)
        lib.sched_rt_timer_clear()
        out = sched_pd.paged_decode(b["q"], b["k_pool"], b["v_pool"], b["block_table"],
                                    b["ctx_lens"], out_dtype=torch.float32, rt_tables=True,
                                    workers=W)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert int((timer_rows(lib, n) > 0).sum()) == n
    lib.sched_rt_set_num_tasks(0)
    lib.sched_rt_push_ctrl()
    lib.sched_rt_disarm()


def test_occupancy_queries(lib):
    assert lib.paged_softmax_occupancy() > 0
    assert lib.sched_pd_cu_count() > 0


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    return hip


def _write_slot(hip, addr, value):
    v = ctypes.c_uint64(value)
    assert hip.hipMemcpy(ctypes.c_void_p(addr), ctypes.byref(v), 8, 1) == 0  # host to device


def test_slots_written_directly_on_the_device_take_effect(lib):
    """The reference's mechanism: the app writes a __sched_* slot itself
    (cudaMemcpyToSymbol). Here the slot's device address comes from
    sched_rt_slot_addresses and a plain copy writes it; the next launch reads
    it. A reversed order and a fresh timer buffer written that way take
    effect (same bits, rows in the new buffer); a device-side disarm of ctrl
    and queue under a queue grid of fewer workers than tasks still serves
    every task (stock path over the whole grid)."""
    f = Fixture(fixture_paged_decode)
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(0)
    lib.sched_rt_timer_clear()
    assert lib.sched_rt_push_ctrl()
    golden = f.launch(lib)
    assert close(golden.cpu(), f.reference())
    lib.sched_rt_timer_clear()        # the golden launch filled the runtime's rows
    addrs = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slot_addresses(addrs) and all(addrs)
    held = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slots(held)
    hip = _hip()
    order = torch.arange(4096, dtype=torch.int32, device="cuda")
    order[:f.nseq] = torch.arange(f.nseq - 1, -1, -1, dtype=torch.int32, device="cuda")
    timer = torch.zeros(4096, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    _write_slot(hip, addrs[0], order.data_ptr())
    _write_slot(hip, addrs[2], timer.data_ptr())
    now = (ctypes.c_uint64 * 4)()
    assert lib.sched_rt_slots(now)
    assert now[0] == order.data_ptr() and now[2] == timer.data_ptr()
    assert torch.equal(f.launch(lib), golden)
    assert int((timer[:f.nseq] > 0).sum()) == f.nseq          # the kernel wrote the new rows
    assert int((timer_rows(lib, f.nseq) > 0).sum()) == 0      # not the runtime's own
    # the queue armed on the host (num_tasks pushed) and launched with 7
    # workers, then ctrl and queue nulled on the device: the stock path
    lib.sched_rt_set_num_tasks(f.nseq)
    assert lib.sched_rt_push_ctrl()
    assert lib.sched_rt_queue_reset(7)
    _write_slot(hip, addrs[1], 0)
    _write_slot(hip, addrs[3], 0)
    args = sched_pd.build_args(f.q, f.kv.view(-1, 1, f.pt, 2 * SD)[..., :SD],
                               f.kv.view(-1, 1, f.pt, 2 * SD)[..., SD:], f.bt, f.nbl,
                               out=f.out, v_layout="tokmajor", sm_scale=0.125,
                               tau_scope=abi.TAU_PER_PAGE, flags=abi.FLAG_CTX_IN_PAGES,
                               rt_tables=True, workers=7)
    f.out.zero_()
    sched_pd.launch(args)
    torch.cuda.synchronize()
    assert torch.equal(f.out, golden)
    # restore what sched_rt armed
    for i in range(4):
        _write_slot(hip, addrs[i], held[i])
    lib.sched_rt_set_num_tasks(0)
    assert lib.sched_rt_push_ctrl()


def test_timer_host_mirror_for_external_readers(lib):
    """Opt-in host copy of the timer rows: after a launch on the runtime's
    tables the published timer_host_va holds the device rows, readable with no
    GPU call; off again publishes 0."""
    import json
    import os
    f = Fixture(fixture_paged_decode)
    assert lib.sched_rt_init()
    lib.sched_rt_set_num_tasks(0)
    assert lib.sched_rt_push_ctrl()
    assert lib.sched_rt_set_timer_host_mirror(True)
    va = lib.sched_rt_timer_host_va()
    assert va
    pub = json.load(open(f"/tmp/sched_rt_{os.getpid()}.json"))
    assert pub["timer_host_va"] == va and pub["timer_bytes"] == 4096 * 8
    lib.sched_rt_timer_clear()
    f.launch(lib)                      # synchronises: the mirror copy is done
    host = np.frombuffer(ctypes.string_at(va, 4096 * 8), np.uint64)
    dev = timer_rows(lib, 4096)
    assert np.array_equal(host, dev) and int((host[:f.nseq] > 0).sum()) == f.nseq
    assert lib.sched_rt_set_timer_host_mirror(False)
    assert lib.sched_rt_timer_host_va() == 0
    assert json.load(open(f"/tmp/sched_rt_{os.getpid()}.json"))["timer_host_va"] == 0
