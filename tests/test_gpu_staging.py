"""Host-to-device staging of the per-step uploads (sched_pd.upload /
upload_into through a pinned ring per stream) and the asynchronous timer
readout: the bytes arrive intact while the ring wraps several times over,
with uploads inside one chunk and spanning chunks, with the device queue
kept busy, on two streams, and for arrays too large for the ring. The
copy out of staging memory (a kernel up to 1 MiB, the copy engine above)
moves exactly the bytes asked for at every alignment, and sees the host's
latest writes to the same bytes."""
import ctypes

import numpy as np
import pytest
import torch

import sched_abi as abi
import sched_pd
from sched_rt import SchedPlane

pytestmark = pytest.mark.gpu


def _busy(n=4096):
    # keep the stream's queue non-empty so that uploads really overlap
    a = torch.randn(n, n, device="cuda")
    return a @ a


def test_uploads_survive_ring_wraps():
    rng = np.random.default_rng(1)
    sent, got = [], []
    total = 0
    while total < 3 * sched_pd._StagingRing.BYTES:
        # mostly small, every 20th spanning several chunks
        n = int(rng.integers(1, 40000)) if len(sent) % 20 else int(rng.integers(300_000, 900_000))
        a = rng.integers(-2**31, 2**31 - 1, n, dtype=np.int64).astype(np.int32)
        if len(sent) % 25 == 0:
            _busy(1024)
        sent.append(a)
        got.append(sched_pd.upload(a, "cuda"))
        total += a.nbytes
    torch.cuda.synchronize()
    for a, t in zip(sent, got):
        assert np.array_equal(t.cpu().numpy(), a)
    print(f"{len(sent)} uploads, {total} B")


def test_upload_on_two_streams_and_large_arrays():
    rng = np.random.default_rng(2)
    s1 = torch.cuda.Stream()
    big = rng.standard_normal(5_000_000).astype(np.float32)     # 20 MB: its own pinned copy
    with torch.cuda.stream(s1):
        _busy(2048)
        a1 = [rng.integers(0, 1000, 5000).astype(np.int32) for _ in range(20)]
        t1 = [sched_pd.upload(a, "cuda") for a in a1]
        tb = sched_pd.upload(big, "cuda")
    a0 = [rng.integers(0, 1000, 7000).astype(np.int64) for _ in range(20)]
    t0 = [sched_pd.upload(a, "cuda") for a in a0]
    torch.cuda.synchronize()
    for a, t in list(zip(a1, t1)) + list(zip(a0, t0)):
        assert np.array_equal(t.cpu().numpy(), a)
    assert np.array_equal(tb.cpu().numpy(), big)
    dst = torch.zeros(64, dtype=torch.int32, device="cuda")
    sched_pd.upload_into(dst[8:40], np.arange(32, dtype=np.int32))
    torch.cuda.synchronize()
    want = np.zeros(64, np.int32)
    want[8:40] = np.arange(32)
    assert np.array_equal(dst.cpu().numpy(), want)
    with pytest.raises(ValueError):
        sched_pd.upload_into(dst[:4], np.arange(5, dtype=np.int32))


def test_async_timer_readout_matches_sync():
    p = SchedPlane(max_tasks=256)
    p.use_device_timer()
    p._timer_view().copy_(torch.arange(256, dtype=torch.int64, device="cuda") * 7 + 3)
    torch.cuda.synchronize()
    rows, ev = p.read_timer_async()
    ev.synchronize()
    assert torch.equal(rows.clone(), p.read_timer())
    assert int(rows[255]) == 255 * 7 + 3


def test_staging_copy_sizes_alignments_and_rewrites():
    lib = abi.load_library()
    n = (1 << 20) + 64
    base = lib.sched_pd_staging_alloc(ctypes.c_uint64(n))
    assert base, abi.last_error()
    host = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(base))
    dst = torch.zeros(n, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    rng = np.random.default_rng(5)
    cases = 0
    for size in (1, 3, 4, 7, 8, 9, 255, 256, 2049, 65541, 1 << 20, (1 << 20) + 1):
        for so, do in ((0, 0), (4, 4), (8, 0), (1, 3), (3, 8), (0, 5), (16, 1)):
            if so + size > n or do + size > n:
                continue
            data = rng.integers(0, 256, size, dtype=np.uint8)
            host[so:so + size] = data                 # rewrites bytes an earlier case copied
            dst.zero_()
            _busy(512)
            rc = lib.sched_pd_copy_to_device(ctypes.c_void_p(dst.data_ptr() + do),
                                             ctypes.c_void_p(base + so), ctypes.c_uint64(size),
                                             ctypes.c_void_p(stream.cuda_stream))
            assert rc == 0, abi.last_error()
            got = dst.cpu().numpy()
            assert np.array_equal(got[do:do + size], data), (size, so, do)
            assert not got[:do].any() and not got[do + size:].any(), (size, so, do)
            cases += 1
    print(f"{cases} copies")


def test_staged_copy_captured_in_a_graph_reads_the_host_bytes_at_each_replay():
    """A serving step captured with its uploads: the copy kernel node reads
    the staging memory when it runs, so each replay moves the bytes the host
    wrote last (two copies: 8-byte aligned, and unaligned with an odd
    size)."""
    lib = abi.load_library()
    n = 8192
    base = lib.sched_pd_staging_alloc(ctypes.c_uint64(n))
    assert base, abi.last_error()
    host = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(base))
    host[:] = 0
    dst = torch.zeros(n, dtype=torch.uint8, device="cuda")
    spans = [(0, 0, 4096), (4096 + 3, 4096 + 1, 2001)]        # (src off, dst off, bytes)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream()
        for so, do, size in spans:
            rc = lib.sched_pd_copy_to_device(ctypes.c_void_p(dst.data_ptr() + do),
                                             ctypes.c_void_p(base + so), ctypes.c_uint64(size),
                                             ctypes.c_void_p(s.cuda_stream))
            assert rc == 0, abi.last_error()
    torch.cuda.synchronize()
    rng = np.random.default_rng(9)
    for rep in range(4):
        host[:] = rng.integers(0, 256, n, dtype=np.uint8)
        want = np.zeros(n, np.uint8)
        for so, do, size in spans:
            want[do:do + size] = host[so:so + size]
        dst.zero_()
        _busy(256)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy(), want), rep


def test_ring_without_staging_memory_falls_back_to_the_copy_engine(monkeypatch):
    """When the library has no staging region left, a ring takes torch's
    pinned memory and the same uploads arrive through hipMemcpyAsync."""
    lib = abi.load_library()
    monkeypatch.setattr(lib, "sched_pd_staging_alloc", lambda n: None)
    ring = sched_pd._StagingRing(torch.cuda.current_stream())
    assert ring.buf is not None
    rng = np.random.default_rng(4)
    sent = [rng.integers(0, 2**31 - 1, int(k), dtype=np.int64).astype(np.int32)
            for k in rng.integers(1, 5000, 30)]
    got = []
    for a in sent:
        out = torch.empty(a.size, dtype=torch.int32, device="cuda")
        assert ring.put(torch.from_numpy(a), out)
        got.append(out)
    torch.cuda.synchronize()
    for a, t in zip(sent, got):
        assert np.array_equal(t.cpu().numpy(), a)
