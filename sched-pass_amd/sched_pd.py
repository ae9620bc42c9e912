"""paged_decode(): one decode step on torch-ROCm tensors through the C ABI
(`sched_paged_decode` in include/sched_pd.h).

Pool layout (HND pages):
    k_pool [num_pages, Hkv, page_size, d]    token rows, dims contiguous
    v_pool [num_pages, Hkv, page_size, d]    token-major ("tokmajor"; what
                                             kv_cache.PagedKvCache stores)
        or [num_pages, Hkv, d, page_size]    d-major ("dmajor", build_args'
                                             default argument)
Both V layouts run on the MFMA kernel for bf16 / fp16 / fp8 with d 128.
Any strides are accepted as long as the innermost listed dim is contiguous;
they are passed to the kernel in elements.

The call goes straight to the HIP library; there is no CPU path. Levers come
from a SchedPlane (its device tables), from the C runtime's armed slots
(rt_tables=True), or are absent (stock decode).
"""
from __future__ import annotations

import collections
import ctypes
import functools
import threading

import numpy as np
import torch

import sched_abi as abi

_DT = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}
if hasattr(torch, "float8_e4m3fn"):
    _DT[torch.float8_e4m3fn] = abi.FP8_E4M3


class _StagingRing:
    """Pinned host ring for the uploads of one stream (page-table rows and
    updates, context lengths, split plans, orders): a copy into the ring,
    then an asynchronous copy to the device on the stream, with no host
    allocation per upload. The ring's memory comes from
    sched_pd_staging_alloc (mapped into the device), so an upload of up to
    1 MiB runs as a copy kernel on the stream rather than on the copy
    engine (past the library's 64 staging regions, torch's pinned memory
    and the copy engine). The ring is cut into CHUNKS chunks. An upload
    that does not fit in the rest of the current chunk starts at the next
    chunk boundary and may span several chunks. Leaving a chunk, and
    finishing an upload that spans chunks, records an event on the stream
    after the copies out of them; a chunk is written again only once the
    event of its previous lap has completed (a wait only when the device lags
    a whole ring behind the host)."""
    BYTES = 16 << 20
    CHUNKS = 16
    ALIGN = 256

    def __init__(self, stream, memory=None):
        lib = abi.load_library()
        if memory is not None:                     # a retired ring's memory
            self.base, self.np, self.buf = memory
        else:
            base = lib.sched_pd_staging_alloc(ctypes.c_uint64(self.BYTES))
            if base:                               # held until the process ends
                self.buf = None
                self.np = np.ctypeslib.as_array((ctypes.c_uint8 * self.BYTES).from_address(base))
            else:
                # the library's regions are used up: torch's pinned memory,
                # which the copy engine moves
                self.buf = torch.empty(self.BYTES, dtype=torch.uint8, pin_memory=True)
                self.np = self.buf.numpy()
                base = self.buf.data_ptr()
            self.base = base
        self.copy = lib.sched_pd_copy_to_device
        self.stream = stream
        self.lock = threading.Lock()
        self.chunk = self.BYTES // self.CHUNKS
        self.cur = 0
        self.head = 0
        self.done = [None] * self.CHUNKS
        self.retired = False

    def put(self, t: torch.Tensor, out: torch.Tensor) -> bool:
        """Stage contiguous host `t` and copy it into contiguous device `out`
        (same bytes); False if `t` is too large for the ring."""
        n = t.numel() * t.element_size()
        if n > (self.CHUNKS - 1) * self.chunk:
            return False
        if n == 0:
            return True
        with self.lock:
            if self.retired:        # its memory went to another ring meanwhile
                return False
            self._put(t, out, n)
        return True

    def _enter(self, c: int) -> None:
        if self.done[c] is not None:
            self.done[c].synchronize()
            self.done[c] = None

    def _put(self, t: torch.Tensor, out: torch.Tensor, n: int) -> None:
        start = -(-self.head // self.ALIGN) * self.ALIGN
        span = None
        if start + n > (self.cur + 1) * self.chunk:
            ev = torch.cuda.Event()
            ev.record(self.stream)
            self.done[self.cur] = ev
            k = -(-n // self.chunk)                 # chunks the upload covers
            c0 = self.cur + 1
            if c0 + k > self.CHUNKS:
                c0 = 0
            for c in range(c0, c0 + k):
                self._enter(c)
            self.cur = c0 + k - 1
            start = c0 * self.chunk
            if k > 1:
                span = range(c0, c0 + k - 1)
        self.head = start + n
        # numpy into the pinned bytes, then one copy on the stream (torch's
        # copy_ pair costs ~20 us of dispatch per small upload)
        self.np[start:start + n] = t.reshape(-1).view(torch.uint8).numpy()
        rc = self.copy(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(self.base + start),
                       ctypes.c_uint64(n), ctypes.c_void_p(self.stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(abi.last_error())
        if span is not None:
            # the chunks before the last one are left now: mark them
            ev = torch.cuda.Event()
            ev.record(self.stream)
            for c in span:
                self.done[c] = ev


    def retire(self):
        """Wait until every copy out of the ring has run (everything queued
        on its stream so far) and hand back its memory for another ring."""
        with self.lock:
            ev = torch.cuda.Event()
            ev.record(self.stream)
            ev.synchronize()
            self.done = [None] * self.CHUNKS
            self.retired = True
            return self.base, self.np, self.buf


# One ring per (device, stream handle), least recently used first. A process
# that keeps making streams reuses the memory of the ring used longest ago
# (after its copies have run) once _RINGS_MAX rings exist, so the pinned
# memory held stays at _RINGS_MAX x 16 MiB.
_RINGS: "collections.OrderedDict" = collections.OrderedDict()
_RINGS_MAX = 16
_RINGS_LOCK = threading.Lock()


def _ring(dev: torch.device) -> _StagingRing:
    stream = torch.cuda.current_stream(dev)
    key = (dev.index, stream.cuda_stream)
    with _RINGS_LOCK:
        ring = _RINGS.get(key)
        if ring is None:
            memory = None
            if len(_RINGS) >= _RINGS_MAX:
                _, old = _RINGS.popitem(last=False)
                memory = old.retire()
            ring = _RINGS[key] = _StagingRing(stream, memory)
        else:
            _RINGS.move_to_end(key)
    # the live stream object (a handle can be reused by a later stream)
    ring.stream = stream
    return ring


def upload_into(dst: torch.Tensor, src) -> None:
    """Copy host `src` (numpy or CPU tensor, same bytes) into the contiguous
    device tensor `dst` through the current stream's pinned ring, without
    waiting for the device (see upload)."""
    t = torch.from_numpy(np.ascontiguousarray(src)) if isinstance(src, np.ndarray) else src
    t = t.contiguous()
    if t.numel() * t.element_size() != dst.numel() * dst.element_size() or not dst.is_contiguous():
        raise ValueError("upload_into: source and destination differ in size or layout")
    if not dst.is_cuda:
        dst.view(-1).view(torch.uint8).copy_(t.reshape(-1).view(torch.uint8))
        return
    if not _ring(dst.device).put(t, dst):
        dst.view(-1).view(torch.uint8).copy_(t.reshape(-1).view(torch.uint8).pin_memory(),
                                             non_blocking=True)


def upload(a, device) -> torch.Tensor:
    """A host array (numpy or CPU tensor) on `device`, without waiting for the
    device: staged through a pinned ring of the current stream and copied
    asynchronously on it (arrays over 15 MiB, more than the ring takes,
    through pinned memory of their own). A copy from pageable memory would first wait for every kernel
    already queued, so a serving loop's host work would never overlap its GPU
    work."""
    t = torch.from_numpy(np.ascontiguousarray(a)) if isinstance(a, np.ndarray) else a
    dev = torch.device(device)
    if dev.type != "cuda":
        return t.to(dev)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    t = t.contiguous()
    out = torch.empty(t.shape, dtype=t.dtype, device=dev)
    if not _ring(dev).put(t, out):
        out.copy_(t.pin_memory(), non_blocking=True)
    return out


def _dtype_code(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DT:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}")
    return _DT[t.dtype]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need_cuda(t: torch.Tensor, what: str) -> None:
    if t is not None and not t.is_cuda:
        raise ValueError(f"{what} must be a device tensor (got {t.device})")


def _on_launch_stream(fn):
    """Run `fn` with its `stream` argument current, so that what it queues
    on the device (uploads of host arrays, workspace clears, the queue
    counter's priming) is ordered with the launch on that stream."""
    @functools.wraps(fn)
    def run(*a, stream=None, **kw):
        if stream is None:
            return fn(*a, stream=None, **kw)
        with torch.cuda.stream(stream):
            return fn(*a, stream=stream, **kw)
    return run


@_on_launch_stream
def build_args(q, k_pool, v_pool, block_table, ctx_lens, *, out,
               mode=abi.SOFTMAX, v_layout="dmajor", page_indptr=None,
               sm_scale=None, k_scale=None, v_scale=None,
               tau_scope=abi.TAU_PREFIX, lin_w=None, lin_w_period=0,
               plane=None, rt_tables=False, workers=0, pf_dist=0, flags=0,
               policy=(1.0, 1.0, 0.25), tiles=None, tile_pages=0,
               workspace=None, check_tables=False, stream=None) -> abi.SchedDecodeArgs:
    """Fill a SchedDecodeArgs from tensors (no launch). With `tiles` (from
    plan_tiles, or a host array from plan_tiles_host or plan_ranges_host,
    which is uploaded here; built from these ctx_lens) long tasks run as
    several work items: [n, 2] (task, chunk) rows of tile_pages pages, or
    [n, 4] ranged rows (task, chunk | nchunks << 16, p0, p1). The workspace
    is taken from a cache with one per (device, stream) unless one is given.
    `stream` is the stream the launch will use (default: the current one);
    what this call queues on the device goes there too (the plan's upload,
    workspace clears, the queue counter's priming). The kernels trust the
    page table (as the reference's do);
    check_tables=True verifies it on the host first (check_page_table; this
    synchronises)."""
    a = abi.default_args()
    linear = mode == abi.LINEAR
    a.mode = mode
    a.kv_dtype = _dtype_code(v_pool, "v_pool")
    num_pages, hkv = v_pool.shape[0], v_pool.shape[1]
    if v_layout == "dmajor":
        d, ps = v_pool.shape[2], v_pool.shape[3]
        a.v_page_stride, a.v_head_stride = v_pool.stride(0), v_pool.stride(1)
        a.v_dim_stride, a.v_tok_stride = v_pool.stride(2), v_pool.stride(3)
    elif v_layout == "tokmajor":
        ps, d = v_pool.shape[2], v_pool.shape[3]
        a.v_page_stride, a.v_head_stride = v_pool.stride(0), v_pool.stride(1)
        a.v_tok_stride, a.v_dim_stride = v_pool.stride(2), v_pool.stride(3)
    else:
        raise ValueError(f"v_layout {v_layout!r}")
    a.num_kv_heads, a.head_dim, a.page_size = hkv, d, ps
    a.num_requests = ctx_lens.numel()
    if not linear:
        if k_pool.dtype != v_pool.dtype or tuple(k_pool.shape) != (num_pages, hkv, ps, d):
            raise ValueError(f"k_pool {tuple(k_pool.shape)} {k_pool.dtype} does not match "
                             f"v_pool ({num_pages}, {hkv}, {ps}, {d}) {v_pool.dtype}")
        if k_pool.stride(3) != 1:
            raise ValueError("k_pool dims must be contiguous")
        a.k_page_stride, a.k_head_stride, a.k_tok_stride = (
            k_pool.stride(0), k_pool.stride(1), k_pool.stride(2))
        if q.dim() != 3 or q.shape[0] != a.num_requests or q.shape[2] != d:
            raise ValueError(f"q must be [num_requests, Hq, {d}], got {tuple(q.shape)}")
        if not q.is_contiguous():
            raise ValueError("q must be contiguous")
        a.num_q_heads = q.shape[1]
        a.q_dtype = _dtype_code(q, "q")
        a.q = _ptr(q)
        a.k_pool = _ptr(k_pool)
        rows = a.num_q_heads
    else:
        if lin_w is None:
            raise ValueError("linear mode needs lin_w")
        a.num_q_heads = hkv
        a.lin_w = _ptr(lin_w)
        a.lin_w_period = lin_w_period
        rows = hkv
    if tuple(out.shape) != (a.num_requests, rows, d) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{a.num_requests}, {rows}, {d}], "
                         f"got {tuple(out.shape)}")
    a.o_dtype = _dtype_code(out, "out")
    a.out = _ptr(out)
    a.v_pool = _ptr(v_pool)
    for t, what in ((q, "q"), (k_pool, "k_pool"), (v_pool, "v_pool"), (out, "out"),
                    (block_table, "block_table"), (ctx_lens, "ctx_lens"),
                    (page_indptr, "page_indptr"), (k_scale, "k_scale"),
                    (v_scale, "v_scale"), (lin_w, "lin_w")):
        if t is not None and not (linear and what in ("q", "k_pool")):
            _need_cuda(t, what)
    for t, what in ((block_table, "block_table"), (ctx_lens, "ctx_lens"),
                    (page_indptr, "page_indptr")):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError(f"{what} must be contiguous int32")
    a.block_table = _ptr(block_table)
    a.ctx_lens = _ptr(ctx_lens)
    if page_indptr is not None:
        a.page_indptr = _ptr(page_indptr)
    else:
        if block_table.dim() != 2:
            raise ValueError("block_table must be [num_requests, max_pages] without page_indptr")
        a.bt_stride = block_table.stride(0)
    a.k_scale, a.v_scale = _ptr(k_scale), _ptr(v_scale)
    if check_tables:
        check_page_table(block_table, ctx_lens, ps, num_pages, page_indptr=page_indptr,
                         ctx_in_pages=bool(flags & abi.FLAG_CTX_IN_PAGES))
        if a.kv_dtype == abi.FP8_E4M3:
            for t, what in ((k_scale, "k_scale"), (v_scale, "v_scale")):
                if t is None or t.numel() < num_pages * hkv:
                    raise ValueError(f"fp8 pools need {what} with {num_pages * hkv} entries")
    a.sm_scale = 0.0 if sm_scale is None else float(sm_scale)
    a.tau_scope = tau_scope
    a.pf_dist = pf_dist
    a.policy_dT, a.policy_dR, a.policy_H = (float(x) for x in policy)
    a.flags = flags
    if isinstance(tiles, np.ndarray):
        # a host plan (plan_tiles_host, plan_ranges_host): uploaded here,
        # without waiting, and held by the arguments until they are dropped
        if tiles.ndim == 2 and tiles.shape[1] == 4:
            check_ranged_plan(tiles)
        elif tiles.ndim == 2 and tiles.shape[1] == 2:
            check_pair_plan(tiles)
        tiles = upload(np.ascontiguousarray(tiles, dtype=np.int32), k_pool.device)
        a._tiles = tiles
    if tiles is not None:
        _need_cuda(tiles, "tiles")
        if tiles.dtype != torch.int32 or tiles.dim() != 2 or tiles.shape[1] not in (2, 4) \
                or not tiles.is_contiguous():
            raise ValueError("tiles must be a contiguous int32 [num_tiles, 2] or "
                             "[num_tiles, 4] tensor")
        a.tiles = _ptr(tiles)
        a.num_tiles = tiles.shape[0]
        a.tile_format = abi.TILES_RANGED if tiles.shape[1] == 4 else abi.TILES_PAIRS
        a.tile_pages = int(tile_pages) if tiles.shape[1] == 2 else 0
        need = abi.load_library().sched_paged_decode_workspace_bytes(ctypes.byref(a))
        if need < 0:
            raise RuntimeError(abi.last_error())
        if workspace is None:
            workspace = workspace_for(need, v_pool.device,
                                      count_bytes=WS_COUNTERS_OFF + 4 * a.num_requests *
                                      a.num_kv_heads, stream=stream)
        elif workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace holds {workspace.numel()} bytes, needs {need}")
        a.workspace = _ptr(workspace)
        a.workspace_bytes = workspace.numel() * workspace.element_size()
        # held by the arguments: a later launch that needs a larger one
        # replaces the cached workspace, and these arguments must not then
        # point into memory the allocator has handed to another tensor (the
        # old workspace's counters stay zero, as each launch leaves them)
        a._ws = workspace
    if rt_tables:
        a.flags |= abi.FLAG_RT_TABLES
        a.workers = workers
    elif plane is not None:
        t = plane.tables()
        a.order, a.ctrl, a.timer, a.queue = (ctypes.c_void_p(t[k]) for k in
                                             ("order", "ctrl", "timer", "queue"))
        a.max_tasks = plane.N
        # num_tasks == 0 is the per-step disarm of the claim loop; the stock
        # path serves one task per workgroup, so launch the full grid then.
        a.workers = workers if plane.num_tasks > 0 else 0
        if a.workers:
            nitems = a.num_tiles if tiles is not None else a.num_requests * a.num_kv_heads
            if plane.num_tasks != nitems:
                # the queue hands out items [0, num_tasks): any other count
                # would skip items or leave workers idle on missing ones
                raise ValueError(f"plane.num_tasks is {plane.num_tasks}, this launch has "
                                 f"{nitems} work items: push the item count (or 0) first")
            plane.prime_queue(a.workers)
    else:
        a.max_tasks = 0
        a.workers = 0
    return a


_WS = {}


def check_page_table(block_table, ctx_lens, page_size: int, num_pages: int, *,
                     page_indptr=None, ctx_in_pages: bool = False) -> None:
    """Raise ValueError unless every page a request's context reaches is in
    its table row (2-D block table) or CSR segment, and is a pool page id in
    [0, num_pages). Host-side check (copies the tables; synchronises)."""
    ctx = ctx_lens.detach().cpu().numpy().astype(np.int64)
    if (ctx < 0).any():
        raise ValueError(f"negative context length for request {int(np.argmax(ctx < 0))}")
    need = ctx if ctx_in_pages else -(-ctx // page_size)
    bt = block_table.detach().cpu().numpy()
    if page_indptr is None:
        bt = bt.reshape(ctx.size, -1)
        if ctx.size and need.max(initial=0) > bt.shape[1]:
            r = int(np.argmax(need > bt.shape[1]))
            raise ValueError(f"request {r} needs {need[r]} pages, its table row has {bt.shape[1]}")
        rows = [bt[r, :need[r]] for r in range(ctx.size)]
    else:
        ind = page_indptr.detach().cpu().numpy().astype(np.int64)
        if ind.size != ctx.size + 1 or (np.diff(ind) < 0).any() or ind[0] < 0 \
                or ind[-1] > bt.size:
            raise ValueError("page_indptr is not a CSR index over the page list")
        have = np.diff(ind)
        if (need > have).any():
            r = int(np.argmax(need > have))
            raise ValueError(f"request {r} needs {need[r]} pages, its segment has {have[r]}")
        rows = [bt.reshape(-1)[ind[r]:ind[r] + need[r]] for r in range(ctx.size)]
    for r, ids in enumerate(rows):
        if ids.size and (ids.min() < 0 or ids.max() >= num_pages):
            raise ValueError(f"request {r} has a page id outside [0, {num_pages})")


# Workspace layout (include/sched_pd.h): a u32 stale-plan counter at byte 0,
# the per-task arrival counters from byte 256, then the partials.
WS_COUNTERS_OFF = 256


def workspace_for(nbytes: int, device, count_bytes: int = 0, stream=None) -> torch.Tensor:
    """A device workspace of at least `nbytes` whose first `count_bytes` (the
    stale counter and the per-task arrival counters) are zero, cached per
    (device, stream): launches on one stream are ordered, launches on two
    streams get two workspaces. A launch leaves its counters zero but writes
    partials right after them, so the zeroed prefix is tracked and cleared
    again when a launch needs more counters (which also clears the stale
    counter)."""
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    key = (dev.type, dev.index, int(s.cuda_stream))
    ent = _WS.get(key)
    if ent is None or ent[0].numel() < nbytes:
        ent = [torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev), 0]
        ent[1] = ent[0].numel()
        _WS[key] = ent
    need_zero = -(-count_bytes // 256) * 256
    if need_zero > ent[1]:
        ent[0][:need_zero].zero_()
    ent[1] = need_zero
    return ent[0]


def stale_plan_count(workspace: torch.Tensor, reset: bool = False) -> int:
    """Tasks the launches on `workspace` found with a stale plan (a context
    needing more chunks than the tile list held; their output rows are NaN).
    Synchronises; reset=True zeroes the counter (stream-ordered)."""
    n = int(workspace[:4].view(torch.int32).item())
    if reset:
        workspace[:4].zero_()
    return n


def workspace_of(args: abi.SchedDecodeArgs) -> torch.Tensor | None:
    """The cached workspace tensor `args` points at (None without tiles or
    for a caller-owned workspace)."""
    for ent in _WS.values():
        if args.workspace and ent[0].data_ptr() == args.workspace:
            return ent[0]
    return None


# The last plan built per (page size, tile size, kv-heads), a few at most: a
# serving loop re-plans every step, and a request's chunk count changes only
# every tile_pages * page_size tokens.
_PLANS = {}
_PLANS_MAX = 4


def plan_tiles_host(ctx_lens, page_size: int, tile_pages: int, num_kv_heads: int) -> np.ndarray:
    """The plan of plan_tiles as a host int32 array [num_tiles, 2] (a new
    array each call)."""
    ctx = np.asarray(ctx_lens.cpu() if isinstance(ctx_lens, torch.Tensor) else ctx_lens,
                     dtype=np.int64)
    npg = (ctx + page_size - 1) // page_size
    nch = np.maximum(1, (npg + tile_pages - 1) // tile_pages)
    key = (int(page_size), int(tile_pages), int(num_kv_heads))
    last = _PLANS.get(key)
    if last is not None and np.array_equal(last[0], nch):
        return last[1].copy()
    per_task = np.repeat(nch, num_kv_heads)
    tasks = np.repeat(np.arange(per_task.size, dtype=np.int32), per_task)
    starts = np.cumsum(per_task) - per_task
    plan = np.empty((tasks.size, 2), np.int32)
    plan[:, 0] = tasks
    plan[:, 1] = np.arange(tasks.size, dtype=np.int64) - np.repeat(starts, per_task)
    if key not in _PLANS and len(_PLANS) >= _PLANS_MAX:
        _PLANS.pop(next(iter(_PLANS)))
    _PLANS[key] = (nch, plan)
    return plan.copy()


def plan_tiles(ctx_lens, page_size: int, tile_pages: int, num_kv_heads: int,
               device="cuda") -> torch.Tensor:
    """Task-major split-KV plan: one (task, chunk) row per work item, chunk c
    of task (r, h) covering pages [c*tile_pages, (c+1)*tile_pages). A task has
    max(1, ceil(ceil(ctx/page_size) / tile_pages)) chunks. ctx_lens: host
    sequence (the plan is built where the lengths are known, like a serving
    scheduler's plan step), the lengths the launch will see."""
    return upload(plan_tiles_host(ctx_lens, page_size, tile_pages, num_kv_heads), device)


def plan_ranges_host(ctx_lens, page_size: int, num_kv_heads: int, task_order=None,
                     tile_pages: int = 128, tail_pages: int = 32,
                     tail_frac: float = 0.1, tau=None) -> np.ndarray:
    """A task-major ranged plan (int32 [num_tiles, 4] rows (task, chunk |
    nchunks << 16, p0, p1)) whose chunk size shrinks at the end of a claim
    order. `task_order` lists the tasks in the order a ticket queue will
    reach them (e.g. by urgency; None = task index). Tasks that start in the
    first 1 - tail_frac of the order's pages are cut into tile_pages-page
    chunks, the rest into tail_pages-page chunks: the work items claimed last
    are short, so the workers finish closer together. Each chunk but a task's
    last holds exactly its size; a task with no pages has one empty chunk.
    `tau`: per-task prefix budgets in tokens (0 = no cap), for launches that
    skip the pages past them: only the pages read are cut into chunks and
    counted, and each task's last range runs on to its context's last page,
    so no work item is empty and the plan still covers the context.
    ctx_lens: the lengths the launch will see."""
    ctx = np.asarray(ctx_lens.cpu() if isinstance(ctx_lens, torch.Tensor) else ctx_lens,
                     dtype=np.int64)
    if tile_pages < 1 or tail_pages < 1 or not 0.0 <= tail_frac <= 1.0:
        raise ValueError("tile_pages and tail_pages must be >= 1, tail_frac in [0, 1]")
    n = np.repeat(ctx, num_kv_heads)
    npg_ctx = (n + page_size - 1) // page_size
    if tau is not None:
        tau = np.asarray(tau, dtype=np.int64)
        if tau.shape != n.shape:
            raise ValueError(f"tau needs one budget per task ({n.size})")
        n = np.where(tau > 0, np.minimum(n, tau), n)
    npg = (n + page_size - 1) // page_size
    ntask = npg.size
    order = np.arange(ntask) if task_order is None else np.asarray(task_order, dtype=np.int64)
    if order.shape != (ntask,) or not np.array_equal(np.sort(order), np.arange(ntask)):
        raise ValueError(f"task_order must be a permutation of the {ntask} tasks")
    # pages claimed before each task starts, in claim order
    before = np.empty(ntask, np.int64)
    before[order] = np.cumsum(npg[order]) - npg[order]
    size = np.where(before < (1.0 - tail_frac) * npg.sum(), tile_pages, tail_pages)
    nch = np.maximum(1, (npg + size - 1) // size)
    if nch.max(initial=1) > 0xFFFF:
        raise ValueError("a task needs more than 65535 chunks; raise the chunk sizes")
    tasks = np.repeat(np.arange(ntask, dtype=np.int64), nch)
    starts = np.cumsum(nch) - nch
    chunk = np.arange(tasks.size, dtype=np.int64) - np.repeat(starts, nch)
    p0 = chunk * size[tasks]
    p1 = np.where(chunk == nch[tasks] - 1, npg_ctx[tasks],
                  np.minimum(p0 + size[tasks], npg[tasks]))
    return np.stack([tasks, chunk | (nch[tasks] << 16), p0, p1], 1).astype(np.int32)


def plan_graded_host(ctx_lens, page_size: int, num_kv_heads: int, task_order=None,
                     sizes=((0.0, 320), (0.9, 128), (0.98, 32)), tau=None) -> np.ndarray:
    """A task-major ranged plan (int32 [num_tiles, 4] rows (task, chunk |
    nchunks << 16, p0, p1)) whose chunk size is set per chunk by where the
    chunk starts in the claim order: `task_order` lists the tasks in the
    order a ticket queue reaches them (None = task index), so the pages of
    the step line up in that order, and `sizes` = [(f_0 = 0, s_0), (f_1,
    s_1), ...] (f ascending) cuts the pages that start in [f_i, f_i+1) of
    that line into chunks of s_i pages. A task crossing a boundary is cut
    there and its later pages take the smaller size. Large chunks early
    keep the per-item cost low; small ones at the very end let the workers
    finish close together. Each task's last range runs on to its context's
    last page, so the plan covers the context; a task with no pages has one
    empty chunk. `tau`: per-task prefix budgets in tokens (0 = no cap), for
    launches that skip the pages past them: only the pages read are lined
    up and cut. ctx_lens: the lengths the launch will see."""
    ctx = np.asarray(ctx_lens.cpu() if isinstance(ctx_lens, torch.Tensor) else ctx_lens,
                     dtype=np.int64)
    fr = np.asarray([f for f, _ in sizes], np.float64)
    sz = np.asarray([p for _, p in sizes], np.int64)
    if fr.size == 0 or fr[0] != 0.0 or (np.diff(fr) <= 0).any() or fr[-1] >= 1.0 \
            or (sz < 1).any():
        raise ValueError("sizes must start at fraction 0, ascend below 1, with sizes >= 1")
    n = np.repeat(ctx, num_kv_heads)
    npg_ctx = (n + page_size - 1) // page_size
    if tau is not None:
        tau = np.asarray(tau, dtype=np.int64)
        if tau.shape != n.shape:
            raise ValueError(f"tau needs one budget per task ({n.size})")
        n = np.where(tau > 0, np.minimum(n, tau), n)
    npg = (n + page_size - 1) // page_size
    ntask = npg.size
    order = np.arange(ntask) if task_order is None else np.asarray(task_order, dtype=np.int64)
    if order.shape != (ntask,) or not np.array_equal(np.sort(order), np.arange(ntask)):
        raise ValueError(f"task_order must be a permutation of the {ntask} tasks")
    # each task's pages as [a, e) on the line of the step's pages in claim order
    a = np.empty(ntask, np.int64)
    a[order] = np.cumsum(npg[order]) - npg[order]
    e = a + npg
    bounds = np.ceil(fr * npg.sum()).astype(np.int64)             # level starts on the line
    ends = np.append(bounds[1:], np.iinfo(np.int64).max)
    # segment (task, level): the task's pages on that level, then its chunks
    s0 = np.maximum(a[:, None], bounds[None, :])
    s1 = np.minimum(e[:, None], ends[None, :])
    seg = np.maximum(0, s1 - s0)
    nseg = -(-seg // sz[None, :])
    nch = np.maximum(1, nseg.sum(1))
    if nch.max(initial=1) > 0xFFFF:
        raise ValueError("a task needs more than 65535 chunks; raise the chunk sizes")
    # rows per (task, level) in task-major, level order; an empty task gets
    # one chunk of level 0
    cnt = nseg.copy()
    cnt[:, 0] += (nseg.sum(1) == 0)
    flat = cnt.ravel()
    t_of = np.repeat(np.repeat(np.arange(ntask), sz.size), flat)
    lv_of = np.repeat(np.tile(np.arange(sz.size), ntask), flat)
    first = np.cumsum(flat) - flat                               # first row of each segment
    j = np.arange(flat.sum()) - np.repeat(first, flat)           # chunk index in the segment
    base = (s0 - a[:, None]).ravel()                             # segment start, task pages
    seg_end = (s0 - a[:, None] + seg).ravel()
    p0 = np.repeat(base, flat) + j * sz[lv_of]
    p1 = np.minimum(p0 + sz[lv_of], np.repeat(seg_end, flat))
    empty = npg[t_of] == 0
    p0 = np.where(empty, 0, p0)
    p1 = np.where(empty, 0, p1)
    tstart = np.cumsum(nch) - nch
    chunk = np.arange(t_of.size) - np.repeat(tstart, nch)
    p1 = np.where(chunk == nch[t_of] - 1, npg_ctx[t_of], p1)
    return np.stack([t_of, chunk | (nch[t_of] << 16), p0, p1], 1).astype(np.int32)


class _PlanFacts:
    """What the host checks established about the last few host plans,
    keyed by content. A serving loop launches one plan for many steps (a
    request's chunk count changes every tile_pages * page_size tokens), so
    a plan is validated once and its per-task reach computed once; a lookup
    compares the array with the remembered copies (a few microseconds)."""
    MAX = 4

    def __init__(self):
        self.items = []          # [(array copy, facts dict)], most recent first
        self.lock = threading.Lock()

    def get(self, t: np.ndarray) -> dict:
        with self.lock:
            for i, (a, f) in enumerate(self.items):
                if a.shape == t.shape and a.dtype == t.dtype and np.array_equal(a, t):
                    if i:
                        self.items.insert(0, self.items.pop(i))
                    return f
            f = {}
            self.items.insert(0, (t.copy(), f))
            del self.items[self.MAX:]
            return f


_FACTS = _PlanFacts()


def check_ranged_plan(tiles) -> None:
    """Raise ValueError unless `tiles` ([n, 4] ranged rows) is task-major:
    each task's chunks consecutive, numbered 0..nchunks-1 with one nchunks,
    their page ranges contiguous from page 0. (Coverage of the context is
    the launch's check: a task whose context passes its last range is
    stale.)"""
    raw = np.asarray(tiles)
    if raw.ndim != 2 or raw.shape[1] != 4 or raw.shape[0] == 0:
        raise ValueError("ranged tiles must be a non-empty [num_tiles, 4] array")
    facts = _FACTS.get(raw)
    if facts.get("task_major"):
        return
    t = raw.astype(np.int64)
    task, chunk, nch = t[:, 0], t[:, 1] & 0xFFFF, t[:, 1] >> 16
    p0, p1 = t[:, 2], t[:, 3]
    first = chunk == 0
    start = np.maximum.accumulate(np.where(first, np.arange(len(t)), 0))
    ok = (nch >= 1) & (chunk < nch) & (p0 <= p1) & (p0 >= 0) & (task >= 0)
    ok &= chunk == np.arange(len(t)) - start          # chunk c sits c rows after chunk 0
    ok &= (task == task[start]) & (nch == nch[start])
    ok &= np.where(first, p0 == 0, p0 == np.roll(p1, 1))
    last = chunk == nch - 1
    ok &= np.where(last, True, np.roll(chunk, -1) == chunk + 1)
    if not ok.all():
        i = int(np.flatnonzero(~ok)[0])
        raise ValueError(f"ranged tiles row {i} {t[i].tolist()} is not task-major with "
                         "contiguous ranges from page 0")
    _check_one_group_per_task(task[first], "ranged")
    facts["task_major"] = True


def _check_one_group_per_task(first_tasks, what: str) -> None:
    """A task may start (chunk 0) on one row only: a second group of its rows
    would merge into the same arrival counter and could leave it nonzero."""
    u, n = np.unique(first_tasks, return_counts=True)
    if (n > 1).any():
        raise ValueError(f"{what} tiles list task {int(u[np.argmax(n > 1)])} in more than "
                         "one group of rows")


def check_plan_covers(tiles, ctx_lens, page_size: int, num_kv_heads: int,
                      tile_pages: int = 0) -> None:
    """Raise ValueError unless the host plan `tiles` ([n, 2] pair rows of
    tile_pages pages, or [n, 4] ranged rows) reaches every page of the
    contexts `ctx_lens` (tokens): the check the kernels make per task (a
    task it fails is stale: NaN output rows), made on the host before a
    launch that must not run stale, such as a fused append."""
    raw = np.asarray(tiles)
    ctx = np.asarray(ctx_lens.cpu() if isinstance(ctx_lens, torch.Tensor) else ctx_lens,
                     dtype=np.int64)
    npg = np.repeat((ctx + page_size - 1) // page_size, num_kv_heads)
    ntask = npg.size
    if raw.shape[1] != 4 and tile_pages <= 0:
        raise ValueError("pair rows need tile_pages > 0")
    facts = _FACTS.get(raw)
    key = ("reach", ntask, 0 if raw.shape[1] == 4 else int(tile_pages))
    reach = facts.get(key)
    if reach is None:
        t = raw.astype(np.int64)
        if t.shape[1] == 4:
            last = (t[:, 1] & 0xFFFF) == (t[:, 1] >> 16) - 1
            reach = np.full(ntask, -1, np.int64)
            lt = t[last]
            ok = (lt[:, 0] >= 0) & (lt[:, 0] < ntask)
            np.maximum.at(reach, lt[ok, 0], lt[ok, 3])
        else:
            ok = (t[:, 0] >= 0) & (t[:, 0] < ntask)
            nch = np.bincount(t[ok, 0], minlength=ntask)[:ntask]
            reach = np.where(nch > 0, nch * tile_pages, -1)
        facts[key] = reach
    short = reach < npg
    if short.any():
        k = int(np.argmax(short))
        raise ValueError(f"the split plan is stale: task {k} (request {k // num_kv_heads}) "
                         f"has {int(npg[k])} pages, the plan reaches {max(int(reach[k]), 0)}")


def check_pair_plan(tiles) -> None:
    """Raise ValueError unless `tiles` ([n, 2] (task, chunk) rows) is
    task-major: each task's chunks consecutive and numbered from 0, each
    task in one group of rows. (Coverage is the launch's check.)"""
    raw = np.asarray(tiles)
    if raw.ndim != 2 or raw.shape[1] != 2 or raw.shape[0] == 0:
        raise ValueError("pair tiles must be a non-empty [num_tiles, 2] array")
    facts = _FACTS.get(raw)
    if facts.get("task_major"):
        return
    t = raw.astype(np.int64)
    task, chunk = t[:, 0], t[:, 1]
    first = chunk == 0
    start = np.maximum.accumulate(np.where(first, np.arange(len(t)), 0))
    ok = (task >= 0) & (chunk >= 0) & (chunk == np.arange(len(t)) - start)
    ok &= task == task[start]
    if not ok.all():
        i = int(np.flatnonzero(~ok)[0])
        raise ValueError(f"pair tiles row {i} {t[i].tolist()} is not task-major")
    _check_one_group_per_task(task[first], "pair")
    facts["task_major"] = True


def desc_order(cost) -> np.ndarray:
    """Indices of `cost` from the largest value to the smallest, ties in
    ascending index: np.argsort(-cost, kind="stable"), as int64. Values
    that are exact in float32 (page counts, float32 costs) sort as one
    packed 64-bit key per entry, the order-preserving float32 bits above
    the index (all keys distinct, so any sort gives the stable order),
    about 3x faster than the stable float sort; other inputs take that
    sort."""
    c = np.asarray(cost, dtype=np.float64).ravel()
    n = c.size
    f = c.astype(np.float32) + np.float32(0.0)          # -0.0 ties with +0.0
    if n >= 1 << 32 or not np.array_equal(f, c):        # (NaN is never equal)
        return np.argsort(-c, kind="stable")
    bits = f.view(np.uint32).astype(np.uint64)
    # ascending order-preserving map of the float32 bits, then descending
    up = np.where(bits >> np.uint64(31), ~bits & np.uint64(0xFFFFFFFF), bits | np.uint64(1 << 31))
    keys = ((np.uint64(0xFFFFFFFF) - up) << np.uint64(32)) | np.arange(n, dtype=np.uint64)
    return (np.sort(keys) & np.uint64(0xFFFFFFFF)).astype(np.int64)


def tile_order_by_task_key(tiles: torch.Tensor, key, descending=True) -> torch.Tensor:
    """pi over work items that follows a per-task key (e.g. urgency or
    predicted cost): tiles of higher-key tasks first, chunk order kept."""
    t = tiles[:, 0].cpu().numpy() if isinstance(tiles, torch.Tensor) else np.asarray(tiles)[:, 0]
    k = np.asarray(key, dtype=np.float64)[t]
    return torch.from_numpy(desc_order(k if descending else -k).astype(np.int32))


def tile_pages_loaded(tiles: torch.Tensor, ctx_lens, page_size: int, tile_pages: int,
                      num_kv_heads: int, tau=None, tau_scope: int = abi.TAU_PREFIX) -> np.ndarray:
    """Pages each work item of a plan_tiles() or plan_ranges_host() plan
    reads when shed pages are skipped: task t reads ceil(n_t / page_size) pages, n_t = ctx, or
    min(ctx, tau_t) under a prefix budget (tau_t = 0: no cap; the per-page
    scope reads every page). Chunk c holds the pages of [c*tile_pages,
    (c+1)*tile_pages) among them, a ranged row those of [p0, p1) (0 for a
    chunk wholly past the budget)."""
    t = tiles.cpu().numpy() if isinstance(tiles, torch.Tensor) else np.asarray(tiles)
    ctx = np.asarray(ctx_lens.cpu() if isinstance(ctx_lens, torch.Tensor) else ctx_lens,
                     dtype=np.int64)
    n = np.repeat(ctx, num_kv_heads)
    if tau is not None and tau_scope == abi.TAU_PREFIX:
        tau = np.asarray(tau, dtype=np.int64)[:n.size]
        n = np.where(tau > 0, np.minimum(n, tau), n)
    pages = (n + page_size - 1) // page_size
    if t.shape[1] == 4:         # ranged rows: pages [p0, p1) of those read
        load = pages[t[:, 0]]
        p1 = np.minimum(t[:, 3].astype(np.int64), load)
        return np.maximum(0, p1 - np.minimum(t[:, 2].astype(np.int64), p1))
    return np.clip(pages[t[:, 0]] - t[:, 1].astype(np.int64) * tile_pages, 0, tile_pages)


def tile_order_lpt(cost) -> torch.Tensor:
    """pi over work items, heaviest first (ties keep index order): the
    longest-processing-time list order for the ticket queue."""
    return torch.from_numpy(desc_order(cost).astype(np.int32))


def launch(args: abi.SchedDecodeArgs, stream=None) -> None:
    """Launch one decode step described by `args` on `stream` (default: the
    current torch stream). Raises RuntimeError with the library's message."""
    lib = abi.load_library()
    s = torch.cuda.current_stream() if stream is None else stream
    rc = lib.sched_paged_decode(ctypes.byref(args), ctypes.c_void_p(s.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"sched_paged_decode failed ({rc}): {abi.last_error()}")


def launch_with_append(args: abi.SchedDecodeArgs, append_args, stream=None) -> None:
    """One launch that writes each request's new token (the one-token-per-
    request append `append_args`, a SchedKvAppendArgs) and decodes `args`
    over contexts that include it (sched_paged_decode_append): bf16, fp16 or
    fp8 caches with token-major V on the MFMA kernel. Raises RuntimeError with
    the library's message for anything else."""
    lib = abi.load_library()
    s = torch.cuda.current_stream() if stream is None else stream
    rc = lib.sched_paged_decode_append(ctypes.byref(args), ctypes.byref(append_args),
                                       ctypes.c_void_p(s.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"sched_paged_decode_append failed ({rc}): {abi.last_error()}")


def paged_decode(q, k_pool, v_pool, block_table, ctx_lens, *, out=None,
                 out_dtype=None, mode=abi.SOFTMAX, stream=None, **kw) -> torch.Tensor:
    """One decode step; returns `out` ([R, Hq, d] softmax, [R, Hkv, d] linear).
    Keyword arguments are those of build_args()."""
    if out is None:
        d = v_pool.shape[2] if kw.get("v_layout", "dmajor") == "dmajor" else v_pool.shape[3]
        rows = q.shape[1] if mode == abi.SOFTMAX else v_pool.shape[1]
        dt = out_dtype or (q.dtype if q is not None else torch.float32)
        out = torch.empty(ctx_lens.numel(), rows, d, dtype=dt, device=v_pool.device)
    args = build_args(q, k_pool, v_pool, block_table, ctx_lens, out=out, mode=mode,
                      stream=stream, **kw)
    launch(args, stream)
    return out


def kernel_kind(args: abi.SchedDecodeArgs) -> str:
    """'mfma', 'valu' (the general VALU kernel) or 'wave' (one wave per task,
    G = 1): which kernel the library picks for `args`."""
    k = abi.load_library().sched_paged_decode_kernel_kind(ctypes.byref(args))
    if k < 0:
        raise RuntimeError(abi.last_error())
    return {0: "valu", 1: "mfma", 2: "wave"}[k]


def prefetch_range(args: abi.SchedDecodeArgs) -> tuple:
    """(stock, deepest): pages in flight per wave of the kernel `args`
    selects, for stock tasks and at most for urgent ones; pf_dist may be 0 (the
    deepest) or any depth in between. (0, 0) for the VALU kernel."""
    lo, hi = abi._u32(), abi._u32()
    rc = abi.load_library().sched_paged_decode_prefetch_range(ctypes.byref(args),
                                                              ctypes.byref(lo), ctypes.byref(hi))
    if rc != 0:
        raise RuntimeError(abi.last_error())
    return lo.value, hi.value


def occupancy(args: abi.SchedDecodeArgs) -> int:
    return abi.load_library().sched_paged_decode_occupancy(ctypes.byref(args))


def cu_count() -> int:
    return abi.load_library().sched_pd_cu_count()
