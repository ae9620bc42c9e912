"""The paged KV cache the decode kernels read: page allocator, per-request
page lists, and the append path (`sched_kv_append` in include/sched_kv.h).

Formats (what the reference's tests build around FlashInfer,
test/py/eval_pi_makespan.py:46-60):
  * CSR page table: page_indptr [R+1], page indices, last_page_len [R]
    (ctx = (pages - 1) * page_size + last_page_len);
  * 2-D block table [R, max_pages] (vLLM style) with ctx_lens [R];
  * pools k [P, Hkv, page, d] and v [P, Hkv, d, page] (d-major, the MFMA
    kernel's layout) or v [P, Hkv, page, d] (token-major);
  * FlashInfer's NHD cache [P, 2, page, Hkv, d] is readable in place through
    nhd_views() (strided pools, token-major V).

Appends run on the GPU through the C ABI; there is no CPU path.
"""
from __future__ import annotations

import contextlib
import ctypes

from collections.abc import MutableMapping

import numpy as np
import torch

import sched_abi as abi
import sched_pd

_DT = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}
_SRC_DT = (torch.float32, torch.bfloat16, torch.float16)
if hasattr(torch, "float8_e4m3fn"):
    _DT[torch.float8_e4m3fn] = abi.FP8_E4M3


class OutOfPages(RuntimeError):
    """The pool has fewer free pages than an allocation needs."""


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def append(k_new, v_new, append_indptr, ctx_lens, k_pool, v_pool, block_table, *,
           page_indptr=None, v_layout="dmajor", k_scale=None, v_scale=None,
           max_append=0, errors=None, heads_per_group=0, stream=None) -> None:
    """Write source rows k_new/v_new [T, Hkv, d] (fp32, bf16 or fp16, dims
    contiguous) into the pools (fp32, bf16, fp16 or fp8 e4m3fn): request r's rows append_indptr[r] ..
    append_indptr[r+1]-1 go to positions ctx_lens[r] - n_r .. ctx_lens[r]-1
    (ctx_lens counts tokens after the append). An fp8 pool needs k_scale /
    v_scale [P * Hkv] float32 (read and written). `errors` (int32/uint32 [1],
    optional) counts (token, kv-head) pairs the kernel could not place."""
    a = build_append_args(k_new, v_new, append_indptr, ctx_lens, k_pool, v_pool, block_table,
                          page_indptr=page_indptr, v_layout=v_layout, k_scale=k_scale,
                          v_scale=v_scale, max_append=max_append, errors=errors,
                          heads_per_group=heads_per_group)
    launch_append(a, stream if stream is not None else torch.cuda.current_stream(k_pool.device))


def launch_append(a: abi.SchedKvAppendArgs, stream) -> None:
    """Launch a prepared append on a torch stream (the tensors behind `a`
    must stay alive until it has run)."""
    lib = abi.load_library()
    if lib.sched_kv_append(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream)) != 0:
        raise RuntimeError(abi.last_error())


def build_append_args(k_new, v_new, append_indptr, ctx_lens, k_pool, v_pool, block_table, *,
                      page_indptr=None, v_layout="dmajor", k_scale=None, v_scale=None,
                      max_append=0, errors=None, heads_per_group=0) -> abi.SchedKvAppendArgs:
    """Validate and fill a SchedKvAppendArgs (no launch); see append()."""
    a = abi.default_kv_args()
    if k_new.dtype not in _SRC_DT or v_new.dtype != k_new.dtype:
        raise TypeError(f"sources must both be float32, bfloat16 or float16, got "
                        f"{k_new.dtype}, {v_new.dtype}")
    if k_pool.dtype not in _DT or v_pool.dtype != k_pool.dtype:
        raise TypeError(f"pool dtypes {k_pool.dtype}, {v_pool.dtype}")
    if k_new.dim() != 3 or k_new.shape != v_new.shape or k_new.stride() != v_new.stride():
        raise ValueError("k_new and v_new must be [T, Hkv, d] with the same strides")
    if k_new.stride(2) != 1:
        raise ValueError("source dims must be contiguous")
    P, hkv, ps, d = k_pool.shape
    if k_new.shape[1:] != (hkv, d):
        raise ValueError(f"sources {tuple(k_new.shape)} vs pool heads/dims ({hkv}, {d})")
    if k_pool.stride(3) != 1:
        raise ValueError("k_pool dims must be contiguous")
    a.src_dtype = _DT[k_new.dtype]
    a.kv_dtype = _DT[k_pool.dtype]
    a.num_requests = ctx_lens.numel()
    a.num_kv_heads, a.head_dim, a.page_size = hkv, d, ps
    a.num_tokens = k_new.shape[0]
    a.max_append = int(max_append)
    a.num_pages = P
    a.src_tok_stride, a.src_head_stride = k_new.stride(0), k_new.stride(1)
    a.k_page_stride, a.k_head_stride, a.k_tok_stride = k_pool.stride()[:3]
    if v_layout == "dmajor":
        if tuple(v_pool.shape) != (P, hkv, d, ps):
            raise ValueError(f"d-major v_pool must be {(P, hkv, d, ps)}, got {tuple(v_pool.shape)}")
        a.v_page_stride, a.v_head_stride = v_pool.stride(0), v_pool.stride(1)
        a.v_dim_stride, a.v_tok_stride = v_pool.stride(2), v_pool.stride(3)
    elif v_layout == "tokmajor":
        if tuple(v_pool.shape) != (P, hkv, ps, d):
            raise ValueError(f"token-major v_pool must be {(P, hkv, ps, d)}, "
                             f"got {tuple(v_pool.shape)}")
        a.v_page_stride, a.v_head_stride = v_pool.stride(0), v_pool.stride(1)
        a.v_tok_stride, a.v_dim_stride = v_pool.stride(2), v_pool.stride(3)
    else:
        raise ValueError(f"v_layout {v_layout!r}")
    for t, what in ((k_new, "k_new"), (v_new, "v_new"), (k_pool, "k_pool"), (v_pool, "v_pool"),
                    (append_indptr, "append_indptr"), (ctx_lens, "ctx_lens"),
                    (block_table, "block_table"), (page_indptr, "page_indptr"),
                    (k_scale, "k_scale"), (v_scale, "v_scale"), (errors, "errors")):
        if t is not None and not t.is_cuda:
            raise ValueError(f"{what} must be a device tensor (got {t.device})")
    for t, what in ((append_indptr, "append_indptr"), (ctx_lens, "ctx_lens"),
                    (block_table, "block_table"), (page_indptr, "page_indptr")):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError(f"{what} must be contiguous int32")
    if append_indptr.numel() != a.num_requests + 1:
        raise ValueError("append_indptr needs num_requests + 1 entries")
    if page_indptr is None:
        if block_table.dim() != 2:
            raise ValueError("block_table must be [num_requests, max_pages] without page_indptr")
        a.bt_stride = block_table.stride(0)
    elif page_indptr.numel() != a.num_requests + 1:
        raise ValueError("page_indptr needs num_requests + 1 entries")
    if a.kv_dtype == abi.FP8_E4M3:
        check_scales(k_scale, v_scale, P * hkv)
    if errors is not None and (errors.dtype not in (torch.int32, torch.uint32)
                               or errors.numel() < 1):
        raise ValueError("errors must be a 32-bit integer tensor")
    a.k_src, a.v_src = _ptr(k_new), _ptr(v_new)
    a.append_indptr, a.ctx_lens = _ptr(append_indptr), _ptr(ctx_lens)
    a.block_table, a.page_indptr = _ptr(block_table), _ptr(page_indptr)
    a.k_pool, a.v_pool = _ptr(k_pool), _ptr(v_pool)
    if a.kv_dtype == abi.FP8_E4M3:
        a.k_scale, a.v_scale = _ptr(k_scale), _ptr(v_scale)
    a.errors = _ptr(errors)
    a.heads_per_group = int(heads_per_group)
    return a


def ctx_lens_from_last_page_len(page_indptr, last_page_len, page_size: int):
    """CSR page counts + last-page fill -> token counts (0 pages -> 0)."""
    pages = page_indptr[1:] - page_indptr[:-1]
    ctx = (pages - 1) * page_size + last_page_len
    return torch.where(pages > 0, ctx, torch.zeros_like(ctx)).to(torch.int32)


def nhd_views(kv):
    """FlashInfer's NHD paged cache [P, 2, page, Hkv, d] as (k_pool, v_pool)
    views [P, Hkv, page, d] for paged_decode(..., v_layout="tokmajor")."""
    if kv.dim() != 5 or kv.shape[1] != 2:
        raise ValueError(f"expected [P, 2, page, Hkv, d], got {tuple(kv.shape)}")
    return kv[:, 0].permute(0, 2, 1, 3), kv[:, 1].permute(0, 2, 1, 3)


class PageAllocator:
    """LIFO free list over page ids 0..num_pages-1 (host side). Freed pages
    are reused first, which keeps a steady-state batch on recently touched
    pages."""

    def __init__(self, num_pages: int):
        self.num_pages = int(num_pages)
        self._stack = np.arange(self.num_pages - 1, -1, -1, dtype=np.int32)
        self._top = self.num_pages
        self._used = np.zeros(self.num_pages, dtype=bool)

    @property
    def num_free(self) -> int:
        return self._top

    def alloc(self, n: int) -> np.ndarray:
        n = int(n)
        if n < 0:
            raise ValueError("negative page count")
        if n > self._top:
            raise OutOfPages(f"need {n} pages, {self._top} free of {self.num_pages}")
        pages = self._stack[self._top - n:self._top][::-1].copy()
        self._top -= n
        self._used[pages] = True
        return pages

    def free(self, pages) -> None:
        pages = np.asarray(pages, dtype=np.int32).ravel()
        if pages.size == 0:
            return
        if pages.min() < 0 or pages.max() >= self.num_pages:
            raise ValueError("page id outside the pool")
        if np.unique(pages).size != pages.size or not self._used[pages].all():
            raise ValueError("freeing a page that is not allocated (double free?)")
        self._used[pages] = False
        self._stack[self._top:self._top + pages.size] = pages[::-1]
        self._top += pages.size


class _Lengths(MutableMapping):
    """PagedKvCache.lens: request id -> tokens held. A dict-like view of the
    cache's per-request length array (writes go to the array). Requests come
    and go through add_request / release."""

    def __init__(self, cache):
        self._c = cache

    def __getitem__(self, rid):
        return int(self._c._len[self._c._slot[rid]])

    def __setitem__(self, rid, value):
        if rid not in self._c._slot:
            raise KeyError(f"request {rid!r} not in the cache (add_request first)")
        self._c._len[self._c._slot[rid]] = int(value)

    def __delitem__(self, rid):
        raise TypeError("release(rid) removes a request")

    def __iter__(self):
        return iter(self._c._slot)

    def __len__(self):
        return len(self._c._slot)


def paired_scales(n: int, device) -> tuple:
    """Zeroed fp32 scales for n (page, kv-head)s as (K, V) pairs: one [n, 2]
    tensor, returned as its two columns (k_scale, v_scale). The kernels see
    v_scale == k_scale + 1 and read a (page, head)'s two scales from one
    cache line (separate [n] arrays take a line each)."""
    pairs = torch.zeros(n, 2, dtype=torch.float32, device=device)
    return pairs[:, 0], pairs[:, 1]


def check_scales(k_scale, v_scale, n: int) -> None:
    """Raise ValueError unless k_scale / v_scale hold float32 scales for n
    (page, kv-head)s: two contiguous arrays, or the two columns of one
    [n, 2] (K, V) pair array (paired_scales)."""
    for t, what in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        if t is None or t.dtype != torch.float32 or t.numel() < n:
            raise ValueError(f"an fp8 pool needs float32 {what} for {n} (page, kv-head)s")
    if k_scale.is_contiguous() and v_scale.is_contiguous():
        return
    paired = (k_scale.dim() >= 1 and k_scale.stride(-1) == 2 and v_scale.stride(-1) == 2
              and v_scale.data_ptr() == k_scale.data_ptr() + 4
              and tuple(k_scale.shape) == tuple(v_scale.shape)
              and (k_scale.dim() == 1 or k_scale.stride(-2) == 2 * k_scale.shape[-1]))
    if not paired:
        raise ValueError("k_scale / v_scale must be contiguous, or the (K, V) columns of one "
                         "pair array")


def _on_stream(stream):
    """The stream a step's work goes to: `stream`, or the current one."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _host_plan(tiles):
    """A host split plan to upload with the step's other arrays (ranged rows
    checked first), or None for no plan or one already on the device."""
    if not isinstance(tiles, np.ndarray):
        return None
    if tiles.ndim == 2 and tiles.shape[1] == 4:
        sched_pd.check_ranged_plan(tiles)
    elif tiles.ndim == 2 and tiles.shape[1] == 2:
        sched_pd.check_pair_plan(tiles)
    return tiles


class PagedKvCache:
    """Pools + allocator + per-request page lists for one layer's KV.

    k_pool [P, Hkv, page, d]; v_pool [P, Hkv, d, page] (d-major) or
    [P, Hkv, page, d] (token-major); for an fp8 cache k_scale / v_scale
    [P * Hkv] (index page * Hkv + head).

    v_layout "auto" is token-major V for every page size and dtype, chosen by
    what a serving step costs (the writer appends each request's token, then
    the decode reads the batch; Llama-3-8B batch, 64 x 2048 tokens):
    - 16-token pages: bf16 87.8 us token-major against 90.7 us d-major (the
      decode alone is ~1% faster d-major, but a d-major append writes one
      token as a 128-row column, 7.7x its bytes); fp8 55.5 against 55.9 us;
    - larger pages: a 16-token block of a d-major V row is a partial row, and
      the decode alone measured 98 / 109 / 109 us for 32- / 64- / 128-token
      bf16 pages against 87 / 86 / 86 us token-major, fp8 54 / 62 us against
      48 / 48;
    - fp32 caches (the VALU kernels) read token-major rows with coalesced
      loads.
    "dmajor" stays available."""

    def __init__(self, num_pages: int, num_kv_heads: int, head_dim: int, page_size: int = 16,
                 dtype=torch.bfloat16, device="cuda", v_layout: str = "auto"):
        self.page_size, self.num_kv_heads, self.head_dim = page_size, num_kv_heads, head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        if v_layout == "auto":
            v_layout = "tokmajor"
        if v_layout not in ("dmajor", "tokmajor"):
            raise ValueError(f"v_layout {v_layout!r}")
        self.v_layout = v_layout
        self.k_pool = torch.zeros(num_pages, num_kv_heads, page_size, head_dim, dtype=dtype,
                                  device=self.device)
        vshape = (head_dim, page_size) if v_layout == "dmajor" else (page_size, head_dim)
        self.v_pool = torch.zeros(num_pages, num_kv_heads, *vshape, dtype=dtype,
                                  device=self.device)
        fp8 = dtype == getattr(torch, "float8_e4m3fn", None)
        # fp8: (K, V) scale pairs per (page, kv-head), k_scale / v_scale
        # being the pair array's columns
        self.k_scale, self.v_scale = paired_scales(num_pages * num_kv_heads, self.device) \
            if fp8 else (None, None)
        self.allocator = PageAllocator(num_pages)
        # Per request: its page list (pages[rid]) and, in arrays indexed by a
        # slot, its token count and page count, so that a step's bookkeeping
        # over a batch is array arithmetic rather than a loop over requests.
        self.pages: dict = {}
        self._slot: dict = {}
        self._free_slots: list = []
        self._len = np.zeros(64, np.int64)
        self._npg = np.zeros(64, np.int64)
        self.lens = _Lengths(self)
        self._batch = (None, None)   # (rids as a tuple, their slots): a batch repeats
        self._table = None       # the device block table of the last request list

    # -- bookkeeping ----------------------------------------------------------
    def add_request(self, rid) -> None:
        if rid in self.pages:
            raise KeyError(f"request {rid!r} already present")
        if self._free_slots:
            slot = self._free_slots.pop()
        else:
            slot = len(self._slot)
            if slot >= self._len.size:
                self._len = np.concatenate([self._len, np.zeros_like(self._len)])
                self._npg = np.concatenate([self._npg, np.zeros_like(self._npg)])
        self._slot[rid] = slot
        self._len[slot] = 0
        self._npg[slot] = 0
        self.pages[rid] = []
        self._batch = (None, None)

    def release(self, rid) -> None:
        self.allocator.free(self.pages.pop(rid))
        slot = self._slot.pop(rid)
        self._len[slot] = 0
        self._npg[slot] = 0
        self._free_slots.append(slot)
        self._batch = (None, None)
        self._table = None

    def truncate(self, rids, lens) -> None:
        """Drop request rids[i]'s tokens past lens[i] (at most its length) and
        free the pages they alone used (a rejected speculation, or a replay
        from an earlier state)."""
        key, s = self._slots(rids)
        new = np.asarray(lens, np.int64)
        if new.size != len(key) or (new < 0).any() or (new > self._len[s]).any():
            raise ValueError("truncate: lengths must be within the requests' lengths")
        keep = -(-new // self.page_size)
        for i in np.nonzero(keep < self._npg[s])[0]:
            pages = self.pages[key[i]]
            self.allocator.free(pages[keep[i]:])
            del pages[keep[i]:]
        self._len[s] = new
        self._npg[s] = np.minimum(self._npg[s], keep)
        self._table = None

    def _batch_distinct(self) -> bool:
        """Whether the last batch _slots() looked up names each request once
        (checked once per batch)."""
        key, s = self._batch
        if getattr(self, "_distinct", (None,))[0] is not s:
            self._distinct = (s, np.unique(s).size == s.size)
        return self._distinct[1]

    def _slots(self, rids) -> tuple:
        """(rids as a tuple, their slots), cached for a repeated list."""
        key = tuple(rids)
        if key != self._batch[0]:
            try:
                slots = np.fromiter((self._slot[r] for r in key), np.int64, len(key))
            except KeyError as e:
                raise KeyError(f"request {e.args[0]!r} not in the cache") from None
            self._batch = (key, slots)
        return self._batch

    def lengths(self, rids) -> np.ndarray:
        """Tokens each request holds, as an int64 array in rids' order (a
        copy; one gather instead of a lookup per request)."""
        return self._len[self._slots(rids)[1]]

    def reserve(self, rids, counts) -> None:
        """Allocate pages so that each request has room for counts[i] more
        tokens; all or nothing."""
        key, s = self._slots(rids)
        want = -(-(self._len[s] + np.asarray(counts, np.int64)) // self.page_size)
        need = np.maximum(want - self._npg[s], 0)
        total = int(need.sum())
        if total > self.allocator.num_free:
            raise OutOfPages(f"need {total} pages, {self.allocator.num_free} free")
        if total == 0:
            return
        fresh = self.allocator.alloc(total).tolist()
        at = 0
        for i in np.nonzero(need)[0]:       # only the requests that cross a page
            k = int(need[i])
            self.pages[key[i]].extend(fresh[at:at + k])
            at += k
        np.add.at(self._npg, s, need)

    # -- tables ---------------------------------------------------------------
    def block_table(self, rids):
        """(block_table [R, width] int32, ctx_lens [R] int32) on the device;
        unused entries are -1, width >= every request's page count.

        The table for a list of requests stays on the device between calls:
        a call with the same list uploads only the entries of pages added
        since (a decode step adds at most one page per request), so a serving
        step does not rebuild and copy R x max_pages entries. The update is
        stream-ordered after the launches that read the previous contents. A
        different list, a request that outgrew the width, or a released page
        rebuilds the table (width with headroom)."""
        key, s = self._slots(rids)
        bt, ctx, _ = self._table_step(key, s)
        return bt, ctx

    def _table_step(self, key, s, extra=()):
        """block_table() for the batch (key, s), with the host int32 arrays
        `extra` uploaded in the same copy as the lengths and the table
        update; returns (table, ctx_lens, [extra on the device])."""
        counts = self._npg[s]
        ctx = self._len[s].astype(np.int32)
        t = self._table
        parts, upd_n = [ctx], 0
        if (t is None or t["key"] != key or t["counts"].size != counts.size
                or (counts.size and (counts.max() > t["width"]
                                     or (counts < t["counts"]).any()))):
            width = max(int(counts.max()) if counts.size else 1, 1)
            width = -(-(width + width // 4 + 1) // 64) * 64     # headroom for growth
            bt = np.full((len(key), width), -1, dtype=np.int32)
            for i, r in enumerate(key):
                bt[i, :counts[i]] = self.pages[r]
            t = {"key": key, "width": width, "counts": counts,
                 "dev": sched_pd.upload(bt, self.device)}
            self._table = t
        else:
            grew = np.nonzero(counts > t["counts"])[0]
            if grew.size:
                rows, cols, vals = [], [], []
                for i in grew:
                    lo, hi = int(t["counts"][i]), int(counts[i])
                    rows.extend([i] * (hi - lo))
                    cols.extend(range(lo, hi))
                    vals.extend(self.pages[key[i]][lo:hi])
                parts.append(np.array([rows, cols, vals], np.int32).ravel())
                upd_n = len(rows)
                t["counts"] = counts
        extra = [np.ascontiguousarray(e, dtype=np.int32) for e in extra]
        parts.extend(e.ravel() for e in extra)
        # one copy for the lengths, the table update and the extras
        dev = sched_pd.upload(np.concatenate(parts) if len(parts) > 1 else ctx, self.device)
        n = len(key)
        ctx_dev, off = dev[:n], n
        if upd_n:
            upd = dev[off:off + 3 * upd_n]
            tab = t["dev"]
            if tab.is_cuda:
                # one small kernel of the library (torch's indexed assignment
                # would add two index conversions and an index_put per step)
                rc = abi.load_library().sched_kv_table_update(
                    ctypes.c_void_p(tab.data_ptr()), tab.shape[0], tab.shape[1],
                    ctypes.c_void_p(upd.data_ptr()), upd_n,
                    ctypes.c_void_p(torch.cuda.current_stream(tab.device).cuda_stream))
                if rc != 0:
                    raise RuntimeError(abi.last_error())
            else:
                u = upd.view(3, upd_n).long()
                tab[u[0], u[1]] = u[2].int()
            off += 3 * upd_n
        out = []
        for e in extra:
            out.append(dev[off:off + e.size].view(e.shape))
            off += e.size
        return t["dev"], ctx_dev, out

    def csr(self, rids):
        """(page_indptr [R+1], indices, last_page_len [R]) int32 on the device."""
        counts = np.array([len(self.pages[r]) for r in rids], dtype=np.int64)
        indptr = np.zeros(len(rids) + 1, dtype=np.int32)
        indptr[1:] = np.cumsum(counts)
        indices = np.array([p for r in rids for p in self.pages[r]], dtype=np.int32)
        last = np.array([self.lens[r] - (len(self.pages[r]) - 1) * self.page_size
                         if self.pages[r] else 0 for r in rids], dtype=np.int32)
        to = lambda x: sched_pd.upload(x, self.device)  # noqa: E731
        return to(indptr), to(indices if indices.size else np.zeros(1, np.int32)), to(last)

    # -- writes and reads -----------------------------------------------------
    def append(self, rids, k_new, v_new, counts=None, errors=None) -> None:
        """Append counts[i] rows (default 1 each) of k_new / v_new [T, Hkv, d]
        to request rids[i], rows in request order."""
        key, s = self._slots(rids)
        counts = (np.ones(len(key), np.int64) if counts is None
                  else np.asarray([int(c) for c in counts], np.int64))
        if counts.size != len(key):
            raise ValueError(f"{counts.size} counts for {len(key)} requests")
        if np.unique(s).size != s.size:
            raise ValueError("a request appears twice in one append")
        if (counts < 0).any() or int(counts.sum()) != k_new.shape[0]:
            raise ValueError(f"counts sum to {int(counts.sum())}, sources have "
                             f"{k_new.shape[0]} rows")
        held = self._npg[s].copy()
        self.reserve(key, counts)
        try:
            self._len[s] += counts
            app = np.zeros(len(key) + 1, dtype=np.int32)
            app[1:] = np.cumsum(counts)
            bt, ctx, (app_dev,) = self._table_step(key, s, (app,))
            append(k_new, v_new, app_dev, ctx, self.k_pool,
                   self.v_pool, bt, v_layout=self.v_layout, k_scale=self.k_scale,
                   v_scale=self.v_scale,
                   max_append=int(counts.max()) if counts.size else 0, errors=errors)
        except Exception:
            # a rejected launch leaves the cache as it was
            self._len[s] -= counts
            for i in np.nonzero(self._npg[s] != held)[0]:
                rid = key[i]
                self.allocator.free(self.pages[rid][held[i]:])
                del self.pages[rid][held[i]:]
            self._npg[s] = held
            self._table = None
            raise

    def decode_step(self, q, rids, k_new, v_new, **kw):
        """One serving step: append each request's new token (k_new / v_new
        [R, Hkv, d], row i for rids[i]) and decode over the contexts that now
        hold it. A bf16, fp16 or fp8 cache with token-major V and head dim
        128 does both in one launch (the decode writes the token into its
        page before reading it, an fp8 page's scale grown as the writer
        grows it); a d-major V runs the writer, then the decode. Keyword
        arguments are those of decode() (`out`, `plane`, `tiles`, ...); a
        split plan must be built from the lengths after the append. With
        `stream`, the step's uploads, table update and launches all go to
        that stream."""
        with _on_stream(kw.get("stream")):
            return self._decode_step(q, rids, k_new, v_new, **kw)

    def _decode_step(self, q, rids, k_new, v_new, **kw):
        # the MFMA kernel's shapes (16-bit Q of the cache's type, bf16 Q for
        # an fp8 cache, 1..16 q-heads per kv-head, head dim 128)
        G = q.shape[1] // self.num_kv_heads if q.shape[1] % self.num_kv_heads == 0 else 0
        fp8 = self.k_scale is not None
        q_ok = q.dtype == torch.bfloat16 if fp8 else q.dtype == self.dtype
        fusable = (q_ok and (fp8 or self.dtype in (torch.bfloat16, torch.float16))
                   and 1 <= G <= 16 and self.v_layout == "tokmajor" and self.head_dim == 128
                   and self.page_size in (16, 32, 64, 128, 256)
                   and kw.get("mode", abi.SOFTMAX) == abi.SOFTMAX
                   and not (kw.get("flags", 0) & (abi.FLAG_FORCE_VALU | abi.FLAG_CTX_IN_PAGES)))
        if not fusable:
            self.append(rids, k_new, v_new)
            return self.decode(q, rids, **kw)
        key, s = self._slots(rids)
        if k_new.shape[0] != len(key) or v_new.shape[0] != len(key):
            raise ValueError(f"{k_new.shape[0]} source rows for {len(key)} requests")
        if not self._batch_distinct():
            raise ValueError("a request appears twice in one step")
        held = self._npg[s].copy()
        self.reserve(key, np.ones(len(key), np.int64))
        try:
            self._len[s] += 1
            tiles = _host_plan(kw.get("tiles"))
            if tiles is not None:
                # a stale plan would leave this step's output rows NaN: refuse
                # it before anything is written
                sched_pd.check_plan_covers(tiles, self._len[s], self.page_size,
                                           self.num_kv_heads, kw.get("tile_pages", 0))
            bt, ctx, ex = self._table_step(key, s, () if tiles is None else (tiles,))
            if tiles is not None:
                kw["tiles"] = ex[0]      # uploaded with the lengths and table update
            kw.setdefault("v_layout", self.v_layout)
            out = kw.pop("out", None)
            if out is None:
                dt = kw.pop("out_dtype", None) or q.dtype
                out = torch.empty(len(key), q.shape[1], self.head_dim, dtype=dt,
                                  device=self.device)
            args = sched_pd.build_args(q, self.k_pool, self.v_pool, bt, ctx, out=out,
                                       k_scale=self.k_scale, v_scale=self.v_scale, **kw)
            if getattr(self, "_app_indptr", None) is None or \
                    self._app_indptr.numel() != len(key) + 1:
                self._app_indptr = torch.arange(len(key) + 1, dtype=torch.int32,
                                                device=self.device)
            app = build_append_args(k_new, v_new, self._app_indptr, ctx, self.k_pool,
                                    self.v_pool, bt, v_layout=self.v_layout, max_append=1,
                                    k_scale=self.k_scale, v_scale=self.v_scale)
            sched_pd.launch_with_append(args, app, kw.get("stream"))
        except Exception:
            self._len[s] -= 1
            for i in np.nonzero(self._npg[s] != held)[0]:
                rid = key[i]
                self.allocator.free(self.pages[rid][held[i]:])
                del self.pages[rid][held[i]:]
            self._npg[s] = held
            self._table = None
            raise
        return out

    def decode(self, q, rids, **kw):
        """One decode step over the requests' current contexts. A host split
        plan (`tiles` from sched_pd.plan_tiles_host or plan_ranges_host) is
        uploaded together with the lengths and table update. With `stream`,
        the uploads, table update and launch all go to that stream."""
        with _on_stream(kw.get("stream")):
            return self._decode(q, rids, **kw)

    def _decode(self, q, rids, **kw):
        key, s = self._slots(rids)
        tiles = _host_plan(kw.get("tiles"))
        bt, ctx, ex = self._table_step(key, s, () if tiles is None else (tiles,))
        if tiles is not None:
            kw["tiles"] = ex[0]
        kw.setdefault("v_layout", self.v_layout)
        return sched_pd.paged_decode(q, self.k_pool, self.v_pool, bt, ctx, k_scale=self.k_scale,
                                     v_scale=self.v_scale, **kw)
