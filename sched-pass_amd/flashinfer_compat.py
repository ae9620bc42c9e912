"""flashinfer_compat.py -- FlashInfer's batch-decode wrapper, as the
reference's serving tests call it, on this library's decode kernels.

The reference drives FlashInfer's decode with (test/py/test_flashinfer_arm.py:
51-54, test/py/eval_pi_makespan.py:56-60, test/py/eval_timer_overhead.py:
56-59):

    w = flashinfer.BatchDecodeWithPagedKVCacheWrapper(workspace_u8, "NHD")
    w.plan(indptr, indices, last_page_len, num_qo_heads, num_kv_heads,
           head_dim, page_size, data_type=torch.float16,
           q_data_type=torch.float16)
    out = w.run(q, kv_cache)

and arms the levers by baking the plane's addresses into FlashInfer's JIT
build. Here the same three calls run sched_paged_decode on the cache in
place (NHD [P, 2, page, Hkv, d], HND [P, 2, Hkv, page, d], or a (k, v)
pair of either), and the levers come from a SchedPlane handed to the wrapper
(pi, policy rows, tau, timer and the ticket queue act on (request, kv-head)
tasks). Only the arguments the reference passes are taken; options that
would change the arithmetic (positional encodings, logits soft-capping,
windowed attention) are rejected rather than ignored.
"""
from __future__ import annotations

import torch

import kv_cache
import sched_pd


def _dtype(x):
    """A torch dtype, or its name as FlashInfer also accepts ("float16")."""
    if x is None or isinstance(x, torch.dtype):
        return x
    t = getattr(torch, str(x).replace("torch.", ""), None)
    if not isinstance(t, torch.dtype):
        raise ValueError(f"unknown dtype {x!r}")
    return t


class BatchDecodeWithPagedKVCacheWrapper:
    """plan() once per batch shape, run() per step (FlashInfer's contract).
    `workspace` is accepted for signature compatibility; the split-KV
    workspace is the library's own."""

    def __init__(self, workspace: torch.Tensor | None = None, kv_layout: str = "NHD", *,
                 plane=None, workers: int = 0, rt_tables: bool = False):
        if kv_layout not in ("NHD", "HND"):
            raise ValueError(f"kv_layout {kv_layout!r} (NHD or HND)")
        self.kv_layout = kv_layout
        self.plane = plane
        self.workers = int(workers)
        self.rt_tables = bool(rt_tables)
        self._plan = None

    def plan(self, indptr, indices, last_page_len, num_qo_heads: int, num_kv_heads: int,
             head_dim: int, page_size: int, *, pos_encoding_mode: str = "NONE",
             window_left: int = -1, logits_soft_cap: float | None = None,
             data_type=None, q_data_type=None, kv_data_type=None,
             sm_scale: float | None = None, **unused) -> None:
        if pos_encoding_mode != "NONE" or window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise ValueError("only plain softmax attention is supported (no positional "
                             "encoding, window or soft cap)")
        if num_qo_heads % num_kv_heads:
            raise ValueError(f"num_qo_heads {num_qo_heads} is not a multiple of "
                             f"num_kv_heads {num_kv_heads}")
        for t, what in ((indptr, "indptr"), (indices, "indices"),
                        (last_page_len, "last_page_len")):
            if not isinstance(t, torch.Tensor) or t.dtype != torch.int32:
                raise ValueError(f"{what} must be an int32 tensor")
        if data_type is not None and kv_data_type is not None and \
                _dtype(data_type) != _dtype(kv_data_type):
            raise ValueError(f"data_type {data_type} and kv_data_type {kv_data_type} differ")
        kv_dt = _dtype(kv_data_type) or _dtype(data_type) or torch.float16
        dev = indices.device
        indptr = indptr.to(dev).contiguous()
        last = last_page_len.to(dev).contiguous()
        self._plan = {
            "indptr": indptr, "indices": indices.contiguous(),
            "ctx": kv_cache.ctx_lens_from_last_page_len(indptr, last, page_size).contiguous(),
            "hq": int(num_qo_heads), "hkv": int(num_kv_heads), "d": int(head_dim),
            "page": int(page_size), "kv_dtype": kv_dt,
            "q_dtype": _dtype(q_data_type) or kv_dt, "sm_scale": sm_scale,
        }

    def _views(self, kv):
        p = self._plan
        if isinstance(kv, (tuple, list)):
            k, v = kv
            if self.kv_layout == "NHD":           # [P, page, Hkv, d] each
                return k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)
            return k, v                           # [P, Hkv, page, d] each
        if kv.dim() != 5 or kv.shape[1] != 2:
            raise ValueError(f"expected a [P, 2, ...] paged cache, got {tuple(kv.shape)}")
        if self.kv_layout == "NHD":
            return kv_cache.nhd_views(kv)
        return kv[:, 0], kv[:, 1]                 # HND: [P, Hkv, page, d]

    def _scales(self, kv_pool, k_scale, v_scale):
        """FlashInfer's fp8 scales are one float per tensor (default 1); the
        kernels read one per (page, kv-head): expand (kept per value)."""
        n = kv_pool.shape[0] * self._plan["hkv"]
        if isinstance(k_scale, torch.Tensor) or isinstance(v_scale, torch.Tensor):
            out = []
            for x in (k_scale, v_scale):
                if isinstance(x, torch.Tensor) and x.numel() == n:
                    out.append(x.to(torch.float32).contiguous())
                else:
                    val = 1.0 if x is None else float(x)
                    out.append(torch.full((n,), val, dtype=torch.float32,
                                          device=kv_pool.device))
            return out
        # two per-tensor values: expanded once into (K, V) pairs per
        # (page, kv-head), the layout whose two scales share a cache line
        kv = (1.0 if k_scale is None else float(k_scale),
              1.0 if v_scale is None else float(v_scale))
        key = (n, kv, str(kv_pool.device))
        cache = self.__dict__.setdefault("_scale_cache", {})
        if key not in cache:
            pairs = torch.tensor(kv, dtype=torch.float32, device=kv_pool.device).repeat(n, 1)
            cache[key] = (pairs[:, 0], pairs[:, 1])
        return list(cache[key])

    def run(self, q: torch.Tensor, paged_kv_cache, *, out: torch.Tensor | None = None,
            k_scale=None, v_scale=None, **kw) -> torch.Tensor:
        """k_scale / v_scale (fp8 caches): a float per tensor as FlashInfer
        takes them, or [P * Hkv] per-(page, kv-head) scales."""
        p = self._plan
        if p is None:
            raise RuntimeError("plan() must be called before run()")
        k, v = self._views(paged_kv_cache)
        if tuple(k.shape[1:]) != (p["hkv"], p["page"], p["d"]):
            raise ValueError(f"cache heads/page/dim {tuple(k.shape[1:])} do not match the "
                             f"plan ({p['hkv']}, {p['page']}, {p['d']})")
        if k.dtype != p["kv_dtype"] or q.dtype != p["q_dtype"]:
            raise ValueError(f"dtypes (q {q.dtype}, kv {k.dtype}) differ from the plan "
                             f"(q {p['q_dtype']}, kv {p['kv_dtype']})")
        if out is None:
            out = torch.empty(q.shape[0], p["hq"], p["d"], dtype=q.dtype, device=q.device)
        if k.dtype == getattr(torch, "float8_e4m3fn", None):
            kw["k_scale"], kw["v_scale"] = self._scales(k, k_scale, v_scale)
        elif k_scale is not None or v_scale is not None:
            raise ValueError("k_scale / v_scale apply to fp8 caches only")
        return sched_pd.paged_decode(q.contiguous(), k, v, p["indices"], p["ctx"], out=out,
                                     page_indptr=p["indptr"], v_layout="tokmajor",
                                     sm_scale=p["sm_scale"], plane=self.plane,
                                     workers=self.workers, rt_tables=self.rt_tables, **kw)

    forward = run
