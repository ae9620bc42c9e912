"""Oracle for the paged-decode hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import
this module, and only for expected values / the timed CPU baseline; no product code
path imports, loads or calls anything under oracle/.

The KV-cache writer's restatement is kv_append() (kv_oracle.c), with the
fp8 encoder and scale rule it uses exposed for their own pins.

Two independent CPU restatements of the reference's truncated attention:
  * decode(): liboracle.so (oracle.c), the reference's online-softmax loop
    (test/paged_decode.cu:124-153, test/py/test_dynamic_loop.py:77-100) in
    fp64 (the expected values) or fp32 (the CPU baseline), OpenMP over tasks;
  * numpy_decode(): the closed form out = sum_{t in kept} e^{s_t - max} v_t /
    sum_{t in kept} e^{s_t - max} in float64 numpy, written from the layout
    semantics (no argument block), used on small inputs to pin decode().
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "liboracle.so")
sys.path.insert(0, os.path.join(ROOT, "sched-pass_amd"))

import sched_abi as abi  # noqa: E402  (the ABI mirror: ctypes only, no GPU)

F64, F32 = 0, 1
_lib = None


def build() -> str:
    """Compile liboracle.so with gcc (OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is None:
        srcs = [os.path.join(HERE, f) for f in ("oracle.c", "kv_oracle.c")]
        if not os.path.exists(LIB_PATH) or (
                os.path.getmtime(LIB_PATH) < max(os.path.getmtime(f) for f in srcs)):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_decode.restype = ctypes.c_int
        lib.oracle_decode.argtypes = [ctypes.POINTER(abi.SchedDecodeArgs), ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_int]
        lib.oracle_bf16_to_float.restype = ctypes.c_float
        lib.oracle_bf16_to_float.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_float.restype = ctypes.c_float
        lib.oracle_f16_to_float.argtypes = [ctypes.c_uint16]
        lib.oracle_fp8_e4m3_to_float.restype = ctypes.c_float
        lib.oracle_fp8_e4m3_to_float.argtypes = [ctypes.c_uint8]
        lib.oracle_max_threads.restype = ctypes.c_int
        lib.oracle_args_layout.restype = ctypes.c_int
        lib.oracle_args_layout.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int]
        lib.oracle_kv_args_layout.restype = ctypes.c_int
        lib.oracle_kv_args_layout.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int]
        lib.oracle_kv_append.restype = ctypes.c_long
        lib.oracle_kv_append.argtypes = [ctypes.POINTER(abi.SchedKvAppendArgs)]
        lib.oracle_fp8_e4m3_from_float.restype = ctypes.c_uint8
        lib.oracle_fp8_e4m3_from_float.argtypes = [ctypes.c_float]
        lib.oracle_float_to_bf16.restype = ctypes.c_uint16
        lib.oracle_float_to_bf16.argtypes = [ctypes.c_float]
        lib.oracle_float_to_f16.restype = ctypes.c_uint16
        lib.oracle_float_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_pow2_scale.restype = ctypes.c_float
        lib.oracle_pow2_scale.argtypes = [ctypes.c_float]
        _lib = lib
    return _lib


_NP_CODE = {np.dtype(np.float32): abi.F32}


def _host(x, dtype=None):
    """torch tensor / numpy array -> contiguous numpy array (bf16 and fp8
    torch tensors become their raw uint16 / uint8 bit patterns)."""
    if x is None:
        return None, None
    try:
        import torch
        if isinstance(x, torch.Tensor):
            t = x.detach().cpu().contiguous()
            if t.dtype == torch.bfloat16:
                return t.view(torch.int16).numpy().view(np.uint16), abi.BF16
            if t.dtype == torch.float16:
                return t.view(torch.int16).numpy().view(np.uint16), abi.F16
            if hasattr(torch, "float8_e4m3fn") and t.dtype == torch.float8_e4m3fn:
                return t.view(torch.uint8).numpy(), abi.FP8_E4M3
            x = t.numpy()
    except ImportError:
        pass
    a = np.ascontiguousarray(x if dtype is None else np.asarray(x, dtype=dtype))
    return a, _NP_CODE.get(a.dtype)


def decode(q, k_pool, v_pool, block_table, ctx_lens, *, mode=abi.SOFTMAX,
           v_layout="dmajor", page_indptr=None, sm_scale=None, k_scale=None,
           v_scale=None, tau_scope=abi.TAU_PREFIX, lin_w=None, lin_w_period=0,
           ctrl=None, max_tasks=abi.SCHED_MAX_TASKS, ctx_in_pages=False,
           precision=F64, threads=0):
    """Reference output for one decode step, on host copies of the inputs.
    ctrl: SchedCtrl bytes (bytes / uint8 array) or None (no shed).
    Returns float64 (F64) or float32 (F32) [R, rows, d]."""
    lib = load()
    keep = []  # keep numpy buffers alive for the call

    def ptr(x, dtype=None):
        a, code = _host(x, dtype)
        if a is None:
            return None, None, None
        keep.append(a)
        return ctypes.c_void_p(a.ctypes.data), code, a

    a = abi.default_args()
    a.mode = mode
    vp, a.kv_dtype, varr = ptr(v_pool)
    num_pages, hkv = varr.shape[0], varr.shape[1]
    st = [s // varr.itemsize for s in varr.strides]
    if v_layout == "dmajor":
        d, ps = varr.shape[2], varr.shape[3]
        a.v_page_stride, a.v_head_stride, a.v_dim_stride, a.v_tok_stride = st
    else:
        ps, d = varr.shape[2], varr.shape[3]
        a.v_page_stride, a.v_head_stride, a.v_tok_stride, a.v_dim_stride = st
    a.v_pool = vp
    a.num_kv_heads, a.head_dim, a.page_size = hkv, d, ps
    ctx_p, _, ctx_arr = ptr(ctx_lens, np.int32)
    a.ctx_lens = ctx_p
    a.num_requests = ctx_arr.size
    if mode == abi.SOFTMAX:
        kp, kcode, karr = ptr(k_pool)
        st = [s // karr.itemsize for s in karr.strides]
        a.k_page_stride, a.k_head_stride, a.k_tok_stride = st[0], st[1], st[2]
        a.k_pool = kp
        qp, a.q_dtype, qarr = ptr(q)
        a.q = qp
        a.num_q_heads = qarr.shape[1]
        rows = a.num_q_heads
    else:
        wp, _, _ = ptr(lin_w, np.float32)
        a.lin_w = wp
        a.lin_w_period = lin_w_period
        a.num_q_heads = hkv
        rows = hkv
    bp, _, barr = ptr(block_table, np.int32)
    a.block_table = bp
    if page_indptr is not None:
        a.page_indptr = ptr(page_indptr, np.int32)[0]
    else:
        a.bt_stride = barr.shape[1]
    a.k_scale = ptr(k_scale, np.float32)[0]
    a.v_scale = ptr(v_scale, np.float32)[0]
    a.sm_scale = 0.0 if sm_scale is None else float(sm_scale)
    a.tau_scope = tau_scope
    a.max_tasks = max_tasks
    if ctx_in_pages:
        a.flags |= abi.FLAG_CTX_IN_PAGES
    cp = None
    if ctrl is not None:
        c = np.frombuffer(bytes(ctrl), dtype=np.uint8).copy()
        keep.append(c)
        cp = ctypes.c_void_p(c.ctypes.data)
    shape = (a.num_requests, rows, d)
    if precision == F64:
        out = np.full(shape, np.nan, dtype=np.float64)
        rc = lib.oracle_decode(ctypes.byref(a), cp, ctypes.c_void_p(out.ctypes.data), None,
                               F64, threads)
    else:
        out = np.full(shape, np.nan, dtype=np.float32)
        rc = lib.oracle_decode(ctypes.byref(a), cp, None, ctypes.c_void_p(out.ctypes.data),
                               F32, threads)
    if rc != 0:
        raise ValueError("oracle_decode rejected the arguments")
    return out


# --- dequantisation tables (pinned against torch in the tests) --------------

def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def fp8_e4m3_table() -> np.ndarray:
    lib = load()
    return np.array([lib.oracle_fp8_e4m3_to_float(i) for i in range(256)], dtype=np.float32)


def _dequant(x):
    a, code = _host(x)
    if code == abi.BF16:
        return bf16_to_float(a).astype(np.float64)
    if code == abi.F16:
        return a.view(np.float16).astype(np.float64)
    if code == abi.FP8_E4M3:
        return fp8_e4m3_table()[a].astype(np.float64)
    return a.astype(np.float64)


def numpy_decode(q, k_pool, v_pool, block_table, ctx_lens, *, mode=abi.SOFTMAX,
                 sm_scale=None, k_scale=None, v_scale=None, tau=None,
                 tau_scope=abi.TAU_PREFIX, lin_w=None, lin_w_period=0):
    """Closed-form truncated attention in float64 numpy, for small inputs.
    Layout: k_pool [P, Hkv, ps, d], v_pool [P, Hkv, d, ps] (d-major).
    tau: per-task budgets (len R*Hkv, 0 = none) or None."""
    K = _dequant(k_pool) if mode == abi.SOFTMAX else None
    V = _dequant(v_pool)
    P_, hkv, d, ps = V.shape
    bt = np.asarray(_host(block_table)[0])
    ctx = np.asarray(_host(ctx_lens)[0]).astype(np.int64)
    R = ctx.size
    ks = None if k_scale is None else np.asarray(_host(k_scale)[0], np.float64).reshape(P_, hkv)
    vs = None if v_scale is None else np.asarray(_host(v_scale)[0], np.float64).reshape(P_, hkv)
    if mode == abi.SOFTMAX:
        Q = _dequant(q)
        hq = Q.shape[1]
        G = hq // hkv
        out = np.zeros((R, hq, d))
        scale = 1.0 / np.sqrt(d) if sm_scale is None else float(sm_scale)
    else:
        w = np.asarray(_host(lin_w)[0], np.float64)
        out = np.zeros((R, hkv, d))
    for r in range(R):
        n = int(ctx[r])
        pos = np.arange(n)
        pages = bt[r, pos // ps]
        i = pos % ps
        for h in range(hkv):
            b = 0 if tau is None else int(tau[r * hkv + h])
            ctr = pos if tau_scope == abi.TAU_PREFIX else i
            kept = np.ones(n, bool) if b == 0 else ctr < b
            Vt = V[pages, h, :, i]                      # [n, d]
            if vs is not None:
                Vt = Vt * vs[pages, h][:, None]
            if mode == abi.LINEAR:
                wt = w[pos % lin_w_period] if lin_w_period else w[pos]
                out[r, h] = (wt[kept, None] * Vt[kept]).sum(0)
                continue
            Kt = K[pages, h, i, :]                      # [n, d]
            if ks is not None:
                Kt = Kt * ks[pages, h][:, None]
            for g in range(G):
                s = scale * (Kt[kept] @ Q[r, h * G + g])
                if s.size == 0:
                    out[r, h * G + g] = np.nan
                    continue
                e = np.exp(s - s.max())
                out[r, h * G + g] = (e[:, None] * Vt[kept]).sum(0) / e.sum()
    return out


def fp8_e4m3_encode(x) -> np.ndarray:
    """The oracle's e4m3fn encoder (RNE, saturating at 448) over an array."""
    lib = load()
    x = np.asarray(x, np.float32).ravel()
    return np.array([lib.oracle_fp8_e4m3_from_float(float(v)) for v in x], np.uint8)


def f16_encode(x) -> np.ndarray:
    """The oracle's binary16 encoder (RNE) over an array, as raw bits."""
    lib = load()
    x = np.asarray(x, np.float32).ravel()
    return np.array([lib.oracle_float_to_f16(float(v)) for v in x], np.uint16)


def pow2_scale(a: float) -> float:
    return load().oracle_pow2_scale(float(a))


def kv_append(k_src, v_src, append_indptr, ctx_lens, k_pool, v_pool, block_table, *,
              page_indptr=None, v_layout="dmajor", k_scale=None, v_scale=None,
              num_tokens=None):
    """Restated sched_kv_append on host copies. Pools: k [P, Hkv, ps, d];
    v [P, Hkv, d, ps] (dmajor) or [P, Hkv, ps, d] (tokmajor); sources
    [T, Hkv, d]. Returns (k_pool, v_pool, k_scale, v_scale, errors) as numpy
    arrays of the pools' raw element bits (uint16 for bf16/fp16, uint8 for fp8)
    and float32 scales (None without scales)."""
    lib = load()
    ks, src_code = _host(k_src)
    vs, _ = _host(v_src)
    kp, kv_code = _host(k_pool)
    vp, _ = _host(v_pool)
    kp, vp = kp.copy(), vp.copy()
    app, _ = _host(append_indptr, np.int32)
    ctx, _ = _host(ctx_lens, np.int32)
    bt, _ = _host(block_table, np.int32)
    pi, _ = _host(page_indptr, np.int32)
    ksc = None if k_scale is None else _host(k_scale, np.float32)[0].copy()
    vsc = None if v_scale is None else _host(v_scale, np.float32)[0].copy()
    a = abi.default_kv_args()
    a.src_dtype, a.kv_dtype = src_code, kv_code
    P, hkv, ps, d = kp.shape
    a.num_requests = ctx.size
    a.num_kv_heads, a.head_dim, a.page_size = hkv, d, ps
    a.num_tokens = ks.shape[0] if num_tokens is None else num_tokens
    a.num_pages = P
    a.src_tok_stride, a.src_head_stride = hkv * d, d
    a.k_page_stride, a.k_head_stride, a.k_tok_stride = hkv * ps * d, ps * d, d
    a.v_page_stride, a.v_head_stride = hkv * ps * d, ps * d
    if v_layout == "dmajor":
        a.v_tok_stride, a.v_dim_stride = 1, ps
    else:
        a.v_tok_stride, a.v_dim_stride = d, 1
    a.bt_stride = bt.shape[1] if bt.ndim == 2 else 0
    vp_ = lambda x: None if x is None else ctypes.c_void_p(x.ctypes.data)  # noqa: E731
    a.k_src, a.v_src = vp_(ks), vp_(vs)
    a.append_indptr, a.ctx_lens, a.block_table = vp_(app), vp_(ctx), vp_(bt)
    a.page_indptr = vp_(pi)
    a.k_pool, a.v_pool = vp_(kp), vp_(vp)
    a.k_scale, a.v_scale = vp_(ksc), vp_(vsc)
    errors = lib.oracle_kv_append(ctypes.byref(a))
    return kp, vp, ksc, vsc, int(errors)
