"""ctypes mirror of include/sched_pd.h and include/sched_kv.h, and the
loader of libschedpd.so.

Pure ctypes: importing this module touches no GPU. The library is loaded from
next to this file (built in-tree by build_lib.py); a missing library is an
error, never a silent fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libschedpd.so")

# --- runtime contract (include/sched_pd.h; reference runtime/sched_rt.h) ----
SCHED_MAX_TASKS = 4096
RT_BIND_MAX_TASKS = 16384   # SCHED_RT_BIND_MAX_TASKS
CTRL_NUM_TASKS_OFF = 4
CTRL_LAMBDA_OFF = 8
CTRL_FLAGS_OFF = 24
CTRL_ORDER_SIZE_OFF = 28
CTRL_ROWS_OFF = 32
ROW_SIZE = 8
ROW_Q_OFF = 0
ROW_TAU_OFF = 4
ROW_HINT_OFF = 6
FLAG_TIMER_OFF = 1
HINT_AUTO, HINT_URGENT, HINT_POLITE = 0, 1, 2

# --- decode launcher ---------------------------------------------------------
ABI_VERSION = 1
SOFTMAX, LINEAR = 0, 1
F32, BF16, FP8_E4M3, F16 = 0, 1, 2, 3
TAU_PREFIX, TAU_PER_PAGE = 0, 1
FLAG_RT_TABLES = 0x1
FLAG_WALLCLOCK = 0x2
FLAG_FORCE_VALU = 0x4
FLAG_CTX_IN_PAGES = 0x8
FLAG_SHED_LOADS = 0x10
FLAG_NO_WAVE = 0x20
FLAG_NO_MFMA = 0x40
TILES_PAIRS, TILES_RANGED = 0, 1

_u32, _f32, _i64, _p = ctypes.c_uint32, ctypes.c_float, ctypes.c_int64, ctypes.c_void_p


class SchedDecodeArgs(ctypes.Structure):
    """Field-for-field mirror of `SchedDecodeArgs` in include/sched_pd.h."""
    _fields_ = [
        ("abi_version", _u32), ("mode", _u32), ("kv_dtype", _u32),
        ("q_dtype", _u32), ("o_dtype", _u32), ("num_requests", _u32),
        ("num_q_heads", _u32), ("num_kv_heads", _u32), ("head_dim", _u32),
        ("page_size", _u32), ("bt_stride", _u32), ("tau_scope", _u32),
        ("workers", _u32), ("pf_dist", _u32), ("flags", _u32),
        ("max_tasks", _u32),
        ("sm_scale", _f32), ("policy_dT", _f32), ("policy_dR", _f32),
        ("policy_H", _f32),
        ("lin_w_period", _u32), ("tile_pages", _u32),
        ("q", _p), ("out", _p), ("k_pool", _p), ("v_pool", _p),
        ("k_page_stride", _i64), ("k_head_stride", _i64), ("k_tok_stride", _i64),
        ("v_page_stride", _i64), ("v_head_stride", _i64), ("v_tok_stride", _i64),
        ("v_dim_stride", _i64),
        ("k_scale", _p), ("v_scale", _p),
        ("block_table", _p), ("page_indptr", _p), ("ctx_lens", _p),
        ("lin_w", _p),
        ("order", _p), ("ctrl", _p), ("timer", _p), ("queue", _p),
        ("tiles", _p), ("num_tiles", _u32), ("tile_format", _u32),
        ("workspace", _p), ("workspace_bytes", ctypes.c_uint64),
    ]


def default_args() -> SchedDecodeArgs:
    """Same defaults as sched_pd_default_args() in C."""
    a = SchedDecodeArgs()
    a.abi_version = ABI_VERSION
    a.kv_dtype = a.q_dtype = a.o_dtype = F32
    a.tau_scope = TAU_PREFIX
    a.max_tasks = SCHED_MAX_TASKS
    a.policy_dT = 1.0
    a.policy_dR = 1.0
    a.policy_H = 0.25
    return a


# --- KV-cache writer (include/sched_kv.h) --------------------------------------
KV_ABI_VERSION = 1


class SchedKvAppendArgs(ctypes.Structure):
    """Field-for-field mirror of `SchedKvAppendArgs` in include/sched_kv.h."""
    _fields_ = [
        ("abi_version", _u32), ("src_dtype", _u32), ("kv_dtype", _u32),
        ("num_requests", _u32), ("num_kv_heads", _u32), ("head_dim", _u32),
        ("page_size", _u32), ("bt_stride", _u32), ("max_append", _u32),
        ("num_tokens", _u32), ("num_pages", ctypes.c_uint64),
        ("k_src", _p), ("v_src", _p),
        ("src_tok_stride", _i64), ("src_head_stride", _i64),
        ("append_indptr", _p), ("ctx_lens", _p), ("block_table", _p),
        ("page_indptr", _p),
        ("k_pool", _p), ("v_pool", _p),
        ("k_page_stride", _i64), ("k_head_stride", _i64), ("k_tok_stride", _i64),
        ("v_page_stride", _i64), ("v_head_stride", _i64), ("v_tok_stride", _i64),
        ("v_dim_stride", _i64),
        ("k_scale", _p), ("v_scale", _p), ("errors", _p),
        ("heads_per_group", _u32), ("_pad0", _u32),
    ]


def default_kv_args() -> SchedKvAppendArgs:
    """Same defaults as sched_kv_default_args() in C."""
    a = SchedKvAppendArgs()
    a.abi_version = KV_ABI_VERSION
    a.src_dtype = a.kv_dtype = BF16
    return a


# Every function include/*.h declares: name -> (restype, argtypes).
_c_bool = ctypes.c_bool
SIGNATURES = {
    "sched_rt_init": (_c_bool, []),
    "sched_rt_disarm": (_c_bool, []),
    "sched_rt_set_order": (_c_bool, [ctypes.POINTER(ctypes.c_int32), ctypes.c_uint]),
    "sched_rt_set_lambda": (None, [_f32, _f32, _f32, _f32]),
    "sched_rt_set_task": (None, [ctypes.c_uint, _f32, ctypes.c_uint16, ctypes.c_uint8]),
    "sched_rt_set_tau": (None, [ctypes.c_uint, ctypes.c_uint16]),
    "sched_rt_set_num_tasks": (None, [_u32]),
    "sched_rt_set_order_size": (None, [_u32]),
    "sched_rt_set_timer_enabled": (None, [_c_bool]),
    "sched_rt_push_ctrl": (_c_bool, []),
    "sched_rt_queue_reset": (_c_bool, [_u32]),
    "sched_rt_timer": (ctypes.c_ulonglong, [ctypes.c_uint]),
    "sched_rt_timer_clear": (None, []),
    "sched_rt_slots": (_c_bool, [ctypes.POINTER(ctypes.c_uint64)]),
    "sched_rt_timer_read": (_c_bool, [ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_uint]),
    "sched_rt_set_timer_host_mirror": (_c_bool, [_c_bool]),
    "sched_rt_slot_addresses": (_c_bool, [ctypes.POINTER(ctypes.c_uint64)]),
    "sched_rt_timer_host_va": (ctypes.c_uint64, []),
    "sched_rt_bind_tables": (_c_bool, [_p, _p, _p, _p, _u32]),
    "sched_pd_default_args": (None, [ctypes.POINTER(SchedDecodeArgs)]),
    "sched_paged_decode": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs), _p]),
    "sched_paged_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs), _p]),
    "sched_paged_decode_occupancy": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs)]),
    "sched_paged_decode_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(SchedDecodeArgs)]),
    "sched_paged_decode_kernel_kind": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs)]),
    "sched_paged_decode_prefetch_range": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs),
                                                         ctypes.POINTER(_u32),
                                                         ctypes.POINTER(_u32)]),
    "sched_pd_cu_count": (ctypes.c_int, []),
    "sched_pd_copy_to_device": (ctypes.c_int, [_p, _p, ctypes.c_uint64, _p]),
    "sched_pd_staging_alloc": (_p, [ctypes.c_uint64]),
    "sched_pd_read_probe": (ctypes.c_int, [_p, ctypes.c_uint64, _p, _p]),
    "sched_pd_read_probe_blocks": (ctypes.c_int, [_p, ctypes.c_uint64, _p, _u32, _u32, _p, _p]),
    "sched_pd_last_error": (ctypes.c_char_p, []),
    "sched_kv_default_args": (None, [ctypes.POINTER(SchedKvAppendArgs)]),
    "sched_kv_append": (ctypes.c_int, [ctypes.POINTER(SchedKvAppendArgs), _p]),
    "sched_paged_decode_append": (ctypes.c_int, [ctypes.POINTER(SchedDecodeArgs),
                                                 ctypes.POINTER(SchedKvAppendArgs), _p]),
    "sched_kv_table_update": (ctypes.c_int, [_p, ctypes.c_int64, ctypes.c_int64, _p, _u32, _p]),
    "launch_paged_softmax": (None, [_p, _p, _p, _p, _p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, _p]),
    "paged_softmax_occupancy": (ctypes.c_int, []),
}

_LIB = None


class SchedLibraryError(RuntimeError):
    """libschedpd.so is missing, unloadable or lacks a declared symbol."""


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libschedpd.so once and bind every declared signature. Raises
    SchedLibraryError when the library is absent: there is no CPU fallback."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise SchedLibraryError(
            f"{path} not built: run `python sched-pass_amd/build_lib.py` "
            f"(or __graft_entry__.build()) first")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:
        raise SchedLibraryError(f"cannot load {path}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as e:
            raise SchedLibraryError(f"{path} does not export {name}") from e
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error() -> str:
    msg = load_library().sched_pd_last_error()
    return msg.decode() if msg else ""
