"""ctypes binding of libtpr_attn.so (the C ABI declared in include/tpr_attn.h).

The library is built in-tree by ``bridge_amd._build``; loading fails loudly when
it is missing -- there is no CPU or eager fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libtpr_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 6

TPR_OK = 0
TPR_ERR_INVALID_ARGUMENT = 1
TPR_ERR_UNSUPPORTED = 2
TPR_ERR_BUFFER_TOO_SMALL = 3
TPR_ERR_LAUNCH = 4

TPR_DTYPE_BF16 = 0
TPR_DTYPE_FP32 = 1

TPR_PLAN_RECOMPUTE_DQ = 1
TPR_PLAN_MASKED = 2                       # plan for calls with a physical key mask (SIMT kernels)
TPR_DS_STORE_DEFAULT = -1                 # TprTreeDesc.ds_store_max_bytes: the library's default budget
TPR_DS_STORE_DEFAULT_BYTES = 8 << 30      # ... which is 8 GiB

EXPORTED_SYMBOLS = (
    "tpr_attn_abi_version",
    "tpr_attn_last_error",
    "tpr_attn_plan",
    "tpr_attn_bwd_workspace_bytes",
    "tpr_attn_fwd",
    "tpr_attn_bwd",
    "tpr_attn_bwd_phases",
    "tpr_attn_bwd_noalloc",
    "tpr_attn_bwd_noalloc_max_workspace_bytes",
)

TPR_BWD_DELTA = 1
TPR_BWD_DKDV = 2
TPR_BWD_DQ = 4
TPR_BWD_DKDV_TILES = 8
TPR_BWD_DKDV_REDUCE = 16
TPR_BWD_ACCUMULATE_PREFIX_F32 = 1  # TprBwdParams.flags: add prefix grads into fp32 buffers

_p = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)


class TprTreeDesc(ctypes.Structure):
    _fields_ = [
        ("num_leaves", ctypes.c_int32),
        ("num_nodes", ctypes.c_int32),
        ("max_depth", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("cu_seqlens_q", _p),
        ("node_offsets", _p),
        ("leaf_ancestors", _p),
        ("ds_store_max_bytes", ctypes.c_int64),
    ]


class TprFwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("reserved_f", ctypes.c_float),
        ("plan_host", _p),
        ("plan_device", _p),
        ("q", _p),
        ("k", _p),
        ("v", _p),
        ("prefix_k", _p),
        ("prefix_v", _p),
        ("out", _p),
        ("lse", _p),
        ("q_row_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("mask", _p),
        ("mask_row_stride", ctypes.c_int64),
    ]


class TprBwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("reserved_f", ctypes.c_float),
        ("plan_host", _p),
        ("plan_device", _p),
        ("q", _p),
        ("k", _p),
        ("v", _p),
        ("prefix_k", _p),
        ("prefix_v", _p),
        ("out", _p),
        ("dout", _p),
        ("lse", _p),
        ("delta", _p),
        ("dq", _p),
        ("dk", _p),
        ("dv", _p),
        ("dprefix_k", _p),
        ("dprefix_v", _p),
        ("workspace", _p),
        ("workspace_bytes", ctypes.c_size_t),
        ("q_row_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("mask", _p),
        ("mask_row_stride", ctypes.c_int64),
    ]


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return os.environ.get("TPR_ATTN_LIB", LIB_PATH)


def load():
    """Load and type the shared library (once). Raises RuntimeError if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{LIB_NAME} is not built at {path}; build it with `python -m bridge_amd._build` "
                "(bridge_amd has no fallback path)")
        lib = ctypes.CDLL(path)
        lib.tpr_attn_abi_version.restype = ctypes.c_int
        lib.tpr_attn_abi_version.argtypes = []
        lib.tpr_attn_last_error.restype = ctypes.c_char_p
        lib.tpr_attn_last_error.argtypes = []
        lib.tpr_attn_plan.restype = ctypes.c_int
        lib.tpr_attn_plan.argtypes = [ctypes.POINTER(TprTreeDesc), _p, ctypes.c_int64,
                                      ctypes.POINTER(ctypes.c_int64)]
        lib.tpr_attn_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.tpr_attn_bwd_workspace_bytes.argtypes = [_p]
        lib.tpr_attn_fwd.restype = ctypes.c_int
        lib.tpr_attn_fwd.argtypes = [ctypes.POINTER(TprFwdParams), _p]
        lib.tpr_attn_bwd.restype = ctypes.c_int
        lib.tpr_attn_bwd.argtypes = [ctypes.POINTER(TprBwdParams), _p]
        lib.tpr_attn_bwd_phases.restype = ctypes.c_int
        lib.tpr_attn_bwd_phases.argtypes = [ctypes.POINTER(TprBwdParams), ctypes.c_int, _p]
        lib.tpr_attn_bwd_noalloc.restype = ctypes.c_int
        lib.tpr_attn_bwd_noalloc.argtypes = [ctypes.POINTER(TprBwdParams), _p]
        lib.tpr_attn_bwd_noalloc_max_workspace_bytes.restype = ctypes.c_size_t
        lib.tpr_attn_bwd_noalloc_max_workspace_bytes.argtypes = []
        version = lib.tpr_attn_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raise the Python exception matching a TprStatus."""
    if status == TPR_OK:
        return
    message = load().tpr_attn_last_error().decode("utf-8", "replace")
    text = f"{what}: {message}" if message else f"{what} failed with status {status}"
    if status in (TPR_ERR_INVALID_ARGUMENT, TPR_ERR_BUFFER_TOO_SMALL):
        raise ValueError(text)
    if status == TPR_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)
