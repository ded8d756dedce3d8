"""ctypes binding of libtileinfer_hip.so (the C ABI declared in include/tileinfer_hip.h).

The shared library is built in-tree by tileinfer.jl_amd/build.py. Loading it never touches
the GPU; every entry point validates its arguments on the host first, so the argument
checks work on a machine without a GPU.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtileinfer_hip.so")

TI_OK, TI_ERR_INVALID_ARG, TI_ERR_UNSUPPORTED, TI_ERR_WORKSPACE, TI_ERR_LAUNCH = range(5)
TI_F32, TI_BF16 = 0, 1
TI_KV_DENSE, TI_KV_INT8 = 0, 1
(TI_PATH_AUTO, TI_PATH_DECODE, TI_PATH_PREFILL, TI_PATH_PREFILL_STAGED, TI_PATH_PREFILL_DIRECT,
 TI_PATH_PREFILL_PINGPONG, TI_PATH_PREFILL_PAIRED, TI_PATH_PREFILL_PAIRED16) = range(8)

# Every symbol include/tileinfer_hip.h declares.
EXPORTS = ("ti_version", "ti_status_string", "ti_attention_workspace_bytes", "ti_attention",
           "ti_attention_noalloc", "ti_store_kv", "ti_rmsnorm", "ti_rope", "ti_attention_inputs")
NOALLOC_SCRATCH_BYTES = 32 << 20   # TI_NOALLOC_SCRATCH_BYTES


class KVCache(ctypes.Structure):
    """ti_kv_cache: one layer's dense pools or INT8 layer arrays (device pointers)."""
    _fields_ = [("kind", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("page_size", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
                ("num_pages", ctypes.c_int32), ("k_pages", ctypes.c_void_p),
                ("v_pages", ctypes.c_void_p), ("layer_q", ctypes.c_void_p),
                ("layer_scale", ctypes.c_void_p), ("smooth", ctypes.c_void_p)]


class AttentionArgs(ctypes.Structure):
    """ti_attention_args."""
    _fields_ = [("dtype", ctypes.c_int32), ("q_heads", ctypes.c_int32),
                ("num_seqs", ctypes.c_int32), ("max_query_len", ctypes.c_int32),
                ("total_tokens", ctypes.c_int32), ("block_table_stride", ctypes.c_int32),
                ("q", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("positions", ctypes.c_void_p), ("query_start_loc", ctypes.c_void_p),
                ("block_tables", ctypes.c_void_p), ("scale", ctypes.c_float),
                ("causal", ctypes.c_int32), ("path", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t)]


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python tileinfer.jl_amd/build.py`")
    L = ctypes.CDLL(path)
    vp, i32, P = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER
    L.ti_version.restype = ctypes.c_char_p
    L.ti_version.argtypes = []
    L.ti_status_string.restype = ctypes.c_char_p
    L.ti_status_string.argtypes = [i32]
    L.ti_attention_workspace_bytes.restype = i32
    L.ti_attention_workspace_bytes.argtypes = [P(AttentionArgs), P(KVCache), P(ctypes.c_size_t)]
    L.ti_attention.restype = i32
    L.ti_attention.argtypes = [P(AttentionArgs), P(KVCache), vp]
    L.ti_attention_noalloc.restype = i32
    L.ti_attention_noalloc.argtypes = [P(AttentionArgs), P(KVCache), vp]
    L.ti_store_kv.restype = i32
    L.ti_store_kv.argtypes = [i32, P(KVCache), vp, vp, vp, i32, vp]
    L.ti_rmsnorm.restype = i32
    L.ti_rmsnorm.argtypes = [i32, vp, vp, vp, i32, i32, ctypes.c_float, vp]
    L.ti_rope.restype = i32
    L.ti_rope.argtypes = [i32, vp, vp, vp, vp, i32, vp, i32, i32, i32, vp]
    L.ti_attention_inputs.restype = i32
    L.ti_attention_inputs.argtypes = [i32, vp, P(KVCache), vp, vp, vp, vp, i32, vp, vp, i32, i32,
                                      ctypes.c_float, vp]
    _lib = L
    return L


class TileInferError(RuntimeError):
    """A non-argument failure reported by the library (e.g. a failed launch)."""


class ArgumentError(ValueError):
    """Invalid arguments, as the reference's ArgumentError (e.g. src/ops/quant.jl:132-133)."""


class WorkspaceError(ArgumentError):
    """Workspace missing or smaller than ti_attention_workspace_bytes."""


def check(status: int) -> None:
    if status == TI_OK:
        return
    msg = load().ti_status_string(status).decode()
    if status == TI_ERR_WORKSPACE:
        raise WorkspaceError(msg)
    if status in (TI_ERR_INVALID_ARG, TI_ERR_UNSUPPORTED):
        raise ArgumentError(msg)
    raise TileInferError(msg)
