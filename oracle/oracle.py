"""ctypes front end of the CPU oracle (liboracle.so, built from ref_attention.c).

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker or the timed CPU baseline, never as the product.
The HIP library and the tileinfer_hip package never import it.

Every function restates a reference function (cited per function); arrays are numpy,
C-order, with bf16 values carried as float32 that are exactly representable in bf16.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP), every time (-B)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB) or os.path.getmtime(_LIB) < os.path.getmtime(
                os.path.join(_HERE, "ref_attention.c")):
            build()
        _lib = ctypes.CDLL(_LIB)
    return _lib


F = ctypes.POINTER(ctypes.c_float)
I32 = ctypes.POINTER(ctypes.c_int32)
I8 = ctypes.POINTER(ctypes.c_int8)


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(F)


def _i(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(I32)


def _b(a):
    assert a.dtype == np.int8 and a.flags.c_contiguous
    return a.ctypes.data_as(I8)


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    out[nan] = x[nan]
    return out


def rope(x, cos, sin, positions, bf16: bool):
    """rope(::RefBackend): src/ops/reference.jl:32-39. x [n][H][D], cos/sin [L][D]."""
    x = np.ascontiguousarray(x, np.float32)
    n, H, D = x.shape
    y = np.empty_like(x)
    lib().or_rope(int(bf16), _f(y), _f(x), _f(np.ascontiguousarray(cos, np.float32)),
                  _f(np.ascontiguousarray(sin, np.float32)),
                  _i(np.ascontiguousarray(positions, np.int32)), n, H, D)
    return y


def store_kv(k_pages, v_pages, k, v, slots):
    """store_kv!(::RefBackend) dense, in place: src/ops/reference.jl:64-74."""
    pages, H, P, D = k_pages.shape
    n = k.shape[0]
    lib().or_store_kv(_f(k_pages), _f(v_pages), _f(np.ascontiguousarray(k, np.float32)),
                      _f(np.ascontiguousarray(v, np.float32)),
                      _i(np.ascontiguousarray(slots, np.int32)), n, D, P, H)


def quantize_vector(x):
    """quantize_columns of one vector: src/ops/quant.jl:141-145 -> (int8[D], scale)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape[0], np.int8)
    s = ctypes.c_float()
    lib().or_quantize_vector(_f(x), x.shape[0], _b(q), ctypes.byref(s))
    return q, np.float32(s.value)


def store_kv_int8(layer_q, layer_scale, smooth, k, v, slots):
    """store_kv!(::RefBackend, ::Int8Pages, ...) in place: src/ops/quant.jl:147-159.
    layer_q [2][pages][H][P][D] int8, layer_scale [2][pages][H][P] f32."""
    _, pages, H, P, D = layer_q.shape
    n = k.shape[0]
    lib().or_store_kv_int8(_b(layer_q), _f(layer_scale), _f(np.ascontiguousarray(smooth, np.float32)),
                           _f(np.ascontiguousarray(k, np.float32)),
                           _f(np.ascontiguousarray(v, np.float32)),
                           _i(np.ascontiguousarray(slots, np.int32)), n, D, P, H, pages)


def attention_inputs(qkv, q_norm, k_norm, cos_sin, positions, slots, nq, nkv, eps, bf16,
                     k_pages=None, v_pages=None, layer_q=None, layer_scale=None, smooth=None):
    """attention_inputs! (src/ops/interface.jl:169-179; src/ops/tile/fused.jl:15-130).
    qkv [n][nq+2nkv][D]; cos_sin [L][2][D]. Writes the pools in place, returns q."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    n, _, D = qkv.shape
    q = np.zeros((n, nq, D), np.float32)
    int8 = layer_q is not None
    norm = q_norm is not None
    dummy = np.zeros(D, np.float32)
    if int8:
        _, pages, _, P, _ = layer_q.shape
        kp = vp = np.zeros(1, np.float32)
        lq, ls, sm = layer_q, layer_scale, np.ascontiguousarray(smooth, np.float32)
    else:
        pages, _, P, _ = k_pages.shape
        kp, vp = k_pages, v_pages
        lq, ls, sm = np.zeros(1, np.int8), np.zeros(1, np.float32), dummy
    lib().or_attention_inputs(
        int(bf16), _f(q), _f(kp), _f(vp), _b(lq), _f(ls), _f(sm), int(int8), _f(qkv),
        _f(np.ascontiguousarray(q_norm if norm else dummy, np.float32)),
        _f(np.ascontiguousarray(k_norm if norm else dummy, np.float32)), int(norm),
        _f(np.ascontiguousarray(cos_sin, np.float32)), _i(np.ascontiguousarray(positions, np.int32)),
        _i(np.ascontiguousarray(slots, np.int32)), n, nq, nkv, D, P, pages, ctypes.c_float(eps))
    return q


lib_set = False


def _setup():
    global lib_set
    if lib_set:
        return
    L = lib()
    L.or_attention.argtypes = [ctypes.c_int, ctypes.c_int, F, F, F, F, I8, F, F, ctypes.c_int,
                               ctypes.c_int, I32, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                               ctypes.c_int]
    L.or_bf16.restype = ctypes.c_float
    L.or_bf16.argtypes = [ctypes.c_float]
    lib_set = True


def attention(q, block_table, start, scale, causal=True, k_pages=None, v_pages=None,
              layer_q=None, layer_scale=None, smooth=None, exact=True, bf16=False):
    """attention(::RefBackend) of ONE sequence: src/ops/reference.jl:95-121.
    q [n][Hq][D]; pools [pages][Hk][P][D] or INT8 layer arrays (gather_pages dequantizes,
    src/ops/quant.jl:165-170). exact=True: double-accumulated, unrounded (the tolerance
    reference); exact=False: the eager op's rounding points in T (bf16 flag)."""
    _setup()
    q = np.ascontiguousarray(q, np.float32)
    n, Hq, D = q.shape
    out = np.empty_like(q)
    bt = np.ascontiguousarray(block_table, np.int32)
    int8 = layer_q is not None
    if int8:
        _, pages, Hk, P, _ = layer_q.shape
        kp = vp = np.zeros(1, np.float32)
        lq, ls, sm = layer_q, np.ascontiguousarray(layer_scale, np.float32), np.ascontiguousarray(smooth, np.float32)
    else:
        pages, Hk, P, _ = k_pages.shape
        kp, vp = np.ascontiguousarray(k_pages, np.float32), np.ascontiguousarray(v_pages, np.float32)
        lq, ls, sm = np.zeros(1, np.int8), np.zeros(1, np.float32), np.zeros(1, np.float32)
    lib().or_attention(0 if exact else 1, int(bf16), _f(out), _f(q), _f(kp), _f(vp), _b(lq), _f(ls),
                       _f(sm), int(int8), pages, _i(bt), int(start), n, Hq, Hk, D, P,
                       float(scale), int(causal))
    return out


_cpu_lib = None


def cpu_lib():
    """The CPU baseline (cpu_baseline.c), compiled for THIS host (-O3 -march=native
    -ffast-math, OpenMP) into a private temporary directory on first use: the library
    built for one machine's instruction set is never carried to another."""
    global _cpu_lib
    if _cpu_lib is None:
        import tempfile
        out = os.path.join(tempfile.mkdtemp(prefix="ti_cpu_baseline_"), "liboracle_cpu.so")
        subprocess.run(["make", "-s", "-C", _HERE, f"CPU_LIB={out}", "cpu"], check=True)
        L = ctypes.CDLL(out)
        L.cb_attention_f32_batch.argtypes = [F, F, F, F, I32, ctypes.c_int, I32, I32, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_float, ctypes.c_int, ctypes.c_int]
        _cpu_lib = L
    return _cpu_lib


def attention_f32_batch(q, k_pages, v_pages, block_tables, starts, counts, scale, causal=True,
                        threads=None):
    """CPU baseline: the eager op in Float32 over a batch (cpu_baseline.c), OpenMP over
    (sequence, KV head). Timed by bench.py; not a checker."""
    q = np.ascontiguousarray(q, np.float32)
    T, Hq, D = q.shape
    pages, Hk, P, _ = k_pages.shape
    out = np.empty_like(q)
    bts = np.ascontiguousarray(block_tables, np.int32)
    threads = threads or os.cpu_count() or 1
    cpu_lib().cb_attention_f32_batch(_f(out), _f(q), _f(np.ascontiguousarray(k_pages, np.float32)),
                                     _f(np.ascontiguousarray(v_pages, np.float32)), _i(bts), bts.shape[1],
                                     _i(np.ascontiguousarray(starts, np.int32)),
                                     _i(np.ascontiguousarray(counts, np.int32)), len(starts), Hq, Hk,
                                     D, P, float(scale), int(causal), int(threads))
    return out
