"""HipBackend: the reference's op interface (src/ops/interface.jl) on the gfx950 kernels.

Each function mirrors one method of the reference for its TileBackend (same name with `!`
spelled as a trailing `_`, same argument order and meaning) and calls one entry point of
libtileinfer_hip.so through ctypes. torch tensors only carry device memory and the
current stream; all compute is in the HIP library, and there is no fallback: if the
library is missing, the first call raises.

Shapes are C order (the reference's column-major shapes reversed):
q, out [n][heads][D]; k, v [n][kv_heads][D]; dense pools [pages][kv_heads][P][D];
qkv [n][(heads + 2 kv_heads) D]; block_table int32 [>= pages of the sequence], 1-based,
zero-padded; positions int32 [n], 0-based; slots int32 [n], 1-based.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from ._lib import ArgumentError, AttentionArgs, KVCache, check
from .kv import Int8Pages, layer_arrays
from .rope import RotaryTable


class HipBackend:
    """Selects the MI355X kernels, as TileBackend selects the cuTile ones
    (src/ops/interface.jl:15-21)."""

    def __repr__(self) -> str:
        return "HipBackend()"


_OPS = {"attention", "attention!", "store_kv!", "rmsnorm", "rmsnorm!", "rope", "rope!", "attention_inputs!"}


def supports_graphs(be: HipBackend) -> bool:
    """In-place ops neither allocate nor synchronize (src/ops/interface.jl:282-288)."""
    return True


def has_kernel(be: HipBackend, op) -> bool:
    """Whether the backend implements op itself (src/ops/interface.jl:290-295)."""
    name = op if isinstance(op, str) else getattr(op, "__name__", "")
    return name.rstrip("_") in {o.rstrip("!") for o in _OPS} or name in _OPS


def _dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.TI_BF16
    if t.dtype == torch.float32:
        return _lib.TI_F32
    raise ArgumentError(f"unsupported element type {t.dtype} (bfloat16 or float32)")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dev(*ts):
    for t in ts:
        if t is not None:
            if not t.is_cuda:
                raise ArgumentError("tensors must be on the GPU")
            if not t.is_contiguous():
                raise ArgumentError("tensors must be contiguous")


def _i32(t: torch.Tensor, name: str):
    if t.dtype != torch.int32:
        raise ArgumentError(f"{name} must be int32")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def kv_cache_struct(k_pages, v_pages, dtype: Optional[torch.dtype] = None) -> KVCache:
    """The ti_kv_cache of a layer: dense pools [pages][H][P][D] or an Int8Pages pair."""
    c = KVCache()
    if isinstance(k_pages, Int8Pages) or isinstance(v_pages, Int8Pages):
        lq, ls, sm = layer_arrays(k_pages, v_pages)
        _dev(lq, ls, sm)
        _, pages, H, P, D = lq.shape
        c.kind, c.layer_q, c.layer_scale, c.smooth = _lib.TI_KV_INT8, lq.data_ptr(), ls.data_ptr(), sm.data_ptr()
    else:
        _dev(k_pages, v_pages)
        if k_pages.shape != v_pages.shape or k_pages.dim() != 4 or k_pages.dtype != v_pages.dtype:
            raise ArgumentError("k_pages and v_pages must be matching [pages][kv_heads][P][D] pools")
        if dtype is not None and k_pages.dtype != dtype:
            raise ArgumentError("pools must have the activations' element type")
        pages, H, P, D = k_pages.shape
        c.kind, c.k_pages, c.v_pages = _lib.TI_KV_DENSE, k_pages.data_ptr(), v_pages.data_ptr()
    c.head_dim, c.page_size, c.kv_heads, c.num_pages = D, P, H, pages
    return c


def _attention_args(out, q, block_tables, positions, scale, causal, path, num_seqs,
                    max_query_len, query_start_loc, workspace) -> AttentionArgs:
    a = AttentionArgs()
    a.dtype = _dtype(q)
    a.q_heads = q.shape[1]
    a.num_seqs = num_seqs
    a.max_query_len = max_query_len
    a.total_tokens = q.shape[0]
    a.block_table_stride = block_tables.shape[-1]
    a.q, a.out = _ptr(q), _ptr(out)
    a.positions = _ptr(positions)
    a.query_start_loc = _ptr(query_start_loc)
    a.block_tables = _ptr(block_tables)
    a.scale = float(scale)
    a.causal = int(bool(causal))
    a.path = int(path)
    a.workspace = _ptr(workspace)
    a.workspace_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return a


def workspace_bytes(q, k_pages, num_seqs: int = 1, max_query_len: Optional[int] = None,
                    path: int = _lib.TI_PATH_AUTO) -> int:
    """Bytes of split-KV scratch ti_attention needs for these query shapes (0 for none)."""
    # A shape-only query: the library validates and sizes, it never dereferences pointers.
    c = KVCache()
    if isinstance(k_pages, Int8Pages):
        pages, H, P, D = k_pages.q.shape
        c.kind, c.layer_q, c.layer_scale, c.smooth = _lib.TI_KV_INT8, 1, 1, 1
    else:
        pages, H, P, D = k_pages.shape
        c.kind, c.k_pages, c.v_pages = _lib.TI_KV_DENSE, 1, 1
    c.head_dim, c.page_size, c.kv_heads, c.num_pages = D, P, H, pages
    n = max_query_len if max_query_len is not None else q.shape[0] // num_seqs
    a = AttentionArgs()
    a.dtype, a.q_heads, a.num_seqs, a.max_query_len = _dtype(q), q.shape[1], num_seqs, n
    a.total_tokens, a.block_table_stride = num_seqs * n, 1
    a.q = a.out = a.positions = a.block_tables = 1
    a.scale, a.causal, a.path = 1.0, 1, int(path)
    size = ctypes.c_size_t(0)
    check(_lib.load().ti_attention_workspace_bytes(ctypes.byref(a), ctypes.byref(c), ctypes.byref(size)))
    return size.value


def attention_workspace(be: HipBackend, q, k_pages, num_seqs: int = 1,
                        max_query_len: Optional[int] = None, path: int = _lib.TI_PATH_AUTO):
    """Scratch for attention_ with queries shaped like q, or None
    (attention_workspace, src/ops/tile/attention.jl:351-352). A byte tensor."""
    n = workspace_bytes(q, k_pages, num_seqs, max_query_len, path)
    return None if n == 0 else torch.empty(n, dtype=torch.uint8, device=q.device)


def paged_attention_(be: HipBackend, out, workspace, q, k_pages, v_pages, block_tables,
                     positions, scale: float, causal: bool = True,
                     query_start_loc: Optional[torch.Tensor] = None,
                     max_query_len: Optional[int] = None, path: int = _lib.TI_PATH_AUTO):
    """Batched attention_: sequence b owns tokens [qsl[b], qsl[b+1]) of q (or equal
    shares when query_start_loc is None) and block table row block_tables[b]."""
    bts = block_tables if block_tables.dim() == 2 else block_tables.view(1, -1)
    B = bts.shape[0]
    _dev(out, q, bts, positions, query_start_loc, workspace)
    _i32(bts, "block_tables")
    _i32(positions, "positions")
    if q.dim() != 3 or out.shape != q.shape or out.dtype != q.dtype:
        raise ArgumentError("q and out must be matching [n][heads][D] tensors")
    if positions.numel() != q.shape[0]:
        raise ArgumentError("one position per query token")
    c = kv_cache_struct(k_pages, v_pages, None if isinstance(k_pages, Int8Pages) else q.dtype)
    if q.shape[2] != c.head_dim:
        raise ArgumentError("q's head_dim differs from the pools'")
    if query_start_loc is not None:
        _i32(query_start_loc, "query_start_loc")
        if max_query_len is None:
            raise ArgumentError("max_query_len is required with query_start_loc")
    n = max_query_len if max_query_len is not None else q.shape[0] // B
    a = _attention_args(out, q, bts, positions, scale, causal, path, B, n, query_start_loc,
                        workspace)
    check(_lib.load().ti_attention(ctypes.byref(a), ctypes.byref(c), _stream(q)))
    return out


def attention_(be: HipBackend, out, workspace, q, k_pages, v_pages, block_table, positions,
               scale: float, causal: bool = True, path: int = _lib.TI_PATH_AUTO):
    """attention!(::TileBackend, out, workspace, q, k_pages, v_pages, block_table,
    positions, scale; causal) (src/ops/tile/attention.jl:359-366) for one sequence."""
    return paged_attention_(be, out, workspace, q, k_pages, v_pages, block_table.view(1, -1),
                            positions, scale, causal, path=path)


def attention(be: HipBackend, q, k_pages, v_pages, block_table, positions, scale: float,
              causal: bool = True):
    """Allocating attention (src/ops/tile/attention.jl:368-371)."""
    out = torch.empty_like(q)
    return attention_(be, out, attention_workspace(be, q, k_pages), q, k_pages, v_pages,
                      block_table, positions, scale, causal)


def store_kv_(be: HipBackend, k_pages, v_pages, k, v, slots):
    """store_kv!(::TileBackend, k_pages, v_pages, k, v, slots)
    (src/ops/tile/elementwise.jl:133-140, :180-188)."""
    _dev(k, v, slots)
    _i32(slots, "slots")
    if k.shape != v.shape or k.dtype != v.dtype or k.dim() != 3:
        raise ArgumentError("k and v must be matching [n][kv_heads][D] tensors")
    c = kv_cache_struct(k_pages, v_pages, None if isinstance(k_pages, Int8Pages) else k.dtype)
    if k.shape[1] != c.kv_heads or k.shape[2] != c.head_dim or slots.numel() != k.shape[0]:
        raise ArgumentError("k/v/slots shapes do not match the pools")
    check(_lib.load().ti_store_kv(_dtype(k), ctypes.byref(c), _ptr(k), _ptr(v), _ptr(slots),
                                  k.shape[0], _stream(k)))


def rmsnorm_(be: HipBackend, y, x, w, eps: float):
    """rmsnorm!(::TileBackend, y, x, w, eps) (src/ops/tile/norm.jl:31-38): every row of the
    last dimension of x normalized as rnd(rnd(x inv_rms) w). y may be x."""
    _dev(y, x, w)
    if y.shape != x.shape or y.dtype != x.dtype or w.dtype != x.dtype or w.dim() != 1 \
            or w.shape[0] != x.shape[-1] or not (x.is_contiguous() and y.is_contiguous()):
        raise ArgumentError("rmsnorm shapes/types mismatch")
    H = x.shape[-1]
    check(_lib.load().ti_rmsnorm(_dtype(x), _ptr(y), _ptr(x), _ptr(w), x.numel() // H, H, float(eps),
                                 _stream(x)))
    return y


def rmsnorm(be: HipBackend, x, w, eps: float):
    return rmsnorm_(be, torch.empty_like(x), x, w, eps)


def rope_(be: HipBackend, y, x, cos, sin, positions):
    """rope!(::TileBackend, y, x, cos, sin, positions) (src/ops/tile/elementwise.jl:29-36).
    cos/sin: [max_len][D]."""
    _dev(y, x, cos, sin, positions)
    _i32(positions, "positions")
    if x.dim() != 3 or y.shape != x.shape or y.dtype != x.dtype or cos.dtype != x.dtype \
            or sin.dtype != x.dtype or cos.shape != sin.shape or cos.shape[1] != x.shape[2]:
        raise ArgumentError("rope shapes/types mismatch")
    n, H, D = x.shape
    if positions.numel() != n:
        raise ArgumentError("one position per token")
    check(_lib.load().ti_rope(_dtype(x), _ptr(y), _ptr(x), _ptr(cos), _ptr(sin), cos.shape[0],
                              _ptr(positions), n, H, D, _stream(x)))
    return y


def rope(be: HipBackend, x, cos, sin, positions):
    return rope_(be, torch.empty_like(x), x, cos, sin, positions)


def attention_inputs_(be: HipBackend, q, k_pages, v_pages, qkv, q_norm, k_norm,
                      table: RotaryTable, positions, slots, eps: float):
    """attention_inputs!(::TileBackend, q, k_pages, v_pages, qkv, q_norm, k_norm, table,
    positions, slots, eps) (src/ops/tile/fused.jl:94-130): optional q/k RMSNorm, RoPE,
    queries into q, keys and values into the cache; returns q."""
    _dev(q, qkv, q_norm, k_norm, table.cos_sin, positions, slots)
    _i32(positions, "positions")
    _i32(slots, "slots")
    n, nq, D = q.shape
    c = kv_cache_struct(k_pages, v_pages, None if isinstance(k_pages, Int8Pages) else q.dtype)
    if qkv.dtype != q.dtype or qkv.numel() != n * (nq + 2 * c.kv_heads) * D or D != c.head_dim:
        raise ArgumentError("qkv must be [n][(heads + 2 kv_heads) D] in q's element type")
    if table.cos_sin.dtype != q.dtype or table.cos_sin.shape[1:] != (2, D):
        raise ArgumentError("rotary table must be [max_len][2][D] in q's element type")
    if (q_norm is None) != (k_norm is None):
        raise ArgumentError("q_norm and k_norm go together")
    if positions.numel() != n or slots.numel() != n:
        raise ArgumentError("one position and one slot per token")
    check(_lib.load().ti_attention_inputs(
        _dtype(q), _ptr(q), ctypes.byref(c), _ptr(qkv), _ptr(q_norm), _ptr(k_norm),
        _ptr(table.cos_sin), table.cos_sin.shape[0], _ptr(positions), _ptr(slots), n, nq,
        float(eps), _stream(q)))
    return q
