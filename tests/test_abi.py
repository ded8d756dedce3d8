"""The C ABI library without a GPU: it loads, exports every symbol include/*.h declares,
and rejects bad arguments with status codes before touching the device."""
import ctypes
import glob
import os
import re

import pytest

import tileinfer_hip as ti
from tileinfer_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(ti_\w+)\s*\(", text))
    return names


def test_exports_every_declared_symbol():
    L = ti.load_library()
    names = declared_symbols()
    assert names, "no declarations found"
    assert names == set(_lib.EXPORTS)
    for n in names:
        assert hasattr(L, n), n


def test_version_and_status_strings():
    L = ti.load_library()
    assert L.ti_version().decode().startswith("tileinfer_hip")
    assert L.ti_status_string(0) == b"ok"
    assert L.ti_status_string(3).startswith(b"workspace")
    assert L.ti_status_string(99) == b"unknown status"


def _cache(**kw):
    c = _lib.KVCache()
    c.kind, c.head_dim, c.page_size, c.kv_heads, c.num_pages = 0, 128, 16, 8, 100
    c.k_pages = c.v_pages = 0x1000
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _args(**kw):
    a = _lib.AttentionArgs()
    a.dtype, a.q_heads, a.num_seqs, a.max_query_len, a.total_tokens = 1, 32, 4, 1, 4
    a.block_table_stride = 64
    a.q = a.out = a.positions = a.block_tables = 0x1000
    a.scale, a.causal, a.path = 0.088, 1, 0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def ws(a, c):
    size = ctypes.c_size_t(7)
    st = ti.load_library().ti_attention_workspace_bytes(ctypes.byref(a), ctypes.byref(c), ctypes.byref(size))
    return st, size.value


def test_workspace_bytes_decode_and_prefill():
    st, n = ws(_args(), _cache())
    # 4 seqs x 8 KV heads -> 8 splits (256 work-groups), 4 packed rows, (D + 2) floats,
    # shared out by length (flat mode): a {first work-group, pieces} pair per sequence
    assert st == 0 and n == 4 * 8 * 8 * 4 * 130 * 4 + 4 * 2 * 4
    # one sequence: its splits are fixed, no table
    assert ws(_args(num_seqs=1, total_tokens=1), _cache()) == (0, 1 * 8 * 16 * 4 * 130 * 4)
    # 32 seqs x 8 KV heads: one split per (sequence, KV head) writes the output directly
    assert ws(_args(num_seqs=32, total_tokens=32), _cache()) == (0, 0)
    st, n = ws(_args(max_query_len=512, total_tokens=2048), _cache())
    assert st == 0 and n == 0                   # prefill needs none
    # fp32 (matrix-core decode): 4 seqs x 8 KV heads = 32 pairs -> 16 key splits (512
    # work-groups), 4 packed rows each
    st, n = ws(_args(dtype=0), _cache())
    assert st == 0 and n == 4 * 8 * 16 * 4 * 130 * 4
    # 32 seqs: 256 pairs -> 2 splits
    assert ws(_args(dtype=0, num_seqs=32, total_tokens=32), _cache()) == (0, 32 * 8 * 2 * 4 * 130 * 4)
    # fp32 with 8-token pages runs the VALU kernel: 1024 query waves need no splits
    assert ws(_args(dtype=0, num_seqs=32, total_tokens=32), _cache(page_size=8)) == (0, 0)
    # fp32 multi-token steps: 16-row q-tiles are work-groups too. One sequence of 4 tokens at
    # G = 4 is one q-tile (8 items -> 32 splits); a 512-token prefill (128 q-tiles per KV
    # head) and the verify shape (16 seqs x 4 q-tiles) fill 512 work-groups unsplit.
    assert ws(_args(dtype=0, num_seqs=1, max_query_len=4, total_tokens=4), _cache()) == (0, 8 * 32 * 16 * 130 * 4)
    assert ws(_args(dtype=0, num_seqs=1, max_query_len=512, total_tokens=512), _cache()) == (0, 0)
    assert ws(_args(dtype=0, num_seqs=16, max_query_len=16, total_tokens=256), _cache()) == (0, 0)
    # two 16-token sequences at G = 4: 2 x 8 x 4 = 64 items -> 8 splits of 64 rows each
    assert ws(_args(dtype=0, num_seqs=2, max_query_len=16, total_tokens=32), _cache()) == (0, 2 * 8 * 8 * 64 * 130 * 4)
    # independent of context length / pool size: same for a larger pool
    assert ws(_args(), _cache(num_pages=100000))[1] == ws(_args(), _cache())[1]


@pytest.mark.parametrize("bad", [
    dict(a=dict(q_heads=30)), dict(a=dict(num_seqs=0)), dict(a=dict(q=0)),
    dict(a=dict(total_tokens=5)), dict(a=dict(causal=2)), dict(a=dict(dtype=7)),
    dict(a=dict(path=9)), dict(c=dict(k_pages=0)), dict(c=dict(kind=5)), dict(c=dict(page_size=0)),
])
def test_invalid_arguments(bad):
    a, c = _args(**bad.get("a", {})), _cache(**bad.get("c", {}))
    L = ti.load_library()
    assert L.ti_attention(ctypes.byref(a), ctypes.byref(c), None) == _lib.TI_ERR_INVALID_ARG
    assert ws(a, c)[0] == _lib.TI_ERR_INVALID_ARG


def test_scale_must_be_finite_and_positive():
    L = ti.load_library()
    for bad in (0.0, -0.088, float("nan"), float("inf")):
        a = _args(scale=bad)
        assert L.ti_attention(ctypes.byref(a), ctypes.byref(_cache()), None) == _lib.TI_ERR_INVALID_ARG
        assert ws(a, _cache())[0] == _lib.TI_ERR_INVALID_ARG


def test_unsupported_shapes_and_workspace():
    L = ti.load_library()
    c = _cache(head_dim=96)
    assert L.ti_attention(ctypes.byref(_args()), ctypes.byref(c), None) == _lib.TI_ERR_UNSUPPORTED
    # forcing the decode kernel past its 64 packed rows
    a = _args(max_query_len=32, total_tokens=128, path=_lib.TI_PATH_DECODE)
    assert L.ti_attention(ctypes.byref(a), ctypes.byref(_cache()), None) == _lib.TI_ERR_UNSUPPORTED
    # decode without (enough) workspace fails before any launch
    assert L.ti_attention(ctypes.byref(_args()), ctypes.byref(_cache()), None) == _lib.TI_ERR_WORKSPACE
    a = _args(workspace=0x1000, workspace_bytes=10)
    assert L.ti_attention(ctypes.byref(a), ctypes.byref(_cache()), None) == _lib.TI_ERR_WORKSPACE
    # sequences and prefill q-tiles live in grid dimensions of at most 65535
    a = _args(num_seqs=70000, total_tokens=70000)
    assert L.ti_attention(ctypes.byref(a), ctypes.byref(_cache()), None) == _lib.TI_ERR_UNSUPPORTED
    assert ws(a, _cache())[0] == _lib.TI_ERR_UNSUPPORTED
    # G = 64 packs two queries per four-wave q-tile: 140000 tokens are 70000 tiles; the
    # 8-wave kernel packs four (35000 tiles, supported), so 300000 tokens exceed both
    c = _cache(kv_heads=1)
    a = _args(q_heads=64, num_seqs=1, max_query_len=300000, total_tokens=300000)
    assert ws(a, c)[0] == _lib.TI_ERR_UNSUPPORTED
    assert L.ti_attention(ctypes.byref(a), ctypes.byref(c), None) == _lib.TI_ERR_UNSUPPORTED
    a = _args(q_heads=64, num_seqs=1, max_query_len=140000, total_tokens=140000)
    assert ws(a, c)[0] == _lib.TI_OK
    # the four-wave kernel pinned: 70000 q-tiles exceed the grid
    for path in (_lib.TI_PATH_PREFILL_STAGED, _lib.TI_PATH_PREFILL_DIRECT):
        a = _args(q_heads=64, num_seqs=1, max_query_len=140000, total_tokens=140000, path=path)
        assert ws(a, c)[0] == _lib.TI_ERR_UNSUPPORTED
        assert L.ti_attention(ctypes.byref(a), ctypes.byref(c), None) == _lib.TI_ERR_UNSUPPORTED
    a = _args(q_heads=64, num_seqs=1, max_query_len=140000, total_tokens=140000,
              path=_lib.TI_PATH_PREFILL_PINGPONG)
    assert ws(a, c)[0] == _lib.TI_OK


def test_paired_prefill_grid_counts_pairs():
    """A paired prefill holds two q-tiles per work-group: its grid y is (q-tiles + 1) / 2,
    so a pinned 16-row paired step of 65536-131070 q-tiles (G = 32: one position per
    q-tile) fits the grid, and one of 131072 does not."""
    L = ti.load_library()
    c = _cache(kv_heads=1, num_pages=10000)
    for n, want in ((100000, _lib.TI_OK), (131070, _lib.TI_OK), (131072, _lib.TI_ERR_UNSUPPORTED)):
        a = _args(q_heads=32, num_seqs=1, max_query_len=n, total_tokens=n, block_table_stride=8192,
                  path=_lib.TI_PATH_PREFILL_PAIRED16)
        assert ws(a, c)[0] == want, n
        if want != _lib.TI_OK:
            assert L.ti_attention(ctypes.byref(a), ctypes.byref(c), None) == want


def test_store_rope_inputs_validation():
    L = ti.load_library()
    c = _cache()
    assert L.ti_store_kv(1, ctypes.byref(c), None, None, None, 0, None) == 0   # n = 0: no-op
    assert L.ti_store_kv(1, ctypes.byref(c), None, None, None, 3, None) == _lib.TI_ERR_INVALID_ARG
    assert L.ti_store_kv(3, ctypes.byref(c), 1, 1, 1, 3, None) == _lib.TI_ERR_INVALID_ARG
    assert L.ti_rope(1, 1, 1, 1, 1, 10, 1, 3, 4, 127, None) == _lib.TI_ERR_INVALID_ARG   # odd D
    assert L.ti_rope(1, None, 1, 1, 1, 10, 1, 3, 4, 128, None) == _lib.TI_ERR_INVALID_ARG
    assert L.ti_attention_inputs(1, 1, ctypes.byref(c), 1, 1, None, 1, 10, 1, 1, 2, 16, 1e-6,
                                 None) == _lib.TI_ERR_INVALID_ARG                        # q_norm without k_norm
    c8 = _cache(kind=1, layer_q=0, layer_scale=0x10, smooth=0x10)
    assert L.ti_store_kv(1, ctypes.byref(c8), 1, 1, 1, 3, None) == _lib.TI_ERR_INVALID_ARG


def test_python_layer_rejects_host_tensors():
    import torch
    q = torch.zeros((1, 4, 64), dtype=torch.bfloat16)
    with pytest.raises(ti.ArgumentError):
        ti.attention_(ti.HipBackend(), q, None, q, torch.zeros((2, 2, 4, 64), dtype=torch.bfloat16),
                      torch.zeros((2, 2, 4, 64), dtype=torch.bfloat16), torch.zeros(4, dtype=torch.int32),
                      torch.zeros(1, dtype=torch.int32), 0.1)


def test_noalloc_validates_before_any_hip_call():
    """ti_attention_noalloc checks arguments and its scratch limit on the host first, so
    these return without a GPU: invalid arguments as ti_attention, and shapes whose
    workspace exceeds TI_NOALLOC_SCRATCH_BYTES with TI_ERR_WORKSPACE."""
    L = ti.load_library()
    assert L.ti_attention_noalloc(ctypes.byref(_args(q_heads=30)), ctypes.byref(_cache()), None) == \
        _lib.TI_ERR_INVALID_ARG
    assert L.ti_attention_noalloc(None, ctypes.byref(_cache()), None) == _lib.TI_ERR_INVALID_ARG
    assert L.ti_attention_noalloc(ctypes.byref(_args()), ctypes.byref(_cache(head_dim=96)), None) == \
        _lib.TI_ERR_UNSUPPORTED
    # the ping-pong kernel pinned on a 512-token prefill of one KV head with G = 8: 16
    # work-groups, so 16 key splits of 4096 packed rows: 16 * 4096 * 130 * 4 B > 32 MiB
    c = _cache(kv_heads=1)
    a = _args(q_heads=8, num_seqs=1, max_query_len=512, total_tokens=512,
              path=_lib.TI_PATH_PREFILL_PINGPONG)
    st, need = ws(a, c)
    assert st == _lib.TI_OK and need > _lib.NOALLOC_SCRATCH_BYTES
    # (such a prefill runs unsplit through ti_attention_noalloc, as ti_attention does without
    # a workspace: tests/test_zz_no_alloc.py runs it on the GPU)
    # 256 tokens: half the rows, within the scratch (not launched here: no GPU)
    a = _args(q_heads=8, num_seqs=1, max_query_len=256, total_tokens=256,
              path=_lib.TI_PATH_PREFILL_PINGPONG)
    st, need = ws(a, c)
    assert st == _lib.TI_OK and 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
