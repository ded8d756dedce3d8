"""KV pools larger than 2^31 elements (a Qwen3-4B layer pool of 139264 pages: 4.6 GB per
bf16 pool), with every used page above element 2^31, so any 32-bit page or slot
arithmetic in the write or attention kernels would land on the wrong rows.

The sequence's K and V are written through `store_kv_` at their slots (slot = (page - 1)
P + offset + 1, src/kv/block_manager.jl:58-100) and read back by decode, prefill (both
tile loaders) and the verify shape; the oracle runs on a compact copy of the used pages
with the same block-table order. Tolerances as the other attention tests: max abs <=
2e-2 (bf16, INT8-KV) against the double-accumulated oracle."""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import randn, rng, smoothing
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()

D, HQ, HK, P = 128, 32, 8, 16
PAGES = (1 << 31) // (HK * P * D) + 8192      # 139264 pages: 2.28e9 elements per pool
L = 2048                                     # cached + new positions of the sequence


def _setup(g):
    used = L // P
    hi0 = (1 << 31) // (HK * P * D) + 1      # first 1-based page id whose rows start past 2^31
    ids = (g.permutation(PAGES - hi0)[:used] + hi0 + 1).astype(np.int32)
    k = randn(g, L, HK, D, bf16=True)
    v = randn(g, L, HK, D, bf16=True)
    pos = np.arange(L)
    slots = ((ids[pos // P] - 1) * P + pos % P + 1).astype(np.int32)
    return ids, k, v, slots


def _check(q, start, n, ref_fn, kd, vd, bt, paths):
    scale = 1 / math.sqrt(D)
    ref = ref_fn(q, start, scale)
    qd = torch.from_numpy(q).bfloat16().cuda()
    pos = torch.arange(start, start + n, dtype=torch.int32, device="cuda")
    btd = torch.from_numpy(bt).cuda()
    for path in paths:
        ws = ti.attention_workspace(BE, qd, kd, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.attention_(BE, out, ws, qd, kd, vd, btd, pos, scale, True, path=path)
        err = float(np.max(np.abs(ref - out.float().cpu().numpy())))
        assert err <= 2e-2, f"start {start} n {n} path {path}: max abs err {err}"


# (start, n): decode, a 512-token prefill on a cached prefix, the verify shape
STEPS = [(L - 1, 1), (L - 512, 512), (L - 16, 16)]
PATHS = [ti.TI_PATH_AUTO, ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT, ti.TI_PATH_PREFILL_PAIRED,
         ti.TI_PATH_PREFILL_PAIRED16]


def test_bf16_pool_past_2_31_elements(gpu):
    g = rng(9100)
    ids, k, v, slots = _setup(g)
    print(f"pool {PAGES} pages, used ids {ids.min()}..{ids.max()}", flush=True)
    kd = torch.empty((PAGES, HK, P, D), dtype=torch.bfloat16, device="cuda")
    vd = torch.empty_like(kd)
    ti.store_kv_(BE, kd, vd, torch.from_numpy(k).bfloat16().cuda(), torch.from_numpy(v).bfloat16().cuda(),
                 torch.from_numpy(slots).cuda())
    # the written pages, copied out in block-table order, against the host data
    back = kd[torch.from_numpy(ids - 1).long().cuda()].float().cpu().numpy()
    assert np.array_equal(back.transpose(0, 2, 1, 3).reshape(L, HK, D), k)
    kp_c = k.reshape(-1, P, HK, D).transpose(0, 2, 1, 3)            # compact [page][Hk][P][D]
    vp_c = v.reshape(-1, P, HK, D).transpose(0, 2, 1, 3)
    bt_c = np.arange(1, L // P + 1, dtype=np.int32)
    for start, n in STEPS:
        q = randn(g, n, HQ, D, bf16=True)
        ref_fn = lambda qq, s, sc: orc.attention(qq, bt_c, s, sc, True, kp_c, vp_c)
        paths = PATHS if n > 1 else PATHS[:1] + [ti.TI_PATH_DECODE]
        _check(q, start, n, ref_fn, kd, vd, ids, paths)
    del kd, vd
    torch.cuda.empty_cache()


def test_int8_pool_past_2_31_elements(gpu):
    g = rng(9200)
    ids, k, v, slots = _setup(g)
    cs = smoothing(g, D)
    kq, vq = ti.int8_kv_pools(D, P, HK, PAGES, key_smoothing=torch.from_numpy(cs))
    ti.store_kv_(BE, kq, vq, torch.from_numpy(k).bfloat16().cuda(), torch.from_numpy(v).bfloat16().cuda(),
                 torch.from_numpy(slots).cuda())
    sel = torch.from_numpy(ids - 1).long().cuda()
    lq = kq.layer_q[:, sel].cpu().numpy()                          # [2][used][Hk][P][D]
    ls = kq.layer_scale[:, sel].cpu().numpy()                      # [2][used][Hk][P]
    # the oracle's INT8 store of the same tokens into a compact pool gives the same bytes
    lq_ref = np.zeros((2, L // P, HK, P, D), np.int8)
    ls_ref = np.zeros((2, L // P, HK, P), np.float32)
    orc.store_kv_int8(lq_ref, ls_ref, cs, k, v, np.arange(1, L + 1, dtype=np.int32))
    assert np.array_equal(lq, lq_ref) and np.array_equal(ls, ls_ref)
    bt_c = np.arange(1, L // P + 1, dtype=np.int32)
    for start, n in STEPS:
        q = randn(g, n, HQ, D, bf16=True)
        ref_fn = lambda qq, s, sc: orc.attention(qq, bt_c, s, sc, True, layer_q=lq, layer_scale=ls, smooth=cs)
        _check(q, start, n, ref_fn, kq, vq, ids, [ti.TI_PATH_AUTO, ti.TI_PATH_PREFILL])
    del kq, vq
    torch.cuda.empty_cache()


def test_fused_write_past_2_31_elements(gpu):
    """attention_inputs_ (RoPE, theta 1e6, no norm) writing 512 tokens into pages past
    element 2^31 of a bf16 and of an INT8 pool: the written pages are bit-identical to the
    oracle's fused write into a compact pool (slots in the same page order)."""
    g = rng(9300)
    n, nq = 512, HQ
    ids, _, _, _ = _setup(g)
    ids = ids[: n // P]
    positions = np.arange(n, dtype=np.int32)
    slots = ((ids[positions // P] - 1) * P + positions % P + 1).astype(np.int32)
    table = ti.RotaryTable.build(D, n, 1e6, torch.bfloat16)
    cos_sin = table.cos_sin.float().cpu().numpy()
    qkv = randn(g, n, nq + 2 * HK, D, bf16=True)
    qkv_d = torch.from_numpy(qkv).bfloat16().cuda()
    pos_d, slots_d = torch.from_numpy(positions).cuda(), torch.from_numpy(slots).cuda()
    compact = np.arange(1, n + 1, dtype=np.int32)
    sel = torch.from_numpy(ids - 1).long().cuda()

    kd = torch.empty((PAGES, HK, P, D), dtype=torch.bfloat16, device="cuda")
    vd = torch.empty_like(kd)
    q = torch.empty((n, nq, D), dtype=torch.bfloat16, device="cuda")
    ti.attention_inputs_(BE, q, kd, vd, qkv_d, None, None, table, pos_d, slots_d, 1e-6)
    rkp = np.zeros((n // P, HK, P, D), np.float32)
    rvp = np.zeros_like(rkp)
    rq = orc.attention_inputs(qkv, None, None, cos_sin, positions, compact, nq, HK, 1e-6, True,
                              k_pages=rkp, v_pages=rvp)
    assert np.array_equal(q.float().cpu().numpy(), rq)
    assert np.array_equal(kd[sel].float().cpu().numpy(), rkp)
    assert np.array_equal(vd[sel].float().cpu().numpy(), rvp)
    del kd, vd

    kq, vq = ti.int8_kv_pools(D, P, HK, PAGES)
    ti.attention_inputs_(BE, q, kq, vq, qkv_d, None, None, table, pos_d, slots_d, 1e-6)
    lq = np.zeros((2, n // P, HK, P, D), np.int8)
    ls = np.zeros((2, n // P, HK, P), np.float32)
    orc.attention_inputs(qkv, None, None, cos_sin, positions, compact, nq, HK, 1e-6, True,
                         layer_q=lq, layer_scale=ls, smooth=np.ones(D, np.float32))
    assert np.array_equal(kq.layer_q[:, sel].cpu().numpy(), lq)
    assert np.array_equal(kq.layer_scale[:, sel].cpu().numpy(), ls)
    del kq, vq
    torch.cuda.empty_cache()
