"""RoPE, KV-cache writes and the fused attention-input op on the GPU vs the CPU oracle.

All bit-exact (test/ops/tile.jl:41-47, :63-89, :111-146), except the q/k RMSNorm path,
whose sum of squares runs in a different order (<= 1 bf16 ulp, as the reference's own
tolerance for it, test/ops/tile.jl:133-134).
"""
import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import randn, rng, smoothing, ulps
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()
DT = {False: torch.float32, True: torch.bfloat16}


def dev(x, bf16=False):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DT[bf16]).cuda()


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("dims", [(128, 16, 1), (128, 8, 7), (64, 24, 3)])
def test_rope_bit_exact(gpu, bf16, dims):
    D, H, n = dims
    g = rng(100 + D + H + n)
    x = randn(g, n, H, D, bf16=bf16)
    theta = g.random((50, D // 2), dtype=np.float32) * 100
    c, s = np.cos(np.concatenate([theta, theta], 1)), np.sin(np.concatenate([theta, theta], 1))
    c, s = (orc.bf16_round(c), orc.bf16_round(s)) if bf16 else (c.astype(np.float32), s.astype(np.float32))
    pos = g.integers(0, 50, n).astype(np.int32)
    y = ti.rope(BE, dev(x, bf16), dev(c, bf16), dev(s, bf16), torch.from_numpy(pos).cuda())
    assert np.array_equal(host(y), orc.rope(x, c, s, pos, bf16))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("D", [128, 64, 96])
def test_store_kv_bit_exact(gpu, bf16, D):
    P, H, pages, n = 4, 8, 6, 9
    g = rng(200 + bf16 + D)
    k, v = randn(g, n, H, D, bf16=bf16), randn(g, n, H, D, bf16=bf16)
    slots = np.array([13, 14, 15, 16, 5, 6, 7, 8, 21], np.int32)
    kp = torch.zeros((pages, H, P, D), dtype=DT[bf16], device="cuda")
    vp = torch.zeros_like(kp)
    ti.store_kv_(BE, kp, vp, dev(k, bf16), dev(v, bf16), torch.from_numpy(slots).cuda())
    rk, rv = np.zeros((pages, H, P, D), np.float32), np.zeros((pages, H, P, D), np.float32)
    orc.store_kv(rk, rv, k, v, slots)
    assert np.array_equal(host(kp), rk) and np.array_equal(host(vp), rv)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("smooth", [False, True])
@pytest.mark.parametrize("D", [128, 64, 96])
def test_store_kv_int8_bit_exact(gpu, bf16, smooth, D):
    P, H, pages, n = 4, 8, 6, 9
    g = rng(300 + 2 * bf16 + smooth + D)
    k, v = randn(g, n, H, D, bf16=bf16), randn(g, n, H, D, bf16=bf16)
    slots = np.array([13, 14, 15, 16, 5, 6, 7, 8, 21], np.int32)
    c = smoothing(g, D) if smooth else np.ones(D, np.float32)
    kq, vq = ti.int8_kv_pools(D, P, H, pages, key_smoothing=torch.from_numpy(c) if smooth else None)
    ti.store_kv_(BE, kq, vq, dev(k, bf16), dev(v, bf16), torch.from_numpy(slots).cuda())
    lq = np.zeros((2, pages, H, P, D), np.int8)
    ls = np.zeros((2, pages, H, P), np.float32)
    orc.store_kv_int8(lq, ls, c, k, v, slots)
    assert np.array_equal(kq.layer_q.cpu().numpy(), lq)
    assert np.array_equal(kq.layer_scale.cpu().numpy(), ls)
    # known answers (test/ops/tile.jl:76-81) on slot 13 = offset 0 of page 4
    x = k[0, 0] / c
    s = ls[0, 3, 0, 0]
    assert s == pytest.approx(np.abs(x).max() / 127, rel=1e-6)
    assert np.abs(lq[0, 3, 0, 0].astype(np.int32)).max() == 127


def _table(g, D, L, bf16):
    theta = g.random((L, D // 2), dtype=np.float32) * 100
    ang = np.concatenate([theta, theta], 1)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    if bf16:
        c, s = orc.bf16_round(c), orc.bf16_round(s)
    return c, s, ti.RotaryTable.from_arrays(torch.from_numpy(c), torch.from_numpy(s), DT[bf16])


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("qk_norm", [False, True])
def test_attention_inputs(gpu, bf16, qk_norm):
    # test/ops/tile.jl:111-146: positions [3,17,18,40,0], slots [13,14,15,16,70].
    D, nq, nkv, P, pages, L = 128, 16, 8, 16, 6, 64
    g = rng(400 + 2 * bf16 + qk_norm)
    positions = np.array([3, 17, 18, 40, 0], np.int32)
    slots = np.array([13, 14, 15, 16, 70], np.int32)
    n = len(positions)
    c, s, table = _table(g, D, L, bf16)
    qkv = randn(g, n, nq + 2 * nkv, D, bf16=bf16)
    qn, kn = (randn(g, D, bf16=bf16), randn(g, D, bf16=bf16)) if qk_norm else (None, None)
    pos_d, slots_d = torch.from_numpy(positions).cuda(), torch.from_numpy(slots).cuda()

    q = torch.zeros((n, nq, D), dtype=DT[bf16], device="cuda")
    kp = torch.zeros((pages, nkv, P, D), dtype=DT[bf16], device="cuda")
    vp = torch.zeros_like(kp)
    ti.attention_inputs_(BE, q, kp, vp, dev(qkv, bf16), None if qn is None else dev(qn, bf16),
                         None if kn is None else dev(kn, bf16), table, pos_d, slots_d, 1e-6)
    rkp, rvp = np.zeros((pages, nkv, P, D), np.float32), np.zeros((pages, nkv, P, D), np.float32)
    rq = orc.attention_inputs(qkv, qn, kn, np.stack([c, s], 1), positions, slots, nq, nkv, 1e-6, bf16,
                              k_pages=rkp, v_pages=rvp)
    if not qk_norm:
        assert np.array_equal(host(q), rq)
        assert np.array_equal(host(kp), rkp) and np.array_equal(host(vp), rvp)
        # fused == the primitive ops chained (rope_ then store_kv_), bit-identical
        kp2, vp2 = torch.zeros_like(kp), torch.zeros_like(kp)
        qkv_d = dev(qkv, bf16)
        qs = qkv_d[:, :nq].contiguous()
        kk = qkv_d[:, nq:nq + nkv].contiguous()
        vv = qkv_d[:, nq + nkv:].contiguous()
        q2 = ti.rope(BE, qs, table.cos, table.sin, pos_d)
        ti.store_kv_(BE, kp2, vp2, ti.rope(BE, kk, table.cos, table.sin, pos_d), vv, slots_d)
        assert torch.equal(q2, q) and torch.equal(kp2, kp) and torch.equal(vp2, vp)
    else:
        worst = max(ulps(r, host(f)) for r, f in ((rq, q), (rkp, kp), (rvp, vp)))
        assert worst <= (1 if bf16 else 32)

    # into an INT8 cache: quantized as store_kv! quantizes (known when no norm: bit-exact)
    cs = smoothing(g, D)
    kq, vq = ti.int8_kv_pools(D, P, nkv, pages, key_smoothing=torch.from_numpy(cs))
    q8 = torch.zeros_like(q)
    ti.attention_inputs_(BE, q8, kq, vq, dev(qkv, bf16), None if qn is None else dev(qn, bf16),
                         None if kn is None else dev(kn, bf16), table, pos_d, slots_d, 1e-6)
    lq = np.zeros((2, pages, nkv, P, D), np.int8)
    ls = np.zeros((2, pages, nkv, P), np.float32)
    orc.attention_inputs(qkv, qn, kn, np.stack([c, s], 1), positions, slots, nq, nkv, 1e-6, bf16,
                         layer_q=lq, layer_scale=ls, smooth=cs)
    assert torch.equal(q8, q)
    if not qk_norm:
        assert np.array_equal(kq.layer_q.cpu().numpy(), lq)
        assert np.array_equal(kq.layer_scale.cpu().numpy(), ls)
    else:
        assert np.abs(kq.layer_q.cpu().numpy().astype(np.int32) - lq).max() <= 1
        assert np.allclose(kq.layer_scale.cpu().numpy(), ls, rtol=1e-2)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_attention_inputs_norm_equals_unfused_chain(gpu, bf16, D):
    """Fused q/k RMSNorm + RoPE + KV write == rmsnorm_ -> rope -> store_kv_ run one by one,
    bit-identical (test/ops/tile.jl:109-146; the generic chain src/ops/interface.jl:169-179),
    into a dense and an INT8 cache."""
    nq, nkv, P, pages, L = 8, 2, 16, 6, 64
    g = rng(480 + 2 * D + bf16)
    positions = np.array([3, 17, 18, 40, 0], np.int32)
    slots = np.array([13, 14, 15, 16, 70], np.int32)
    n = len(positions)
    c, s, table = _table(g, D, L, bf16)
    qkv = randn(g, n, nq + 2 * nkv, D, bf16=bf16)
    qn, kn = randn(g, D, bf16=bf16), randn(g, D, bf16=bf16)
    pos_d, slots_d = torch.from_numpy(positions).cuda(), torch.from_numpy(slots).cuda()
    qkv_d, qn_d, kn_d = dev(qkv, bf16), dev(qn, bf16), dev(kn, bf16)

    q = torch.zeros((n, nq, D), dtype=DT[bf16], device="cuda")
    kp = torch.zeros((pages, nkv, P, D), dtype=DT[bf16], device="cuda")
    vp = torch.zeros_like(kp)
    ti.attention_inputs_(BE, q, kp, vp, qkv_d, qn_d, kn_d, table, pos_d, slots_d, 1e-6)

    qs = ti.rmsnorm(BE, qkv_d[:, :nq].contiguous(), qn_d, 1e-6)
    ks = ti.rmsnorm(BE, qkv_d[:, nq:nq + nkv].contiguous(), kn_d, 1e-6)
    vv = qkv_d[:, nq + nkv:].contiguous()
    q2 = ti.rope(BE, qs, table.cos, table.sin, pos_d)
    k2 = ti.rope(BE, ks, table.cos, table.sin, pos_d)
    kp2, vp2 = torch.zeros_like(kp), torch.zeros_like(kp)
    ti.store_kv_(BE, kp2, vp2, k2, vv, slots_d)
    assert torch.equal(q, q2) and torch.equal(kp, kp2) and torch.equal(vp, vp2)

    cs = smoothing(g, D)
    kq, vq = ti.int8_kv_pools(D, P, nkv, pages, key_smoothing=torch.from_numpy(cs))
    kq2, vq2 = ti.int8_kv_pools(D, P, nkv, pages, key_smoothing=torch.from_numpy(cs))
    ti.attention_inputs_(BE, torch.zeros_like(q), kq, vq, qkv_d, qn_d, kn_d, table, pos_d, slots_d, 1e-6)
    ti.store_kv_(BE, kq2, vq2, k2, vv, slots_d)
    assert torch.equal(kq.layer_q, kq2.layer_q) and torch.equal(kq.layer_scale, kq2.layer_scale)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("H", [128, 100, 2560])
def test_rmsnorm(gpu, bf16, H):
    """rmsnorm_ rows (src/ops/tile/norm.jl:5-38) against the formula in float64 with the
    reference's rounding points: within one rounding of T (the Float32 sum order differs)."""
    g = rng(900 + H + bf16)
    x = randn(g, 7, H, bf16=bf16)
    w = randn(g, H, bf16=bf16)
    y = ti.rmsnorm(BE, dev(x, bf16), dev(w, bf16), 1e-6).float().cpu().numpy()
    inv = 1.0 / np.sqrt((x.astype(np.float64) ** 2).sum(1, keepdims=True) / H + 1e-6)
    rnd = orc.bf16_round if bf16 else (lambda a: a.astype(np.float32))
    ref = rnd(rnd((x * inv).astype(np.float32)) * w[None, :])
    assert ulps(ref, y) <= 1 if bf16 else np.allclose(ref, y, rtol=1e-5, atol=1e-6)


def test_out_of_range_slots_are_skipped(gpu):
    D, P, H, pages = 64, 4, 2, 3
    k = torch.ones((3, H, D), dtype=torch.bfloat16, device="cuda")
    kp = torch.zeros((pages, H, P, D), dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    ti.store_kv_(BE, kp, vp, k, k, torch.tensor([0, 13, 2], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert kp.sum().item() == H * D                     # only slot 2 was written
    assert kp[0, :, 1].float().eq(1).all()


@pytest.mark.parametrize("int8", [False, True], ids=["dense", "int8"])
@pytest.mark.parametrize("D", [64, 128])
def test_attention_inputs_out_of_range(gpu, D, int8):
    """Tokens whose slot lies outside the pool write no K/V row, tokens whose position
    lies outside the rotary table write nothing (the q rows keep what they held); every
    other token is written as the oracle writes it. Both head dims run the D / 8 lanes per
    head kernel; on INT8 pages the untouched rows and scales keep their prior contents."""
    nq, nkv, P, pages, L = 4, 2, 4, 3, 32
    g = rng(700 + D + (1 if int8 else 0))
    positions = np.array([3, 5, 40, 7], np.int32)            # 40 is past the table
    slots = np.array([2, 13, 5, 0], np.int32)                # 13 and 0 are outside the pool
    n = len(positions)
    c, s, table = _table(g, D, L, True)
    qkv = randn(g, n, nq + 2 * nkv, D, bf16=True)
    q = torch.full((n, nq, D), 7.0, dtype=torch.bfloat16, device="cuda")
    if int8:
        cs = (g.random(D, dtype=np.float32) + 0.5).astype(np.float32)
        kp, vp = ti.int8_kv_pools(D, P, nkv, pages, key_smoothing=torch.from_numpy(cs))
        kp.layer_q.fill_(55)                                 # prior contents
        kp.layer_scale.fill_(0.25)
    else:
        kp = torch.zeros((pages, nkv, P, D), dtype=torch.bfloat16, device="cuda")
        vp = torch.zeros_like(kp)
    ti.attention_inputs_(BE, q, kp, vp, dev(qkv, True), None, None, table,
                         torch.from_numpy(positions).cuda(), torch.from_numpy(slots).cuda(), 1e-6)
    keep = np.array([0, 1, 3])                               # tokens with an in-table position
    cs_tab = np.stack([c, s], 1)
    scratch = [np.zeros((pages, nkv, P, D), np.float32) for _ in range(2)]
    rq = orc.attention_inputs(qkv[keep], None, None, cs_tab, positions[keep], np.ones(3, np.int32),
                              nq, nkv, 1e-6, True, k_pages=scratch[0], v_pages=scratch[1])
    got_q = host(q)
    assert np.array_equal(got_q[keep], rq)
    assert (got_q[2] == 7.0).all()
    # only token 0 has both an in-table position and an in-pool slot
    if int8:
        rlq = np.full((2, pages, nkv, P, D), 55, np.int8)
        rls = np.full((2, pages, nkv, P), 0.25, np.float32)
        orc.attention_inputs(qkv[:1], None, None, cs_tab, positions[:1], slots[:1], nq, nkv, 1e-6, True,
                             layer_q=rlq, layer_scale=rls, smooth=cs)
        assert np.array_equal(kp.layer_q.cpu().numpy(), rlq)
        assert np.array_equal(kp.layer_scale.cpu().numpy(), rls)
        assert (rlq != 55).any()                             # the in-range token was written
    else:
        rkp, rvp = np.zeros((pages, nkv, P, D), np.float32), np.zeros((pages, nkv, P, D), np.float32)
        orc.attention_inputs(qkv[:1], None, None, cs_tab, positions[:1], slots[:1], nq, nkv, 1e-6, True,
                             k_pages=rkp, v_pages=rvp)
        assert np.array_equal(host(kp), rkp) and np.array_equal(host(vp), rvp)
