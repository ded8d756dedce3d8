"""Pins the CPU oracle (oracle/ref_attention.c) before it is trusted as the checker.

Each check is independent of the oracle's own code path: the reference's known-answer
loops (test/ops/reference.jl), closed forms (dense, unpaged numpy attention in float64),
invariants of softmax attention, INT8 known answers (test/ops/tile.jl:76-81), and torch's
bf16 conversion for the rounding helper. CPU only.
"""
import math

import numpy as np
import pytest
import torch

from helpers import block_table, randn, rng, smoothing
from oracle import oracle as orc


def test_bf16_round_matches_torch():
    g = rng(1)
    x = np.concatenate([randn(g, 10000) * 1e3, randn(g, 1000) * 1e-30,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 65504.0], np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(orc.bf16_round(x), want)
    L = orc.lib()
    orc._setup()
    assert all(L.or_bf16(float(v)) == float(w) for v, w in zip(x[:200], want[:200]))


def test_rope_closed_form():
    # test/ops/reference.jl:29-42: element i rotates with i + D/2 by angle theta[i, pos].
    g = rng(2)
    D, H, L = 8, 2, 10
    positions = np.array([7, 2, 9], np.int32)
    x = randn(g, 3, H, D)
    theta = g.random((L, D // 2), dtype=np.float32)
    c = np.cos(np.concatenate([theta, theta], 1)).astype(np.float32)
    s = np.sin(np.concatenate([theta, theta], 1)).astype(np.float32)
    y = orc.rope(x, c, s, positions, bf16=False)
    for t, p in enumerate(positions):
        for h in range(H):
            for i in range(D // 2):
                a, b, phi = float(x[t, h, i]), float(x[t, h, i + D // 2]), float(theta[p, i])
                assert y[t, h, i] == pytest.approx(a * math.cos(phi) - b * math.sin(phi), rel=1e-5, abs=1e-6)
                assert y[t, h, i + D // 2] == pytest.approx(b * math.cos(phi) + a * math.sin(phi), rel=1e-5, abs=1e-6)


def test_rope_bf16_rounding_points():
    # In bf16 every op rounds (src/ops/reference.jl:38): compare with torch bf16 ops.
    g = rng(3)
    x = randn(g, 5, 4, 16, bf16=True)
    theta = g.random((20, 8), dtype=np.float32) * 100
    c = orc.bf16_round(np.cos(np.concatenate([theta, theta], 1)))
    s = orc.bf16_round(np.sin(np.concatenate([theta, theta], 1)))
    pos = np.array([0, 19, 3, 3, 7], np.int32)
    y = orc.rope(x, c, s, pos, bf16=True)
    tx = torch.from_numpy(x).bfloat16()
    tc = torch.from_numpy(c[pos]).bfloat16()[:, None, :]
    ts = torch.from_numpy(s[pos]).bfloat16()[:, None, :]
    rot = torch.cat([-tx[..., 8:], tx[..., :8]], -1)
    want = (tx * tc + rot * ts).float().numpy()       # torch bf16 ops round each result
    assert np.array_equal(y, want)


def test_store_kv_known_answer():
    # test/ops/reference.jl:91-99: table [5,2,4], P = 4, 10 positions, 2 heads, 5 pages.
    g = rng(4)
    D, P, H, pages, L = 8, 4, 2, 5, 10
    table = np.array([5, 2, 4], np.int32)
    kv = randn(g, L, H, D)
    slot_ids = np.array([(table[p // P] - 1) * P + p % P + 1 for p in range(L)], np.int32)
    kp = np.zeros((pages, H, P, D), np.float32)
    vp = np.zeros_like(kp)
    orc.store_kv(kp, vp, kv, np.zeros_like(kv), slot_ids)
    for p in range(L):
        for h in range(H):
            assert np.array_equal(kp[table[p // P] - 1, h, p % P], kv[p, h])
    assert not kp[[0, 2]].any()                         # pages 1 and 3 untouched
    assert not vp.any()


def test_store_kv_slots_out_of_order():
    # test/ops/tile.jl:63-70 slots [13,14,15,16,5,6,7,8,21], P = 4, H = 8, 6 pages.
    g = rng(5)
    D, P, H, pages = 128, 4, 8, 6
    slots = np.array([13, 14, 15, 16, 5, 6, 7, 8, 21], np.int32)
    k, v = randn(g, 9, H, D), randn(g, 9, H, D)
    kp = np.zeros((pages, H, P, D), np.float32)
    vp = np.zeros_like(kp)
    orc.store_kv(kp, vp, k, v, slots)
    for t, s in enumerate(slots):
        page, off = (s - 1) // P, (s - 1) % P
        assert np.array_equal(kp[page, :, off], k[t]) and np.array_equal(vp[page, :, off], v[t])
    assert np.count_nonzero(kp.any(axis=3)) == 9 * H


def test_quantize_known_answers():
    # test/ops/tile.jl:76-81: s = max|x|/127, |s q - x| <= s/2, max|q| = 127; zero -> 0.
    g = rng(6)
    for _ in range(50):
        x = randn(g, 128) * np.float32(g.random() * 10 + 1e-3)
        q, s = orc.quantize_vector(x.astype(np.float32))
        assert s == pytest.approx(np.abs(x).max() / 127, rel=1e-6)
        assert np.max(np.abs(s * q.astype(np.float64) - x)) <= s / 2 * (1 + 1e-5)
        assert np.abs(q.astype(np.int32)).max() == 127
    q, s = orc.quantize_vector(np.zeros(64, np.float32))
    assert s == 0 and not q.any()
    # Round half up exactly at the formula's float32 steps: floor(x*inv + 0.5).
    x = np.array([127.0, -127.0, 63.5, -63.5, 0.25, -0.25, 1.0], np.float32)
    q, s = orc.quantize_vector(x)
    assert list(q) == [127, -127, 64, -63, 0, 0, 1]


def test_store_kv_int8_matches_quantize_and_smoothing():
    g = rng(7)
    D, P, H, pages = 128, 4, 8, 6
    slots = np.array([13, 14, 15, 16, 5, 6, 7, 8, 21], np.int32)
    k, v = randn(g, 9, H, D, bf16=True), randn(g, 9, H, D, bf16=True)
    c = smoothing(g, D)
    lq = np.zeros((2, pages, H, P, D), np.int8)
    ls = np.zeros((2, pages, H, P), np.float32)
    orc.store_kv_int8(lq, ls, c, k, v, slots)
    for t, s in enumerate(slots):
        page, off = (s - 1) // P, (s - 1) % P
        for h in range(H):
            kq, ks = orc.quantize_vector((k[t, h] / c).astype(np.float32))
            vq, vs = orc.quantize_vector(v[t, h])
            assert np.array_equal(lq[0, page, h, off], kq) and ls[0, page, h, off] == ks
            assert np.array_equal(lq[1, page, h, off], vq) and ls[1, page, h, off] == vs
            # dequantized keys, re-smoothed, approximate the input within half a step
            deq = lq[0, page, h, off].astype(np.float64) * ls[0, page, h, off] * c
            assert np.all(np.abs(deq - k[t, h]) <= ls[0, page, h, off] / 2 * c * (1 + 1e-5))


def paged(kv, table, P, pages):
    """Pages of a contiguous [len][H][D] tensor scattered over a pool via the table,
    through the oracle's store_kv (test/ops/reference.jl:77-86)."""
    L, H, D = kv.shape
    pool = np.zeros((pages, H, P, D), np.float32)
    slot_ids = np.array([(table[p // P] - 1) * P + p % P + 1 for p in range(L)], np.int32)
    orc.store_kv(pool, np.zeros_like(pool), kv, np.zeros_like(kv), slot_ids)
    return pool


def dense_attention(q, kc, vc, start, causal):
    """Unpaged closed form in float64: softmax(scale q.k) v over visible keys."""
    n, Hq, D = q.shape
    Hk = kc.shape[1]
    G = Hq // Hk
    out = np.zeros((n, Hq, D))
    for h in range(Hq):
        gk = h // G
        for t in range(n):
            keys = np.arange(start + t + 1) if causal else np.arange(start + n)
            s = kc[keys, gk].astype(np.float64) @ q[t, h].astype(np.float64) / math.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[t, h] = p @ vc[keys, gk].astype(np.float64)
    return out


@pytest.mark.parametrize("start", [0, 5])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_known_answer(start, causal):
    # test/ops/reference.jl:101-119: D = 16, H = 4, KVH = 2, n = 3, P = 4, table [3,1,6].
    g = rng(10 + start + int(causal))
    D, H, KVH, n, P = 16, 4, 2, 3, 4
    L = start + n
    q = randn(g, n, H, D)
    kc, vc = randn(g, L, KVH, D), randn(g, L, KVH, D)
    table = np.array([3, 1, 6], np.int32)[: -(-L // P)]
    kp, vp = paged(kc, table, P, 6), paged(vc, table, P, 6)
    padded = np.concatenate([table, np.zeros(5, np.int32)])
    o = orc.attention(q, padded, start, 1 / math.sqrt(D), causal, kp, vp)
    assert np.allclose(o, dense_attention(q, kc, vc, start, causal), rtol=1e-5, atol=1e-6)


def test_attention_invariants():
    g = rng(20)
    D, Hq, Hk, P, pages, start, n = 32, 8, 2, 4, 12, 17, 5
    L = start + n
    bt = block_table(g, L, P, pages)
    q = randn(g, n, Hq, D)
    kp = randn(g, pages, Hk, P, D)
    # constant V -> output = that constant
    vp = np.full((pages, Hk, P, D), 0.75, np.float32)
    o = orc.attention(q, bt, start, 0.3, True, kp, vp)
    assert np.allclose(o, 0.75, atol=1e-12)
    # V = KV-head index + 1 -> output of head h is h // G + 1 (GQA mapping, reference.jl:109)
    vp = np.broadcast_to((np.arange(Hk, dtype=np.float32) + 1)[None, :, None, None], kp.shape).copy()
    o = orc.attention(q, bt, start, 0.3, True, kp, vp)
    for h in range(Hq):
        assert np.allclose(o[:, h], h // (Hq // Hk) + 1)
    # q = 0 -> mean of the visible values
    vp = randn(g, pages, Hk, P, D)
    o = orc.attention(np.zeros_like(q), bt, start, 0.3, True, kp, vp)
    for t in range(n):
        rows = [((bt[i // P] - 1), i % P) for i in range(start + t + 1)]
        for gk in range(Hk):
            mean = np.mean([vp[pg, gk, off] for pg, off in rows], axis=0)
            assert np.allclose(o[t, gk * 4], mean, atol=1e-6)
    # a single visible key (start 0, first query, causal) -> that key's value
    o = orc.attention(q, bt, 0, 0.3, True, kp, vp)
    assert np.allclose(o[0, 0], vp[bt[0] - 1, 0, 0])
    # permuting the pool's pages together with the table leaves the output unchanged
    perm = g.permutation(pages)
    inv = np.argsort(perm)
    bt2 = bt.copy()
    used = bt > 0
    bt2[used] = inv[bt[used] - 1] + 1
    o1 = orc.attention(q, bt, start, 0.3, True, kp, vp)
    o2 = orc.attention(q, bt2, start, 0.3, True, kp[perm], vp[perm])
    assert np.array_equal(o1, o2)


def test_attention_eager_mode_close_to_exact():
    g = rng(21)
    D, Hq, Hk, P, pages, start, n = 64, 4, 2, 16, 8, 60, 4
    bt = block_table(g, start + n, P, pages)
    q = randn(g, n, Hq, D, bf16=True)
    kp, vp = randn(g, pages, Hk, P, D, bf16=True), randn(g, pages, Hk, P, D, bf16=True)
    ex = orc.attention(q, bt, start, 1 / 8, True, kp, vp)
    ea = orc.attention(q, bt, start, 1 / 8, True, kp, vp, exact=False, bf16=True)
    assert np.max(np.abs(ex - ea)) < 2e-2
    assert np.array_equal(ea, orc.bf16_round(ea))


def test_attention_int8_dequantizes_like_gather_pages():
    # gather_pages(::Int8Pages) (src/ops/quant.jl:165-170): K = (q s) c, V = q s.
    g = rng(22)
    D, Hq, Hk, P, pages, start, n = 32, 4, 2, 4, 6, 9, 3
    c = smoothing(g, D)
    lq = g.integers(-127, 128, (2, pages, Hk, P, D), dtype=np.int8)
    ls = (g.random((2, pages, Hk, P), dtype=np.float32) * 0.05).astype(np.float32)
    kd = ((lq[0].astype(np.float32) * ls[0][..., None]) * c).astype(np.float32)
    vd = (lq[1].astype(np.float32) * ls[1][..., None]).astype(np.float32)
    bt = block_table(g, start + n, P, pages)
    q = randn(g, n, Hq, D)
    o8 = orc.attention(q, bt, start, 0.2, True, layer_q=lq, layer_scale=ls, smooth=c)
    od = orc.attention(q, bt, start, 0.2, True, kd, vd)
    assert np.allclose(o8, od, rtol=1e-6, atol=1e-7)


def test_attention_inputs_composes_rope_and_store():
    # attention_inputs! without norm == store_kv!(rope(k)) and rope(q)
    # (generic chain src/ops/interface.jl:169-179).
    g = rng(23)
    D, nq, nkv, P, pages = 64, 4, 2, 16, 6
    positions = np.array([3, 17, 18, 40, 0], np.int32)
    slots = np.array([13, 14, 15, 16, 70], np.int32)
    n = len(positions)
    theta = g.random((64, D // 2), dtype=np.float32) * 100
    c = orc.bf16_round(np.cos(np.concatenate([theta, theta], 1)))
    s = orc.bf16_round(np.sin(np.concatenate([theta, theta], 1)))
    cs = np.stack([c, s], 1)
    qkv = randn(g, n, nq + 2 * nkv, D, bf16=True)
    kp = np.zeros((pages, nkv, P, D), np.float32)
    vp = np.zeros_like(kp)
    q = orc.attention_inputs(qkv, None, None, cs, positions, slots, nq, nkv, 1e-6, True,
                             k_pages=kp, v_pages=vp)
    assert np.array_equal(q, orc.rope(qkv[:, :nq], c, s, positions, True))
    kp2, vp2 = np.zeros_like(kp), np.zeros_like(kp)
    orc.store_kv(kp2, vp2, orc.rope(qkv[:, nq:nq + nkv], c, s, positions, True),
                 qkv[:, nq + nkv:].copy(), slots)
    assert np.array_equal(kp, kp2) and np.array_equal(vp, vp2)


def _torch_norm_rope(x, w, c, s, pos, eps):
    """Qwen3 q/k RMSNorm then rope with torch ops: inv_rms in Float32, x inv_rms rounded to
    bf16, times w rounded to bf16 (src/ops/reference.jl:17-21, src/ops/tile/fused.jl:15-34),
    then rope with every bf16 op rounding (src/ops/reference.jl:32-39)."""
    x32 = torch.from_numpy(x).float()
    inv = 1.0 / torch.sqrt((x32 * x32).sum(-1, keepdim=True) / x.shape[-1] + eps)
    h = x.shape[-1] // 2
    tx = (x32 * inv).bfloat16() * torch.from_numpy(w).bfloat16()
    tc = torch.from_numpy(c[pos]).bfloat16()[:, None, :]
    ts = torch.from_numpy(s[pos]).bfloat16()[:, None, :]
    rot = torch.cat([-tx[..., h:], tx[..., :h]], -1)
    return (tx * tc + rot * ts).float().numpy()


def test_attention_inputs_norm_rounding_points():
    # With q/k norm: the oracle's rounding points equal torch bf16 ops exactly. The sums of
    # squares are made exact in any order (bf16 inputs that are small multiples of 1/8,
    # so every square and partial sum is a float32 integer multiple of 1/64), so inv_rms
    # is the same Float32 number on both sides and no tolerance is needed.
    g = rng(24)
    D, nq, nkv, P, pages = 128, 4, 2, 16, 6
    positions = np.array([3, 17, 18, 40, 0, 63], np.int32)
    slots = np.array([13, 14, 15, 16, 70, 2], np.int32)
    n = len(positions)
    theta = g.random((64, D // 2), dtype=np.float32) * 100
    c = orc.bf16_round(np.cos(np.concatenate([theta, theta], 1)))
    s = orc.bf16_round(np.sin(np.concatenate([theta, theta], 1)))
    cs = np.stack([c, s], 1)
    qkv = (g.integers(-64, 65, (n, nq + 2 * nkv, D)) / 8.0).astype(np.float32)
    qn, kn = randn(g, D, bf16=True), randn(g, D, bf16=True)
    kp = np.zeros((pages, nkv, P, D), np.float32)
    vp = np.zeros_like(kp)
    for eps in (1e-6, 0.25):
        q = orc.attention_inputs(qkv, qn, kn, cs, positions, slots, nq, nkv, eps, True,
                                 k_pages=kp, v_pages=vp)
        assert np.array_equal(q, _torch_norm_rope(qkv[:, :nq], qn, c, s, positions, eps))
        k_want = _torch_norm_rope(qkv[:, nq:nq + nkv], kn, c, s, positions, eps)
        for t, sl in enumerate(slots):
            page, off = (sl - 1) // P, (sl - 1) % P
            if page < pages:
                assert np.array_equal(kp[page, :, off], k_want[t])
                assert np.array_equal(vp[page, :, off], qkv[t, nq + nkv:])


def test_attention_inputs_norm_random_within_one_ulp():
    # Random bf16 inputs: the sum of squares' order differs (the oracle sums in double),
    # so inv_rms may differ by a Float32 ulp: within one bf16 ulp of torch everywhere,
    # equal almost everywhere.
    g = rng(25)
    D, nq, nkv, P, pages = 128, 8, 2, 16, 4
    positions = g.integers(0, 64, 40).astype(np.int32)
    n = len(positions)
    theta = g.random((64, D // 2), dtype=np.float32) * 100
    c = orc.bf16_round(np.cos(np.concatenate([theta, theta], 1)))
    s = orc.bf16_round(np.sin(np.concatenate([theta, theta], 1)))
    qkv = randn(g, n, nq + 2 * nkv, D, bf16=True, scale=3.0)
    qn = randn(g, D, bf16=True)
    kp = np.zeros((pages, nkv, P, D), np.float32)
    q = orc.attention_inputs(qkv, qn, qn, np.stack([c, s], 1), positions, np.arange(1, n + 1, dtype=np.int32), nq, nkv,
                             1e-6, True, k_pages=kp, v_pages=kp.copy())
    want = _torch_norm_rope(qkv[:, :nq], qn, c, s, positions, 1e-6)
    from helpers import bf16_eps
    assert np.all(np.abs(q - want) <= bf16_eps(want) + 1e-30)
    assert np.mean(q == want) >= 0.99
