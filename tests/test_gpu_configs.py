"""The BASELINE configs at full size on the GPU.

Inputs are generated on the GPU from a seeded torch generator; a sample of sequences is
checked against the oracle (their pages gathered to the host into a compact pool with a
renumbered block table, which the oracle's block-table invariance makes equivalent).
Tolerances: max abs error <= 2e-2 for bf16 / INT8-KV and <= 1e-4 for fp32, against the
double-accumulated oracle.
"""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()


def make_batch(gen, lens, n, Hq, Hk, D, P, dtype=torch.bfloat16, slack=3):
    """Pools, block tables (shuffled pages, zero-padded) and queries for sequences whose
    step's n queries sit at positions L_b - n .. L_b - 1."""
    per = [-(-L // P) for L in lens]
    pages = sum(per) + slack
    perm = (torch.randperm(pages, generator=gen) + 1).to(torch.int32)
    width = max(per) + 16
    bts = torch.zeros((len(lens), width), dtype=torch.int32)
    off = 0
    for b, u in enumerate(per):
        bts[b, :u] = perm[off:off + u]
        off += u
    dg = torch.Generator(device="cuda").manual_seed(int(torch.randint(0, 2 ** 31, (1,), generator=gen)))
    k = torch.randn((pages, Hk, P, D), generator=dg, device="cuda").to(dtype)
    v = torch.randn((pages, Hk, P, D), generator=dg, device="cuda").to(dtype)
    q = torch.randn((len(lens) * n, Hq, D), generator=dg, device="cuda").to(dtype)
    pos = torch.cat([torch.arange(L - n, L, dtype=torch.int32) for L in lens]).cuda()
    return k, v, q, bts.cuda(), pos


def compact(pool, bt_row, L, P):
    """The sequence's pages as a compact host pool [used][Hk][P][D] and table 1..used."""
    used = -(-L // P)
    idx = bt_row[:used].long() - 1
    return pool[idx].float().cpu().numpy(), np.arange(1, used + 1, dtype=np.int32)


def check_seqs(out, q, k, v, bts, lens, n, P, scale, tol, samples, causal=True):
    got = out.float().cpu().numpy()
    qh = q.float().cpu().numpy()
    for b in samples:
        kp, bt = compact(k, bts[b], lens[b], P)
        vp, _ = compact(v, bts[b], lens[b], P)
        ref = orc.attention(qh[b * n:(b + 1) * n], bt, lens[b] - n, scale, causal, kp, vp)
        err = float(np.max(np.abs(ref - got[b * n:(b + 1) * n])))
        assert err <= tol, f"seq {b} (L={lens[b]}): max abs err {err}"
        if tol <= 1e-4:
            # fp32: the reference's bound, isapprox(y, exact; rtol = 1e-5) (test/ops/tile.jl:240)
            y = got[b * n:(b + 1) * n].astype(np.float64)
            d = float(np.linalg.norm(ref - y))
            assert d <= 1e-5 * max(float(np.linalg.norm(ref)), float(np.linalg.norm(y))), f"seq {b}: norm err {d}"


@pytest.mark.parametrize("B", [1, 8, 32])
def test_config2_qwen3_4b_decode(gpu, B):
    """bf16 paged decode, 32/8 heads, D 128, 16-token pages, L ~ U[1024, 8192]."""
    gen = torch.Generator().manual_seed(2000 + B)
    lens = torch.randint(1024, 8193, (B,), generator=gen).tolist()
    k, v, q, bts, pos = make_batch(gen, lens, 1, 32, 8, 128, 16)
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, num_seqs=B, max_query_len=1)
    ti.paged_attention_(BE, out, ws, q, k, v, bts, pos, 1 / math.sqrt(128), True, max_query_len=1)
    check_seqs(out, q, k, v, bts, lens, 1, 16, 1 / math.sqrt(128), 2e-2,
               sorted({0, B // 2, B - 1}))


def test_config2_target_batch32_ctx4096(gpu):
    """The headline shape: B = 32 x 4096 (single-split, direct-output decode)."""
    gen = torch.Generator().manual_seed(2032)
    lens = [4096] * 32
    k, v, q, bts, pos = make_batch(gen, lens, 1, 32, 8, 128, 16)
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, num_seqs=32, max_query_len=1)
    ti.paged_attention_(BE, out, ws, q, k, v, bts, pos, 1 / math.sqrt(128), True, max_query_len=1)
    check_seqs(out, q, k, v, bts, lens, 1, 16, 1 / math.sqrt(128), 2e-2, [0, 13, 31])


def test_config1_qwen3_06b_fp32(gpu):
    """fp32, batch 1, 16/8 heads, 1024 positions in 16-token pages, tolerance 1e-4."""
    gen = torch.Generator().manual_seed(1001)
    k, v, q, bts, pos = make_batch(gen, [1024], 1, 16, 8, 128, 16, dtype=torch.float32)
    out = ti.attention(BE, q, k, v, bts[0], pos, 1 / math.sqrt(128))
    check_seqs(out, q, k, v, bts, [1024], 1, 16, 1 / math.sqrt(128), 1e-4, [0])


@pytest.mark.parametrize("start", [0, 1024])
def test_config3_prefill_with_fused_rope_kv_write(gpu, start):
    """512 new tokens (from scratch, or after a 1024-token cached prefix): fused RoPE
    (theta 1e6) + KV page write of the new tokens from qkv, then causal attention."""
    gen = torch.Generator().manual_seed(3000 + start)
    Hq, Hk, D, P, n = 32, 8, 128, 16, 512
    L = start + n
    k, v, _, bts, pos = make_batch(gen, [L], n, Hq, Hk, D, P)
    qkv = torch.randn((n, (Hq + 2 * Hk) * D), generator=gen).to(torch.bfloat16).cuda()
    table = ti.RotaryTable.build(D, 4096, 1e6, torch.bfloat16)
    bt_host = bts[0].cpu().numpy()
    slots = np.array([(bt_host[p // P] - 1) * P + p % P + 1 for p in range(start, L)], np.int32)
    q = torch.empty((n, Hq, D), dtype=torch.bfloat16, device="cuda")
    k_before = k.float().cpu().numpy()
    v_before = v.float().cpu().numpy()
    ti.attention_inputs_(BE, q, k, v, qkv, None, None, table, pos, torch.from_numpy(slots).cuda(), 1e-6)
    out = ti.attention(BE, q, k, v, bts[0], pos, 1 / math.sqrt(D))
    # oracle chain on the same inputs
    rk, rv = k_before.copy(), v_before.copy()
    rq = orc.attention_inputs(qkv.float().cpu().numpy().reshape(n, Hq + 2 * Hk, D), None, None,
                              table.cos_sin.float().cpu().numpy(), pos.cpu().numpy(), slots, Hq, Hk,
                              1e-6, True, k_pages=rk, v_pages=rv)
    assert np.array_equal(q.float().cpu().numpy(), rq)
    assert np.array_equal(k.float().cpu().numpy(), rk) and np.array_equal(v.float().cpu().numpy(), rv)
    ref = orc.attention(rq, bt_host, start, 1 / math.sqrt(D), True, rk, rv)
    err = float(np.max(np.abs(ref - out.float().cpu().numpy())))
    assert err <= 2e-2, err


def test_config4_llama3_8b_int8_decode(gpu):
    """INT8 cache, batch 8 x 32768 positions, K/V ~ N(0,1) quantized per (token, KV head)."""
    gen = torch.Generator().manual_seed(4000)
    Hq, Hk, D, P, B, L = 32, 8, 128, 16, 8, 32768
    lens = [L] * B
    per = L // P
    pages = B * per
    perm = (torch.randperm(pages, generator=gen) + 1).to(torch.int32)
    bts = perm.view(B, per).cuda()
    kq, vq = ti.int8_kv_pools(D, P, Hk, pages)
    dg = torch.Generator(device="cuda").manual_seed(4001)
    chunk = 65536                     # quantize the pool in slot chunks through the GPU store
    for s0 in range(0, pages * P, chunk):
        kk = torch.randn((chunk, Hk, D), generator=dg, device="cuda").to(torch.bfloat16)
        vv = torch.randn((chunk, Hk, D), generator=dg, device="cuda").to(torch.bfloat16)
        ti.store_kv_(BE, kq, vq, kk, vv, torch.arange(s0 + 1, s0 + chunk + 1, dtype=torch.int32, device="cuda"))
    q = torch.randn((B, Hq, D), generator=gen).to(torch.bfloat16).cuda()
    pos = torch.full((B,), L - 1, dtype=torch.int32).cuda()
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, kq, num_seqs=B, max_query_len=1)
    ti.paged_attention_(BE, out, ws, q, kq, vq, bts, pos, 1 / math.sqrt(D), True, max_query_len=1)
    got = out.float().cpu().numpy()
    for b in (0, B - 1):
        idx = bts[b].long() - 1
        lq = kq.layer_q[:, idx].cpu().numpy()
        ls = kq.layer_scale[:, idx].cpu().numpy()
        ref = orc.attention(q[b:b + 1].float().cpu().numpy(), np.arange(1, per + 1, dtype=np.int32), L - 1,
                            1 / math.sqrt(D), True, layer_q=np.ascontiguousarray(lq),
                            layer_scale=np.ascontiguousarray(ls), smooth=np.ones(D, np.float32))
        err = float(np.max(np.abs(ref - got[b:b + 1])))
        assert err <= 2e-2, f"seq {b}: {err}"


def test_config5_qwen3_8b_verify(gpu):
    """Speculative verify: batch 16, 16 causal query tokens on 4096 cached positions."""
    gen = torch.Generator().manual_seed(5000)
    n, B = 16, 16
    lens = [4096 + n] * B
    k, v, q, bts, pos = make_batch(gen, lens, n, 32, 8, 128, 16)
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, num_seqs=B, max_query_len=n)
    ti.paged_attention_(BE, out, ws, q, k, v, bts, pos, 1 / math.sqrt(128), True, max_query_len=n)
    check_seqs(out, q, k, v, bts, lens, n, 16, 1 / math.sqrt(128), 2e-2, [0, 7, 15])
