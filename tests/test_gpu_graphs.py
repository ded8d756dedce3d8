"""Graph capture: attention and the fused KV write recorded once in a HIP graph stay
valid as the sequences grow, because the kernels read the step's positions and block
tables from device memory and their launch shapes depend only on host shapes
(src/ops/tile/attention.jl:14-17; test/engine/runner.jl:16-33 checks replay == eager).
Each replay is compared with an eager call on the same state, with eager work and
synchronizations between replays."""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()


@pytest.mark.parametrize("B,n", [(4, 1), (40, 1), (2, 16)])
def test_decode_step_graph_replays_as_sequences_grow(gpu, B, n):
    Hq, Hk, D, P = 32, 8, 128, 16
    torch.manual_seed(B * 100 + n)
    lens = [700 + 37 * b for b in range(B)]
    steps = 5
    width = (max(lens) + n * steps) // P + 2
    pages = B * width
    k = torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    bts = (torch.randperm(pages, dtype=torch.int32) + 1).view(B, width).cuda()
    pos = torch.zeros(B * n, dtype=torch.int32, device="cuda")
    q = torch.randn((B * n, Hq, D), device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, num_seqs=B, max_query_len=n)
    scale = 1 / math.sqrt(D)

    def set_positions(step):
        p = torch.cat([torch.arange(L + step * n, L + step * n + n, dtype=torch.int32) for L in lens])
        pos.copy_(p.cuda())

    set_positions(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ti.paged_attention_(BE, out, ws, q, k, v, bts, pos, scale, True, max_query_len=n)
    for step in range(steps):
        set_positions(step)                     # the sequences grew by n positions
        q.normal_()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = torch.empty_like(q)
        ti.paged_attention_(BE, ref, ws, q, k, v, bts, pos, scale, True, max_query_len=n)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {step} differs from eager"


@pytest.mark.parametrize("path,n", [(ti.TI_PATH_AUTO, 128), (ti.TI_PATH_PREFILL_PINGPONG, 128),
                                    (ti.TI_PATH_AUTO, 512)])
def test_prefill_and_kv_write_graph(gpu, path, n):
    """AUTO's choice (128 new tokens: the four-wave kernel with key splits; 512: the 16-row
    paired kernel), and the 8-wave ping-pong prefill kernel pinned."""
    Hq, Hk, D, P = 32, 8, 128, 16
    torch.manual_seed(7)
    pages = 64
    k = torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    bt = (torch.randperm(pages, dtype=torch.int32) + 1).cuda()
    table = ti.RotaryTable.build(D, 2048, 1e6, torch.bfloat16)
    qkv = torch.randn((n, (Hq + 2 * Hk) * D), device="cuda", dtype=torch.bfloat16)
    q = torch.empty((n, Hq, D), device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(q)
    pos = torch.zeros(n, dtype=torch.int32, device="cuda")
    slots = torch.zeros(n, dtype=torch.int32, device="cuda")
    bt_host = bt.cpu()

    def set_step(start):
        p = torch.arange(start, start + n, dtype=torch.int32)
        pos.copy_(p.cuda())
        slots.copy_(torch.tensor([(int(bt_host[x // P]) - 1) * P + x % P + 1 for x in p.tolist()],
                                 dtype=torch.int32).cuda())

    def step():
        ti.attention_inputs_(BE, q, k, v, qkv, None, None, table, pos, slots, 1e-6)
        ti.attention_(BE, out, None, q, k, v, bt, pos, 1 / math.sqrt(D), path=path)

    set_step(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i, start in enumerate((0, 128, 256, 384)):    # chunked prefill: the prefix grows
        set_step(start)
        qkv.normal_()
        k2, v2 = k.clone(), v.clone()
        g.replay()
        torch.cuda.synchronize()
        got, kg, vg = out.clone(), k.clone(), v.clone()
        k.copy_(k2)
        v.copy_(v2)
        step()
        torch.cuda.synchronize()
        assert torch.equal(got, out) and torch.equal(kg, k) and torch.equal(vg, v), f"replay {i}"


def _pools(kind, pages, Hk, P, D):
    """Two identical caches (random contents stand for the cached prefix)."""
    if kind in ("bf16", "fp32"):
        k = torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16 if kind == "bf16" else torch.float32)
        v = torch.randn_like(k)
        return (k, v), (k.clone(), v.clone())
    kq, vq = ti.int8_kv_pools(D, P, Hk, pages, torch.rand(D) + 0.5)
    kq.layer_q.copy_(torch.randint(-127, 128, kq.layer_q.shape, dtype=torch.int8))
    kq.layer_scale.copy_(torch.rand(kq.layer_scale.shape) * 0.02 + 0.001)
    lq, ls, sm = kq.layer_q.clone(), kq.layer_scale.clone(), kq.smooth.clone()
    other = (ti.Int8Pages(lq, ls, sm, 0), ti.Int8Pages(lq, ls, vq.smooth.clone(), 1))
    return (kq, vq), other


def _pool_tensors(kv):
    k, v = kv
    return (k.layer_q, k.layer_scale) if isinstance(k, ti.Int8Pages) else (k, v)


@pytest.mark.parametrize("B,n,kind", [(4, 1, "bf16"), (2, 16, "bf16"), (1, 64, "bf16"), (4, 1, "int8"),
                                      (4, 1, "fp32"), (2, 16, "fp32")])
def test_runner_step_graph_with_block_table_rewrites(gpu, B, n, kind):
    """The reference's runner step (src/model/decoder.jl:137-196, test/engine/runner.jl:
    16-33): pages are reserved from a shared BlockManager as the sequences grow, so new
    page ids appear in the block tables step by step. Each step's host staging (zero-padded
    block tables, positions, slots) is copied to a device buffer; the captured graph copies
    it into the tables, positions and slots the kernels read (device-to-device copies
    recorded before the launches), writes the step's K/V through attention_inputs_ and
    runs attention. Every replay must equal an eager step on a second cache, bit for bit,
    and its attention must match the oracle."""
    Hq, Hk, D, P = 32, 8, 128, 16
    torch.manual_seed(1000 * B + n)
    steps = {1: 24, 16: 5, 64: 4}[n]
    lens0 = [13 + 29 * b for b in range(B)]
    pages = sum(-(-(L + steps * n) // P) for L in lens0) + 8
    width = max(-(-(L + steps * n) // P) for L in lens0) + 2
    bm = ti.BlockManager(pages, P)
    seqs = [ti.Sequence() for _ in range(B)]
    for b, L in enumerate(lens0):
        ti.reserve(bm, seqs[b], L)
        seqs[b].tokens.extend([0] * L)
    cache, eager = _pools(kind, pages, Hk, P, D)
    dt = torch.float32 if kind == "fp32" else torch.bfloat16
    table = ti.RotaryTable.build(D, 2048, 1e6, dt)
    T = B * n
    qkv = torch.empty((T, (Hq + 2 * Hk) * D), device="cuda", dtype=dt)
    q = torch.empty((T, Hq, D), device="cuda", dtype=dt)
    out = torch.empty_like(q)
    staging = torch.zeros(2 * T + B * width, dtype=torch.int32, device="cuda")
    pos = torch.zeros(T, dtype=torch.int32, device="cuda")
    slots = torch.zeros(T, dtype=torch.int32, device="cuda")
    bts = torch.zeros((B, width), dtype=torch.int32, device="cuda")
    ws = ti.attention_workspace(BE, q, cache[0], num_seqs=B, max_query_len=n)
    scale = 1 / math.sqrt(D)

    def prepare():
        """reserve + host staging (prepare_step!): one copy to the device."""
        h = torch.zeros(2 * T + B * width, dtype=torch.int32)
        for b, s in enumerate(seqs):
            start = len(s)
            ti.reserve(bm, s, n)
            h[b * n:(b + 1) * n] = torch.arange(start, start + n, dtype=torch.int32)
            h[T + b * n:T + (b + 1) * n] = torch.tensor(ti.slots(bm, s, start, n), dtype=torch.int32)
            h[2 * T + b * width:2 * T + b * width + len(s.block_table)] = torch.tensor(s.block_table,
                                                                                    dtype=torch.int32)
        staging.copy_(h.cuda())

    def step(kv, o):
        pos.copy_(staging[:T])
        slots.copy_(staging[T:2 * T])
        bts.copy_(staging[2 * T:].view(B, width))
        ti.attention_inputs_(BE, q, kv[0], kv[1], qkv, None, None, table, pos, slots, 1e-6)
        ti.paged_attention_(BE, o, ws, q, kv[0], kv[1], bts, pos, scale, True, max_query_len=n)

    qkv.normal_()
    prepare()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(cache, out)
    for s in seqs:
        s.tokens.extend([0] * n)                     # the reservation above was for step 0
    ref_out = torch.empty_like(q)
    grew = 0
    for it in range(steps):
        if it > 0:
            old = [len(s.block_table) for s in seqs]
            qkv.normal_()
            prepare()
            grew += sum(len(s.block_table) - o for s, o in zip(seqs, old))
            for s in seqs:
                s.tokens.extend([0] * n)
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        step(eager, ref_out)                         # the same step, eager, on the second cache
        torch.cuda.synchronize()
        assert torch.equal(got, ref_out), f"replay {it} attention differs from eager"
        for a, e in zip(_pool_tensors(cache), _pool_tensors(eager)):
            assert torch.equal(a, e), f"replay {it} cache differs from eager"
        if kind != "int8":
            # sequence 0's attention against the oracle over the cache the step wrote
            s = seqs[0]
            start = len(s) - n
            kp, vp = cache[0].float().cpu().numpy(), cache[1].float().cpu().numpy()
            ref = orc.attention(q[:n].float().cpu().numpy(), np.array(s.block_table, np.int32), start,
                                scale, True, kp, vp)
            err = float(np.max(np.abs(ref - got[:n].float().cpu().numpy())))
            assert err <= (2e-2 if kind == "bf16" else 1e-4), f"replay {it}: max abs err {err} vs oracle"
    assert grew > 0, "no step reserved a new page"
