"""Graph capture: attention and the fused KV write recorded once in a HIP graph stay
valid as the sequences grow, because the kernels read the step's positions and block
tables from device memory and their launch shapes depend only on host shapes
(src/ops/tile/attention.jl:14-17; test/engine/runner.jl:16-33 checks replay == eager).
Each replay is compared with an eager call on the same state, with eager work and
synchronizations between replays."""
import math

import pytest
import torch

import tileinfer_hip as ti

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


@pytest.mark.parametrize("pp", [None, "1"])
def test_prefill_and_kv_write_graph(gpu, pp, monkeypatch):
    """pp = "1": the 8-wave ping-pong prefill kernel (TI_PREFILL_PP=1), else AUTO's choice."""
    if pp is not None:
        monkeypatch.setenv("TI_PREFILL_PP", pp)
    Hq, Hk, D, P, n = 32, 8, 128, 16, 128
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
        ti.attention_(BE, out, None, q, k, v, bt, pos, 1 / math.sqrt(D))

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
