"""The 8-wave ping-pong prefill kernel (pa_prefill_pp.hip) against the oracle.

AUTO takes it only for large grids (a 4096-token prefill); TI_PATH_PREFILL_PINGPONG pins it for
every shape it accepts (bf16 dense cache, head_dim 128, power-of-two pages of >= 16
tokens, heads per KV head dividing 256), so these cases cover its masks, ragged last
tiles, key splits, the prologue with one or two key tiles and batched calls. Tolerance:
max abs <= 2e-2 against the double-accumulated oracle, and <= 5 bf16 ulps (the
reference's bound, test/ops/tile.jl:237-259) up to 512 query tokens, the longest step its
cases hold: longer causal prefills round more probabilities to bf16 and both prefill
kernels reach 5.0-5.7 ulps at 1024-2048 tokens (same elements, same errors)."""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import block_table, randn, rng, ulps
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()


# Every call pins the ping-pong kernel (TI_PATH_PREFILL_PINGPONG).
PP = ti.TI_PATH_PREFILL_PINGPONG


# (heads, kv_heads, page_size, start, n, causal, block-table width in pages or 0)
CASES = [(32, 8, 16, 0, 1, True, 0),          # one key tile, one query
         (32, 8, 16, 0, 31, True, 0),         # one partial key tile
         (32, 8, 16, 0, 33, True, 0),         # two key tiles, ragged
         (32, 8, 16, 5, 70, True, 0),         # start inside the first tile
         (32, 8, 16, 0, 512, True, 0),        # the BASELINE prefill, split keys
         (32, 8, 16, 1024, 512, True, 0),     # chunked prefill on a cached prefix
         (32, 8, 64, 200, 300, True, 0),      # 64-token pages
         (16, 8, 64, 0, 512, True, 0),        # G = 2 (128 positions per work-group)
         (8, 8, 16, 77, 300, True, 0),        # G = 1
         (64, 8, 32, 120, 40, True, 0),       # G = 8
         (32, 8, 16, 1000, 16, False, 0),     # non-causal
         (32, 8, 16, 300, 250, False, 0),     # non-causal, ragged
         (32, 8, 16, 0, 16, True, 512),       # wide block table: most splits empty
         (16, 4, 16, 0, 2048, True, 0)]       # a long prefill (128 work-groups)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_prefill_pp(gpu, case):
    H, KVH, P, start, n, causal, width = case
    D = 128
    g = rng(4400 + start + n + H)
    L = start + n
    pages = -(-L // P) + 2
    bt = block_table(g, L, P, pages)
    if width:
        wide = np.zeros(width, np.int32)
        wide[:len(bt)] = bt
        bt = wide
    q = randn(g, n, H, D, bf16=True)
    kp, vp = randn(g, pages, KVH, P, D, bf16=True), randn(g, pages, KVH, P, D, bf16=True)
    ref = orc.attention(q, bt, start, 1 / math.sqrt(D), causal, kp, vp)
    qd = torch.from_numpy(q).bfloat16().cuda()
    kd, vd = torch.from_numpy(kp).bfloat16().cuda(), torch.from_numpy(vp).bfloat16().cuda()
    pos = torch.arange(start, L, dtype=torch.int32, device="cuda")
    btd = torch.from_numpy(bt).cuda()
    print(f"case {case}", flush=True)
    for with_ws in (True, False):
        ws = ti.attention_workspace(BE, qd, kd, path=PP) if with_ws else None
        out = torch.full_like(qd, float("nan"))
        ti.attention_(BE, out, ws, qd, kd, vd, btd, pos, 1 / math.sqrt(D), causal, path=PP)
        got = out.float().cpu().numpy()
        err = float(np.max(np.abs(ref - got)))
        assert err <= 2e-2, f"workspace {with_ws}: max abs err {err}"
        if n <= 512:
            assert ulps(ref, got) <= 5


def test_prefill_pp_nan_pages(gpu):
    """Keys past the step's last key in its last tile read allocated pool rows that may
    hold any bits: NaN there must not reach the output (their values are zeroed)."""
    H, KVH, P, D, start, n = 32, 8, 16, 128, 0, 40
    g = rng(4500)
    pages = 6
    bt = block_table(g, start + n, P, pages)
    q = randn(g, n, H, D, bf16=True)
    kp, vp = randn(g, pages, KVH, P, D, bf16=True), randn(g, pages, KVH, P, D, bf16=True)
    ref = orc.attention(q, bt, start, 1 / math.sqrt(D), True, kp, vp)
    kd, vd = torch.from_numpy(kp).bfloat16().cuda(), torch.from_numpy(vp).bfloat16().cuda()
    last = int(bt[(start + n - 1) // P]) - 1
    off = (start + n) % P
    kd[last, :, off:, :] = float("nan")
    vd[last, :, off:, :] = float("nan")
    qd = torch.from_numpy(q).bfloat16().cuda()
    out = torch.empty_like(qd)
    ti.attention_(BE, out, None, qd, kd, vd, torch.from_numpy(bt).cuda(),
                  torch.arange(start, start + n, dtype=torch.int32, device="cuda"), 1 / math.sqrt(D), True,
                  path=PP)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert float(np.max(np.abs(ref - got))) <= 2e-2


def test_prefill_pp_batched(gpu):
    """Ragged batch (one empty sequence) in one call."""
    g = rng(4600)
    D, H, KVH, P = 128, 32, 8, 16
    starts, counts = [700, 0, 33, 2000, 5], [40, 130, 0, 1, 300]
    nmax = max(counts)
    pages = sum(-(-(s + n) // P) for s, n in zip(starts, counts)) + 3
    perm = g.permutation(pages) + 1
    width = 160
    bts = np.zeros((len(starts), width), np.int32)
    off = 0
    for b, (s, n) in enumerate(zip(starts, counts)):
        used = -(-(s + n) // P)
        bts[b, :used] = perm[off:off + used]
        off += used
    kp, vp = randn(g, pages, KVH, P, D, bf16=True), randn(g, pages, KVH, P, D, bf16=True)
    q = randn(g, sum(counts), H, D, bf16=True)
    qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    positions = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, counts)]).astype(np.int32)
    qd = torch.from_numpy(q).bfloat16().cuda()
    out = torch.zeros_like(qd)
    kd, vd = torch.from_numpy(kp).bfloat16().cuda(), torch.from_numpy(vp).bfloat16().cuda()
    ws = ti.attention_workspace(BE, qd, kd, num_seqs=len(starts), max_query_len=nmax, path=PP)
    ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(),
                        torch.from_numpy(positions).cuda(), 1 / math.sqrt(D), True,
                        query_start_loc=torch.from_numpy(qsl).cuda(), max_query_len=nmax,
                        path=PP)
    got = out.float().cpu().numpy()
    for b, (s, n) in enumerate(zip(starts, counts)):
        if n == 0:
            continue
        ref = orc.attention(q[qsl[b]:qsl[b + 1]], bts[b], s, 1 / math.sqrt(D), True, kp, vp)
        assert float(np.max(np.abs(ref - got[qsl[b]:qsl[b + 1]]))) <= 2e-2
