"""Paged attention on the GPU (split-KV decode, MFMA prefill, fp32 path) vs the oracle.

Tolerances: max abs error <= 1e-4 for fp32 and <= 2e-2 for bf16 and
INT8-KV, against the double-accumulated oracle; also the reference's own ulp bounds
(test/ops/tile.jl:237-259: bf16 <= 5 ulps of exact attention, INT8 <= 14 ulps of exact
attention over the dequantized cache, whole-op relative L2 < 0.02 vs unquantized).
"""
import math

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import block_table, randn, rng, smoothing, ulps
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()
TOL = {False: 1e-4, True: 2e-2}

# (head_dim, heads, kv_heads, page_size, start, n, causal): test/ops/tile.jl:217-222.
REF_CASES = [(128, 16, 8, 64, 1023, 1, True), (128, 16, 8, 64, 63, 2, True),
             (128, 16, 8, 64, 100, 8, True), (128, 16, 8, 64, 0, 512, True),
             (128, 16, 8, 64, 200, 300, True), (128, 32, 8, 64, 700, 3, True),
             (64, 12, 4, 16, 40, 5, True), (128, 32, 8, 64, 950, 16, True),
             (128, 32, 8, 64, 63, 12, True), (128, 32, 8, 64, 1000, 16, False),
             (128, 32, 8, 64, 300, 30, False)]
# Shapes the BASELINE configs add: 16-token pages, tiny pages, page-straddling steps.
EXTRA_CASES = [(128, 32, 8, 16, 1500, 1, True), (128, 32, 8, 16, 4000, 16, True),
               (128, 32, 8, 4, 37, 9, True), (128, 8, 8, 16, 77, 3, True),
               (128, 64, 8, 16, 120, 8, True), (64, 8, 2, 32, 0, 1, True),
               (128, 32, 8, 16, 1024, 512, True), (128, 16, 8, 16, 0, 100, False),
               # 48-token pages: whole 16-key tiles per page, but not a power of two
               (128, 32, 8, 48, 700, 5, True), (128, 16, 8, 48, 100, 200, True)]


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()


def make_case(case, bf16, seed):
    D, H, KVH, P, start, n, causal = case
    g = rng(seed)
    L = start + n
    pages = -(-L // P) + 2
    bt = block_table(g, L, P, pages)
    q = randn(g, n, H, D, bf16=bf16)
    kp, vp = randn(g, pages, KVH, P, D, bf16=bf16), randn(g, pages, KVH, P, D, bf16=bf16)
    return dict(q=q, kp=kp, vp=vp, bt=bt, start=start, n=n, causal=causal, D=D, g=g)


def run_gpu(c, dtype, path=ti.TI_PATH_AUTO, k=None, v=None):
    q = dev(c["q"], dtype)
    k = dev(c["kp"], dtype) if k is None else k
    v = dev(c["vp"], dtype) if v is None else v
    out = torch.empty_like(q)
    ws = ti.attention_workspace(BE, q, k, path=path)
    pos = torch.arange(c["start"], c["start"] + c["n"], dtype=torch.int32, device="cuda")
    ti.attention_(BE, out, ws, q, k, v, torch.from_numpy(c["bt"]).cuda(), pos,
                  1 / math.sqrt(c["D"]), c["causal"], path=path)
    return out.float().cpu().numpy()


def exact(c, **kw):
    if "layer_q" in kw:
        return orc.attention(c["q"], c["bt"], c["start"], 1 / math.sqrt(c["D"]), c["causal"], **kw)
    return orc.attention(c["q"], c["bt"], c["start"], 1 / math.sqrt(c["D"]), c["causal"],
                         kw.get("kp", c["kp"]), kw.get("vp", c["vp"]))


def check(ref, got, bf16):
    err = float(np.max(np.abs(ref - got)))
    assert err <= TOL[bf16], f"max abs err {err}"
    if bf16:
        u = ulps(ref, got)
        assert u <= 5, f"{u} ulps"
    else:
        # the reference's Float32 bound, isapprox(y, exact; rtol = 1e-5) (test/ops/tile.jl:240)
        d = float(np.linalg.norm((ref - got).astype(np.float64)))
        nrm = max(float(np.linalg.norm(ref.astype(np.float64))), float(np.linalg.norm(got.astype(np.float64))))
        assert d <= 1e-5 * nrm, f"relative norm err {d / nrm}"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", REF_CASES + EXTRA_CASES, ids=str)
def test_attention(gpu, case, bf16):
    c = make_case(case, bf16, seed=hash(case) % 10000 + bf16)
    dtype = torch.bfloat16 if bf16 else torch.float32
    ref = exact(c)
    check(ref, run_gpu(c, dtype), bf16)
    if bf16:
        D, H, KVH, P, start, n, causal = case
        # both MFMA kernels wherever their shape limits allow
        if (H // KVH) * n <= 64:
            check(ref, run_gpu(c, dtype, ti.TI_PATH_DECODE), True)
        if n <= 16:
            check(ref, run_gpu(c, dtype, ti.TI_PATH_PREFILL), True)


# The largest shapes the paths take: a 128k-token context (8192 pages of 16), one KV head
# shared by 64 query heads (G = 64: 64 packed rows on the decode kernel, 192 on the
# prefill kernel), head_dim 64 at G = 64, and a 16-query verify step on a 64k context.
LIMIT_CASES = [(128, 8, 2, 16, 131071, 1, True), (128, 64, 1, 16, 5000, 1, True),
               (128, 64, 1, 16, 3000, 3, True), (64, 64, 1, 16, 2000, 1, True),
               (128, 8, 2, 16, 65543, 16, True)]


@pytest.mark.parametrize("case", LIMIT_CASES, ids=str)
def test_attention_limits(gpu, case):
    D, H, KVH, P, start, n, causal = case
    print(f"case {case}", flush=True)
    c = make_case(case, True, seed=hash(case) % 10000 + 11)
    ref = exact(c)
    check(ref, run_gpu(c, torch.bfloat16), True)
    if (H // KVH) * n <= 64:
        check(ref, run_gpu(c, torch.bfloat16, ti.TI_PATH_DECODE), True)
    check(ref, run_gpu(c, torch.bfloat16, ti.TI_PATH_PREFILL), True)


@pytest.mark.parametrize("case", [LIMIT_CASES[0], LIMIT_CASES[1], LIMIT_CASES[2], LIMIT_CASES[4]], ids=str)
def test_attention_limits_fp32(gpu, case):
    """The fp32 matrix-core kernel at the largest shapes: a 128k-token context (32 key splits),
    64 query heads per KV head (4 q-tiles per token), and a 16-query step on a 64k context."""
    print(f"case {case}", flush=True)
    c = make_case(case, False, seed=hash(case) % 10000 + 13)
    check(exact(c), run_gpu(c, torch.float32), False)


@pytest.mark.parametrize("case", REF_CASES + EXTRA_CASES[:5], ids=str)
def test_attention_int8(gpu, case):
    """INT8 cache (bf16 activations), keys scaled like the smoothing factors."""
    D, H, KVH, P, start, n, causal = case
    c = make_case(case, True, seed=hash(case) % 10000 + 7)
    g = c["g"]
    cs = smoothing(g, D)
    pages = c["kp"].shape[0]
    k_src = orc.bf16_round(c["kp"] * orc.bf16_round(cs)[None, None, None, :])
    kq, vq = ti.int8_kv_pools(D, P, KVH, pages, key_smoothing=torch.from_numpy(cs))
    # every position of the pool, through the GPU store (bit-exact vs the oracle's)
    kk = dev(k_src.transpose(0, 2, 1, 3).reshape(-1, KVH, D), torch.bfloat16)
    vv = dev(c["vp"].transpose(0, 2, 1, 3).reshape(-1, KVH, D), torch.bfloat16)
    ti.store_kv_(BE, kq, vq, kk, vv, torch.arange(1, P * pages + 1, dtype=torch.int32, device="cuda"))
    lq, ls = kq.layer_q.cpu().numpy(), kq.layer_scale.cpu().numpy()
    ref8 = exact(c, layer_q=lq, layer_scale=ls, smooth=cs)
    paths = [ti.TI_PATH_AUTO]
    if (H // KVH) * n <= 64 and n > 16:
        paths.append(ti.TI_PATH_DECODE)
    if n <= 16:
        paths.append(ti.TI_PATH_PREFILL)
    for path in paths:
        y8 = run_gpu(c, torch.bfloat16, path, kq, vq)
        assert float(np.max(np.abs(ref8 - y8))) <= 2e-2
        assert ulps(ref8, y8) <= 14
        src = exact(c, kp=k_src, vp=c["vp"])
        rel = math.sqrt(float(np.sum((y8 - src) ** 2)) / float(np.sum(src ** 2)))
        assert rel < 0.02



# configs[2]'s shapes (and a 64-token-page and a 1024-token case) on an INT8 cache: AUTO
# takes the 16-row paired kernel, its tiles staged through registers as bf16.
INT8_PAIRED_CASES = [(128, 32, 8, 16, 0, 512, True), (128, 32, 8, 16, 1024, 512, True),
                     (128, 16, 8, 64, 0, 512, True), (128, 32, 8, 16, 0, 1024, True)]


@pytest.mark.parametrize("case", INT8_PAIRED_CASES, ids=str)
def test_attention_int8_paired16(gpu, case):
    """INT8 cache through TI_PATH_PREFILL_PAIRED16 (AUTO's pick here) against the oracle over
    the dequantized cache, with the reference's INT8 bounds (test/ops/tile.jl:237-259)."""
    D, H, KVH, P, start, n, causal = case
    c = make_case(case, True, seed=hash(case) % 10000 + 11)
    g = c["g"]
    cs = smoothing(g, D)
    pages = c["kp"].shape[0]
    k_src = orc.bf16_round(c["kp"] * orc.bf16_round(cs)[None, None, None, :])
    kq, vq = ti.int8_kv_pools(D, P, KVH, pages, key_smoothing=torch.from_numpy(cs))
    kk = dev(k_src.transpose(0, 2, 1, 3).reshape(-1, KVH, D), torch.bfloat16)
    vv = dev(c["vp"].transpose(0, 2, 1, 3).reshape(-1, KVH, D), torch.bfloat16)
    ti.store_kv_(BE, kq, vq, kk, vv, torch.arange(1, P * pages + 1, dtype=torch.int32, device="cuda"))
    lq, ls = kq.layer_q.cpu().numpy(), kq.layer_scale.cpu().numpy()
    ref8 = exact(c, layer_q=lq, layer_scale=ls, smooth=cs)
    y16 = run_gpu(c, torch.bfloat16, ti.TI_PATH_PREFILL_PAIRED16, kq, vq)
    assert np.array_equal(y16, run_gpu(c, torch.bfloat16, ti.TI_PATH_AUTO, kq, vq))
    assert float(np.max(np.abs(ref8 - y16))) <= 2e-2
    if n <= 512:
        assert ulps(ref8, y16) <= 14
    src = exact(c, kp=k_src, vp=c["vp"])
    assert math.sqrt(float(np.sum((y16 - src) ** 2)) / float(np.sum(src ** 2))) < 0.02

@pytest.mark.parametrize("path", [ti.TI_PATH_AUTO, ti.TI_PATH_PREFILL, ti.TI_PATH_PREFILL_PAIRED16])
def test_batched_ragged(gpu, path):
    """B sequences of different lengths and query counts (one empty) in one call. The
    paired 16-row kernel runs its work-groups past a short sequence's queries through to the
    end (no early exit): they must write nothing, and every other row must match."""
    g = rng(900 + path)
    D, H, KVH, P = 128, 32, 8, 16
    starts = [700, 0, 33, 2000, 5]
    counts = [3, 16, 0, 1, 9] if path == ti.TI_PATH_AUTO else [40, 130, 0, 1, 64]
    print(f"batched ragged path {path} counts {counts}", flush=True)
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
    T = sum(counts)
    q = randn(g, T, H, D, bf16=True)
    qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    positions = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, counts)]).astype(np.int32)
    qd = dev(q, torch.bfloat16)
    out = torch.full_like(qd, float("nan"))
    kd, vd = dev(kp, torch.bfloat16), dev(vp, torch.bfloat16)
    ws = ti.attention_workspace(BE, qd, kd, num_seqs=len(starts), max_query_len=nmax, path=path)
    ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(),
                        torch.from_numpy(positions).cuda(), 1 / math.sqrt(D), True,
                        query_start_loc=torch.from_numpy(qsl).cuda(), max_query_len=nmax, path=path)
    got = out.float().cpu().numpy()
    for b, (s, n) in enumerate(zip(starts, counts)):
        if n == 0:
            continue
        ref = orc.attention(q[qsl[b]:qsl[b + 1]], bts[b], s, 1 / math.sqrt(D), True, kp, vp)
        check(ref, got[qsl[b]:qsl[b + 1]], True)


def _run_batch(g, starts, counts, use_qsl, KVH=8, H=32, D=128, P=16, bf16=True, causal=True):
    """One call over sequences at `starts` with `counts` query tokens each; returns
    (q, kp, vp, bts, qsl, out). Without `use_qsl` every sequence has max(counts) tokens."""
    nmax = max(counts)
    pages = sum(-(-(s + n) // P) for s, n in zip(starts, counts)) + 3
    perm = g.permutation(pages) + 1
    width = max(-(-(s + n) // P) for s, n in zip(starts, counts)) + 2
    bts = np.zeros((len(starts), width), np.int32)
    off = 0
    for b, (s, n) in enumerate(zip(starts, counts)):
        used = -(-(s + n) // P)
        bts[b, :used] = perm[off:off + used]
        off += used
    kp, vp = randn(g, pages, KVH, P, D, bf16=bf16), randn(g, pages, KVH, P, D, bf16=bf16)
    q = randn(g, sum(counts), H, D, bf16=bf16)
    qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    positions = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, counts)]).astype(np.int32)
    dt = torch.bfloat16 if bf16 else torch.float32
    qd = dev(q, dt)
    out = torch.zeros_like(qd)
    kd, vd = dev(kp, dt), dev(vp, dt)
    ws = ti.attention_workspace(BE, qd, kd, num_seqs=len(starts), max_query_len=nmax)
    ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(),
                        torch.from_numpy(positions).cuda(), 1 / math.sqrt(D), causal,
                        query_start_loc=torch.from_numpy(qsl).cuda() if use_qsl else None,
                        max_query_len=nmax)
    return q, kp, vp, bts, qsl, out.float().cpu().numpy()


# Split batches of 4-64 sequences with at least 4 splits each share their work-groups out
# by length: one long sequence among short ones (most work-groups on one sequence), an
# empty sequence, 64 sequences (the largest such batch) and 65 (one split count for all),
# multi-token steps through query_start_loc and through the uniform layout.
FLAT_CASES = {
    "one_long": ([8000, 15, 16, 17], [1, 1, 1, 1], True),
    "empty_and_multi": ([3000, 700, 0, 40], [3, 0, 5, 8], True),
    "b64": (None, 64, True),     # with 1 KV head (64 pairs: 4 splits each)
    "b65": (None, 65, True),
    "uniform_layout": ([100, 5000, 2000, 64, 900, 1], [2, 2, 2, 2, 2, 2], False),
}


@pytest.mark.parametrize("name", list(FLAT_CASES))
def test_split_shares_by_length(gpu, name):
    g = rng(950 + list(FLAT_CASES).index(name))
    starts, counts, use_qsl = FLAT_CASES[name]
    if starts is None:
        B = counts
        starts = [int(x) for x in g.integers(0, 3000, size=B)]
        counts = [1] * B
        q, kp, vp, bts, qsl, got = _run_batch(g, starts, counts, use_qsl, KVH=1, H=4)
    else:
        q, kp, vp, bts, qsl, got = _run_batch(g, starts, counts, use_qsl)
    nmax = max(counts)
    for b, (s, n) in enumerate(zip(starts, counts)):
        if n == 0:
            continue
        lo = qsl[b] if use_qsl else b * nmax
        ref = orc.attention(q[lo:lo + n], bts[b], s, 1 / math.sqrt(128), True, kp, vp)
        check(ref, got[lo:lo + n], True)


# fp32 batches on the matrix-core decode kernel (dense pools, 2^k >= 16-token pages, at most
# 16 packed rows): contexts either side of the 16-key tile and of the 4-tile minimum split
# (one split alone writes the output; longer ones merge only the splits that held keys), 16
# packed rows (G = 2 x 8 tokens), G = 8 x 2 tokens in the uniform layout, head_dim 64 on
# 64-token pages, a non-causal multi-token step, and empty sequences (the last one too).
# name: (starts, counts, use_qsl, dict(KVH, H, D, P, causal))
F32_BATCHES = {
    "split_edges": ([0, 14, 15, 63, 64, 1000, 4100], [1] * 7, True, dict(KVH=8, H=16)),
    "rows16": ([30, 2000, 500], [8, 8, 3], True, dict(KVH=8, H=16)),
    "g8_uniform": ([3000, 17], [2, 2], False, dict(KVH=4, H=32)),
    "d64_p64": ([5000, 60, 191], [1, 1, 1], True, dict(KVH=2, H=8, D=64, P=64)),
    "non_causal": ([700, 33], [4, 4], True, dict(KVH=8, H=32, causal=False)),
    "empty_sequences": ([0, 900, 0, 60], [0, 3, 1, 0], True, dict(KVH=8, H=16)),
}


@pytest.mark.parametrize("name", list(F32_BATCHES))
def test_fp32_decode_batches(gpu, name):
    g = rng(990 + list(F32_BATCHES).index(name))
    starts, counts, use_qsl, kw = F32_BATCHES[name]
    causal = kw.get("causal", True)
    q, kp, vp, bts, qsl, got = _run_batch(g, starts, counts, use_qsl, bf16=False, **kw)
    nmax = max(counts)
    D = kw.get("D", 128)
    for b, (s, n) in enumerate(zip(starts, counts)):
        if n == 0:
            continue
        lo = qsl[b] if use_qsl else b * nmax
        ref = orc.attention(q[lo:lo + n], bts[b], s, 1 / math.sqrt(D), causal, kp, vp)
        check(ref, got[lo:lo + n], False)


# (head_dim, heads, kv_heads, page_size, start, n, causal, block-table width in pages)
SPLIT_CASES = [(128, 32, 8, 16, 0, 16, True, 512),      # most splits hold no keys
               (128, 32, 8, 16, 2048, 16, True, 160),   # the verify shape on a long prefix
               (128, 32, 8, 16, 1500, 40, False, 160),  # non-causal, ragged last tile
               (64, 12, 4, 16, 900, 12, True, 128)]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_prefill_key_splits(gpu, case):
    """The prefill kernel with its keys split across work-groups (partials merged by the
    combine kernel), through AUTO and the forced prefill path; without a workspace the
    prefill path runs unsplit (the reference runs its prefill kernel exactly when
    attention! gets no workspace, src/ops/tile/attention.jl:354-366)."""
    D, H, KVH, P, start, n, causal, width = case
    c = make_case((D, H, KVH, P, start, n, causal), True, 1200 + start + n)
    used = -(-(start + n) // P)
    bt = np.zeros(width, np.int32)
    bt[:used] = c["bt"][:used]
    c["bt"] = bt
    ref = exact(c)
    q = dev(c["q"], torch.bfloat16)
    k, v = dev(c["kp"], torch.bfloat16), dev(c["vp"], torch.bfloat16)
    pos = torch.arange(start, start + n, dtype=torch.int32, device="cuda")
    btd = torch.from_numpy(bt).cuda()
    assert ti.workspace_bytes(q, k, path=ti.TI_PATH_PREFILL) > 0     # this shape splits
    for path, with_ws in ((ti.TI_PATH_AUTO, True), (ti.TI_PATH_PREFILL, True), (ti.TI_PATH_PREFILL, False)):
        ws = ti.attention_workspace(BE, q, k, path=path) if with_ws else None
        out = torch.full_like(q, float("nan"))
        ti.attention_(BE, out, ws, q, k, v, btd, pos, 1 / math.sqrt(D), causal, path=path)
        check(ref, out.float().cpu().numpy(), True)


def test_workspace_errors(gpu):
    c = make_case((128, 16, 8, 16, 100, 1, True), True, 1)
    q = dev(c["q"], torch.bfloat16)
    k = dev(c["kp"], torch.bfloat16)
    out = torch.empty_like(q)
    pos = torch.tensor([100], dtype=torch.int32, device="cuda")
    bt = torch.from_numpy(c["bt"]).cuda()
    with pytest.raises(ti.WorkspaceError):
        ti.attention_(BE, out, None, q, k, k, bt, pos, 0.1)
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(ti.WorkspaceError):
        ti.attention_(BE, out, small, q, k, k, bt, pos, 0.1)


# (head_dim, heads, kv_heads, page_size, start, n, causal, batch)
LOADER_CASES = [(128, 32, 8, 16, 0, 512, True, 1), (128, 32, 8, 16, 1024, 512, True, 1),
                (128, 32, 8, 16, 4096, 16, True, 4), (128, 32, 8, 64, 300, 250, False, 1),
                (128, 24, 8, 32, 77, 301, True, 1), (128, 32, 8, 16, 0, 2048, True, 1),
                # odd q-tile counts: the paired kernel's middle q-tile pairs with itself
                (128, 32, 8, 16, 0, 200, True, 2), (128, 16, 8, 16, 37, 100, True, 3)]


@pytest.mark.parametrize("case", LOADER_CASES, ids=str)
def test_prefill_tile_loaders_bit_identical(gpu, case):
    """The four-wave prefill kernel's two tile loaders (register-staged loads + LDS stores,
    TI_PATH_PREFILL_STAGED; direct global -> LDS loads into swizzled rows,
    TI_PATH_PREFILL_DIRECT; and the same with paired heavy / light q-tiles,
    TI_PATH_PREFILL_PAIRED, where causal shapes allow it) feed
    the same operands to the same arithmetic: outputs must be bit-identical, and within
    the tolerances of the oracle."""
    D, H, KVH, P, start, n, causal, B = case
    g = rng(1300 + n + start + B)
    L = start + n
    per = -(-L // P)
    pages = B * per + 2
    perm = g.permutation(pages) + 1
    bts = np.zeros((B, per + 3), np.int32)
    for b in range(B):
        bts[b, :per] = perm[b * per:(b + 1) * per]
    q = randn(g, B * n, H, D, bf16=True)
    kp, vp = randn(g, pages, KVH, P, D, bf16=True), randn(g, pages, KVH, P, D, bf16=True)
    qd = dev(q, torch.bfloat16)
    kd, vd = dev(kp, torch.bfloat16), dev(vp, torch.bfloat16)
    pos = torch.arange(start, L, dtype=torch.int32, device="cuda").repeat(B)
    outs = []
    for path in (ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT, ti.TI_PATH_PREFILL_PAIRED):
        ws = ti.attention_workspace(BE, qd, kd, num_seqs=B, max_query_len=n, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(), pos, 1 / math.sqrt(D),
                            causal, max_query_len=n, path=path)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(outs[1], outs[2])
    got = outs[2].float().cpu().numpy()
    for b in range(B):
        ref = orc.attention(q[b * n:(b + 1) * n], bts[b], start, 1 / math.sqrt(D), causal, kp, vp)
        assert float(np.max(np.abs(ref - got[b * n:(b + 1) * n]))) <= 2e-2



# Shapes on which AUTO takes the 16-row paired kernel: causal, unsplit, at most 512 pairs of
# q-tiles (start, n, B); the other LOADER_CASES pin it where AUTO picks another kernel.
PAIRED16_AUTO = {(0, 512, 1), (1024, 512, 1), (0, 200, 2), (0, 1024, 1)}


@pytest.mark.parametrize("case", LOADER_CASES + [(128, 32, 8, 16, 0, 1024, True, 1)], ids=str)
def test_prefill_paired16(gpu, case):
    """The paired work-groups on 16-row waves (TI_PATH_PREFILL_PAIRED16, AUTO's pick for
    causal steps of up to 512 pairs of q-tiles) against the oracle and the 32-row paired
    kernel: the same attention with a different MFMA shape (16x16x32 instead of 32x32x16),
    so equal within the tolerances, not bit for bit. The reference's ulp bound is stated for
    its shapes (n <= 512); at 1024 new tokens every prefill variant gives the same 5.6 ulps
    on this seed (the bf16 probabilities of long causal rows), so there the absolute
    tolerance applies alone."""
    D, H, KVH, P, start, n, causal, B = case
    g = rng(1400 + n + start + B)
    L = start + n
    per = -(-L // P)
    pages = B * per + 2
    perm = g.permutation(pages) + 1
    bts = np.zeros((B, per + 3), np.int32)
    for b in range(B):
        bts[b, :per] = perm[b * per:(b + 1) * per]
    q = randn(g, B * n, H, D, bf16=True)
    kp, vp = randn(g, pages, KVH, P, D, bf16=True), randn(g, pages, KVH, P, D, bf16=True)
    qd = dev(q, torch.bfloat16)
    kd, vd = dev(kp, torch.bfloat16), dev(vp, torch.bfloat16)
    pos = torch.arange(start, L, dtype=torch.int32, device="cuda").repeat(B)
    outs = []
    for path in (ti.TI_PATH_PREFILL_PAIRED16, ti.TI_PATH_PREFILL_PAIRED, ti.TI_PATH_AUTO):
        ws = ti.attention_workspace(BE, qd, kd, num_seqs=B, max_query_len=n, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(), pos, 1 / math.sqrt(D),
                            causal, max_query_len=n, path=path)
        outs.append(out)
    if (start, n, B) in PAIRED16_AUTO:
        assert torch.equal(outs[0], outs[2])             # AUTO takes it
    got = outs[0].float().cpu().numpy()
    assert float(np.max(np.abs(got - outs[1].float().cpu().numpy()))) <= 2e-2
    for b in range(B):
        ref = orc.attention(q[b * n:(b + 1) * n], bts[b], start, 1 / math.sqrt(D), causal, kp, vp)
        if n <= 512:
            check(ref, got[b * n:(b + 1) * n], True)
        else:
            assert float(np.max(np.abs(ref - got[b * n:(b + 1) * n]))) <= TOL[True]

# (head_dim, heads, kv_heads, page_size, start, n, table width in pages, dtype)
NARROW_CASES = [(128, 32, 8, 16, 200, 1, 5, "bf16"), (128, 32, 8, 16, 0, 300, 7, "bf16"),
                (128, 32, 8, 48, 100, 5, 1, "bf16"), (128, 32, 8, 16, 90, 16, 2, "bf16"),
                (64, 8, 2, 16, 70, 3, 2, "fp32")]


@pytest.mark.parametrize("case", NARROW_CASES, ids=str)
def test_block_table_narrower_than_context(gpu, case):
    """Out of contract: a block-table row holding fewer pages than the context needs. No
    access may leave the row (the table tensor here is exactly that row, so a read past it
    leaves the allocation); page indices past the row clamp to its last entry, so the
    result equals attention over a table whose missing entries repeat that last page."""
    D, H, KVH, P, start, n, width, kind = case
    bf16 = kind == "bf16"
    dtype = torch.bfloat16 if bf16 else torch.float32
    g = rng(2100 + start + n + width)
    L = start + n
    pages = width + 4
    bt = (g.permutation(pages)[:width] + 1).astype(np.int32)
    need = -(-L // P)
    bt_full = np.concatenate([bt, np.full(max(need - width, 0), bt[-1], np.int32)])
    q = randn(g, n, H, D, bf16=bf16)
    kp, vp = randn(g, pages, KVH, P, D, bf16=bf16), randn(g, pages, KVH, P, D, bf16=bf16)
    ref = orc.attention(q, bt_full, start, 1 / math.sqrt(D), True, kp, vp)
    qd, kd, vd = dev(q, dtype), dev(kp, dtype), dev(vp, dtype)
    btd = torch.from_numpy(bt).cuda()
    pos = torch.arange(start, L, dtype=torch.int32, device="cuda")
    paths = [ti.TI_PATH_AUTO]
    if bf16:
        paths += ([ti.TI_PATH_DECODE] if n <= 16 else []) + [
            ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT, ti.TI_PATH_PREFILL_PINGPONG]
    for path in paths:
        print(f"narrow table {case} path {path}", flush=True)
        ws = ti.attention_workspace(BE, qd, kd, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.attention_(BE, out, ws, qd, kd, vd, btd, pos, 1 / math.sqrt(D), True, path=path)
        err = float(np.max(np.abs(ref - out.float().cpu().numpy())))
        assert err <= TOL[bf16], f"path {path}: max abs err {err}"


@pytest.mark.parametrize("n", [1, 40])
def test_negative_position_reads_as_zero(gpu, n):
    """Out of contract: a negative first position. The kernels read it as 0 (no access
    before the block-table row or the pool), so the result is the start-0 attention."""
    D, H, KVH, P = 128, 32, 8, 16
    g = rng(2200 + n)
    bt = block_table(g, n, P, 8)
    q = randn(g, n, H, D, bf16=True)
    kp, vp = randn(g, 8, KVH, P, D, bf16=True), randn(g, 8, KVH, P, D, bf16=True)
    ref = orc.attention(q, bt, 0, 1 / math.sqrt(D), True, kp, vp)
    qd, kd, vd = dev(q, torch.bfloat16), dev(kp, torch.bfloat16), dev(vp, torch.bfloat16)
    # positions -50 .. : the kernels take the first; the step is n consecutive tokens
    pos = torch.arange(-50, -50 + n, dtype=torch.int32, device="cuda")
    for path in (ti.TI_PATH_AUTO, ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT):
        print(f"negative position n {n} path {path}", flush=True)
        ws = ti.attention_workspace(BE, qd, kd, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bt).cuda(), pos, 1 / math.sqrt(D), True,
                      path=path)
        err = float(np.max(np.abs(ref - out.float().cpu().numpy())))
        assert err <= 2e-2, f"path {path}: max abs err {err}"


@pytest.mark.parametrize("kind", ["bf16", "fp32"])
def test_sequences_longer_than_max_query_len(gpu, kind):
    """Out of contract: query_start_loc gives sequences more tokens than max_query_len. Every
    kernel takes a sequence's first max_query_len tokens (n_b capped, so no split partial or
    grid index leaves what the host sized): those rows equal the oracle's (causal), and the
    rows past them are never written (their NaN sentinels survive)."""
    bf16 = kind == "bf16"
    D, P = 128, 16
    H, KVH = (32, 8) if bf16 else (16, 8)
    nmax = 8
    starts, counts = [100, 40, 0, 300], [5, 12, 3, 20]
    g = rng(2300 + bf16)
    pages = sum(-(-(s + n) // P) for s, n in zip(starts, counts)) + 2
    perm = g.permutation(pages) + 1
    width = max(-(-(s + n) // P) for s, n in zip(starts, counts))
    bts = np.zeros((len(starts), width), np.int32)
    off = 0
    for b, (s, n) in enumerate(zip(starts, counts)):
        used = -(-(s + n) // P)
        bts[b, :used] = perm[off:off + used]
        off += used
    dt = torch.bfloat16 if bf16 else torch.float32
    kp, vp = randn(g, pages, KVH, P, D, bf16=bf16), randn(g, pages, KVH, P, D, bf16=bf16)
    q = randn(g, sum(counts), H, D, bf16=bf16)
    qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    positions = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, counts)]).astype(np.int32)
    qd, kd, vd = dev(q, dt), dev(kp, dt), dev(vp, dt)
    paths = [ti.TI_PATH_AUTO]
    if bf16:
        paths += [ti.TI_PATH_DECODE, ti.TI_PATH_PREFILL, ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT,
                  ti.TI_PATH_PREFILL_PAIRED, ti.TI_PATH_PREFILL_PAIRED16, ti.TI_PATH_PREFILL_PINGPONG]
    for path in paths:
        print(f"n_b > max_query_len, {kind} path {path}", flush=True)
        ws = ti.attention_workspace(BE, qd, kd, num_seqs=len(starts), max_query_len=nmax, path=path)
        out = torch.full_like(qd, float("nan"))
        ti.paged_attention_(BE, out, ws, qd, kd, vd, torch.from_numpy(bts).cuda(),
                            torch.from_numpy(positions).cuda(), 1 / math.sqrt(D), True,
                            query_start_loc=torch.from_numpy(qsl).cuda(), max_query_len=nmax, path=path)
        got = out.float().cpu().numpy()
        for b, (s, n) in enumerate(zip(starts, counts)):
            lo, k = qsl[b], min(n, nmax)
            ref = orc.attention(q[lo:lo + k], bts[b], s, 1 / math.sqrt(D), True, kp, vp)
            check(ref, got[lo:lo + k], bf16)
            assert np.isnan(got[lo + k:lo + n]).all(), f"path {path}: seq {b} rows past max_query_len written"
