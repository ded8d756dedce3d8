"""Benchmark of the paged flash-attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one call of the headline workload: Qwen3-4B-shaped bf16 paged decode attention
(32 query heads, 8 KV heads, head_dim 128, 16-token pages, shuffled block tables) over a
batch of 32 sequences of 4096 cached positions, inputs resident in HBM. Two copies of the
KV pools alternate between steps (2 x 537 MB, over 4x the 256 MB Infinity Cache) so every
step streams its pages from HBM. Prints ONE JSON line: decode GB/s as `value`, with the
decode figures at batch 1, 8 and 32 with context lengths drawn from [1024, 8192] (the
config as stated), prefill TFLOP/s, INT8-KV decode, speculative-verify and fused RoPE +
KV-write figures of the other BASELINE configs alongside, the roofline of the decode kernel and the CPU
baseline (the oracle's Float32 op on the host cores, a bounded sample). The headline is
timed call by call (HIP events around K steps); the other legs replay a HIP graph of 20
captured calls, which removes host launch overhead from their microsecond-scale figures,
after half a second of replays so that each leg is timed at steady state.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tileinfer.jl_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3       # MI355X dense fp32 MFMA, TFLOP/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_calls(fn, iters, warmup):
    """Average ms per call over `iters` back-to-back calls (HIP events on the stream the
    kernels are launched on: torch's current stream), after `warmup` calls."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters


def time_graph(fn, calls=20, replays=10, settle_s=0.5):
    """Average ms per call with `calls` calls captured in one HIP graph, replayed `replays`
    times after the graph has been replayed for about `settle_s` seconds: GPU time without
    host launch overhead, as a graph-capturing runner sees it, at steady state (a leg's
    first fraction of a second runs up to 15 % slower while the GPU's clocks settle)."""
    import torch
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / (replays * calls)


CACHE_BYTES = 256 << 20      # MI355X Infinity Cache (the L2s are far smaller)


def decode_setup(B, L, n, Hq, Hk, D, P, copies, gen, int8=False, cold=True):
    """Pools, block tables, q/out and workspace for B sequences of L positions each with
    n new query tokens at positions L-n .. L-1. At least `copies` independent copies of
    the pools; with `cold`, enough that the calls cycle through twice the Infinity Cache,
    so every call reads its K and V from HBM (prefill legs read the K and V the fused
    write just stored, and stay warm)."""
    import torch
    import tileinfer_hip as ti
    per = -(-L // P)
    pages = B * per
    copy_bytes = 2 * pages * Hk * P * (D + 4 if int8 else 2 * D)
    if cold:
        copies = max(copies, min(64, -(-2 * CACHE_BYTES // copy_bytes)))
    perm = torch.randperm(pages, generator=gen) + 1
    bts = perm.view(B, per).to(torch.int32).cuda()
    pools = []
    for _ in range(copies):
        if int8:
            kq, vq = ti.int8_kv_pools(D, P, Hk, pages)
            kq.layer_q.random_(-127, 128)
            kq.layer_scale.uniform_(0.015, 0.03)
            pools.append((kq, vq))
        else:
            k = torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16)
            v = torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16)
            pools.append((k, v))
    q = torch.randn((B * n, Hq, D), device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(q)
    pos = (torch.arange(L - n, L, dtype=torch.int32).repeat(B)).cuda()
    ws = ti.attention_workspace(ti.HipBackend(), q, pools[0][0], num_seqs=B, max_query_len=n)
    return dict(pools=pools, bts=bts, q=q, out=out, pos=pos, ws=ws, n=n, B=B, L=L)


def ragged_setup(B, Hq, Hk, D, P, seed):
    """BASELINE configs[1] as stated: B sequences with context lengths drawn uniformly from
    [1024, 8192] (seeded), one query token each at position L_b - 1, shuffled pages,
    block tables as wide as the longest sequence (zero-padded), pool copies cycling past
    the Infinity Cache."""
    import numpy as np
    import torch
    import tileinfer_hip as ti
    g = np.random.default_rng(seed)
    lens = g.integers(1024, 8193, size=B)
    per = -(-lens // P)
    pages = int(per.sum())
    copy_bytes = 2 * pages * Hk * P * 2 * D
    copies = max(2, min(64, -(-2 * CACHE_BYTES // copy_bytes)))
    perm = torch.from_numpy(g.permutation(pages).astype(np.int32) + 1)
    bts = torch.zeros((B, int(per.max())), dtype=torch.int32)
    off = 0
    for b in range(B):
        bts[b, :per[b]] = perm[off:off + per[b]]
        off += int(per[b])
    pools = [(torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16),
              torch.randn((pages, Hk, P, D), device="cuda", dtype=torch.bfloat16)) for _ in range(copies)]
    q = torch.randn((B, Hq, D), device="cuda", dtype=torch.bfloat16)
    pos = torch.from_numpy((lens - 1).astype(np.int32)).cuda()
    ws = ti.attention_workspace(ti.HipBackend(), q, pools[0][0], num_seqs=B, max_query_len=1)
    nbytes = int(lens.sum()) * 2 * Hk * D * 2 + B * 2 * Hq * D * 2
    return dict(pools=pools, bts=bts.cuda(), q=q, out=torch.empty_like(q), pos=pos, ws=ws, n=1, B=B,
                lens=lens, bytes=nbytes)


def decode_call(s, i, scale, path=0):
    import tileinfer_hip as ti
    k, v = s["pools"][i % len(s["pools"])]
    ti.paged_attention_(ti.HipBackend(), s["out"], s["ws"], s["q"], k, v, s["bts"], s["pos"],
                        scale, True, max_query_len=s["n"], path=path)


def decode_bytes(B, L, n, Hq, Hk, D, kv_elt_bytes):
    """Algorithmic bytes (bench/suite.jl:248-253): read K and V once, read q, write out."""
    return B * (2 * L * Hk * kv_elt_bytes + 2 * n * Hq * D * 2)


def measured_traffic():
    """HBM bytes per headline launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (copy-calibrated), or None when it is absent."""
    path = os.path.join(ROOT, "profiles", "decode_b32_ctx4096_pmc.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_cores():
    """Cores this process may use: the cgroup CPU quota when one is set (a GPU box grants
    each GPU a share of its host), else the CPUs in the affinity mask."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_baseline(B, L, Hq, Hk, D, P, budget_s=10.0):
    """The reference's eager op in Float32 (cpu_baseline.c: gather pages, K^T q, softmax,
    V p; src/ops/reference.jl:76-121) on every core this process may use, built -O3
    -march=native for this host, over a sample of the headline workload repeated for about
    budget_s seconds; the rate is in the headline's units (bf16 algorithmic bytes of the
    sampled sequences per second)."""
    import numpy as np
    from oracle import oracle as orc
    g = np.random.Generator(np.random.PCG64(7))
    threads = cpu_cores()
    Bs = min(B, max(4, threads))
    per = -(-L // P)
    pages = Bs * per
    kp = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    vp = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    bts = (g.permutation(pages) + 1).astype(np.int32).reshape(Bs, per)
    q = g.standard_normal((Bs, Hq, D), dtype=np.float32)
    starts = np.full(Bs, L - 1, np.int32)
    counts = np.ones(Bs, np.int32)
    orc.attention_f32_batch(q, kp, vp, bts, starts, counts, 1 / math.sqrt(D), True, threads)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        orc.attention_f32_batch(q, kp, vp, bts, starts, counts, 1 / math.sqrt(D), True, threads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    gbs = decode_bytes(Bs, L, 1, Hq, Hk, D, D * 2) / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "host_cpus": os.cpu_count(),
            "kind": "port", "build": "gcc -O3 -march=native -ffast-math -fopenmp (oracle/cpu_baseline.c)",
            "sample": f"{Bs} of the {B} sequences ({L} positions each, Float32 copies of the pools), "
                      f"{reps} passes in {reps * dt:.1f} s; {dt * 1e3:.2f} ms per pass"}


def cpu_baseline_config0(budget_s=5.0):
    """BASELINE configs[0], the canonical CPU point: Qwen3-0.6B-shaped Float32 decode
    attention, batch 1, 16 query / 8 KV heads, head_dim 128, 1024 positions in 16-token
    pages (seeded permutation block table), scale 1/sqrt(128); the same op and build as
    cpu_baseline, timed per call."""
    import numpy as np
    from oracle import oracle as orc
    g = np.random.Generator(np.random.PCG64(0))
    L, Hq, Hk, D, P = 1024, 16, 8, 128, 16
    pages = L // P
    kp = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    vp = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    bt = (g.permutation(pages) + 1).astype(np.int32)[None]
    q = g.standard_normal((1, Hq, D), dtype=np.float32)
    args = (q, kp, vp, bt, np.array([L - 1], np.int32), np.ones(1, np.int32), 1 / math.sqrt(D), True)
    threads = min(cpu_cores(), Hk)                 # the op parallelizes over KV heads
    best = {}
    for th in sorted({1, threads}):
        orc.attention_f32_batch(*args, th)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s / 2:
            orc.attention_f32_batch(*args, th)
            reps += 1
        best[th] = (time.perf_counter() - t0) / reps
    th = min(best, key=best.get)
    us = best[th] * 1e6
    nbytes = 2 * L * Hk * D * 4 + 2 * Hq * D * 4
    return {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 2), "cores": th,
            "us_by_threads": {str(k): round(v * 1e6, 2) for k, v in best.items()}, "kind": "port",
            "build": "gcc -O3 -march=native -ffast-math -fopenmp (oracle/cpu_baseline.c)",
            "workload": "configs[0]: Qwen3-0.6B fp32 decode, B=1, 16/8 heads, D=128, 1024 positions"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="",
                    help="comma list: decode,ragged,fp32,verify,int8,prefill (= prefill512,chunked,prefill4096),kvwrite; "
                         "'none' runs the headline only")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy a 512 MiB buffer 5 times (reference for rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (decode would shard "
              "by sequence or KV head with no exchange); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel() * 2}))
        return
    import tileinfer_hip as ti
    ti.load_library()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    only = set(filter(None, args.only.split(",")))
    want = lambda k: not only or k in only
    gen = torch.Generator().manual_seed(20261201)
    torch.manual_seed(20261201)
    Hq, Hk, D, P = 32, 8, 128, 16
    scale = 1 / math.sqrt(D)
    result = {}

    # ---- headline: bf16 decode, B = 32 x 4096 ----
    B, L = 32, 4096
    s = decode_setup(B, L, 1, Hq, Hk, D, P, 2, gen)
    nbytes = decode_bytes(B, L, 1, Hq, Hk, D, D * 2)
    for i in range(args.warmup):
        decode_call(s, i, scale)
    torch.cuda.synchronize()
    # An event after every WIN calls of the timed region: the spread (min, median) is over
    # those windows' per-call means, whose average is the mean itself (events around single
    # calls would add the gap between launches to every call).
    WIN = 5
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps // WIN + 2)]
    t0 = time.perf_counter()
    marks[0].record()
    nm = 1
    for i in range(args.steps):
        decode_call(s, i, scale)
        if (i + 1) % WIN == 0 or i + 1 == args.steps:
            marks[nm].record()
            nm += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = marks[0].elapsed_time(marks[nm - 1]) / args.steps
    bounds = [min(WIN * w, args.steps) for w in range(nm)]
    bounds[-1] = args.steps
    per_call = sorted(marks[w].elapsed_time(marks[w + 1]) * 1e3 / (bounds[w + 1] - bounds[w])
                      for w in range(nm - 1) if bounds[w + 1] > bounds[w])
    nwin = len(per_call)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"decode B={B} L={L}: {ms * 1e3:.1f} us/call, {gbs:.0f} GB/s ({wall:.2f} s wall)")
    del s
    torch.cuda.empty_cache()

    extra = {}
    if want("decode"):
        for Bx in (1, 8):
            sx = decode_setup(Bx, L, 1, Hq, Hk, D, P, 2, gen)
            msx = time_graph(lambda i: decode_call(sx, i, scale))
            bx = decode_bytes(Bx, L, 1, Hq, Hk, D, D * 2)
            extra[f"decode_b{Bx}"] = {"us": round(msx * 1e3, 2), "GB/s": round(bx / msx / 1e6, 1),
                                      "pct_hbm_peak": round(100 * bx / msx / 1e6 / HBM_PEAK_GBS, 1)}
            del sx
    if want("decode") or want("ragged"):
        for Bx in (1, 8, 32):
            sx = ragged_setup(Bx, Hq, Hk, D, P, 20261201 + Bx)
            msx = time_graph(lambda i: decode_call(sx, i, scale))
            gx = sx["bytes"] / msx / 1e6
            extra[f"decode_ragged_b{Bx}"] = {"us": round(msx * 1e3, 2), "GB/s": round(gx, 1),
                                             "pct_hbm_peak": round(100 * gx / HBM_PEAK_GBS, 1),
                                             "context_sum": int(sx["lens"].sum()), "context_max": int(sx["lens"].max())}
            log(f"decode ragged B={Bx}: {msx * 1e3:.1f} us, {gx:.0f} GB/s")
            del sx
        torch.cuda.empty_cache()
    if want("fp32"):
        # configs[0]'s shape on the fp32 path: B = 1, 16 query / 8 KV heads, 1024 positions
        import tileinfer_hip as ti
        L1, H1, K1 = 1024, 16, 8
        copies = 32                                  # 8.4 MB per copy: cycle past the cache
        per1 = L1 // P
        pools1 = [(torch.randn((per1, K1, P, D), device="cuda"), torch.randn((per1, K1, P, D), device="cuda"))
                  for _ in range(copies)]
        bt1 = (torch.randperm(per1, generator=gen) + 1).to(torch.int32).cuda()
        q1 = torch.randn((1, H1, D), device="cuda")
        o1 = torch.empty_like(q1)
        pos1 = torch.tensor([L1 - 1], dtype=torch.int32, device="cuda")
        be = ti.HipBackend()
        ws1 = ti.attention_workspace(be, q1, pools1[0][0])
        ms1 = time_graph(lambda i: ti.attention_(be, o1, ws1, q1, pools1[i % copies][0], pools1[i % copies][1],
                                                 bt1, pos1, scale))
        b1 = 2 * L1 * K1 * D * 4 + 2 * H1 * D * 4
        extra["decode_fp32_qwen3_06b_ctx1024"] = {"us": round(ms1 * 1e3, 2), "GB/s": round(b1 / ms1 / 1e6, 1)}
        del pools1
        # the fp32 path on a 512-token causal prefill at the same head shape (not a BASELINE
        # config: the fp32 matrix-core kernel's multi-token mode)
        n2 = 512
        k2 = torch.randn((n2 // P, K1, P, D), device="cuda")
        v2 = torch.randn_like(k2)
        bt2 = (torch.randperm(n2 // P, generator=gen) + 1).to(torch.int32).cuda()
        q2 = torch.randn((n2, H1, D), device="cuda")
        o2 = torch.empty_like(q2)
        pos2 = torch.arange(n2, dtype=torch.int32, device="cuda")
        ws2 = ti.attention_workspace(be, q2, k2)
        ms2 = time_graph(lambda i: ti.attention_(be, o2, ws2, q2, k2, v2, bt2, pos2, scale))
        tf2 = 4 * D * H1 * (n2 * (n2 + 1) // 2) / (ms2 * 1e-3) / 1e12
        extra["prefill_fp32_qwen3_06b_512"] = {"us": round(ms2 * 1e3, 2), "TFLOP/s": round(tf2, 1),
                                               "pct_fp32_mfma_peak": round(100 * tf2 / FP32_PEAK_TFLOPS, 1)}
        del k2, v2
    if want("verify"):
        sv = decode_setup(16, 4096 + 16, 16, 32, 8, D, P, 2, gen)
        msv = time_graph(lambda i: decode_call(sv, i, scale))
        bv = decode_bytes(16, 4096 + 16, 16, 32, 8, D, D * 2)
        extra["verify_qwen3_8b_b16_n16_ctx4096"] = {"us": round(msv * 1e3, 2), "GB/s": round(bv / msv / 1e6, 1),
                                                   "pct_hbm_peak": round(100 * bv / msv / 1e6 / HBM_PEAK_GBS, 1)}
        del sv
    if want("int8"):
        s8 = decode_setup(8, 32768, 1, 32, 8, D, P, 2, gen, int8=True)
        ms8 = time_graph(lambda i: decode_call(s8, i, scale))
        b8 = decode_bytes(8, 32768, 1, 32, 8, D, D + 4)
        extra["int8_decode_llama3_8b_b8_ctx32768"] = {"us": round(ms8 * 1e3, 2), "GB/s": round(b8 / ms8 / 1e6, 1),
                                                     "pct_hbm_peak": round(100 * b8 / ms8 / 1e6 / HBM_PEAK_GBS, 1)}
        del s8
    torch.cuda.empty_cache()
    for start, n, leg in ((0, 512, "prefill512"), (1024, 512, "chunked"), (0, 4096, "prefill4096")):
        if want("prefill") or want(leg):
            sp = decode_setup(1, start + n, n, Hq, Hk, D, P, 1, gen, cold=False)
            msp = time_graph(lambda i: decode_call(sp, i, scale))
            visited = n * start + n * (n + 1) // 2
            flops = 4 * D * Hq * visited
            tf = flops / (msp * 1e-3) / 1e12
            key = {"prefill512": "prefill_512", "chunked": "chunked_prefill_512_on_1024",
                   "prefill4096": "prefill_4096"}[leg]
            extra[key] = {"us": round(msp * 1e3, 2), "TFLOP/s": round(tf, 1),
                          "pct_mfma_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2), "gflop": round(flops / 1e9, 3)}
            log(f"{key}: {msp * 1e3:.1f} us, {tf:.1f} TFLOP/s")
            del sp
    if want("kvwrite"):
        n = 512
        table = ti.RotaryTable.build(D, 4096, 1e6, torch.bfloat16)
        qkv = torch.randn((n, (Hq + 2 * Hk) * D), device="cuda", dtype=torch.bfloat16)
        qo = torch.empty((n, Hq, D), device="cuda", dtype=torch.bfloat16)
        kpool = torch.zeros((64 + 32, Hk, P, D), device="cuda", dtype=torch.bfloat16)
        vpool = torch.zeros_like(kpool)
        positions = torch.arange(1024, 1024 + n, dtype=torch.int32, device="cuda")
        slots_t = torch.arange(1024 + 1, 1024 + n + 1, dtype=torch.int32, device="cuda")
        be = ti.HipBackend()
        msk = time_graph(lambda i: ti.attention_inputs_(be, qo, kpool, vpool, qkv, None, None, table,
                                                        positions, slots_t, 1e-6))
        kb = (n * (Hq + 2 * Hk) * D * 2) + (n * Hq * D * 2) + 2 * n * Hk * D * 2 + n * 2 * D * 2
        extra["rope_kv_write_512"] = {"us": round(msk * 1e3, 2), "GB/s": round(kb / msk / 1e6, 1)}
        # the unfused ops of the same step (the reference's generic chain): store_kv into
        # dense bf16 and INT8 pages, and rope on the queries
        kk = torch.randn((n, Hk, D), device="cuda", dtype=torch.bfloat16)
        vv = torch.randn_like(kk)
        mss = time_graph(lambda i: ti.store_kv_(be, kpool, vpool, kk, vv, slots_t))
        sb = 2 * n * Hk * D * 2 * 2 + n * 4                       # read k, v; write both; slots
        extra["store_kv_bf16_512"] = {"us": round(mss * 1e3, 2), "GB/s": round(sb / mss / 1e6, 1)}
        kq, vq = ti.int8_kv_pools(D, P, Hk, 64 + 32)
        msf = time_graph(lambda i: ti.attention_inputs_(be, qo, kq, vq, qkv, None, None, table,
                                                        positions, slots_t, 1e-6))
        fb = (n * (Hq + 2 * Hk) * D * 2) + (n * Hq * D * 2) + 2 * n * Hk * (D + 4) + n * 2 * D * 2
        extra["rope_kv_write_int8_512"] = {"us": round(msf * 1e3, 2), "GB/s": round(fb / msf / 1e6, 1)}
        msq = time_graph(lambda i: ti.store_kv_(be, kq, vq, kk, vv, slots_t))
        qb = 2 * n * Hk * D * 2 + 2 * n * Hk * (D + 4) + n * 4    # read bf16 k, v; write int8 + scales
        extra["store_kv_int8_512"] = {"us": round(msq * 1e3, 2), "GB/s": round(qb / msq / 1e6, 1)}
        xr = torch.randn((n, Hq, D), device="cuda", dtype=torch.bfloat16)
        yr = torch.empty_like(xr)
        msr = time_graph(lambda i: ti.rope_(be, yr, xr, table.cos, table.sin, positions))
        rb = 2 * n * Hq * D * 2 + n * 2 * D * 2 + n * 4           # read x, write y; cos, sin rows
        extra["rope_q_512"] = {"us": round(msr * 1e3, 2), "GB/s": round(rb / msr / 1e6, 1)}

    result = {
        "metric": "decode attn GB/s (% of HBM peak) & prefill attn TFLOP/s at Qwen3-4B shape",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_call": round(ms * 1e3, 2),
        "us_per_call_min": round(per_call[0], 2),
        "us_per_call_median": round(per_call[len(per_call) // 2], 2),
        "us_per_call_spread": f"min and median over the {nwin} windows of up to {WIN} back-to-back calls that make up "
                              "the timed K steps (per-call mean of each window; us_per_call is their overall mean)",
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 pools, shuffled 16-token pages)",
        "config": {"workload": "Qwen3-4B paged decode attention (BASELINE configs[1], batch 32 x 4096 context)",
                   "global_batch": B, "context": L, "q_heads": Hq, "kv_heads": Hk, "head_dim": D,
                   "page_size": P, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "note": "achieved = algorithmic bytes per call / HIP-event time per call; the call is "
                             "one decode_kernel launch (one split per sequence and KV head, no combine); "
                             "traffic = rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated"},
    }
    result.update(extra)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(B, L, Hq, Hk, D, P)
        result["cpu_baseline_config0"] = cpu_baseline_config0()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
