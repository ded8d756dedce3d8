"""Seeded random shapes through every attention path against the oracle, in one process.

Each case draws head_dim, heads per KV head, page size, cached prefix, query count,
causality and cache type, builds a fragmented block table, and compares the GPU output
with the double-accumulated oracle: max abs <= 2e-2 (bf16), <= 2e-2 + one bf16 unit of the
reference value and <= 14 ulps (INT8-KV), or <= 1e-4 (fp32, and the reference's relative
2-norm bound 1e-5).
The case parameters are printed before each call so a failure names its shape.
TI_RANDOM_SHAPES sets the number of cases (default 60)."""
import math
import os

import numpy as np
import pytest
import torch

import tileinfer_hip as ti
from helpers import block_table, randn, rng, smoothing, ulps
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
BE = ti.HipBackend()


def draw(g):
    D = int(g.choice([64, 128]))
    Hk = int(g.choice([1, 2, 4, 8]))
    G = int(g.choice([1, 2, 3, 4, 8]))
    P = int(g.choice([4, 16, 32, 48, 64]))
    start = int(g.choice([0, int(g.integers(1, 200)), int(g.integers(200, 3000))]))
    n = int(g.choice([1, int(g.integers(2, 17)), int(g.integers(17, 300))]))
    causal = bool(g.random() < 0.8)
    kind = str(g.choice(["bf16", "bf16", "fp32", "int8"]))
    return D, Hk, G, P, start, n, causal, kind


# TI_RANDOM_SHAPES cases from seed TI_RANDOM_SHAPES_FROM (default: 60 from seed 0)
_FROM = int(os.environ.get("TI_RANDOM_SHAPES_FROM", "0"))


@pytest.mark.parametrize("seed", list(range(_FROM, _FROM + int(os.environ.get("TI_RANDOM_SHAPES", "60")))))
def test_random_shape(gpu, seed):
    g = rng(7000 + seed)
    D, Hk, G, P, start, n, causal, kind = draw(g)
    H = Hk * G
    L = start + n
    pages = -(-L // P) + 3
    bt = block_table(g, L, P, pages)
    bf = kind != "fp32"
    q = randn(g, n, H, D, bf16=bf)
    kp, vp = randn(g, pages, Hk, P, D, bf16=bf), randn(g, pages, Hk, P, D, bf16=bf)
    scale = 1 / math.sqrt(D)
    print(f"seed {seed}: D={D} Hk={Hk} G={G} P={P} start={start} n={n} causal={causal} {kind}", flush=True)
    dtype = torch.float32 if kind == "fp32" else torch.bfloat16
    qd = torch.from_numpy(q).to(dtype).cuda()
    pos = torch.arange(start, L, dtype=torch.int32, device="cuda")
    btd = torch.from_numpy(bt).cuda()
    if kind == "int8":
        cs = smoothing(g, D)
        k_src = orc.bf16_round(kp * orc.bf16_round(cs)[None, None, None, :])
        kq, vq = ti.int8_kv_pools(D, P, Hk, pages, key_smoothing=torch.from_numpy(cs))
        kk = torch.from_numpy(np.ascontiguousarray(k_src.transpose(0, 2, 1, 3).reshape(-1, Hk, D))).to(dtype).cuda()
        vv = torch.from_numpy(np.ascontiguousarray(vp.transpose(0, 2, 1, 3).reshape(-1, Hk, D))).to(dtype).cuda()
        ti.store_kv_(BE, kq, vq, kk, vv, torch.arange(1, P * pages + 1, dtype=torch.int32, device="cuda"))
        ref = orc.attention(q, bt, start, scale, causal, layer_q=kq.layer_q.cpu().numpy(),
                            layer_scale=kq.layer_scale.cpu().numpy(), smooth=cs)
        k, v = kq, vq
    else:
        ref = orc.attention(q, bt, start, scale, causal, kp, vp)
        k, v = torch.from_numpy(kp).to(dtype).cuda(), torch.from_numpy(vp).to(dtype).cuda()
    paths = [ti.TI_PATH_AUTO]
    if kind != "fp32":
        if G * n <= 64:
            paths.append(ti.TI_PATH_DECODE)
        paths.append(ti.TI_PATH_PREFILL)
    tol = 1e-4 if kind == "fp32" else 2e-2
    if kind == "bf16":
        # the prefill path through both prefill kernels (PINGPONG takes the 8-wave kernel
        # wherever its shape limits allow) and through both tile loaders of the four-wave
        # kernel (STAGED: register-staged loads; DIRECT: direct global -> LDS loads
        # wherever they apply)
        paths += [ti.TI_PATH_PREFILL_PINGPONG, ti.TI_PATH_PREFILL_STAGED, ti.TI_PATH_PREFILL_DIRECT,
                  ti.TI_PATH_PREFILL_PAIRED, ti.TI_PATH_PREFILL_PAIRED16]
    for path in paths:
        out = torch.full_like(qd, float("nan"))
        ws = ti.attention_workspace(BE, qd, k, path=path)
        ti.attention_(BE, out, ws, qd, k, v, btd, pos, scale, causal, path=path)
        got = out.float().cpu().numpy()
        if kind == "int8":
            # INT8: 2e-2 plus one bf16 unit of the reference value (the output's own rounding),
            # and the reference's INT8 bound of 14 ulps (test/ops/tile.jl:256). Its algorithm
            # rounds p * s_v to bf16, so where outputs reach |o| ~ 2.4 the exact result is out of
            # a flat 2e-2 at times: seed 18373, 1 case in ~4500, 0.021 at o = -2.354 on every
            # prefill kernel alike (10 ulps), where the reference's own eager op is 0.018 off
            # (27 ulps) on the same inputs.
            excess = float(np.max(np.abs(ref - got) - (tol + np.abs(ref) * 2.0 ** -8)))
            assert excess <= 0, f"path {path}: abs err over 2e-2 + |ref| 2^-8 by {excess}"
            u = ulps(ref, got)
            assert u <= 14, f"path {path}: {u} ulps"
        else:
            err = float(np.max(np.abs(ref - got)))
            assert err <= tol, f"path {path}: max abs err {err}"
        if kind == "fp32":
            # the reference's Float32 bound, isapprox(y, exact; rtol = 1e-5) (test/ops/tile.jl:240)
            d = float(np.linalg.norm((ref - got).astype(np.float64)))
            assert d <= 1e-5 * max(float(np.linalg.norm(ref)), float(np.linalg.norm(got))), f"path {path}: norm err {d}"
