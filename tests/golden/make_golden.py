"""Write the golden fixtures in this directory from the CPU oracle (test infrastructure).

    python tests/golden/make_golden.py

The reference holds no golden vectors for its attention path (its tests draw random
inputs from Julia's RNG), so these are the build's own: small seeded inputs and the
oracle's outputs, pinned so that a change in the oracle or a kernel shows up against
stored numbers. Every fixture is an .npz of plain arrays (no pickles).

  attention_bf16.npz       paged GQA attention on bf16-valued inputs, causal and
                           non-causal, a ragged last page (src/ops/reference.jl:95-121)
  attention_int8.npz       attention over an INT8 cache with key smoothing
                           (src/ops/quant.jl:56-72, :165-170)
  store_kv_int8.npz        INT8 quantizing store incl. a zero vector and a halfway case
                           (src/ops/quant.jl:141-159)
  attention_inputs.npz     fused q/k RMSNorm + RoPE + KV page write, bf16 rounding points
                           (src/ops/interface.jl:169-179, src/ops/tile/fused.jl:15-130)
  config1_fp32.npz         BASELINE configs[0]: fp32 decode, 16/8 heads, 1024 positions in
                           16-token pages; the pools are regenerated from the stored seed
                           (their SHA-256 is stored) and q and the output are stored
"""
from __future__ import annotations

import hashlib
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def bf16n(g, *shape):
    return orc.bf16_round(g.standard_normal(shape, dtype=np.float32))


def table(g, L, P, pages, width):
    used = -(-L // P)
    t = np.zeros(width, np.int32)
    t[:used] = g.permutation(pages)[:used] + 1
    return t


def config1_pools(seed=20261201):
    """configs[0] inputs: q, pools, block table from one PCG64 stream."""
    g = rng(seed)
    Hq, Hk, D, P, L = 16, 8, 128, 16, 1024
    pages = L // P + 4
    q = g.standard_normal((1, Hq, D), dtype=np.float32)
    k = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    v = g.standard_normal((pages, Hk, P, D), dtype=np.float32)
    bt = table(g, L, P, pages, 64)
    return q, k, v, bt


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), np.uint8)


def main():
    # ---- paged attention, bf16-valued inputs ----
    g = rng(101)
    D, Hq, Hk, P, pages, start, n = 64, 8, 2, 4, 14, 33, 7
    L = start + n
    kp, vp = bf16n(g, pages, Hk, P, D), bf16n(g, pages, Hk, P, D)
    q = bf16n(g, n, Hq, D)
    bt = table(g, L, P, pages, 16)
    scale = np.float32(1 / math.sqrt(D))
    out_c = orc.attention(q, bt, start, scale, True, kp, vp)
    out_nc = orc.attention(q, bt, start, scale, False, kp, vp)
    np.savez_compressed(os.path.join(HERE, "attention_bf16.npz"), q=q, k_pages=kp, v_pages=vp,
                        block_table=bt, start=np.int32(start), scale=scale,
                        out_causal=out_c, out_noncausal=out_nc)

    # ---- INT8 cache with key smoothing ----
    g = rng(202)
    D, Hq, Hk, P, pages, start, n = 128, 4, 1, 16, 6, 66, 4
    L = start + n
    smooth = (0.5 + g.random(D, dtype=np.float32)).astype(np.float32)
    lq = np.zeros((2, pages, Hk, P, D), np.int8)
    ls = np.zeros((2, pages, Hk, P), np.float32)
    k = bf16n(g, pages * P, Hk, D)
    v = bf16n(g, pages * P, Hk, D)
    orc.store_kv_int8(lq, ls, smooth, k, v, np.arange(1, pages * P + 1, dtype=np.int32))
    q = bf16n(g, n, Hq, D)
    bt = table(g, L, P, pages, 16)
    scale = np.float32(1 / math.sqrt(D))
    out = orc.attention(q, bt, start, scale, True, layer_q=lq, layer_scale=ls, smooth=smooth)
    np.savez_compressed(os.path.join(HERE, "attention_int8.npz"), q=q, layer_q=lq, layer_scale=ls,
                        smooth=smooth, block_table=bt, start=np.int32(start), scale=scale, out=out)

    # ---- INT8 store: zero vector, a halfway value, random ----
    g = rng(303)
    D, Hk, P, pages, n = 64, 2, 4, 3, 5
    k = bf16n(g, n, Hk, D)
    v = bf16n(g, n, Hk, D)
    k[1, 0] = 0.0                                  # zero vector: q = 0, s = 0
    v[2, 1] = 0.0
    v[3, 1, :] = 0.0
    v[3, 1, 0], v[3, 1, 1] = 127.0, 0.5            # x * 127 / max = 0.5 exactly: floor(1.0) = 1
    smooth = (0.75 + 0.5 * g.random(D, dtype=np.float32)).astype(np.float32)
    slots = np.array([3, 12, 1, 7, 10], np.int32)
    lq = np.zeros((2, pages, Hk, P, D), np.int8)
    ls = np.zeros((2, pages, Hk, P), np.float32)
    orc.store_kv_int8(lq, ls, smooth, k, v, slots)
    np.savez_compressed(os.path.join(HERE, "store_kv_int8.npz"), k=k, v=v, smooth=smooth, slots=slots,
                        layer_q=lq, layer_scale=ls)

    # ---- fused q/k RMSNorm + RoPE + KV write (bf16) ----
    g = rng(404)
    D, nq, nkv, P, pages, n, max_len = 64, 4, 2, 4, 6, 6, 48
    qkv = bf16n(g, n, nq + 2 * nkv, D)
    q_norm = orc.bf16_round((1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float32))
    k_norm = orc.bf16_round((1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float32))
    inv = 1.0 / (1e6 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.outer(np.arange(max_len, dtype=np.float64), inv)
    cos = orc.bf16_round(np.cos(np.concatenate([ang, ang], 1)).astype(np.float32))
    sin = orc.bf16_round(np.sin(np.concatenate([ang, ang], 1)).astype(np.float32))
    cos_sin = np.stack([cos, sin], 1).astype(np.float32)          # [max_len][2][D]
    positions = np.array([17, 18, 19, 20, 21, 40], np.int32)
    slots = np.array([2, 3, 4, 5, 9, 23], np.int32)
    kp = np.zeros((pages, nkv, P, D), np.float32)
    vp = np.zeros((pages, nkv, P, D), np.float32)
    qo = orc.attention_inputs(qkv, q_norm, k_norm, cos_sin, positions, slots, nq, nkv, 1e-6, True,
                              k_pages=kp, v_pages=vp)
    np.savez_compressed(os.path.join(HERE, "attention_inputs.npz"), qkv=qkv, q_norm=q_norm,
                        k_norm=k_norm, cos_sin=cos_sin, positions=positions, slots=slots,
                        eps=np.float32(1e-6), q=qo, k_pages=kp, v_pages=vp)

    # ---- fp32 decode ----
    seed = 20261201
    q, k, v, bt = config1_pools(seed)
    scale = np.float32(1 / math.sqrt(128))
    out = orc.attention(q, bt, 1023, scale, True, k, v)
    np.savez_compressed(os.path.join(HERE, "config1_fp32.npz"), seed=np.int64(seed), q=q,
                        block_table=bt, start=np.int32(1023), scale=scale, out=out,
                        pools_sha256=digest(k, v))
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
