"""Shared input builders and error metrics for the tests (seeded, numpy-based)."""
from __future__ import annotations

import math

import numpy as np

from oracle import oracle as orc


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def randn(g, *shape, bf16=False, scale=1.0):
    x = (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)
    return orc.bf16_round(x) if bf16 else x


def block_table(g, len_, P, pages, pad_to=16):
    """Fragmented, out-of-order 1-based table of cld(len, P) pages of a pool of `pages`,
    zero-padded to a multiple of pad_to entries (as test/ops/tile.jl:226-227 and
    src/model/decoder.jl:109 pad it)."""
    used = -(-len_ // P)
    t = (g.permutation(pages)[:used] + 1).astype(np.int32)
    width = max(pad_to, -(-used // pad_to) * pad_to)
    return np.concatenate([t, np.zeros(width - used, np.int32)])


def bf16_eps(x):
    """Spacing of bf16 numbers at |x| (Julia's eps(BFloat16(x)))."""
    a = np.abs(np.asarray(x, np.float64))
    a = np.maximum(a, 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def ulps(ref, got):
    """Largest difference in units of bf16 precision at each element's size, the unit
    floored at the reference's RMS (test/ops/tile.jl:16-20)."""
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64)
    floor_ulp = bf16_eps(math.sqrt(float(np.mean(ref * ref))))
    return float(np.max(np.abs(ref - got) / np.maximum(bf16_eps(ref), floor_ulp), initial=0.0))


def smoothing(g, D):
    """Key smoothing factors with RMS 1 spanning two orders of magnitude, equal on both
    channels of a rotary pair (test/ops/tile.jl:25-29)."""
    c = np.exp(g.standard_normal(D // 2).astype(np.float32) * np.float32(1.5)).astype(np.float32)
    c = (c / np.float32(math.sqrt(float(np.sum(c.astype(np.float64) ** 2)) / len(c)))).astype(np.float32)
    return np.concatenate([c, c]).astype(np.float32)
