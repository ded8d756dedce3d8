"""Paged KV cache: host-side page allocation and the device page pools.

Mirrors src/kv/block_manager.jl (BlockManager, Sequence, reserve!, truncate!, release!,
slots, OutOfPagesError), src/kv/paged_cache.jl (PagedKVCache) and the INT8 cache types of
src/ops/quant.jl:56-135 (Int8Pages, int8_kv_pools, key_smoothing, layer_arrays).

Pools are torch tensors in C order, the reference's column-major shapes reversed:
dense (head_dim, page_size, kv_heads, pages) -> [pages][kv_heads][page_size][head_dim];
an INT8 layer's values `layer_q` (D, P, H, pages, 2) -> [2][pages][H][P][D] (keys first)
and scales `layer_scale` (P, H, pages, 2) -> [2][pages][H][P]. Page ids and slots are
1-based, as in the reference, so block tables and slots pass through unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch

from ._lib import ArgumentError

DEFAULT_PAGE_SIZE = 64  # src/kv/paged_cache.jl:7


class OutOfPagesError(Exception):
    """Raised by reserve when the pool has fewer free pages than a step needs
    (src/kv/block_manager.jl:26-32)."""

    def __init__(self, needed: int, free: int):
        super().__init__(f"KV cache full: need {needed} more pages, {free} free")
        self.needed, self.free = needed, free


@dataclass
class Sequence:
    """A sequence's block table (1-based page ids) and cached token ids
    (src/kv/block_manager.jl:13-18)."""
    block_table: List[int] = field(default_factory=list)
    tokens: List[int] = field(default_factory=list)

    def __len__(self) -> int:
        return len(self.tokens)


class BlockManager:
    """Hands out the pages of a pool of num_pages pages of page_size positions
    (src/kv/block_manager.jl:39-50). The free list is a stack, reversed so pages are
    handed out in increasing order."""

    def __init__(self, num_pages: int, page_size: int):
        self.num_pages, self.page_size = int(num_pages), int(page_size)
        self.free: List[int] = list(range(self.num_pages, 0, -1))

    def num_free_pages(self) -> int:
        return len(self.free)


def _cld(a: int, b: int) -> int:
    return -(-a // b)


def reserve(b: BlockManager, seq: Sequence, n: int) -> Sequence:
    """Pages for n more positions of seq; raises OutOfPagesError before changing anything
    (src/kv/block_manager.jl:58-65)."""
    needed = _cld(len(seq) + n, b.page_size) - len(seq.block_table)
    if needed > b.num_free_pages():
        raise OutOfPagesError(needed, b.num_free_pages())
    for _ in range(max(needed, 0)):
        seq.block_table.append(b.free.pop())
    return seq


def truncate(b: BlockManager, seq: Sequence, n: int) -> Sequence:
    """Keep the first n cached positions; unused pages go back to the pool
    (src/kv/block_manager.jl:74-81)."""
    if not 0 <= n <= len(seq):
        raise ArgumentError(f"cannot truncate a sequence of length {len(seq)} to {n}")
    del seq.tokens[n:]
    keep = _cld(n, b.page_size)
    b.free.extend(reversed(seq.block_table[keep:]))
    del seq.block_table[keep:]
    return seq


def release(b: BlockManager, seq: Sequence) -> Sequence:
    """Return all pages of seq (src/kv/block_manager.jl:88)."""
    return truncate(b, seq, 0)


def slots(b: BlockManager, seq: Sequence, start: int, n: int) -> List[int]:
    """1-based cache slots of positions start .. start+n-1: (page - 1) P + offset + 1
    (src/kv/block_manager.jl:97-100)."""
    P = b.page_size
    return [(seq.block_table[p // P] - 1) * P + p % P + 1 for p in range(start, start + n)]


class Int8Pages:
    """One half (keys or values) of an INT8 layer (src/ops/quant.jl:86-92): `q`
    [pages][H][P][D] int8 and `scale` [pages][H][P] f32 are views of the layer arrays
    `layer_q` [2][pages][H][P][D] and `layer_scale` [2][pages][H][P]; `smooth` [D] holds
    the keys' smoothing factors (ones for values)."""

    def __init__(self, layer_q: torch.Tensor, layer_scale: torch.Tensor, smooth: torch.Tensor,
                 half: int):
        self.layer_q, self.layer_scale, self.smooth, self.half = layer_q, layer_scale, smooth, half
        self.q = layer_q[half]
        self.scale = layer_scale[half]

    @property
    def shape(self):
        return tuple(self.q.shape)

    def size(self, d: Optional[int] = None):
        return self.q.size() if d is None else self.q.size(d)


def int8_kv_pools(head_dim: int, page_size: int, kv_heads: int, num_pages: int,
                  key_smoothing: Optional[torch.Tensor] = None, device="cuda"):
    """The zeroed key and value Int8Pages of one layer (src/ops/quant.jl:104-109)."""
    q = torch.zeros((2, num_pages, kv_heads, page_size, head_dim), dtype=torch.int8, device=device)
    s = torch.zeros((2, num_pages, kv_heads, page_size), dtype=torch.float32, device=device)
    ks = (key_smoothing.to(device=device, dtype=torch.float32).contiguous() if key_smoothing is not None
          else torch.ones(head_dim, dtype=torch.float32, device=device))
    return Int8Pages(q, s, ks, 0), Int8Pages(q, s, torch.ones(head_dim, dtype=torch.float32, device=device), 1)


def key_smoothing(k_norm: torch.Tensor) -> torch.Tensor:
    """max(|w_i|, |w_j|) for each rotary pair (i, j = i + D/2), 1 where both are zero
    (src/ops/quant.jl:118-124)."""
    w = k_norm.float().abs()
    half = w.numel() // 2
    c = torch.maximum(w[:half], w[half:2 * half])
    c = torch.where(c > 0, c, torch.ones_like(c))
    return torch.cat([c, c])


def layer_arrays(k: Int8Pages, v: Int8Pages):
    """The layer arrays behind a key/value pair; both must be the halves of one layer
    made by int8_kv_pools (src/ops/quant.jl:131-135)."""
    if not (isinstance(k, Int8Pages) and isinstance(v, Int8Pages) and k.layer_q is v.layer_q
            and k.half == 0 and v.half == 1):
        raise ArgumentError("keys and values must be the halves of one layer's pools (int8_kv_pools)")
    return k.layer_q, k.layer_scale, k.smooth


class PagedKVCache:
    """Key/value pools for every layer and their page allocator (src/kv/paged_cache.jl:18-36).
    quantize=None: pools in `dtype`; quantize="int8": Int8Pages pairs."""

    def __init__(self, num_layers: int, head_dim: int, kv_heads: int, num_pages: int,
                 page_size: int = DEFAULT_PAGE_SIZE, dtype=torch.bfloat16, quantize=None,
                 key_smoothing=None, device="cuda"):
        self.blocks = BlockManager(num_pages, page_size)
        self.quantize = quantize
        if quantize is None:
            shape = (num_pages, kv_heads, page_size, head_dim)
            self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
            self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        elif quantize == "int8":
            pairs = [int8_kv_pools(head_dim, page_size, kv_heads, num_pages,
                                   None if key_smoothing is None else key_smoothing[l], device)
                     for l in range(num_layers)]
            self.k = [p[0] for p in pairs]
            self.v = [p[1] for p in pairs]
        else:
            raise ArgumentError(f"unsupported KV cache quantization {quantize} (only 'int8')")

    def page_size(self) -> int:
        return self.blocks.page_size

    def num_pages(self) -> int:
        return self.blocks.num_pages

    def new_sequence(self) -> Sequence:
        return Sequence()


def bytes_per_token(num_layers: int, kv_heads: int, head_dim: int, elt_bytes: int = 2,
                    quantize=None) -> int:
    """Cache bytes per cached position (src/kv/paged_cache.jl:43-47)."""
    if quantize == "int8":
        return 2 * num_layers * kv_heads * (head_dim + 4)
    return 2 * num_layers * kv_heads * head_dim * elt_bytes
