"""Rotary tables, built once on the host as src/model/rope.jl:9-48 builds them:
inverse frequencies and angles in Float32, cos/sin evaluated in Float64 on the Float32
angle, rounded to Float32, then to the model's element type.

`cos_sin` is [max_len][2][D] (row 2p = cos of position p, row 2p + 1 = its sin), the
C-order form of the reference's interleaved (D, 2 max_len) table; `cos`/`sin` are
[max_len][D]. The table is an input of the kernels, so kernel parity does not depend on
how it is built (libm's powf here, Julia's `^` in the reference).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch


@dataclass
class Llama3RopeScaling:
    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position_embeddings: int


def inverse_frequencies(head_dim: int, theta: float,
                        scaling: Optional[Llama3RopeScaling] = None) -> np.ndarray:
    """1 / theta^(i/D) for i = 0, 2, ..., D-2, in Float32 (src/model/rope.jl:15-21)."""
    ex = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv = np.float32(1.0) / np.power(np.float32(theta), ex, dtype=np.float32)
    return inv if scaling is None else llama3_scaled(inv, scaling)


def llama3_scaled(inv_freq: np.ndarray, s: Llama3RopeScaling) -> np.ndarray:
    """transformers' _compute_llama3_parameters (src/model/rope.jl:27-38), in Float32."""
    f32 = np.float32
    factor, low, high = f32(s.factor), f32(s.low_freq_factor), f32(s.high_freq_factor)
    old_len = f32(s.original_max_position_embeddings)
    low_wl, high_wl = old_len / low, old_len / high
    out = np.empty_like(inv_freq)
    for i, f in enumerate(inv_freq.astype(np.float32)):
        wl = f32(2) * f32(np.pi) / f
        if wl < high_wl:
            out[i] = f
        elif wl > low_wl:
            out[i] = f / factor
        else:
            smooth = (old_len / wl - low) / (high - low)
            out[i] = (f32(1) - smooth) * f / factor + smooth * f
    return out


class RotaryTable:
    """Per-position cos/sin tables on the device (src/model/rope.jl:9-13, 40-48)."""

    def __init__(self, cos: torch.Tensor, sin: torch.Tensor, cos_sin: torch.Tensor):
        self.cos, self.sin, self.cos_sin = cos, sin, cos_sin

    def __len__(self) -> int:
        return self.cos.shape[0]

    @classmethod
    def build(cls, head_dim: int, max_len: int, theta: float, dtype=torch.bfloat16,
              scaling: Optional[Llama3RopeScaling] = None, device="cuda") -> "RotaryTable":
        inv = inverse_frequencies(head_dim, theta, scaling)
        pos = np.arange(max_len, dtype=np.float32)
        ang = (pos[:, None] * inv[None, :]).astype(np.float32)        # [max_len][D/2]
        ang = np.concatenate([ang, ang], axis=1)                          # both halves
        c = np.cos(ang.astype(np.float64)).astype(np.float32)
        s = np.sin(ang.astype(np.float64)).astype(np.float32)
        return cls.from_arrays(torch.from_numpy(c), torch.from_numpy(s), dtype, device)

    @classmethod
    def from_arrays(cls, cos: torch.Tensor, sin: torch.Tensor, dtype=torch.bfloat16,
                    device="cuda") -> "RotaryTable":
        c = cos.to(dtype).to(device).contiguous()
        s = sin.to(dtype).to(device).contiguous()
        cs = torch.stack([c, s], dim=1).contiguous()                     # [max_len][2][D]
        return cls(c, s, cs)
