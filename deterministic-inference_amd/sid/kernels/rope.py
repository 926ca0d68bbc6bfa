"""Rotary position embedding, NeoX rotate-half (Qwen3), applied in place to Q and K.

Table layout follows sid/kernels/rope.py:40-48 of the reference: fp32 [max_pos, D] =
[cos(D/2) | sin(D/2)] with inv_freq = theta^(-i / (D/2)). The table is computed once in
float64 on the device and rounded to fp32.
"""

from __future__ import annotations

import torch

from sid.kernels.jit import load_ext


def rope_table(head_dim: int, max_positions: int, theta: float, device) -> torch.Tensor:
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float64, device=device) / half))
    pos = torch.arange(max_positions, dtype=torch.float64, device=device)
    freqs = torch.outer(pos, inv_freq)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).to(torch.float32).contiguous()


class RotaryEmbedding:
    def __init__(self, head_dim: int, max_positions: int, theta: float, device: str):
        self.head_dim = head_dim
        self.max_positions = max_positions
        self.cos_sin = rope_table(head_dim, max_positions, theta, device)

    def apply(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor) -> None:
        """In place. q: [T, HQ, D] bf16, k: [T, HKV, D] bf16, positions: int64 [T]."""
        t, _, head_dim = q.shape
        assert head_dim == self.head_dim and q.is_contiguous() and k.is_contiguous()
        if t == 0:
            return
        load_ext().rope_apply(q, k, positions, self.cos_sin)
