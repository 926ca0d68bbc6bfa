"""RMSNorm / RoPE / SwiGLU oracles (fp32, CPU).

rmsnorm_ref          restates tests/test_01_triton_ops.py:13-15 and the kernel
                     sid/kernels/rmsnorm.py:14-24. Pinned by closed forms: a constant row
                     c maps to sign(c) * w (up to eps), scaling x by a leaves the output
                     unchanged, and mean(y^2 / w^2) == 1.
fused_add_rmsnorm_ref  restates sid/kernels/rmsnorm.py:27-42 (the residual is stored as
                     bf16; the norm reads the fp32 sum). Pinned by: residual == bf16(x + r)
                     exactly, and output == rmsnorm_ref of the fp32 sum.
rope_table_ref / rope_ref  restate sid/kernels/rope.py:41-48 and the HF NeoX formula of
                     tests/test_01_triton_ops.py:72-81. Pinned by: position 0 is the
                     identity, every (x_i, x_{i+D/2}) pair keeps its norm, and rotating by
                     p1 then p2 equals rotating by p1 + p2 (angle additivity).
silu_mul_ref         restates sid/model/qwen3.py:85 (F.silu(gate) * up in bf16). Pinned by
                     silu(0) = 0, silu(x) -> x for large x, and gate/up halves swapped
                     giving a different result (catches a transposed chunk).
"""

from __future__ import annotations

import torch


def rmsnorm_ref(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def fused_add_rmsnorm_ref(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor, eps: float):
    """-> (normed fp32, new residual bf16)."""
    r = x.float() + residual.float()
    return rmsnorm_ref(r, w, eps), r.to(torch.bfloat16)


def rope_table_ref(head_dim: int, max_positions: int, theta: float) -> torch.Tensor:
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float64) / half))
    freqs = torch.outer(torch.arange(max_positions, dtype=torch.float64), inv_freq)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).float()


def rope_ref(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """x [T, H, D] -> fp32 rotated copy (HF rotate-half convention)."""
    d = x.shape[-1]
    half = d // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float64) / half))
    freqs = positions.double()[:, None] * inv_freq[None, :]
    cos = freqs.cos().float()[:, None, :]
    sin = freqs.sin().float()[:, None, :]
    xf = x.float()
    x1, x2 = xf[..., :half], xf[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def silu_mul_ref(gate_up: torch.Tensor) -> torch.Tensor:
    """bf16 [T, 2I] -> bf16 [T, I] with torch's bf16 rounding of each op."""
    gate, up = gate_up.chunk(2, dim=-1)
    return torch.nn.functional.silu(gate) * up
