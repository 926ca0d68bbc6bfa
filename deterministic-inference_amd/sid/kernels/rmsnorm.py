"""RMSNorm ops (sid/kernels/rmsnorm.py of the reference): plain, fused residual-add, and
per-head q/k-norm. fp32 math with a fixed in-row reduction order, so results are
invariant to batch composition and row position in every mode."""

from __future__ import annotations

import torch

from sid.kernels.jit import load_ext


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x: [..., hidden] bf16 -> new tensor of the same shape."""
    shape = x.shape
    x2 = x.view(-1, shape[-1])
    assert x2.is_contiguous()
    out = torch.empty_like(x2)
    load_ext().rmsnorm(x2, weight, out, eps)
    return out.view(shape)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """In place: residual += x; x = rmsnorm(residual). Returns (x, residual)."""
    assert x.is_contiguous() and residual.is_contiguous()
    assert x.shape == residual.shape
    load_ext().fused_add_rmsnorm(x, residual, weight, eps)
    return x, residual


def qk_head_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-head RMSNorm (Qwen3 q/k-norm). x: [T, H, head_dim] -> same shape."""
    t, h, d = x.shape
    return rmsnorm(x.view(t * h, d), weight, eps).view(t, h, d)
