"""Small fused ops of the decode step that replace torch glue in sid/model/qwen3.py:
embedding lookup (:93), silu(gate) * up (:85), sampled-row gather (:113) and greedy
argmax (sid/engine/sampler.py:37)."""

from __future__ import annotations

import torch

from sid.kernels.jit import load_ext


def embedding(ids: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """F.embedding(ids, table) for int64 ids and a bf16 [V, H] table (bit copy)."""
    out = torch.empty(ids.numel(), table.shape[1], dtype=table.dtype, device=table.device)
    load_ext().gather_rows(table, ids.reshape(-1), out)
    return out.view(*ids.shape, table.shape[1])


def gather_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x[idx] for a 2-D bf16 x and int64 idx (bit copy)."""
    return embedding(idx, x)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """[T, 2I] -> [T, I]: F.silu(gate) * up with gate, up = gate_up.chunk(2, -1)."""
    t, two_i = gate_up.shape
    out = torch.empty(t, two_i // 2, dtype=gate_up.dtype, device=gate_up.device)
    load_ext().silu_mul(gate_up, out)
    return out


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """torch.argmax(logits, -1) for fp32 [R, V] (first index on ties)."""
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    load_ext().argmax_rows(logits, out)
    return out


def sample_rows(logits: torch.Tensor, temperatures: torch.Tensor, top_ks: torch.Tensor,
                top_ps: torch.Tensor, seeds: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Per-row greedy / temperature + top-k + top-p + seeded Gumbel-max draw (HIP)."""
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    load_ext().sample_rows(logits.contiguous(), temperatures.float().contiguous(),
                           top_ks.long().contiguous(), top_ps.float().contiguous(),
                           seeds.long().contiguous(), positions.long().contiguous(), out)
    return out


def silu_mul_partials(partials: torch.Tensor) -> torch.Tensor:
    """SwiGLU straight from the gate_up projection's chunk partials [C, T, 2I] -> [T, I]."""
    _, t, two_i = partials.shape
    out = torch.empty(t, two_i // 2, dtype=torch.bfloat16, device=partials.device)
    load_ext().silu_mul_partials(partials, out)
    return out


def fused_add_rmsnorm_partials(partials: torch.Tensor, residual: torch.Tensor,
                               weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """residual += bf16(fold(partials)); returns (rmsnorm(residual), residual)."""
    out = torch.empty_like(residual)
    load_ext().fused_add_rmsnorm_partials(partials, residual, weight, out, eps)
    return out, residual


def qkv_post(qkv_or_partials: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float,
             positions: torch.Tensor, cos_sin: torch.Tensor, slots: torch.Tensor,
             k_cache: torch.Tensor, v_cache: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    """Fused q/k-norm + RoPE + KV-cache write of a QKV projection (bf16 [T, W] or chunk
    partials [C, T, W]); returns q [T, HQ, D]."""
    partial = qkv_or_partials.dtype == torch.float32
    t = qkv_or_partials.shape[1] if partial else qkv_or_partials.shape[0]
    d = k_cache.shape[2]
    q = torch.empty(t, num_q_heads, d, dtype=torch.bfloat16, device=k_cache.device)
    load_ext().qkv_post(None if partial else qkv_or_partials, qkv_or_partials if partial else None,
                        q_norm, k_norm, eps, positions, cos_sin, slots, q, k_cache, v_cache)
    return q
