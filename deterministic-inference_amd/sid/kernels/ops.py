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
