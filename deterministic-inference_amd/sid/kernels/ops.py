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


# ---- the decode-step chain (csrc/decode_chain.hip) -----------------------------------------

def r32_positions(hidden: int) -> torch.Tensor:
    """Where column c of an r32 row is stored (int64 [hidden]): the RMSNorm lane order of
    csrc/decode_chain.hip (element 8 v + e, v = j + 64 i, at i*512 + (e//4)*256 + 4 j + e%4),
    so `r32[:, r32_positions(h)]` is the row in column order."""
    col = torch.arange(hidden)
    v, e = col >> 3, col & 7
    return (v >> 6) * 512 + (e >> 2) * 256 + 4 * (v & 63) + (e & 3)


def pack_decode_weight(weight: torch.Tensor, gate_up: bool = False) -> torch.Tensor:
    """The fragment-packed copy of a [N, K] projection weight that the decode-chain kernels
    read (same shape and values, another order; gate_up: [gate rows | up rows])."""
    out = torch.empty_like(weight)
    load_ext().pack_decode_weight(weight.contiguous(), out, gate_up)
    return out


def linear_residual(x: torch.Tensor, packed: torch.Tensor, residual: torch.Tensor,
                    r32: torch.Tensor) -> None:
    """In place: r = residual + bf16(x @ weight^T) (fp32), residual = bf16(r), r32 = r stored
    in the RMSNorm lane order (r32_positions): the projection plus the residual half of
    fused_add_rmsnorm (sid/kernels/rmsnorm.py:27-42). packed = pack_decode_weight(weight)."""
    load_ext().linear_residual(x, packed, residual, r32)


def rmsnorm_linear_silu_mul(src: torch.Tensor, norm_w: torch.Tensor, eps: float,
                            weight: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up of bf16(rmsnorm(src) * norm_w) @ gate_up^T; src an r32 (fp32, lane
    order) or bf16 rows in column order, [T, H]; weight = pack_decode_weight(gate_up,
    gate_up=True)."""
    out = torch.empty(src.shape[0], weight.shape[0] // 2, dtype=torch.bfloat16, device=src.device)
    load_ext().rmsnorm_linear_silu_mul(src, norm_w, eps, weight, out)
    return out


def rmsnorm_qkv_post(src: torch.Tensor, norm_w: torch.Tensor, eps: float, weight: torch.Tensor,
                     q_norm: torch.Tensor, k_norm: torch.Tensor, positions: torch.Tensor,
                     cos_sin: torch.Tensor, slots: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    """qkv_post of the qkv projection of bf16(rmsnorm(src) * norm_w); returns q [T, HQ, D].
    weight = pack_decode_weight(qkv)."""
    d = k_cache.shape[2]
    q = torch.empty(src.shape[0], num_q_heads, d, dtype=torch.bfloat16, device=src.device)
    load_ext().rmsnorm_qkv_post(src, norm_w, eps, weight, q_norm, k_norm, positions, cos_sin,
                                slots, q, k_cache, v_cache)
    return q


def rmsnorm_f32(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16(rmsnorm(x) * weight) for r32 rows (fp32 in the lane order of r32_positions);
    sid.kernels.rmsnorm.rmsnorm's bits on the same values."""
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    load_ext().rmsnorm_f32(x, weight, out, eps)
    return out


def decode_chain_supported(rows: int, hidden: int, intermediate: int, q_size: int,
                           head_dim: int) -> bool:
    """Whether the fused decode chain serves this model shape (rows: decode batch size)."""
    return (1 <= rows <= DECODE_CHAIN_MAX_ROWS and hidden in (512, 1024) and head_dim == 128
            and intermediate % 24 == 0 and intermediate % 256 == 0
            and q_size % 256 == 0 and q_size <= 4096 and intermediate <= 4096 and hidden % 128 == 0)


# Decode batches up to this many rows take the fused chain; larger ones the split-K /
# tiled projections with separate norm kernels (identical bits either way). The chain's
# workgroups re-read their weight tiles once per 16 (32) rows, so large batches favour the
# tiled GEMMs. 28-layer chain without attention, weights from HBM, graph-timed (us per
# layer, chain vs split-K path): 32 rows 26.9 vs 30.1, 64: 27.0 vs 36.1, 128: 31.0 vs 45.4
# (32-column workgroups from 96 rows); above 128 rows (32-row qkv and 64-column o / down
# workgroups) whole decode steps: 160 rows 7.83 vs 7.96 ms, 192: 8.57 vs 8.70, 256: 11.12 vs
# 11.30. Past 256 rows the chain's workgroups outnumber the CUs again.
DECODE_CHAIN_MAX_ROWS = 256
