"""Varlen causal attention over the paged pool (prefill, DVR verify, decode fallback).

Same contract as sid/kernels/extend_attention.py:115-144 of the reference: the extend
tokens' K/V are already in the pool (reshape_and_cache ran first), kv_indptr covers the
full sequence (prefix + extend), query j of a request is at absolute position prefix + j.
Keys are reduced in 256-position splits anchored at absolute position 0 and folded in split
order, which makes every query's result bitwise invariant to the window offset and to
co-batched requests (the DVR requirement); small grids fan the splits out over more
workgroups with the same bits.
"""

from __future__ import annotations

import torch

from sid.kernels.jit import load_ext


def extend_attention_fwd(q_extend: torch.Tensor, k_buffer: torch.Tensor, v_buffer: torch.Tensor,
                         qo_indptr: torch.Tensor, kv_indptr: torch.Tensor,
                         kv_indices: torch.Tensor, max_extend_len: int,
                         sm_scale: float, max_kv_len: int | None = None) -> torch.Tensor:
    """max_kv_len (an extension of the reference signature): an upper bound of every
    request's kv length; defaults to kv_indices.numel(), which needs no device sync."""
    assert q_extend.is_contiguous()
    assert k_buffer.is_contiguous() and v_buffer.is_contiguous()
    ext = load_ext()
    if max_kv_len is None or max_kv_len <= 0:
        max_kv_len = kv_indices.numel()
    o_extend = torch.empty_like(q_extend)
    need = ext.extend_attention_workspace_bytes(qo_indptr.numel() - 1, q_extend.shape[0],
                                                q_extend.shape[1], k_buffer.shape[1],
                                                max_extend_len, max_kv_len)
    ws = torch.empty(need, dtype=torch.uint8, device=q_extend.device) if need else None
    ext.extend_attention_fwd(q_extend, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices,
                             max_extend_len, sm_scale, o_extend, max_kv_len, ws)
    return o_extend
