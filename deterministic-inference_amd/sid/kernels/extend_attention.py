"""Varlen causal attention over the paged pool (prefill, DVR verify, decode fallback).

Same contract as sid/kernels/extend_attention.py:115-144 of the reference: the extend
tokens' K/V are already in the pool (reshape_and_cache ran first), kv_indptr covers the
full sequence (prefix + extend), query j of a request is at absolute position prefix + j.
Key tiles are anchored at absolute position 0, which makes every query's result bitwise
invariant to the window offset and to co-batched requests (the DVR requirement).
"""

from __future__ import annotations

import torch

from sid.kernels.jit import load_ext


def extend_attention_fwd(q_extend: torch.Tensor, k_buffer: torch.Tensor, v_buffer: torch.Tensor,
                         qo_indptr: torch.Tensor, kv_indptr: torch.Tensor,
                         kv_indices: torch.Tensor, max_extend_len: int,
                         sm_scale: float) -> torch.Tensor:
    assert q_extend.is_contiguous()
    assert k_buffer.is_contiguous() and v_buffer.is_contiguous()
    o_extend = torch.empty_like(q_extend)
    load_ext().extend_attention_fwd(q_extend, k_buffer, v_buffer, qo_indptr, kv_indptr,
                                    kv_indices, max_extend_len, sm_scale, o_extend)
    return o_extend
