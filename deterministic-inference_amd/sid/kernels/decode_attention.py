"""Decode attention: split-KV HIP kernel plus the num_splits policy.

Policy (kept exactly as sid/kernels/decode_attention.py:1-17, 56-85 of the reference,
with the device's compute-unit count as its input):

* nondet / dvr: ``splits = clamp(ceil(2 * CUs / (B * HKV)), 1, max_kv_splits)``, then per
  request ``min(splits, ceil(len / 32))``; the grid has ``splits`` slots. The split count
  depends on the batch size, so a request's bits depend on its co-tenants: this is the
  designed nondeterminism of the fast path.
* batch_invariant: fixed 256-token splits, ``ceil(len / 256)`` per request, grid
  ``ceil(max_len / 256)``; a request's result depends only on its own length.

On MI355X (256 CUs) a batch of 64 with 8 KV heads gets one split per request; the
kernel then writes the output directly and skips the merge pass.
"""

from __future__ import annotations

import functools

import torch

from sid.kernels.jit import load_ext


@functools.lru_cache(maxsize=8)
def _cu_count(device_index: int) -> int:
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def heuristic_splits(batch: int, num_kv_heads: int, cu_count: int, max_kv_splits: int) -> int:
    """Grid split count of the nondet/dvr policy (reference decode_attention.py:73-74)."""
    splits = -(-2 * cu_count // (batch * num_kv_heads))
    return max(1, min(splits, max_kv_splits))


class DecodeAttention:
    """Owns the persistent split workspace (fixed pointers across steps)."""

    def __init__(self, max_batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 max_kv_splits: int, invariant_split_size: int, max_seq_len: int, device: str):
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_kv_splits = max_kv_splits
        self.invariant_split_size = invariant_split_size
        self.invariant_max_splits = -(-max_seq_len // invariant_split_size)
        self.ws_splits = max(max_kv_splits, self.invariant_max_splits)
        self.part_o = torch.empty(max_batch, num_q_heads, self.ws_splits, head_dim,
                                  dtype=torch.float32, device=device)
        self.part_lse = torch.empty(max_batch, num_q_heads, self.ws_splits,
                                    dtype=torch.float32, device=device)
        self.device = torch.device(device)
        self.ext = load_ext()
        self._plan_src = None
        self._plan = None

    def reset_plan(self) -> None:
        """Forget the cached split plan (called at the start of every forward)."""
        self._plan_src = None
        self._plan = None

    def cu_count(self) -> int:
        idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
        return _cu_count(idx)

    def plan(self, seq_lens: torch.Tensor, max_seq_len: int, invariant: bool):
        """(num_splits int32 [B] on device, grid splits, fixed split size)."""
        bs = seq_lens.shape[0]
        if invariant:
            tile = self.invariant_split_size
            num_splits = ((seq_lens + tile - 1) // tile).to(torch.int32)
            return num_splits, max(1, -(-max_seq_len // tile)), tile
        splits = heuristic_splits(bs, self.num_kv_heads, self.cu_count(), self.max_kv_splits)
        num_splits = torch.clamp((seq_lens + 31) // 32, max=splits).to(torch.int32)
        return num_splits, splits, 0

    def forward(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                kv_indptr: torch.Tensor, kv_indices: torch.Tensor, seq_lens: torch.Tensor,
                max_seq_len: int, sm_scale: float, invariant: bool) -> torch.Tensor:
        """q: [B, HQ, D] bf16 -> o: [B, HQ, D] bf16 (max_seq_len is host-side, no sync)."""
        bs = q.shape[0]
        assert bs <= self.part_o.shape[0], "decode batch exceeds workspace"
        # One plan per forward: every layer sees the same seq_lens tensor.
        key = (invariant, max_seq_len, bs)
        if self._plan_src is seq_lens and self._plan[0] == key:
            num_splits, grid_splits, fixed = self._plan[1]
        else:
            num_splits, grid_splits, fixed = self.plan(seq_lens, max_seq_len, invariant)
            self._plan_src, self._plan = seq_lens, (key, (num_splits, grid_splits, fixed))
        o = torch.empty_like(q)
        self.ext.flash_decode_fwd(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                                  grid_splits, fixed, sm_scale, self.part_o, self.part_lse, o)
        return o
