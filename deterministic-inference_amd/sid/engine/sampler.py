"""Row-independent sampler shared by decode and the DVR verifier (sid/engine/sampler.py).

Greedy rows: argmax with first-index ties (HIP kernel). Stochastic rows: top-k / top-p,
then seeded Gumbel-max whose uniform is a hash of (seed, sample position, vocab id), so a
request's draw at a position is the same in any batch and on either path. No reduction
crosses rows. When the caller knows every row is greedy (`all_greedy`), no device->host
synchronisation happens here.
"""

from __future__ import annotations

from typing import Optional

import torch

from sid.kernels.ops import argmax_rows

_EPS = 1e-10


def _seeded_gumbel(seeds: torch.Tensor, sample_pos: torch.Tensor, num_cols: int) -> torch.Tensor:
    step = seeds * 19349663 ^ sample_pos * 73856093
    cols = torch.arange(num_cols, dtype=torch.int64, device=seeds.device)
    hashed = step.unsqueeze(-1) * 8589934591 ^ cols * 479001599
    uniform = (hashed % (2 ** 24)).float() / (2 ** 24)
    return -torch.log(-torch.log(uniform + _EPS) + _EPS)


def sample(logits: torch.Tensor, temperatures: torch.Tensor, top_ks: torch.Tensor,
           top_ps: torch.Tensor, seeds: torch.Tensor, sample_pos: torch.Tensor,
           all_greedy: Optional[bool] = None) -> torch.Tensor:
    """logits fp32 [R, V] -> int64 [R]."""
    if logits.is_cuda:
        greedy = argmax_rows(logits.contiguous())
    else:
        greedy = torch.argmax(logits, dim=-1)
    if all_greedy is None:
        all_greedy = not bool((temperatures > 0).any())
    if all_greedy:
        return greedy
    stochastic = temperatures > 0
    temps = torch.where(stochastic, temperatures, torch.ones_like(temperatures))
    probs = torch.softmax(logits / temps.unsqueeze(-1), dim=-1)
    probs_sort, probs_idx = probs.sort(dim=-1, descending=True)
    cum = torch.cumsum(probs_sort, dim=-1)
    drop = (cum - probs_sort) > top_ps.unsqueeze(-1)
    vocab = probs.shape[-1]
    ranks = torch.arange(vocab, device=probs.device).expand_as(probs_sort)
    k = torch.where(top_ks > 0, top_ks, torch.full_like(top_ks, vocab))
    drop |= ranks >= k.unsqueeze(-1)
    drop[:, 0] = False
    keep = torch.zeros_like(drop)
    keep.scatter_(-1, probs_idx, ~drop)
    log_probs = torch.where(keep, torch.log(probs + _EPS), torch.full_like(probs, float("-inf")))
    sampled = torch.argmax(log_probs + _seeded_gumbel(seeds, sample_pos, vocab), dim=-1)
    return torch.where(stochastic, sampled, greedy)
