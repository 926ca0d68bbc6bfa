"""Row-independent sampler shared by decode and the DVR verifier (sid/engine/sampler.py).

Every row is drawn by one HIP kernel (`sid_sample_rows`): greedy rows (temperature 0) take
the argmax with first-index ties; stochastic rows take softmax(logits / T), the top-k /
top-p truncation of the reference (sid/engine/sampler.py:45-58, with the mass before a
rank summed exactly in fixed point), and the seeded Gumbel-max draw whose noise is a hash
of (seed, sample position, vocab id) (sampler.py:22-29), so a request's draw at a position
is the same in any batch and on either path. No reduction crosses rows. An all-greedy batch
(`all_greedy`, known on the host) takes the plain argmax kernel; nothing here synchronises
with the device.
"""

from __future__ import annotations

from typing import Optional

import torch

from sid.kernels.ops import argmax_rows, sample_rows


def sample(logits: torch.Tensor, temperatures: torch.Tensor, top_ks: torch.Tensor,
           top_ps: torch.Tensor, seeds: torch.Tensor, sample_pos: torch.Tensor,
           all_greedy: Optional[bool] = None) -> torch.Tensor:
    """logits fp32 [R, V] on the GPU -> int64 [R] token ids."""
    if not logits.is_cuda:
        raise RuntimeError("sample: logits must be on the GPU (the sampler is a HIP kernel)")
    if all_greedy:
        return argmax_rows(logits.contiguous())
    return sample_rows(logits, temperatures, top_ks, top_ps, seeds, sample_pos)
