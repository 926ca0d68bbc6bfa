"""GEMM oracle: y = x @ w^T (+ bias) in fp32 on the CPU.

Restates F.linear as used at sid/model/qwen3.py:49, 80, 84, 86, 114 and the math of
sid/kernels/matmul_persistent.py:82-113. Pinned by float64 matmul (tests compare the
fp32 result against it) and by an identity weight returning x exactly.
The tolerance of the reference's own GEMM test is tests/test_10_batch_invariant.py:24
(atol 3e-1, rtol 3e-2 against cuBLAS bf16).
"""

from __future__ import annotations

import torch


def linear_ref(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    y = x.float() @ w.float().t()
    if bias is not None:
        y = y + bias.float()
    return y
