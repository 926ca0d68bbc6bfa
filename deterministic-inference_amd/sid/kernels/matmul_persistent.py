"""Decode-step GEMMs on bf16 MFMA with a fixed, M-independent reduction order.

`linear` replaces F.linear on the model path; `bi_linear` / `matmul_persistent` keep the
names and signatures of sid/kernels/matmul_persistent.py:82-113. Every output element is
reduced in the same order whatever M is (K in 256-wide chunks, chunk sums folded in
increasing order), so `bi_linear` and `linear` are the same kernel: rows are bitwise
batch-invariant in every mode, and the batch_invariant mode costs nothing extra here.
"""

from __future__ import annotations

from typing import Optional

import torch

from sid.kernels.jit import load_ext

def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out_fp32: bool = False) -> torch.Tensor:
    """y = x @ weight^T (+ bias). x: [..., K] bf16, weight: [N, K] bf16 -> [..., N].

    out_fp32=True returns fp32 holding the bf16-rounded result (F.linear(...).float())."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    n = weight.shape[0]
    y = torch.empty(x2.shape[0], n, device=x.device,
                    dtype=torch.float32 if out_fp32 else torch.bfloat16)
    load_ext().linear(x2, weight, bias, y, out_fp32)
    return y.view(*shape[:-1], n)


def matmul_persistent(a: torch.Tensor, b: torch.Tensor,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C = A @ B (+ bias). A: [M, K], B: [K, N] (a transposed [N, K] view is used as is)."""
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    w = b.t()
    if not w.is_contiguous():
        w = w.contiguous()
    return linear(a, w, bias)


def bi_linear(x: torch.Tensor, weight: torch.Tensor,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Drop-in for F.linear(x, weight, bias) with batch-invariant reduction."""
    return linear(x, weight, bias)


def linear_partials(x: torch.Tensor, weight: torch.Tensor,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Split-K chunk sums fp32 [K/256, M, N] of x @ weight^T (fold in order + round to bf16
    = linear(x, weight) bit for bit); consumed by the *_partials fused ops."""
    m, k = x.shape
    n = weight.shape[0]
    if out is None:
        out = torch.empty(k // 256, m, n, dtype=torch.float32, device=x.device)
    load_ext().linear_partials(x, weight, out)
    return out


# sid_linear_silu_mul (gate_up projection + SwiGLU in one launch, no projection written)
# serves every row count at K = 1024: up to 95 rows a kernel in which every workgroup reads
# its rows' whole x for 16 output columns (against the split-K pair it saves a launch and the
# fp32 partials' round trip: M=1 8.0 -> 5.2 us, M=32 9.9 -> 6.8, M=64 12.5 -> 9.3), from 96
# rows the tiled GEMM with the SwiGLU in its epilogue (M=128 15.6 -> 12.8 us, M=192
# 20.7 -> 12.5, M=2048 48.2 -> 38.4 against linear + silu_mul). Same bits everywhere.
def linear_silu_mul_preferred(m: int, k: int) -> bool:
    """Shapes where linear_silu_mul is used for the MLP's first half (K = 1024)."""
    return m >= 1 and k == 1024


def linear_silu_mul(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.silu(gate) * up of (gate, up) = (x @ weight^T).chunk(2, -1), as one launch: the same
    bits as silu_mul_partials(linear_partials(x, weight)). x [M, 1024] bf16 -> [M, N/2]."""
    out = torch.empty(x.shape[0], weight.shape[0] // 2, dtype=torch.bfloat16, device=x.device)
    load_ext().linear_silu_mul(x, weight, out)
    return out


def linear_argmax_supported(m: int, k: int) -> bool:
    """Shapes the fused lm_head + greedy argmax takes: any row count (up to 64 rows one
    streaming pass over the weights, more rows the tiled GEMM with the argmax in its
    epilogue; neither writes logits unless asked), K a multiple of 256."""
    return m >= 1 and k > 0 and k % 256 == 0


def linear_argmax(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                  logits: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """argmax(x @ weight^T + bias, dim=-1) as int64 [M], the logits being exactly those of
    linear(..., out_fp32=True) (written to `logits` when given). Greedy sampling fused into
    the lm_head GEMM; needs linear_argmax_supported(M, K)."""
    m, k = x.shape
    ext = load_ext()
    if workspace is None:
        workspace = torch.empty(ext.linear_argmax_workspace_bytes(m), dtype=torch.uint8,
                                device=x.device)
    if out is None:
        out = torch.empty(m, dtype=torch.int64, device=x.device)
    ext.linear_argmax(x, weight, bias, logits, workspace, out)
    return out


def linear_sample_supported(m: int, k: int, tiles: Optional[bool] = None) -> bool:
    """Shapes the fused lm_head + sampler kernel takes for a grouping (see linear_sample):
    K = 1024; M <= 256 for the streaming waves (tiles=False), M <= 4096 otherwise (above
    64 rows tiles=None means the tiles)."""
    return k == 1024 and 1 <= m <= (256 if tiles is False else 4096)


def linear_sample(x: torch.Tensor, weight: torch.Tensor, temperatures: torch.Tensor,
                  seeds: torch.Tensor, positions: torch.Tensor,
                  workspace: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None,
                  recompute_all: bool = False, tiles: Optional[bool] = None,
                  logits: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Tokens int64 [M] drawn from the logits x @ weight^T: greedy rows (temperature 0) take
    the argmax, the others the seeded Gumbel-max draw of sid/engine/sampler.py:32-69 with no
    top-k / top-p limit. The logits are exactly those of linear(..., out_fp32=True) (written
    to `logits` when given, else not at all); needs linear_sample_supported(M, K).
    A row's token depends on the row and on how the softmax sum is grouped: tiles=None picks
    by speed (streaming waves up to 64 rows, 128-column tiles above or with logits);
    tiles=True / False fix the tiles / the streaming waves, for callers whose tokens must not
    depend on the batch size. recompute_all scores every column exactly instead of
    certifying per-group candidates (a check; slow)."""
    m, k = x.shape
    ext = load_ext()
    if workspace is None:
        workspace = torch.empty(ext.linear_sample_workspace_bytes(m), dtype=torch.uint8,
                                device=x.device)
    if out is None:
        out = torch.empty(m, dtype=torch.int64, device=x.device)
    ext.linear_sample(x, weight, temperatures.float().contiguous(), seeds.long().contiguous(),
                      positions.long().contiguous(), workspace, out, recompute_all, tiles, logits)
    return out
