"""Decode-step GEMMs (HIP MFMA) vs fp32, and the M-invariance of every row (bitwise).
Shapes: the reference's tests/test_10_batch_invariant.py:18-38 plus the Qwen3-0.6B decode
(M=64) and verify (M=128) projections."""

from __future__ import annotations

import pytest
import torch

from oracle.gemm import linear_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k", [
    (1, 1024, 1024), (7, 3072, 1024), (128, 151936, 1024), (500, 1024, 3072),
    (64, 4096, 1024), (64, 1024, 2048), (64, 6144, 1024), (64, 1024, 3072), (64, 151936, 1024),
    (128, 6144, 1024), (33, 64, 256), (200, 128, 512), (64, 2048, 1024),
])
def test_linear_vs_fp32(m, n, k):
    from sid.kernels.matmul_persistent import linear
    torch.manual_seed(0)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(n, k, device="cuda") * 0.05).to(torch.bfloat16)
    out = linear(x, w)
    ref = linear_ref(x.cpu(), w.cpu())
    torch.testing.assert_close(out.float().cpu(), ref, atol=3e-2, rtol=2e-2)


def test_bias_and_fp32_output():
    from sid.kernels.matmul_persistent import bi_linear, linear, matmul_persistent
    torch.manual_seed(1)
    x = torch.randn(9, 512, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(128, 512, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(128, device="cuda", dtype=torch.bfloat16)
    y = bi_linear(x, w, b)
    torch.testing.assert_close(y.float().cpu(), linear_ref(x.cpu(), w.cpu(), b.cpu()), atol=2e-1, rtol=2e-2)
    y32 = linear(x, w, b, out_fp32=True)
    assert y32.dtype == torch.float32 and torch.equal(y32.to(torch.bfloat16), y)
    assert torch.equal(matmul_persistent(x, w.t(), b), y)


def test_row_invariance():
    from sid.kernels.matmul_persistent import bi_linear
    torch.manual_seed(2)
    x0 = torch.randn(1, 1024, device="cuda", dtype=torch.bfloat16)
    for n in (3072, 151936):
        w = (torch.randn(n, 1024, device="cuda") * 0.05).to(torch.bfloat16)
        alone = bi_linear(x0, w)
        for m in (2, 64, 65, 333):
            x = torch.cat([torch.randn(m - 1, 1024, device="cuda", dtype=torch.bfloat16), x0])
            assert torch.equal(alone[0], bi_linear(x, w)[-1]), (n, m)


def test_strided_input_rows():
    from sid.kernels.matmul_persistent import linear
    torch.manual_seed(3)
    big = torch.randn(16, 2048, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(64, 1024, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(linear(big[:, :1024], w), linear(big[:, :1024].contiguous(), w))


@pytest.mark.parametrize("m,n,k", [(64, 4096, 1024), (64, 1024, 2048), (64, 6144, 1024),
                                   (64, 1024, 3072), (5, 1024, 3072), (1, 4096, 1024),
                                   (100, 1024, 2048), (512, 1024, 2048), (1024, 1024, 3072),
                                   (300, 4096, 1024)])
def test_partials_fold_equals_linear(m, n, k):
    """Chunk partials folded in increasing chunk order and rounded to bf16 equal sid_linear
    bit for bit (the contract the *_partials consumers rely on)."""
    from sid.kernels.matmul_persistent import linear, linear_partials
    torch.manual_seed(4)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(n, k, device="cuda") * 0.05).to(torch.bfloat16)
    p = linear_partials(x, w)
    assert p.shape == (k // 256, m, n)
    fold = p[0].clone()
    for c in range(1, p.shape[0]):
        fold += p[c]
    assert torch.equal(fold.to(torch.bfloat16), linear(x, w))


@pytest.mark.parametrize("m", [1, 16, 33, 64, 100, 128, 256])
def test_stream_lm_head_path_bitwise_matches_tiled(m):
    """lm_head-shaped GEMMs (K=1024, N >= 32768, M<=256 in 64-row groups) take the persistent
    streaming kernel;
    its bits equal the tiled kernel's (checked on the first and last 4096 columns, which
    the tiled kernel computes separately), for fp32 and bf16 outputs."""
    from sid.kernels.matmul_persistent import linear
    torch.manual_seed(6)
    print(f"m={m}", flush=True)
    x = torch.randn(m, 1024, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(151936, 1024, device="cuda") * 0.05).to(torch.bfloat16)
    full = linear(x, w, out_fp32=True)              # streaming kernel
    head = linear(x, w[:4096].contiguous(), out_fp32=True)  # tiled kernel (small N)
    tail = linear(x, w[-4096:].contiguous(), out_fp32=True)
    assert torch.equal(full[:, :4096], head)
    assert torch.equal(full[:, -4096:], tail)
    assert torch.equal(linear(x, w), full.to(torch.bfloat16))
    ref = x.float().cpu() @ w[:2048].float().cpu().t()
    torch.testing.assert_close(full[:, :2048].cpu(), ref, atol=3e-2, rtol=2e-2)


@pytest.mark.parametrize("m,n,k", [(1, 151936, 1024), (7, 151936, 1024), (33, 65536, 1024),
                                   (64, 151936, 1024), (64, 4096, 1024), (65, 151936, 1024),
                                   (128, 151936, 1024), (200, 65536, 1024), (300, 151936, 1024),
                                   (512, 151936, 1024), (100, 1088, 512), (3, 4096, 2048)])
def test_linear_argmax_matches_linear_then_argmax(m, n, k):
    """Fused lm_head + greedy argmax == argmax_rows(linear(..., out_fp32=True)), and the
    optional logits output equals linear's: the streaming path (up to 64 rows, K = 1024)
    and the tiled GEMM's argmax epilogue (more rows, other K, a ragged last column tile)."""
    from sid.kernels.matmul_persistent import linear, linear_argmax
    from sid.kernels.ops import argmax_rows
    torch.manual_seed(7 + m)
    print(f"m={m} n={n} k={k}", flush=True)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(n, k, device="cuda") * 0.05).to(torch.bfloat16)
    logits = linear(x, w, out_fp32=True)
    want = argmax_rows(logits)
    assert torch.equal(linear_argmax(x, w), want)
    lg = torch.empty(m, n, device="cuda")
    assert torch.equal(linear_argmax(x, w, logits=lg), want)
    assert torch.equal(lg, logits)


@pytest.mark.parametrize("m", [4, 130])
def test_linear_argmax_ties_and_nan(m):
    """Equal maxima -> first column; a NaN logit wins over every number, first NaN first
    (torch.argmax semantics), also when the tied columns land in different waves (streaming
    path) or column tiles (tiled path)."""
    from sid.kernels.matmul_persistent import linear_argmax
    torch.manual_seed(8)
    n = 151936
    x = torch.randn(m, 1024, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(n, 1024, device="cuda") * 0.01).to(torch.bfloat16)
    hot = (x[0].float() / x[0].float().norm()).to(torch.bfloat16)
    for c in (150000, 70001, 70000, 123):   # identical rows: identical logits for every x
        w[c] = hot
    got = linear_argmax(x, w).cpu()
    assert got[0].item() == 123
    want = torch.argmax(x.float().cpu() @ w.float().cpu().t(), dim=-1)
    assert got[0].item() == want[0].item()
    w[90000, 5] = float("nan")
    w[80000, 7] = float("nan")
    got = linear_argmax(x, w).cpu()
    assert (got == 80000).all()



@pytest.mark.parametrize("m,n,k", [(256, 1024, 1024), (300, 1024, 2048), (1000, 6144, 1024),
                                   (2048, 4096, 1024), (777, 192, 512), (4100, 1024, 3072)])
def test_tiled_large_m_bitwise_matches_row_group_kernel(m, n, k):
    """M >= 64 takes the LDS-tiled MFMA kernel (128 x 128 or 128 x 64 tiles); its bits
    equal the 64-row-group kernel's on row slices of fewer than 64 rows, and its own on a
    129-row slice, with bias, both output dtypes, ragged M and N tails."""
    from sid.kernels.matmul_persistent import linear
    torch.manual_seed(m + n)
    print(f"m={m} n={n} k={k}", flush=True)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(n, k, device="cuda") * 0.05).to(torch.bfloat16)
    b = torch.randn(n, device="cuda", dtype=torch.bfloat16)
    for bias in (None, b):
        full = linear(x, w, bias)
        for lo, hi in ((0, 63), (m - 33, m), (m // 2, m // 2 + 129)):
            assert torch.equal(full[lo:hi], linear(x[lo:hi].contiguous(), w, bias)), (lo, hi)
    f32 = linear(x, w, out_fp32=True)
    assert torch.equal(f32.to(torch.bfloat16), linear(x, w))
    ref = x[:64].float().cpu() @ w.float().cpu().t()
    torch.testing.assert_close(f32[:64].cpu(), ref, atol=3e-2, rtol=2e-2)
