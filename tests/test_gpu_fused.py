"""Fused decode-path kernels are bit-identical to the unfused op sequences they replace:
  qkv_post  == split + contiguous + qk_head_rmsnorm(q), (k) + RoPE + reshape_and_cache
               (sid/model/qwen3.py:49-61), fed by linear or by linear_partials;
  fused_add_rmsnorm_partials == linear + fused_add_rmsnorm;
  silu_mul_partials          == linear + silu_mul;
  linear_silu_mul            == linear_partials + silu_mul_partials."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _ext():
    from sid.kernels.jit import load_ext
    return load_ext()


@pytest.mark.parametrize("t", [1, 7, 64, 300])
@pytest.mark.parametrize("use_partials", [False, True])
def test_qkv_post_matches_unfused(t, use_partials):
    from sid.kernels.matmul_persistent import linear, linear_partials
    from sid.kernels.ops import qkv_post
    from sid.kernels.rmsnorm import qk_head_rmsnorm
    from sid.kernels.rope import RotaryEmbedding
    torch.manual_seed(t)
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn((HQ + 2 * HKV) * D, 1024, device="cuda") * 0.03).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    rope = RotaryEmbedding(D, 4096, 1e6, "cuda")
    pos = torch.randint(0, 4096, (t,), device="cuda")
    pos[0] = 5000 if t > 1 else pos[0]  # out of the table: left unrotated by both paths
    slots = torch.randperm(1000, device="cuda")[:t] + 1
    if t > 2:
        slots[1] = -1  # skipped by both paths
    # unfused reference path
    qkv = linear(x, w)
    q, k, v = qkv.split([HQ * D, HKV * D, HKV * D], dim=-1)
    q = qk_head_rmsnorm(q.contiguous().view(t, HQ, D), qn, 1e-6)
    k = qk_head_rmsnorm(k.contiguous().view(t, HKV, D), kn, 1e-6)
    v = v.contiguous().view(t, HKV, D)
    rope.apply(q, k, pos)
    kc0 = torch.zeros(1024, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc0 = torch.zeros_like(kc0)
    _ext().reshape_and_cache(k, v, kc0, vc0, slots)
    # fused
    kc1 = torch.zeros_like(kc0)
    vc1 = torch.zeros_like(kc0)
    src = linear_partials(x, w) if use_partials else qkv
    q1 = qkv_post(src, qn, kn, 1e-6, pos, rope.cos_sin, slots, kc1, vc1, HQ)
    assert torch.equal(q1, q)
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0)


@pytest.mark.parametrize("t,k", [(1, 2048), (64, 2048), (33, 3072), (300, 3072), (1024, 2048),
                                 (1024, 3072)])
def test_fused_add_rmsnorm_partials_matches_unfused(t, k):
    from sid.kernels.matmul_persistent import linear, linear_partials
    from sid.kernels.ops import fused_add_rmsnorm_partials
    from sid.kernels.rmsnorm import fused_add_rmsnorm
    torch.manual_seed(k + t)
    x = torch.randn(t, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(1024, k, device="cuda") * 0.03).to(torch.bfloat16)
    nw = torch.randn(1024, device="cuda", dtype=torch.bfloat16)
    res = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    h, r0 = fused_add_rmsnorm(linear(x, w), res.clone(), nw, 1e-6)
    out, r1 = fused_add_rmsnorm_partials(linear_partials(x, w), res.clone(), nw, 1e-6)
    assert torch.equal(r1, r0) and torch.equal(out, h)


@pytest.mark.parametrize("t", [1, 64])
def test_silu_mul_partials_matches_unfused(t):
    from sid.kernels.matmul_persistent import linear, linear_partials
    from sid.kernels.ops import silu_mul, silu_mul_partials
    torch.manual_seed(t)
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(6144, 1024, device="cuda") * 0.05).to(torch.bfloat16)
    assert torch.equal(silu_mul_partials(linear_partials(x, w)), silu_mul(linear(x, w)))


@pytest.mark.parametrize("t", [1, 5, 16, 33, 64, 65, 128, 200, 256, 300, 1000, 2048])
@pytest.mark.parametrize("inter", [3072, 192, 96])
def test_linear_silu_mul_matches_unfused(t, inter):
    """gate_up projection + SwiGLU in one launch == linear_partials + silu_mul_partials (and
    == linear + silu_mul), bit for bit, on full and ragged 64-row groups; from 256 rows the
    tiled GEMM with the SwiGLU epilogue in each of its tile shapes (inter 96 keeps the small-M
    kernel)."""
    from sid.kernels.matmul_persistent import linear, linear_partials, linear_silu_mul
    from sid.kernels.ops import silu_mul, silu_mul_partials
    print(f"linear_silu_mul t={t} inter={inter}", flush=True)
    torch.manual_seed(1000 * t + inter)
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(2 * inter, 1024, device="cuda") * 0.05).to(torch.bfloat16)
    fused = linear_silu_mul(x, w)
    assert torch.equal(fused, silu_mul_partials(linear_partials(x, w)))
    assert torch.equal(fused, silu_mul(linear(x, w)))
    # torch fp32 reference of the same op (bf16 tolerance)
    gu = (x.float() @ w.float().t())
    ref = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    assert (fused.float() - ref).abs().max().item() <= 2e-2 * max(1.0, ref.abs().max().item())
