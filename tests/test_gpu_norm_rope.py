"""RMSNorm / fused add-norm / q-k head norm / RoPE / SwiGLU (HIP) vs the fp32 oracle
(the reference's tests/test_01_triton_ops.py cases) and row-invariance (bitwise)."""

from __future__ import annotations

import pytest
import torch

from oracle.norms import fused_add_rmsnorm_ref, rmsnorm_ref, rope_ref, silu_mul_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t", [1, 7, 32, 128, 4096])
def test_rmsnorm(t):
    from sid.kernels.rmsnorm import rmsnorm
    torch.manual_seed(0)
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(1024, device="cuda", dtype=torch.bfloat16)
    out = rmsnorm(x, w, 1e-6)
    torch.testing.assert_close(out.float().cpu(), rmsnorm_ref(x.cpu(), w.cpu(), 1e-6), atol=2e-2, rtol=2e-2)
    # a row's bits do not depend on how many rows are normalised with it
    assert torch.equal(rmsnorm(x[:1].clone(), w, 1e-6)[0], out[0])


@pytest.mark.parametrize("t", [1, 7, 32, 128, 4096])
def test_fused_add_rmsnorm(t):
    from sid.kernels.rmsnorm import fused_add_rmsnorm
    torch.manual_seed(1)
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    r = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(1024, device="cuda", dtype=torch.bfloat16)
    ref_out, ref_res = fused_add_rmsnorm_ref(x.cpu(), r.cpu(), w.cpu(), 1e-6)
    out, res = fused_add_rmsnorm(x.clone(), r.clone(), w, 1e-6)
    assert torch.equal(res.cpu(), ref_res)  # bf16(x + r): exact
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("t", [1, 33, 500])
def test_qk_head_rmsnorm(t):
    from sid.kernels.rmsnorm import qk_head_rmsnorm
    torch.manual_seed(2)
    x = torch.randn(t, 16, 128, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(128, device="cuda", dtype=torch.bfloat16)
    out = qk_head_rmsnorm(x, w, 1e-6)
    torch.testing.assert_close(out.float().cpu(), rmsnorm_ref(x.cpu(), w.cpu(), 1e-6), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("t", [1, 5, 257])
def test_rope_matches_hf(t):
    from sid.kernels.rope import RotaryEmbedding
    torch.manual_seed(3)
    rope = RotaryEmbedding(128, 8192, 1e6, "cuda")
    q = torch.randn(t, 16, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(t, 8, 128, device="cuda", dtype=torch.bfloat16)
    pos = torch.randint(0, 8192, (t,), device="cuda", dtype=torch.int64)
    rq, rk = rope_ref(q.cpu(), pos.cpu(), 1e6), rope_ref(k.cpu(), pos.cpu(), 1e6)
    rope.apply(q, k, pos)
    torch.testing.assert_close(q.float().cpu(), rq, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(k.float().cpu(), rk, atol=2e-2, rtol=2e-2)


def test_rope_out_of_range_position_untouched():
    from sid.kernels.rope import RotaryEmbedding
    rope = RotaryEmbedding(128, 64, 1e6, "cuda")
    q = torch.randn(2, 16, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 8, 128, device="cuda", dtype=torch.bfloat16)
    q0, k0 = q.clone(), k.clone()
    rope.apply(q, k, torch.tensor([64, 0], device="cuda"))
    assert torch.equal(q[0], q0[0]) and torch.equal(k[0], k0[0])
    assert torch.equal(q[1], q0[1])  # position 0 is the identity rotation


def test_silu_mul():
    from sid.kernels.ops import silu_mul
    torch.manual_seed(4)
    gu = (torch.randn(64, 6144, device="cuda") * 3).to(torch.bfloat16)
    out = silu_mul(gu)
    ref = silu_mul_ref(gu.cpu())
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=2e-2, rtol=2e-2)
    exact = (out.cpu() == ref).float().mean().item()
    assert exact > 0.99, exact


@pytest.mark.parametrize("hidden", [1024, 2048, 4096, 96 * 8])
def test_rmsnorm_row_layouts_bitwise(hidden):
    """Below 1024 rows each row gets its own 256-thread workgroup; from 1024 rows up, the
    lane-group kernel runs. Both must give the same bits for a row (batch invariance)."""
    from sid.kernels.rmsnorm import fused_add_rmsnorm, rmsnorm
    torch.manual_seed(hidden)
    x = torch.randn(1100, hidden, device="cuda", dtype=torch.bfloat16) * 3
    r = torch.randn(1100, hidden, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(hidden, device="cuda", dtype=torch.bfloat16)
    print(f"hidden={hidden}", flush=True)
    big = rmsnorm(x, w, 1e-6)
    small = rmsnorm(x[:70].clone(), w, 1e-6)
    assert torch.equal(small, big[:70])
    hb, rb = fused_add_rmsnorm(x.clone(), r.clone(), w, 1e-6)
    hs, rs = fused_add_rmsnorm(x[:5].clone(), r[:5].clone(), w, 1e-6)
    assert torch.equal(rs, rb[:5]) and torch.equal(hs, hb[:5])


def test_fused_add_rmsnorm_partials_row_layouts_bitwise():
    from sid.kernels.matmul_persistent import linear_partials
    from sid.kernels.ops import fused_add_rmsnorm_partials
    torch.manual_seed(5)
    x = torch.randn(1030, 3072, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(1024, 3072, device="cuda") * 0.03).to(torch.bfloat16)
    nw = torch.randn(1024, device="cuda", dtype=torch.bfloat16)
    res = torch.randn(1030, 1024, device="cuda", dtype=torch.bfloat16)
    hb, rb = fused_add_rmsnorm_partials(linear_partials(x, w), res.clone(), nw, 1e-6)
    hs, rs = fused_add_rmsnorm_partials(linear_partials(x[:64].clone(), w), res[:64].clone(), nw, 1e-6)
    assert torch.equal(rs, rb[:64]) and torch.equal(hs, hb[:64])
