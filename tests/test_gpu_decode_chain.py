"""The fused decode chain (csrc/decode_chain.hip) is bit-identical to the unfused op
sequences it replaces (sid/model/qwen3.py:43-115 for one token per request):
  linear_residual + rmsnorm_f32   == linear + fused_add_rmsnorm     (residual and normed x)
  rmsnorm_linear_silu_mul         == rmsnorm / fused_add_rmsnorm + linear_silu_mul
  rmsnorm_qkv_post                == rmsnorm + linear + qkv_post     (q and both pools)
and a whole decode forward through the chain equals the unfused forward bit for bit. The
unfused ops are themselves pinned against the fp32 oracle (test_gpu_fused, test_gpu_gemm,
test_gpu_norm_rope); a torch fp32 check of each fused op is added here too."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D, H = 16, 8, 128, 1024
ROWS = [1, 5, 16, 37, 64, 100, 128, 161, 200, 256]


def _w(n, k, scale=0.03):
    return (torch.randn(n, k, device="cuda") * scale).to(torch.bfloat16)


@pytest.mark.parametrize("t", ROWS)
@pytest.mark.parametrize("k", [2048, 3072])
def test_linear_residual_matches_unfused(t, k):
    from sid.kernels.matmul_persistent import linear
    from sid.kernels.ops import linear_residual, pack_decode_weight, r32_positions, rmsnorm_f32
    from sid.kernels.rmsnorm import fused_add_rmsnorm
    inv = torch.argsort(r32_positions(H)).cuda()  # column order -> r32 order
    print(f"linear_residual t={t} k={k}", flush=True)
    torch.manual_seed(7 * t + k)
    x = torch.randn(t, k, device="cuda", dtype=torch.bfloat16)
    w = _w(H, k)
    nw = (1 + 0.1 * torch.randn(H, device="cuda")).to(torch.bfloat16)
    res = torch.randn(t, H, device="cuda", dtype=torch.bfloat16)
    h0, r0 = fused_add_rmsnorm(linear(x, w), res.clone(), nw, 1e-6)
    r1 = res.clone()
    r32 = torch.full((t, H), float("nan"), device="cuda")
    linear_residual(x, pack_decode_weight(w), r1, r32)
    r32_raw = r32.clone()
    assert torch.equal(r1, r0)
    r32 = r32[:, r32_positions(H).cuda()]  # column order
    assert torch.equal(r32.to(torch.bfloat16), r0)
    assert torch.equal(r32[:, inv], r32_raw)
    assert torch.equal(rmsnorm_f32(r32_raw, nw, 1e-6), h0)
    # fp32 torch reference of the residual sum (bf16 tolerance)
    ref = res.float() + (x.float() @ w.float().t())
    assert (r32 - ref).abs().max().item() <= 2e-2 * max(1.0, ref.abs().max().item())


@pytest.mark.parametrize("t", ROWS)
@pytest.mark.parametrize("src_fp32", [True, False])
def test_rmsnorm_linear_silu_mul_matches_unfused(t, src_fp32):
    from sid.kernels.matmul_persistent import linear_silu_mul
    from sid.kernels.ops import pack_decode_weight, rmsnorm_f32, rmsnorm_linear_silu_mul
    from sid.kernels.rmsnorm import rmsnorm
    print(f"rmsnorm_linear_silu_mul t={t} f32={src_fp32}", flush=True)
    torch.manual_seed(11 * t + src_fp32)
    src = torch.randn(t, H, device="cuda") * 3
    if not src_fp32:
        src = src.to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(H, device="cuda")).to(torch.bfloat16)
    w = _w(6144, H, 0.05)
    x = rmsnorm_f32(src, nw, 1e-6) if src_fp32 else rmsnorm(src, nw, 1e-6)
    want = linear_silu_mul(x, w)
    got = rmsnorm_linear_silu_mul(src, nw, 1e-6, pack_decode_weight(w, gate_up=True))
    assert torch.equal(got, want)


@pytest.mark.parametrize("t", ROWS)
@pytest.mark.parametrize("src_fp32", [True, False])
def test_rmsnorm_qkv_post_matches_unfused(t, src_fp32):
    from sid.kernels.matmul_persistent import linear
    from sid.kernels.ops import pack_decode_weight, qkv_post, rmsnorm_f32, rmsnorm_qkv_post
    from sid.kernels.rmsnorm import rmsnorm
    from sid.kernels.rope import RotaryEmbedding
    print(f"rmsnorm_qkv_post t={t} f32={src_fp32}", flush=True)
    torch.manual_seed(13 * t + src_fp32)
    src = torch.randn(t, H, device="cuda") * 2
    if not src_fp32:
        src = src.to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(H, device="cuda")).to(torch.bfloat16)
    w = _w((HQ + 2 * HKV) * D, H)
    qn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    rope = RotaryEmbedding(D, 4096, 1e6, "cuda")
    pos = torch.randint(0, 4096, (t,), device="cuda")
    if t > 1:
        pos[0] = 5000  # outside the table: left unrotated by both paths
    slots = torch.randperm(1000, device="cuda")[:t] + 1
    if t > 2:
        slots[1] = -1  # skipped by both paths
    x = rmsnorm_f32(src, nw, 1e-6) if src_fp32 else rmsnorm(src, nw, 1e-6)
    kc0 = torch.zeros(1024, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc0 = torch.zeros_like(kc0)
    q0 = qkv_post(linear(x, w), qn, kn, 1e-6, pos, rope.cos_sin, slots, kc0, vc0, HQ)
    kc1 = torch.zeros_like(kc0)
    vc1 = torch.zeros_like(kc0)
    q1 = rmsnorm_qkv_post(src, nw, 1e-6, pack_decode_weight(w), qn, kn, pos, rope.cos_sin, slots,
                          kc1, vc1, HQ)
    assert torch.equal(q1, q0)
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0)


@pytest.mark.parametrize("t", [3, 40, 128])
def test_hidden_512_chain_matches_unfused(t):
    """The hidden-512 instantiations (two 256-wide chunks per row): norm + gate_up + SwiGLU
    against rmsnorm + linear + silu_mul, norm + qkv + post against rmsnorm + linear +
    qkv_post, and the o-shaped residual projection (K = 1024) against linear +
    fused_add_rmsnorm, bitwise."""
    from sid.kernels.matmul_persistent import linear
    from sid.kernels.ops import (linear_residual, pack_decode_weight, qkv_post, r32_positions,
                                 rmsnorm_f32, rmsnorm_linear_silu_mul, rmsnorm_qkv_post, silu_mul)
    from sid.kernels.rmsnorm import fused_add_rmsnorm
    from sid.kernels.rope import RotaryEmbedding
    h = 512
    print(f"hidden 512 t={t}", flush=True)
    torch.manual_seed(17 + t)
    nw = (1 + 0.1 * torch.randn(h, device="cuda")).to(torch.bfloat16)
    # residual projection (K = 1024 -> N = 512) and the fp32 sum it leaves
    x = torch.randn(t, 1024, device="cuda", dtype=torch.bfloat16)
    wo = _w(h, 1024)
    res = torch.randn(t, h, device="cuda", dtype=torch.bfloat16)
    xn0, r0 = fused_add_rmsnorm(linear(x, wo), res.clone(), nw, 1e-6)
    r1, r32 = res.clone(), torch.empty(t, h, device="cuda")
    linear_residual(x, pack_decode_weight(wo), r1, r32)
    assert torch.equal(r1, r0)
    assert torch.equal(r32[:, r32_positions(h).cuda()].to(torch.bfloat16), r0)
    assert torch.equal(rmsnorm_f32(r32, nw, 1e-6), xn0)
    # norm + gate_up + SwiGLU from that sum
    wg = _w(2 * 1536, h, 0.05)
    want = silu_mul(linear(xn0, wg))
    got = rmsnorm_linear_silu_mul(r32, nw, 1e-6, pack_decode_weight(wg, gate_up=True))
    assert torch.equal(got, want)
    # norm + qkv + q/k-norm + RoPE + cache write (8 q heads, 4 kv heads)
    hq, hkv = 8, 4
    wq = _w((hq + 2 * hkv) * D, h)
    qn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    rope = RotaryEmbedding(D, 4096, 1e6, "cuda")
    pos = torch.randint(0, 4096, (t,), device="cuda")
    slots = torch.randperm(300, device="cuda")[:t]
    kc0 = torch.zeros(300, hkv, D, device="cuda", dtype=torch.bfloat16)
    vc0 = torch.zeros_like(kc0)
    q0 = qkv_post(linear(xn0, wq), qn, kn, 1e-6, pos, rope.cos_sin, slots, kc0, vc0, hq)
    kc1, vc1 = torch.zeros_like(kc0), torch.zeros_like(kc0)
    q1 = rmsnorm_qkv_post(r32, nw, 1e-6, pack_decode_weight(wq), qn, kn, pos, rope.cos_sin,
                          slots, kc1, vc1, hq)
    assert torch.equal(q1, q0)
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0)


def test_decode_chain_rows_are_batch_invariant():
    """A row's chain outputs do not depend on the batch around it (M-invariance), across the
    workgroup shapes the row count selects (16/32-column, 32/64-column, 16/32-row)."""
    from sid.kernels.ops import linear_residual, pack_decode_weight, rmsnorm_linear_silu_mul
    torch.manual_seed(3)
    big = torch.randn(200, 3072, device="cuda", dtype=torch.bfloat16)
    w = pack_decode_weight(_w(H, 3072))
    res = torch.randn(200, H, device="cuda", dtype=torch.bfloat16)
    wg = pack_decode_weight(_w(6144, H, 0.05), gate_up=True)
    nw = (1 + 0.1 * torch.randn(H, device="cuda")).to(torch.bfloat16)
    r_all, f_all = res.clone(), torch.empty(200, H, device="cuda")
    linear_residual(big, w, r_all, f_all)
    act_all = rmsnorm_linear_silu_mul(f_all, nw, 1e-6, wg)
    for lo, hi in ((0, 1), (17, 18), (40, 57), (100, 200), (199, 200)):
        r_part, f_part = res[lo:hi].clone(), torch.empty(hi - lo, H, device="cuda")
        linear_residual(big[lo:hi].contiguous(), w, r_part, f_part)
        assert torch.equal(r_part, r_all[lo:hi]) and torch.equal(f_part, f_all[lo:hi])
        assert torch.equal(rmsnorm_linear_silu_mul(f_part, nw, 1e-6, wg), act_all[lo:hi])
    # the qkv kernel (16-row workgroups up to 128 rows, 32-row ones above)
    from sid.kernels.ops import rmsnorm_qkv_post
    from sid.kernels.rope import RotaryEmbedding
    wq = pack_decode_weight(_w((HQ + 2 * HKV) * D, H))
    qn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    rope = RotaryEmbedding(D, 4096, 1e6, "cuda")
    pos = torch.randint(0, 4096, (200,), device="cuda")
    slots = torch.randperm(400, device="cuda")[:200]

    def qkv(lo, hi):
        kc = torch.zeros(400, HKV, D, device="cuda", dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        q = rmsnorm_qkv_post(f_all[lo:hi].contiguous(), nw, 1e-6, wq, qn, kn, pos[lo:hi],
                             rope.cos_sin, slots[lo:hi], kc, vc, HQ)
        return q, kc[slots[lo:hi]], vc[slots[lo:hi]]

    q_all, k_all, v_all = qkv(0, 200)
    for lo, hi in ((0, 1), (40, 57), (100, 200), (199, 200)):
        q, k, v = qkv(lo, hi)
        assert torch.equal(q, q_all[lo:hi]) and torch.equal(k, k_all[lo:hi])
        assert torch.equal(v, v_all[lo:hi])


def test_pack_decode_weight_layout():
    """packed[b][c][s][lane] = row(b, lane % 16), cols 256 c + 32 s + 8 (lane // 16) .. +7."""
    from sid.kernels.ops import pack_decode_weight
    torch.manual_seed(4)
    for n, k, gu in ((64, 512, False), (48, 768, True)):
        w = torch.randn(n, k, device="cuda").to(torch.bfloat16)
        p = pack_decode_weight(w, gate_up=gu).cpu().view(n // 16, k // 256, 8, 64, 8)
        wc = w.cpu()
        if gu:  # block b = [gate rows 8b..8b+7 | up rows inter + 8b..]
            inter = n // 2
            wc = torch.cat([wc[:inter].view(inter // 8, 8, k), wc[inter:].view(inter // 8, 8, k)],
                           1).view(n, k)
        want = wc.view(n // 16, 16, k // 256, 8, 4, 8).permute(0, 2, 3, 4, 1, 5).reshape(p.shape)
        assert torch.equal(p, want)


@pytest.mark.parametrize("bs", [1, 13, 64, 100, 200])
def test_decode_forward_chain_equals_unfused(bs):
    """Whole decode forward (2 layers of the Qwen3-0.6B shape): chain == unfused, bitwise,
    logits and KV pools."""
    from sid.config import ModelConfig
    from sid.engine.batch import ForwardBatch, ForwardMode
    from sid.kernels.decode_attention import DecodeAttention
    from sid.model.loader import random_weights
    from sid.model.qwen3 import Qwen3Model
    print(f"decode chain forward bs={bs}", flush=True)
    mcfg = ModelConfig(num_layers=2)
    w = random_weights(mcfg, "cuda", seed=5)
    torch.manual_seed(bs)
    ctx = 40
    slots_per = ctx + 1
    pools = [torch.randn(bs * slots_per + 16, HKV, D, device="cuda").to(torch.bfloat16)
             for _ in range(4)]

    class Pool:
        def __init__(self, p):
            self.p = p

        def layer(self, i):
            return self.p[2 * i], self.p[2 * i + 1]

    lens = torch.randint(1, ctx + 1, (bs,))
    indptr = torch.zeros(bs + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(lens, 0)
    idx = torch.cat([torch.arange(i * slots_per, i * slots_per + int(n)) for i, n in
                     enumerate(lens)]).to(torch.int32)
    out_slots = torch.tensor([i * slots_per + int(n) - 1 for i, n in enumerate(lens)])
    fb = ForwardBatch(mode=ForwardMode.DECODE,
                      input_ids=torch.randint(0, mcfg.vocab_size, (bs,), device="cuda"),
                      positions=(lens - 1).cuda(), out_slots=out_slots.cuda(),
                      kv_indptr=indptr.cuda(), kv_indices=idx.cuda(),
                      seq_lens=lens.to(torch.int32).cuda(), max_seq_len=int(lens.max()))
    attn = DecodeAttention(max(bs, 64), HQ, HKV, D, 32, 256, 4096, "cuda")
    outs = []
    for chain in (False, True):
        model = Qwen3Model(mcfg, w, "cuda")
        model.decode_chain = chain
        pool = Pool([p.clone() for p in pools])
        logits = model.forward(fb, pool, attn, decode_backend="hip")
        outs.append((logits, pool.p))
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)
