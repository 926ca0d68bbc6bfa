"""Pins the CPU oracle itself: every oracle function is checked against something other
than its own formula (brute force, closed forms, invariants, the reference tests' known
answers), chosen so that a dropped term, a wrong sign/index or a transposed operand fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import cache as C
from oracle import gemm as G
from oracle import norms as N

torch.manual_seed(0)


# ---- attention ----------------------------------------------------------------------

@pytest.mark.parametrize("causal", [None, 0, 2])
def test_ref_attention_matches_brute_force(causal):
    g = torch.Generator().manual_seed(1)
    q = torch.randn(3, 4, 8, generator=g)
    k = torch.randn(5, 2, 8, generator=g)
    v = torch.randn(5, 2, 8, generator=g)
    ref = A.ref_attention(q, k, v, 0.3, causal_offset=causal)
    brute = A.brute_attention(q, k, v, 0.3, causal_offset=causal)
    torch.testing.assert_close(ref, brute, atol=1e-5, rtol=1e-5)


def test_ref_attention_closed_forms():
    g = torch.Generator().manual_seed(2)
    v = torch.randn(7, 2, 16, generator=g)
    # all-zero q -> uniform weights -> mean of V (GQA: q heads 0,1 -> kv 0; 2,3 -> kv 1)
    q = torch.zeros(1, 4, 16)
    k = torch.randn(7, 2, 16, generator=g)
    out = A.ref_attention(q, k, v, 1.0)
    torch.testing.assert_close(out[0, 0], v[:, 0].mean(0))
    torch.testing.assert_close(out[0, 3], v[:, 1].mean(0))
    # one visible key -> that V row exactly
    out = A.ref_attention(torch.randn(1, 4, 16, generator=g), k, v, 1.0, causal_offset=0)
    torch.testing.assert_close(out[0, 2], v[0, 1])
    # key permutation invariance (full visibility)
    perm = torch.randperm(7, generator=g)
    q = torch.randn(2, 4, 16, generator=g)
    torch.testing.assert_close(A.ref_attention(q, k, v, 0.5), A.ref_attention(q, k[perm], v[perm], 0.5),
                               atol=1e-6, rtol=1e-5)


def test_decode_ref_gathers_by_indices():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 8, generator=g)
    kc = torch.randn(20, 2, 8, generator=g)
    vc = torch.randn(20, 2, 8, generator=g)
    idx = torch.tensor([5, 3, 9, 1, 0, 7], dtype=torch.int32)
    indptr = torch.tensor([0, 4, 6], dtype=torch.int32)
    out = A.decode_attention_ref(q, kc, vc, indptr, idx, 0.4)
    for b, sl in enumerate([[5, 3, 9, 1], [0, 7]]):
        sel = torch.tensor(sl)
        torch.testing.assert_close(out[b], A.brute_attention(q[b:b + 1], kc[sel], vc[sel], 0.4)[0],
                                   atol=1e-5, rtol=1e-5)


def test_split_geometry_known_values():
    # hand-computed: len 1000 in 3 splits -> ceil(334/32)*32 = 352
    assert A.kv_per_split(1000, 3, 0) == 352
    assert A.kv_per_split(33, 1, 0) == 64
    assert A.kv_per_split(31, 32, 0) == 32
    assert A.kv_per_split(5000, 7, 256) == 256
    # MI355X heuristic: 256 CUs, 8 kv heads: B=1 -> 64 -> capped 32; B=32 -> 2; B=64 -> 1
    assert A.plan_heuristic([1024], 256, 8, 32) == ([32], 32)
    assert A.plan_heuristic([100] * 32, 256, 8, 32)[1] == 2
    assert A.plan_heuristic([2049] * 64, 256, 8, 32) == ([1] * 64, 1)
    assert A.plan_heuristic([5, 100], 256, 8, 32) == ([1, 4], 32)
    assert A.plan_fixed([255, 256, 257, 1]) == ([1, 1, 2, 1], 2)


@pytest.mark.parametrize("seq_len", [1, 31, 32, 33, 255, 256, 257, 1000, 4097])
@pytest.mark.parametrize("n,fixed", [(1, 0), (3, 0), (8, 0), (32, 0), (64, 256)])
def test_split_ranges_tile_the_sequence(seq_len, n, fixed):
    n_req = n if fixed == 0 else -(-seq_len // fixed)
    rs = A.split_ranges(seq_len, min(n_req, -(-seq_len // 32)) if fixed == 0 else n_req, fixed)
    assert rs[0][0] == 0 and rs[-1][1] == seq_len
    assert all(a < b for a, b in rs)
    assert all(rs[i][1] == rs[i + 1][0] for i in range(len(rs) - 1))


@pytest.mark.parametrize("n_splits", [1, 2, 5, 17])
def test_split_merge_equals_full_softmax(n_splits):
    g = torch.Generator().manual_seed(4)
    L = 300
    q = torch.randn(4, 16, generator=g)
    k = torch.randn(L, 2, 16, generator=g)
    v = torch.randn(L, 2, 16, generator=g)
    ranges = A.split_ranges(L, n_splits, 0)
    merged = A.split_merge_ref(q, k, v, 0.25, ranges)
    full = A.ref_attention(q[None], k, v, 0.25)[0].double()
    torch.testing.assert_close(merged, full, atol=1e-5, rtol=1e-5)


def test_extend_ref_prefix_zero_is_causal_self_attention():
    g = torch.Generator().manual_seed(5)
    T = 9
    q = torch.randn(T, 4, 8, generator=g)
    kb = torch.randn(T + 3, 2, 8, generator=g)
    vb = torch.randn(T + 3, 2, 8, generator=g)
    idx = torch.tensor([4, 2, 11, 0, 7, 1, 3, 9, 5], dtype=torch.int32)
    qo = torch.tensor([0, T], dtype=torch.int32)
    out = A.extend_attention_ref(q, kb, vb, qo, qo, idx, 0.5)
    brute = A.brute_attention(q, kb[idx.long()], vb[idx.long()], 0.5, causal_offset=0)
    torch.testing.assert_close(out, brute, atol=1e-5, rtol=1e-5)
    # the last extend row with prefix p == decode attention over all p + e keys
    p, e = 5, 4
    qo2 = torch.tensor([0, e], dtype=torch.int32)
    kv2 = torch.tensor([0, p + e], dtype=torch.int32)
    ext = A.extend_attention_ref(q[:e], kb, vb, qo2, kv2, idx, 0.5)
    dec = A.decode_attention_ref(q[e - 1:e], kb, vb, kv2, idx, 0.5)
    torch.testing.assert_close(ext[-1], dec[0])


# ---- norms / rope / gemm -----------------------------------------------------------------

def test_rmsnorm_closed_forms():
    w = torch.randn(64)
    x = torch.full((1, 64), -3.0)
    torch.testing.assert_close(N.rmsnorm_ref(x, w, 0.0)[0], -w)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(5, 64, generator=g)
    torch.testing.assert_close(N.rmsnorm_ref(7.5 * x, w, 0.0), N.rmsnorm_ref(x, w, 0.0),
                               atol=1e-5, rtol=1e-5)
    y = N.rmsnorm_ref(x, torch.ones(64), 0.0)
    torch.testing.assert_close(y.pow(2).mean(-1), torch.ones(5), atol=1e-5, rtol=1e-5)


def test_fused_add_rmsnorm_semantics():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, 32, generator=g).to(torch.bfloat16)
    r = torch.randn(4, 32, generator=g).to(torch.bfloat16)
    w = torch.randn(32, generator=g).to(torch.bfloat16)
    out, res = N.fused_add_rmsnorm_ref(x, r, w, 1e-6)
    assert torch.equal(res, (x.float() + r.float()).to(torch.bfloat16))
    torch.testing.assert_close(out, N.rmsnorm_ref(x.float() + r.float(), w, 1e-6))


def test_rope_identity_norm_and_additivity():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(3, 2, 16, generator=g)
    theta = 1e6
    torch.testing.assert_close(N.rope_ref(x, torch.zeros(3, dtype=torch.int64), theta), x)
    pos = torch.tensor([1, 50, 999])
    y = N.rope_ref(x, pos, theta)
    n0 = x[..., :8] ** 2 + x[..., 8:] ** 2
    n1 = y[..., :8] ** 2 + y[..., 8:] ** 2
    torch.testing.assert_close(n0, n1, atol=1e-4, rtol=1e-4)
    z = N.rope_ref(N.rope_ref(x, pos, theta), torch.tensor([7, 7, 7]), theta)
    torch.testing.assert_close(z, N.rope_ref(x, pos + 7, theta), atol=1e-4, rtol=1e-4)
    # table layout [cos | sin]
    tab = N.rope_table_ref(16, 10, theta)
    assert tab.shape == (10, 16)
    torch.testing.assert_close(tab[3, 0], torch.tensor(math.cos(3.0)))
    torch.testing.assert_close(tab[3, 8], torch.tensor(math.sin(3.0)))


def test_silu_mul_halves():
    gu = torch.tensor([[0.0, 20.0, 2.0, 3.0]], dtype=torch.bfloat16)  # gate [0, 20], up [2, 3]
    out = N.silu_mul_ref(gu).float()
    assert out[0, 0] == 0.0
    assert abs(out[0, 1] - 60.0) < 0.5
    swapped = N.silu_mul_ref(torch.cat([gu[:, 2:], gu[:, :2]], -1)).float()
    assert not torch.equal(out, swapped)


def test_linear_ref_vs_float64():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(7, 96, generator=g).to(torch.bfloat16)
    w = torch.randn(40, 96, generator=g).to(torch.bfloat16)
    b = torch.randn(40, generator=g).to(torch.bfloat16)
    ref = G.linear_ref(x, w, b)
    exact = x.double() @ w.double().t() + b.double()
    torch.testing.assert_close(ref.double(), exact, atol=1e-4, rtol=1e-4)
    eye = torch.eye(96, dtype=torch.bfloat16)
    assert torch.equal(G.linear_ref(x, eye), x.float())


# ---- cache / indexing -----------------------------------------------------------------------

def test_reshape_and_cache_ref_reference_cases():
    # roundtrip + untouched slots stay zero (tests/test_04_reshape_and_cache.py:8-30)
    rng = np.random.default_rng(0)
    k = rng.integers(-30000, 30000, size=(10, 8, 128), dtype=np.int16)
    v = rng.integers(-30000, 30000, size=(10, 8, 128), dtype=np.int16)
    kc = np.zeros((50, 8, 128), np.int16)
    vc = np.zeros((50, 8, 128), np.int16)
    slots = rng.permutation(49)[:10] + 1
    C.reshape_and_cache_ref(k, v, kc, vc, slots)
    assert (kc[slots] == k).all() and (vc[slots] == v).all()
    mask = np.ones(50, bool)
    mask[slots] = False
    assert not kc[mask].any()
    # overwrite (:33-53) and -1 skip (:56-67)
    k2 = k + 1
    C.reshape_and_cache_ref(k2, v, kc, vc, slots)
    assert (kc[slots] == k2).all()
    kc[:] = 0
    C.reshape_and_cache_ref(k[:2], v[:2], kc, vc, np.array([-1, 2]))
    assert (kc[2] == k[1]).all() and not kc[0].any() and not kc[1].any()


def test_block_table_expansion_brute_force():
    rng = np.random.default_rng(1)
    bt = rng.permutation(256)[:64]
    idx = C.block_table_to_indices(bt, 1000)
    for pos in (0, 15, 16, 17, 999):
        assert idx[pos] == bt[pos // 16] * 16 + pos % 16
    assert len(set(idx.tolist())) == 1000


def test_decode_indices_brute_force():
    # page_size 1: the block table is the reference's request -> token table
    r2t = np.arange(40, dtype=np.int32).reshape(4, 10) * 3
    indptr, idx = C.decode_indices_ref(r2t, [2, 0], [3, 5])
    assert indptr.tolist() == [0, 3, 8]
    assert idx.tolist() == [60, 63, 66, 0, 3, 6, 9, 12]
    # pages of 4 slots: row 1 holds pages 7, 2, 9
    bt = np.zeros((3, 5), dtype=np.int32)
    bt[1, :3] = [7, 2, 9]
    indptr, idx = C.decode_indices_ref(bt, [1], [10], page_size=4)
    assert idx.tolist() == [28, 29, 30, 31, 8, 9, 10, 11, 36, 37]
