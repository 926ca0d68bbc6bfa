"""Bit-exact byte kernels vs the numpy oracle: reshape_and_cache (the reference's
tests/test_04_reshape_and_cache.py cases plus out-of-range slots), row gathers
(embedding / sampled rows), device-side decode index construction, argmax."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HKV, D
from oracle.cache import decode_indices_ref, reshape_and_cache_ref

pytestmark = pytest.mark.gpu


def _ext():
    from sid.kernels.jit import load_ext
    return load_ext()


def _i16(t):
    return t.cpu().view(torch.int16).numpy()


def test_scatter_roundtrip_untouched_zero():
    torch.manual_seed(0)
    t, slots = 100, 500
    k = torch.randn(t, HKV, D, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(t, HKV, D, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(slots, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    mapping = (torch.randperm(slots - 1, device="cuda")[:t] + 1).to(torch.int64)
    _ext().reshape_and_cache(k, v, kc, vc, mapping)
    rk, rv = np.zeros((slots, HKV, D), np.int16), np.zeros((slots, HKV, D), np.int16)
    reshape_and_cache_ref(_i16(k), _i16(v), rk, rv, mapping.cpu().numpy())
    assert (_i16(kc) == rk).all() and (_i16(vc) == rv).all()
    assert torch.equal(kc[mapping], k) and torch.equal(vc[mapping], v)


def test_overwrite_same_slots():
    torch.manual_seed(1)
    t = 32
    kc = torch.zeros(t + 8, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    mapping = torch.arange(1, t + 1, device="cuda", dtype=torch.int64)
    for _ in range(2):
        k = torch.randn(t, HKV, D, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(t, HKV, D, device="cuda", dtype=torch.bfloat16)
        _ext().reshape_and_cache(k, v, kc, vc, mapping)
    assert torch.equal(kc[mapping], k) and torch.equal(vc[mapping], v)


def test_negative_and_out_of_range_slots_skipped():
    k = torch.randn(3, HKV, D, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(3, HKV, D, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(4, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    _ext().reshape_and_cache(k, v, kc, vc, torch.tensor([-1, 2, 4], device="cuda"))
    assert torch.equal(kc[2], k[1]) and torch.equal(vc[2], v[1])
    assert torch.count_nonzero(kc[[0, 1, 3]]) == 0


def test_large_pool_scatter_bit_exact():
    """T=128 rows (a verify pass) into a 524,288-slot pool, int64 slot addressing."""
    torch.manual_seed(2)
    slots = 32768 * 16
    kc = torch.zeros(slots, HKV, D, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    mapping = (torch.randperm(slots - 1, device="cuda")[:128] + 1).to(torch.int64)
    k = torch.randn(128, HKV, D, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(128, HKV, D, device="cuda", dtype=torch.bfloat16)
    _ext().reshape_and_cache(k, v, kc, vc, mapping)
    assert torch.equal(kc[mapping], k) and torch.equal(vc[mapping], v)
    assert int(torch.count_nonzero(kc.view(slots, -1).any(1))) <= 128


def test_gather_rows_and_embedding():
    from sid.kernels.ops import embedding
    torch.manual_seed(3)
    table = torch.randn(1000, 1024, device="cuda", dtype=torch.bfloat16)
    ids = torch.tensor([5, 0, 999, 5, 17], device="cuda")
    assert torch.equal(embedding(ids, table), table[ids])
    bad = torch.tensor([3, -1, 1000], device="cuda")
    out = embedding(bad, table)
    assert torch.equal(out[0], table[3]) and torch.count_nonzero(out[1:]) == 0


def test_build_decode_indices_vs_oracle():
    rng = np.random.default_rng(4)
    r2t = rng.integers(1, 10 ** 6, size=(8, 300)).astype(np.int32)
    rows = [3, 1, 6]
    lens = [5, 300, 1]
    new = [777, 888, 999]
    r2t_after = r2t.copy()
    for r, L, s in zip(rows, lens, new):
        r2t_after[r, L - 1] = s
    want_ptr, want_idx = decode_indices_ref(r2t_after, rows, lens)
    dev = torch.from_numpy(r2t).cuda()
    ptr = torch.from_numpy(want_ptr).cuda()
    out = torch.full((int(want_ptr[-1]),), -7, dtype=torch.int32, device="cuda")
    _ext().build_decode_indices(dev, torch.tensor(rows, device="cuda"),
                                torch.tensor(new, device="cuda"), ptr, out)
    assert out.cpu().numpy().tolist() == want_idx.tolist()
    assert (dev.cpu().numpy() == r2t_after).all()


def test_argmax_first_index_and_nan():
    from sid.kernels.ops import argmax_rows
    torch.manual_seed(5)
    x = torch.randn(7, 151936, device="cuda")
    x[1, 100] = x[1, 90000] = 1e9
    x[2] = 0.0
    x[3, 5000] = float("nan")
    x[3, 7000] = float("nan")
    x[4, -1] = float("inf")
    got = argmax_rows(x)
    assert got.tolist() == torch.argmax(x.cpu(), dim=-1).tolist()
    assert got[1] == 100 and got[2] == 0 and got[3] == 5000
