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


@pytest.mark.parametrize("page_size", [1, 16])
def test_build_paged_decode_indices_vs_oracle(page_size):
    """Bit-exact vs the block-table expansion; a request whose new token opens a page gets
    that page recorded in its table row, and no other table entry changes."""
    rng = np.random.default_rng(4)
    rows_n, max_pages = 8, 300 // page_size + 2
    tables = rng.integers(1, 5000, size=(rows_n, max_pages)).astype(np.int32)
    rows = [3, 1, 6, 2]
    lens = [5, 300, 1, 2 * page_size + 1]
    # new token slots: position L-1 of each request; a page-opening position gets a fresh page
    after = tables.copy()
    new = []
    for r, L in zip(rows, lens):
        pos = L - 1
        if pos % page_size == 0:
            page = 9000 + r
            after[r, pos // page_size] = page
        else:
            page = tables[r, pos // page_size]
        new.append(page * page_size + pos % page_size)
    want_ptr, want_idx = decode_indices_ref(after, rows, lens, page_size)
    dev = torch.from_numpy(tables).cuda()
    ptr = torch.from_numpy(want_ptr).cuda()
    out = torch.full((int(want_ptr[-1]),), -7, dtype=torch.int32, device="cuda")
    _ext().build_paged_decode_indices(dev, page_size, torch.tensor(rows, device="cuda"),
                                      torch.tensor(new, device="cuda"), ptr, out)
    assert out.cpu().numpy().tolist() == want_idx.tolist()
    assert (dev.cpu().numpy() == after).all()


def test_paged_kv_cache_decode_matches_block_tables():
    """The engine's page allocator + device index build over several decode steps with a
    rollback in between: every step's kv_indices equal the host block tables' expansion
    (oracle), and a rollback returns exactly the pages that became empty."""
    from sid.config import EngineConfig, ModelConfig
    from sid.engine.batch import build_decode_batch
    from sid.engine.kv_cache import KVCache
    from sid.engine.request import Request
    from sid.config import SamplingParams
    cfg = EngineConfig(kv_pool_tokens=64 * 16, max_reqs=8, max_seq_len=256, kv_page_size=16)
    kv = KVCache(cfg, ModelConfig(num_layers=1), "cuda")
    kv.scatter_free_pages(3)
    reqs = []
    for i, (p, n) in enumerate([(15, 1), (16, 1), (40, 3)]):
        r = Request(i, list(range(p)), SamplingParams(max_new_tokens=100), (0,))
        r.req_row = kv.open_row()
        kv.grow(r.req_row, p + n - 1)
        r.output_ids = [5] * n
        reqs.append(r)
    kv.sync_rows([r.req_row for r in reqs])
    free0 = kv.free_pages
    for step in range(40):
        fb = build_decode_batch(reqs, kv, "cuda", invariant=False)
        lens = [r.kv_len + 1 for r in reqs]
        want_ptr, want_idx = decode_indices_ref(kv.tables, [r.req_row for r in reqs], lens, 16)
        assert fb.kv_indices.cpu().numpy().tolist() == want_idx.tolist(), step
        assert fb.out_slots.cpu().tolist() == [int(want_idx[e - 1]) for e in want_ptr[1:]]
        for r in reqs:
            r.output_ids.append(7)
        if step == 25:  # roll request 2 back by 20 tokens
            r = reqs[2]
            del r.output_ids[-20:]
            before = int(kv.held[r.req_row])
            kv.shrink(r.req_row, r.kv_len)
            assert kv.held[r.req_row] == kv.pages_for(r.kv_len) < before
    assert kv.free_pages == free0 - sum(kv.pages_for(r.kv_len) - kv.pages_for(p + n - 1)
                                        for r, (p, n) in zip(reqs, [(15, 1), (16, 1), (40, 3)]))
    for r in reqs:
        kv.close_row(r.req_row)
    assert kv.free_pages == kv.num_pages - 1


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


@pytest.mark.parametrize("cols", [33, 4001, 8192 * 4 + 3, 151936])
def test_argmax_row_widths(cols):
    """Every column path of the row loop: whole 8192-vector passes, the guarded last pass,
    unaligned rows (odd widths) and the scalar tail; the maximum placed in each region."""
    from sid.kernels.ops import argmax_rows
    torch.manual_seed(cols)
    x = torch.randn(6, cols, device="cuda")
    for r, c in enumerate((0, cols // 3, cols - 5, cols - 1, min(cols - 1, 4 * 8192), 2)):
        x[r, c] = 100.0
    got = argmax_rows(x)
    assert got.tolist() == torch.argmax(x.cpu(), dim=-1).tolist()
