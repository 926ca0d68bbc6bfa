"""Sampler: the known answers of the reference's tests/test_07_sampler.py:25-80, run on the
product sampler (CPU tensors) and on the oracle; the int64 hash against a big-int scalar
restatement."""

from __future__ import annotations

import torch

from oracle.sampler import sample_ref, seeded_gumbel_ref, seeded_uniform_ref
from sid.engine.sampler import _seeded_gumbel, sample


def _one(fn, logits, temp, seed, pos, top_k=-1, top_p=1.0):
    r = logits.shape[0]
    return fn(logits, torch.full((r,), temp), torch.full((r,), top_k, dtype=torch.int64),
              torch.full((r,), top_p), torch.full((r,), seed, dtype=torch.int64),
              torch.as_tensor(pos, dtype=torch.int64))


def test_hash_matches_big_integer_restatement():
    seeds = torch.tensor([0, 42, 1234, 2 ** 40 + 7, -5], dtype=torch.int64)
    pos = torch.tensor([0, 17, 250, 8191, 3], dtype=torch.int64)
    cols = [0, 1, 2, 999, 151935]
    g = seeded_gumbel_ref(seeds, pos, 151936)
    gp = _seeded_gumbel(seeds, pos, 151936)
    assert torch.equal(g, gp)
    for i in range(5):
        for c in cols:
            u = seeded_uniform_ref(int(seeds[i]), int(pos[i]), c)
            assert 0.0 <= u < 1.0
            want = -torch.log(-torch.log(torch.tensor(u, dtype=torch.float32) + 1e-10) + 1e-10)
            assert torch.equal(g[i, c], want), (i, c)


def test_greedy_first_index_tie():
    logits = torch.zeros(2, 100)
    logits[0, 7] = 5.0
    logits[1, 3] = 2.0
    logits[1, 42] = 2.0
    for fn in (sample, sample_ref):
        assert _one(fn, logits, 0.0, 42, [10, 11]).tolist() == [7, 3]


def test_seeded_draw_invariant_to_batch_shape():
    torch.manual_seed(0)
    row = torch.randn(1, 5000)
    alone = _one(sample, row, 0.8, 1234, [17])
    assert alone.item() == sample_ref(row, [0.8], [-1], [1.0], [1234], [17]).item()
    for batch in (2, 7, 33):
        logits = torch.cat([torch.randn(batch - 1, 5000), row])
        toks = _one(sample, logits, 0.8, 1234, list(range(100, 100 + batch - 1)) + [17])
        assert toks[-1].item() == alone.item()


def test_position_changes_draws():
    torch.manual_seed(1)
    logits = torch.randn(1, 1000).repeat(64, 1)
    assert len(set(_one(sample, logits, 1.5, 42, list(range(64))).tolist())) > 1


def test_decode_and_verify_paths_agree():
    torch.manual_seed(2)
    W, seed, base = 32, 777, 250
    logits = torch.randn(W, 4000)
    verify = _one(sample, logits, 0.7, seed, list(range(base, base + W)), top_k=50, top_p=0.9)
    for j in (0, 1, W // 2, W - 1):
        dec = _one(sample, logits[j:j + 1], 0.7, seed, [base + j], top_k=50, top_p=0.9)
        assert dec.item() == verify[j].item()
    ref = sample_ref(logits, [0.7] * W, [50] * W, [0.9] * W, [seed] * W, list(range(base, base + W)))
    assert torch.equal(verify, ref)


def test_top_k_top_p_respected():
    logits = torch.tensor([[10.0, 9.0, 8.0, -20.0, -20.0]])
    for pos in range(200):
        assert _one(sample, logits, 2.0, 5, [pos], top_k=3).item() in (0, 1, 2)
    peaked = torch.tensor([[10.0, 0.0, 0.0, 0.0, 0.0]])
    for pos in range(100):
        assert _one(sample, peaked, 1.0, 5, [pos], top_p=0.5).item() == 0


def test_mixed_rows_greedy_and_stochastic():
    torch.manual_seed(3)
    logits = torch.randn(6, 300)
    temps = torch.tensor([0.0, 0.9, 0.0, 1.3, 0.5, 0.0])
    args = (torch.full((6,), 20, dtype=torch.int64), torch.full((6,), 0.95),
            torch.arange(6, dtype=torch.int64) + 11, torch.arange(6, dtype=torch.int64) * 3)
    out = sample(logits, temps, *args)
    ref = sample_ref(logits, temps, *args)
    assert torch.equal(out, ref)
    assert out[0] == logits[0].argmax() and out[5] == logits[5].argmax()
