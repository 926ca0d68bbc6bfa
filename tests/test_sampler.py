"""Sampler oracle (CPU): the known answers of the reference's tests/test_07_sampler.py:25-80
on sample_ref (the reference's float-cumsum rule) and on sample_exact_ref (the exact rule the
HIP sampler implements); the int64 hash against a big-int scalar restatement; the exact rule
against brute-force enumeration; and that the product sampler refuses CPU tensors (it is a
HIP kernel, there is no CPU path)."""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle.sampler import (kept_mask_exact, sample_exact_ref, sample_ref, seeded_gumbel_ref,
                            seeded_uniform_ref)

REFS = (sample_ref, sample_exact_ref)


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
    for i in range(5):
        for c in cols:
            u = seeded_uniform_ref(int(seeds[i]), int(pos[i]), c)
            assert 0.0 <= u < 1.0
            want = -torch.log(-torch.log(torch.tensor(u, dtype=torch.float32) + 1e-10) + 1e-10)
            assert torch.equal(g[i, c], want), (i, c)


@pytest.mark.parametrize("fn", REFS)
def test_greedy_first_index_tie(fn):
    logits = torch.zeros(2, 100)
    logits[0, 7] = 5.0
    logits[1, 3] = 2.0
    logits[1, 42] = 2.0
    assert _one(fn, logits, 0.0, 42, [10, 11]).tolist() == [7, 3]


def test_seeded_draw_invariant_to_batch_shape():
    torch.manual_seed(0)
    row = torch.randn(1, 5000)
    alone = _one(sample_exact_ref, row, 0.8, 1234, [17])
    assert alone.item() == _one(sample_ref, row, 0.8, 1234, [17]).item()
    for batch in (2, 7):
        logits = torch.cat([torch.randn(batch - 1, 5000), row])
        toks = _one(sample_exact_ref, logits, 0.8, 1234, list(range(100, 100 + batch - 1)) + [17])
        assert toks[-1].item() == alone.item()


@pytest.mark.parametrize("fn", REFS)
def test_top_k_top_p_respected(fn):
    logits = torch.tensor([[10.0, 9.0, 8.0, -20.0, -20.0]])
    for pos in range(100):
        assert _one(fn, logits, 2.0, 5, [pos], top_k=3).item() in (0, 1, 2)
    peaked = torch.tensor([[10.0, 0.0, 0.0, 0.0, 0.0]])
    for pos in range(50):
        assert _one(fn, peaked, 1.0, 5, [pos], top_p=0.5).item() == 0


def test_exact_rule_equals_reference_rule_without_ambiguity():
    """Random distinct logits (no ties, cut far from rounding): both rules, same tokens."""
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(12, 3000, generator=g) * 3
    temps = torch.tensor([0.0, 0.7, 1.0, 1.3] * 3)
    ks = torch.tensor([-1, 20, -1, 5, 100, -1, 1, 50, -1, -1, 7, 2000], dtype=torch.int64)
    ps = torch.tensor([1.0, 0.9, 0.5, 1.0, 0.95, 0.3, 1.0, 0.8, 0.99, 0.6, 1.0, 0.7])
    seeds = torch.arange(12, dtype=torch.int64) * 7 + 1
    pos = torch.arange(12, dtype=torch.int64) + 40
    assert torch.equal(sample_exact_ref(logits, temps, ks, ps, seeds, pos),
                       sample_ref(logits, temps, ks, ps, seeds, pos))


def test_exact_mask_brute_force_tiny_vocab():
    """kept_mask_exact vs enumerating ranks by hand on tiny vocabularies with ties."""
    rng = np.random.default_rng(4)
    for _ in range(300):
        v = int(rng.integers(1, 7))
        p = rng.choice([0.5, 0.25, 0.125, 0.0625, 0.03125, 0.0], size=v).astype(np.float32)
        k = int(rng.integers(-1, v + 2))
        tp = float(rng.choice([0.0, 0.1, 0.25, 0.5, 0.75, 0.875, 1.0]))
        ranks = sorted(range(v), key=lambda i: (-float(p[i]), i))
        want = np.zeros(v, dtype=bool)
        mass = 0
        for rk, i in enumerate(ranks):
            keep = rk == 0 or ((k <= 0 or rk < k) and (tp >= 1.0 or mass <= math.floor(tp * 2 ** 48)))
            want[i] = keep
            mass += math.floor(float(p[i]) * 2 ** 48)
        assert np.array_equal(kept_mask_exact(p, k, tp), want), (p, k, tp)


def test_product_sampler_refuses_cpu_tensors():
    from sid.engine.sampler import sample
    with pytest.raises(RuntimeError, match="GPU"):
        _one(sample, torch.zeros(1, 10), 0.7, 1, [0])
