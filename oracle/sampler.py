"""Sampler oracle (CPU).

seeded_uniform_ref  restates the integer hash of sid/engine/sampler.py:22-29 with Python
                    big integers, explicit 64-bit two's-complement wraparound and floor
                    modulo 2^24, independently of torch's int64 arithmetic.
sample_ref          restates sid/engine/sampler.py:32-69: greedy argmax (first index on
                    ties); stochastic rows: softmax(l / T), descending sort, top-p drop when
                    the mass before a token exceeds top_p, top-k drop by rank, keep-mask
                    scattered back to vocab order, argmax(log(p + 1e-10) + gumbel).
                    Pinned by the known answers of tests/test_07_sampler.py:25-80
                    (restated in tests/test_sampler.py).
sample_exact_ref    the same draw with the truncation made exact, as the HIP sampler
                    defines it: ranks by (p descending, index ascending) (a stable order,
                    where torch's sort leaves ties unordered) and the mass before a rank
                    summed exactly in units of 2^-48 (each p rounded down) instead of a
                    float cumsum; top_p >= 1 keeps every rank. Pinned against sample_ref
                    on inputs with no tie or rounding ambiguity at the cut, and against
                    brute-force enumeration of the kept set on tiny vocabularies.
"""

from __future__ import annotations

import math

import numpy as np
import torch

EPS = 1e-10
_M64 = (1 << 64) - 1


def _wrap64(x: int) -> int:
    x &= _M64
    return x - (1 << 64) if x >= (1 << 63) else x


def seeded_uniform_ref(seed: int, pos: int, col: int) -> float:
    step = _wrap64(_wrap64(seed * 19349663) ^ _wrap64(pos * 73856093))
    h = _wrap64(_wrap64(step * 8589934591) ^ _wrap64(col * 479001599))
    return (h % (1 << 24)) / float(1 << 24)


def seeded_gumbel_ref(seeds: torch.Tensor, positions: torch.Tensor, num_cols: int) -> torch.Tensor:
    """Vectorised (torch int64 wraps the same way); the scalar form above checks it."""
    step = seeds.long() * 19349663 ^ positions.long() * 73856093
    cols = torch.arange(num_cols, dtype=torch.int64)
    h = step.unsqueeze(-1) * 8589934591 ^ cols * 479001599
    u = (h % (1 << 24)).float() / float(1 << 24)
    return -torch.log(-torch.log(u + EPS) + EPS)


def sample_ref(logits, temperatures, top_ks, top_ps, seeds, positions) -> torch.Tensor:
    logits = logits.float().cpu()
    out = []
    for r in range(logits.shape[0]):
        row = logits[r]
        t = float(temperatures[r])
        if t <= 0:
            out.append(int(torch.argmax(row)))
            continue
        probs = torch.softmax(row / t, dim=-1)
        ps, pi = probs.sort(descending=True)
        cum = torch.cumsum(ps, dim=-1)
        drop = (cum - ps) > float(top_ps[r])
        k = int(top_ks[r])
        if k > 0:
            drop |= torch.arange(row.numel()) >= k
        drop[0] = False
        keep = torch.zeros_like(drop)
        keep[pi] = ~drop
        lp = torch.where(keep, torch.log(probs + EPS), torch.full_like(probs, -math.inf))
        g = seeded_gumbel_ref(torch.tensor([int(seeds[r])]), torch.tensor([int(positions[r])]),
                              row.numel())[0]
        out.append(int(torch.argmax(lp + g)))
    return torch.tensor(out, dtype=torch.int64)


MASS_UNIT = 1 << 48


def kept_mask_exact(p: np.ndarray, top_k: int, top_p: float) -> np.ndarray:
    """Keep-mask of one row under the exact rule (p: float32 probabilities)."""
    v = p.size
    order = np.lexsort((np.arange(v), -p.astype(np.float64)))  # p desc, index asc
    # NaN probabilities (a +inf logit: inf - inf in the softmax) cast to unspecified
    # masses; only the no-limit rule (every column kept) is pinned for such rows.
    with np.errstate(invalid="ignore"):
        q = np.floor(p.astype(np.float64)[order] * MASS_UNIT).astype(np.uint64)
    before = np.concatenate([[0], np.cumsum(q)[:-1]]).astype(np.uint64)
    keep_rank = np.ones(v, dtype=bool)
    if top_k > 0:
        keep_rank &= np.arange(v) < top_k
    if top_p < 1.0:
        lim = np.uint64(math.floor(max(top_p, 0.0) * MASS_UNIT))
        keep_rank &= before <= lim
    keep_rank[0] = True
    keep = np.zeros(v, dtype=bool)
    keep[order] = keep_rank
    return keep


def sample_exact_ref(logits, temperatures, top_ks, top_ps, seeds, positions) -> torch.Tensor:
    logits = logits.float().cpu()
    out = []
    for r in range(logits.shape[0]):
        row = logits[r]
        t = float(temperatures[r])
        if t <= 0:
            out.append(int(torch.argmax(row)))
            continue
        probs = torch.softmax(row / t, dim=-1)
        keep = torch.from_numpy(kept_mask_exact(probs.numpy(), int(top_ks[r]), float(top_ps[r])))
        lp = torch.where(keep, torch.log(probs + EPS), torch.full_like(probs, -math.inf))
        g = seeded_gumbel_ref(torch.tensor([int(seeds[r])]), torch.tensor([int(positions[r])]),
                              row.numel())[0]
        out.append(int(torch.argmax(lp + g)))
    return torch.tensor(out, dtype=torch.int64)
