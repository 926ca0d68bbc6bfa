"""Attention oracles (fp32, CPU).

ref_attention            restates tests/conftest.py:11-32 (GQA, optional causal offset).
                         Pinned by: a scalar pure-Python brute force on tiny inputs; the
                         uniform-logit special case (output = mean of V); the one-key case
                         (output = that V row); permutation invariance of the keys.
decode_attention_ref     restates tests/test_02_flash_decode.py:50-58 (gather by kv_indices,
                         full visibility). Pinned by ref_attention + gather brute force.
kv_per_split / plan_*    restate sid/csrc/flash_decode.cu:56-60 and
                         sid/kernels/decode_attention.py:65-76. Pinned by hand-computed
                         values (tests) and the covering property (splits tile [0, len)).
split_merge_ref          restates the stage1/stage2 math of sid/csrc/flash_decode.cu:216-229
                         and :252-272 (per-split normalised partial + lse, max-shifted
                         merge over valid splits). Pinned by the identity: merge of splits
                         == full softmax attention, for every split count.
extend_attention_ref     restates tests/test_03_extend_attention.py:44-53 (query j sees keys
                         <= prefix + j). Pinned by ref_attention with causal_offset and by
                         the prefix-0 case equalling causal self-attention.
"""

from __future__ import annotations

import math

import torch


def ref_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float,
                  causal_offset: int | None = None) -> torch.Tensor:
    """q [Tq, HQ, D], k/v [Tk, HKV, D] -> fp32 [Tq, HQ, D]; q head h uses kv head h // (HQ/HKV).
    causal_offset c: query i sees keys j <= c + i; None: every key."""
    tq, hq, d = q.shape
    tk, hkv, _ = k.shape
    group = hq // hkv
    qf, kf, vf = q.float(), k.float(), v.float()
    out = torch.zeros(tq, hq, d, dtype=torch.float32)
    if tk == 0:
        return out
    for h in range(hq):
        kh = h // group
        scores = (qf[:, h] @ kf[:, kh].t()) * sm_scale
        if causal_offset is not None:
            qi = torch.arange(tq).unsqueeze(1)
            kj = torch.arange(tk).unsqueeze(0)
            scores = scores.masked_fill(kj > causal_offset + qi, float("-inf"))
        out[:, h] = torch.softmax(scores, dim=-1) @ vf[:, kh]
    return out


def brute_attention(q, k, v, sm_scale, causal_offset=None):
    """Scalar pure-Python attention (tiny inputs only): the check on ref_attention."""
    tq, hq, d = q.shape
    tk, hkv, _ = k.shape
    group = hq // hkv
    ql, kl, vl = q.double().tolist(), k.double().tolist(), v.double().tolist()
    out = [[[0.0] * d for _ in range(hq)] for _ in range(tq)]
    for i in range(tq):
        for h in range(hq):
            kh = h // group
            keys = [j for j in range(tk) if causal_offset is None or j <= causal_offset + i]
            logits = [sum(ql[i][h][e] * kl[j][kh][e] for e in range(d)) * sm_scale for j in keys]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            z = sum(w)
            for e in range(d):
                out[i][h][e] = sum(w[n] * vl[keys[n]][kh][e] for n in range(len(keys))) / z
    return torch.tensor(out, dtype=torch.float32)


def decode_attention_ref(q, k_cache, v_cache, kv_indptr, kv_indices, sm_scale):
    """q [B, HQ, D]; every request attends to all of its kv_indices rows. fp32 [B, HQ, D]."""
    kv_indptr = kv_indptr.cpu().long()
    kv_indices = kv_indices.cpu().long()
    q, k_cache, v_cache = q.cpu(), k_cache.cpu(), v_cache.cpu()
    outs = []
    for b in range(q.shape[0]):
        idx = kv_indices[kv_indptr[b]:kv_indptr[b + 1]]
        outs.append(ref_attention(q[b:b + 1], k_cache[idx], v_cache[idx], sm_scale))
    return torch.cat(outs) if outs else torch.zeros(0, *q.shape[1:])


def kv_per_split(seq_len: int, n_splits: int, fixed_split_size: int) -> int:
    """Tokens per split: fixed size, or ceil(ceil(len / n) / 32) * 32 (flash_decode.cu:56-60)."""
    if fixed_split_size > 0:
        return fixed_split_size
    return -(-(-(-seq_len // n_splits)) // 32) * 32


def plan_heuristic(seq_lens: list[int], cu_count: int, num_kv_heads: int,
                   max_kv_splits: int) -> tuple[list[int], int]:
    """(per-request num_splits, grid splits) of the nondet/dvr policy (decode_attention.py:72-76)."""
    bs = len(seq_lens)
    splits = -(-2 * cu_count // (bs * num_kv_heads))
    splits = max(1, min(splits, max_kv_splits))
    return [min(-(-s // 32), splits) for s in seq_lens], splits


def plan_fixed(seq_lens: list[int], tile: int = 256) -> tuple[list[int], int]:
    """(per-request num_splits, grid splits) of the batch_invariant policy (:66-70)."""
    return [-(-s // tile) for s in seq_lens], -(-max(seq_lens) // tile)


def split_ranges(seq_len: int, n_splits: int, fixed_split_size: int) -> list[tuple[int, int]]:
    """Non-empty [start, end) token ranges of the splits a request actually uses."""
    if n_splits <= 0 or seq_len <= 0:
        return []
    chunk = kv_per_split(seq_len, n_splits, fixed_split_size)
    out = []
    for s in range(n_splits):
        start = s * chunk
        if start >= seq_len:
            break
        out.append((start, min(start + chunk, seq_len)))
    return out


def split_merge_ref(q, k, v, sm_scale, ranges):
    """Stage-1 partials over each range, then the stage-2 lse merge (fp64 for the check).
    q [HQ, D], k/v [L, HKV, D] -> [HQ, D] float64."""
    hq, d = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    qd, kd, vd = q.double(), k.double(), v.double()
    out = torch.zeros(hq, d, dtype=torch.float64)
    for h in range(hq):
        kh = h // group
        parts, lses = [], []
        for (a, b) in ranges:
            logits = (kd[a:b, kh] @ qd[h]) * sm_scale
            m = logits.max()
            p = torch.exp(logits - m)
            parts.append((p @ vd[a:b, kh]) / p.sum())
            lses.append(m + torch.log(p.sum()))
        if not parts:
            continue
        lse = torch.stack(lses)
        w = torch.exp(lse - lse.max())
        out[h] = (w[:, None] * torch.stack(parts)).sum(0) / w.sum()
    return out


def extend_attention_ref(q, k_buf, v_buf, qo_indptr, kv_indptr, kv_indices, sm_scale):
    """q [Text, HQ, D]: per request, query j sees keys <= prefix + j. fp32 [Text, HQ, D]."""
    qo = qo_indptr.cpu().long().tolist()
    kvp = kv_indptr.cpu().long().tolist()
    idx_all = kv_indices.cpu().long()
    q, k_buf, v_buf = q.cpu(), k_buf.cpu(), v_buf.cpu()
    outs = []
    for i in range(len(qo) - 1):
        qi = q[qo[i]:qo[i + 1]]
        idx = idx_all[kvp[i]:kvp[i + 1]]
        prefix = (kvp[i + 1] - kvp[i]) - (qo[i + 1] - qo[i])
        outs.append(ref_attention(qi, k_buf[idx], v_buf[idx], sm_scale, causal_offset=prefix))
    return torch.cat(outs) if outs else torch.zeros(0, *q.shape[1:])
