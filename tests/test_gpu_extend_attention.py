"""Extend (prefill / verify) attention (HIP, MFMA) vs the fp32 oracle, and the two bitwise
properties DVR rests on: window-offset invariance and batch-slot invariance.
Cases follow the reference's tests/test_03_extend_attention.py:56-152."""

from __future__ import annotations

import pytest
import torch

from conftest import HKV, HQ, D, SCALE, assert_close_bf16
from oracle.attention import extend_attention_ref

pytestmark = pytest.mark.gpu


def _fwd(*a):
    from sid.kernels.extend_attention import extend_attention_fwd
    return extend_attention_fwd(*a)


def _make(specs, seed=0):
    g = torch.Generator().manual_seed(seed)
    total_kv = sum(p + e for p, e in specs)
    total_q = sum(e for _, e in specs)
    slots = total_kv + 16
    q = torch.randn(total_q, HQ, D, generator=g).to(torch.bfloat16)
    kb = torch.randn(slots, HKV, D, generator=g).to(torch.bfloat16)
    vb = torch.randn(slots, HKV, D, generator=g).to(torch.bfloat16)
    idx = (torch.randperm(slots - 1, generator=g)[:total_kv] + 1).to(torch.int32)
    qo = torch.zeros(len(specs) + 1, dtype=torch.int32)
    qo[1:] = torch.cumsum(torch.tensor([e for _, e in specs]), 0)
    kvp = torch.zeros(len(specs) + 1, dtype=torch.int32)
    kvp[1:] = torch.cumsum(torch.tensor([p + e for p, e in specs]), 0)
    return [t.cuda() for t in (q, kb, vb, qo, kvp, idx)]


@pytest.mark.parametrize("specs", [
    [(0, 1)], [(0, 32)], [(0, 64)], [(0, 100)], [(0, 500)],
    [(1, 1)], [(100, 32)], [(1000, 64)],
    [(100, 32), (0, 17), (999, 1), (5, 64)],
    [(31, 32), (32, 32), (33, 32), (256, 32)],
    [(7, 1), (100, 1), (5000, 1)],
    [(2048, 32), (2049, 32), (2070, 32), (0, 32)],
], ids=str)
def test_extend_vs_oracle(specs):
    q, kb, vb, qo, kvp, idx = _make(specs)
    out = _fwd(q, kb, vb, qo, kvp, idx, max(e for _, e in specs), SCALE)
    ref = extend_attention_ref(q, kb, vb, qo, kvp, idx, SCALE)
    assert_close_bf16(out, ref)


def test_window_offset_invariance():
    torch.manual_seed(11)
    L = 300
    q_all = torch.randn(L, HQ, D, device="cuda", dtype=torch.bfloat16)
    kb = torch.randn(L + 32, HKV, D, device="cuda", dtype=torch.bfloat16)
    vb = torch.randn(L + 32, HKV, D, device="cuda", dtype=torch.bfloat16)
    idx = (torch.randperm(L + 31, device="cuda")[:L] + 1).to(torch.int32)

    def run(prefix):
        e = L - prefix
        qo = torch.tensor([0, e], dtype=torch.int32, device="cuda")
        kvp = torch.tensor([0, L], dtype=torch.int32, device="cuda")
        return _fwd(q_all[prefix:].contiguous(), kb, vb, qo, kvp, idx, e, SCALE)

    base = run(268)
    for prefix in (233, 245, 267, 269, 236, 0, 100):
        other = run(prefix)
        common = max(268, prefix)
        n = L - common
        assert torch.equal(base[common - 268:common - 268 + n], other[common - prefix:common - prefix + n]), prefix


def test_position_invariance_within_batch():
    torch.manual_seed(7)
    p, e = 100, 32
    q0 = torch.randn(e, HQ, D, device="cuda", dtype=torch.bfloat16)
    kb = torch.randn(4096, HKV, D, device="cuda", dtype=torch.bfloat16)
    vb = torch.randn(4096, HKV, D, device="cuda", dtype=torch.bfloat16)
    idx0 = (torch.randperm(4095, device="cuda")[:p + e] + 1).to(torch.int32)

    def run(slot, others):
        specs, qs, idxs = [], [], []
        g = torch.Generator(device="cuda").manual_seed(1234)
        for i in range(others + 1):
            if i == slot:
                specs.append((p, e)); qs.append(q0); idxs.append(idx0)
            else:
                pe, ee = 40 + 13 * i, 8 + i
                specs.append((pe, ee))
                qs.append(torch.randn(ee, HQ, D, device="cuda", generator=g).to(torch.bfloat16))
                idxs.append(torch.randint(1, 4096, (pe + ee,), device="cuda", generator=g,
                                          dtype=torch.int32))
        qo = torch.zeros(len(specs) + 1, dtype=torch.int32)
        qo[1:] = torch.cumsum(torch.tensor([s[1] for s in specs]), 0)
        kvp = torch.zeros(len(specs) + 1, dtype=torch.int32)
        kvp[1:] = torch.cumsum(torch.tensor([s[0] + s[1] for s in specs]), 0)
        out = _fwd(torch.cat(qs), kb, vb, qo.cuda(), kvp.cuda(), torch.cat(idxs),
                   max(s[1] for s in specs), SCALE)
        return out[qo[slot]:qo[slot] + e]

    base = run(0, 0)
    for slot, others in [(0, 3), (2, 3), (3, 3), (1, 7)]:
        assert torch.equal(base, run(slot, others)), (slot, others)


def test_decode_shape_matches_decode_kernel_numerically():
    """Extend with one query per request == decode attention (tolerance; different kernels)."""
    from oracle.attention import decode_attention_ref
    specs = [(63, 1), (500, 1), (0, 1)]
    q, kb, vb, qo, kvp, idx = _make(specs, seed=5)
    out = _fwd(q, kb, vb, qo, kvp, idx, 1, SCALE)
    assert_close_bf16(out, decode_attention_ref(q, kb, vb, kvp, idx, SCALE))


@pytest.mark.parametrize("specs", [
    [(2048, 32), (2049, 32), (2070, 32), (0, 32)],   # the verify shape with 2k prefixes
    [(100, 32), (0, 17), (999, 1), (5, 64)],
    [(0, 300)],
], ids=str)
def test_split_fanout_bitwise_equals_sequential_fold(specs):
    """With a workspace the kernel gives every 256-key split its own workgroup and folds the
    split states afterwards; without one a workgroup folds them itself: same bits."""
    from sid.kernels.jit import load_ext
    ext = load_ext()
    q, kb, vb, qo, kvp, idx = _make(specs, seed=9)
    max_e = max(e for _, e in specs)
    max_kv = max(p + e for p, e in specs)
    need = ext.extend_attention_workspace_bytes(len(specs), q.shape[0], HQ, HKV, max_e, max_kv)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    a = torch.empty_like(q)
    b = torch.empty_like(q)
    ext.extend_attention_fwd(q, kb, vb, qo, kvp, idx, max_e, SCALE, a, max_kv, ws)
    ext.extend_attention_fwd(q, kb, vb, qo, kvp, idx, max_e, SCALE, b, max_kv, None)
    assert torch.equal(a, b)
    # a looser bound (more, empty splits in the grid) changes nothing either
    ws2 = torch.empty(ext.extend_attention_workspace_bytes(len(specs), q.shape[0], HQ, HKV, max_e,
                                                           4 * max_kv), dtype=torch.uint8, device="cuda")
    c = torch.empty_like(q)
    ext.extend_attention_fwd(q, kb, vb, qo, kvp, idx, max_e, SCALE, c, 4 * max_kv, ws2)
    assert torch.equal(a, c)
