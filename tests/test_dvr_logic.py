"""DVR bookkeeping on the CPU: the verify pass the Verifier builds and its commit rule,
against the literal expectations of the reference's tests/test_08_dvr_logic.py:56-304
(window construction, padding rows, KV slot reuse, rollback arithmetic, EOS cleared and
re-finished, u = 1, two sequences in one pass, monotone verified_len), plus this build's
pass bucketing and deferral.

Everything runs on the real host objects: a KVCache with CPU tensors (4-slot pages, so
windows cross page boundaries) and the runner's own verify-buffer layout; no GPU work.
"""

from __future__ import annotations

import types

import numpy as np
import pytest

from sid.config import DUMMY_TOKEN_ID, EngineConfig, Mode, ModelConfig, SamplingParams
from sid.engine.dvr import Verifier
from sid.engine.kv_cache import KVCache
from sid.engine.model_runner import ModelRunner
from sid.engine.request import Request

W = 8
EOS = 9
PAGE = 4


def _stack(group=2, buckets=False, min_verify=1):
    """(kv, verify buffers, verifier). The default is the reference's schedule: every pass
    padded to G = 2 sequences, verify whatever is ready."""
    cfg = EngineConfig(mode=Mode.DVR, dvr_window_size=W, dvr_group_size=group, device="cpu",
                       dvr_verify_buckets=buckets, dvr_min_verify=min_verify,
                       kv_pool_tokens=4096, kv_page_size=PAGE, max_reqs=32, max_seq_len=256)
    kv = KVCache(cfg, ModelConfig(num_layers=1, num_kv_heads=1, head_dim=8), "cpu")
    buffers = ModelRunner._alloc_verify_buffers(cfg, "cpu")
    ver = Verifier(cfg, types.SimpleNamespace(verify_buffers=buffers), kv)
    return kv, buffers, ver


def _running(kv, rid, prompt_len, outputs, verified):
    """A deterministic request that has decoded `outputs` (KV for P + N - 1 positions)."""
    r = Request(rid, [100 + k for k in range(prompt_len)],
                SamplingParams(is_deterministic=True, max_new_tokens=1000), eos_token_ids=(EOS,))
    r.output_ids = list(outputs)
    r.verified_len = verified
    r.req_row = kv.open_row()
    kv.grow(r.req_row, r.kv_len)
    r.check_finished()
    return r


def _verdict(per_seq: dict, group=2):
    """Verifier output rows: sequence i's predictions in rows i*W .. i*W + len - 1."""
    out = np.zeros(group * W, dtype=np.int64)
    for i, toks in per_seq.items():
        out[i * W:i * W + len(toks)] = toks
    import torch
    return torch.from_numpy(out)


def test_full_window_construction():
    kv, buf, ver = _stack()
    p, v = 5, 1
    outs = list(range(50, 59))
    r = _running(kv, 0, p, outs, v)
    assert r.unverified() == W
    fb, meta = ver.build_verify_batch([r])
    assert buf["input_ids"][:W].tolist() == outs[0:8]
    assert buf["positions"][:W].tolist() == list(range(p + v - 1, p + v - 1 + W))
    assert buf["sample_positions"][:W].tolist() == list(range(p + v, p + v + W))
    window = kv.slot_range(r.req_row, p + v - 1, p + v - 1 + W).tolist()
    assert buf["out_slots"][:W].tolist() == window          # decode's slots, overwritten
    assert buf["kv_indptr"].tolist()[:2] == [0, p + v - 1 + W]
    assert buf["kv_indices"][:p + v - 1].tolist() == kv.slot_range(r.req_row, 0, p + v - 1).tolist()
    assert buf["kv_indices"][p + v - 1:p + v - 1 + W].tolist() == window
    assert buf["input_ids"][W:2 * W].tolist() == [DUMMY_TOKEN_ID] * W   # dummy sequence
    assert buf["qo_indptr"].tolist()[:3] == [0, W, 2 * W]
    assert meta.window_lens == [W] and meta.windows == [outs[1:9]]
    assert fb.max_extend_len == W and fb.kv_indices.numel() == p + v - 1 + 2 * W


def test_finished_window_padding():
    kv, buf, ver = _stack()
    p = 5
    outs = [50, 51, 52, 53, 54, EOS]
    r = _running(kv, 1, p, outs, verified=3)
    assert r.finished_reason == "stop" and r.unverified() == 3
    ver.build_verify_batch([r])
    assert buf["input_ids"][:W].tolist() == outs[2:5] + [DUMMY_TOKEN_ID] * (W - 3)
    mine = kv.slot_range(r.req_row, 0, r.kv_len).tolist()
    got = buf["out_slots"][:W].tolist()
    assert got[:3] == kv.slot_range(r.req_row, p + 2, p + 5).tolist()
    assert not set(got[3:]) & set(mine) and len(set(got)) == W
    # padding rows repeat the last real position
    assert buf["positions"][:W].tolist() == [p + 2, p + 3, p + 4] + [p + 4] * (W - 3)


def test_all_match_advances():
    kv, _, ver = _stack()
    outs = list(range(50, 59))
    r = _running(kv, 2, 5, outs, 1)
    held = int(kv.held[r.req_row])
    _, meta = ver.build_verify_batch([r])
    ver.compare_and_rollback(meta, _verdict({0: outs[1:9]}))
    assert r.verified_len == 9 and r.output_ids == outs
    assert r.num_rollbacks == 0 and kv.held[r.req_row] == held


def test_mismatch_middle_rolls_back():
    kv, _, ver = _stack()
    p, v = 5, 1
    outs = list(range(50, 59))
    r = _running(kv, 3, p, outs, v)
    free0 = kv.free_pages
    _, meta = ver.build_verify_batch([r])
    got = outs[1:9]
    got[3] = 777
    ver.compare_and_rollback(meta, _verdict({0: got}))
    assert r.output_ids == outs[:4] + [777]
    assert r.verified_len == 5 and r.num_rollbacks == 1 and r.epoch == 1
    assert r.tokens_rolled_back == len(outs) - (v + 3)
    assert r.kv_len == p + len(r.output_ids) - 1 == 9 and r.finished_reason is None
    # KV positions 9 .. 12 were dropped: 13 -> 9 positions is 4 -> 3 pages of 4
    assert kv.held[r.req_row] == 3 and kv.free_pages == free0 + 1


def test_mismatch_at_zero_still_progresses():
    kv, _, ver = _stack()
    outs = list(range(50, 59))
    r = _running(kv, 4, 5, outs, 1)
    _, meta = ver.build_verify_batch([r])
    ver.compare_and_rollback(meta, _verdict({0: [666] + outs[2:9]}))
    assert r.output_ids == [50, 666] and r.verified_len == 2


def test_mismatch_last_frees_nothing():
    kv, _, ver = _stack()
    outs = list(range(50, 59))
    r = _running(kv, 5, 5, outs, 1)
    free0 = kv.free_pages
    _, meta = ver.build_verify_batch([r])
    got = outs[1:9]
    got[-1] = 888
    ver.compare_and_rollback(meta, _verdict({0: got}))
    assert r.output_ids == outs[:8] + [888] and r.verified_len == 9
    assert kv.free_pages == free0


def test_eos_cleared_then_refinished():
    kv, _, ver = _stack()
    outs = [50, 51, 52, 53, 54, EOS]
    r = _running(kv, 6, 5, outs, verified=3)
    _, meta = ver.build_verify_batch([r])
    ver.compare_and_rollback(meta, _verdict({0: [EOS, 54, EOS]}))
    assert r.output_ids == [50, 51, 52, EOS]
    assert r.finished_reason == "stop" and r.verified_len == 4 and r.unverified() == 0


def test_eos_cleared_and_decoding_resumes():
    kv, _, ver = _stack()
    outs = [50, 51, 52, 53, 54, EOS]
    r = _running(kv, 7, 5, outs, verified=3)
    _, meta = ver.build_verify_batch([r])
    ver.compare_and_rollback(meta, _verdict({0: [53, 54, 42]}))
    assert r.output_ids[-1] == 42 and r.finished_reason is None
    assert r.verified_len == len(r.output_ids)


def test_u_equals_one():
    kv, buf, ver = _stack()
    r = _running(kv, 8, 5, [50, EOS], verified=1)
    assert r.unverified() == 1
    _, meta = ver.build_verify_batch([r])
    assert buf["input_ids"][:W].tolist() == [50] + [DUMMY_TOKEN_ID] * (W - 1)
    ver.compare_and_rollback(meta, _verdict({0: [EOS]}))
    assert r.verified_len == 2 and r.output_ids == [50, EOS]


def test_two_requests_grouped():
    kv, _, ver = _stack()
    r1 = _running(kv, 10, 4, list(range(50, 59)), 1)
    r2 = _running(kv, 11, 7, list(range(70, 79)), 1)
    _, meta = ver.build_verify_batch([r1, r2])
    bad = list(range(71, 79))
    bad[2] = 999
    ver.compare_and_rollback(meta, _verdict({0: list(range(51, 59)), 1: bad}))
    assert r1.verified_len == 9 and r1.num_rollbacks == 0
    assert r2.output_ids == [70, 71, 72, 999] and r2.verified_len == 4


def test_verified_len_monotone():
    kv, _, ver = _stack()
    r = _running(kv, 12, 5, list(range(50, 59)), 1)
    history = [r.verified_len]
    for trial in range(3):
        if r.unverified() < 1:
            break
        _, meta = ver.build_verify_batch([r])
        u = meta.window_lens[0]
        got = list(meta.windows[0])
        if trial == 0 and u > 2:
            got[2] = 300
        ver.compare_and_rollback(meta, _verdict({0: got[:u]}))
        history.append(r.verified_len)
        while r.unverified() < W and r.num_output < 20:   # decode more
            r.output_ids.append(60 + r.num_output)
            kv.grow(r.req_row, r.kv_len)
    assert history == sorted(history) and len(history) == 4


def test_collect_ready_groups_by_rid():
    kv, _, ver = _stack()
    reqs = [_running(kv, rid, 3, list(range(50, 50 + n)), 1)
            for rid, n in ((5, 9), (2, 9), (7, 3), (1, 9))]
    # rid 7 has 2 unverified tokens and is still decoding: not ready; the rest by rid, G = 2
    assert [[r.rid for r in g] for g in ver.collect_ready(reqs)] == [[1, 2], [5]]


def test_bucketed_verify_shapes():
    """With dvr_verify_buckets a pass holds the next power of two >= its ready sequences
    (at most G): no dummy sequence for one request, one for three with G = 4."""
    kv, _, ver = _stack(group=4, buckets=True)
    p, v = 5, 1
    r = _running(kv, 0, p, list(range(50, 59)), v)
    fb, _ = ver.build_verify_batch([r])
    assert fb.input_ids.numel() == W and fb.qo_indptr.tolist() == [0, W]
    assert fb.kv_indptr.tolist() == [0, p + v - 1 + W]
    assert fb.kv_indices.numel() == p + v - 1 + W and fb.sample_indices.numel() == W
    reqs = [_running(kv, 1 + i, p, list(range(50, 59)), v) for i in range(3)]
    fb, meta = ver.build_verify_batch(reqs)
    assert fb.input_ids.numel() == 4 * W
    assert fb.qo_indptr.tolist() == [0, W, 2 * W, 3 * W, 4 * W]
    assert fb.input_ids[3 * W:].tolist() == [DUMMY_TOKEN_ID] * W
    assert fb.kv_indices.numel() == 3 * (p + v - 1 + W) + W
    assert meta.window_lens == [W] * 3


def test_collect_ready_waits_for_a_full_pass():
    """With dvr_min_verify = 3, two ready windows wait; a finished request or a 2 W backlog
    is verified at once, together with every other ready request."""
    kv, _, ver = _stack(group=4, min_verify=3)
    a = _running(kv, 1, 3, list(range(50, 59)), 1)               # W unverified
    b = _running(kv, 2, 3, list(range(50, 59)), 1)
    assert ver.collect_ready([a, b]) == []
    c = _running(kv, 3, 3, list(range(50, 50 + 2 * W + 1)), 1)  # 2 W unverified
    assert [[r.rid for r in g] for g in ver.collect_ready([a, b, c])] == [[1, 2, 3]]
    d = _running(kv, 4, 3, [50, 51, EOS], 1)                      # finished, 2 unverified
    assert [[r.rid for r in g] for g in ver.collect_ready([a, d])] == [[1, 4]]
    e = _running(kv, 5, 3, list(range(50, 59)), 1)
    assert [[r.rid for r in g] for g in ver.collect_ready([a, b, e])] == [[1, 2, 5]]


@pytest.mark.parametrize("page", [1, 4, 16])
def test_page_allocator_round_trip(page):
    """Pages: growth takes whole pages, shrinking returns only emptied ones, closing a row
    returns all of them; the debug owner check accepts every step."""
    import os
    os.environ["SID_DEBUG_ALLOC"] = "1"
    try:
        cfg = EngineConfig(kv_pool_tokens=64 * page, kv_page_size=page, max_reqs=4,
                           max_seq_len=48 * page, device="cpu")
        kv = KVCache(cfg, ModelConfig(num_layers=1, num_kv_heads=1, head_dim=8), "cpu")
    finally:
        del os.environ["SID_DEBUG_ALLOC"]
    kv.scatter_free_pages(0)
    total = kv.free_pages
    a, b = kv.open_row(), kv.open_row()
    kv.grow(a, 5 * page + 1)
    kv.grow(b, 3)
    assert kv.held[a] == 6 and kv.held[b] == kv.pages_for(3)
    sa = kv.slot_range(a, 0, 5 * page + 1)
    sb = kv.slot_range(b, 0, 3)
    assert len(set(sa.tolist()) | set(sb.tolist())) == sa.size + sb.size  # no slot shared
    assert ((sa // page)[::page] == kv.tables[a, :6]).all()
    kv.shrink(a, 5 * page)          # the last page held only position 5 * page
    assert kv.held[a] == 5
    kv.shrink(a, 5 * page - 1)      # page 4 keeps position 5 * page - 1 (for page > 1)
    assert kv.held[a] == kv.pages_for(5 * page - 1) == (5 if page > 1 else 4)
    kv.grow(a, 5 * page)
    slots = kv.decode_slots(np.array([a, b]), np.array([5 * page, 3]))
    assert slots[0] // page == kv.tables[a, 5] and kv.held[a] == 6
    kv.close_row(a)
    kv.close_row(b)
    assert kv.free_pages == total
    with pytest.raises(AssertionError):
        kv._give_back(np.array([kv._stack[0]], dtype=np.int32), 1)   # not owned by row 1
