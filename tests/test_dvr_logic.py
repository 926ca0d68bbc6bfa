"""DVR bookkeeping on the CPU with fake KV / runner: the literal expectations of the
reference's tests/test_08_dvr_logic.py:56-304 (window construction, padding, slot reuse,
rollback arithmetic, EOS clear / re-finish, u = 1, grouped offsets, monotone verified_len),
run against this build's Verifier."""

from __future__ import annotations

import torch

from sid.config import DUMMY_TOKEN_ID, EngineConfig, Mode, SamplingParams
from sid.engine.dvr import Verifier
from sid.engine.request import Request

W, G = 8, 2
EOS = 9


class FakeKV:
    def __init__(self, rows=32, width=256):
        self.req_to_token = torch.zeros(rows, width, dtype=torch.int32)
        self.device = "cpu"
        self._next = 1
        self.freed: list = []

    def alloc(self, n):
        out = torch.arange(self._next, self._next + n, dtype=torch.int64)
        self._next += n
        return out

    def free(self, slots):
        self.freed.extend(slots.tolist())


class FakeRunner:
    def __init__(self, cfg):
        gw, g = cfg.dvr_group_size * cfg.dvr_window_size, cfg.dvr_group_size
        z = torch.zeros
        self.verify_buffers = {
            "input_ids": z(gw, dtype=torch.int64), "positions": z(gw, dtype=torch.int64),
            "out_slots": z(gw, dtype=torch.int64), "sample_positions": z(gw, dtype=torch.int64),
            "temperatures": z(gw), "top_ks": z(gw, dtype=torch.int64), "top_ps": z(gw),
            "seeds": z(gw, dtype=torch.int64), "qo_indptr": z(g + 1, dtype=torch.int32),
            "kv_indptr": z(g + 1, dtype=torch.int32), "kv_indices": z(g * 256, dtype=torch.int32),
        }


def setup():
    # the reference's fixed verify shape (every pass padded to G sequences)
    cfg = EngineConfig(mode=Mode.DVR, dvr_window_size=W, dvr_group_size=G, device="cpu",
                       dvr_verify_buckets=False, dvr_min_verify=1)
    kv = FakeKV()
    runner = FakeRunner(cfg)
    return cfg, kv, runner, Verifier(cfg, runner, kv)


def make_request(kv, rid, prompt_len, outputs, verified, row):
    req = Request(rid, list(range(100, 100 + prompt_len)),
                  SamplingParams(is_deterministic=True, max_new_tokens=1000), eos_token_ids=(EOS,))
    req.output_ids = list(outputs)
    req.verified_len = verified
    req.req_row = row
    kv_len = prompt_len + len(outputs) - 1
    kv.req_to_token[row, :kv_len] = torch.arange(1000, 1000 + kv_len, dtype=torch.int32)
    req.check_finished()
    return req


def tokens_for(rows: dict) -> torch.Tensor:
    t = torch.zeros(G * W, dtype=torch.int64)
    for g, vals in rows.items():
        t[g * W:g * W + len(vals)] = torch.tensor(vals)
    return t


def test_full_window_construction():
    _, kv, runner, ver = setup()
    p, v = 5, 1
    outs = list(range(50, 59))
    req = make_request(kv, 0, p, outs, v, row=3)
    assert req.unverified() == W
    fb, meta = ver.build_verify_batch([req])
    buf = runner.verify_buffers
    assert buf["input_ids"][:W].tolist() == [outs[0]] + outs[1:8]
    assert buf["positions"][:W].tolist() == list(range(p + v - 1, p + v - 1 + W))
    assert buf["sample_positions"][:W].tolist() == list(range(p + v, p + v + W))
    slots = kv.req_to_token[3, p + v - 1:p + v - 1 + W].tolist()
    assert buf["out_slots"][:W].tolist() == slots
    assert buf["kv_indptr"].tolist()[:2] == [0, p + v - 1 + W]
    assert buf["kv_indices"][:p + v - 1].tolist() == kv.req_to_token[3, :p + v - 1].tolist()
    assert buf["kv_indices"][p + v - 1:p + v - 1 + W].tolist() == slots
    assert buf["input_ids"][W:2 * W].tolist() == [DUMMY_TOKEN_ID] * W
    assert buf["qo_indptr"].tolist() == [0, W, 2 * W]
    assert meta.window_lens == [W] and meta.windows == [outs[1:9]]
    assert fb.max_extend_len == W and fb.kv_indices.numel() == p + v - 1 + 2 * W


def test_finished_window_padding():
    _, kv, runner, ver = setup()
    p = 5
    outs = [50, 51, 52, 53, 54, EOS]
    req = make_request(kv, 1, p, outs, verified=3, row=4)
    assert req.finished_reason == "stop" and req.unverified() == 3
    ver.build_verify_batch([req])
    buf = runner.verify_buffers
    assert buf["input_ids"][:W].tolist() == [outs[2]] + outs[3:5] + [DUMMY_TOKEN_ID] * (W - 3)
    kv_len = p + len(outs) - 1
    real = kv.req_to_token[4, p + 2:p + 2 + 3].tolist()
    got = buf["out_slots"][:W].tolist()
    assert got[:3] == real
    assert all(s not in kv.req_to_token[4, :kv_len].tolist() for s in got[3:])
    # padding rows repeat the last real position
    assert buf["positions"][:W].tolist() == [p + 2, p + 3, p + 4] + [p + 4] * (W - 3)


def test_all_match_advances():
    _, kv, _, ver = setup()
    outs = list(range(50, 59))
    req = make_request(kv, 2, 5, outs, 1, row=5)
    _, meta = ver.build_verify_batch([req])
    ver.compare_and_rollback(meta, tokens_for({0: outs[1:9]}))
    assert req.verified_len == 9 and req.output_ids == outs
    assert req.num_rollbacks == 0 and kv.freed == []


def test_mismatch_middle_rolls_back():
    _, kv, _, ver = setup()
    p, v = 5, 1
    outs = list(range(50, 59))
    req = make_request(kv, 3, p, outs, v, row=6)
    _, meta = ver.build_verify_batch([req])
    got = outs[1:9].copy()
    got[3] = 777
    ver.compare_and_rollback(meta, tokens_for({0: got}))
    assert req.output_ids == outs[:4] + [777]
    assert req.verified_len == 5 and req.num_rollbacks == 1
    assert req.tokens_rolled_back == len(outs) - (v + 3)
    assert kv.freed == kv.req_to_token[6, 9:13].tolist()
    assert req.kv_len == p + len(req.output_ids) - 1 and req.finished_reason is None


def test_mismatch_at_zero_still_progresses():
    _, kv, _, ver = setup()
    outs = list(range(50, 59))
    req = make_request(kv, 4, 5, outs, 1, row=7)
    _, meta = ver.build_verify_batch([req])
    ver.compare_and_rollback(meta, tokens_for({0: [666] + outs[2:9]}))
    assert req.output_ids == outs[:1] + [666] and req.verified_len == 2


def test_mismatch_last_frees_nothing():
    _, kv, _, ver = setup()
    outs = list(range(50, 59))
    req = make_request(kv, 5, 5, outs, 1, row=8)
    _, meta = ver.build_verify_batch([req])
    got = outs[1:9].copy()
    got[-1] = 888
    ver.compare_and_rollback(meta, tokens_for({0: got}))
    assert req.output_ids == outs[:8] + [888] and req.verified_len == 9 and kv.freed == []


def test_eos_cleared_then_refinished():
    _, kv, _, ver = setup()
    outs = [50, 51, 52, 53, 54, EOS]
    req = make_request(kv, 6, 5, outs, verified=3, row=9)
    _, meta = ver.build_verify_batch([req])
    ver.compare_and_rollback(meta, tokens_for({0: [EOS, 54, EOS]}))
    assert req.output_ids == outs[:3] + [EOS]
    assert req.finished_reason == "stop" and req.verified_len == 4 and req.unverified() == 0


def test_eos_cleared_and_decoding_resumes():
    _, kv, _, ver = setup()
    outs = [50, 51, 52, 53, 54, EOS]
    req = make_request(kv, 7, 5, outs, verified=3, row=10)
    _, meta = ver.build_verify_batch([req])
    ver.compare_and_rollback(meta, tokens_for({0: [53, 54, 42]}))
    assert req.output_ids[-1] == 42 and req.finished_reason is None
    assert req.verified_len == len(req.output_ids)


def test_u_equals_one():
    _, kv, runner, ver = setup()
    req = make_request(kv, 8, 5, [50, EOS], verified=1, row=11)
    assert req.unverified() == 1
    _, meta = ver.build_verify_batch([req])
    assert runner.verify_buffers["input_ids"][:W].tolist() == [50] + [DUMMY_TOKEN_ID] * (W - 1)
    ver.compare_and_rollback(meta, tokens_for({0: [EOS]}))
    assert req.verified_len == 2 and req.output_ids == [50, EOS]


def test_two_requests_grouped():
    _, kv, _, ver = setup()
    r1 = make_request(kv, 10, 4, list(range(50, 59)), 1, row=12)
    r2 = make_request(kv, 11, 7, list(range(70, 79)), 1, row=13)
    _, meta = ver.build_verify_batch([r1, r2])
    bad = r2.output_ids[1:9].copy()
    bad[2] = 999
    ver.compare_and_rollback(meta, tokens_for({0: r1.output_ids[1:9], 1: bad}))
    assert r1.verified_len == 9 and r1.num_rollbacks == 0
    assert r2.output_ids == list(range(70, 73)) + [999] and r2.verified_len == 4


def test_verified_len_monotone():
    _, kv, _, ver = setup()
    req = make_request(kv, 12, 5, list(range(50, 59)), 1, row=14)
    hist = [req.verified_len]
    for trial in range(3):
        if req.unverified() < 1:
            break
        _, meta = ver.build_verify_batch([req])
        u = meta.window_lens[0]
        got = meta.windows[0].copy()
        if trial == 0 and u > 2:
            got[2] = 300
        ver.compare_and_rollback(meta, tokens_for({0: got[:u]}))
        hist.append(req.verified_len)
        while req.unverified() < W and len(req.output_ids) < 20:
            req.output_ids.append(60 + len(req.output_ids))
            pos = req.prompt_len + len(req.output_ids) - 2
            kv.req_to_token[14, pos] = 2000 + pos
    assert hist == sorted(hist)


def test_collect_ready_groups_by_rid():
    _, kv, _, ver = setup()
    reqs = [make_request(kv, rid, 3, list(range(50, 50 + n)), 1, row=rid + 1)
            for rid, n in ((5, 9), (2, 9), (7, 3), (1, 9))]
    groups = ver.collect_ready(reqs)
    # rid 7 has 2 unverified and is not finished -> not ready; the rest sorted by rid, G=2
    assert [[r.rid for r in g] for g in groups] == [[1, 2], [5]]


def test_bucketed_verify_shapes():
    """With dvr_verify_buckets a pass holds the next power of two >= its ready sequences
    (at most G): no dummy sequence for one request, one for three with G = 4."""
    cfg = EngineConfig(mode=Mode.DVR, dvr_window_size=W, dvr_group_size=4, device="cpu",
                       dvr_verify_buckets=True)
    kv = FakeKV()
    runner = FakeRunner(cfg)
    ver = Verifier(cfg, runner, kv)
    p, v = 5, 1
    req = make_request(kv, 0, p, list(range(50, 59)), v, row=3)
    fb, _ = ver.build_verify_batch([req])
    assert fb.input_ids.numel() == W and fb.qo_indptr.tolist() == [0, W]
    assert fb.kv_indptr.tolist() == [0, p + v - 1 + W]
    assert fb.kv_indices.numel() == p + v - 1 + W
    assert fb.sample_indices.numel() == W
    reqs = [make_request(kv, i, p, list(range(50, 59)), v, row=4 + i) for i in range(3)]
    fb, meta = ver.build_verify_batch(reqs)
    assert fb.input_ids.numel() == 4 * W and fb.qo_indptr.tolist() == [0, W, 2 * W, 3 * W, 4 * W]
    assert fb.input_ids[3 * W:].tolist() == [DUMMY_TOKEN_ID] * W
    assert fb.kv_indices.numel() == 3 * (p + v - 1 + W) + W
    assert meta.window_lens == [W] * 3


def test_collect_ready_waits_for_a_full_pass():
    """With dvr_min_verify = 3, two ready windows wait; a finished request or a 2 W backlog
    is verified at once, together with every other ready request."""
    cfg = EngineConfig(mode=Mode.DVR, dvr_window_size=W, dvr_group_size=4, device="cpu",
                       dvr_min_verify=3)
    kv = FakeKV()
    ver = Verifier(cfg, FakeRunner(cfg), kv)
    a = make_request(kv, 1, 3, list(range(50, 59)), 1, row=1)    # W unverified
    b = make_request(kv, 2, 3, list(range(50, 59)), 1, row=2)
    assert ver.collect_ready([a, b]) == []
    c = make_request(kv, 3, 3, list(range(50, 50 + 2 * W + 1)), 1, row=3)  # 2 W unverified
    assert [[r.rid for r in g] for g in ver.collect_ready([a, b, c])] == [[1, 2, 3]]
    d = make_request(kv, 4, 3, [50, 51, EOS], 1, row=4)          # finished, 2 unverified
    assert [[r.rid for r in g] for g in ver.collect_ready([a, d])] == [[1, 4]]
    e = make_request(kv, 5, 3, list(range(50, 59)), 1, row=5)
    assert [[r.rid for r in g] for g in ver.collect_ready([a, b, e])] == [[1, 2, 5]]
