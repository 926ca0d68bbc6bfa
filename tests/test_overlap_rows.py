"""Host logic of the overlapped decode and of the per-shape split-K rule (no GPU): which
requests the next decode step takes, and from where each takes its newest token."""

from __future__ import annotations

from types import SimpleNamespace

from sid.config import SamplingParams
from sid.engine.engine import Engine, _InFlight
from sid.engine.request import Request
from sid.model.qwen3 import SPLIT_K_MAX_TOKENS, split_k_preferred


def _req(rid, n_out, max_new):
    r = Request(rid, [1, 2, 3], SamplingParams(max_new_tokens=max_new, ignore_eos=True), (0,))
    r.output_ids = list(range(10, 10 + n_out))
    return r


def _next_rows(decode, inflight):
    fake = SimpleNamespace(scheduler=SimpleNamespace(decode_reqs=lambda: decode))
    return Engine._next_rows(fake, inflight)


def test_next_rows_continue_from_the_step_in_flight():
    a, b, c = _req(0, 3, 10), _req(1, 3, 10), _req(2, 9, 10)
    step = _InFlight([a, b, c], [0, 0, 0], None, None, None)
    reqs, rows = _next_rows([a, b, c], step)
    # c's in-flight token is its 10th and last: it does not continue
    assert reqs == [a, b] and rows == [0, 1]


def test_next_rows_after_rollback_and_resume():
    a, b, c = _req(0, 3, 10), _req(1, 3, 10), _req(2, 4, 10)
    step = _InFlight([a, b], [0, 0], None, None, None)
    b.epoch = 1  # rolled back after the launch: its in-flight row is stale
    reqs, rows = _next_rows([a, b, c], step)  # c resumed (not in the step in flight)
    assert reqs == [a, b, c] and rows == [0, -1, -1]


def test_next_rows_skip_stopped_requests():
    a, b = _req(0, 3, 10), _req(1, 3, 10)
    step = _InFlight([a, b], [0, 0], None, None, None)
    # b stopped on EOS at the previous step: the scheduler no longer lists it
    reqs, rows = _next_rows([a], step)
    assert reqs == [a] and rows == [0]
    assert _next_rows([a, b], None) == ([a, b], [-1, -1])


def test_split_k_rule():
    w = SPLIT_K_MAX_TOKENS
    assert split_k_preferred(3 * w, 1024) and not split_k_preferred(3 * w + 1, 1024)
    assert split_k_preferred(5 * w // 8 - 1, 4096) and not split_k_preferred(5 * w // 8, 4096)
    assert split_k_preferred(w - 1, 6144) and not split_k_preferred(w, 6144)
    assert not split_k_preferred(1, 1024, wide_max=0)
