"""Prefill grouping (sid/engine/scheduler.py:63-86 of the reference isolates dvr-mode
deterministic requests): one-request groups with dvr_isolated_prefill, shared batches
otherwise, always under max_prefill_tokens. CPU only (no KV pool needed)."""

from __future__ import annotations

from sid.config import EngineConfig, Mode, SamplingParams
from sid.engine.request import Request
from sid.engine.scheduler import Scheduler


def _reqs(lens, det):
    return [Request(i, list(range(n)), SamplingParams(is_deterministic=d), (0,))
            for i, (n, d) in enumerate(zip(lens, det))]


def _groups(isolated, mode=Mode.DVR, max_tokens=100):
    cfg = EngineConfig(mode=mode, max_prefill_tokens=max_tokens, dvr_isolated_prefill=isolated)
    reqs = _reqs([30, 40, 50, 20, 10], [True, False, True, False, True])
    return [[r.rid for r in g] for g in Scheduler(cfg, kv=None).prefill_groups(reqs)]


def test_isolated_deterministic_prefill():
    # deterministic 0, 2, 4 alone; 1 and 3 share a batch
    assert _groups(True) == [[0], [2], [4], [1, 3]]


def test_shared_prefill_batches_respect_token_budget():
    # 30 + 40 fit, + 50 would exceed 100; 50 + 20 + 10 fit
    assert _groups(False) == [[0, 1], [2, 3, 4]]


def test_isolation_flag_only_applies_in_dvr_mode():
    assert _groups(True, Mode.NONDET) == [[0, 1], [2, 3, 4]]
