"""Overlapped decode (EngineConfig.overlap_decode): step N+1 is launched before step N's
tokens are read back, taking them on the device. In batch_invariant mode the tokens must
equal the synchronous engine's bit for bit, including requests that stop on a stop token
mid-stream (their row of the step already in flight is discarded), under a decode batch
limit that forces admissions (which drain the pipeline), with greedy and seeded sampling;
every KV slot must come back. nondet mode: same lengths and slot accounting."""

from __future__ import annotations

import pytest
import torch

from sid.config import EngineConfig, Mode, SamplingParams
from sid.engine.engine import Engine

pytestmark = pytest.mark.gpu


def _engine(mode, overlap, max_batch=6):
    cfg = EngineConfig(mode=mode, kv_pool_tokens=32768, max_reqs=32, max_seq_len=2048,
                       max_decode_batch=max_batch, num_layers=4, seed=7,
                       overlap_decode=overlap)
    return Engine(cfg)


def _prompts(n, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 151936, (int(torch.randint(8, 90, (1,), generator=g)),),
                          generator=g).tolist() for _ in range(n)]


def _params(n, temperature, stops=None, ignore_eos=True):
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(5, 40, (n,), generator=g).tolist()
    return [SamplingParams(max_new_tokens=lens[i], temperature=temperature, seed=100 + i,
                           ignore_eos=ignore_eos,
                           stop_token_ids=[] if stops is None else [stops[i]])
            for i in range(n)]


def _run(mode, overlap, prompts, params, max_batch=6):
    eng = _engine(mode, overlap, max_batch)
    free0 = eng.kv.free_count
    outs = eng.generate(prompts, params)
    assert eng._inflight is None
    assert eng.kv.free_count == free0, "KV slots leaked"
    return [o.token_ids for o in outs], [o.finish_reason for o in outs]


@pytest.mark.parametrize("temperature", [0.0, 0.7])
def test_overlap_matches_synchronous_batch_invariant(temperature):
    prompts = _prompts(14, 11)
    print(f"overlap batch_invariant T={temperature}", flush=True)
    base, _ = _run(Mode.BATCH_INVARIANT, False, prompts, _params(14, temperature))
    # stop tokens that occur mid-stream: each request's 4th token (or none for short ones)
    stops = [t[3] if len(t) > 6 else 151935 for t in base]
    params = _params(14, temperature, stops, ignore_eos=False)
    a, ra = _run(Mode.BATCH_INVARIANT, False, prompts, params)
    b, rb = _run(Mode.BATCH_INVARIANT, True, prompts, params)
    assert a == b and ra == rb
    assert "stop" in ra and "length" in ra  # both finish kinds exercised
    c, _ = _run(Mode.BATCH_INVARIANT, True, prompts, _params(14, temperature))
    assert c == base


def test_overlap_nondet_lengths_and_slots():
    prompts = _prompts(10, 12)
    print("overlap nondet", flush=True)
    params = _params(10, 0.7)
    toks, reasons = _run(Mode.NONDET, True, prompts, params, max_batch=4)
    assert [len(t) for t in toks] == [p.max_new_tokens for p in params]
    assert set(reasons) == {"length"}


def test_overlap_dvr_deterministic_tokens_unchanged():
    """dvr: verify passes run beside the overlapped decode; rollbacks arrive while the next
    step is in flight (its rows for rolled-back requests are discarded). The deterministic
    requests' tokens equal the synchronous engine's; every slot comes back."""
    prompts = _prompts(16, 13)
    print("overlap dvr", flush=True)
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(20, 90, (16,), generator=g).tolist()
    params = [SamplingParams(max_new_tokens=lens[i], temperature=0.7 if i % 3 else 0.0,
                             seed=7 + i, is_deterministic=i % 2 == 0, ignore_eos=True)
              for i in range(16)]

    def run(overlap):
        eng = _engine(Mode.DVR, overlap, max_batch=8)
        free0 = eng.kv.free_count
        outs = eng.generate(prompts, params)
        assert eng._inflight is None
        assert eng.kv.free_count == free0, "KV slots leaked"
        return outs

    a, b = run(False), run(True)
    for i, (x, y) in enumerate(zip(a, b)):
        assert len(y.token_ids) == params[i].max_new_tokens
        if params[i].is_deterministic:
            assert x.token_ids == y.token_ids, f"request {i}"
    assert sum(o.num_rollbacks for o in b) > 0  # the rollback path ran


def test_overlap_manual_step_loop_returns_every_slot():
    """Driving step() by hand until Engine.has_work() is False applies the last launched
    step too (its rows may belong only to requests that already stopped on EOS)."""
    prompts = _prompts(8, 14)
    print("overlap manual step loop", flush=True)
    base, _ = _run(Mode.BATCH_INVARIANT, False, prompts, _params(8, 0.0))
    stops = [t[2] if len(t) > 4 else 151935 for t in base]
    params = _params(8, 0.0, stops, ignore_eos=False)
    want, _ = _run(Mode.BATCH_INVARIANT, False, prompts, params)
    eng = _engine(Mode.BATCH_INVARIANT, True)
    free0 = eng.kv.free_count
    rids = [eng.add_request(prompt_ids=p, params=sp) for p, sp in zip(prompts, params)]
    while eng.has_work():
        eng.step()
    got = [eng.get_output(r).token_ids for r in rids]
    assert got == want
    assert eng.kv.free_count == free0


def test_overlap_dvr_stop_tokens_and_rollbacks():
    """dvr with stop tokens: a deterministic request may stop on a fast-path token while the
    next step is in flight and be rolled back later (its finish cleared, decoding resumed,
    the in-flight row discarded under the bumped epoch). Deterministic requests' tokens and
    finish reasons equal the synchronous engine's, and every KV page comes back."""
    prompts = _prompts(16, 15)
    print("overlap dvr with stop tokens", flush=True)
    g = torch.Generator().manual_seed(6)
    lens = torch.randint(30, 90, (16,), generator=g).tolist()

    def params(stops):
        return [SamplingParams(max_new_tokens=lens[i], temperature=0.7 if i % 3 else 0.0,
                               seed=11 + i, is_deterministic=i % 2 == 0,
                               ignore_eos=stops is None,
                               stop_token_ids=None if stops is None else [stops[i]])
                for i in range(16)]

    def run(overlap, ps):
        eng = _engine(Mode.DVR, overlap, max_batch=8)
        free0 = eng.kv.free_count
        outs = eng.generate(prompts, ps)
        assert eng._inflight is None
        assert eng.kv.free_count == free0, "KV pages leaked"
        return outs

    base = run(False, params(None))
    # a deterministic request's 6th committed token stops it (when it is not earlier too)
    stops = [151935] * 16
    for i in range(0, 16, 2):
        t = base[i].token_ids
        if len(t) > 8 and t[5] not in t[:5]:
            stops[i] = t[5]
    assert sum(s != 151935 for s in stops) >= 3
    a, b = run(False, params(stops)), run(True, params(stops))
    for i in range(0, 16, 2):
        assert a[i].token_ids == b[i].token_ids, f"request {i}"
        assert a[i].finish_reason == b[i].finish_reason
    assert any(a[i].finish_reason == "stop" for i in range(0, 16, 2))
    assert sum(o.num_rollbacks for o in b) > 0
