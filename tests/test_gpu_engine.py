"""End-to-end determinism on a random-init Qwen3-0.6B-shape model (4 layers to keep the
test short): the watched request's tokens are SHA-256-identical whether its decode batch
is 1, 4, 8 or 16 wide with random co-tenants, in dvr mode (greedy and T=0.7 seeded
sampling) and in batch_invariant mode. Mirrors the reference's tests/test_09_dvr_e2e.py
and tests/test_10_batch_invariant.py:41-74, with token-id prompts (no tokenizer offline)."""

from __future__ import annotations

import hashlib

import pytest
import torch

from sid.config import EngineConfig, Mode, SamplingParams
from sid.engine.engine import Engine

pytestmark = pytest.mark.gpu

WIDTHS = (1, 4, 8, 16)


def _prompts(n, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 151936, (int(torch.randint(8, 120, (1,), generator=g)),),
                          generator=g).tolist() for _ in range(n)]


def _engine(mode):
    cfg = EngineConfig(mode=mode, kv_pool_tokens=32768, max_reqs=64, max_seq_len=2048,
                       max_decode_batch=64, num_layers=4, seed=7)
    return Engine(cfg)


def _hashes(engine, temperature, max_new=80):
    watched = _prompts(1, 100)[0]
    fillers = _prompts(16, 200)
    out = {}
    for width in WIDTHS:
        comp = [watched] + fillers[:width - 1]
        # the watched request sits at a different batch slot each time
        pos = {1: 0, 4: 2, 8: 5, 16: 11}[width]
        comp[0], comp[pos] = comp[pos], comp[0]
        params = [SamplingParams(max_new_tokens=max_new, temperature=temperature,
                                 top_p=0.95 if temperature > 0 else 1.0, seed=1234,
                                 is_deterministic=True, ignore_eos=True) for _ in comp]
        res = engine.generate(comp, params)
        w = res[pos]
        assert len(w.token_ids) == max_new
        out[width] = (hashlib.sha256(str(w.token_ids).encode()).hexdigest(), w)
    return out


@pytest.mark.parametrize("temperature", [0.0, 0.7])
def test_dvr_identical_across_batch_widths(temperature):
    eng = _engine(Mode.DVR)
    out = _hashes(eng, temperature)
    hashes = {h for h, _ in out.values()}
    assert len(hashes) == 1, {k: v[1].token_ids[:16] for k, v in out.items()}
    assert all(w.num_windows > 0 for _, w in out.values())


def test_batch_invariant_identical_across_batch_widths():
    out = _hashes(_engine(Mode.BATCH_INVARIANT), 0.0)
    assert len({h for h, _ in out.values()}) == 1


def test_batch_invariant_row_path_ignores_co_tenants_limits():
    """batch_invariant, T = 0.7: a request without top-k / top-p limits draws every token
    with the lm_head-fused sampler (the engine's choice at max_decode_batch <= 256) whether
    its co-tenants have limits or not; the rows with limits use the sampler kernel. The two
    paths can disagree at float near-ties, so the path must follow from the row alone. Its
    first token (the prefill batch's) likewise: the lm_head-fused sampler with 128-column
    tiles, with the logits also written when co-tenants have limits."""
    from sid.engine.model_runner import ModelRunner
    eng = _engine(Mode.BATCH_INVARIANT)
    calls = []
    prefill_calls = []
    orig = ModelRunner.forward

    def spy(self, fb, greedy=False, sample=False, with_logits=False):
        if fb.mode.name == "DECODE":
            calls.append((sample, with_logits))
        elif fb.mode.name == "PREFILL":
            prefill_calls.append((sample, with_logits, fb.sample_tiles))
        return orig(self, fb, greedy, sample, with_logits)

    watched = _prompts(1, 101)[0]
    fillers = _prompts(5, 201)
    free = SamplingParams(max_new_tokens=40, temperature=0.7, seed=99, ignore_eos=True)
    tokens = {}
    ModelRunner.forward = spy
    try:
        for limits in ("none", "top_k", "top_p"):
            params = [free] + [SamplingParams(
                max_new_tokens=40, temperature=0.7, seed=5 + i, ignore_eos=True,
                top_k=20 if limits == "top_k" else -1,
                top_p=0.9 if limits == "top_p" else 1.0) for i in range(len(fillers))]
            calls.clear()
            prefill_calls.clear()
            tokens[limits] = eng.generate([watched] + fillers, params)[0].token_ids
            decode_calls = set(calls)
            if limits == "none":
                assert decode_calls == {(True, False)}, decode_calls
                assert set(prefill_calls) == {(True, False, True)}, prefill_calls
            else:
                assert decode_calls == {(True, True)}, decode_calls
                assert set(prefill_calls) == {(True, True, True)}, prefill_calls
    finally:
        ModelRunner.forward = orig
    assert tokens["none"] == tokens["top_k"] == tokens["top_p"]


def test_engine_step_api_and_release():
    eng = _engine(Mode.DVR)
    free0 = eng.kv.free_count
    rid = eng.add_request(prompt_ids=_prompts(1, 5)[0],
                          params=SamplingParams(max_new_tokens=40, is_deterministic=True,
                                                ignore_eos=True))
    while eng.has_work():
        eng.step()
    out = eng.get_output(rid)
    assert out is not None and len(out.token_ids) == 40 and out.finish_reason == "length"
    assert eng.get_output(rid) is None
    assert eng.kv.free_count == free0  # every slot returned
    with pytest.raises(ValueError):
        eng.add_request(prompt_ids=[1] * 10, params=SamplingParams(max_new_tokens=10 ** 6))


def test_dvr_schedule_does_not_change_tokens():
    """This engine's DVR schedule (deterministic prompts in shared prefill batches, verify
    passes of up to 16 sequences padded to a power of two, passes deferred until 8 windows
    are ready, run on a side stream beside the step's decode) commits exactly the tokens of
    the reference's schedule (one-request prefill groups, every pass padded to G = 4,
    verify whatever is ready after every decode step)."""
    prompts = _prompts(10, 300)
    params = [SamplingParams(max_new_tokens=70, temperature=0.7, seed=50 + i,
                             is_deterministic=i % 2 == 0, ignore_eos=True)
              for i in range(len(prompts))]
    reference = dict(dvr_isolated_prefill=True, dvr_group_size=4, dvr_verify_buckets=False,
                     dvr_min_verify=1, dvr_overlap_verify=False)
    outs = {}
    for name, extra in (("reference", reference), ("default", {})):
        cfg = EngineConfig(mode=Mode.DVR, kv_pool_tokens=32768, max_reqs=64, max_seq_len=2048,
                           max_decode_batch=64, num_layers=4, seed=7, **extra)
        print(f"schedule={name}", flush=True)
        res = Engine(cfg).generate(prompts, params)
        outs[name] = [o.token_ids for o in res]
        assert all(o.num_windows > 0 for o, p in zip(res, params) if p.is_deterministic)
    for i in range(0, len(prompts), 2):
        assert outs["reference"][i] == outs["default"][i], i


def test_dvr_shared_prefill_equals_isolated_prefill():
    """A prompt prefilled inside a shared batch gets the same logits, bit for bit, as when
    prefilled alone (the reference's isolated dvr prefill, scheduler.py:63-86), and the
    same K/V in the pool: every prefill kernel is batch-invariant."""
    from sid.engine.batch import build_prefill_batch
    from sid.engine.model_runner import ModelRunner
    from sid.engine.request import Request
    cfg = EngineConfig(mode=Mode.DVR, kv_pool_tokens=32768, max_reqs=64, max_seq_len=2048,
                       max_decode_batch=64, num_layers=4, seed=7)
    runner = ModelRunner(cfg, "cuda")
    prompts = _prompts(5, 77)

    def prefill(groups):
        logits, kv = {}, {}
        for grp in groups:
            reqs = []
            for i in grp:
                r = Request(i, prompts[i], SamplingParams(is_deterministic=True), (0,))
                r.req_row = runner.kv_cache.open_row()
                reqs.append(r)
            fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
            out = runner.forward(fb)
            for k, r in enumerate(reqs):
                logits[r.rid] = out[k].clone()
                slots = torch.from_numpy(runner.kv_cache.slot_range(r.req_row, 0, r.prompt_len))
                kv[r.rid] = runner.kv_cache.k_pools[-1][slots.cuda()].clone()
                runner.kv_cache.close_row(r.req_row)
        return logits, kv

    alone = prefill([[i] for i in range(5)])
    shared = prefill([[3, 0, 4, 1, 2]])
    for i in range(5):
        assert torch.equal(alone[0][i], shared[0][i]), i
        assert torch.equal(alone[1][i], shared[1][i]), i
