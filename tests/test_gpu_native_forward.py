"""The native extend-forward executor (sid_qwen3_extend_forward) is bit-identical to the
op-by-op Python driver of Qwen3Model.forward: logits, greedy tokens and the KV written to
the pool, for prefill batches on both sides of the split-K threshold (256 tokens), with and
without sampled-row gathers, and for a DVR verify batch."""

from __future__ import annotations

import pytest
import torch

from sid.config import EngineConfig, Mode, SamplingParams
from sid.engine.batch import build_prefill_batch
from sid.engine.model_runner import ModelRunner
from sid.engine.request import Request

pytestmark = pytest.mark.gpu


def _runner():
    cfg = EngineConfig(mode=Mode.DVR, kv_pool_tokens=16384, max_reqs=16, max_seq_len=2048,
                       max_decode_batch=16, num_layers=3, seed=5, use_graphs=False)
    return ModelRunner(cfg, "cuda")


def _reqs(runner, lens, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = []
    for rid, p in enumerate(lens):
        r = Request(rid, torch.randint(0, 151936, (p,), generator=g).tolist(),
                    SamplingParams(max_new_tokens=40, is_deterministic=True, ignore_eos=True),
                    runner.mcfg.eos_token_ids)
        r.req_row = runner.kv_cache.open_row()
        out.append(r)
    return out


def _both(runner, fb, greedy):
    """Python driver, then the native executor from the same starting pool state."""
    model = runner.model
    pools = [runner.kv_cache.layer(i) for i in range(runner.mcfg.num_layers)]
    start = [(k.clone(), v.clone()) for k, v in pools]
    model.native_extend = False
    a = runner.model.forward(fb, runner.kv_cache, runner.decode_attn, greedy=greedy).clone()
    kv_a = [(k.clone(), v.clone()) for k, v in pools]
    for (k, v), (k0, v0) in zip(pools, start):
        k.copy_(k0)
        v.copy_(v0)
    model.native_extend = True
    b = runner.model.forward(fb, runner.kv_cache, runner.decode_attn, greedy=greedy)
    kv_b = [(k.clone(), v.clone()) for k, v in pools]
    return a, b, kv_a, kv_b


@pytest.mark.parametrize("lens", [[5], [40, 3, 100], [300], [200, 180]])
@pytest.mark.parametrize("greedy", [False, True])
def test_prefill_native_equals_python(lens, greedy):
    runner = _runner()
    reqs = _reqs(runner, lens)
    fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
    print(f"lens={lens} tokens={sum(lens)} greedy={greedy}", flush=True)
    a, b, kv_a, kv_b = _both(runner, fb, greedy)
    assert torch.equal(a, b)
    for (ka, va), (kb, vb) in zip(kv_a, kv_b):
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_all_rows_and_verify_batch_native_equals_python():
    from sid.engine.dvr import Verifier
    runner = _runner()
    reqs = _reqs(runner, [64, 90], seed=1)
    fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
    fb.sample_indices = None  # every token row: R = T
    a, b, _, _ = _both(runner, fb, greedy=False)
    assert a.shape[0] == 154 and torch.equal(a, b)
    # prefill for real, decode until 20 unverified tokens, then a verify batch
    runner = _runner()
    reqs = _reqs(runner, [40, 90], seed=3)
    ver = Verifier(runner.cfg, runner, runner.kv_cache)
    for r in reqs:
        fb = build_prefill_batch([r], runner.kv_cache, "cuda", invariant=False)
        r.output_ids.append(runner.step(fb).item())
        r.verified_len = 1
    while any(r.unverified() < 20 for r in reqs):
        fb = runner.prepare_decode(reqs, False)
        for r, t in zip(reqs, runner.step(fb).tolist()):
            r.output_ids.append(t)
    fb, _ = ver.build_verify_batch(reqs)
    for greedy in (False, True):
        print(f"verify greedy={greedy}", flush=True)
        a, b, kv_a, kv_b = _both(runner, fb, greedy)
        assert torch.equal(a, b)
        for (ka, va), (kb, vb) in zip(kv_a, kv_b):
            assert torch.equal(ka, kb) and torch.equal(va, vb)
