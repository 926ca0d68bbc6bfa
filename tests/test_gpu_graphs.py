"""HIP-graph replays of the decode and verify forwards are bit-identical to eager forwards
(same weights, same requests), across steps, batch sizes (one graph each) and modes."""

from __future__ import annotations

import pytest
import torch

from sid.config import EngineConfig, Mode, SamplingParams
from sid.engine.batch import build_prefill_batch
from sid.engine.model_runner import ModelRunner
from sid.engine.request import Request

pytestmark = pytest.mark.gpu


def _runner(graphs, mode=Mode.NONDET):
    cfg = EngineConfig(mode=mode, kv_pool_tokens=8192, max_reqs=16, max_seq_len=1024,
                       max_decode_batch=16, num_layers=2, seed=11, use_graphs=graphs)
    return ModelRunner(cfg, "cuda")


def _requests(runner, lens, seed=0):
    g = torch.Generator().manual_seed(seed)
    reqs = []
    for rid, p in enumerate(lens):
        r = Request(rid, torch.randint(0, 151936, (p,), generator=g).tolist(),
                    SamplingParams(max_new_tokens=64), runner.mcfg.eos_token_ids)
        r.req_row = runner.kv_cache.open_row()
        reqs.append(r)
    return reqs


@pytest.mark.parametrize("invariant", [False, True])
def test_decode_graph_equals_eager(invariant):
    # A decode graph runs its batch padded to the bucket size (5 -> 8, 3 -> 4); the nondet
    # split policy follows the real request count, so padded and eager runs agree bitwise
    # in both modes.
    lens = [30, 300, 7, 64, 129]
    outs = {}
    for graphs in (False, True):
        runner = _runner(graphs)
        reqs = _requests(runner, lens)
        fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
        for r, t in zip(reqs, runner.sample(fb, runner.forward(fb)).tolist()):
            r.output_ids.append(t)
        logs = []
        for step in range(6):
            active = reqs if step < 3 else reqs[:3]
            fb = runner.prepare_decode(active, invariant)
            assert (fb.graph_key is not None) == graphs
            lg = runner.forward(fb)
            logs.append(lg.clone())
            toks = runner.sample(fb, lg).tolist()
            # fused lm_head + argmax (its own graph) picks the same tokens
            assert fb.all_greedy and runner.step(fb).tolist() == toks
            for r, t in zip(active, toks):
                r.output_ids.append(t)
        outs[graphs] = (logs, [r.output_ids for r in reqs])
    assert outs[True][1] == outs[False][1]
    for a, b in zip(outs[True][0], outs[False][0]):
        assert torch.equal(a, b)


def test_verify_graph_equals_eager():
    from sid.engine.dvr import Verifier
    results = {}
    for graphs in (False, True):
        runner = _runner(graphs, Mode.DVR)
        reqs = _requests(runner, [40, 90], seed=3)
        for r in reqs:
            r.params.is_deterministic = True
        ver = Verifier(runner.cfg, runner, runner.kv_cache)
        fb = build_prefill_batch(reqs[:1], runner.kv_cache, "cuda", invariant=False)
        reqs[0].output_ids.append(runner.sample(fb, runner.forward(fb)).item())
        fb = build_prefill_batch(reqs[1:], runner.kv_cache, "cuda", invariant=False)
        reqs[1].output_ids.append(runner.sample(fb, runner.forward(fb)).item())
        for r in reqs:
            r.verified_len = 1
        logs = []
        for _ in range(2):  # two verify passes: the graph is captured, then replayed
            while any(r.unverified() < 20 for r in reqs):
                fb = runner.prepare_decode(reqs, False)
                for r, t in zip(reqs, runner.sample(fb, runner.forward(fb)).tolist()):
                    r.output_ids.append(t)
            fb, meta = ver.build_verify_batch(reqs)
            runner.tag_verify(fb)
            lg = runner.forward(fb)
            logs.append(lg.clone())
            ver.compare_and_rollback(meta, runner.sample(fb, lg))
        results[graphs] = (logs, [r.output_ids for r in reqs])
    assert results[True][1] == results[False][1]
    for a, b in zip(results[True][0], results[False][0]):
        assert torch.equal(a, b)


def test_decode_graph_near_max_seq_len():
    """A request just past a length bucket near max_seq_len (8194 tokens, bucket 12288,
    max_seq_len 9000): the graph's plan is bounded by max_seq_len, so its grid fits the
    split workspace, and the graph replay equals the eager forward bitwise."""
    outs = {}
    for graphs in (False, True):
        cfg = EngineConfig(mode=Mode.NONDET, kv_pool_tokens=9200, max_reqs=2, max_seq_len=9000,
                           max_decode_batch=2, num_layers=2, seed=11, use_graphs=graphs)
        runner = ModelRunner(cfg, "cuda")
        reqs = _requests(runner, [8193])
        fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
        reqs[0].output_ids.append(int(runner.sample(fb, runner.forward(fb))[0]))
        fb = runner.prepare_decode(reqs, False)
        print(f"graphs={graphs} max_seq_len={fb.max_seq_len} geometry={fb.decode_geometry}",
              flush=True)
        outs[graphs] = runner.forward(fb).clone()
    assert torch.equal(outs[True], outs[False])


@pytest.mark.parametrize("graphs", [False, True])
def test_decode_worker_launch_equals_grid(graphs, monkeypatch):
    """A decode batch whose attention plan is an 8 x 2 grid with between half the CUs and
    the CU count of non-empty segments runs stage 1 as one worker workgroup per CU
    (stage1_workers); its logits are bitwise those of the same step with the grid launch."""
    import sid.engine.model_runner as mr
    lens = [2596, 2019, 1680, 1028, 1131, 410, 503, 344]
    cfg = EngineConfig(mode=Mode.NONDET, kv_pool_tokens=16384, max_reqs=16, max_seq_len=4096,
                       max_decode_batch=16, num_layers=2, seed=13, use_graphs=graphs)
    runner = ModelRunner(cfg, "cuda")
    reqs = _requests(runner, lens, seed=5)
    fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
    for r, t in zip(reqs, runner.sample(fb, runner.forward(fb)).tolist()):
        r.output_ids.append(t)
    fb = runner.prepare_decode(reqs, False)
    if fb.decode_workers == 0:
        pytest.skip(f"this device's CU count gives no worker plan for these lengths")
    print(f"workers={fb.decode_workers} variant={fb.decode_variant} geom={fb.decode_geometry}",
          flush=True)
    worker = runner.forward(fb).clone()
    monkeypatch.setattr(mr, "stage1_workers", lambda *a: 0)
    fb = runner.prepare_decode(reqs, False)
    assert fb.decode_workers == 0
    grid = runner.forward(fb)
    assert torch.equal(worker, grid)


def test_decode_worker_graph_replays_follow_each_steps_order():
    """Decode steps through a captured graph whose attention runs as a worker launch: the
    order (with its empty-item flags) is refilled every step, so replays of one graph for
    batches with different non-empty segments give the eager forward's logits bitwise."""
    import numpy as np

    from sid.kernels.decode_attention import ORDER_EMPTY
    lens = [2596, 2019, 1680, 1028, 1131, 410, 503, 344]
    logs, keys, flags = {}, {}, {}
    for graphs in (False, True):
        cfg = EngineConfig(mode=Mode.NONDET, kv_pool_tokens=16384, max_reqs=16,
                           max_seq_len=4096, max_decode_batch=16, num_layers=2, seed=13,
                           use_graphs=graphs)
        runner = ModelRunner(cfg, "cuda")
        reqs = _requests(runner, lens, seed=5)
        fb = build_prefill_batch(reqs, runner.kv_cache, "cuda", invariant=False)
        for r, t in zip(reqs, runner.sample(fb, runner.forward(fb)).tolist()):
            r.output_ids.append(t)
        logs[graphs], keys[graphs], flags[graphs] = [], [], []
        for step in range(70):
            fb = runner.prepare_decode(reqs, False)
            keys[graphs].append((fb.graph_key, fb.decode_workers))
            if fb.decode_workers:
                order = fb.decode_wg_order.cpu().numpy()
                flags[graphs].append(int((order & ORDER_EMPTY != 0).sum()))
            lg = runner.forward(fb)
            logs[graphs].append(lg.clone())
            for r, t in zip(reqs, runner.sample(fb, lg).tolist()):
                r.output_ids.append(t)
    for a, b in zip(logs[True], logs[False]):
        assert torch.equal(a, b)
    used = [k for k in keys[True] if k[1]]
    if not used:
        pytest.skip("this device's CU count gives no worker plan for these lengths")
    # one graph served steps with different sets of empty items
    by_key = {}
    for (k, w), f in zip(used, flags[True]):
        by_key.setdefault(k, set()).add(f)
    print({str(k)[:60]: sorted(v) for k, v in by_key.items()}, flush=True)
    assert any(len(v) > 1 for v in by_key.values())
