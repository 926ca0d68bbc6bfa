"""Which decode batches draw their tokens inside the lm_head (ModelRunner.fused_sample), on
the host: nothing here launches a kernel. The fused and the logits + sampler paths agree
except at float near-ties, so in batch_invariant mode the choice must not depend on the
batch (one answer per engine; a batch mixing rows with and without top-k / top-p limits
still takes the fused path for the latter, tests/test_gpu_engine.py), while nondet/dvr
pick the faster path by row count."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from sid.engine.batch import ForwardBatch, ForwardMode
from sid.engine.model_runner import ModelRunner


def _runner(max_decode_batch):
    r = SimpleNamespace(cfg=SimpleNamespace(max_decode_batch=max_decode_batch),
                        mcfg=SimpleNamespace(hidden_size=1024))
    r._invariant_fused = lambda: ModelRunner._invariant_fused(r)
    return r


def _fb(rows, invariant, untruncated=True, mode=ForwardMode.DECODE):
    z = torch.zeros(rows, dtype=torch.int64)
    return ForwardBatch(mode=mode, input_ids=z, positions=z, out_slots=z,
                        invariant=invariant, untruncated=untruncated)


@pytest.mark.parametrize("max_batch,expect", [(64, True), (256, True), (512, False)])
def test_batch_invariant_choice_is_one_per_engine(max_batch, expect):
    r = _runner(max_batch)
    got = {ModelRunner.fused_sample(r, _fb(rows, True)) for rows in (1, 7, 64, 129, max_batch)}
    assert got == {expect}


def test_nondet_picks_by_rows():
    r = _runner(256)
    assert ModelRunner.fused_sample(r, _fb(1, False))
    assert ModelRunner.fused_sample(r, _fb(128, False))
    assert not ModelRunner.fused_sample(r, _fb(129, False))
    assert not ModelRunner.fused_sample(r, _fb(256, False))


def test_truncated_or_non_decode_batches_never_fuse():
    r = _runner(256)
    assert not ModelRunner.fused_sample(r, _fb(8, False, untruncated=False))
    assert not ModelRunner.fused_sample(r, _fb(8, True, untruncated=False))
    assert not ModelRunner.fused_sample(r, _fb(8, True, mode=ForwardMode.VERIFY))
