"""Which decode batches draw their tokens inside the lm_head (ModelRunner.fused_sample), on
the host: nothing here launches a kernel. The fused and the logits + sampler paths agree
except at float near-ties, so in batch_invariant mode the choice must not depend on the
batch (one answer per engine; a batch mixing rows with and without top-k / top-p limits
still takes the fused path for the latter, tests/test_gpu_engine.py) and the grouping is
fixed (streaming waves); nondet/dvr decode batches fuse up to the kernel's 256 rows with the
grouping left to the row count; DVR verify passes always fuse, with 128-column tiles."""

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


def test_invariant_grouping_is_fixed():
    r = _runner(256)
    for rows in (1, 64, 65, 256):
        fb = _fb(rows, True)
        assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is False


def test_nondet_fuses_up_to_256_rows():
    r = _runner(512)
    for rows in (1, 128, 129, 256):
        fb = _fb(rows, False)
        assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is None
    assert not ModelRunner.fused_sample(r, _fb(257, False))


def test_verify_passes_fuse_with_tiles():
    r = _runner(256)
    for rows in (1, 32, 128, 256):
        fb = _fb(rows, True, mode=ForwardMode.VERIFY)
        assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is True


def test_truncated_or_prefill_batches_never_fuse():
    r = _runner(256)
    assert not ModelRunner.fused_sample(r, _fb(8, False, untruncated=False))
    assert not ModelRunner.fused_sample(r, _fb(8, True, untruncated=False))
    assert not ModelRunner.fused_sample(r, _fb(8, True, untruncated=False, mode=ForwardMode.VERIFY))
    assert not ModelRunner.fused_sample(r, _fb(8, False, mode=ForwardMode.PREFILL))
