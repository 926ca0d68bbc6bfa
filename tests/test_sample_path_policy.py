"""Which decode batches draw their tokens inside the lm_head (ModelRunner.fused_sample), on
the host: nothing here launches a kernel. The fused and the logits + sampler paths agree
except at float near-ties, so in batch_invariant mode the choice must not depend on the
batch (one answer per engine; a batch mixing rows with and without top-k / top-p limits
still takes the fused path for the latter, tests/test_gpu_engine.py) and the grouping is
fixed (streaming waves); nondet/dvr decode batches fuse up to the kernel's 4096 rows with the
grouping left to the row count; prefill and DVR verify passes always fuse, with 128-column
tiles."""

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
    r._sampled_rows = lambda fb: ModelRunner._sampled_rows(r, fb)
    r._tiles_always = lambda fb: ModelRunner._tiles_always(r, fb)
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


def test_nondet_fuses_up_to_the_kernels_rows():
    r = _runner(512)
    for rows in (1, 128, 129, 256, 512):
        fb = _fb(rows, False)
        assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is None
    assert not ModelRunner.fused_sample(r, _fb(4097, False))


@pytest.mark.parametrize("mode", [ForwardMode.VERIFY, ForwardMode.PREFILL])
def test_verify_and_prefill_passes_fuse_with_tiles(mode):
    r = _runner(256)
    for rows in (1, 32, 128, 256, 512, 4096):
        for invariant in (False, True):
            fb = _fb(rows, invariant, mode=mode)
            assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is True


def test_prefill_rows_are_the_sampled_ones():
    r = _runner(256)
    fb = _fb(5000, False, mode=ForwardMode.PREFILL)  # 5000 prompt tokens, 3 sequences
    fb.sample_indices = torch.tensor([99, 2999, 4999])
    assert ModelRunner.fused_sample(r, fb) and fb.sample_tiles is True


def test_truncated_batches_never_fuse():
    r = _runner(256)
    assert not ModelRunner.fused_sample(r, _fb(8, False, untruncated=False))
    assert not ModelRunner.fused_sample(r, _fb(8, True, untruncated=False))
    for mode in (ForwardMode.VERIFY, ForwardMode.PREFILL):
        assert not ModelRunner.fused_sample(r, _fb(8, True, untruncated=False, mode=mode))


def test_engine_config_bounds_sampled_rows():
    """Prefill batches and verify passes larger than the fused sampler's 4096 rows would move
    their untruncated rows to the sampler kernel: such configurations are refused."""
    from sid.config import MAX_SAMPLED_ROWS, EngineConfig
    from sid.kernels.matmul_persistent import linear_sample_supported
    assert linear_sample_supported(MAX_SAMPLED_ROWS, 1024)
    assert not linear_sample_supported(MAX_SAMPLED_ROWS + 1, 1024)
    EngineConfig(max_decode_batch=MAX_SAMPLED_ROWS, dvr_group_size=128, dvr_window_size=32)
    with pytest.raises(ValueError, match="max_decode_batch"):
        EngineConfig(max_decode_batch=MAX_SAMPLED_ROWS + 1)
    with pytest.raises(ValueError, match="verify pass"):
        EngineConfig(dvr_group_size=256, dvr_window_size=32)
