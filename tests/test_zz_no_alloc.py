"""The allocation-free decode attention entry point (sid_flash_decode_segments_fwd_noalloc,
split partials in the library's static per-GPU scratch) against the workspace entry point
(sid_flash_decode_segments_fwd) on the same inputs: bit-identical outputs on two calls in a
row, the second with a smaller batch, for multi-slot plans of both split policies; and a
call whose partials exceed the scratch is rejected with an error."""

from __future__ import annotations

import pytest
import torch

from conftest import D, HKV, HQ, SCALE, decode_inputs

pytestmark = pytest.mark.gpu


def _ext():
    from sid.kernels.jit import load_ext
    return load_ext()


def _plan(lens, invariant, attn):
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    return attn.plan(seq, max(lens), invariant)


@pytest.mark.parametrize("invariant", [False, True])
def test_noalloc_matches_workspace_entry(invariant):
    from sid.kernels.decode_attention import DecodeAttention
    ext = _ext()
    attn = DecodeAttention(16, HQ, HKV, D, 32, 256, 8192, "cuda")
    for call, lens in enumerate(([700, 2049, 33, 1500, 4000, 257, 1, 96],   # first call
                                 [1200, 64, 3000])):                       # then smaller
        print(f"noalloc call {call}: invariant={invariant} lens={lens}", flush=True)
        q, k, v, indptr, idx = decode_inputs(lens, seed=10 + call)
        num_splits, grid, fixed, seg, slots = _plan(lens, invariant, attn)
        assert slots > 1
        want = torch.empty_like(q)
        ext.flash_decode_fwd(q, k, v, indptr, idx, num_splits, grid, fixed, SCALE,
                             attn.part_o, attn.part_lse, want, segment_size=seg,
                             grid_slots=slots)
        got = torch.full_like(q, float("nan"))
        ext.flash_decode_fwd_noalloc(q, k, v, indptr, idx, num_splits, grid, fixed, SCALE, got,
                                     segment_size=seg, grid_slots=slots)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_rejects_partials_beyond_scratch():
    ext = _ext()
    cap = int(ext.lib.sid_flash_decode_noalloc_scratch_bytes())
    b, slots = 64, 1024
    assert b * HQ * slots * (D + 1) * 4 > cap
    q, k, v, indptr, idx = decode_inputs([300] * b, seed=3)
    num_splits = torch.ones(b, dtype=torch.int32, device="cuda")
    o = torch.empty_like(q)
    with pytest.raises(RuntimeError, match="scratch"):
        ext.flash_decode_fwd_noalloc(q, k, v, indptr, idx, num_splits, 32, 0, SCALE, o,
                                     segment_size=64, grid_slots=slots)
