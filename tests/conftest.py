"""Test setup: import paths, the `gpu` marker, shared input builders.

GPU tests (marked `gpu`) call the HIP kernels through the C-ABI library and compare them
with the CPU oracle (oracle/) on the same seeded inputs. CPU tests cover the oracle, the
host logic and the library's exported symbols.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "deterministic-inference_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running end-to-end test")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


HQ, HKV, D = 16, 8, 128
SCALE = D ** -0.5


def assert_close_bf16(actual: torch.Tensor, ref: torch.Tensor, atol=2e-2, rtol=2e-2):
    torch.testing.assert_close(actual.float().cpu(), ref.float().cpu(), atol=atol, rtol=rtol)


def decode_inputs(seq_lens, seed=0, device="cuda", extra_slots=64):
    """q, k/v pools with shuffled non-contiguous slots (slot 0 reserved), kv_indptr/indices.
    Same construction as tests/test_02_flash_decode.py:19-31 of the reference."""
    g = torch.Generator().manual_seed(seed)
    bs, total = len(seq_lens), sum(seq_lens)
    num_slots = total + extra_slots
    q = torch.randn(bs, HQ, D, generator=g).to(torch.bfloat16)
    k = torch.randn(num_slots, HKV, D, generator=g).to(torch.bfloat16)
    v = torch.randn(num_slots, HKV, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_slots - 1, generator=g)[:total] + 1
    indptr = torch.zeros(bs + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(seq_lens, dtype=torch.int64), 0).to(torch.int32)
    t = [x.to(device) for x in (q, k, v, indptr, perm.to(torch.int32))]
    return tuple(t)
