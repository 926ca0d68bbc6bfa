"""lm_head with the sampler fused into its epilogue (sid_linear_sample): no logits are
written, yet the tokens are those of the exact-rule oracle (oracle/sampler.py
sample_exact_ref) applied to the logits of the same GEMM, for greedy and stochastic rows
(top_k <= 0, top_p >= 1) at the real lm_head shape, across row counts (one and several
64-row groups). The per-wave candidate certificate is checked against recomputing every
column exactly, and non-finite logits take the exact path."""

from __future__ import annotations

import math

import pytest
import torch

from oracle.sampler import sample_exact_ref
from test_gpu_sampler import _score

pytestmark = pytest.mark.gpu

V, K = 151936, 1024


@pytest.fixture(scope="module")
def lm_head():
    g = torch.Generator(device="cuda").manual_seed(5)
    return (torch.randn(V, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)


def _rows(m, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = (torch.randn(m, K, device="cuda", generator=g) * 3.0).to(torch.bfloat16)
    temps = torch.tensor([[0.0, 0.7, 1.0, 1.5, 0.3][i % 5] for i in range(m)], device="cuda")
    seeds = torch.arange(m, device="cuda", dtype=torch.int64) * 977 + seed
    pos = torch.arange(m, device="cuda", dtype=torch.int64) * 13 + 300
    return x, temps, seeds, pos


@pytest.mark.parametrize("m,tiles", [(1, None), (5, None), (64, None), (100, None),
                                     (5, True), (64, True), (128, None), (256, None),
                                     (100, False), (256, False), (512, None), (600, True)])
def test_fused_sample_equals_oracle(lm_head, m, tiles):
    """Streaming-wave groups up to 64 rows (tiles=None) or at any size (False); 128-column
    tile groups above 64 rows (None) or at any size (True: the grouping verify passes
    use; above 256 rows only these)."""
    from sid.kernels.matmul_persistent import linear, linear_sample
    x, temps, seeds, pos = _rows(m, 10 + m)
    print(f"fused sampler m={m} tiles={tiles}", flush=True)
    got = linear_sample(x, lm_head, temps, seeds, pos, tiles=tiles).cpu()
    logits = linear(x, lm_head, out_fp32=True).cpu()
    n = torch.full((m,), -1, dtype=torch.int64)
    ones = torch.ones(m)
    want = sample_exact_ref(logits, temps.cpu(), n, ones, seeds.cpu(), pos.cpu())
    _assert_near_ties(got, want, logits, temps.cpu(), seeds.cpu(), pos.cpu())
    # the unfused HIP path (logits + sid_sample_rows) on the same logits: per row the same
    # token, or a near-tie under the same rule
    from sid.engine.sampler import sample
    unfused = sample(logits.cuda(), temps, n.cuda(), ones.cuda(), seeds, pos).cpu()
    _assert_near_ties(got, unfused, logits, temps.cpu(), seeds.cpu(), pos.cpu())


def _assert_near_ties(got, want, logits, temps, seeds, pos):
    """Every row where the fused token differs must be a stochastic row whose fused token
    scores within 1e-4 of the other one under the exact rule (the exp/log ulps of torch's
    CPU kernels and of the device differ; nothing else may)."""
    for r in range(got.shape[0]):
        if got[r] == want[r]:
            continue
        t = float(temps[r])
        assert t > 0, f"greedy row {r}: {int(got[r])} != {int(want[r])}"
        a = _score(logits[r], t, -1, 1.0, int(seeds[r]), int(pos[r]), int(got[r]))
        b = _score(logits[r], t, -1, 1.0, int(seeds[r]), int(pos[r]), int(want[r]))
        assert math.isfinite(a) and abs(a - b) < 1e-4, (r, int(got[r]), int(want[r]), a, b)


@pytest.mark.parametrize("m,tiles", [(64, None), (64, True), (200, None), (200, False),
                                     (300, True)])
def test_certificate_equals_full_recompute(lm_head, m, tiles):
    from sid.kernels.matmul_persistent import linear_sample
    x, temps, seeds, pos = _rows(m, 3)
    a = linear_sample(x, lm_head, temps, seeds, pos, tiles=tiles)
    b = linear_sample(x, lm_head, temps, seeds, pos, recompute_all=True, tiles=tiles)
    assert torch.equal(a, b)


def test_tiled_sampler_writes_the_logits(lm_head):
    """With a logits buffer the tiled sampler writes sid_linear's fp32 logits and draws the
    same tokens as without it."""
    from sid.kernels.matmul_persistent import linear, linear_sample
    x, temps, seeds, pos = _rows(70, 9)
    lg = torch.full((70, V), float("nan"), device="cuda")
    a = linear_sample(x, lm_head, temps, seeds, pos, logits=lg)
    b = linear_sample(x, lm_head, temps, seeds, pos, tiles=True)
    assert torch.equal(lg, linear(x, lm_head, out_fp32=True))
    assert torch.equal(a, b)


def test_non_finite_logits_follow_the_reference(lm_head):
    """A +inf logit makes every probability NaN in the reference (inf - inf); its argmax of
    NaN scores is the first column. Greedy rows keep torch.argmax's NaN rule."""
    from sid.kernels.matmul_persistent import linear_sample
    w = lm_head.clone()
    w[777] = float("inf")
    x, temps, seeds, pos = _rows(4, 8)
    x = x.abs()  # every logit of column 777 is +inf
    got = linear_sample(x, w, temps, seeds, pos).cpu()
    from sid.kernels.matmul_persistent import linear
    logits = linear(x, w, out_fp32=True).cpu()
    n, ones = torch.full((4,), -1), torch.ones(4)
    want = sample_exact_ref(logits, temps.cpu(), n, ones, seeds.cpu(), pos.cpu())
    assert got.tolist() == want.tolist()


@pytest.mark.parametrize("tiles", [False, True])
def test_fused_sample_is_row_independent(lm_head, tiles):
    """A row's token does not depend on the other rows of the batch (or on its slot), for a
    fixed grouping (streaming waves or tiles, at any size)."""
    from sid.kernels.matmul_persistent import linear_sample
    n = 600 if tiles else 80
    x, temps, seeds, pos = _rows(n, 21)
    full = linear_sample(x, lm_head, temps, seeds, pos, tiles=tiles)
    for j in (0, 17, 63, 64, 79, 300, n - 1):
        if j >= n:
            continue
        one = linear_sample(x[j:j + 1], lm_head, temps[j:j + 1], seeds[j:j + 1], pos[j:j + 1],
                            tiles=tiles)
        assert one.item() == full[j].item()


def test_row_limits_per_grouping(lm_head):
    """The streaming waves take at most 256 rows, the tiles at most 4096: beyond, the call
    fails with an error (nothing launched) and the workspace query answers 0."""
    from sid.kernels.jit import load_ext
    from sid.kernels.matmul_persistent import linear_sample, linear_sample_supported
    ext = load_ext()
    assert ext.linear_sample_workspace_bytes(4096) > 0
    assert ext.linear_sample_workspace_bytes(4097) == 0
    assert linear_sample_supported(4096, K) and not linear_sample_supported(4097, K)
    assert not linear_sample_supported(257, K, tiles=False)
    x, temps, seeds, pos = _rows(257, 4)
    ws = torch.empty(ext.linear_sample_workspace_bytes(257), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="M <= 256"):
        linear_sample(x, lm_head, temps, seeds, pos, workspace=ws, tiles=False)
