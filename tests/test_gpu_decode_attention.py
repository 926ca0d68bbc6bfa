"""Split-KV decode attention (HIP) vs the fp32 CPU oracle, plus its bitwise invariants.

Cases follow the reference's tests/test_02_flash_decode.py:61-118 (split boundaries
31/32/33, 255/256/257, ragged batches, 5 split policies, shuffled slots), the BASELINE
configs 1 and 2 (page_size-16 block tables over large pools), empty requests, and the
determinism contract: fixed splits are run-to-run bitwise stable, fixed-256 results do
not depend on the batch, and different split counts change low-order bits.
Tolerance: max abs/rel error 2e-2 against fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HKV, HQ, D, SCALE, assert_close_bf16, decode_inputs
from oracle.attention import decode_attention_ref, plan_fixed, plan_heuristic
from oracle.cache import block_table_to_indices

pytestmark = pytest.mark.gpu


def _ext():
    from sid.kernels.jit import load_ext
    return load_ext()


def _run(q, k, v, indptr, idx, num_splits, grid, fixed, seg=0, slots=None, variant=0):
    bs = q.shape[0]
    slots = grid if slots is None else slots
    part_o = torch.full((bs, HQ, max(slots, 1), D), float("nan"), device="cuda")
    part_lse = torch.full((bs, HQ, max(slots, 1)), float("nan"), device="cuda")
    o = torch.empty_like(q)
    ns = torch.tensor(num_splits, dtype=torch.int32, device="cuda")
    _ext().flash_decode_fwd(q, k, v, indptr, idx, ns, grid, fixed, SCALE, part_o, part_lse, o,
                            segment_size=seg, grid_slots=slots, variant=variant)
    return o


def _run_ordered(q, k, v, indptr, idx, nst, grid, fixed, seg, slots, variant, order):
    """A grid launch with a workgroup order, into NaN-prefilled workspaces."""
    bs = q.shape[0]
    part_o = torch.full((bs, HQ, slots, D), float("nan"), device="cuda")
    part_lse = torch.full((bs, HQ, slots), float("nan"), device="cuda")
    o = torch.empty_like(q)
    _ext().flash_decode_fwd(q, k, v, indptr, idx, nst, grid, fixed, SCALE, part_o, part_lse, o,
                            segment_size=seg, grid_slots=slots, variant=variant, wg_order=order)
    return o


def _slots(seq_lens, num_splits, fixed, seg):
    """Partial slots the segmented grid needs (max over requests of n_splits * sps)."""
    best = 1
    for n, s in zip(seq_lens, num_splits):
        if n <= 0 or s <= 0:
            continue
        chunk = fixed if fixed > 0 else -(-(-(-n // s)) // 32) * 32
        sl = min(seg, chunk) if seg > 0 else chunk
        best = max(best, s * -(-chunk // sl))
    return best


def _policy(seq_lens, policy):
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    if policy == "heuristic":
        ns, grid = plan_heuristic(seq_lens, cu, HKV, 32)
        return ns, grid, 0
    if policy == "fixed256":
        ns, grid = plan_fixed(seq_lens)
        return ns, grid, 256
    s = int(policy.replace("splits", ""))
    return [min(-(-x // 32), s) for x in seq_lens], s, 0


CASES = [
    [1], [31], [32], [33], [255], [256], [257], [300, 5], [1000, 32, 999], [100] * 8,
    [17 * i + 1 for i in range(17)], [50] * 64, [5000],
]


@pytest.mark.parametrize("seq_lens", CASES, ids=lambda s: f"b{len(s)}_max{max(s)}")
@pytest.mark.parametrize("policy", ["heuristic", "fixed256", "splits1", "splits8", "splits32"])
def test_decode_vs_oracle(seq_lens, policy):
    q, k, v, indptr, idx = decode_inputs(seq_lens)
    ns, grid, fixed = _policy(seq_lens, policy)
    out = _run(q, k, v, indptr, idx, ns, grid, fixed)
    ref = decode_attention_ref(q, k, v, indptr, idx, SCALE)
    assert_close_bf16(out, ref)


@pytest.mark.parametrize("seq_lens", CASES, ids=lambda s: f"b{len(s)}_max{max(s)}")
@pytest.mark.parametrize("policy", ["heuristic", "fixed256", "splits1", "splits8"])
@pytest.mark.parametrize("seg", [64, 128, 256])
@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_decode_segments_vs_oracle(seq_lens, policy, seg, variant):
    """Splits cut into segments of <= seg tokens (one workgroup each), merged in token
    order by stage 2, for every stage-1 workgroup shape. Workspace pre-filled with NaN: a
    slot read but never written, or a token dropped, shows up."""
    q, k, v, indptr, idx = decode_inputs(seq_lens)
    ns, grid, fixed = _policy(seq_lens, policy)
    slots = _slots(seq_lens, ns, fixed, seg)
    print(f"lens={seq_lens[:4]} policy={policy} seg={seg} slots={slots} variant={variant}",
          flush=True)
    out = _run(q, k, v, indptr, idx, ns, grid, fixed, seg, slots, variant)
    ref = decode_attention_ref(q, k, v, indptr, idx, SCALE)
    assert_close_bf16(out, ref)


@pytest.mark.parametrize("variant", [1, 2, 3])
def test_variant_changes_bits_but_is_run_to_run_stable(variant):
    """The workgroup shape is part of the reduction order: another shape gives other bits
    (within tolerance), the same shape the same bits on every run."""
    lens = [1500, 2049, 700]
    q, k, v, indptr, idx = decode_inputs(lens, seed=9)
    ns, grid, fixed = _policy(lens, "fixed256")
    slots = _slots(lens, ns, fixed, 256)
    base = _run(q, k, v, indptr, idx, ns, grid, fixed, 256, slots, 0)
    a = _run(q, k, v, indptr, idx, ns, grid, fixed, 256, slots, variant)
    b = _run(q, k, v, indptr, idx, ns, grid, fixed, 256, slots, variant)
    assert torch.equal(a, b) and not torch.equal(a, base)
    assert_close_bf16(a, base)


@pytest.mark.parametrize("invariant", [False, True])
@pytest.mark.parametrize("lens", [[1, 2049, 300], [4096] * 3, [33] * 70, [777] * 9])
def test_planned_decode_vs_oracle(invariant, lens):
    """DecodeAttention's own plan (splits, segment size, grid slots) covers every token."""
    from sid.kernels.decode_attention import DecodeAttention
    q, k, v, indptr, idx = decode_inputs(lens, seed=5)
    attn = DecodeAttention(len(lens), HQ, HKV, D, 16, 256, 8192, "cuda")
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    _, _, _, seg, slots = attn.plan(seq, max(lens), invariant)
    print(f"lens={lens[:3]} invariant={invariant} seg={seg} slots={slots}", flush=True)
    out = attn.forward(q, k, v, indptr, idx, seq, max(lens), SCALE, invariant)
    assert_close_bf16(out, decode_attention_ref(q, k, v, indptr, idx, SCALE))


@pytest.mark.parametrize("lens", [[1024] * 256, [2048] * 256, [8192] * 64, [1025] * 256,
                                  [2049] * 96, [8192] * 32,
                                  [int(x) for x in (np.minimum(np.random.default_rng(3).lognormal(
                                      np.log(700), 0.8, 256), 8192) + 1).astype(int)],
                                  [int(x) for x in (np.minimum(np.random.default_rng(4).lognormal(
                                      np.log(512), 0.8, 32), 8192) + 300).astype(int)]],
                         ids=["b256x1024", "b256x2048", "b64x8192", "b256x1025", "b96x2049",
                              "b32x8192", "b256_lognormal", "b32_lognormal"])
def test_planned_geometries_vs_oracle(lens):
    """plan_variant's plans from real lengths (wide 8 x 2 workgroups for single-split grids,
    the multi-split plan below 64 requests) with the workgroup shape it picks, run through
    DecodeAttention.forward, against the oracle."""
    from sid.kernels.decode_attention import DecodeAttention, plan_variant
    q, k, v, indptr, idx = decode_inputs(lens, seed=8)
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    geom, variant = plan_variant(lens, max(lens), HKV, cu, 32, invariant=False)
    print(f"B={len(lens)} max={max(lens)} geometry={geom} variant={variant}", flush=True)
    attn = DecodeAttention(len(lens), HQ, HKV, D, 32, 256, 8192, "cuda")
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = attn.forward(q, k, v, indptr, idx, seq, max(lens), SCALE, False, variant=variant,
                       geometry=geom)
    torch.set_num_threads(16)
    assert_close_bf16(out, decode_attention_ref(q, k, v, indptr, idx, SCALE))


@pytest.mark.parametrize("policy", ["heuristic", "fixed256", "seg64"])
def test_workgroup_order_does_not_change_bits(policy):
    """The heaviest-first workgroup order (wg_order) only moves segments between workgroups:
    outputs are bitwise those of the grid's own order, for ragged batches with empty
    requests, through the workspace and the allocation-free entry points (NaN-prefilled
    workspaces: every partial the merge reads is written in the same call)."""
    from sid.kernels.decode_attention import segment_tokens, workgroup_order
    ext = _ext()
    rng = np.random.default_rng(12)
    lens = [int(x) for x in np.minimum(rng.lognormal(np.log(400), 1.0, 40), 6000).astype(int)]
    lens[3] = 0
    lens[17] = 1
    q, k, v, indptr, idx = decode_inputs(lens, seed=13)
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    if policy == "fixed256":
        ns, grid = plan_fixed(lens)
        fixed, seg, slots = 256, 256, grid
    else:
        ns, grid = plan_heuristic(lens, cu, HKV, 32)
        fixed, seg = 0, (256 if policy == "heuristic" else 64)
        slots = _slots(lens, ns, fixed, seg)
    tok = segment_tokens(lens, len(lens), grid, fixed, seg, slots)
    order = torch.from_numpy(workgroup_order(tok, cu)).cuda()
    print(f"policy={policy} slots={slots} busy={(tok > 0).sum()}", flush=True)
    plain = _run(q, k, v, indptr, idx, ns, grid, fixed, seg=seg, slots=slots)
    part_o = torch.full((len(lens), HQ, slots, D), float("nan"), device="cuda")
    part_lse = torch.full((len(lens), HQ, slots), float("nan"), device="cuda")
    o = torch.empty_like(q)
    nst = torch.tensor(ns, dtype=torch.int32, device="cuda")
    ext.flash_decode_fwd(q, k, v, indptr, idx, nst, grid, fixed, SCALE, part_o, part_lse, o,
                         segment_size=seg, grid_slots=slots, wg_order=order)
    assert torch.equal(o, plain)
    o2 = torch.empty_like(q)
    ext.flash_decode_fwd_noalloc(q, k, v, indptr, idx, nst, grid, fixed, SCALE, o2,
                                 segment_size=seg, grid_slots=slots, wg_order=order)
    assert torch.equal(o2, plain)
    assert (o[3] == 0).all()
    assert_close_bf16(o, decode_attention_ref(q, k, v, indptr, idx, SCALE))


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("policy", ["heuristic", "fixed256", "seg64"])
def test_worker_launch_equals_grid(policy, variant):
    """sid_flash_decode_workers_fwd: stage 1 by a fixed number of workgroups, each computing
    the items dealt to it in turn, gives bitwise the grid launch's output, for worker counts
    below, at and above the item count (ragged batch with an empty request and a one-token
    request; NaN-prefilled workspaces, so every partial the merge reads is written), and
    stays within the fp32 oracle's tolerance."""
    from sid.kernels.decode_attention import (ORDER_EMPTY, segment_tokens, worker_order,
                                              workgroup_order)
    ext = _ext()
    rng = np.random.default_rng(21)
    lens = [int(x) for x in np.minimum(rng.lognormal(np.log(400), 1.0, 24), 5000).astype(int)]
    lens[5] = 0
    lens[11] = 1
    q, k, v, indptr, idx = decode_inputs(lens, seed=23)
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    if policy == "fixed256":
        ns, grid = plan_fixed(lens)
        fixed, seg, slots = 256, 256, grid
    else:
        ns, grid = plan_heuristic(lens, cu, HKV, 32)
        fixed, seg = 0, (256 if policy == "heuristic" else 64)
        slots = _slots(lens, ns, fixed, seg)
    tok = segment_tokens(lens, len(lens), grid, fixed, seg, slots)
    plain = _run(q, k, v, indptr, idx, ns, grid, fixed, seg=seg, slots=slots, variant=variant)
    nst = torch.tensor(ns, dtype=torch.int32, device="cuda")
    items = len(lens) * slots
    for workers in (1, 7, cu, items + 5):
        # plain dealing, and worker_order's (empty items flagged when they all trail)
        for order_np in (workgroup_order(tok, workers), worker_order(tok, workers)):
            order = torch.from_numpy(order_np).cuda()
            flagged = int((order_np & ORDER_EMPTY != 0).sum())
            print(f"policy={policy} variant={variant} slots={slots} workers={workers} "
                  f"flagged={flagged}", flush=True)
            part_o = torch.full((len(lens), HQ, slots, D), float("nan"), device="cuda")
            part_lse = torch.full((len(lens), HQ, slots), float("nan"), device="cuda")
            o = torch.empty_like(q)
            ext.flash_decode_fwd(q, k, v, indptr, idx, nst, grid, fixed, SCALE, part_o,
                                 part_lse, o, segment_size=seg, grid_slots=slots,
                                 variant=variant, wg_order=order, workers=workers)
            assert torch.equal(o, plain), (workers, flagged)
    # the grid launch ignores the flag
    order = torch.from_numpy(worker_order(tok, items + 5)).cuda()
    o = _run_ordered(q, k, v, indptr, idx, nst, grid, fixed, seg, slots, variant, order)
    assert torch.equal(o, plain)
    assert (o[5] == 0).all()
    assert_close_bf16(o, decode_attention_ref(q, k, v, indptr, idx, SCALE))


def test_worker_launch_needs_an_order():
    lens = [300, 40]
    q, k, v, indptr, idx = decode_inputs(lens, seed=3)
    part_o = torch.empty((2, HQ, 4, D), device="cuda")
    part_lse = torch.empty((2, HQ, 4), device="cuda")
    with pytest.raises(RuntimeError, match="wg_order"):
        _ext().flash_decode_fwd(q, k, v, indptr, idx, None, 4, 0, SCALE, part_o, part_lse,
                                torch.empty_like(q), segment_size=64, grid_slots=4, workers=8)


@pytest.mark.parametrize("policy", ["heuristic", "fixed256", "splits8"])
def test_device_derived_split_counts_equal_explicit(policy):
    """num_splits = None: the kernel derives each request's split count from its length
    (the reference's policies); bitwise the same output as the explicit array, empty
    requests included."""
    ext = _ext()
    lens = [1, 31, 32, 33, 255, 257, 1000, 0, 4097, 64]
    q, k, v, indptr, idx = decode_inputs(lens, seed=17)
    ns, grid, fixed = _policy(lens, policy)  # the oracle's split counts
    slots = _slots(lens, ns, fixed, 64)
    want = _run(q, k, v, indptr, idx, ns, grid, fixed, seg=64, slots=slots)
    part_o = torch.full((len(lens), HQ, slots, D), float("nan"), device="cuda")
    part_lse = torch.full((len(lens), HQ, slots), float("nan"), device="cuda")
    got = torch.empty_like(q)
    ext.flash_decode_fwd(q, k, v, indptr, idx, None, grid, fixed, SCALE, part_o, part_lse, got,
                         segment_size=64, grid_slots=slots)
    assert torch.equal(got, want)
    assert (got[7] == 0).all()
    got2 = torch.empty_like(q)
    ext.flash_decode_fwd_noalloc(q, k, v, indptr, idx, None, grid, fixed, SCALE, got2,
                                 segment_size=64, grid_slots=slots)
    assert torch.equal(got2, want)


def test_direct_single_split_equals_two_stage():
    """Grid 1 writes o directly; a grid of 2 with every request on one split runs the
    merge pass. Both must give the same bits (merge of one split is the identity)."""
    lens = [37, 300, 1]
    q, k, v, indptr, idx = decode_inputs(lens, seed=3)
    a = _run(q, k, v, indptr, idx, [1, 1, 1], 1, 0)
    b = _run(q, k, v, indptr, idx, [1, 1, 1], 2, 0)
    assert torch.equal(a, b)


def test_empty_request_gives_zeros():
    q, k, v, indptr, idx = decode_inputs([5, 7], seed=4)
    indptr = torch.tensor([0, 0, 7], dtype=torch.int32, device="cuda")
    for grid in (1, 4):
        out = _run(q, k, v, indptr, idx, [0, 1], grid, 0)
        assert torch.count_nonzero(out[0]) == 0
        ref = decode_attention_ref(q[1:], k, v, torch.tensor([0, 7]), idx.cpu(), SCALE)
        assert_close_bf16(out[1:], ref)


def test_fixed_splits_run_to_run_bitwise():
    lens = [123, 456, 789, 7]
    q, k, v, indptr, idx = decode_inputs(lens)
    ns, grid = plan_fixed(lens)
    a = _run(q, k, v, indptr, idx, ns, grid, 256)
    for _ in range(3):
        assert torch.equal(a, _run(q, k, v, indptr, idx, ns, grid, 256))


def test_split_count_changes_bits():
    q, k, v, indptr, idx = decode_inputs([4096])
    outs = [_run(q, k, v, indptr, idx, [min(128, s)], s, 0) for s in (1, 3, 8, 32)]
    for o in outs[1:]:
        assert_close_bf16(o, outs[0].float(), atol=3e-2, rtol=3e-2)
    assert any(not torch.equal(outs[0], o) for o in outs[1:])


def test_fixed256_is_batch_invariant():
    """A request's fixed-256 output is bitwise identical alone and inside other batches
    (the grid size changes with the batch's max length; its result must not)."""
    g = torch.Generator().manual_seed(9)
    pool = 20000
    k = torch.randn(pool, HKV, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(pool, HKV, D, generator=g).to(torch.bfloat16).cuda()
    q0 = torch.randn(1, HQ, D, generator=g).to(torch.bfloat16).cuda()
    idx0 = torch.randperm(pool - 1, generator=g)[:1500] + 1

    def run(others):
        qs, idxs, lens = [], [], []
        for pos, L in enumerate(others):
            if L is None:
                qs.append(q0)
                idxs.append(idx0)
                lens.append(1500)
            else:
                qs.append(torch.randn(1, HQ, D, generator=g).to(torch.bfloat16).cuda())
                idxs.append(torch.randint(1, pool, (L,), generator=g))
                lens.append(L)
        indptr = torch.zeros(len(lens) + 1, dtype=torch.int32)
        indptr[1:] = torch.cumsum(torch.tensor(lens), 0)
        ns, grid = plan_fixed(lens)
        out = _run(torch.cat(qs), k, v, indptr.cuda(), torch.cat(idxs).to(torch.int32).cuda(),
                   ns, grid, 256)
        return out[others.index(None)]

    base = run([None])
    for comp in ([None, 100], [4000, None, 3], [7] * 15 + [None]):
        assert torch.equal(base, run(comp))


@pytest.mark.parametrize("plan", [(0, 32, 0), (0, 32, 64), (256, 0, 64), (256, 0, 0), (0, 5, 32),
                                  (0, 6, 0), (0, 12, 0), (0, 16, 0), (0, 24, 0)],
                         ids=["heur32", "heur32_seg64", "fixed256_seg64", "fixed256", "split5_seg32",
                              "heur6", "heur12", "heur16", "heur24"])
def test_stage2_latency_kernel_bits_equal_batch_kernel(plan):
    """Batches of at most 4 requests merge with the latency-oriented stage 2 and larger ones
    with the throughput ones (grids of up to 32 slots: one load batch per workgroup, sized
    4 / 8 / 12 / 16 / 24 / 32; more: the slot loop); all fold the same slots in the same
    order, so a request's output must be bitwise the same alone (B=1) and among 7 others
    (B=8), for 1 to 128 used slots (more than one 32-slot load chunk)."""
    fixed, max_splits, seg = plan
    g = torch.Generator().manual_seed(21)
    pool = 40000
    k = torch.randn(pool, HKV, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(pool, HKV, D, generator=g).to(torch.bfloat16).cuda()

    def splits(n):
        return -(-n // fixed) if fixed else min(-(-n // 32), max_splits)

    for L in (1, 33, 1024, 2047, 8192):
        q0 = torch.randn(1, HQ, D, generator=g).to(torch.bfloat16).cuda()
        idx0 = (torch.randperm(pool - 1, generator=g)[:L] + 1).to(torch.int32)
        others = [int(x) for x in torch.randint(1, 3000, (7,), generator=g)]
        outs = []
        for lens in ([L], others[:3] + [L] + others[3:]):
            qs, idxs = [], []
            for n in lens:
                if n == L and len(qs) == (0 if len(lens) == 1 else 3):
                    qs.append(q0)
                    idxs.append(idx0)
                else:
                    qs.append(torch.randn(1, HQ, D, generator=g).to(torch.bfloat16).cuda())
                    idxs.append(torch.randint(1, pool, (n,), generator=g, dtype=torch.int32))
            indptr = torch.zeros(len(lens) + 1, dtype=torch.int32)
            indptr[1:] = torch.cumsum(torch.tensor(lens), 0)
            ns = [splits(n) for n in lens]
            slots = _slots(lens, ns, fixed, seg)
            o = _run(torch.cat(qs), k, v, indptr.cuda(), torch.cat(idxs).cuda(), ns, max(ns), fixed,
                     seg=seg, slots=slots)
            outs.append(o[0 if len(lens) == 1 else 3])
        assert torch.isfinite(outs[0].float()).all()
        assert torch.equal(outs[0], outs[1]), f"L={L}"


def _paged_case(num_pages, seq_lens, seed):
    rng = np.random.default_rng(seed)
    bs = len(seq_lens)
    pages_needed = [-(-L // 16) for L in seq_lens]
    perm = rng.permutation(num_pages)
    tables, off = [], 0
    for n in pages_needed:
        tables.append(perm[off:off + n])
        off += n
    idx = np.concatenate([block_table_to_indices(t, L) for t, L in zip(tables, seq_lens)])
    indptr = np.zeros(bs + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(seq_lens)
    return torch.from_numpy(idx).cuda(), torch.from_numpy(indptr.astype(np.int32)).cuda()


def test_config1_paged_single_request():
    """q [1,16,128], ctx 1024, page 16, 256-page pool, randperm table."""
    torch.manual_seed(1)
    q = torch.randn(1, HQ, D, device="cuda").to(torch.bfloat16)
    k = torch.randn(256 * 16, HKV, D, device="cuda").to(torch.bfloat16)
    v = torch.randn(256 * 16, HKV, D, device="cuda").to(torch.bfloat16)
    idx, indptr = _paged_case(256, [1024], seed=1)
    ref = decode_attention_ref(q, k, v, indptr, idx, SCALE)
    for policy in ("heuristic", "fixed256"):
        ns, grid, fixed = _policy([1024], policy)
        assert_close_bf16(_run(q, k, v, indptr, idx, ns, grid, fixed), ref)


def test_config2_cache_write_then_decode():
    """B=32, ctx ~ U[128, 4096], 32k-page x 16 pool, new K/V written by
    reshape_and_cache (bit-exact) then attended with both split policies."""
    rng = np.random.default_rng(2)
    lens = rng.integers(128, 4097, size=32).tolist()
    slots_total = 32768 * 16
    torch.manual_seed(2)
    k = torch.randn(slots_total, HKV, D, device="cuda").to(torch.bfloat16)
    v = torch.randn(slots_total, HKV, D, device="cuda").to(torch.bfloat16)
    q = torch.randn(32, HQ, D, device="cuda").to(torch.bfloat16)
    idx, indptr = _paged_case(32768, lens, seed=2)
    ends = indptr[1:].long() - 1
    new_slots = idx[ends].long()
    k_new = torch.randn(32, HKV, D, device="cuda").to(torch.bfloat16)
    v_new = torch.randn(32, HKV, D, device="cuda").to(torch.bfloat16)
    keep = torch.ones(idx.numel(), dtype=torch.bool, device="cuda")
    keep[ends] = False
    others = idx[keep].long()
    before_k, before_v = k[others].clone(), v[others].clone()
    _ext().reshape_and_cache(k_new, v_new, k, v, new_slots)
    assert torch.equal(k[new_slots], k_new) and torch.equal(v[new_slots], v_new)
    assert torch.equal(k[others], before_k) and torch.equal(v[others], before_v)
    used = idx.long()
    ref = decode_attention_ref(q.cpu(), k[used].cpu(), v[used].cpu(), indptr.cpu(),
                               torch.arange(used.numel(), dtype=torch.int32), SCALE)
    outs = {}
    for policy in ("heuristic", "fixed256"):
        ns, grid, fixed = _policy(lens, policy)
        outs[policy] = _run(q, k, v, indptr, idx, ns, grid, fixed)
        assert_close_bf16(outs[policy], ref)
