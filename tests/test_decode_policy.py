"""Host-side decode-attention policy (no GPU): split heuristic, segment size, the grid's
slot count covering every request's segments, and the graph-key sequence buckets."""

from __future__ import annotations

import random

import pytest

from sid.kernels.decode_attention import length_bucket as seq_bucket
from sid.kernels.decode_attention import (MAX_GRID_SLOTS, SEGMENT_SIZES, heuristic_splits,
                                          nondet_geometry, segment_size, workspace_slots)


def _segments(n: int, splits: int, fixed: int, seg: int) -> list[tuple[int, int]]:
    """Token ranges of a request's segments, by walking its splits token by token."""
    s = min(splits, -(-n // 32)) if fixed == 0 else -(-n // fixed)
    if fixed:
        chunk = fixed
    else:
        per = -(-n // s)
        chunk = -(-per // 32) * 32
    out = []
    for i in range(s):
        a, b = i * chunk, min((i + 1) * chunk, n)
        while a < b:
            out.append((a, min(a + seg, b)))
            a = min(a + seg, b)
    return out


def test_heuristic_splits_matches_reference_formula_cases():
    # reference decode_attention.py:73-74 on 256 CUs, 8 KV heads, max 16 splits
    assert heuristic_splits(64, 8, 256, 16) == 1
    assert heuristic_splits(8, 8, 256, 16) == 8
    assert heuristic_splits(1, 8, 256, 16) == 16
    assert heuristic_splits(3, 8, 256, 16) == 16
    assert heuristic_splits(33, 8, 256, 16) == 2


def test_segment_size_prefers_long_segments_when_grid_is_full():
    # largest segment with >= 1.5 workgroups per CU (384 on 256 CUs)
    assert segment_size(64, 2049, 256) == 256   # 64 x 9 = 576
    assert segment_size(32, 2049, 256) == 128   # 32 x 9 = 288 < 384; 32 x 17 = 544
    assert segment_size(8, 2049, 256) == 64
    assert segment_size(4, 8192, 256) == 64     # 4 x 64 = 256 < 384 at 128
    assert segment_size(48, 1025, 256) == 128   # 48 x 5 = 240; 48 x 9 = 432
    assert segment_size(1, 10, 256) == SEGMENT_SIZES[-1]


@pytest.mark.parametrize("seed", range(20))
def test_nondet_slots_cover_every_request(seed):
    rng = random.Random(seed)
    bs = rng.choice([1, 2, 3, 8, 17, 64, 200])
    max_len = rng.choice([1, 31, 32, 33, 255, 256, 257, 1000, 2049, 8191])
    lens = [rng.randint(1, max_len) for _ in range(bs)]
    lens[0] = max_len
    splits, seg, slots = nondet_geometry(bs, max_len, 8, 256, 16)
    need = max(len(_segments(n, splits, 0, seg)) for n in lens)
    assert need <= slots <= workspace_slots(max_len, 16, 256)
    assert sum(b - a for a, b in _segments(max_len, splits, 0, seg)) == max_len


def test_invariant_segments_are_the_256_splits():
    for n in (1, 255, 256, 257, 5000):
        segs = _segments(n, 0, 256, 256)
        assert len(segs) == -(-n // 256) and all(b - a <= 256 for a, b in segs)


def test_workspace_slots_capped():
    assert workspace_slots(10 ** 6, 16, 256) == MAX_GRID_SLOTS


def test_seq_bucket():
    prev = 0
    for n in range(1, 20000, 7):
        b = seq_bucket(n)
        assert b >= n and b >= prev
        prev = b
    assert [seq_bucket(n) for n in (1, 256, 257, 384, 385, 2049, 3073)] == [
        256, 256, 384, 384, 512, 3072, 4096]


def test_batch_bucket():
    from sid.engine.batch import batch_bucket
    sizes = set()
    for bs in range(1, 257):
        b = batch_bucket(bs, 256)
        assert bs <= b <= 256
        sizes.add(b)
    assert len(sizes) <= 24  # few graphs for any mix of batch sizes
    assert [batch_bucket(n, 256) for n in (1, 3, 5, 9, 64, 65, 129, 250)] == [
        1, 4, 8, 16, 64, 80, 160, 256]
    assert batch_bucket(100, 96) == 100  # never below the real size


def test_decode_backend_names():
    """The reference's names select the same paths; anything else is an error."""
    import pytest
    from sid.config import EngineConfig
    assert EngineConfig(decode_backend="cuda").decode_backend == "hip"
    assert EngineConfig(decode_backend="hip").decode_backend == "hip"
    assert EngineConfig(decode_backend="triton").decode_backend == "extend"
    assert EngineConfig().decode_backend == "hip"
    with pytest.raises(ValueError):
        EngineConfig(decode_backend="cuDNN")


def test_nonempty_workgroups_brute_force():
    """Counted segment by segment with the oracle's split ranges."""
    import numpy as np
    from oracle.attention import kv_per_split, split_ranges
    from sid.kernels.decode_attention import nonempty_workgroups
    rng = np.random.default_rng(0)
    for _ in range(200):
        lens = rng.integers(0, 5000, size=int(rng.integers(1, 20))).tolist()
        splits = int(rng.integers(1, 33))
        seg = int(rng.choice([64, 128, 256]))
        want = 0
        for n in lens:
            ns = min(splits, -(-n // 32))
            if n == 0:
                continue
            sl = min(seg, kv_per_split(n, ns, 0))
            for a, b in split_ranges(n, ns, 0):
                want += len(range(a, b, sl))
        assert nonempty_workgroups(lens, splits, seg) == want, (lens, splits, seg)


def test_stage1_variant_rule():
    from sid.kernels.decode_attention import stage1_variant
    assert stage1_variant(576, 256, invariant=False) == 1     # >= 2 per CU
    assert stage1_variant(512, 256, invariant=False) == 1
    assert stage1_variant(576, 256, invariant=True) == 2      # invariant: one fixed shape
    assert stage1_variant(3, 256, invariant=True) == 2
    assert stage1_variant(230, 256, invariant=False) == 2     # fewer than the CUs
    assert stage1_variant(32, 256, invariant=False) == 2
    assert stage1_variant(256, 256, invariant=False) == 3     # one to two per CU
    assert stage1_variant(511, 256, invariant=False) == 3


def test_multi_split_plans():
    """For multi-split grids (fewer than 64 requests) plan_variant takes the longest of
    512/256/128/64-token segments with >= 0.75 half-full workgroups per CU, counted over the
    batch's real lengths, and the shape stage1_variant gives that count; batches with less
    work keep the size-based segment."""
    import numpy as np

    from sid.kernels.decode_attention import (heuristic_splits, nondet_geometry,
                                              nonempty_workgroups, plan_variant)
    cu = 256
    assert heuristic_splits(32, 8, cu, 32) == 2

    def plan(lens):
        geom, variant = plan_variant(lens, max(lens), 8, cu, 32, invariant=False)
        return geom, variant

    assert plan([8192] * 32) == ((2, 512, 16), 1)      # 32 x 2 x 8 = 512 workgroups
    assert plan([2048] * 48) == ((2, 512, 4), 2)       # 192 full 512-token workgroups
    assert plan([2048] * 24)[0][1] == 256              # 3 splits of 683: 216 workgroups
    # a lognormal batch: the longest segment with 0.75 half-full workgroups per CU
    rng = np.random.default_rng(7)
    lens = (np.minimum(rng.lognormal(np.log(512), 0.8, 32), 8192) + 300).astype(int).tolist()
    (splits, seg, _), variant = plan(lens)
    assert splits == 2 and seg <= nondet_geometry(32, max(lens), 8, cu, 32)[1]
    assert nonempty_workgroups(lens, 2, seg, seg // 2) >= 0.75 * cu
    assert nonempty_workgroups(lens, 2, 2 * seg, seg) < 0.75 * cu
    # one request of 1024 tokens (config 1): 32 splits of 32 tokens; the size-based plan
    assert plan([1024]) == ((32, 64, 32), 2)
    assert plan_variant([1024] * 4, 1024, 8, cu, 32, invariant=True) == (None, 2)


def test_wide_plans_for_single_split_batches():
    """From 64 requests up (one split each) plan_variant takes the wide-workgroup plan: the
    longest segment with >= 0.6 half-full workgroups per CU, a longest workgroup of at most
    1/170 of the batch's tokens and (once every CU has one) balanced CUs; 8 x 2 below two
    workgroups per CU, 4 x 1 from two; segments of 512+ at about one per CU halved into 4 x 1
    when the halves fill every CU twice."""
    import numpy as np

    from sid.kernels.decode_attention import _wide_plan, plan_variant
    cu = 256

    def plan(lens):
        geom, variant = plan_variant(lens, max(lens), 8, cu, 32, invariant=False)
        assert geom[0] == 1 and geom[2] == -(-(-(-max(lens) // 32) * 32) // geom[1])
        return geom[1], variant

    assert plan([2049] * 64) == (256, 1)      # config 3: 512-token halves into 256 x 4 x 1
    assert plan([1025] * 256) == (2048, 2)    # one 8 x 2 workgroup per request
    assert plan([520] * 256) == (1024, 2)
    assert plan([2049] * 96) == (1024, 2)     # 192 full 1024-token workgroups
    assert plan([2049] * 128) == (512, 1)     # 256 x 1024 -> 512 x 512 of 4 x 1
    assert plan([2049] * 256) == (1024, 1)
    assert plan([4097] * 192) == (1024, 1)    # 2048: 384 workgroups leave CUs uneven
    # Too little work for 0.6 half-full workgroups per CU at any size: the segment rules.
    assert _wide_plan(np.array([100] * 64), cu) is None
    assert plan([100] * 64) == (64, 2)
    # A few requests far longer than the rest: their workgroups would set the time, so the
    # segment is cut until the longest holds <= 1/170 of the tokens.
    lens = [300] * 200 + [8192] * 4
    seg, _ = plan(lens)
    assert seg * 170 <= sum(lens) < 1024 * 170 and seg < 1024


def test_workgroup_counts_match_the_partition():
    """nonempty_workgroups(..., min_tokens) == the number of slots of segment_tokens (the
    kernel's partition, itself checked against a walk of the splits) holding at least
    min_tokens tokens."""
    import numpy as np

    from sid.kernels.decode_attention import nonempty_workgroups, segment_tokens
    rng = np.random.default_rng(3)
    for _ in range(300):
        b = int(rng.integers(1, 80))
        lens = rng.integers(0, 5000, b)
        splits = int(rng.integers(1, 33))
        seg = int(rng.choice([64, 128, 256, 512, 1024, 2048]))
        mx = max(int(lens.max()), 1)
        chunk_max = max(32, -(-(-(-mx // splits)) // 32) * 32)
        slots = splits * max(1, -(-chunk_max // seg))
        tok = segment_tokens(lens, b, splits, 0, seg, slots)
        for min_tokens in (1, seg // 4, seg // 2, seg):
            assert nonempty_workgroups(lens, splits, seg, min_tokens) == int(
                (tok >= max(min_tokens, 1)).sum())


def _walk_tokens(n, splits, fixed, seg):
    """Token count of every partial slot of one request, walking its splits and segments."""
    if n <= 0:
        return []
    if fixed:
        s, chunk = -(-n // fixed), fixed
    else:
        s = min(splits, -(-n // 32))
        chunk = -(-(-(-n // s)) // 32) * 32
    sl = min(seg, chunk) if seg > 0 else chunk
    sps = -(-chunk // sl)
    out = []
    for i in range(s):
        a, b = i * chunk, min((i + 1) * chunk, n)
        for j in range(sps):
            st = a + j * sl
            out.append(max(0, min(st + sl, b) - st))
    return out


@pytest.mark.parametrize("plan", [(1, 0, 256), (32, 0, 64), (4, 0, 128), (0, 256, 256), (2, 0, 512)])
def test_segment_tokens_match_the_kernel_partition(plan):
    """segment_tokens (the host mirror of the kernel's segment_range) gives every slot's token
    count: the slot-by-slot walk of each request's splits and segments, zeros for padding
    rows and for slots past a request's last segment."""
    import numpy as np

    from sid.kernels.decode_attention import segment_tokens
    splits, fixed, seg = plan
    rng = random.Random(7)
    lens = [rng.randint(1, 5000) for _ in range(37)] + [1, 31, 32, 33, 255, 256, 257]
    walks = [_walk_tokens(n, splits, fixed, seg) for n in lens]
    slots = max(len(w) for w in walks) + 3
    tok = segment_tokens(lens, len(lens) + 5, splits, fixed, seg, slots)
    assert tok.shape == (slots, len(lens) + 5)
    for b, w in enumerate(walks):
        assert tok[:len(w), b].tolist() == w
        assert not tok[len(w):, b].any()
    assert not tok[:, len(lens):].any()
    assert int(tok.sum()) == sum(lens)


def test_workgroup_order_is_a_balanced_permutation():
    """workgroup_order is a permutation of the grid (request << 12 | slot), heaviest segments
    first in rounds of cu_count with every other full round of unequal segments reversed,
    ties in the grid's own order (so a uniform batch keeps the grid's order)."""
    import numpy as np

    from sid.kernels.decode_attention import ORDER_SLOT_BITS, workgroup_order
    rng = np.random.default_rng(3)
    slots, rows, cu = 11, 50, 16
    tok = rng.integers(0, 300, size=(slots, rows))
    tok[rng.random((slots, rows)) < 0.3] = 0
    order = workgroup_order(tok, cu)
    b, y = order >> ORDER_SLOT_BITS, order & ((1 << ORDER_SLOT_BITS) - 1)
    assert sorted((y * rows + b).tolist()) == list(range(slots * rows))
    work = tok[y, b]
    n = order.size
    ranked = []
    for k in range(0, n, cu):
        chunk = work[k:k + cu].tolist()
        rnd = k // cu
        if rnd % 2 == 1 and k + cu <= n and len(set(chunk)) > 1:
            chunk = chunk[::-1]
        ranked += chunk
    assert ranked == sorted(work.tolist(), reverse=True)
    # equal work keeps the grid's order (request fastest), over several full rounds too
    flat = np.full((4, 6), 7, dtype=np.int64)
    assert workgroup_order(flat, 4).tolist() == [(b << ORDER_SLOT_BITS) | y
                                                for y in range(4) for b in range(6)]


def test_stage1_workers_rule():
    """Worker launches only for 8 x 2 plans of several slots whose non-empty items number
    more than half the CUs and at most the CU count (one worker per CU)."""
    from sid.kernels.decode_attention import WORKERS_VARIANT, stage1_workers
    cu = 256
    assert WORKERS_VARIANT == 2
    assert stage1_workers(241, 2, 7, cu) == cu
    assert stage1_workers(129, 2, 20, cu) == cu
    assert stage1_workers(256, 2, 16, cu) == cu
    assert stage1_workers(128, 2, 32, cu) == 0   # half the CUs or fewer: the grid
    assert stage1_workers(257, 2, 16, cu) == 0   # more items than CUs: the grid
    assert stage1_workers(241, 1, 7, cu) == 0    # 4 x 1 / 4 x 2 / 4 x 4 keep the grid
    assert stage1_workers(241, 3, 7, cu) == 0
    assert stage1_workers(241, 0, 7, cu) == 0
    assert stage1_workers(200, 2, 1, cu) == 0    # single-slot grids write o directly


def test_worker_dealing_covers_every_item_once():
    """A worker launch's wg_order (workgroup_order over the workers): worker w takes the
    entries w, w + W, ...; every (request, slot) item, empty ones included, is dealt to
    exactly one worker, and the workers' token loads differ by at most one item's tokens
    beyond a perfect split of the heaviest-first rounds."""
    import numpy as np

    from sid.kernels.decode_attention import ORDER_SLOT_BITS, workgroup_order
    rng = np.random.default_rng(9)
    slots, rows = 9, 40
    tok = rng.integers(0, 512, size=(slots, rows))
    tok[rng.random((slots, rows)) < 0.4] = 0
    for workers in (1, 5, 64, 300, slots * rows + 3):
        order = workgroup_order(tok, workers)
        assert order.size == slots * rows
        seen = set()
        loads = np.zeros(workers, dtype=np.int64)
        for w in range(workers):
            for e in order[w::workers]:
                b, y = int(e) >> ORDER_SLOT_BITS, int(e) & ((1 << ORDER_SLOT_BITS) - 1)
                assert (b, y) not in seen
                seen.add((b, y))
                loads[w] += tok[y, b]
        assert len(seen) == slots * rows
        assert loads.max() - loads.min() <= tok.max()


def test_worker_order_flags_only_trailing_empty_items():
    """worker_order flags the empty items (ORDER_EMPTY) when the non-empty ones fit one round
    of the dealing; then in every worker's sequence (entries w, w + W, ...) the flagged
    entries are exactly the empty items and come after all the others. With more non-empty
    items than workers nothing is flagged."""
    import numpy as np

    from sid.kernels.decode_attention import (ORDER_EMPTY, ORDER_SLOT_BITS, worker_order,
                                              workgroup_order)
    rng = np.random.default_rng(4)
    for trial in range(40):
        slots, rows = int(rng.integers(1, 20)), int(rng.integers(1, 40))
        tok = rng.integers(1, 500, size=(slots, rows))
        tok[rng.random((slots, rows)) < rng.random()] = 0
        workers = int(rng.integers(1, 300))
        order = worker_order(tok, workers)
        plain = workgroup_order(tok, workers)
        assert ((order & ~ORDER_EMPTY) == plain).all()
        nonempty = int(np.count_nonzero(tok))
        flag = (order & ORDER_EMPTY) != 0
        if nonempty > workers:
            assert not flag.any()
            continue
        entry = order & ~ORDER_EMPTY
        b, y = entry >> ORDER_SLOT_BITS, entry & ((1 << ORDER_SLOT_BITS) - 1)
        assert (flag == (tok[y, b] == 0)).all()
        for w in range(workers):
            f = flag[w::workers]
            if f.any():
                assert f[int(np.argmax(f)):].all()
