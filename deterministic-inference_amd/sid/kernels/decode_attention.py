"""Decode attention: split-KV HIP kernel plus the num_splits policy.

Policy (kept exactly as sid/kernels/decode_attention.py:1-17, 56-85 of the reference,
with the device's compute-unit count as its input):

* nondet / dvr: ``splits = clamp(ceil(2 * CUs / (B * HKV)), 1, max_kv_splits)``, then per
  request ``min(splits, ceil(len / 32))``; the grid has ``splits`` slots. The split count
  depends on the batch size, so a request's bits depend on its co-tenants: this is the
  designed nondeterminism of the fast path.
* batch_invariant: fixed 256-token splits, ``ceil(len / 256)`` per request, grid
  ``ceil(max_len / 256)``; a request's result depends only on its own length.

MI355X addition: the kernel's workgroup reads all KV heads of a token range (whole
2 KiB pool rows), so a split is further cut into segments of at most ``seg`` tokens,
one workgroup each. batch_invariant uses seg = 256 = the split size (the reference's
partition, independent of the batch); nondet/dvr take the largest of 256/128/64 that
still gives 1.5 workgroups per CU for the batch's longest request, rounded up to a
length bucket (so a HIP graph captured for a bucket computes the same plan). From the
batch's real lengths, plan_variant gives single-split grids (64 requests and more) wide
8 x 2 workgroups of up to 2048 tokens when there is work for them (_wide_plan), and
multi-split grids the longest of 512-64 tokens that still gives 0.75 half-full workgroups
per CU (_multi_split_plan). The stage-1 workgroup shape is picked with the plan.

B in the policy is the number of real requests. A caller that pads its batch with empty
requests (graph replay at a fixed size) passes the real count as ``policy_batch``, so
padded and unpadded runs of the same requests pick the same splits and give the same bits.
"""

from __future__ import annotations

import functools

import numpy as np
import torch

from sid.kernels.jit import load_ext


@functools.lru_cache(maxsize=8)
def _cu_count(device_index: int) -> int:
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def heuristic_splits(batch: int, num_kv_heads: int, cu_count: int, max_kv_splits: int) -> int:
    """Grid split count of the nondet/dvr policy (reference decode_attention.py:73-74)."""
    splits = -(-2 * cu_count // (batch * num_kv_heads))
    return max(1, min(splits, max_kv_splits))


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


SEGMENT_SIZES = (256, 128, 64)
MAX_GRID_SLOTS = 1024  # kernel limit on partial slots per request


def segment_size(batch: int, max_len: int, cu_count: int) -> int:
    """nondet/dvr segment length: the largest of SEGMENT_SIZES whose grid
    (batch x segments of the longest request) has at least 1.5 workgroups per CU. (Measured
    on B = 4..160 at lengths 1k-8k, uniform and mixed: this picks the fastest segment in
    all but one case, B = 24 at 2k, 4% off; a 1-per-CU rule chose 256 for B = 32 at 2k,
    18% slower than 128.)"""
    for seg in SEGMENT_SIZES:
        if 2 * batch * -(-max_len // seg) >= 3 * cu_count:
            return seg
    return SEGMENT_SIZES[-1]


def length_bucket(n: int) -> int:
    """Smallest of 256 * {1, 1.5, 2, 3, 4, 6, ...} >= n."""
    b = 256
    while True:
        if b >= n:
            return b
        if b + b // 2 >= n:
            return b + b // 2
        b *= 2


def nondet_geometry(batch: int, max_len: int, num_kv_heads: int, cu_count: int,
                    max_kv_splits: int) -> tuple[int, int, int]:
    """(grid splits, segment size, grid slots) of the nondet/dvr plan. A request of length
    n <= max_len gets s = min(splits, ceil(n/32)) splits of chunk
    ceil(ceil(n/s)/32)*32 <= chunk_max tokens, each cut into ceil(chunk/seg) segments, so
    splits * ceil(chunk_max/seg) slots cover every request."""
    splits = heuristic_splits(batch, num_kv_heads, cu_count, max_kv_splits)
    chunk_max = max(32, _cdiv(_cdiv(max_len, splits), 32) * 32)
    seg = segment_size(batch, length_bucket(max_len), cu_count)
    return splits, seg, splits * max(1, _cdiv(chunk_max, seg))


def nonempty_workgroups(lengths, splits: int, seg: int, min_tokens: int = 1) -> int:
    """Stage-1 workgroups of a nondet/dvr plan that hold at least min_tokens tokens: per
    request of length n, its min(splits, ceil(n/32)) splits of kv_per_split tokens, each cut
    into segments of at most seg (host-side, from the requests' lengths)."""
    lens = np.asarray(lengths, dtype=np.int64)
    lens = lens[lens > 0]
    if lens.size == 0:
        return 0
    min_tokens = max(int(min_tokens), 1)
    n = np.minimum(splits, -(-lens // 32))
    chunk = -(-(-(-lens // n)) // 32) * 32
    sl = np.minimum(seg, chunk)
    total = 0
    for s in range(int(n.max())):
        part = np.clip(lens - s * chunk, 0, chunk) * (s < n)
        full = part // sl
        tail = part - full * sl
        total += int((full * (sl >= min_tokens)).sum() + (tail >= min_tokens).sum())
    return total


# Stage-1 workgroup shapes (sid_flash_decode_segments_fwd `variant`): 0 = 4 waves x 4 tokens
# per iteration, 1 = 4 x 1, 2 = 8 x 2, 3 = 4 x 2. The shape is part of the in-segment
# reduction order. batch_invariant uses one shape for every batch (results depend on the
# request alone): 8 x 2, which with the heaviest-first order is the fastest fixed choice
# (0.935 x the time of 4 x 4 over 11 shapes from one request to B = 256: small batches 10-15%
# faster, config 3's shape 2.5%, lognormal B = 128 8%; B = 256 x 1024 0.4% slower). nondet/dvr
# pick by the number of non-empty workgroups W against the CU count.
# Fewer workgroups than CUs are bound by each workgroup's chain of round trips: 8 x 2 (B = 1,
# ctx 1024, 13.3 -> 12.5 us; lognormal B = 64 77.7 -> 60.1 us). One to two per CU: 4 x 2
# (config 2, 59.3 -> 56.1 us). Two or more per CU are HBM-bound and run best with the fewest
# registers: 4 x 1 (config 3, 91.5 -> 88.9 us). Ragged batches used to keep 4 x 4, which
# copes best with CUs left idle at the end; with the heaviest-first workgroup order
# (workgroup_order, used from W >= CUs) the W rule alone is as fast or faster on all 15
# shapes measured (lognormal B = 256 154.2 -> 145.6 us, B = 128 84.3 -> 81.4 us).
INVARIANT_VARIANT = 2


def stage1_variant(workgroups: int, cu_count: int, invariant: bool) -> int:
    """The stage-1 workgroup shape for a plan with `workgroups` non-empty workgroups."""
    if invariant:
        return INVARIANT_VARIANT
    if workgroups < cu_count:
        return 2
    if workgroups < 2 * cu_count:
        return 3
    return 1


# Wide-workgroup plans for single-split grids (64 requests and more). An 8 x 2 workgroup
# keeps four times the bytes of a 4 x 1 one in flight, so a few hundred of them already
# stream at the chip's rate; then fewer, longer segments win (fewer partials, a shorter
# merge, no near-empty tails). Measured on whole decode steps (15 uniform shapes and 6
# lognormal batches at B = 64-256, against eight fixed plans each): the plans below average
# 1.1% from the best plan of each shape, against 2.8% for the segment rules alone, e.g.
# B = 192 x 1024 5.83 -> 5.32 ms per step, B = 96 x 2048 5.33 -> 5.13 ms, lognormal B = 128
# 3.96 -> 3.84 ms; config 3's shape keeps 256-token segments of 4 x 1.
WIDE_SEGMENTS = (2048, 1024, 512, 256, 128)
WIDE_MIN_PER_CU = 0.6        # 8 x 2 workgroups holding at least half a segment
WIDE_TOKENS_PER_LONGEST = 170  # the longest workgroup holds <= 1/170 of the batch's tokens
WIDE_MAX_IMBALANCE = 1.3     # busiest CU / mean CU load, once they cover every CU


def _cu_imbalance(sizes: np.ndarray, cu_count: int) -> float:
    """Busiest CU's tokens over the mean when `sizes` (workgroup tokens) are dealt
    heaviest first, every other round reversed, as workgroup_order deals them."""
    w = np.sort(sizes[sizes > 0])[::-1]
    if w.size == 0:
        return 1.0
    rounds = _cdiv(w.size, cu_count)
    m = np.zeros(rounds * cu_count, dtype=np.int64)
    m[:w.size] = w
    m = m.reshape(rounds, cu_count)
    m[1::2] = m[1::2, ::-1]
    loads = m.sum(axis=0)
    return float(loads.max()) / max(float(loads.mean()), 1.0)


def _wide_plan(lens: np.ndarray, cu_count: int):
    """(segment, variant) of the wide-workgroup plan of a single-split batch, or None. Takes
    the longest segment whose half-full workgroups number at least 0.6 per CU, whose longest
    workgroup is a small share of the batch, and which, once every CU has one, balances;
    segments of 512 or more that leave about one workgroup per CU become half-size 4 x 1
    workgroups when those fill every CU twice. Two or more workgroups per CU run 4 x 1
    (enough in flight already; isolated B = 256 x 4096 with 2048-token segments: 638 us with
    4 x 1, 654 us with 8 x 2)."""
    total = int(lens.sum())
    longest = int(lens.max())
    for seg in WIDE_SEGMENTS:
        full, tail = lens // seg, lens % seg
        carrying = int(full.sum() + (tail >= seg // 2).sum())
        if carrying < WIDE_MIN_PER_CU * cu_count:
            continue
        if min(seg, longest) * WIDE_TOKENS_PER_LONGEST > total:
            continue
        if carrying >= cu_count:
            sizes = np.concatenate([np.full(int(full.sum()), seg, dtype=np.int64), tail])
            if _cu_imbalance(sizes, cu_count) > WIDE_MAX_IMBALANCE:
                continue
        if seg >= 512 and 4 * carrying <= 5 * cu_count:
            half = seg // 2
            if int((lens // half).sum() + (lens % half >= half // 2).sum()) >= 2 * cu_count:
                return half, 1
        return seg, (1 if carrying >= 2 * cu_count else 2)
    return None


# Plans for multi-split grids (fewer than 64 requests), from the real lengths: the longest
# of MULTI_SPLIT_SEGMENTS whose half-full workgroups number at least 0.75 per CU, with the
# shape stage1_variant gives that count. The size-based segment counts every request as long
# as the (bucketed) longest, so a few long requests among short ones left half the chip
# idle: lognormal B = 32 2.53 -> 1.87 ms per step, B = 48 2.73 -> 2.25 ms. Measured on whole
# steps (21 uniform shapes B = 1-48 x 512-8192, 8 lognormal batches, 15 fixed plans each):
# 1.1% from the best plan of each shape on average, against 5.6% before.
MULTI_SPLIT_SEGMENTS = (512, 256, 128, 64)
MULTI_SPLIT_MIN_PER_CU = 0.75


def _multi_split_plan(lens: np.ndarray, splits: int, cu_count: int):
    for seg in MULTI_SPLIT_SEGMENTS:
        carrying = nonempty_workgroups(lens, splits, seg, seg // 2)
        if carrying >= MULTI_SPLIT_MIN_PER_CU * cu_count:
            return seg, stage1_variant(carrying, cu_count, invariant=False)
    return None


def plan_variant(lengths, max_len: int, num_kv_heads: int, cu_count: int, max_kv_splits: int,
                 invariant: bool) -> tuple:
    """(nondet geometry or None, stage-1 variant) for a batch of known lengths; max_len is
    the (possibly bucketed) bound the plan is built for. The geometry (grid splits, segment
    size, grid slots) is what DecodeAttention.forward runs when given it: the wide plan for
    single-split grids, the multi-split plan otherwise, and the size-based segment (with the
    shape for its non-empty workgroups) for batches too small for either."""
    if invariant:
        return None, INVARIANT_VARIANT
    lens = np.asarray(lengths, dtype=np.int64)
    geom = nondet_geometry(len(lens), max_len, num_kv_heads, cu_count, max_kv_splits)
    splits, seg, slots = geom
    if lens.size and int(lens.min()) > 0:
        pick = (_wide_plan(lens, cu_count) if splits == 1
                else _multi_split_plan(lens, splits, cu_count))
        if pick is not None:
            chunk_max = max(32, _cdiv(_cdiv(max_len, splits), 32) * 32)
            return (splits, pick[0], splits * max(1, _cdiv(chunk_max, pick[0]))), pick[1]
    return geom, stage1_variant(nonempty_workgroups(lens, splits, seg), cu_count, invariant=False)


ORDER_SLOT_BITS = 12  # sid_flash_decode_segments_fwd wg_order entries: request << 12 | slot
ORDER_EMPTY = 1 << 30  # wg_order entry flag of a worker launch: the item holds no tokens


def segment_tokens(lengths, rows: int, splits: int, fixed_split: int, seg: int,
                   slots: int) -> np.ndarray:
    """int64 [slots, rows]: tokens of partial slot y of request b, as the kernel's
    segment_range cuts them (rows past len(lengths) are empty padding). fixed_split > 0 is
    the batch_invariant plan (one segment per fixed split); else the nondet plan of
    `splits` grid splits, min(splits, ceil(len/32)) per request, segments of at most seg."""
    lens = np.zeros(rows, dtype=np.int64)
    lens[:len(lengths)] = np.asarray(lengths, dtype=np.int64)
    pos = lens > 0
    safe = np.maximum(lens, 1)
    if fixed_split > 0:
        n = -(-lens // fixed_split)
        chunk = np.full(rows, fixed_split, dtype=np.int64)
    else:
        n = np.where(pos, np.minimum(splits, -(-safe // 32)), 0)
        chunk = -(-(-(-safe // np.maximum(n, 1))) // 32) * 32
    sl = np.minimum(seg, chunk) if seg > 0 else chunk
    sps = -(-chunk // sl)
    y = np.arange(slots, dtype=np.int64)[:, None]
    s = y // sps
    split_start = s * chunk
    split_end = np.minimum(split_start + chunk, lens)
    start = split_start + (y % sps) * sl
    end = np.minimum(start + sl, split_end)
    return np.where(s < n, np.maximum(end - start, 0), 0)


def workgroup_order(tokens: np.ndarray, cu_count: int) -> np.ndarray:
    """The stage-1 workgroup order (wg_order) for segment sizes tokens[slot, request]:
    heaviest segments first (ties in the grid's own order, request fastest), dealt to
    linear ids in rounds of cu_count, every other full round reversed when its segments
    differ in size, so the segments that share a CU balance (the longest-processing-time
    rule; empty slots go last). Uniform batches keep the grid's order. Only the placement
    changes, never a result. Measured on ragged batches: lognormal lengths B = 64 54.8 ->
    33.9 us, B = 128 112.5 -> 83.6, B = 256 200.7 -> 167.6; config 2 53.2 -> 47.8."""
    slots, rows = tokens.shape
    n = slots * rows
    flat = tokens.reshape(-1)  # index = y * rows + b = the grid's linear id
    rank = np.lexsort((np.arange(n), -flat))
    p = max(int(cu_count), 1)
    r = np.arange(n)
    rnd, j = r // p, r % p
    work = flat[rank]
    nr = -(-n // p)
    pad = np.full(nr * p, work[-1] if n else 0, dtype=work.dtype)
    pad[:n] = work
    varied = pad.reshape(nr, p).max(axis=1) != pad.reshape(nr, p).min(axis=1)
    flip = (rnd % 2 == 1) & ((rnd + 1) * p <= n) & varied[rnd]
    pos = rnd * p + np.where(flip, p - 1 - j, j)
    order = np.empty(n, dtype=np.int32)
    order[pos] = ((rank % rows) << ORDER_SLOT_BITS) | (rank // rows)
    return order


# Worker launches (sid_flash_decode_workers_fwd): stage 1 as one workgroup per CU, each
# computing in turn the (request, slot) items dealt to it (workgroup_order over the workers),
# instead of one workgroup per item. Same items, same arithmetic: the same bits; only the
# placement differs. Measured over 33 batch shapes (B = 1-256, uniform and config-5-like
# lognormal lengths, nondet and batch_invariant plans, 4 KV pools rotated, graph-timed): an
# 8 x 2 grid whose non-empty workgroups number between half the CUs and the CU count runs
# 1.27-1.65x slower than the worker form (e.g. B = 96 lognormal, 241 non-empty 512-token
# segments: 106.4 -> 70.4 us; batch_invariant B = 32 lognormal: 52.0 -> 31.6 us), while below
# that band and above it the two are within a few percent (the worker form 0.94-1.03x of the
# grid), and 4 x 1 / 4 x 2 grids lose with one worker per CU (0.66-0.80x).
WORKERS_VARIANT = 2


def stage1_workers(nonempty: int, variant: int, slots: int, cu_count: int) -> int:
    """Workgroups of a worker launch for a plan with `nonempty` non-empty (request, slot)
    items in `slots` slots per request with stage-1 shape `variant`, or 0 for the grid."""
    if slots > 1 and variant == WORKERS_VARIANT and cu_count < 2 * nonempty <= 2 * cu_count:
        return cu_count
    return 0


def worker_order(tokens: np.ndarray, workers: int) -> np.ndarray:
    """The wg_order of a worker launch: workgroup_order dealt over the workers, with the
    entries of items that hold no tokens flagged ORDER_EMPTY when they all come after every
    worker's non-empty ones (true when the non-empty items fit one round of the dealing,
    which is never reversed), so each worker marks its empty tail in one pass."""
    order = workgroup_order(tokens, workers)
    nonempty = int(np.count_nonzero(tokens))
    if nonempty <= workers:
        order[nonempty:] |= ORDER_EMPTY
    return order


def workspace_slots(max_seq_len: int, max_kv_splits: int, invariant_split_size: int) -> int:
    """Partial slots per request the workspace must hold for any plan."""
    nondet = -(-max_seq_len // SEGMENT_SIZES[-1]) + max_kv_splits
    inv = -(-max_seq_len // invariant_split_size)
    return min(max(nondet, inv), MAX_GRID_SLOTS)


class DecodeAttention:
    """Owns the persistent split workspace (fixed pointers across steps)."""

    def __init__(self, max_batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 max_kv_splits: int, invariant_split_size: int, max_seq_len: int, device: str):
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_kv_splits = max_kv_splits
        self.invariant_split_size = invariant_split_size
        self.invariant_max_splits = -(-max_seq_len // invariant_split_size)
        self.ws_splits = workspace_slots(max_seq_len, max_kv_splits, invariant_split_size)
        self.part_o = torch.empty(max_batch, num_q_heads, self.ws_splits, head_dim,
                                  dtype=torch.float32, device=device)
        self.part_lse = torch.empty(max_batch, num_q_heads, self.ws_splits,
                                    dtype=torch.float32, device=device)
        self.device = torch.device(device)
        self.ext = load_ext()
        self._plan_src = None
        self._plan = None

    def reset_plan(self) -> None:
        """Forget the cached split plan (called at the start of every forward)."""
        self._plan_src = None
        self._plan = None

    def cu_count(self) -> int:
        idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
        return _cu_count(idx)

    def plan(self, seq_lens: torch.Tensor, max_seq_len: int, invariant: bool,
             policy_batch: int | None = None, geometry: tuple | None = None):
        """(num_splits, grid splits, fixed split size, segment size, grid slots).
        num_splits is None: the kernel derives each request's split count from its length
        (ceil(len / fixed split) for fixed splits, min(ceil(len / 32), grid splits) for the
        heuristic), so a step launches no elementwise kernels for it. max_seq_len bounds
        every request's length (host-side, no sync); policy_batch: the real request count when seq_lens has padding rows; geometry: the
        nondet (grid splits, segment size, grid slots) chosen by plan_variant, if any."""
        bs = seq_lens.shape[0] if policy_batch is None else int(policy_batch)
        max_len = max(int(max_seq_len), 1)
        if invariant:
            tile = self.invariant_split_size
            grid = max(1, -(-max_len // tile))
            return None, grid, tile, tile, grid
        if geometry is None:
            geometry = nondet_geometry(bs, max_len, self.num_kv_heads, self.cu_count(),
                                       self.max_kv_splits)
        splits, seg, slots = geometry
        return None, splits, 0, seg, slots

    def forward(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                kv_indptr: torch.Tensor, kv_indices: torch.Tensor, seq_lens: torch.Tensor,
                max_seq_len: int, sm_scale: float, invariant: bool,
                policy_batch: int | None = None, variant: int | None = None,
                geometry: tuple | None = None,
                wg_order: torch.Tensor | None = None, workers: int = 0) -> torch.Tensor:
        """q: [B, HQ, D] bf16 -> o: [B, HQ, D] bf16 (max_seq_len is host-side, no sync).
        policy_batch: real requests among the B rows (the rest are empty padding); variant:
        the stage-1 workgroup shape (stage1_variant; None: INVARIANT_VARIANT in batch_invariant
        mode, else 0); geometry:
        plan_variant's nondet geometry for this batch (None: from the batch size and
        max_seq_len alone); wg_order: workgroup_order of this plan, on the device (None: the
        grid's own order); workers > 0: stage 1 by that many workgroups, each computing the
        items of wg_order dealt to it (then a permutation of every (request, slot) item; see
        worker_order)."""
        if variant is None:
            variant = INVARIANT_VARIANT if invariant else 0
        assert not invariant or variant == INVARIANT_VARIANT, \
            "batch_invariant mode runs one fixed workgroup shape"
        bs = q.shape[0]
        assert bs <= self.part_o.shape[0], "decode batch exceeds workspace"
        # One plan per forward: every layer sees the same seq_lens tensor.
        key = (invariant, max_seq_len, bs, policy_batch, geometry)
        if self._plan_src is seq_lens and self._plan[0] == key:
            plan = self._plan[1]
        else:
            plan = self.plan(seq_lens, max_seq_len, invariant, policy_batch, geometry)
            self._plan_src, self._plan = seq_lens, (key, plan)
        num_splits, grid_splits, fixed, seg, slots = plan
        assert slots <= self.part_o.shape[2], "decode plan exceeds the split workspace"
        o = torch.empty_like(q)
        self.ext.flash_decode_fwd(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                                  grid_splits, fixed, sm_scale, self.part_o, self.part_lse, o,
                                  segment_size=seg, grid_slots=slots, variant=variant,
                                  wg_order=wg_order, workers=workers)
        return o
