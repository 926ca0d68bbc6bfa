"""ForwardBatch and the prefill / decode batch builders (sid/engine/batch.py).

sample_pos is the absolute position of the token being generated, on every path:
prefill of P tokens generates position P; a decode step feeding output_ids[N-1] (at
position P+N-1) generates P+N; verify row j of a window starting at verified_len v
generates P+v+j. (A mismatch here would make every verify window fail at index 0.)

Host work per decode step is O(B) Python plus one host->device copy (graph-static
buffers; three without them); the kv_indices of the whole batch are built on the device
from the requests' block tables by one kernel.
"""

from __future__ import annotations

import enum
import itertools
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from sid.config import DUMMY_TOKEN_ID
from sid.engine.request import Request
from sid.kernels.jit import load_ext


class ForwardMode(enum.Enum):
    PREFILL = "prefill"
    DECODE = "decode"
    VERIFY = "verify"


@dataclass
class ForwardBatch:
    mode: ForwardMode
    input_ids: torch.Tensor       # int64 [T]
    positions: torch.Tensor       # int64 [T]
    out_slots: torch.Tensor       # int64 [T] (KV write targets; < 0 skips)
    kv_indptr: Optional[torch.Tensor] = None   # int32 [B+1], full sequence (prefix + new)
    kv_indices: Optional[torch.Tensor] = None  # int32
    seq_lens: Optional[torch.Tensor] = None    # int32 [B] (decode)
    max_seq_len: int = 0                        # host-side max(seq_lens)
    qo_indptr: Optional[torch.Tensor] = None   # int32 [B+1] (extend paths)
    max_extend_len: int = 0
    max_kv_len: int = 0                         # host-side bound of every kv length (extend)
    sample_indices: Optional[torch.Tensor] = None    # int64 [R]; None = every row
    sample_positions: Optional[torch.Tensor] = None  # int64 [R]
    temperatures: Optional[torch.Tensor] = None      # fp32 [R]
    top_ks: Optional[torch.Tensor] = None            # int64 [R]
    top_ps: Optional[torch.Tensor] = None            # fp32 [R]
    seeds: Optional[torch.Tensor] = None             # int64 [R]
    invariant: bool = False
    all_greedy: Optional[bool] = None  # host-known: every row has temperature 0
    untruncated: Optional[bool] = None  # host-known: no row has a top-k / top-p limit
    # softmax-sum grouping of the lm_head-fused sampler (linear_sample's `tiles`): None = by
    # row count; True / False = fixed, for tokens that must not depend on the batch size
    sample_tiles: Optional[bool] = None
    graph_key: Optional[tuple] = None  # set when the inputs live in graph-static buffers
    real_rows: Optional[int] = None    # rows of real requests when padded (decode graphs)
    # decode batches in the graph-static buffers: build_paged_decode_indices arguments, run at the
    # start of the forward (inside the graph) instead of by the builder
    index_build: Optional[tuple] = None
    new_slots_host: Optional[np.ndarray] = None  # decode: the KV slot each row writes
    seq_lens_host: Optional[np.ndarray] = None  # decode: kv length of each real row
    decode_variant: int = 0  # decode: stage-1 workgroup shape of the attention kernel
    decode_geometry: Optional[tuple] = None  # decode, nondet: plan_variant's attention geometry
    decode_wg_order: Optional[torch.Tensor] = None  # decode: the attention's workgroup order
    decode_workers: int = 0  # decode: workgroups of a worker launch of the attention (0: grid)

    def build_indices(self) -> None:
        """Enqueue the deferred kv_indices build (a no-op when the builder already ran it).
        The forward calls this first; a caller that reads kv_indices without a forward
        calls it itself."""
        if self.index_build is not None:
            load_ext().build_paged_decode_indices(*self.index_build)


class DecodeStatic:
    """Fixed-address device buffers for decode batches of up to max_bs requests, shared by
    every captured decode graph (replays are ordered on one stream). All per-step inputs
    live in one pinned host block and one device block, so a step is one asynchronous
    host->device copy; the host block is reused only after the event of its previous copy
    has completed."""

    def __init__(self, max_bs: int, kv_capacity: int, device, max_slots: int = 1):
        self.max_bs = max_bs
        n64, n32, nf = 8 * max_bs, 2 * max_bs + 1, 2 * max_bs
        o32 = 8 * n64
        of = o32 + 4 * (n32 + (n32 & 1))  # keep the fp32 block 8-byte aligned
        nbytes = of + 4 * nf
        self.host = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True)
        self.dev = torch.zeros(nbytes, dtype=torch.uint8, device=device)

        def views(buf):
            return (buf[:o32].view(torch.int64).view(8, max_bs),
                    buf[o32:o32 + 4 * n32].view(torch.int32),
                    buf[of:].view(torch.float32).view(2, max_bs))

        self.i64, self.i32, self.f32 = views(self.dev)
        self.h64, self.h32, self.hf32 = (v.numpy() for v in views(self.host))
        self.kv_indices = torch.zeros(kv_capacity, dtype=torch.int32, device=device)
        self.copied = torch.cuda.Event()
        self.copied.record()
        # the attention's workgroup order (known once the step's plan is), its own copy
        self.order_host = torch.zeros(max_bs * max_slots, dtype=torch.int32, pin_memory=True)
        self.order_dev = torch.zeros(max_bs * max_slots, dtype=torch.int32, device=device)
        self.order_copied = torch.cuda.Event()
        self.order_copied.record()

    def set_order(self, order: np.ndarray) -> torch.Tensor:
        """Queue the copy of a step's workgroup order; returns its fixed-address device view."""
        n = order.size
        self.order_copied.synchronize()  # the pinned block is free once its last copy ran
        self.order_host.numpy()[:n] = order
        dst = self.order_dev[:n]
        dst.copy_(self.order_host[:n], non_blocking=True)
        self.order_copied.record()
        return dst


def _sampling_host(reqs, repeat: int = 1):
    """(temperatures, top_ks, top_ps, seeds) of the requests, each repeated `repeat` times.
    (One flat fromiter per dtype: half the host time of building arrays from the tuples.)"""
    n = len(reqs)
    f = np.fromiter(itertools.chain.from_iterable(r.samp_f for r in reqs), dtype=np.float32,
                    count=2 * n).reshape(-1, 2)
    i = np.fromiter(itertools.chain.from_iterable(r.samp_i for r in reqs), dtype=np.int64,
                    count=2 * n).reshape(-1, 2)
    if repeat != 1:
        f = np.repeat(f, repeat, axis=0)
        i = np.repeat(i, repeat, axis=0)
    return f[:, 0], i[:, 0], f[:, 1], i[:, 1]


def _untruncated(top_ks: np.ndarray, top_ps: np.ndarray) -> bool:
    """No row limits its draw (top_k <= 0 and top_p >= 1 everywhere)."""
    return bool((np.asarray(top_ks) <= 0).all() and (np.asarray(top_ps) >= 1.0).all())


def _to_device(arrays: list, dtype, device) -> list:
    """One host->device copy for several same-dtype 1-D arrays; returns device views."""
    sizes = [int(a.size) for a in arrays]
    host = torch.from_numpy(np.concatenate([np.asarray(a, dtype=dtype) for a in arrays]))
    dev = host.to(device)
    out, off = [], 0
    for n in sizes:
        out.append(dev[off:off + n])
        off += n
    return out


def build_prefill_batch(reqs: list, kv, device: str, invariant: bool) -> ForwardBatch:
    """Takes pages for every prompt (block tables copied to the device); extend attention
    with prefix 0."""
    ids, pos, slots, qo = [], [], [], [0]
    for r in reqs:
        p = r.prompt_len
        kv.grow(r.req_row, p)
        ids.append(np.asarray(r.prompt_ids, dtype=np.int64))
        pos.append(np.arange(p, dtype=np.int64))
        slots.append(kv.slot_range(r.req_row, 0, p))
        qo.append(qo[-1] + p)
    kv.sync_rows([r.req_row for r in reqs])
    temps, top_ks, top_ps, seeds = _sampling_host(reqs)
    qo_np = np.asarray(qo, dtype=np.int64)
    i64 = _to_device([np.concatenate(ids), np.concatenate(pos), np.concatenate(slots),
                      qo_np[1:] - 1, np.asarray([r.prompt_len for r in reqs]), top_ks, seeds],
                     np.int64, device)
    i32 = _to_device([qo_np, np.concatenate(slots)], np.int32, device)
    f32 = _to_device([temps, top_ps], np.float32, device)
    return ForwardBatch(
        mode=ForwardMode.PREFILL, input_ids=i64[0], positions=i64[1], out_slots=i64[2],
        qo_indptr=i32[0], kv_indptr=i32[0], kv_indices=i32[1],
        max_extend_len=max(r.prompt_len for r in reqs),
        max_kv_len=max(r.prompt_len for r in reqs),
        sample_indices=i64[3], sample_positions=i64[4],
        temperatures=f32[0], top_ks=i64[5], top_ps=f32[1], seeds=i64[6],
        invariant=invariant, all_greedy=bool((temps == 0).all()),
        untruncated=_untruncated(top_ks, top_ps),
    )


def gather_prev_tokens(static: DecodeStatic, prev_rows: np.ndarray,
                       prev_tokens: torch.Tensor) -> None:
    """Input ids of a batch built with prev_rows: ids[i] = prev_tokens[prev_rows[i]] where
    prev_rows[i] >= 0, on the stream after the batch's host->device copy (so the in-flight
    step that produces prev_tokens has finished when it runs)."""
    bs = len(prev_rows)
    rows, ids = static.i64[7, :bs], static.i64[0, :bs]
    if (prev_rows >= 0).all():
        torch.index_select(prev_tokens, 0, rows, out=ids)
    else:
        got = torch.index_select(prev_tokens, 0, rows.clamp(min=0))
        ids.copy_(torch.where(rows >= 0, got, ids))


def batch_bucket(bs: int, max_bs: int) -> int:
    """Padded decode batch size of a graph: 1, 2, 4, 8, then steps of 8 up to 64, of 16 up
    to 128, of 32 beyond (at most max_bs). Padding rows are empty requests."""
    if bs <= 8:
        b = 1
        while b < bs:
            b *= 2
    else:
        step = 8 if bs <= 64 else 16 if bs <= 128 else 32
        b = -(-bs // step) * step
    return max(bs, min(b, max_bs))


def build_decode_batch(reqs: list, kv, device: str, invariant: bool,
                       static: Optional[DecodeStatic] = None,
                       pad_to: Optional[int] = None,
                       prev_rows: Optional[np.ndarray] = None) -> ForwardBatch:
    """One new token per request; attention covers the full sequence including the
    position being written now. With `static`, the batch lives in its fixed buffers and
    may be padded to `pad_to` rows: padding rows are empty requests (sequence length 0,
    table row -1, KV slot -1, greedy), whose attention output is zero and whose tokens the
    caller ignores; real rows' results do not depend on them.

    prev_rows (static only): prev_rows[i] >= 0 means request i has one more token than its
    output_ids hold, sampled by a step still in flight at that step's row prev_rows[i]; the
    batch feeds it (position one further on) and the caller gathers it on the device
    (`gather_prev_tokens`) after this returns. prev_rows[i] < 0: the newest token is in
    output_ids, as without prev_rows."""
    bs = len(reqs)
    if not all(r.output_ids for r in reqs):
        bad = next(r for r in reqs if not r.output_ids)
        raise AssertionError(f"req {bad.rid}: decode step before any output token")
    # position of the fed token = kv_len = prompt_len + num_output - 1 (request.py)
    pos = np.fromiter((len(r.prompt_ids) + len(r.output_ids) - 1 for r in reqs),
                      dtype=np.int64, count=bs)
    ids = np.fromiter((r.output_ids[-1] for r in reqs), dtype=np.int64, count=bs)
    if prev_rows is not None:
        assert static is not None, "a pending token needs the graph-static buffers"
        pending = prev_rows >= 0
        pos += pending  # the in-flight token sits one position further on
        ids[pending] = DUMMY_TOKEN_ID  # replaced on the device
    rows = np.fromiter((r.req_row for r in reqs), dtype=np.int64, count=bs)
    new_slots = kv.decode_slots(rows, pos)
    seq_lens = pos + 1
    indptr = np.zeros(bs + 1, dtype=np.int64)
    np.cumsum(seq_lens, out=indptr[1:])
    temps, top_ks, top_ps, seeds = _sampling_host(reqs)
    total = int(indptr[-1])
    index_build = None
    if static is None:
        d_ids, d_pos, d_rows, d_slots, d_spos, d_topk, d_seed = _to_device(
            [ids, pos, rows, new_slots, pos + 1, top_ks, seeds], np.int64, device)
        d_indptr, d_lens = _to_device([indptr, seq_lens], np.int32, device)
        d_temps, d_topp = _to_device([temps, top_ps], np.float32, device)
        kv_indices = torch.empty(total, dtype=torch.int32, device=device)
        load_ext().build_paged_decode_indices(kv.block_tables_gpu, kv.page_size, d_rows, d_slots,
                                              d_indptr, kv_indices)
    else:
        n = bs if pad_to is None else pad_to
        assert bs <= n <= static.max_bs and total <= static.kv_indices.numel()
        mb = static.max_bs
        static.copied.synchronize()
        h64 = static.h64
        pad64 = (DUMMY_TOKEN_ID, 0, -1, -1, 1, -1, 0)  # ids, pos, rows, slots, spos, top_k, seed
        for i, a in enumerate((ids, pos, rows, new_slots, seq_lens, top_ks, seeds)):
            h64[i, :bs] = a
            h64[i, bs:n] = pad64[i]
        if prev_rows is not None:
            h64[7, :bs] = prev_rows
        h32 = static.h32
        h32[:bs + 1] = indptr
        h32[bs + 1:n + 1] = indptr[-1]
        h32[mb + 1:mb + 1 + bs] = seq_lens
        h32[mb + 1 + bs:mb + 1 + n] = 0
        hf = static.hf32
        hf[0, :bs] = temps
        hf[1, :bs] = top_ps
        hf[0, bs:n] = 0.0
        hf[1, bs:n] = 1.0
        static.dev.copy_(static.host, non_blocking=True)
        static.copied.record()
        d_ids, d_pos, d_rows, d_slots, d_spos, d_topk, d_seed = (static.i64[i, :n] for i in range(7))
        d_indptr, d_lens = static.i32[:n + 1], static.i32[mb + 1:mb + 1 + n]
        d_temps, d_topp = static.f32[0, :n], static.f32[1, :n]
        kv_indices = static.kv_indices[:total]
        # Every argument lives at a fixed address, so the index build is part of the
        # forward (and of its captured graph): ModelRunner runs it first.
        index_build = (kv.block_tables_gpu, kv.page_size, d_rows, d_slots, d_indptr, kv_indices)
    return ForwardBatch(
        mode=ForwardMode.DECODE, input_ids=d_ids, positions=d_pos, out_slots=d_slots,
        kv_indptr=d_indptr, kv_indices=kv_indices, seq_lens=d_lens,
        max_seq_len=int(seq_lens.max()) if bs else 0,
        qo_indptr=None, max_extend_len=1,
        sample_indices=None, sample_positions=d_spos,
        temperatures=d_temps, top_ks=d_topk, top_ps=d_topp, seeds=d_seed,
        invariant=invariant, all_greedy=bool((temps == 0).all()),
        untruncated=_untruncated(top_ks, top_ps), real_rows=bs if d_ids.shape[0] != bs else None,
        index_build=index_build, new_slots_host=new_slots, seq_lens_host=seq_lens,
    )
