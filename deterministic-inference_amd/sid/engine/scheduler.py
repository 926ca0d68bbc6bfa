"""Admission and batching of requests (the role of sid/engine/scheduler.py).

Policy (the reference's): first come, first served, and a request enters only when the
KV pool can hold the worst case of everything admitted — every active request's
prompt + max_new_tokens plus the newcomer's — so a decode step never runs out of KV and
nothing is ever preempted. Here the reservation is counted in pages: a request's worst case
is pages_for(prompt + max_new_tokens), and what is still owed to the active requests is
their worst case minus the pages their block-table rows already hold.

Prefill batching: newly admitted prompts are packed in arrival order into batches of at
most max_prefill_tokens tokens (a prompt longer than that gets a batch of its own). The
reference prefills every deterministic request of dvr mode alone, since its prefill kernels
depend on the batch; every prefill kernel here is batch-invariant, so deterministic prompts
are packed too unless EngineConfig.dvr_isolated_prefill asks for one-request batches.
"""

from __future__ import annotations

from collections import deque

import numpy as np

from sid.config import EngineConfig, Mode
from sid.engine.request import Request, RequestState


class Scheduler:
    def __init__(self, cfg: EngineConfig, kv):
        self.cfg = cfg
        self.kv = kv
        self.waiting: deque = deque()
        self.active: list = []   # admitted, not yet released (RUNNING or pending verify)

    # ---- KV reservation ------------------------------------------------------------------

    def _worst_pages(self, req: Request) -> int:
        # the KV of P prompt + N outputs covers P + N - 1 positions, N <= max_new_tokens
        return self.kv.pages_for(req.prompt_len + req.params.max_new_tokens)

    def owed_pages(self) -> int:
        """Pages the active requests may still take, at most."""
        if not self.active:
            return 0
        worst = np.fromiter((self._worst_pages(r) for r in self.active), dtype=np.int64,
                            count=len(self.active))
        rows = np.fromiter((r.req_row for r in self.active), dtype=np.int64,
                           count=len(self.active))
        held = np.where(rows > 0, self.kv.held[np.maximum(rows, 0)], 0)
        return int(np.maximum(worst - held, 0).sum())

    def can_admit(self, req: Request) -> bool:
        if len(self.active) >= self.cfg.max_decode_batch or self.kv.free_rows == 0:
            return False
        return self._worst_pages(req) + self.owed_pages() <= self.kv.free_pages

    def admit(self) -> list:
        """Move admissible requests from the head of the queue to the active set; they
        still need their prefill."""
        fresh = []
        while self.waiting and self.can_admit(self.waiting[0]):
            req = self.waiting.popleft()
            req.req_row = self.kv.open_row()
            req.state = RequestState.RUNNING
            self.active.append(req)
            fresh.append(req)
        return fresh

    # ---- batches -------------------------------------------------------------------------

    def prefill_groups(self, new_reqs: list) -> list:
        isolate = self.cfg.mode == Mode.DVR and self.cfg.dvr_isolated_prefill
        alone = [[r] for r in new_reqs if isolate and r.params.is_deterministic]
        packed = [r for r in new_reqs if not (isolate and r.params.is_deterministic)]
        groups = []
        budget = self.cfg.max_prefill_tokens
        for r in packed:
            if groups and groups[-1][1] + r.prompt_len <= budget:
                groups[-1][0].append(r)
                groups[-1][1] += r.prompt_len
            else:
                groups.append([[r], r.prompt_len])
        return alone + [g for g, _ in groups]

    def decode_reqs(self) -> list:
        """Requests that feed a token in the next decode step."""
        return [r for r in self.active
                if r.state is RequestState.RUNNING and r.finished_reason is None]

    # ---- retirement ------------------------------------------------------------------------

    def release_finished(self) -> list:
        """Retire finished requests (in dvr mode a deterministic one only once every
        output is verified: until then it waits as FINISHED_PENDING_VERIFY) and return
        their pages and rows to the cache."""
        dvr = self.cfg.mode == Mode.DVR
        retired, kept = [], []
        for r in self.active:
            if r.finished_reason is None:
                kept.append(r)
                continue
            if dvr and r.params.is_deterministic and r.unverified() > 0:
                r.state = RequestState.FINISHED_PENDING_VERIFY
                kept.append(r)
                continue
            self.kv.close_row(r.req_row)
            r.req_row = -1
            r.state = RequestState.DONE
            retired.append(r)
        self.active = kept
        return retired

    def resume_rolled_back(self) -> None:
        """A verify pass that rolled a pending request back un-finished it: decode again."""
        for r in self.active:
            if r.finished_reason is None and r.state is RequestState.FINISHED_PENDING_VERIFY:
                r.state = RequestState.RUNNING

    def has_work(self) -> bool:
        return bool(self.waiting) or bool(self.active)
