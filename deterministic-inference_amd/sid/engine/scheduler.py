"""FCFS continuous batching with full KV reservation at admission (sid/engine/scheduler.py).

A request is admitted only when the pool covers every active request's worst case
(prompt + max_new_tokens), so decode never runs out of slots. Requests share prefill
batches under max_prefill_tokens. The reference prefills each dvr-mode deterministic
request alone (its token 0 is never re-verified, so its result must not depend on the
batch); every prefill kernel here is batch-invariant, so deterministic requests share
batches too unless EngineConfig.dvr_isolated_prefill asks for one-request groups.
"""

from __future__ import annotations

from collections import deque

from sid.config import EngineConfig, Mode
from sid.engine.request import Request, RequestState


class Scheduler:
    def __init__(self, cfg: EngineConfig, kv):
        self.cfg = cfg
        self.kv = kv
        self.waiting: deque = deque()
        self.active: list = []

    @staticmethod
    def _worst_case_slots(req: Request) -> int:
        return req.prompt_len + req.params.max_new_tokens

    def _future_need(self) -> int:
        return sum(max(0, self._worst_case_slots(r) - r.kv_len) for r in self.active)

    def can_admit(self, req: Request) -> bool:
        if len(self.active) >= self.cfg.max_decode_batch or not self.kv.free_rows:
            return False
        return self.kv.free_count >= self._future_need() + self._worst_case_slots(req)

    def admit(self) -> list:
        admitted = []
        while self.waiting and self.can_admit(self.waiting[0]):
            req = self.waiting.popleft()
            req.req_row = self.kv.alloc_row()
            req.state = RequestState.RUNNING
            self.active.append(req)
            admitted.append(req)
        return admitted

    def prefill_groups(self, new_reqs: list) -> list:
        groups, shared = [], []
        for r in new_reqs:
            if (self.cfg.mode == Mode.DVR and r.params.is_deterministic
                    and self.cfg.dvr_isolated_prefill):
                groups.append([r])
            else:
                shared.append(r)
        cur, cur_tokens = [], 0
        for r in shared:
            if cur and cur_tokens + r.prompt_len > self.cfg.max_prefill_tokens:
                groups.append(cur)
                cur, cur_tokens = [], 0
            cur.append(r)
            cur_tokens += r.prompt_len
        if cur:
            groups.append(cur)
        return groups

    def decode_reqs(self) -> list:
        return [r for r in self.active
                if r.state == RequestState.RUNNING and r.finished_reason is None]

    def release_finished(self) -> list:
        dvr = self.cfg.mode == Mode.DVR
        done = []
        for r in self.active:
            if r.finished_reason is None:
                continue
            if dvr and r.params.is_deterministic and r.unverified() > 0:
                r.state = RequestState.FINISHED_PENDING_VERIFY
                continue
            done.append(r)
        for r in done:
            if r.kv_len > 0:
                self.kv.free(self.kv.req_to_token[r.req_row, :r.kv_len])
            self.kv.free_row(r.req_row)
            r.req_row = -1
            r.state = RequestState.DONE
            self.active.remove(r)
        return done

    def resume_rolled_back(self) -> None:
        for r in self.active:
            if r.state == RequestState.FINISHED_PENDING_VERIFY and r.finished_reason is None:
                r.state = RequestState.RUNNING

    def has_work(self) -> bool:
        return bool(self.waiting or self.active)
