"""Request state machine and the KV-length invariant (as sid/engine/request.py).

  WAITING -> RUNNING -> DONE                                   (nondet / batch_invariant)
  WAITING -> RUNNING <-> FINISHED_PENDING_VERIFY -> DONE        (dvr, is_deterministic)

With P prompt tokens and N >= 1 outputs, the KV covers positions 0 .. P+N-2: the newest
sampled token has no KV until it is fed back in the next decode step.
"""

from __future__ import annotations

import enum
from typing import Optional

from sid.config import SamplingParams


class RequestState(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED_PENDING_VERIFY = "finished_pending_verify"
    DONE = "done"


class Request:
    def __init__(self, rid: int, prompt_ids: list, params: SamplingParams, eos_token_ids: tuple):
        self.rid = rid
        self.prompt_ids = list(prompt_ids)
        self.params = params
        self.eos_token_ids = set(eos_token_ids)
        if params.stop_token_ids:
            self.eos_token_ids.update(params.stop_token_ids)
        self.output_ids: list = []
        # host rows of the per-step sampling arrays (params do not change after admission)
        self.samp_f = (float(params.temperature), float(params.top_p))
        self.samp_i = (int(params.top_k) if params.top_k > 0 else -1, int(params.seed))
        self.state = RequestState.WAITING
        self.finished_reason: Optional[str] = None
        self.req_row = -1
        self.verified_len = 0
        self.num_windows = 0
        self.num_rollbacks = 0
        self.tokens_rolled_back = 0
        self.stream_offset = 0
        # bumped whenever a rollback rewrites output_ids: a decode row launched before the
        # bump (overlapped decode) is stale and is discarded
        self.epoch = 0

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_ids)

    @property
    def num_output(self) -> int:
        return len(self.output_ids)

    @property
    def kv_len(self) -> int:
        return 0 if not self.output_ids else self.prompt_len + self.num_output - 1

    def unverified(self) -> int:
        return self.num_output - self.verified_len

    def gate(self, dvr_mode: bool) -> int:
        """How many output tokens the client may see."""
        return self.verified_len if (dvr_mode and self.params.is_deterministic) else self.num_output

    def check_finished(self) -> None:
        """Derive finished_reason from the current outputs (re-derivable after a rollback)."""
        if not self.output_ids:
            self.finished_reason = None
        elif not self.params.ignore_eos and self.output_ids[-1] in self.eos_token_ids:
            self.finished_reason = "stop"
        elif self.num_output >= self.params.max_new_tokens:
            self.finished_reason = "length"
        else:
            self.finished_reason = None

    def assert_invariants(self, dvr_mode: bool) -> None:
        problems = []
        if not 0 <= self.verified_len <= self.num_output:
            problems.append(f"{self.verified_len} verified of {self.num_output} outputs")
        if self.stream_offset > self.gate(dvr_mode):
            problems.append(f"streamed {self.stream_offset} > visible {self.gate(dvr_mode)}")
        assert not problems, f"request {self.rid} inconsistent: " + "; ".join(problems)

    def __repr__(self) -> str:
        fields = {"rid": self.rid, "state": self.state.value, "prompt": self.prompt_len,
                  "out": self.num_output, "verified": self.verified_len,
                  "reason": self.finished_reason}
        return "<Request " + " ".join(f"{k}={v}" for k, v in fields.items()) + ">"
