"""Decode-verify-rollback (LLM-42 style), as sid/engine/dvr.py.

A verify pass is S sequences x W extend tokens, padded with dummy sequences: S = G (the
reference's fixed shape) or, with EngineConfig.dvr_verify_buckets, the next power of two
>= the ready sequences (at most G). Every kernel of the pass makes each row depend only on
its own sequence (batch-invariant GEMMs and extend attention), so the verifier's tokens are
a function of the request's history alone, whatever S is.

For a real request with prompt length P, verified_len v >= 1 and u = min(unverified, W)
window tokens t[0..u-1] = output_ids[v:v+u]:
  input row  = [output_ids[v-1], t[0], ..., t[u-2]] + [DUMMY] * (W - u)
  positions  = P+v-1 .. P+v+u-2, padding rows repeat the last real position
  prefix     = KV positions 0 .. P+v-2
  out_slots  = the slots decode already wrote for P+v-1 .. P+v+u-2 (overwritten in
               place), then scratch slots for the padding rows
  prediction j is compared with t[j]; its sample position is P+v+j.
At the first mismatch j the request keeps v+j tokens plus the verifier's token (at least
one token of progress per pass) and frees the KV of everything after it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from sid.config import DUMMY_TOKEN_ID, EngineConfig
from sid.engine.batch import ForwardBatch, ForwardMode
from sid.engine.request import Request


def _bucket(n: int) -> int:
    """Power-of-two bound (>= 512) of the longest verify sequence: the verify pass is
    replayed as a graph per bucket, whose attention grid covers every sequence up to it."""
    b = 512
    while b < n:
        b *= 2
    return b


def _pow2_at_least(n: int, cap: int) -> int:
    b = 1
    while b < n:
        b *= 2
    return min(b, cap)


class DummyPool:
    """Scratch KV slots: G*W for dummy sequences, G*(W-1) for window padding."""

    def __init__(self, kv, group_size: int, window_size: int):
        self.dummy_slots = kv.alloc(group_size * window_size)
        self.padding_slots = kv.alloc(group_size * (window_size - 1))
        self.window_size = window_size


@dataclass
class VerifyMeta:
    reqs: list
    window_lens: list
    windows: list


class Verifier:
    def __init__(self, cfg: EngineConfig, runner, kv):
        self.cfg = cfg
        self.runner = runner
        self.kv = kv
        self.W = cfg.dvr_window_size
        self.G = cfg.dvr_group_size
        self.pool = DummyPool(kv, self.G, self.W)
        buf = runner.verify_buffers
        gw = self.G * self.W
        self.device = buf["qo_indptr"].device
        buf["qo_indptr"].copy_(torch.arange(0, gw + 1, self.W, dtype=torch.int32))
        self._sample_indices = torch.arange(gw, dtype=torch.int64, device=self.device)

    @staticmethod
    def ready(req: Request, window_size: int) -> bool:
        if not req.params.is_deterministic or req.unverified() <= 0:
            return False
        return req.unverified() >= window_size or req.finished_reason is not None

    def collect_ready(self, reqs: list) -> list:
        """Ready requests in rid order, in groups of at most G; nothing while fewer than
        dvr_min_verify are ready, unless one of them must be verified now (it finished
        decoding, so only verification can release it, or it holds 2 W unverified tokens)."""
        ready = sorted((r for r in reqs if self.ready(r, self.W)), key=lambda r: r.rid)
        if len(ready) < self.cfg.dvr_min_verify and not any(
                r.finished_reason is not None or r.unverified() >= 2 * self.W for r in ready):
            return []
        return [ready[i:i + self.G] for i in range(0, len(ready), self.G)]

    def build_verify_batch(self, reqs: list) -> tuple:
        assert 1 <= len(reqs) <= self.G
        W, G, kv = self.W, self.G, self.kv
        buf = self.runner.verify_buffers
        ids, positions, spos = [], [], []
        out_slots, kv_lens, kv_chunks = [], [], []
        temps, top_ks, top_ps, seeds = [], [], [], []
        window_lens, windows = [], []
        pad_used = 0

        for r in reqs:
            p, v = r.prompt_len, r.verified_len
            assert v >= 1, f"req {r.rid} entered verify with verified_len 0"
            u = min(r.unverified(), W)
            assert u >= 1
            window = r.output_ids[v:v + u]
            window_lens.append(u)
            windows.append(window)

            ids.extend([r.output_ids[v - 1]] + window[:-1] + [DUMMY_TOKEN_ID] * (W - u))
            positions.extend(range(p + v - 1, p + v - 1 + u))
            positions.extend([p + v + u - 2] * (W - u))
            spos.extend(range(p + v, p + v + W))

            prefix_len = p + v - 1
            end = prefix_len + u
            assert r.kv_len >= end, (
                f"req {r.rid}: window needs KV through position {end - 1}, only {r.kv_len} valid")
            real = kv.req_to_token[r.req_row, prefix_len:end].to(torch.int64)
            pad = W - u
            if pad:
                slots = torch.cat([real, self.pool.padding_slots[pad_used:pad_used + pad]])
                pad_used += pad
            else:
                slots = real
            out_slots.append(slots)
            kv_lens.append(prefix_len + W)
            kv_chunks.append(torch.cat([kv.req_to_token[r.req_row, :prefix_len].to(torch.int32),
                                        slots.to(torch.int32)]))
            temps.extend([r.params.temperature] * W)
            top_ks.extend([r.params.top_k if r.params.top_k > 0 else -1] * W)
            top_ps.extend([r.params.top_p] * W)
            seeds.extend([r.params.seed] * W)

        # Sequences in this pass: G (the reference's fixed shape) or, with bucketed shapes,
        # the next power of two >= len(reqs); dummy sequences fill the rest.
        n_pad = _pow2_at_least(len(reqs), G) if self.cfg.dvr_verify_buckets else G
        rows = n_pad * W
        for d in range(len(reqs), n_pad):
            dummy = self.pool.dummy_slots[d * W:(d + 1) * W]
            ids.extend([DUMMY_TOKEN_ID] * W)
            positions.extend(range(W))
            spos.extend(range(1, W + 1))
            out_slots.append(dummy)
            kv_lens.append(W)
            kv_chunks.append(dummy.to(torch.int32))
            temps.extend([0.0] * W)
            top_ks.extend([-1] * W)
            top_ps.extend([1.0] * W)
            seeds.extend([0] * W)

        v = {k: t[:rows] for k, t in buf.items()
             if k in ("input_ids", "positions", "out_slots", "sample_positions", "temperatures",
                      "top_ks", "top_ps", "seeds")}
        v["input_ids"].copy_(torch.tensor(ids, dtype=torch.int64))
        v["positions"].copy_(torch.tensor(positions, dtype=torch.int64))
        v["out_slots"].copy_(torch.cat(out_slots).to(torch.int64))
        v["sample_positions"].copy_(torch.tensor(spos, dtype=torch.int64))
        v["temperatures"].copy_(torch.tensor(temps, dtype=torch.float32))
        v["top_ks"].copy_(torch.tensor(top_ks, dtype=torch.int64))
        v["top_ps"].copy_(torch.tensor(top_ps, dtype=torch.float32))
        v["seeds"].copy_(torch.tensor(seeds, dtype=torch.int64))
        total_kv = sum(kv_lens)
        buf["kv_indices"][:total_kv].copy_(torch.cat(kv_chunks))
        indptr = torch.zeros(n_pad + 1, dtype=torch.int64)
        indptr[1:] = torch.cumsum(torch.tensor(kv_lens, dtype=torch.int64), dim=0)
        kv_indptr = buf["kv_indptr"][:n_pad + 1]
        kv_indptr.copy_(indptr.to(torch.int32))

        fb = ForwardBatch(
            mode=ForwardMode.VERIFY,
            input_ids=v["input_ids"], positions=v["positions"], out_slots=v["out_slots"],
            qo_indptr=buf["qo_indptr"][:n_pad + 1], kv_indptr=kv_indptr,
            kv_indices=buf["kv_indices"][:total_kv], max_extend_len=W,
            max_kv_len=_bucket(max(kv_lens)),
            sample_indices=self._sample_indices[:rows], sample_positions=v["sample_positions"],
            temperatures=v["temperatures"], top_ks=v["top_ks"], top_ps=v["top_ps"],
            seeds=v["seeds"], invariant=True, all_greedy=all(t == 0 for t in temps),
        )
        return fb, VerifyMeta(reqs=list(reqs), window_lens=window_lens, windows=windows)

    def compare_and_rollback(self, meta: VerifyMeta, verify_tokens: torch.Tensor) -> None:
        W = self.W
        tokens = verify_tokens.tolist()
        for i, r in enumerate(meta.reqs):
            u = meta.window_lens[i]
            window = meta.windows[i]
            got = tokens[i * W:i * W + u]
            j = next((idx for idx in range(u) if got[idx] != window[idx]), u)
            r.num_windows += 1
            v = r.verified_len
            if j < u:
                old_len = r.num_output
                r.output_ids = r.output_ids[:v + j] + [got[j]]
                r.verified_len = v + j + 1
                r.num_rollbacks += 1
                r.epoch += 1
                r.tokens_rolled_back += old_len - (v + j)
                start = r.prompt_len + r.verified_len - 1
                end = r.prompt_len + old_len - 1
                if end > start:
                    self.kv.free(self.kv.req_to_token[r.req_row, start:end])
                r.finished_reason = None
                r.check_finished()
            else:
                r.verified_len = v + u
            r.assert_invariants(dvr_mode=True)
            assert r.kv_len == r.prompt_len + r.num_output - 1
