"""Decode-verify-rollback: the verify pass and its commit rule (the role of sid/engine/dvr.py).

A deterministic request decodes on the fast (batch-dependent) path; every W tokens, or
when it finishes, its unverified tokens are recomputed by a verify pass whose result is a
function of the request's history alone, and the tokens are committed up to the first
disagreement.

A pass is an extend batch of S sequences x W rows. For a real sequence with prompt length
P, verified_len v >= 1 and a window of u = min(unverified, W) tokens output_ids[v:v+u]:
  rows 0 .. u-1   feed output_ids[v-1 .. v+u-2] at positions P+v-1 .. P+v+u-2, and write
                  their K/V over the slots decode wrote for those positions;
  rows u .. W-1   padding: the DUMMY token at the last real position, K/V to scratch slots;
  keys            positions 0 .. P+v-2 (its block table) followed by the W rows' slots;
  row j predicts the token at position P+v+j (its sample position), compared with
  output_ids[v+j].
Dummy sequences (prefix 0, W DUMMY rows at positions 0 .. W-1, all on scratch slots) pad
the pass to S sequences: S = G, the reference's fixed shape, or with
EngineConfig.dvr_verify_buckets the next power of two >= the real sequences (at most G).
Every kernel of the pass makes a row depend only on its own sequence (M-invariant GEMM rows,
extend attention independent of the other sequences), so the verifier's tokens do not
depend on S or on the other sequences.

Commit rule, at the first index j where the verifier disagrees: keep v + j tokens, append
the verifier's token (so a pass always commits at least one token) and give back the KV
pages that only the discarded tokens used; with no disagreement, all u tokens are verified.

The pass is built as arrays (numpy, one row per sequence or per verify row) and copied into
the runner's persistent verify buffers, so its graph replays read fixed addresses.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from sid.config import DUMMY_TOKEN_ID, EngineConfig
from sid.engine.batch import ForwardBatch, ForwardMode
from sid.engine.request import Request


def kv_bucket(n: int) -> int:
    """Power-of-two bound (>= 512) of a pass's longest key list: one verify graph serves
    every pass up to it (its attention grid covers that many keys)."""
    return max(512, 1 << (int(n) - 1).bit_length())


def sequences_in_pass(ready: int, group: int, buckets: bool) -> int:
    if not buckets:
        return group
    return min(group, 1 << (int(ready) - 1).bit_length())


@dataclass
class VerifyMeta:
    reqs: list
    window_lens: list   # u per real sequence
    windows: list       # the tokens each window checks: output_ids[v:v+u]


class Verifier:
    def __init__(self, cfg: EngineConfig, runner, kv):
        self.cfg = cfg
        self.runner = runner
        self.kv = kv
        self.W = W = cfg.dvr_window_size
        self.G = G = cfg.dvr_group_size
        # scratch K/V targets: row j >= 1 of real sequence i pads into pad[i, j - 1]; row j
        # of dummy sequence d writes dummy[d, j]
        scratch = kv.scratch_slots(G * W + G * (W - 1))
        self.dummy_slots = scratch[:G * W].reshape(G, W)
        self.pad_slots = scratch[G * W:].reshape(G, W - 1)
        buf = runner.verify_buffers
        self.device = buf["qo_indptr"].device
        buf["qo_indptr"].copy_(torch.arange(0, G * W + 1, W, dtype=torch.int32))
        self._sample_rows = torch.arange(G * W, dtype=torch.int64, device=self.device)

    # ---- which windows --------------------------------------------------------------------

    def ready(self, req: Request) -> bool:
        """A deterministic request has a window to verify: W unverified tokens, or any
        once it has finished decoding."""
        n = req.unverified()
        return req.params.is_deterministic and n > 0 and (
            n >= self.W or req.finished_reason is not None)

    def collect_ready(self, reqs: list) -> list:
        """Ready requests in rid order, cut into passes of at most G. With
        dvr_min_verify = m, nothing is returned while fewer than m are ready, unless one
        of them cannot wait (it finished decoding, or it has 2 W unverified tokens)."""
        ready = sorted((r for r in reqs if self.ready(r)), key=lambda r: r.rid)
        urgent = any(r.finished_reason is not None or r.unverified() >= 2 * self.W
                     for r in ready)
        if len(ready) < self.cfg.dvr_min_verify and not urgent:
            return []
        return [ready[k:k + self.G] for k in range(0, len(ready), self.G)]

    # ---- the pass ---------------------------------------------------------------------------

    def build_verify_batch(self, reqs: list) -> tuple:
        n, W = len(reqs), self.W
        assert 1 <= n <= self.G, f"{n} sequences for a pass of at most {self.G}"
        S = sequences_in_pass(n, self.G, self.cfg.dvr_verify_buckets)
        j = np.arange(W, dtype=np.int64)

        v = np.array([r.verified_len for r in reqs], dtype=np.int64)
        assert (v >= 1).all(), "a request entered verify before its first token was committed"
        u = np.minimum(np.array([r.unverified() for r in reqs], dtype=np.int64), W)
        assert (u >= 1).all()
        base = np.array([r.prompt_len for r in reqs], dtype=np.int64) + v - 1
        kv_have = np.array([r.kv_len for r in reqs], dtype=np.int64)
        assert (kv_have >= base + u).all(), "a window reaches past the KV decode wrote"

        # per verify row [S, W]
        tokens = np.full((S, W), DUMMY_TOKEN_ID, dtype=np.int64)
        windows = []
        for i, r in enumerate(reqs):
            fed = r.output_ids[v[i] - 1:v[i] - 1 + u[i]]
            tokens[i, :u[i]] = fed
            windows.append(r.output_ids[v[i]:v[i] + u[i]])
        positions = np.empty((S, W), dtype=np.int64)
        positions[:n] = base[:, None] + np.minimum(j[None, :], u[:, None] - 1)
        positions[n:] = j
        sample_pos = np.empty((S, W), dtype=np.int64)
        sample_pos[:n] = base[:, None] + 1 + j
        sample_pos[n:] = j + 1
        slots = np.empty((S, W), dtype=np.int64)
        slots[:n, 1:] = self.pad_slots[:n]
        for i, r in enumerate(reqs):
            slots[i, :u[i]] = self.kv.slot_range(r.req_row, base[i], base[i] + u[i])
        slots[n:] = self.dummy_slots[n:S]

        # keys: each real sequence's prefix, then its W rows' slots; dummies: their rows
        kv_lens = np.full(S, W, dtype=np.int64)
        kv_lens[:n] += base
        chunks = []
        for i, r in enumerate(reqs):
            chunks.append(self.kv.slot_range(r.req_row, 0, base[i]))
            chunks.append(slots[i])
        chunks.extend(slots[n:S])
        kv_indices = np.concatenate(chunks)
        kv_indptr = np.zeros(S + 1, dtype=np.int64)
        np.cumsum(kv_lens, out=kv_indptr[1:])

        # sampling parameters repeat per row; dummy rows are greedy
        temps = np.zeros((S, W), dtype=np.float32)
        top_p = np.ones((S, W), dtype=np.float32)
        top_k = np.full((S, W), -1, dtype=np.int64)
        seeds = np.zeros((S, W), dtype=np.int64)
        for i, r in enumerate(reqs):
            temps[i], top_p[i] = r.samp_f
            top_k[i], seeds[i] = r.samp_i

        rows = S * W
        buf = self.runner.verify_buffers
        dev = {}
        for name, arr in (("input_ids", tokens), ("positions", positions), ("out_slots", slots),
                          ("sample_positions", sample_pos), ("temperatures", temps),
                          ("top_ks", top_k), ("top_ps", top_p), ("seeds", seeds)):
            dst = buf[name][:rows]
            dst.copy_(torch.from_numpy(arr.reshape(-1)).to(dst.dtype))
            dev[name] = dst
        total = int(kv_indptr[-1])
        buf["kv_indices"][:total].copy_(torch.from_numpy(kv_indices.astype(np.int32)))
        buf["kv_indptr"][:S + 1].copy_(torch.from_numpy(kv_indptr.astype(np.int32)))

        fb = ForwardBatch(
            mode=ForwardMode.VERIFY, input_ids=dev["input_ids"], positions=dev["positions"],
            out_slots=dev["out_slots"], qo_indptr=buf["qo_indptr"][:S + 1],
            kv_indptr=buf["kv_indptr"][:S + 1], kv_indices=buf["kv_indices"][:total],
            max_extend_len=W, max_kv_len=kv_bucket(int(kv_lens.max())),
            sample_indices=self._sample_rows[:rows], sample_positions=dev["sample_positions"],
            temperatures=dev["temperatures"], top_ks=dev["top_ks"], top_ps=dev["top_ps"],
            seeds=dev["seeds"], invariant=True, all_greedy=bool((temps == 0).all()),
            untruncated=bool((top_k <= 0).all() and (top_p >= 1.0).all()),
        )
        return fb, VerifyMeta(reqs=list(reqs), window_lens=u.tolist(), windows=windows)

    # ---- commit ----------------------------------------------------------------------------

    def compare_and_rollback(self, meta: VerifyMeta, verify_tokens: torch.Tensor) -> None:
        W = self.W
        got = verify_tokens.reshape(-1)[:len(meta.reqs) * W].view(-1, W).cpu().numpy()
        for i, r in enumerate(meta.reqs):
            u = meta.window_lens[i]
            differ = np.flatnonzero(got[i, :u] != np.asarray(meta.windows[i], dtype=np.int64))
            r.num_windows += 1
            if differ.size == 0:
                r.verified_len += u
            else:
                keep = r.verified_len + int(differ[0])
                r.tokens_rolled_back += r.num_output - keep
                del r.output_ids[keep:]
                r.output_ids.append(int(got[i, differ[0]]))
                r.verified_len = keep + 1
                r.num_rollbacks += 1
                r.epoch += 1
                self.kv.shrink(r.req_row, r.kv_len)
                r.check_finished()
            r.assert_invariants(dvr_mode=True)
            assert r.kv_len == r.prompt_len + r.num_output - 1
