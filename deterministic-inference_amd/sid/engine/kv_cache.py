"""Paged KV cache, token-granular slots (page_size 1), as sid/engine/kv_cache.py:1-12.

  * per-layer K/V pools, bf16 [num_slots, HKV, D] on the device;
  * request -> token table int32 [max_reqs, max_seq_len]: (row, position) -> slot.
    The authoritative copy lives on the host (`req_to_token`), a device mirror
    (`req_to_token_gpu`) feeds the decode-index kernel; decode steps update both;
  * slot allocator: a LIFO free stack on the host, so alloc/free cost no GPU work and no
    synchronisation. Slot 0 and row 0 are reserved null targets.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from sid.config import EngineConfig, ModelConfig
from sid.kernels.jit import load_ext


class KVCache:
    def __init__(self, cfg: EngineConfig, mcfg: ModelConfig, device: str):
        self.num_slots = cfg.kv_pool_tokens
        self.max_reqs = cfg.max_reqs
        self.max_seq_len = cfg.max_seq_len
        self.device = device
        self.ext = load_ext()
        shape = (self.num_slots, mcfg.num_kv_heads, mcfg.head_dim)
        self.k_pools = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                        for _ in range(mcfg.num_layers)]
        self.v_pools = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                        for _ in range(mcfg.num_layers)]

        self._stack = np.arange(1, self.num_slots, dtype=np.int64)
        self.free_count = self.num_slots - 1

        self.req_to_token = torch.zeros(self.max_reqs, self.max_seq_len, dtype=torch.int32)
        self.req_to_token_gpu = torch.zeros(self.max_reqs, self.max_seq_len, dtype=torch.int32,
                                            device=device)
        self.free_rows = list(range(self.max_reqs - 1, 0, -1))

        self.debug = os.environ.get("SID_DEBUG_ALLOC", "0") == "1"
        self._live: set[int] = set()

    def layer(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k_pools[i], self.v_pools[i]

    # ---- slots ---------------------------------------------------------------------

    def alloc(self, n: int) -> torch.Tensor:
        """n free slots as a host int64 tensor."""
        if n > self.free_count:
            raise RuntimeError(f"KV pool exhausted: need {n}, free {self.free_count}")
        out = torch.from_numpy(self._stack[self.free_count - n:self.free_count].copy())
        self.free_count -= n
        if self.debug:
            ids = out.tolist()
            dup = self._live.intersection(ids)
            assert not dup, f"allocator handed out live slots: {sorted(dup)[:5]}"
            self._live.update(ids)
        return out

    def free(self, slots: torch.Tensor) -> None:
        n = slots.numel()
        if n == 0:
            return
        arr = slots.detach().cpu().numpy().astype(np.int64, copy=False).reshape(-1)
        if self.debug:
            ids = arr.tolist()
            foreign = [s for s in ids if s not in self._live]
            assert not foreign, f"freeing slots not allocated: {foreign[:5]}"
            self._live.difference_update(ids)
        self._stack[self.free_count:self.free_count + n] = arr
        self.free_count += n

    # ---- request rows ----------------------------------------------------------------

    def alloc_row(self) -> int:
        if not self.free_rows:
            raise RuntimeError("req_to_token rows exhausted")
        return self.free_rows.pop()

    def free_row(self, row: int) -> None:
        assert 0 < row < self.max_reqs
        self.free_rows.append(row)

    def write_row(self, row: int, start: int, slots: torch.Tensor) -> None:
        """Set positions start.. of a row to `slots` on the host and the device."""
        vals = slots.to(torch.int32).cpu()
        self.req_to_token[row, start:start + vals.numel()] = vals
        self.req_to_token_gpu[row, start:start + vals.numel()].copy_(vals, non_blocking=False)
