"""Paged KV cache: per-layer pools, page allocator and per-request block tables.

Replaces sid/engine/kv_cache.py of the reference, whose pool is token-granular (a GPU free
stack of single slots and an int32 request -> token table [max_reqs, max_seq_len]). Here:

  * pools: per layer, K and V bf16 [num_pages * page_size, HKV, D]. Slot numbering is
    unchanged (slot = page * page_size + offset), so every kernel that takes slots
    (reshape_and_cache, attention through kv_indices) sees the reference's pool format;
  * block tables: int32 [max_reqs, max_pages] page ids per request row. The host copy is
    authoritative; the device mirror feeds the decode-index kernel, which also records the
    page a decode step opens. Prefill writes whole rows to the mirror (`sync_rows`);
  * allocator: whole pages from a host LIFO stack (numpy), so allocation and freeing need
    no GPU work and no synchronisation. A request holds pages 0 .. held-1 of its row;
    shrinking it (a DVR rollback) returns only the pages left empty.

page_size 1 is the reference's token-granular layout; the default 16 is the page layout of
the BASELINE configs (slot(pos) = table[pos // 16] * 16 + pos % 16). Page 0 and row 0 are
reserved, so a stray index lands on memory no request owns.

SID_DEBUG_ALLOC=1 keeps an owner per page and checks every hand-out and return against it.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from sid.config import EngineConfig, ModelConfig
from sid.kernels.jit import load_ext


def _pages(n_tokens, page_size: int):
    """Pages that hold n_tokens positions (works on ints and numpy arrays)."""
    return -(-n_tokens // page_size)


class KVCache:
    def __init__(self, cfg: EngineConfig, mcfg: ModelConfig, device: str):
        ps = int(cfg.kv_page_size)
        if ps < 1 or ps & (ps - 1):
            raise ValueError(f"kv_page_size must be a power of two, got {ps}")
        self.page_size = ps
        self.num_pages = cfg.kv_pool_tokens // ps
        if self.num_pages < 2:
            raise ValueError("the KV pool needs at least two pages (page 0 is reserved)")
        self.num_slots = self.num_pages * ps
        self.max_reqs = cfg.max_reqs
        self.max_seq_len = cfg.max_seq_len
        self.max_pages = _pages(cfg.max_seq_len, ps) + 1
        self.device = device
        self.ext = load_ext()
        shape = (self.num_slots, mcfg.num_kv_heads, mcfg.head_dim)
        self.k_pools = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                        for _ in range(mcfg.num_layers)]
        self.v_pools = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                        for _ in range(mcfg.num_layers)]

        # free pages: stack[:top] (the top of the stack is handed out first)
        self._stack = np.arange(self.num_pages - 1, 0, -1, dtype=np.int32)
        self._top = self.num_pages - 1
        self.tables = np.zeros((self.max_reqs, self.max_pages), dtype=np.int32)
        self.held = np.zeros(self.max_reqs, dtype=np.int64)
        self.block_tables_gpu = torch.zeros(self.max_reqs, self.max_pages, dtype=torch.int32,
                                            device=device)
        self._rows = list(range(self.max_reqs - 1, 0, -1))
        self._owner = (np.full(self.num_pages, -1, dtype=np.int64)
                       if os.environ.get("SID_DEBUG_ALLOC", "0") == "1" else None)

    # ---- pools -----------------------------------------------------------------------

    def layer(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k_pools[i], self.v_pools[i]

    @property
    def free_pages(self) -> int:
        return self._top

    @property
    def free_count(self) -> int:
        """Free capacity in token slots (whole free pages)."""
        return self._top * self.page_size

    @property
    def free_rows(self) -> int:
        return len(self._rows)

    def pages_for(self, n_tokens: int) -> int:
        return _pages(int(n_tokens), self.page_size)

    def scatter_free_pages(self, seed: int) -> None:
        """Shuffle the free-page stack: later allocations land on random pages, as in a
        pool that has served many requests (benchmarks; no effect on results)."""
        rng = np.random.default_rng(seed)
        self._stack[:self._top] = rng.permutation(self._stack[:self._top])

    # ---- page stack --------------------------------------------------------------------

    def _take(self, n: int, owner) -> np.ndarray:
        """n pages off the stack; owner: the row (or one row per page) they go to."""
        if n > self._top:
            raise RuntimeError(f"KV pool out of pages: {n} wanted, {self._top} free "
                               f"(page_size {self.page_size})")
        self._top -= n
        got = self._stack[self._top:self._top + n][::-1].copy()
        if self._owner is not None:
            busy = got[self._owner[got] >= 0]
            assert busy.size == 0, f"page(s) {busy[:4].tolist()} handed out while owned"
            self._owner[got] = owner
        return got

    def _give_back(self, pages: np.ndarray, row: int) -> None:
        if pages.size == 0:
            return
        if self._owner is not None:
            wrong = pages[self._owner[pages] != row]
            assert wrong.size == 0, f"row {row} returned page(s) {wrong[:4].tolist()} it does not own"
            self._owner[pages] = -1
        self._stack[self._top:self._top + pages.size] = pages[::-1]
        self._top += pages.size

    # ---- request rows --------------------------------------------------------------------

    def open_row(self) -> int:
        if not self._rows:
            raise RuntimeError("no free block-table row (raise max_reqs)")
        row = self._rows.pop()
        self.held[row] = 0
        return row

    def close_row(self, row: int) -> None:
        """Return every page of the row, then the row."""
        assert 0 < row < self.max_reqs
        self.shrink(row, 0)
        self._rows.append(row)

    def grow(self, row: int, n_tokens: int) -> None:
        """Hold enough pages for positions 0 .. n_tokens-1 (host table only)."""
        need = self.pages_for(n_tokens) - int(self.held[row])
        if need > 0:
            h = int(self.held[row])
            if h + need > self.max_pages:
                raise RuntimeError(f"row {row}: {n_tokens} tokens exceed max_seq_len")
            self.tables[row, h:h + need] = self._take(need, row)
            self.held[row] = h + need

    def shrink(self, row: int, n_tokens: int) -> None:
        """Keep only the pages that positions 0 .. n_tokens-1 use."""
        keep = self.pages_for(n_tokens)
        h = int(self.held[row])
        if h > keep:
            self._give_back(self.tables[row, keep:h].copy(), row)
            self.held[row] = keep

    def scratch_slots(self, n: int) -> np.ndarray:
        """n slots on pages no request will ever own (verify padding rows and dummy
        sequences write their K/V there). Held until the cache is destroyed."""
        pages = self._take(self.pages_for(n), 0)
        ps = self.page_size
        return (pages.astype(np.int64)[:, None] * ps + np.arange(ps)).reshape(-1)[:n]

    def slot_range(self, row: int, start: int, end: int) -> np.ndarray:
        """Pool slots of positions start .. end-1 of a row (int64)."""
        pos = np.arange(start, end, dtype=np.int64)
        assert end <= int(self.held[row]) * self.page_size, "positions beyond the row's pages"
        return self.tables[row, pos // self.page_size].astype(np.int64) * self.page_size \
            + pos % self.page_size

    def sync_rows(self, rows) -> None:
        """Copy the host tables of `rows` to the device mirror (after a prefill)."""
        idx = np.asarray(rows, dtype=np.int64)
        if idx.size == 0:
            return
        width = int(self.held[idx].max())
        if width == 0:
            return
        src = torch.from_numpy(self.tables[idx, :width]).to(self.device)
        self.block_tables_gpu[torch.from_numpy(idx).to(self.device), :width] = src

    # ---- decode ----------------------------------------------------------------------------

    def decode_slots(self, rows: np.ndarray, positions: np.ndarray) -> np.ndarray:
        """Slots for one new token per row at `positions` (int64 arrays). A row whose
        position is the first of a page it does not hold yet gets that page (host table);
        the decode-index kernel records it in the device mirror."""
        ps = self.page_size
        page_idx = positions // ps
        opens = page_idx >= self.held[rows]
        if opens.any():
            r, pi = rows[opens], page_idx[opens]
            assert (pi == self.held[r]).all(), "a decode step skipped a page"
            assert np.unique(r).size == r.size, "two new tokens for one row in a step"
            self.tables[r, pi] = self._take(r.size, r)
            self.held[r] = pi + 1
        return self.tables[rows, page_idx].astype(np.int64) * ps + positions % ps
