"""Integer / byte oracles of the paged KV cache (numpy, bit-exact).

reshape_and_cache_ref   restates sid/csrc/flash_decode.cu:275-296 (+ the -1 skip at :285):
                        k_cache[slot[t]] = k[t]. Pinned by the reference's own tests
                        tests/test_04_reshape_and_cache.py:8-67 (roundtrip, untouched slots
                        stay zero, overwrite, negative slot skipped), restated in
                        tests/test_oracle.py.
block_table_to_indices  expands a page_size-16 block table into token slots,
                        slot(pos) = table[pos // 16] * 16 + pos % 16 (the BASELINE config's
                        page layout over the reference's token-granular pool,
                        sid/engine/kv_cache.py:1-12). Pinned by a brute-force loop.
decode_indices_ref      restates build_decode_batch's kv_indptr / kv_indices construction,
                        sid/engine/batch.py:110-154, over block tables: request b's keys are
                        block_table_to_indices of its table row. page_size 1 is the
                        reference's request -> token table (sid/engine/kv_cache.py:45-47).
                        Pinned by a brute-force loop and by the page_size 1 special case.
"""

from __future__ import annotations

import numpy as np


def reshape_and_cache_ref(k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                          slot_mapping: np.ndarray) -> None:
    """In place on numpy arrays (any dtype; bf16 tensors can be viewed as int16)."""
    n = k_cache.shape[0]
    for t, s in enumerate(slot_mapping.tolist()):
        if 0 <= s < n:
            k_cache[s] = k[t]
            v_cache[s] = v[t]


def block_table_to_indices(block_table: np.ndarray, seq_len: int, page_size: int = 16) -> np.ndarray:
    pos = np.arange(seq_len, dtype=np.int64)
    return (block_table[pos // page_size].astype(np.int64) * page_size + pos % page_size).astype(np.int32)


def decode_indices_ref(block_tables: np.ndarray, rows: list[int], seq_lens: list[int],
                       page_size: int = 1):
    """-> (kv_indptr int32 [B+1], kv_indices int32 [sum]) for requests on block-table rows."""
    indptr = np.zeros(len(rows) + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(seq_lens)
    idx = np.concatenate([block_table_to_indices(block_tables[r], L, page_size)
                          for r, L in zip(rows, seq_lens)]) if rows else np.zeros(0, np.int32)
    return indptr.astype(np.int32), idx.astype(np.int32)
