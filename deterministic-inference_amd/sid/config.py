"""Engine, model and sampling configuration (same fields and defaults as sid/config.py).

Modes:
  nondet          fast path only; the decode attention split count follows the batch size,
                  so a request's output depends on its co-tenants.
  dvr             decode-verify-rollback: the nondet fast path plus fixed-shape G x W verify
                  passes that make is_deterministic requests reproducible.
  batch_invariant fixed 256-token attention splits; deterministic by construction.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Optional


class Mode(str, enum.Enum):
    NONDET = "nondet"
    DVR = "dvr"
    BATCH_INVARIANT = "batch_invariant"


# Padding token of verify windows and dummy verify sequences (sid/config.py:26).
DUMMY_TOKEN_ID = 32


@dataclass
class ModelConfig:
    model_path: str = "random:qwen3-0.6b"
    num_layers: int = 28
    hidden_size: int = 1024
    num_q_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    eos_token_ids: tuple = (151645, 151643)

    @property
    def q_size(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim


@dataclass
class EngineConfig:
    """Engine settings (the reference's fields, plus this build's schedule and paging knobs)."""

    # "random:<name>" builds a random-init Qwen3-0.6B-shape model (no download); a directory
    # path loads config.json + safetensors from disk.
    model_path: str = "random:qwen3-0.6b"
    mode: Mode = Mode.DVR
    dtype: str = "bfloat16"

    kv_pool_tokens: int = 256 * 1024
    # KV pages: a request holds whole pages of this many consecutive pool slots (a power of
    # two; 1 = the reference's token-granular pool). Slot numbering, and so every kernel's
    # view of the pool, is the same for any page size.
    kv_page_size: int = 16
    max_reqs: int = 256
    max_seq_len: int = 32768
    max_prompt_len: int = 16384

    max_prefill_tokens: int = 8192
    max_decode_batch: int = 256

    dvr_window_size: int = 32
    # Sequences per verify pass. The reference pads every pass to exactly G = 4 sequences
    # (a fixed shape keeps its kernels' reduction orders fixed). Every verify-path kernel
    # here is batch-invariant, so with dvr_verify_buckets a pass takes up to G ready
    # sequences and is padded only to the next power of two (one graph per size): same
    # tokens, fewer and fuller passes. dvr_verify_buckets=False, dvr_group_size=4 is the
    # reference's schedule.
    dvr_group_size: int = 16
    dvr_verify_buckets: bool = True
    # A verify pass costs about the same for 1 and for 16 sequences (weight reads and
    # per-layer launches dominate), so passes wait until this many windows are ready, unless
    # a ready request has finished decoding or holds 2 W unverified tokens (it keeps
    # decoding meanwhile). Committed tokens do not depend on when a window is verified.
    # 1 = the reference's schedule (verify whatever is ready, every step).
    dvr_min_verify: int = 8
    # Run a step's verify passes on a side stream beside its decode step (graphs only; the
    # verify windows are then taken before the decode appends). False: decode, then verify.
    dvr_overlap_verify: bool = True
    # The reference prefills every is_deterministic request alone (a fixed shape, so its
    # first token is reproducible). Every prefill kernel here is batch-invariant (GEMM rows
    # reduce in an M-independent order, extend attention is bitwise independent of
    # co-batched requests), so a deterministic prompt gets the same bits inside a shared
    # prefill batch and is batched by default; True restores one-request groups.
    dvr_isolated_prefill: bool = False

    max_kv_splits: int = 32
    invariant_split_size: int = 256

    # "cuda" (the reference's name) or "hip": the split-KV decode kernel; "triton" (the
    # reference's name) or "extend": decode through the extend kernel (debugging)
    decode_backend: str = "cuda"
    use_graphs: bool = True  # replay decode / verify forwards as HIP graphs
    # nondet / batch_invariant with graphs: launch decode step N+1 before step N's tokens are
    # read back (N+1 takes them on the device), so the host's per-step work overlaps the GPU.
    # A request that stops on EOS at step N has its row of N+1 discarded. Tokens do not
    # change (batch_invariant: bit for bit); False: one synchronous step at a time.
    overlap_decode: bool = True

    device: str = "cuda"
    seed: int = 0  # random-init weight seed
    num_layers: Optional[int] = None  # override (smaller random models for tests)
    vocab_size: Optional[int] = None

    def __post_init__(self):
        self.mode = Mode(self.mode)
        self.decode_backend = decode_backend_kind(self.decode_backend)
        # Prefill batches (at most max_decode_batch sequences) and verify passes (G x W
        # rows) draw their untruncated rows inside the lm_head with one fixed grouping,
        # which takes up to MAX_SAMPLED_ROWS rows per pass; larger passes would switch those
        # rows to the sampler kernel, whose sums differ at float near-ties.
        if self.max_decode_batch > MAX_SAMPLED_ROWS:
            raise ValueError(f"max_decode_batch {self.max_decode_batch} exceeds "
                             f"{MAX_SAMPLED_ROWS}")
        if self.dvr_group_size * self.dvr_window_size > MAX_SAMPLED_ROWS:
            raise ValueError(f"a verify pass of dvr_group_size x dvr_window_size = "
                             f"{self.dvr_group_size * self.dvr_window_size} rows exceeds "
                             f"{MAX_SAMPLED_ROWS}")


# Rows one lm_head-fused sampling pass takes with 128-column tiles (sid_linear_sample).
MAX_SAMPLED_ROWS = 4096

_DECODE_BACKENDS = {"cuda": "hip", "hip": "hip", "triton": "extend", "extend": "extend"}


def decode_backend_kind(name: str) -> str:
    """'hip' (split-KV decode kernel) or 'extend'; accepts the reference's 'cuda'/'triton'."""
    try:
        return _DECODE_BACKENDS[name]
    except KeyError:
        raise ValueError(f"unknown decode_backend {name!r}: use 'cuda' (or 'hip') for the "
                         "split-KV decode kernel, 'triton' (or 'extend') for the extend "
                         "kernel") from None


@dataclass
class SamplingParams:
    temperature: float = 0.0
    top_k: int = -1
    top_p: float = 1.0
    max_new_tokens: int = 128
    seed: int = 42
    is_deterministic: bool = False
    stop_token_ids: Optional[list] = None
    ignore_eos: bool = False

    def __post_init__(self):
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if not (0.0 < self.top_p <= 1.0):
            raise ValueError("top_p must be in (0, 1]")
        if self.max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")
