"""ModelRunner: model, KV cache, decode workspace, verify buffers (sid/engine/model_runner.py).

Numerics: every GEMM, norm and attention kernel on the path is this library's own HIP
code with fixed reduction orders, so no library autotuning or workspace setting can
change bits between runs of the same shape.
"""

from __future__ import annotations

import gc
import logging
import weakref
from collections import OrderedDict

import numpy as np
import torch

from sid.config import EngineConfig, Mode, ModelConfig
from sid.engine.batch import (DecodeStatic, ForwardBatch, ForwardMode, batch_bucket,
                              build_decode_batch, gather_prev_tokens)
from sid.engine.kv_cache import KVCache
from sid.engine.sampler import sample as _sample
from sid.kernels.decode_attention import (INVARIANT_VARIANT, DecodeAttention, length_bucket,
                                          plan_variant, segment_tokens, stage1_workers,
                                          worker_order, workgroup_order)
from sid.kernels.matmul_persistent import linear_sample_supported
from sid.model.loader import build_model_config, load_weights, random_weights
from sid.model.qwen3 import Qwen3Model

logger = logging.getLogger(__name__)


def pin_numerics() -> None:
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False


class ModelRunner:
    def __init__(self, cfg: EngineConfig, device: str = "cuda", weights: dict | None = None):
        pin_numerics()
        self.cfg = cfg
        self.device = device
        self.mcfg: ModelConfig
        self.mcfg, self.model_dir = build_model_config(cfg.model_path, cfg.num_layers,
                                                       cfg.vocab_size)
        logger.info("model %s: %d layers, %d/%d heads, head_dim %d", cfg.model_path,
                    self.mcfg.num_layers, self.mcfg.num_q_heads, self.mcfg.num_kv_heads,
                    self.mcfg.head_dim)
        if weights is None:
            if self.model_dir is None:
                weights = random_weights(self.mcfg, device, seed=cfg.seed)
            else:
                weights = load_weights(self.model_dir, self.mcfg, device)
        self.model = Qwen3Model(self.mcfg, weights, device)
        self.model.set_batch_invariant(cfg.mode == Mode.BATCH_INVARIANT)
        self.kv_cache = KVCache(cfg, self.mcfg, device)
        self.decode_attn = DecodeAttention(
            max_batch=cfg.max_decode_batch, num_q_heads=self.mcfg.num_q_heads,
            num_kv_heads=self.mcfg.num_kv_heads, head_dim=self.mcfg.head_dim,
            max_kv_splits=cfg.max_kv_splits, invariant_split_size=cfg.invariant_split_size,
            max_seq_len=cfg.max_seq_len, device=device)
        self.verify_buffers = self._alloc_verify_buffers(cfg, device) \
            if cfg.mode == Mode.DVR else None
        self.graphs = GraphCache(self) if cfg.use_graphs else None

    @staticmethod
    def _alloc_verify_buffers(cfg: EngineConfig, device: str) -> dict:
        gw = cfg.dvr_group_size * cfg.dvr_window_size
        g = cfg.dvr_group_size

        def z(n, dt):
            return torch.zeros(n, dtype=dt, device=device)

        return {
            "input_ids": z(gw, torch.int64), "positions": z(gw, torch.int64),
            "out_slots": z(gw, torch.int64), "sample_positions": z(gw, torch.int64),
            "temperatures": z(gw, torch.float32), "top_ks": z(gw, torch.int64),
            "top_ps": z(gw, torch.float32), "seeds": z(gw, torch.int64),
            "qo_indptr": z(g + 1, torch.int32), "kv_indptr": z(g + 1, torch.int32),
            # a row's kv_len is prefix + W and a prefix can reach max_seq_len - 1
            "kv_indices": z(g * (cfg.max_seq_len + cfg.dvr_window_size), torch.int32),
        }

    def forward(self, fb: ForwardBatch, greedy: bool = False, sample: bool = False,
                with_logits: bool = False):
        """Logits of the sampled rows, or (greedy=True) their greedy tokens, or (sample=True,
        decode batches) the tokens the lm_head-fused sampler draws, with with_logits=True
        together with the logits as (logits, tokens); rows of batch padding are dropped."""
        if self.graphs is not None and fb.graph_key is not None:
            out = self.graphs.run(fb, greedy, sample, with_logits)
        else:
            out = self._forward_eager(fb, greedy, sample, with_logits)
        if fb.real_rows is None:
            return out
        if isinstance(out, tuple):
            return tuple(o[:fb.real_rows] for o in out)
        return out[:fb.real_rows]

    def _forward_eager(self, fb: ForwardBatch, greedy: bool = False, sample: bool = False,
                       with_logits: bool = False):
        fb.build_indices()
        return self.model.forward(fb, self.kv_cache, self.decode_attn,
                                  decode_backend=self.cfg.decode_backend, greedy=greedy,
                                  sample=sample, with_logits=with_logits)

    def _invariant_fused(self) -> bool:
        """batch_invariant mode's one choice per engine (never per batch) for its decode rows
        without top-k / top-p limits: the lm_head-fused sampler when every decode batch fits
        its streaming grouping (max_decode_batch <= 256). The fused sampler and the sampler
        kernel agree except at float near-ties of the scores (their softmax sums run in
        different orders), so a row's path must follow from the row alone."""
        return linear_sample_supported(self.cfg.max_decode_batch, self.mcfg.hidden_size,
                                       tiles=False)

    def _sampled_rows(self, fb: ForwardBatch) -> int:
        return fb.input_ids.shape[0] if fb.sample_indices is None else fb.sample_indices.shape[0]

    def _tiles_always(self, fb: ForwardBatch) -> bool:
        """Prefill and verify passes draw every row without top-k / top-p limits in the
        lm_head with 128-column tiles at every size (tokens independent of the pass's size
        and makeup; a prefill batch has at most max_decode_batch rows, a verify pass G x W)."""
        return fb.mode in (ForwardMode.PREFILL, ForwardMode.VERIFY) and linear_sample_supported(
            self._sampled_rows(fb), self.mcfg.hidden_size, tiles=True)

    def fused_sample(self, fb: ForwardBatch) -> bool:
        """Whether a batch without top-k / top-p limits draws its tokens inside the lm_head
        (sid_linear_sample) instead of writing logits for the sampler kernel, and with which
        softmax-sum grouping (set on fb.sample_tiles; it is part of a row's result, see
        linear_sample):
          * prefill and verify passes: always, with 128-column tiles at every size (a
            verify pass's tokens are the committed ones, a prefill's first tokens are
            committed directly; neither may depend on the pass's size);
          * batch_invariant decode batches: the engine's one choice (_invariant_fused), with
            the streaming grouping at every size;
          * other decode batches: by speed, grouping by row count (T = 0.7, graph-timed:
            1 row 80 vs 178 us for logits + sampler kernel, 64: 120 vs 205, 128: 158 vs 231,
            256: 284 vs 329); dvr commits only the verifier's tokens, nondet is free."""
        if not fb.untruncated:
            return False
        if fb.mode in (ForwardMode.PREFILL, ForwardMode.VERIFY):
            fb.sample_tiles = True
            return self._tiles_always(fb)
        if not linear_sample_supported(self._sampled_rows(fb), self.mcfg.hidden_size):
            return False
        if fb.invariant:
            fb.sample_tiles = False
            return self._invariant_fused()
        fb.sample_tiles = None
        return True

    def step(self, fb: ForwardBatch) -> torch.Tensor:
        """forward + sample -> int64 tokens [R]. An all-greedy batch takes the fused
        lm_head + argmax path, a batch without top-k / top-p limits the fused lm_head +
        sampler where fused_sample says so (no logits written); the rest writes the logits
        and runs the sampler kernel over them. A batch that mixes rows with and without
        limits and needs the fused sampler's tokens for the latter (a prefill or verify
        pass, or a batch_invariant decode batch on an engine whose choice is the fused
        sampler) gets both: the fused sampler's tokens for the rows without limits (as in
        any other batch), the sampler kernel's for the others."""
        if fb.all_greedy:
            return self.forward(fb, greedy=True)
        if self.fused_sample(fb):
            return self.forward(fb, sample=True)
        mixed_tiles = self._tiles_always(fb)
        mixed_invariant = fb.mode == ForwardMode.DECODE and fb.invariant and self._invariant_fused()
        if mixed_tiles or mixed_invariant:
            fb.sample_tiles = True if mixed_tiles else False
            logits, fused = self.forward(fb, sample=True, with_logits=True)
            r = logits.shape[0]
            free = (fb.top_ks[:r] <= 0) & (fb.top_ps[:r] >= 1.0)
            return torch.where(free, fused, self.sample(fb, logits))
        return self.sample(fb, self.forward(fb))

    def prepare_decode(self, reqs: list, invariant: bool, prev_rows=None,
                       prev_tokens: torch.Tensor | None = None) -> ForwardBatch:
        """build_decode_batch, into the graph-static buffers when graphs are enabled. With
        prev_rows / prev_tokens (graphs only), each request's newest token is still in
        flight: row prev_rows[i] of prev_tokens, gathered on the device."""
        if self.graphs is None:
            assert prev_rows is None or not (prev_rows >= 0).any(), "a pending token needs graphs"
            fb = build_decode_batch(reqs, self.kv_cache, self.device, invariant)
            if invariant:
                fb.decode_variant = INVARIANT_VARIANT
            geom = None if invariant else self._pick_variant(fb, len(reqs), fb.max_seq_len)
            self._attach_order(fb, len(reqs), invariant, fb.max_seq_len, geom)
            return fb
        static = self.graphs.decode_static
        pad = batch_bucket(len(reqs), static.max_bs)
        fb = build_decode_batch(reqs, self.kv_cache, self.device, invariant,
                                static=static, pad_to=pad, prev_rows=prev_rows)
        if prev_rows is not None and (prev_rows >= 0).any():
            gather_prev_tokens(static, prev_rows, prev_tokens)
        # The attention grid depends on the longest request (fixed-256 splits, or the
        # segment count of the heuristic splits): bucket it so a graph serves a range. The
        # nondet plan follows the real request count, so it is part of the key. No request
        # is longer than max_seq_len, which also bounds the split workspace's slots.
        bucket = min(length_bucket(fb.max_seq_len), max(self.cfg.max_seq_len, fb.max_seq_len))
        fb.max_seq_len = bucket
        plan = None
        if invariant:
            fb.decode_variant = INVARIANT_VARIANT
        else:
            plan = self._pick_variant(fb, len(reqs), bucket)
        ordered = self._attach_order(fb, pad, invariant, bucket, plan)
        fb.graph_key = ("decode", pad, invariant, bucket, plan, fb.decode_variant, ordered)
        return fb

    def _attach_order(self, fb: ForwardBatch, rows: int, invariant: bool, max_len: int,
                      geom: tuple | None) -> int:
        """The attention's stage-1 placement for this step, from the host-known lengths and
        the plan the forward will run (fixed splits in batch_invariant mode, else the nondet
        geometry): the heaviest-first workgroup order (workgroup_order, balanced over the
        CUs) for the grid, or for a worker launch (stage1_workers) the same dealing over the
        workers. Grids with fewer non-empty segments than CUs otherwise keep their own order
        (nothing to balance, and reading the order first costs a small batch 0.2-0.4 us).
        Placement never changes a result. Returns 0 (grid order), 1 (order attached) or the
        worker count (fb.decode_workers)."""
        da = self.decode_attn
        if invariant:
            tile = da.invariant_split_size
            splits, fixed, seg, slots = 0, tile, tile, max(1, -(-max(max_len, 1) // tile))
        else:
            (splits, seg, slots), fixed = geom, 0
        tokens = segment_tokens(fb.seq_lens_host, rows, splits, fixed, seg, slots)
        fb.decode_wg_order = None
        fb.decode_workers = 0
        cu = da.cu_count()
        nonempty = int(np.count_nonzero(tokens))
        workers = stage1_workers(nonempty, fb.decode_variant, slots, cu)
        if workers == 0 and nonempty < cu:
            return 0
        order = worker_order(tokens, workers) if workers else workgroup_order(tokens, cu)
        if self.graphs is not None:
            fb.decode_wg_order = self.graphs.decode_static.set_order(order)
        else:
            fb.decode_wg_order = torch.from_numpy(order).to(self.device)
        fb.decode_workers = workers
        return workers or 1

    def _pick_variant(self, fb: ForwardBatch, bs: int, max_len: int) -> tuple:
        """The nondet plan's geometry and its stage-1 workgroup shape (fb.decode_variant),
        from the requests' host-known lengths."""
        geom, fb.decode_variant = plan_variant(fb.seq_lens_host, max_len,
                                               self.mcfg.num_kv_heads,
                                               self.decode_attn.cu_count(),
                                               self.cfg.max_kv_splits, invariant=False)
        fb.decode_geometry = geom
        return geom

    def tag_verify(self, fb: ForwardBatch) -> ForwardBatch:
        """Verify batches always live in the persistent verify buffers: graph them."""
        if self.graphs is not None:
            fb.graph_key = ("verify", fb.input_ids.shape[0], fb.max_kv_len)
        return fb

    def sample(self, fb: ForwardBatch, logits: torch.Tensor) -> torch.Tensor:
        r = logits.shape[0]  # real rows (batch padding already dropped by forward)
        return _sample(logits, fb.temperatures[:r], fb.top_ks[:r], fb.top_ps[:r], fb.seeds[:r],
                       fb.sample_positions[:r], all_greedy=fb.all_greedy)


class GraphCache:
    """HIP graphs of the decode forward (one per batch size and split policy) and of the
    fixed-shape verify forward. Every captured graph reads its inputs from fixed buffers
    (DecodeStatic / the verify buffers), so a step is: host builds the batch into those
    buffers, then one graph replay. Kernels of this library take every size they need from
    device memory or from launch arguments that are fixed per key; nothing in the captured
    region allocates host-side or issues memsets."""

    # The decode key holds the batch bucket, the length bucket and the attention plan, which
    # follows the real lengths, so a long mixed run visits many keys: config 5 (dvr) keeps
    # ~80. With room for 64, a second identical run still re-captured 21 of them (21.9k vs
    # 22.2k tokens/s). Graphs of one kind share a memory pool, so more graphs cost only
    # their command lists.
    def __init__(self, runner: "ModelRunner", max_graphs: int = 128):
        cfg = runner.cfg
        # A weak back-reference: no runner <-> cache cycle, so a dropped runner (and its
        # graphs) is freed at once by reference counting, never by a later garbage
        # collection that could run in the middle of another graph's capture.
        self._runner = weakref.ref(runner)
        self.max_graphs = max_graphs
        self.graphs: OrderedDict = OrderedDict()
        # Graphs of one kind replay in order on one stream and share a memory pool; decode
        # and verify graphs may replay concurrently on two streams, so each kind has its own.
        self.pools = {"decode": torch.cuda.graph_pool_handle(),
                      "verify": torch.cuda.graph_pool_handle()}
        self._warm: set = set()
        self.decode_static = DecodeStatic(cfg.max_decode_batch,
                                          cfg.max_decode_batch * cfg.max_seq_len, runner.device,
                                          max_slots=runner.decode_attn.ws_splits)

    def run(self, fb: ForwardBatch, greedy: bool = False, sample: bool = False,
            with_logits: bool = False):
        key = (fb.graph_key, greedy, sample, with_logits)
        entry = self.graphs.get(key)
        if entry is None:
            entry = self._capture(fb, greedy, sample, with_logits)
            self.graphs[key] = entry
            while len(self.graphs) > self.max_graphs:
                self.graphs.popitem(last=False)
        else:
            self.graphs.move_to_end(key)
        graph, out = entry
        graph.replay()
        return out

    def _capture(self, fb: ForwardBatch, greedy: bool, sample: bool, with_logits: bool = False):
        runner = self._runner()
        kind = fb.graph_key[0]
        if kind not in self._warm:
            # One eager pass before the first capture of a kind, so lazy initialisation
            # (library load, descriptors, torch's first-use work) happens outside a capture;
            # it computes exactly what the replay recomputes. Later captures of the kind run
            # the same host code and skip it.
            runner._forward_eager(fb, greedy, sample, with_logits)
            self._warm.add(kind)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        # No garbage collection inside the capture: a collected object that owns device
        # resources (a graph, an event, pinned memory) would release them with HIP calls
        # that are illegal while a stream is being captured, and the process aborts. The
        # collector is only paused (cycles found later are freed after the capture); a full
        # collection first would cost ~50 ms per capture on a serving process's heap.
        was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(graph, pool=self.pools[fb.graph_key[0]]):
                out = runner._forward_eager(fb, greedy, sample, with_logits)
        finally:
            if was_enabled:
                gc.enable()
        return graph, out
