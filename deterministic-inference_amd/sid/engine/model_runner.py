"""ModelRunner: model, KV cache, decode workspace, verify buffers (sid/engine/model_runner.py).

Numerics: every GEMM, norm and attention kernel on the path is this library's own HIP
code with fixed reduction orders, so no library autotuning or workspace setting can
change bits between runs of the same shape.
"""

from __future__ import annotations

import logging

import torch

from sid.config import EngineConfig, Mode, ModelConfig
from sid.engine.batch import ForwardBatch
from sid.engine.kv_cache import KVCache
from sid.engine.sampler import sample as _sample
from sid.kernels.decode_attention import DecodeAttention
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

    def forward(self, fb: ForwardBatch) -> torch.Tensor:
        return self.model.forward(fb, self.kv_cache, self.decode_attn,
                                  decode_backend=self.cfg.decode_backend)

    def sample(self, fb: ForwardBatch, logits: torch.Tensor) -> torch.Tensor:
        return _sample(logits, fb.temperatures, fb.top_ks, fb.top_ps, fb.seeds,
                       fb.sample_positions, all_greedy=fb.all_greedy)
