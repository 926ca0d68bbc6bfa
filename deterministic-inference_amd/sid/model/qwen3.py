"""Qwen3 dense forward over a ForwardBatch (sid/model/qwen3.py), every op a HIP kernel.

Qwen3 specifics: explicit head_dim 128; per-head q/k RMSNorm after the QKV projection and
BEFORE RoPE; no biases; SwiGLU; pre-norm with fused residual-add RMSNorm; tied lm_head.

Routing: DECODE -> split-KV decode attention; PREFILL / VERIFY (or
decode_backend="extend") -> extend attention. Both read all keys from the pool after
this step's K/V were written by reshape_and_cache.
"""

from __future__ import annotations

import torch

from sid.config import ModelConfig
from sid.engine.batch import ForwardBatch, ForwardMode
from sid.kernels.extend_attention import extend_attention_fwd
from sid.kernels.matmul_persistent import linear
from sid.kernels.ops import embedding, gather_rows, silu_mul
from sid.kernels.rmsnorm import fused_add_rmsnorm, qk_head_rmsnorm, rmsnorm
from sid.kernels.rope import RotaryEmbedding


class Qwen3Model:
    def __init__(self, mcfg: ModelConfig, weights: dict, device: str):
        self.cfg = mcfg
        self.w = weights
        self.device = device
        self.rope = RotaryEmbedding(mcfg.head_dim, mcfg.max_position_embeddings,
                                    mcfg.rope_theta, device)
        self.sm_scale = mcfg.head_dim ** -0.5
        self.invariant_gemm = False

    def set_batch_invariant(self, enabled: bool) -> None:
        # Every GEMM here already reduces in an M-independent order (see
        # sid.kernels.matmul_persistent), so both settings run the same kernel.
        self.invariant_gemm = enabled

    def _attention(self, layer_idx: int, hidden: torch.Tensor, fb: ForwardBatch, kv_cache,
                   decode_attn, decode_backend: str) -> torch.Tensor:
        cfg = self.cfg
        lw = self.w["layers"][layer_idx]
        t = hidden.shape[0]
        qkv = linear(hidden, lw["qkv"])
        q, k, v = qkv.split([cfg.q_size, cfg.kv_size, cfg.kv_size], dim=-1)
        q = q.contiguous().view(t, cfg.num_q_heads, cfg.head_dim)
        k = k.contiguous().view(t, cfg.num_kv_heads, cfg.head_dim)
        v = v.contiguous().view(t, cfg.num_kv_heads, cfg.head_dim)
        q = qk_head_rmsnorm(q, lw["q_norm"], cfg.rms_norm_eps)
        k = qk_head_rmsnorm(k, lw["k_norm"], cfg.rms_norm_eps)
        self.rope.apply(q, k, fb.positions)
        k_pool, v_pool = kv_cache.layer(layer_idx)
        kv_cache.ext.reshape_and_cache(k, v, k_pool, v_pool, fb.out_slots)
        if fb.mode == ForwardMode.DECODE and decode_backend == "hip":
            o = decode_attn.forward(q, k_pool, v_pool, fb.kv_indptr, fb.kv_indices, fb.seq_lens,
                                    fb.max_seq_len, self.sm_scale, invariant=fb.invariant)
        else:
            qo = fb.qo_indptr
            if qo is None:  # decode through the extend kernel: one query per request
                qo = torch.arange(t + 1, dtype=torch.int32, device=hidden.device)
            o = extend_attention_fwd(q, k_pool, v_pool, qo, fb.kv_indptr, fb.kv_indices,
                                     max(fb.max_extend_len, 1), self.sm_scale)
        return linear(o.view(t, cfg.q_size), lw["o"])

    def _mlp(self, layer_idx: int, hidden: torch.Tensor) -> torch.Tensor:
        lw = self.w["layers"][layer_idx]
        return linear(silu_mul(linear(hidden, lw["gate_up"])), lw["down"])

    @torch.inference_mode()
    def forward(self, fb: ForwardBatch, kv_cache, decode_attn,
                decode_backend: str = "hip") -> torch.Tensor:
        """fp32 logits [R, vocab] for the sampled rows (bf16-rounded values)."""
        cfg = self.cfg
        hidden = embedding(fb.input_ids, self.w["embed"])
        residual = None
        for i in range(cfg.num_layers):
            lw = self.w["layers"][i]
            if residual is None:
                residual = hidden
                hidden = rmsnorm(hidden, lw["input_ln"], cfg.rms_norm_eps)
            else:
                hidden, residual = fused_add_rmsnorm(hidden, residual, lw["input_ln"],
                                                     cfg.rms_norm_eps)
            hidden = self._attention(i, hidden, fb, kv_cache, decode_attn, decode_backend)
            hidden, residual = fused_add_rmsnorm(hidden, residual, lw["post_ln"], cfg.rms_norm_eps)
            hidden = self._mlp(i, hidden)
        hidden, _ = fused_add_rmsnorm(hidden, residual, self.w["norm"], cfg.rms_norm_eps)
        rows = hidden if fb.sample_indices is None else gather_rows(hidden, fb.sample_indices)
        return linear(rows, self.w["lm_head"], out_fp32=True)
