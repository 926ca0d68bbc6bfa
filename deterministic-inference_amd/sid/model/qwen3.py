"""Qwen3 dense forward over a ForwardBatch (sid/model/qwen3.py), every op a HIP kernel.

Qwen3 specifics: explicit head_dim 128; per-head q/k RMSNorm after the QKV projection and
BEFORE RoPE; no biases; SwiGLU; pre-norm with fused residual-add RMSNorm; tied lm_head.

Routing: DECODE -> split-KV decode attention (decode_backend "cuda" / "hip"); PREFILL /
VERIFY, or DECODE with decode_backend "triton" / "extend" -> extend attention. Both read all keys from the pool after
this step's K/V were written by reshape_and_cache.
"""

from __future__ import annotations

import torch

from sid.config import ModelConfig, decode_backend_kind
from sid.engine.batch import ForwardBatch, ForwardMode
from sid.kernels.extend_attention import extend_attention_fwd
from sid.kernels.matmul_persistent import (linear, linear_argmax, linear_argmax_supported,
                                            linear_partials, linear_sample, linear_silu_mul,
                                            linear_silu_mul_preferred)
from sid.kernels.ops import (DECODE_CHAIN_MAX_ROWS, argmax_rows, decode_chain_supported, embedding,
                             fused_add_rmsnorm_partials, gather_rows, linear_residual,
                             pack_decode_weight, qkv_post,
                             rmsnorm_f32, rmsnorm_linear_silu_mul, rmsnorm_qkv_post, silu_mul,
                             silu_mul_partials)
from sid.kernels.rmsnorm import fused_add_rmsnorm, rmsnorm
from sid.kernels.rope import RotaryEmbedding


# Split-K projections (chunk partials folded by the consuming fused kernel) or direct GEMMs
# (the tiled kernel from 64 rows): both give identical bits, so this is a speed choice per
# projection shape. With W = SPLIT_K_MAX_TOKENS: outputs of N <= 2048 columns (o, down: few
# output tiles) split up to 3 W rows, N <= 4096 (qkv) below 5 W / 8, wider ones below W.
# The native executor applies the same rule (sid_qwen3_model.split_k_max_tokens). MI355X,
# weights from HBM, consumers included (split vs direct, us): o at 512 rows 18.9 vs 20.1,
# at 1024 27.6 vs 23.4; down 21.8 vs 28.6, 36.8 vs 31.2; qkv at 128 rows 14.5 vs 15.8, at
# 192 17.9 vs 15.8, at 256 20.7 vs 16.2.
SPLIT_K_MAX_TOKENS = 256


def split_k_preferred(rows: int, n: int, wide_max: int = SPLIT_K_MAX_TOKENS) -> bool:
    if n <= 2048:
        return rows <= 3 * wide_max
    if n <= 4096:
        return rows < 5 * wide_max // 8
    return rows < wide_max


class Qwen3Model:
    def __init__(self, mcfg: ModelConfig, weights: dict, device: str):
        self.cfg = mcfg
        self.w = weights
        self.device = device
        self.rope = RotaryEmbedding(mcfg.head_dim, mcfg.max_position_embeddings,
                                    mcfg.rope_theta, device)
        self.sm_scale = mcfg.head_dim ** -0.5
        self.invariant_gemm = False
        # Prefill / verify batches go through the native executor (one library call per
        # forward); False keeps the op-by-op Python driver below (identical bits).
        self.native_extend = True
        self._native = None
        # Decode batches run the fused five-launch layer chain (identical bits); False keeps
        # the split-K projections with separate norm kernels.
        self.decode_chain = True
        self._packed = None

    def set_batch_invariant(self, enabled: bool) -> None:
        # Every GEMM here already reduces in an M-independent order (see
        # sid.kernels.matmul_persistent), so both settings run the same kernels.
        self.invariant_gemm = enabled

    def _attention(self, layer_idx: int, x: torch.Tensor, fb: ForwardBatch, kv_cache,
                   decode_attn, decode_backend: str, split: bool) -> torch.Tensor:
        """qkv projection -> (q/k-norm, RoPE, cache write) -> attention. Returns o [T, HQ*D]."""
        cfg = self.cfg
        lw = self.w["layers"][layer_idx]
        t = x.shape[0]
        k_pool, v_pool = kv_cache.layer(layer_idx)
        proj = linear_partials(x, lw["qkv"]) if split else linear(x, lw["qkv"])
        q = qkv_post(proj, lw["q_norm"], lw["k_norm"], cfg.rms_norm_eps, fb.positions,
                     self.rope.cos_sin, fb.out_slots, k_pool, v_pool, cfg.num_q_heads)
        return self._attend(layer_idx, q, fb, kv_cache, decode_attn, decode_backend)

    def _attend(self, layer_idx: int, q: torch.Tensor, fb: ForwardBatch, kv_cache, decode_attn,
                decode_backend: str) -> torch.Tensor:
        """Attention of q [T, HQ, D] over the pool (this step's K/V already written)."""
        cfg = self.cfg
        t = q.shape[0]
        k_pool, v_pool = kv_cache.layer(layer_idx)
        if fb.mode == ForwardMode.DECODE and decode_backend == "hip":
            o = decode_attn.forward(q, k_pool, v_pool, fb.kv_indptr, fb.kv_indices, fb.seq_lens,
                                    fb.max_seq_len, self.sm_scale, invariant=fb.invariant,
                                    policy_batch=fb.real_rows, variant=fb.decode_variant,
                                    geometry=fb.decode_geometry, wg_order=fb.decode_wg_order,
                                    workers=fb.decode_workers)
        else:
            qo = fb.qo_indptr
            if qo is None:  # decode through the extend kernel: one query per request
                qo = torch.arange(t + 1, dtype=torch.int32, device=q.device)
            o = extend_attention_fwd(q, k_pool, v_pool, qo, fb.kv_indptr, fb.kv_indices,
                                     max(fb.max_extend_len, 1), self.sm_scale,
                                     max_kv_len=fb.max_kv_len or fb.max_seq_len or None)
        return o.view(t, cfg.q_size)

    def _packed_weights(self) -> list:
        """Per layer, the fragment-packed projection weights of the decode chain (made on
        first use; 0.88 GB for Qwen3-0.6B)."""
        if self._packed is None:
            self._packed = [{"qkv": pack_decode_weight(lw["qkv"]),
                             "o": pack_decode_weight(lw["o"]),
                             "gate_up": pack_decode_weight(lw["gate_up"], gate_up=True),
                             "down": pack_decode_weight(lw["down"])}
                            for lw in self.w["layers"]]
        return self._packed

    def _decode_chain(self, fb: ForwardBatch, kv_cache, decode_attn,
                      decode_backend: str) -> torch.Tensor:
        """The decoder stack of a decode batch as five fused launches per layer
        (csrc/decode_chain.hip); returns the final-normed hidden rows. Same bits as the
        unfused sequence in forward()."""
        cfg = self.cfg
        eps = cfg.rms_norm_eps
        layers = self.w["layers"]
        packed = self._packed_weights()
        residual = embedding(fb.input_ids, self.w["embed"])
        r32 = torch.empty(residual.shape, dtype=torch.float32, device=residual.device)
        src = residual  # layer 0 normalises the embedding rows themselves
        for i in range(cfg.num_layers):
            lw, pw = layers[i], packed[i]
            k_pool, v_pool = kv_cache.layer(i)
            q = rmsnorm_qkv_post(src, lw["input_ln"], eps, pw["qkv"], lw["q_norm"], lw["k_norm"],
                                 fb.positions, self.rope.cos_sin, fb.out_slots, k_pool, v_pool,
                                 cfg.num_q_heads)
            o = self._attend(i, q, fb, kv_cache, decode_attn, decode_backend)
            linear_residual(o, pw["o"], residual, r32)
            act = rmsnorm_linear_silu_mul(r32, lw["post_ln"], eps, pw["gate_up"])
            linear_residual(act, pw["down"], residual, r32)
            src = r32
        return rmsnorm_f32(r32, self.w["norm"], eps)

    @torch.inference_mode()
    def forward(self, fb: ForwardBatch, kv_cache, decode_attn,
                decode_backend: str = "cuda", greedy: bool = False,
                sample: bool = False, with_logits: bool = False):
        """fp32 logits [R, vocab] for the sampled rows (bf16-rounded values); with
        greedy=True, the greedy tokens int64 [R] instead (argmax of those logits, fused into
        the lm_head GEMM for decode-sized R); with sample=True (rows without a top-k / top-p
        limit, R within linear_sample_supported), the sampled tokens int64 [R], drawn inside
        the lm_head GEMM without writing the logits (with_logits=True: (logits, those
        tokens)); the draw's grouping is fb.sample_tiles (see linear_sample; prefill and
        verify passes: tiles).

        Same op order as sid/model/qwen3.py:88-115; the residual add + RMSNorm that follows
        each o / down projection consumes the projection directly (fused), and the down
        projection of layer i feeds layer i+1's input norm (or the final norm)."""
        decode_backend = decode_backend_kind(decode_backend)
        if self.native_extend and fb.mode != ForwardMode.DECODE:
            return self._native_forward(fb, kv_cache, greedy, sample, with_logits)
        cfg = self.cfg
        eps = cfg.rms_norm_eps
        layers = self.w["layers"]
        t = fb.input_ids.shape[0]
        h = cfg.hidden_size
        split_qkv = split_k_preferred(t, cfg.q_size + 2 * cfg.kv_size)
        split_o = split_k_preferred(t, h)
        split_gu = split_k_preferred(t, 2 * cfg.intermediate_size)
        split_down = split_k_preferred(t, h)
        decode_attn.reset_plan()
        if self.decode_chain and fb.mode == ForwardMode.DECODE and decode_chain_supported(
                t, h, cfg.intermediate_size, cfg.q_size, cfg.head_dim):
            x = self._decode_chain(fb, kv_cache, decode_attn, decode_backend)
            return self._head(x, fb, greedy, sample, with_logits)
        residual = embedding(fb.input_ids, self.w["embed"])
        x = rmsnorm(residual, layers[0]["input_ln"], eps)
        for i in range(cfg.num_layers):
            lw = layers[i]
            o = self._attention(i, x, fb, kv_cache, decode_attn, decode_backend, split_qkv)
            if split_o:
                x, residual = fused_add_rmsnorm_partials(linear_partials(o, lw["o"]), residual,
                                                         lw["post_ln"], eps)
            else:
                x, residual = fused_add_rmsnorm(linear(o, lw["o"]), residual, lw["post_ln"], eps)
            if linear_silu_mul_preferred(t, x.shape[1]):
                act = linear_silu_mul(x, lw["gate_up"])
            elif split_gu:
                act = silu_mul_partials(linear_partials(x, lw["gate_up"]))
            else:
                act = silu_mul(linear(x, lw["gate_up"]))
            next_w = layers[i + 1]["input_ln"] if i + 1 < cfg.num_layers else self.w["norm"]
            if split_down:
                x, residual = fused_add_rmsnorm_partials(linear_partials(act, lw["down"]),
                                                         residual, next_w, eps)
            else:
                x, residual = fused_add_rmsnorm(linear(act, lw["down"]), residual, next_w, eps)
        return self._head(x, fb, greedy, sample, with_logits)

    def _head(self, x: torch.Tensor, fb: ForwardBatch, greedy: bool, sample: bool,
              with_logits: bool):
        """lm_head (tied) on the sampled rows of the final-normed hidden states x."""
        rows = x if fb.sample_indices is None else gather_rows(x, fb.sample_indices)
        if sample:  # the sampler fused into the lm_head (rows without top-k / top-p)
            r = rows.shape[0]
            args = (rows, self.w["lm_head"], fb.temperatures[:r], fb.seeds[:r],
                    fb.sample_positions[:r])
            if not with_logits:
                return linear_sample(*args, tiles=fb.sample_tiles)
            # also the logits, for the rows that need the sampler kernel: the tiled sampler
            # writes them in its own pass; the streaming grouping cannot
            if fb.sample_tiles is False:
                return linear(rows, self.w["lm_head"], out_fp32=True), linear_sample(*args, tiles=False)
            logits = torch.empty(r, self.cfg.vocab_size, dtype=torch.float32, device=rows.device)
            return logits, linear_sample(*args, tiles=True, logits=logits)
        if greedy:
            if linear_argmax_supported(rows.shape[0], rows.shape[1]):
                return linear_argmax(rows, self.w["lm_head"])
            return argmax_rows(linear(rows, self.w["lm_head"], out_fp32=True))
        return linear(rows, self.w["lm_head"], out_fp32=True)

    def _native_forward(self, fb: ForwardBatch, kv_cache, greedy: bool, sample: bool = False,
                        with_logits: bool = False):
        from sid.model.native import NativeQwen3
        key = (id(kv_cache), tuple(kv_cache.layer(0)[0].shape), self.decode_chain)
        if self._native is None or self._native.key != key:
            self._native = NativeQwen3(self, kv_cache, SPLIT_K_MAX_TOKENS,
                                       DECODE_CHAIN_MAX_ROWS if self.decode_chain else 0)
            self._native.key = key
        return self._native.forward(fb, greedy, sample, with_logits,
                                    sample_tiles=fb.sample_tiles is not False)
