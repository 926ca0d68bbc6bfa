"""ctypes descriptor of a Qwen3 model for the native extend-forward executor
(`sid_qwen3_extend_forward` in csrc/forward.hip): weight and KV-pool pointers, built once
per (model, KV cache); a forward over a prefill / verify batch is then one library call
that issues the whole kernel sequence from C++, bit-identical to the Python driver in
sid/model/qwen3.py."""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from sid.kernels.jit import load_ext

_vp, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float




class Layer(ctypes.Structure):
    _fields_ = [("input_ln", _vp), ("qkv", _vp), ("q_norm", _vp), ("k_norm", _vp), ("o", _vp),
                ("post_ln", _vp), ("gate_up", _vp), ("down", _vp), ("k_cache", _vp),
                ("v_cache", _vp), ("qkv_packed", _vp), ("o_packed", _vp),
                ("gate_up_packed", _vp), ("down_packed", _vp)]


class Model(ctypes.Structure):
    _fields_ = [("num_layers", _i32), ("hidden", _i32), ("num_q_heads", _i32),
                ("num_kv_heads", _i32), ("head_dim", _i32), ("intermediate", _i32),
                ("vocab", _i32), ("rms_eps", _f32), ("sm_scale", _f32),
                ("split_k_max_tokens", _i32), ("chain_max_tokens", _i32), ("num_slots", _i64), ("max_positions", _i64),
                ("cos_sin", _vp), ("embed", _vp), ("final_norm", _vp), ("lm_head", _vp),
                ("layers", ctypes.POINTER(Layer))]


class Batch(ctypes.Structure):
    _fields_ = [("num_tokens", _i64), ("batch", _i32), ("max_extend_len", _i32),
                ("max_kv_len", _i32), ("num_kv_indices", _i64), ("input_ids", _vp),
                ("positions", _vp), ("out_slots", _vp), ("qo_indptr", _vp), ("kv_indptr", _vp),
                ("kv_indices", _vp), ("sample_indices", _vp), ("num_samples", _i64),
                ("temperatures", _vp), ("seeds", _vp), ("sample_positions", _vp),
                ("sample_flags", _i32)]


def _bind(lib) -> None:
    if getattr(lib, "_sid_native_forward_bound", False):
        return
    lib.sid_qwen3_extend_workspace_bytes.restype = _i64
    lib.sid_qwen3_extend_workspace_bytes.argtypes = [ctypes.POINTER(Model), ctypes.POINTER(Batch)]
    lib.sid_qwen3_extend_forward.restype = _i32
    lib.sid_qwen3_extend_forward.argtypes = [ctypes.POINTER(Model), ctypes.POINTER(Batch), _vp,
                                             _i64, _vp, _vp, _vp]
    lib._sid_native_forward_bound = True


class NativeQwen3:
    """Descriptor of one model + KV cache (pointers stay valid while both live)."""

    def __init__(self, model, kv_cache, split_k_max_tokens: int, chain_max_tokens: int = 0):
        """chain_max_tokens > 0: batches up to that many tokens run the decode-step chain
        with the model's packed weights (Qwen3Model._packed_weights)."""
        cfg, w = model.cfg, model.w
        self.ext = load_ext()
        _bind(self.ext.lib)
        layers = w["layers"]
        packed = model._packed_weights() if chain_max_tokens > 0 else None
        self.layers = (Layer * cfg.num_layers)()
        for i, lw in enumerate(layers):
            kp, vp = kv_cache.layer(i)
            pw = ((packed[i]["qkv"].data_ptr(), packed[i]["o"].data_ptr(),
                   packed[i]["gate_up"].data_ptr(), packed[i]["down"].data_ptr())
                  if packed is not None else (None, None, None, None))
            self.layers[i] = Layer(lw["input_ln"].data_ptr(), lw["qkv"].data_ptr(),
                                   lw["q_norm"].data_ptr(), lw["k_norm"].data_ptr(),
                                   lw["o"].data_ptr(), lw["post_ln"].data_ptr(),
                                   lw["gate_up"].data_ptr(), lw["down"].data_ptr(),
                                   kp.data_ptr(), vp.data_ptr(), *pw)
        kp0, _ = kv_cache.layer(0)
        self.model = Model(cfg.num_layers, cfg.hidden_size, cfg.num_q_heads, cfg.num_kv_heads,
                           cfg.head_dim, cfg.intermediate_size, cfg.vocab_size,
                           float(cfg.rms_norm_eps), float(model.sm_scale), split_k_max_tokens,
                           chain_max_tokens, kp0.shape[0], model.rope.cos_sin.shape[0],
                           model.rope.cos_sin.data_ptr(), w["embed"].data_ptr(),
                           w["norm"].data_ptr(), w["lm_head"].data_ptr(), self.layers)
        self.vocab = cfg.vocab_size
        self.key = (id(kv_cache), tuple(kv_cache.layer(0)[0].shape))

    def forward(self, fb, greedy: bool, sample: bool = False, with_logits: bool = False,
                sample_tiles: bool = True):
        """Logits fp32 [R, V] of the sampled rows, or their greedy tokens int64 [R], or
        (sample=True) the tokens the lm_head-fused sampler draws for them (no top-k / top-p;
        grouping: 128-column tiles, or sid_linear_sample's choice by row count when
        sample_tiles is False), with with_logits=True as (logits, tokens)."""
        t = fb.input_ids.numel()
        dev = fb.input_ids.device
        r = fb.sample_indices.numel() if fb.sample_indices is not None else t
        samp = (fb.temperatures[:r].data_ptr(), fb.seeds[:r].data_ptr(),
                fb.sample_positions[:r].data_ptr(), 2 if sample_tiles else 0) if sample \
            else (None, None, None, 0)
        b = Batch(t, fb.qo_indptr.numel() - 1, max(fb.max_extend_len, 1),
                  int(fb.max_kv_len or fb.max_seq_len or 0), fb.kv_indices.numel(),
                  fb.input_ids.data_ptr(), fb.positions.data_ptr(), fb.out_slots.data_ptr(),
                  fb.qo_indptr.data_ptr(), fb.kv_indptr.data_ptr(), fb.kv_indices.data_ptr(),
                  fb.sample_indices.data_ptr() if fb.sample_indices is not None else None, r,
                  *samp)
        lib = self.ext.lib
        need = int(lib.sid_qwen3_extend_workspace_bytes(ctypes.byref(self.model), ctypes.byref(b)))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        logits: Optional[torch.Tensor] = None
        tokens: Optional[torch.Tensor] = None
        if greedy or sample:
            tokens = torch.empty(r, dtype=torch.int64, device=dev)
        if not (greedy or sample) or with_logits:
            logits = torch.empty(r, self.vocab, dtype=torch.float32, device=dev)
        rc = lib.sid_qwen3_extend_forward(
            ctypes.byref(self.model), ctypes.byref(b), ws.data_ptr(), ws.numel(),
            logits.data_ptr() if logits is not None else None,
            tokens.data_ptr() if tokens is not None else None,
            torch.cuda.current_stream(dev).cuda_stream)
        if rc != 0:
            raise RuntimeError(f"sid_qwen3_extend_forward: {lib.sid_last_error().decode()}")
        if tokens is None:
            return logits
        return (logits, tokens) if with_logits else tokens
