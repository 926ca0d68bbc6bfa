"""Model construction: weight dict in the fused layout of sid/model/loader.py:58-107.

{embed, norm, lm_head, layers: [{qkv, o, q_norm, k_norm, input_ln, post_ln, gate_up, down}]}
with qkv = cat[q, k, v] rows and gate_up = cat[gate, up] rows; lm_head is embed when the
embeddings are tied. Offline builds use `random_weights` (projections and embedding
~ N(0, std), norm weights 1, as the HF initialiser does); `load_weights` reads local
safetensors (no download: a missing directory is an error).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from sid.config import ModelConfig


def random_weights(mcfg: ModelConfig, device, seed: int = 0, std: float = 0.02,
                   dtype: torch.dtype = torch.bfloat16) -> dict:
    gen = torch.Generator(device=device).manual_seed(seed)

    def normal(*shape):
        return (torch.randn(*shape, generator=gen, device=device) * std).to(dtype)

    def ones(n):
        return torch.ones(n, dtype=dtype, device=device)

    h, d = mcfg.hidden_size, mcfg.head_dim
    qkv_rows = (mcfg.num_q_heads + 2 * mcfg.num_kv_heads) * d
    w = {"layers": [], "embed": normal(mcfg.vocab_size, h), "norm": ones(h)}
    w["lm_head"] = w["embed"] if mcfg.tie_word_embeddings else normal(mcfg.vocab_size, h)
    for _ in range(mcfg.num_layers):
        w["layers"].append({
            "qkv": normal(qkv_rows, h),
            "o": normal(h, mcfg.num_q_heads * d),
            "q_norm": ones(d),
            "k_norm": ones(d),
            "input_ln": ones(h),
            "post_ln": ones(h),
            "gate_up": normal(2 * mcfg.intermediate_size, h),
            "down": normal(h, mcfg.intermediate_size),
        })
    return w


def load_model_config(model_dir: Path, model_path: str) -> ModelConfig:
    cfg = json.loads((model_dir / "config.json").read_text())
    if cfg.get("model_type") != "qwen3":
        raise ValueError(f"only qwen3 is supported, got {cfg.get('model_type')}")
    eos = [cfg.get("eos_token_id", 151645)]
    gen_path = model_dir / "generation_config.json"
    if gen_path.exists():
        e = json.loads(gen_path.read_text()).get("eos_token_id", eos)
        eos = e if isinstance(e, list) else [e]
    return ModelConfig(
        model_path=model_path,
        num_layers=cfg["num_hidden_layers"],
        hidden_size=cfg["hidden_size"],
        num_q_heads=cfg["num_attention_heads"],
        num_kv_heads=cfg["num_key_value_heads"],
        head_dim=cfg["head_dim"],
        intermediate_size=cfg["intermediate_size"],
        vocab_size=cfg["vocab_size"],
        rms_norm_eps=cfg["rms_norm_eps"],
        rope_theta=cfg["rope_theta"],
        max_position_embeddings=cfg["max_position_embeddings"],
        tie_word_embeddings=cfg.get("tie_word_embeddings", False),
        eos_token_ids=tuple(eos),
    )


def load_weights(model_dir: Path, mcfg: ModelConfig, device,
                 dtype: torch.dtype = torch.bfloat16) -> dict:
    from safetensors.torch import load_file

    raw: dict = {}
    files = sorted(Path(model_dir).glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors under {model_dir}")
    for f in files:
        raw.update(load_file(str(f)))

    def take(name):
        return raw.pop(name).to(device=device, dtype=dtype)

    w = {"layers": [], "embed": take("model.embed_tokens.weight"), "norm": take("model.norm.weight")}
    if mcfg.tie_word_embeddings:
        w["lm_head"] = w["embed"]
        raw.pop("lm_head.weight", None)
    else:
        w["lm_head"] = take("lm_head.weight")
    for i in range(mcfg.num_layers):
        p = f"model.layers.{i}."
        w["layers"].append({
            "qkv": torch.cat([take(p + "self_attn.q_proj.weight"), take(p + "self_attn.k_proj.weight"),
                              take(p + "self_attn.v_proj.weight")], dim=0).contiguous(),
            "o": take(p + "self_attn.o_proj.weight"),
            "q_norm": take(p + "self_attn.q_norm.weight"),
            "k_norm": take(p + "self_attn.k_norm.weight"),
            "input_ln": take(p + "input_layernorm.weight"),
            "post_ln": take(p + "post_attention_layernorm.weight"),
            "gate_up": torch.cat([take(p + "mlp.gate_proj.weight"),
                                  take(p + "mlp.up_proj.weight")], dim=0).contiguous(),
            "down": take(p + "mlp.down_proj.weight"),
        })
    left = [k for k in raw if "rotary" not in k]
    if left:
        raise ValueError(f"unconsumed checkpoint tensors: {left[:5]}")
    return w


def build_model_config(model_path: str, num_layers=None, vocab_size=None) -> tuple[ModelConfig, Path | None]:
    """-> (ModelConfig, model_dir or None for a random-init model)."""
    if model_path.startswith("random:"):
        mcfg = ModelConfig(model_path=model_path)
        model_dir = None
    else:
        model_dir = Path(model_path)
        if not model_dir.is_dir():
            raise FileNotFoundError(
                f"model directory {model_path!r} not found (no network downloads; use "
                "'random:qwen3-0.6b' for a random-init model)")
        mcfg = load_model_config(model_dir, model_path)
    if num_layers is not None:
        mcfg.num_layers = num_layers
    if vocab_size is not None:
        mcfg.vocab_size = vocab_size
    return mcfg, model_dir
