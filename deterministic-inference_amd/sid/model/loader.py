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


# ModelConfig field <- config.json key (HF Qwen3 names); the rest keep ModelConfig defaults.
_CONFIG_FIELDS = (
    ("num_layers", "num_hidden_layers"), ("hidden_size", "hidden_size"),
    ("num_q_heads", "num_attention_heads"), ("num_kv_heads", "num_key_value_heads"),
    ("head_dim", "head_dim"), ("intermediate_size", "intermediate_size"),
    ("vocab_size", "vocab_size"), ("rms_norm_eps", "rms_norm_eps"),
    ("rope_theta", "rope_theta"), ("max_position_embeddings", "max_position_embeddings"),
)


def _read_json(path: Path) -> dict:
    return json.loads(path.read_text()) if path.exists() else {}


def load_model_config(model_dir: Path, model_path: str) -> ModelConfig:
    """ModelConfig of a local Qwen3 checkpoint directory (config.json, and the stop ids of
    generation_config.json when present, as sid/model/loader.py:30-50 reads them)."""
    hf = _read_json(model_dir / "config.json")
    if hf.get("model_type") != "qwen3":
        raise ValueError(f"{model_dir}: model_type {hf.get('model_type')!r} is not qwen3")
    missing = [key for _, key in _CONFIG_FIELDS if key not in hf]
    if missing:
        raise ValueError(f"{model_dir}/config.json lacks {missing}")
    stop = _read_json(model_dir / "generation_config.json").get(
        "eos_token_id", hf.get("eos_token_id", 151645))
    return ModelConfig(model_path=model_path,
                       tie_word_embeddings=bool(hf.get("tie_word_embeddings", False)),
                       eos_token_ids=tuple(stop) if isinstance(stop, list) else (stop,),
                       **{field: hf[key] for field, key in _CONFIG_FIELDS})


# Fused weight -> the checkpoint tensors stacked along dim 0 to build it ({} = layer prefix).
_LAYER_TENSORS = {
    "qkv": ("{}self_attn.q_proj.weight", "{}self_attn.k_proj.weight", "{}self_attn.v_proj.weight"),
    "o": ("{}self_attn.o_proj.weight",),
    "q_norm": ("{}self_attn.q_norm.weight",),
    "k_norm": ("{}self_attn.k_norm.weight",),
    "input_ln": ("{}input_layernorm.weight",),
    "post_ln": ("{}post_attention_layernorm.weight",),
    "gate_up": ("{}mlp.gate_proj.weight", "{}mlp.up_proj.weight"),
    "down": ("{}mlp.down_proj.weight",),
}


def load_weights(model_dir: Path, mcfg: ModelConfig, device,
                 dtype: torch.dtype = torch.bfloat16) -> dict:
    """The fused weight dict from local *.safetensors shards, read tensor by tensor. Every
    tensor of the checkpoint must be used (rotary caches aside): a name the table does not
    know means a different architecture."""
    from safetensors import safe_open

    shards = sorted(Path(model_dir).glob("*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"no safetensors under {model_dir}")
    where = {}
    for shard in shards:
        with safe_open(str(shard), framework="pt") as f:
            where.update({name: shard for name in f.keys()})
    used = set()

    def fetch(*names):
        parts = []
        for name in names:
            if name not in where:
                raise KeyError(f"{model_dir}: checkpoint has no tensor {name}")
            with safe_open(str(where[name]), framework="pt") as f:
                parts.append(f.get_tensor(name))
            used.add(name)
        t = parts[0] if len(parts) == 1 else torch.cat(parts, 0)
        return t.to(device=device, dtype=dtype).contiguous()

    w = {"embed": fetch("model.embed_tokens.weight"), "norm": fetch("model.norm.weight")}
    if mcfg.tie_word_embeddings:
        w["lm_head"] = w["embed"]
        used.add("lm_head.weight")
    else:
        w["lm_head"] = fetch("lm_head.weight")
    w["layers"] = [{key: fetch(*(n.format(f"model.layers.{i}.") for n in names))
                    for key, names in _LAYER_TENSORS.items()}
                   for i in range(mcfg.num_layers)]
    extra = sorted(n for n in where if n not in used and "rotary" not in n)
    if extra:
        raise ValueError(f"{model_dir}: {len(extra)} checkpoint tensors not in the Qwen3 "
                         f"layout, e.g. {extra[:3]}")
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
