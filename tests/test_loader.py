"""Checkpoint loading (sid/model/loader.py): config.json / generation_config.json fields, the
fused weight layout (qkv = [q; k; v], gate_up = [gate; up]) from safetensors shards, and the
rejection of tensors the Qwen3 layout does not use. CPU only, on a tiny synthetic
checkpoint written here."""

from __future__ import annotations

import json

import pytest
import torch

from sid.model.loader import load_model_config, load_weights

SHAPES = {"self_attn.q_proj.weight": (64, 64), "self_attn.k_proj.weight": (32, 64),
          "self_attn.v_proj.weight": (32, 64), "self_attn.o_proj.weight": (64, 64),
          "self_attn.q_norm.weight": (16,), "self_attn.k_norm.weight": (16,),
          "input_layernorm.weight": (64,), "post_attention_layernorm.weight": (64,),
          "mlp.gate_proj.weight": (96, 64), "mlp.up_proj.weight": (96, 64),
          "mlp.down_proj.weight": (64, 96)}


def _checkpoint(tmp_path, tied=True, extra=False, shards=2):
    from safetensors.torch import save_file
    cfg = {"model_type": "qwen3", "num_hidden_layers": 2, "hidden_size": 64,
           "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 16,
           "intermediate_size": 96, "vocab_size": 100, "rms_norm_eps": 1e-6,
           "rope_theta": 1e6, "max_position_embeddings": 128, "tie_word_embeddings": tied,
           "eos_token_id": 7}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": [7, 8]}))
    g = torch.Generator().manual_seed(0)
    t = {"model.embed_tokens.weight": torch.randn(100, 64, generator=g),
         "model.norm.weight": torch.randn(64, generator=g)}
    if not tied:
        t["lm_head.weight"] = torch.randn(100, 64, generator=g)
    for i in range(2):
        for name, shape in SHAPES.items():
            t[f"model.layers.{i}.{name}"] = torch.randn(*shape, generator=g)
    if extra:
        t["model.layers.0.mlp.bias"] = torch.zeros(3)
    names = sorted(t)
    for s in range(shards):
        save_file({n: t[n] for n in names[s::shards]}, str(tmp_path / f"m-{s}.safetensors"))
    return t


@pytest.mark.parametrize("tied", [True, False])
def test_load_fused_layout(tmp_path, tied):
    t = _checkpoint(tmp_path, tied=tied)
    mcfg = load_model_config(tmp_path, str(tmp_path))
    assert mcfg.eos_token_ids == (7, 8) and mcfg.num_layers == 2 and mcfg.head_dim == 16
    assert mcfg.tie_word_embeddings == tied
    w = load_weights(tmp_path, mcfg, "cpu", dtype=torch.float32)
    assert (w["lm_head"] is w["embed"]) == tied
    for i, lw in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        want_qkv = torch.cat([t[p + "self_attn.q_proj.weight"], t[p + "self_attn.k_proj.weight"],
                              t[p + "self_attn.v_proj.weight"]])
        assert torch.equal(lw["qkv"], want_qkv)
        assert torch.equal(lw["gate_up"][:96], t[p + "mlp.gate_proj.weight"])
        assert torch.equal(lw["gate_up"][96:], t[p + "mlp.up_proj.weight"])
        assert torch.equal(lw["down"], t[p + "mlp.down_proj.weight"])
        assert torch.equal(lw["k_norm"], t[p + "self_attn.k_norm.weight"])


def test_unknown_tensor_rejected(tmp_path):
    _checkpoint(tmp_path, extra=True)
    with pytest.raises(ValueError, match="not in the Qwen3 layout"):
        load_weights(tmp_path, load_model_config(tmp_path, str(tmp_path)), "cpu")


def test_wrong_model_type_rejected(tmp_path):
    _checkpoint(tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["model_type"] = "llama"
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="not qwen3"):
        load_model_config(tmp_path, str(tmp_path))
