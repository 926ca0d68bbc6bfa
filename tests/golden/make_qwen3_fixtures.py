"""Write tests/golden/qwen3_hf_logits.pt: logits of transformers' own Qwen3ForCausalLM.

Runs only in the build container (needs `transformers`, which is not used anywhere else; no
network: the model is built from a Qwen3Config object, never fetched). The fixture pins the
full-model oracle oracle/qwen3.py:forward_ref, whose op order restates
sid/model/qwen3.py:43-115 of the reference:
  - q/k RMSNorm before RoPE (qwen3.py:55-58),
  - the fused residual add + RMSNorm (qwen3.py:99-111),
  - the fused gate_up weight with gate rows first (qwen3.py:84-85, loader.py:84-101),
  - the tied lm_head applied to the final-normed rows (qwen3.py:113-115).
transformers' modeling_qwen3.py is an independent implementation of the same architecture, so a
dropped term, a swapped operand or a wrong op order in forward_ref shows up as a mismatch.

Model: the real head geometry (16 q / 8 kv heads, head_dim 128, theta 1e6, eps 1e-6, tied
embeddings) with a small hidden size, intermediate size, vocabulary and layer count. Weights
come from a seeded torch CPU generator in a fixed order (`make_weights`, shared with the test),
rounded to bf16; the fixture stores their SHA-256 so the test detects any drift of the
generator. Norm weights are 1 + 0.2 N(0,1), not ones, so a norm applied at the wrong point
or with the wrong weight changes the logits.

HF runs in fp32 on the bf16 weight values (eager attention), once per sequence over the whole
prompt + next token, so one fixture row set covers both the prefill rows and the decode row.
The same model in bf16 is run too: its distance from the fp32 logits is the scale of bf16
rounding noise the test's tolerance is set against.

    python tests/golden/make_qwen3_fixtures.py
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "qwen3_hf_logits.pt"

DIMS = dict(hidden=256, inter=768, vocab=2048, layers=3, hq=16, hkv=8, d=128,
            eps=1e-6, theta=1e6)
SEED = 1234
PROMPT_LENS = (9, 23)


def make_weights(dims=DIMS, seed=SEED) -> dict:
    """Fused-layout weight dict (sid/model/loader.py:84-101): qkv = cat[q, k, v] rows,
    gate_up = cat[gate, up] rows, lm_head = embed (tied). bf16 CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    h, it, v, d = dims["hidden"], dims["inter"], dims["vocab"], dims["d"]
    hq, hkv = dims["hq"], dims["hkv"]

    def normal(*shape, std):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    def norm_w(n):
        return (1.0 + 0.2 * torch.randn(n, generator=g)).to(torch.bfloat16)

    w = {"embed": normal(v, h, std=0.5), "layers": []}
    for _ in range(dims["layers"]):
        w["layers"].append({
            "qkv": normal((hq + 2 * hkv) * d, h, std=0.08),
            "o": normal(h, hq * d, std=0.03),
            "q_norm": norm_w(d),
            "k_norm": norm_w(d),
            "input_ln": norm_w(h),
            "post_ln": norm_w(h),
            "gate_up": normal(2 * it, h, std=0.08),
            "down": normal(h, it, std=0.05),
        })
    w["norm"] = norm_w(h)
    w["lm_head"] = w["embed"]
    return w


def weights_sha256(w: dict) -> str:
    m = hashlib.sha256()
    m.update(w["embed"].view(torch.int16).numpy().tobytes())
    for lw in w["layers"]:
        for k in ("qkv", "o", "q_norm", "k_norm", "input_ln", "post_ln", "gate_up", "down"):
            m.update(lw[k].view(torch.int16).numpy().tobytes())
    m.update(w["norm"].view(torch.int16).numpy().tobytes())
    return m.hexdigest()


def make_sequences(dims=DIMS, seed=SEED + 1):
    """Each sequence = prompt + one next token (the decode step's input)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, dims["vocab"], (n + 1,), generator=g) for n in PROMPT_LENS]


def _hf_model(w: dict, dtype):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    d = DIMS
    cfg = Qwen3Config(vocab_size=d["vocab"], hidden_size=d["hidden"],
                      intermediate_size=d["inter"], num_hidden_layers=d["layers"],
                      num_attention_heads=d["hq"], num_key_value_heads=d["hkv"],
                      head_dim=d["d"], rms_norm_eps=d["eps"], rope_theta=d["theta"],
                      tie_word_embeddings=True, max_position_embeddings=4096,
                      attention_bias=False)
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).eval()
    qs, ks = d["hq"] * d["d"], d["hkv"] * d["d"]
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"],
          "lm_head.weight": w["embed"]}
    for i, lw in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        q, k, v = lw["qkv"].split([qs, ks, ks], dim=0)
        gate, up = lw["gate_up"].chunk(2, dim=0)
        sd.update({
            p + "self_attn.q_proj.weight": q, p + "self_attn.k_proj.weight": k,
            p + "self_attn.v_proj.weight": v, p + "self_attn.o_proj.weight": lw["o"],
            p + "self_attn.q_norm.weight": lw["q_norm"],
            p + "self_attn.k_norm.weight": lw["k_norm"],
            p + "input_layernorm.weight": lw["input_ln"],
            p + "post_attention_layernorm.weight": lw["post_ln"],
            p + "mlp.gate_proj.weight": gate, p + "mlp.up_proj.weight": up,
            p + "mlp.down_proj.weight": lw["down"],
        })
    sd = {k: t.to(dtype) for k, t in sd.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if "rotary" not in m]
    assert not missing and not unexpected, (missing, unexpected)
    return model.to(dtype)


@torch.no_grad()
def main():
    w = make_weights()
    seqs = make_sequences()
    out = {"dims": DIMS, "seed": SEED, "prompt_lens": list(PROMPT_LENS),
           "weights_sha256": weights_sha256(w), "sequences": seqs}
    fp32 = _hf_model(w, torch.float32)
    bf16 = _hf_model(w, torch.bfloat16)
    out["logits_fp32"] = [fp32(s[None]).logits[0].float() for s in seqs]
    # per-row max |bf16 model - fp32 model|: the size of bf16 rounding noise at each row
    out["bf16_noise"] = [(bf16(s[None]).logits[0].float() - ref).abs().amax(-1)
                         for s, ref in zip(seqs, out["logits_fp32"])]
    FIXTURE.parent.mkdir(parents=True, exist_ok=True)
    torch.save(out, FIXTURE)
    for i, s in enumerate(seqs):
        e = out["bf16_noise"][i].max().item()
        print(f"seq {i}: len {len(s)}  hf bf16 vs fp32 max abs {e:.4f}  "
              f"logit scale {out['logits_fp32'][i].abs().max().item():.3f}")
    print(f"wrote {FIXTURE} ({FIXTURE.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
