"""Pins oracle/qwen3.py:forward_ref (the full-model oracle) on the CPU.

1. Against transformers' Qwen3ForCausalLM: tests/golden/qwen3_hf_logits.pt holds the logits
   of the HF model (built from a Qwen3Config, fp32, eager attention) on seeded weights that
   `make_weights` regenerates here; their SHA-256 is checked first. forward_ref runs the
   prompts as one prefill (extend) batch and then one decode step, and every row must agree
   with HF within the bf16 rounding noise the fixture measured (the same HF model run in
   bf16), with the same argmax.
2. Sensitivity: weights with the gate/up halves swapped, or with the q/k-norm weights
   swapped, miss the fixture by far more than that tolerance, so the check can tell the
   reference's op order (qwen3.py:55-58, 84-85) from a plausible mistake.
3. Identities: a decode step equals, bit for bit, a one-token extend at the same position
   over the same keys; the last row of a prefill equals a decode over the cached prefix
   (within fp32 accumulation noise).
"""

from __future__ import annotations

import copy
from pathlib import Path

import pytest
import torch

from oracle.qwen3 import forward_ref
from sid.config import ModelConfig

GOLDEN = Path(__file__).resolve().parent / "golden"
FIX = GOLDEN / "qwen3_hf_logits.pt"


def _load():
    import sys
    sys.path.insert(0, str(GOLDEN))
    try:
        from make_qwen3_fixtures import make_weights, weights_sha256
    finally:
        sys.path.pop(0)
    fx = torch.load(FIX, weights_only=True)
    w = make_weights(fx["dims"], fx["seed"])
    assert weights_sha256(w) == fx["weights_sha256"], "weight generator drifted"
    d = fx["dims"]
    cfg = ModelConfig(num_layers=d["layers"], hidden_size=d["hidden"], num_q_heads=d["hq"],
                      num_kv_heads=d["hkv"], head_dim=d["d"], intermediate_size=d["inter"],
                      vocab_size=d["vocab"], rms_norm_eps=d["eps"], rope_theta=d["theta"])
    return fx, w, cfg


@pytest.fixture(scope="module")
def fixture():
    return _load()


def _pools(cfg, n_slots=128):
    g = torch.Generator().manual_seed(7)
    shape = (n_slots, cfg.num_kv_heads, cfg.head_dim)
    # garbage in unused slots: nothing may read them
    kp = [torch.randn(*shape, generator=g).to(torch.bfloat16) * 50 for _ in range(cfg.num_layers)]
    vp = [torch.randn(*shape, generator=g).to(torch.bfloat16) * 50 for _ in range(cfg.num_layers)]
    return kp, vp


def _slot_tables(lens, n_slots=128, seed=3):
    """One shuffled slot per position of every sequence (prompt + next token)."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(n_slots, generator=g)
    out, at = [], 0
    for n in lens:
        out.append(perm[at:at + n])
        at += n
    return out


def _prefill_batch(prompts, tables):
    ids = torch.cat(prompts)
    pos = torch.cat([torch.arange(len(p)) for p in prompts])
    slots = torch.cat([t[:len(p)] for p, t in zip(prompts, tables)])
    lens = torch.tensor([0] + [len(p) for p in prompts])
    indptr = torch.cumsum(lens, 0)
    return {"mode": "extend", "input_ids": ids, "positions": pos, "out_slots": slots,
            "kv_indptr": indptr, "kv_indices": slots.clone(), "qo_indptr": indptr.clone(),
            "sample_indices": torch.arange(len(ids))}


def _decode_batch(tokens, positions, tables):
    n = len(tokens)
    slots = torch.stack([t[p] for t, p in zip(tables, positions)])
    kv = [t[:p + 1] for t, p in zip(tables, positions)]
    indptr = torch.cumsum(torch.tensor([0] + [len(k) for k in kv]), 0)
    return {"mode": "decode", "input_ids": torch.as_tensor(tokens),
            "positions": torch.as_tensor(positions), "out_slots": slots,
            "kv_indptr": indptr, "kv_indices": torch.cat(kv), "sample_indices": torch.arange(n)}


def _run(w, cfg, fx):
    """Prefill of every prompt, then one decode step: logits per sequence, rows = positions."""
    seqs = fx["sequences"]
    prompts = [s[:-1] for s in seqs]
    tables = _slot_tables([len(s) for s in seqs])
    kp, vp = _pools(cfg)
    pre = forward_ref(w, cfg, kp, vp, _prefill_batch(prompts, tables))
    dec = forward_ref(w, cfg, kp, vp, _decode_batch([int(s[-1]) for s in seqs],
                                                     [len(p) for p in prompts], tables))
    out, at = [], 0
    for i, p in enumerate(prompts):
        out.append(torch.cat([pre[at:at + len(p)], dec[i:i + 1]]))
        at += len(p)
    return out


def _mismatch(logits, fx):
    """Worst ratio of |oracle - HF fp32| to the fixture's bf16 noise of the same row."""
    worst = 0.0
    for mine, ref, noise in zip(logits, fx["logits_fp32"], fx["bf16_noise"]):
        err = (mine - ref).abs().amax(-1)
        worst = max(worst, (err / noise.clamp_min(1e-3)).max().item())
    return worst


def test_forward_ref_matches_transformers_qwen3(fixture):
    fx, w, cfg = fixture
    logits = _run(w, cfg, fx)
    # forward_ref rounds to bf16 at the GPU path's storage points, HF fp32 does not, so the
    # difference is bf16 rounding noise: within 2x what the whole HF model shows in bf16.
    assert _mismatch(logits, fx) < 2.0
    for mine, ref in zip(logits, fx["logits_fp32"]):
        top2 = ref.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 0.25
        assert clear.sum() >= len(ref) - 2
        assert torch.equal(mine.argmax(-1)[clear], ref.argmax(-1)[clear])


def test_fixture_rejects_swapped_gate_up(fixture):
    fx, w, cfg = fixture
    bad = copy.deepcopy(w)
    for lw in bad["layers"]:
        gate, up = lw["gate_up"].chunk(2, dim=0)
        lw["gate_up"] = torch.cat([up, gate])
    assert _mismatch(_run(bad, cfg, fx), fx) > 10.0


def test_fixture_rejects_swapped_qk_norm(fixture):
    fx, w, cfg = fixture
    bad = copy.deepcopy(w)
    for lw in bad["layers"]:
        lw["q_norm"], lw["k_norm"] = lw["k_norm"], lw["q_norm"]
    assert _mismatch(_run(bad, cfg, fx), fx) > 10.0


def test_decode_equals_one_token_extend(fixture):
    fx, w, cfg = fixture
    seqs = fx["sequences"]
    prompts = [s[:-1] for s in seqs]
    tables = _slot_tables([len(s) for s in seqs])
    kp, vp = _pools(cfg)
    forward_ref(w, cfg, kp, vp, _prefill_batch(prompts, tables))
    kp2, vp2 = [t.clone() for t in kp], [t.clone() for t in vp]
    toks = [int(s[-1]) for s in seqs]
    positions = [len(p) for p in prompts]
    dec_b = _decode_batch(toks, positions, tables)
    dec = forward_ref(w, cfg, kp, vp, dec_b)
    ext_b = dict(dec_b, mode="extend", qo_indptr=torch.arange(len(toks) + 1))
    ext = forward_ref(w, cfg, kp2, vp2, ext_b)
    assert torch.equal(dec, ext)
    for a, b in zip(kp + vp, kp2 + vp2):
        assert torch.equal(a, b)


def test_prefill_last_row_equals_decode_over_prefix(fixture):
    fx, w, cfg = fixture
    seq = fx["sequences"][1]
    table = _slot_tables([len(seq)])[0]
    n = len(seq)
    kp, vp = _pools(cfg)
    full = forward_ref(w, cfg, kp, vp, _prefill_batch([seq], [table]))
    kp, vp = _pools(cfg)
    forward_ref(w, cfg, kp, vp, _prefill_batch([seq[:-1]], [table]))
    last = forward_ref(w, cfg, kp, vp, _decode_batch([int(seq[-1])], [n - 1], [table]))
    # the prefix rows of both runs are the same math; only GEMM blocking (M = n vs n - 1 and 1)
    # may change fp32 accumulation order, which bf16 storage mostly absorbs
    err = (full[-1] - last[0]).abs().max().item()
    assert err < 0.25 * fx["bf16_noise"][1][-1].item() + 1e-3
    assert torch.equal(full[-1].argmax(), last[0].argmax())
