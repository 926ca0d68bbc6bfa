"""Qwen3 forward oracle on the CPU (fp32 math, bf16 storage points).

Restates sid/model/qwen3.py:43-115 op by op in the same order: embedding; per layer
input norm (plain rmsnorm for layer 0, fused residual add after), fused qkv projection
(rows q | k | v, sid/model/loader.py:84-89), per-head q/k RMSNorm BEFORE RoPE, NeoX RoPE,
cache write at out_slots, attention (decode: all keys of the request; extend/verify:
causal by absolute position), o projection, fused add + post norm, SwiGLU MLP with the
fused gate_up weight (gate rows first, qwen3.py:84-85); final fused add + norm; tied
lm_head on the sampled rows, bf16 logits returned as fp32.

Every intermediate that the GPU path stores as bf16 is rounded to bf16 here too, so the
only differences left are accumulation orders (checked by tolerance and argmax agreement).
Pinned by (tests/test_oracle_qwen3.py): transformers' own Qwen3ForCausalLM, built from a
Qwen3Config with the real head geometry and seeded weights (tests/golden/qwen3_hf_logits.pt,
written by tests/golden/make_qwen3_fixtures.py): every prefill and decode row within the bf16
noise of that model and with the same argmax, while swapped gate/up halves or swapped q/k-norm
weights miss it by 10-100x; a decode step equals, bit for bit, a one-token extend over the
same keys; the last prefill row equals a decode over the cached prefix. Each op is also
pinned by its own oracle (tests/test_oracle.py).
"""

from __future__ import annotations

import torch

from oracle.norms import rmsnorm_ref, fused_add_rmsnorm_ref, rope_ref

BF = torch.bfloat16


def _bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(BF)


def _attend(q, k_pool, v_pool, idx, sm_scale, causal_offset):
    """q [Tq, HQ, D] bf16; keys k_pool[idx]. fp32 out."""
    k = k_pool[idx].float()          # [L, HKV, D]
    v = v_pool[idx].float()
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    qf = q.float().view(q.shape[0], hkv, g, q.shape[2])          # [Tq, HKV, g, D]
    s = torch.einsum("thgd,lhd->hgtl", qf, k) * sm_scale          # [HKV, g, Tq, L]
    if causal_offset is not None:
        tq, L = q.shape[0], k.shape[0]
        mask = torch.arange(L)[None, :] > (causal_offset + torch.arange(tq)[:, None])
        s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("hgtl,lhd->thgd", p, v)
    return o.reshape(q.shape[0], hq, q.shape[2])


def forward_ref(w: dict, cfg, k_pools: list, v_pools: list, batch: dict,
                layers: int | None = None) -> torch.Tensor:
    """w: weight dict on the CPU (bf16); k_pools/v_pools: per-layer CPU bf16 pools, written
    in place at batch['out_slots']. batch keys: mode ('decode' | 'extend'), input_ids,
    positions, out_slots, kv_indptr, kv_indices, qo_indptr (extend), sample_indices.
    layers: run only the first `layers` layers (timing samples); logits still produced."""
    eps = cfg.rms_norm_eps
    hq, hkv, d = cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim
    sm_scale = d ** -0.5
    ids = batch["input_ids"].long()
    pos = batch["positions"].long()
    slots = batch["out_slots"].long()
    kvp = batch["kv_indptr"].long().tolist()
    kvi = batch["kv_indices"].long()
    decode = batch["mode"] == "decode"
    qo = list(range(len(kvp))) if decode else batch["qo_indptr"].long().tolist()
    t = ids.shape[0]

    hidden = w["embed"][ids]
    residual = None
    n_layers = cfg.num_layers if layers is None else layers
    for i in range(n_layers):
        lw = w["layers"][i]
        if residual is None:
            residual = hidden
            x = _bf(rmsnorm_ref(hidden, lw["input_ln"], eps))
        else:
            xf, residual = fused_add_rmsnorm_ref(hidden, residual, lw["input_ln"], eps)
            x = _bf(xf)
        qkv = _bf(x.float() @ lw["qkv"].float().t())
        q, k, v = qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
        q = _bf(rmsnorm_ref(q.reshape(t, hq, d), lw["q_norm"], eps))
        k = _bf(rmsnorm_ref(k.reshape(t, hkv, d), lw["k_norm"], eps))
        v = v.reshape(t, hkv, d)
        q = _bf(rope_ref(q, pos, cfg.rope_theta))
        k = _bf(rope_ref(k, pos, cfg.rope_theta))
        kp, vp = k_pools[i], v_pools[i]
        ok = (slots >= 0) & (slots < kp.shape[0])
        kp[slots[ok]] = k[ok]
        vp[slots[ok]] = v[ok]
        o = torch.empty(t, hq, d, dtype=BF)
        for b in range(len(kvp) - 1):
            idx = kvi[kvp[b]:kvp[b + 1]]
            q_rows = slice(qo[b], qo[b + 1])
            n_q = qo[b + 1] - qo[b]
            if n_q == 0:
                continue
            if idx.numel() == 0:
                o[q_rows] = 0
                continue
            off = None if decode else idx.numel() - n_q
            o[q_rows] = _bf(_attend(q[q_rows], kp, vp, idx, sm_scale, off))
        hidden = _bf(o.reshape(t, hq * d).float() @ lw["o"].float().t())
        xf, residual = fused_add_rmsnorm_ref(hidden, residual, lw["post_ln"], eps)
        x = _bf(xf)
        gu = _bf(x.float() @ lw["gate_up"].float().t())
        gate, up = gu.chunk(2, dim=-1)
        act = torch.nn.functional.silu(gate) * up
        hidden = _bf(act.float() @ lw["down"].float().t())
    xf, _ = fused_add_rmsnorm_ref(hidden, residual, w["norm"], eps)
    rows = _bf(xf)[batch["sample_indices"].long()]
    return _bf(rows.float() @ w["lm_head"].float().t()).float()
