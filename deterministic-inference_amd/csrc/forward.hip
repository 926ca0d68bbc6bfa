// Native executor of one Qwen3 forward over an extend batch (prefill or DVR verify): the
// kernel sequence of sid/model/qwen3.py:88-115 (this build's Qwen3Model.forward for
// non-decode batches) issued from C++, so a forward costs ~3 us of host time per launch
// instead of a Python op per kernel. It calls the library's own entry points in the same
// order with the same buffers' contents, so its results are bit-identical to the Python
// driver's (checked by the GPU tests). All temporaries come from one caller workspace.
#include "common.h"

#include <algorithm>

namespace sid {
namespace {


// Whether a projection of t rows and n output columns takes the split-K path (the same bits
// either way). Narrow outputs (n <= 2048: o, down) have few output tiles, so split-K keeps
// the chip busy up to 3x `wide_max` rows; n <= 4096 (qkv) below 5/8 of it; wider ones below
// `wide_max`; beyond, the tiled direct GEMM is faster. (MI355X, weights from HBM, fused
// consumers included, split vs direct: o at 512 rows 18.9 vs 20.1 us, at 1024 27.6 vs 23.4;
// down 21.8 vs 28.6, 36.8 vs 31.2; qkv at 128 rows 14.5 vs 15.8, at 192 17.9 vs 15.8.)
bool split_for(int64_t t, int64_t n, int64_t wide_max) {
  if (n <= 2048) return t <= 3 * wide_max;
  if (n <= 4096) return t < 5 * wide_max / 8;
  return t < wide_max;
}

constexpr int64_t kAlign = 256;

struct Carver {
  char* base;
  int64_t used = 0;
  int64_t cap;
  void* take(int64_t bytes) {
    used = (used + kAlign - 1) / kAlign * kAlign;
    void* p = base ? base + used : nullptr;
    used += bytes;
    return p;
  }
};

struct Layout {
  float* r32;     // the decode chain's fp32 residual sums (r32 order)
  void* resid;
  void* x;
  void* proj;     // split-K partials (fp32) or a bf16 projection output
  void* q;
  void* attn;
  void* act;
  void* ext_ws;
  int64_t ext_ws_bytes;
  void* rows;
  void* argmax_ws;
  int64_t argmax_ws_bytes;
  int64_t total;
};

Layout plan(const sid_qwen3_model* m, const sid_extend_batch* b, void* ws) {
  const int64_t t = b->num_tokens;
  const int64_t h = m->hidden;
  const int64_t wq = static_cast<int64_t>(m->num_q_heads + 2 * m->num_kv_heads) * m->head_dim;
  const int64_t ao = static_cast<int64_t>(m->num_q_heads) * m->head_dim;
  const int64_t inter = m->intermediate;
  const int64_t r = b->sample_indices ? b->num_samples : t;
  Carver c{static_cast<char*>(ws), 0, 0};
  Layout l{};
  l.resid = c.take(t * h * 2);
  l.r32 = static_cast<float*>(c.take(t * h * 4));
  l.x = c.take(t * h * 2);
  // One buffer for the largest projection output: fp32 chunk partials [K/256][t][n] on the
  // split-K path, bf16 [t][n] on the direct one (o and down write straight into x).
  int64_t proj = 0;
  const int64_t shapes[4][2] = {{wq, h}, {h, ao}, {2 * inter, h}, {h, inter}};  // {n, k}
  for (const auto& nk : shapes) {
    const int64_t need = split_for(t, nk[0], m->split_k_max_tokens) ? nk[1] / 256 * nk[0] * t * 4
                                                                      : nk[0] * t * 2;
    proj = std::max(proj, need);
  }
  l.proj = c.take(proj);
  l.q = c.take(t * ao * 2);
  l.attn = c.take(t * ao * 2);
  l.act = c.take(t * inter * 2);
  const int64_t kvmax = b->max_kv_len > 0 ? b->max_kv_len : b->num_kv_indices;
  l.ext_ws_bytes = sid_extend_attention_workspace_bytes(b->batch, t, m->num_q_heads,
                                                        m->num_kv_heads,
                                                        std::max(b->max_extend_len, 1),
                                                        static_cast<int>(kvmax));
  l.ext_ws = l.ext_ws_bytes > 0 ? c.take(l.ext_ws_bytes) : nullptr;
  l.rows = b->sample_indices ? c.take(r * h * 2) : nullptr;
  l.argmax_ws_bytes = b->temperatures ? sid_linear_sample_workspace_bytes(r)
                                      : sid_linear_argmax_workspace_bytes(r);
  l.argmax_ws = l.argmax_ws_bytes > 0 ? c.take(l.argmax_ws_bytes) : nullptr;
  l.total = c.used;
  return l;
}

#define SID_TRY(call)               \
  do {                              \
    const int rc_ = (call);         \
    if (rc_ != SID_OK) return rc_;  \
  } while (0)

// The decode chain serves a batch when every layer has its packed weights and the shapes
// are the chain kernels' (hidden 512 / 1024, head_dim 128, I a multiple of 24 and of 256).
bool use_chain(const sid_qwen3_model* m, int64_t t) {
  if (t > m->chain_max_tokens || m->head_dim != 128) return false;
  if (m->hidden != 512 && m->hidden != 1024) return false;
  if (m->intermediate % 24 != 0 || m->intermediate % 256 != 0 || m->intermediate > 4096) return false;
  const int64_t ao = static_cast<int64_t>(m->num_q_heads) * m->head_dim;
  if (ao % 256 != 0 || ao > 4096) return false;
  for (int i = 0; i < m->num_layers; ++i) {
    const sid_qwen3_layer& lw = m->layers[i];
    if (!lw.qkv_packed || !lw.o_packed || !lw.gate_up_packed || !lw.down_packed) return false;
  }
  return true;
}

// lm_head over the sampled rows of l.x: the greedy argmax fused in (logits written if given)
// or the fp32 logits.
int lm_head(const sid_qwen3_model* m, const sid_extend_batch* b, const Layout& l, float* logits,
            int64_t* greedy_tokens, void* stream) {
  const int64_t t = b->num_tokens;
  const int h = m->hidden;
  const int64_t r = b->sample_indices ? b->num_samples : t;
  const void* rows = l.x;
  if (b->sample_indices) {
    SID_TRY(sid_gather_rows(l.x, b->sample_indices, l.rows, r, h, t, stream));
    rows = l.rows;
  }
  if (greedy_tokens && b->temperatures) {  // the sampler fused into the lm_head
    return sid_linear_sample(rows, h, m->lm_head, r, m->vocab, h, b->temperatures, b->seeds,
                             b->sample_positions, l.argmax_ws, l.argmax_ws_bytes, greedy_tokens,
                             logits, b->sample_flags, stream);
  }
  if (greedy_tokens) {
    return sid_linear_argmax(rows, h, m->lm_head, nullptr, logits, r, m->vocab, h, l.argmax_ws,
                             l.argmax_ws_bytes, greedy_tokens, stream);
  }
  return sid_linear(rows, h, m->lm_head, nullptr, logits, r, m->vocab, h, 1, stream);
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int64_t sid_qwen3_extend_workspace_bytes(const sid_qwen3_model* m,
                                                    const sid_extend_batch* b) {
  if (m == nullptr || b == nullptr || b->num_tokens <= 0) return 0;
  return plan(m, b, nullptr).total;
}

extern "C" int sid_qwen3_extend_forward(const sid_qwen3_model* m, const sid_extend_batch* b,
                                        void* workspace, int64_t workspace_bytes, float* logits,
                                        int64_t* greedy_tokens, void* stream) {
  SID_REQUIRE(m && b, "qwen3_extend_forward: null descriptor");
  SID_REQUIRE(b->num_tokens >= 0 && b->batch >= 0, "qwen3_extend_forward: negative size");
  if (b->num_tokens == 0) return SID_OK;
  SID_REQUIRE(m->layers && m->embed && m->final_norm && m->lm_head && m->cos_sin,
              "qwen3_extend_forward: null weight");
  SID_REQUIRE(b->input_ids && b->positions && b->out_slots && b->qo_indptr && b->kv_indptr &&
                  b->kv_indices,
              "qwen3_extend_forward: null batch field");
  SID_REQUIRE(logits || greedy_tokens, "qwen3_extend_forward: no output");
  SID_REQUIRE(!b->temperatures || (greedy_tokens && b->seeds && b->sample_positions),
              "qwen3_extend_forward: sampling needs tokens, seeds and sample_positions");
  const int64_t t = b->num_tokens;
  const int64_t r = b->sample_indices ? b->num_samples : t;
  SID_REQUIRE(r > 0, "qwen3_extend_forward: no sampled rows");
  const Layout l = plan(m, b, workspace);
  SID_REQUIRE(workspace && workspace_bytes >= l.total,
              "qwen3_extend_forward: workspace %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)l.total);
  const int h = m->hidden;
  const int hq = m->num_q_heads, hkv = m->num_kv_heads, d = m->head_dim;
  const int64_t wq = static_cast<int64_t>(hq + 2 * hkv) * d;
  const int64_t ao = static_cast<int64_t>(hq) * d;
  const int64_t inter = m->intermediate;
  const float eps = m->rms_eps;
  const int64_t smax = m->split_k_max_tokens;
  const bool split_qkv = split_for(t, wq, smax);
  const bool split_o = split_for(t, h, smax);
  const bool split_gu = split_for(t, 2 * inter, smax);
  const bool split_down = split_for(t, h, smax);
  float* part = static_cast<float*>(l.proj);
  const int kvmax = static_cast<int>(b->max_kv_len > 0 ? b->max_kv_len : b->num_kv_indices);

  // residual = embed[ids]; x = rmsnorm(residual, input_ln of layer 0)
  SID_TRY(sid_gather_rows(m->embed, b->input_ids, l.resid, t, h, m->vocab, stream));
  if (use_chain(m, t)) {
    // Five launches per layer, the same bits (csrc/decode_chain.hip).
    for (int i = 0; i < m->num_layers; ++i) {
      const sid_qwen3_layer& lw = m->layers[i];
      const bool first = i == 0;  // layer 0 normalises the embedding rows themselves
      SID_TRY(sid_rmsnorm_qkv_post(first ? l.resid : static_cast<const void*>(l.r32), !first,
                                   lw.input_ln, eps, lw.qkv_packed, t, h, hq, hkv, d,
                                   lw.q_norm, lw.k_norm, b->positions, m->cos_sin,
                                   m->max_positions, b->out_slots, l.q, lw.k_cache, lw.v_cache,
                                   m->num_slots, stream));
      SID_TRY(sid_extend_attention_fwd(l.q, lw.k_cache, lw.v_cache, b->qo_indptr, b->kv_indptr,
                                       b->kv_indices, b->batch, t, hq, hkv, d, m->num_slots,
                                       std::max(b->max_extend_len, 1), kvmax, m->sm_scale,
                                       l.ext_ws, l.ext_ws_bytes, l.attn, stream));
      SID_TRY(sid_linear_residual(l.attn, ao, lw.o_packed, l.resid, l.r32, t, h, ao, stream));
      SID_TRY(sid_rmsnorm_linear_silu_mul(l.r32, 1, lw.post_ln, eps, lw.gate_up_packed, l.act,
                                          t, h, inter, stream));
      SID_TRY(sid_linear_residual(l.act, inter, lw.down_packed, l.resid, l.r32, t, h, inter,
                                  stream));
    }
    SID_TRY(sid_rmsnorm_f32(l.r32, m->final_norm, l.x, t, h, eps, stream));
    return lm_head(m, b, l, logits, greedy_tokens, stream);
  }
  SID_TRY(sid_rmsnorm(l.resid, m->layers[0].input_ln, l.x, t, h, eps, stream));
  for (int i = 0; i < m->num_layers; ++i) {
    const sid_qwen3_layer& lw = m->layers[i];
    // qkv projection -> q/k-norm, RoPE, KV-cache write
    if (split_qkv) {
      SID_TRY(sid_linear_partials(l.x, h, lw.qkv, part, t, wq, h, stream));
      SID_TRY(sid_qkv_post(nullptr, part, h / 256, t, hq, hkv, d, lw.q_norm, lw.k_norm, eps,
                           b->positions, m->cos_sin, m->max_positions, b->out_slots, l.q,
                           lw.k_cache, lw.v_cache, m->num_slots, stream));
    } else {
      SID_TRY(sid_linear(l.x, h, lw.qkv, nullptr, l.proj, t, wq, h, 0, stream));
      SID_TRY(sid_qkv_post(l.proj, nullptr, 0, t, hq, hkv, d, lw.q_norm, lw.k_norm, eps,
                           b->positions, m->cos_sin, m->max_positions, b->out_slots, l.q,
                           lw.k_cache, lw.v_cache, m->num_slots, stream));
    }
    SID_TRY(sid_extend_attention_fwd(l.q, lw.k_cache, lw.v_cache, b->qo_indptr, b->kv_indptr,
                                     b->kv_indices, b->batch, t, hq, hkv, d, m->num_slots,
                                     std::max(b->max_extend_len, 1), kvmax, m->sm_scale,
                                     l.ext_ws, l.ext_ws_bytes, l.attn, stream));
    // o projection; residual += o; x = rmsnorm(residual, post_ln)
    if (split_o) {
      SID_TRY(sid_linear_partials(l.attn, ao, lw.o, part, t, h, ao, stream));
      SID_TRY(sid_fused_add_rmsnorm_partials(part, static_cast<int>(ao / 256), l.resid,
                                             lw.post_ln, l.x, t, h, eps, stream));
    } else {
      SID_TRY(sid_linear(l.attn, ao, lw.o, nullptr, l.x, t, h, ao, 0, stream));
      SID_TRY(sid_fused_add_rmsnorm(l.x, l.resid, lw.post_ln, t, h, eps, stream));
    }
    // act = silu(gate) * up in one launch (K = 1024 shapes; the split-K or direct GEMM +
    // silu_mul pair otherwise)
    if (h == 1024 && inter % 64 == 0) {
      SID_TRY(sid_linear_silu_mul(l.x, lw.gate_up, l.act, t, h, inter, stream));
    } else if (split_gu) {
      SID_TRY(sid_linear_partials(l.x, h, lw.gate_up, part, t, 2 * inter, h, stream));
      SID_TRY(sid_silu_mul_partials(part, h / 256, l.act, t, inter, stream));
    } else {
      SID_TRY(sid_linear(l.x, h, lw.gate_up, nullptr, l.proj, t, 2 * inter, h, 0, stream));
      SID_TRY(sid_silu_mul(l.proj, l.act, t, inter, stream));
    }
    // down projection; residual += down; x = rmsnorm(residual, next input_ln / final norm)
    const void* next_w = i + 1 < m->num_layers ? m->layers[i + 1].input_ln : m->final_norm;
    if (split_down) {
      SID_TRY(sid_linear_partials(l.act, inter, lw.down, part, t, h, inter, stream));
      SID_TRY(sid_fused_add_rmsnorm_partials(part, static_cast<int>(inter / 256), l.resid,
                                             next_w, l.x, t, h, eps, stream));
    } else {
      SID_TRY(sid_linear(l.act, inter, lw.down, nullptr, l.x, t, h, inter, 0, stream));
      SID_TRY(sid_fused_add_rmsnorm(l.x, l.resid, next_w, t, h, eps, stream));
    }
  }
  return lm_head(m, b, l, logits, greedy_tokens, stream);
}
