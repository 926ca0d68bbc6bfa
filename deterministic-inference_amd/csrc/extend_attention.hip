// Varlen causal "extend" attention over the paged KV pool, gfx950 MFMA.
//
// Used for prefill and for the DVR verify pass (sid/kernels/extend_attention.py
// :1-22 states the contract). All keys, prefix and freshly written window, are
// read from the pool through kv_indices, and causality is by absolute position:
// query j of request b is at position prefix_b + j and sees keys <= that.
//
// Determinism: key tiles of 64 are anchored at absolute position 0 and every
// query row is reduced with the same instruction sequence whichever tile slot
// it occupies; tiles beyond a row's position are exact no-ops for it (rescale
// exp(0) = 1, p = 0). So a row's bits depend only on its own q, its absolute
// position and its sequence's keys: invariant to the window offset (how the
// sequence is split into prefix and extend) and to co-batched requests.
//
// Workgroup = (request, kv head, 32-query tile) with 4 waves; the two query
// heads of the GQA pair share every K/V tile (wave w: head w / 2, query rows
// 16 * (w % 2) .. +15). Per 64-key tile:
//   S^T = K Q^T   : 4 key blocks x 4 k-steps of v_mfma_f32_16x16x32_bf16, with
//                   A = K rows from LDS and B = q held in registers. Key rows are
//                   assigned to MFMA rows so that each lane ends up holding 8
//                   consecutive keys for its query, which is exactly the B
//                   operand layout of the PV product (no shuffles needed);
//   softmax       : online, per query row, reductions over the 4 lanes of a
//                   row by xor 16 / xor 32 (max is order-free, sums commute);
//   O^T += V^T P^T: 8 dim blocks x 2 k-steps, A = V^T from a transposed LDS
//                   copy of the V tile, B = bf16(P) (P is rounded to bf16
//                   before the PV product, as sid/kernels/extend_attention.py:106).
#include "common.h"

namespace sid {
namespace {

constexpr int D = 128;
constexpr int BN = 64;          // keys per tile (anchored at absolute position 0)
constexpr int BQ = 32;          // query positions per workgroup (x 2 heads = 64 rows)
constexpr int KS_STRIDE = D + 8;    // bf16 elements per K row in LDS (272 bytes)
constexpr int VT_STRIDE = BN + 8;   // bf16 elements per transposed V row in LDS (144 bytes)
constexpr float NEG_BIG = -1e30f;

__device__ __forceinline__ float xor16(float v) { return lane_xor(v, 16); }
__device__ __forceinline__ float xor32(float v) { return lane_xor(v, 32); }

__global__ void __launch_bounds__(256) extend_attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ qo_indptr,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    int num_q_heads, int num_kv_heads, int64_t num_slots, float sm_scale,
    bf16_t* __restrict__ o) {
  __shared__ __align__(16) bf16_t sK[BN * KS_STRIDE];
  __shared__ __align__(16) bf16_t sVt[D * VT_STRIDE];

  const int b = blockIdx.x;
  const int h_kv = blockIdx.y;
  const int mtile = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;   // query row within the wave's 16 (MFMA column)
  const int g = lane >> 4;   // k-slot group

  const int q_start = qo_indptr[b];
  const int extend_len = qo_indptr[b + 1] - q_start;
  if (mtile * BQ >= extend_len) return;
  const int kv_start = kv_indptr[b];
  const int kv_len = kv_indptr[b + 1] - kv_start;
  const int prefix = kv_len - extend_len;
  if (prefix < 0) return;  // malformed batch: the kv range must cover the extend tokens

  const int hq = h_kv * 2 + (wave >> 1);
  const int qr = mtile * BQ + 16 * (wave & 1) + r;  // extend-local query row of this lane
  const bool row_ok = qr < extend_len;
  const int q_abs = prefix + qr;

  // q fragments (B operand of S^T = K Q^T): row qr, dims 32*ks + 8*g .. +7.
  bf16x8_v qf[4];
  {
    const bf16_t* qp = q + (static_cast<int64_t>(q_start + (row_ok ? qr : 0)) * num_q_heads + hq) * D;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = *reinterpret_cast<const bf16x8_v*>(qp + 32 * ks + 8 * g);
      if (!row_ok) qf[ks] = bf16x8_v{};
    }
  }

  f32x4_v acc[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) acc[db] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = NEG_BIG;
  float l_run = 0.0f;

  const int last_row = min(extend_len, (mtile + 1) * BQ) - 1;
  const int visible_end = min(kv_len, prefix + last_row + 1);
  const int64_t row_stride = static_cast<int64_t>(num_kv_heads) * D;
  const int32_t* idx = kv_indices + kv_start;

  // MFMA row m of key block j holds key 32*(j/2) + 8*(m/4) + 4*(j%2) + m%4.
  const int key_a0 = 8 * (r >> 2) + (r & 3);

  for (int t0 = 0; t0 < visible_end; t0 += BN) {
    __syncthreads();  // previous tile fully consumed
    // K tile, row-major: vector v = tid + 256*i -> key v/16, 16-byte chunk v%16.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      const int key = v >> 4;
      const int ch = v & 15;
      const int pos = t0 + key;
      int64_t slot = pos < kv_len ? static_cast<int64_t>(idx[pos]) : 0;
      if (slot < 0 || slot >= num_slots) slot = 0;
      const uint4 kv = reinterpret_cast<const uint4*>(k_cache + slot * row_stride + h_kv * D)[ch];
      *reinterpret_cast<uint4*>(&sK[key * KS_STRIDE + ch * 8]) = kv;
    }
    // V tile, transposed: lane -> key, wave w -> 16-byte chunks 4w .. 4w+3.
    {
      const int key = lane;
      const int pos = t0 + key;
      int64_t slot = pos < kv_len ? static_cast<int64_t>(idx[pos]) : 0;
      if (slot < 0 || slot >= num_slots) slot = 0;
      const uint4* vp = reinterpret_cast<const uint4*>(v_cache + slot * row_stride + h_kv * D);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ch = 4 * wave + i;
        const uint4 vv = vp[ch];
        const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sVt[(ch * 8 + 2 * e) * VT_STRIDE + key] = static_cast<bf16_t>(w4[e] & 0xffffu);
          sVt[(ch * 8 + 2 * e + 1) * VT_STRIDE + key] = static_cast<bf16_t>(w4[e] >> 16);
        }
      }
    }
    __syncthreads();

    // S^T blocks: lane holds logits of query r for keys 8g..8g+7 (s[0..7])
    // and 32+8g..32+8g+7 (s[8..15]).
    float s[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = 32 * (j >> 1) + 4 * (j & 1) + key_a0;
      f32x4_v st = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8_v kf = *reinterpret_cast<const bf16x8_v*>(&sK[key * KS_STRIDE + 32 * ks + 8 * g]);
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], st, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * j + i] = st[i];
    }

    // Mask by absolute position, scale, online softmax for row r.
    float tmax = NEG_BIG;
    bool vis[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = t0 + 32 * (i >> 3) + 8 * g + (i & 7);
      vis[i] = row_ok && key <= q_abs;
      s[i] = vis[i] ? s[i] * sm_scale : NEG_BIG;
      tmax = fmaxf(tmax, s[i]);
    }
    tmax = fmaxf(tmax, xor16(tmax));
    tmax = fmaxf(tmax, xor32(tmax));
    const float m_new = fmaxf(m_run, tmax);
    const float rescale = __expf(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = vis[i] ? __expf(s[i] - m_new) : 0.0f;
      psum += s[i];
    }
    psum += xor16(psum);
    psum += xor32(psum);
    l_run = l_run * rescale + psum;
    m_run = m_new;

    // P^T as bf16 B operands: kb = 0 -> s[0..7], kb = 1 -> s[8..15].
    bf16x8_v pf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      uint4 u;
      u.x = pack_bf16x2(s[8 * kb + 0], s[8 * kb + 1]);
      u.y = pack_bf16x2(s[8 * kb + 2], s[8 * kb + 3]);
      u.z = pack_bf16x2(s[8 * kb + 4], s[8 * kb + 5]);
      u.w = pack_bf16x2(s[8 * kb + 6], s[8 * kb + 7]);
      pf[kb] = __builtin_bit_cast(bf16x8_v, u);
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      acc[db][0] *= rescale;
      acc[db][1] *= rescale;
      acc[db][2] *= rescale;
      acc[db][3] *= rescale;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8_v vf =
            *reinterpret_cast<const bf16x8_v*>(&sVt[(16 * db + r) * VT_STRIDE + 32 * kb + 8 * g]);
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[kb], acc[db], 0, 0, 0);
      }
    }
  }

  if (!row_ok) return;
  // Lane holds O[row r][dims 16*db + 4*g .. +3].
  bf16_t* op = o + (static_cast<int64_t>(q_start + qr) * num_q_heads + hq) * D;
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    uint2 u;
    u.x = pack_bf16x2(acc[db][0] / l_run, acc[db][1] / l_run);
    u.y = pack_bf16x2(acc[db][2] / l_run, acc[db][3] / l_run);
    *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) = u;
  }
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_extend_attention_fwd(const void* q, const void* k_cache, const void* v_cache,
                                        const int32_t* qo_indptr, const int32_t* kv_indptr,
                                        const int32_t* kv_indices, int batch, int64_t total_q,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int64_t num_slots, int max_extend_len, float sm_scale,
                                        void* o, void* stream) {
  SID_REQUIRE(batch >= 0 && total_q >= 0, "extend_attention: negative size");
  if (batch == 0 || total_q == 0 || max_extend_len <= 0) return SID_OK;
  SID_REQUIRE(q && k_cache && v_cache && qo_indptr && kv_indptr && kv_indices && o,
              "extend_attention: null pointer");
  SID_REQUIRE(head_dim == D, "extend_attention: head_dim must be %d, got %d", D, head_dim);
  SID_REQUIRE(num_kv_heads > 0 && num_q_heads == 2 * num_kv_heads,
              "extend_attention: expected 2 q heads per kv head (got %d q, %d kv)", num_q_heads,
              num_kv_heads);
  SID_REQUIRE(num_slots > 0, "extend_attention: empty KV pool");
  SID_REQUIRE(batch < (1 << 30), "extend_attention: batch too large");
  const int mtiles = ceil_div(max_extend_len, BQ);
  SID_REQUIRE(mtiles <= 65535 && num_kv_heads <= 65535, "extend_attention: grid too large");
  hipLaunchKernelGGL(extend_attention_kernel, dim3(batch, num_kv_heads, mtiles), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (const bf16_t*)q, (const bf16_t*)k_cache,
                     (const bf16_t*)v_cache, qo_indptr, kv_indptr, kv_indices, num_q_heads,
                     num_kv_heads, num_slots, sm_scale, (bf16_t*)o);
  return check_launch("extend_attention");
}
