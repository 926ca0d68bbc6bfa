// Varlen causal "extend" attention over the paged KV pool, gfx950 MFMA.
//
// Used for prefill and for the DVR verify pass (sid/kernels/extend_attention.py
// :1-22 states the contract). All keys, prefix and freshly written window, are
// read from the pool through kv_indices, and causality is by absolute position:
// query j of request b is at position prefix_b + j and sees keys <= that.
//
// Reduction order (what makes results bitwise invariant to the window offset
// and to co-batched requests): keys are cut into splits of KSPLIT = 256
// positions anchored at absolute position 0, each split into 64-key tiles.
// Inside a split a query row runs an online softmax from a fresh state over the
// split's tiles in order; the split states are then folded into the row's
// running state in increasing split order by fold(). Tiles and splits beyond a
// row's position are exact no-ops for it (rescale exp(0) = 1, p = 0, fold
// weight exp(-1e30 - m) = 0). So a row's bits depend only on its q, its
// absolute position and its sequence's keys. A launch either walks a query
// tile's splits sequentially in one workgroup, or (when a workspace is given
// and the grid would be small, e.g. the 4 x 32 verify pass) gives every split
// its own workgroup and folds the saved split states afterwards with the same
// fold() in the same order: identical bits, many more workgroups.
//
// Workgroup = (request, kv head, 32-query tile[, split]) with 4 waves; the two
// query heads of the GQA pair share every K/V tile (wave w: head w / 2, query
// rows 16 * (w % 2) .. +15). Per 64-key tile:
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
constexpr int BN = 64;          // keys per tile
constexpr int BQ = 32;          // query positions per workgroup (x 2 heads = 64 rows)
constexpr int KSPLIT = 256;     // keys per split (4 tiles), anchored at position 0
constexpr int KS_STRIDE = D + 8;    // bf16 elements per K row in LDS (272 bytes)
constexpr int VT_STRIDE = BN + 8;   // bf16 elements per transposed V row in LDS (144 bytes)
constexpr float NEG_BIG = -1e30f;

__device__ __forceinline__ float xor16(float v) { return lane_xor(v, 16); }
__device__ __forceinline__ float xor32(float v) { return lane_xor(v, 32); }

// Per-lane softmax state of one query row (the lane's 32 output dims).
struct RowState {
  float m;
  float l;
  f32x4_v acc[8];
};

__device__ __forceinline__ void fresh(RowState& s) {
  s.m = NEG_BIG;
  s.l = 0.0f;
#pragma unroll
  for (int db = 0; db < 8; ++db) s.acc[db] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
}

// run <- fold(run, part): the one merge used by every path.
__device__ __forceinline__ void fold(RowState& run, float m, float l, const f32x4_v (&a)[8]) {
  const float mn = fmaxf(run.m, m);
  const float alpha = __expf(run.m - mn);
  const float beta = __expf(m - mn);
  run.l = run.l * alpha + l * beta;
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) run.acc[db][i] = run.acc[db][i] * alpha + a[db][i] * beta;
  run.m = mn;
}

struct Ctx {
  const bf16_t* k_cache;
  const bf16_t* v_cache;
  const int32_t* idx;
  int64_t row_stride;
  int64_t num_slots;
  int kv_len;
  int h_kv;
  int q_abs;
  bool row_ok;
  int r, g, wave, lane, tid;
};

// One 64-key tile starting at absolute key t0 folded into `st` (online softmax).
__device__ __forceinline__ void tile_step(RowState& st, const Ctx& c, int t0,
                                          const bf16x8_v (&qf)[4], float sm_scale, bf16_t* sK,
                                          bf16_t* sVt) {
  __syncthreads();  // previous tile fully consumed
  // K tile, row-major: vector v = tid + 256*i -> key v/16, 16-byte chunk v%16.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = c.tid + 256 * i;
    const int key = v >> 4;
    const int ch = v & 15;
    const int pos = t0 + key;
    int64_t slot = pos < c.kv_len ? static_cast<int64_t>(c.idx[pos]) : 0;
    if (slot < 0 || slot >= c.num_slots) slot = 0;
    const uint4 kv =
        reinterpret_cast<const uint4*>(c.k_cache + slot * c.row_stride + c.h_kv * D)[ch];
    *reinterpret_cast<uint4*>(&sK[key * KS_STRIDE + ch * 8]) = kv;
  }
  // V tile, transposed: lane -> key, wave w -> 16-byte chunks 4w .. 4w+3.
  {
    const int key = c.lane;
    const int pos = t0 + key;
    int64_t slot = pos < c.kv_len ? static_cast<int64_t>(c.idx[pos]) : 0;
    if (slot < 0 || slot >= c.num_slots) slot = 0;
    const uint4* vp = reinterpret_cast<const uint4*>(c.v_cache + slot * c.row_stride + c.h_kv * D);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = 4 * c.wave + i;
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

  // S^T blocks: lane holds logits of its query for keys 8g..8g+7 (s[0..7]) and
  // 32+8g..32+8g+7 (s[8..15]). MFMA row m of key block j holds key
  // 32*(j/2) + 8*(m/4) + 4*(j%2) + m%4.
  const int key_a0 = 8 * (c.r >> 2) + (c.r & 3);
  float s[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int key = 32 * (j >> 1) + 4 * (j & 1) + key_a0;
    f32x4_v st4 = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8_v kf = *reinterpret_cast<const bf16x8_v*>(&sK[key * KS_STRIDE + 32 * ks + 8 * c.g]);
      st4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], st4, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s[4 * j + i] = st4[i];
  }

  float tmax = NEG_BIG;
  bool vis[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int key = t0 + 32 * (i >> 3) + 8 * c.g + (i & 7);
    vis[i] = c.row_ok && key <= c.q_abs;
    s[i] = vis[i] ? s[i] * sm_scale : NEG_BIG;
    tmax = fmaxf(tmax, s[i]);
  }
  tmax = fmaxf(tmax, xor16(tmax));
  tmax = fmaxf(tmax, xor32(tmax));
  const float m_new = fmaxf(st.m, tmax);
  const float rescale = __expf(st.m - m_new);
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s[i] = vis[i] ? __expf(s[i] - m_new) : 0.0f;
    psum += s[i];
  }
  psum += xor16(psum);
  psum += xor32(psum);
  st.l = st.l * rescale + psum;
  st.m = m_new;

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
    st.acc[db][0] *= rescale;
    st.acc[db][1] *= rescale;
    st.acc[db][2] *= rescale;
    st.acc[db][3] *= rescale;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bf16x8_v vf = *reinterpret_cast<const bf16x8_v*>(
          &sVt[(16 * db + c.r) * VT_STRIDE + 32 * kb + 8 * c.g]);
      st.acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[kb], st.acc[db], 0, 0, 0);
    }
  }
}

// part_* layout: [split][total_q][HQ]; part_a holds the unnormalised accumulator
// (128 dims), part_ml = (m, l). Lane holds dims 16*db + 4*g .. +3 of its row.
__global__ void __launch_bounds__(256) extend_attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ qo_indptr,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    int num_q_heads, int num_kv_heads, int64_t num_slots, float sm_scale, int mtiles,
    int64_t total_q, bf16_t* __restrict__ o, float* __restrict__ part_a,
    float* __restrict__ part_ml) {
  __shared__ __align__(16) bf16_t sK[BN * KS_STRIDE];
  __shared__ __align__(16) bf16_t sVt[D * VT_STRIDE];

  const int b = blockIdx.x;
  const int h_kv = blockIdx.y;
  const bool fanout = part_a != nullptr;
  const int mtile = fanout ? static_cast<int>(blockIdx.z) % mtiles : static_cast<int>(blockIdx.z);
  const int split = fanout ? static_cast<int>(blockIdx.z) / mtiles : 0;

  Ctx c;
  c.tid = threadIdx.x;
  c.wave = c.tid >> 6;
  c.lane = c.tid & 63;
  c.r = c.lane & 15;
  c.g = c.lane >> 4;

  const int q_start = qo_indptr[b];
  const int extend_len = qo_indptr[b + 1] - q_start;
  if (mtile * BQ >= extend_len) return;
  const int kv_start = kv_indptr[b];
  const int kv_len = kv_indptr[b + 1] - kv_start;
  const int prefix = kv_len - extend_len;
  if (prefix < 0) return;  // malformed batch: the kv range must cover the extend tokens

  const int hq = h_kv * 2 + (c.wave >> 1);
  const int qr = mtile * BQ + 16 * (c.wave & 1) + c.r;  // extend-local query row of this lane
  c.row_ok = qr < extend_len;
  c.q_abs = prefix + qr;
  c.k_cache = k_cache;
  c.v_cache = v_cache;
  c.idx = kv_indices + kv_start;
  c.row_stride = static_cast<int64_t>(num_kv_heads) * D;
  c.num_slots = num_slots;
  c.kv_len = kv_len;
  c.h_kv = h_kv;

  const int last_row = min(extend_len, (mtile + 1) * BQ) - 1;
  const int visible_end = min(kv_len, prefix + last_row + 1);
  const int nsplits = ceil_div(visible_end, KSPLIT);
  if (fanout && split >= nsplits) return;  // the merge never reads this split

  // q fragments (B operand of S^T = K Q^T): row qr, dims 32*ks + 8*g .. +7.
  bf16x8_v qf[4];
  {
    const bf16_t* qp = q + (static_cast<int64_t>(q_start + (c.row_ok ? qr : 0)) * num_q_heads + hq) * D;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = *reinterpret_cast<const bf16x8_v*>(qp + 32 * ks + 8 * c.g);
      if (!c.row_ok) qf[ks] = bf16x8_v{};
    }
  }

  const int64_t prow = static_cast<int64_t>(q_start + (c.row_ok ? qr : 0)) * num_q_heads + hq;
  if (fanout) {
    RowState st;
    fresh(st);
    const int t_end = min(visible_end, (split + 1) * KSPLIT);
    for (int t0 = split * KSPLIT; t0 < t_end; t0 += BN) tile_step(st, c, t0, qf, sm_scale, sK, sVt);
    if (!c.row_ok) return;
    const int64_t pr = static_cast<int64_t>(split) * total_q * num_q_heads + prow;
    float* pa = part_a + pr * D;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<f32x4_v*>(pa + 16 * db + 4 * c.g) = st.acc[db];
    if (c.g == 0) {
      part_ml[2 * pr] = st.m;
      part_ml[2 * pr + 1] = st.l;
    }
    return;
  }

  RowState run;
  fresh(run);
  for (int sp = 0; sp < nsplits; ++sp) {
    RowState st;
    fresh(st);
    const int t_end = min(visible_end, (sp + 1) * KSPLIT);
    for (int t0 = sp * KSPLIT; t0 < t_end; t0 += BN) tile_step(st, c, t0, qf, sm_scale, sK, sVt);
    fold(run, st.m, st.l, st.acc);
  }
  if (!c.row_ok) return;
  bf16_t* op = o + prow * D;
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    uint2 u;
    u.x = pack_bf16x2(run.acc[db][0] / run.l, run.acc[db][1] / run.l);
    u.y = pack_bf16x2(run.acc[db][2] / run.l, run.acc[db][3] / run.l);
    *reinterpret_cast<uint2*>(op + 16 * db + 4 * c.g) = u;
  }
}

// Fold the fanned-out split states of every (query row, head) in split order.
// One 64-lane wave per (row, head): lane (r, g) with r = 0 holds... every lane
// reproduces the per-lane layout of the attention kernel (dims 16*db + 4*g + i)
// so fold() runs on exactly the same operands.
__global__ void __launch_bounds__(256) extend_merge_kernel(
    const int32_t* __restrict__ qo_indptr, const int32_t* __restrict__ kv_indptr, int batch,
    int num_q_heads, int64_t total_q, const float* __restrict__ part_a,
    const float* __restrict__ part_ml, bf16_t* __restrict__ o) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (row, head)
  const int lane = threadIdx.x & 63;
  if (item >= total_q * num_q_heads) return;
  const int64_t row = item / num_q_heads;
  // Locate the row's request (binary search over qo_indptr).
  int lo = 0, hi = batch;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (qo_indptr[mid] <= row) lo = mid; else hi = mid;
  }
  const int b = lo;
  const int extend_len = qo_indptr[b + 1] - qo_indptr[b];
  const int kv_len = kv_indptr[b + 1] - kv_indptr[b];
  const int prefix = kv_len - extend_len;
  const int qr = static_cast<int>(row - qo_indptr[b]);
  const int mtile = qr / BQ;
  const int last_row = min(extend_len, (mtile + 1) * BQ) - 1;
  const int visible_end = min(kv_len, prefix + last_row + 1);
  const int nsplits = ceil_div(visible_end, KSPLIT);
  // Lane layout of the attention kernel: g = lane / 16 owns dims 16*db + 4*g + i.
  const int g = lane >> 4;
  RowState run;
  fresh(run);
  for (int sp = 0; sp < nsplits; ++sp) {
    const int64_t pr = static_cast<int64_t>(sp) * total_q * num_q_heads + item;
    const float* pa = part_a + pr * D;
    f32x4_v a[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) a[db] = *reinterpret_cast<const f32x4_v*>(pa + 16 * db + 4 * g);
    fold(run, part_ml[2 * pr], part_ml[2 * pr + 1], a);
  }
  if ((lane & 15) != 0) return;  // 4 lanes (g = 0..3) write the 128 dims
  bf16_t* op = o + item * D;
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    uint2 u;
    u.x = pack_bf16x2(run.acc[db][0] / run.l, run.acc[db][1] / run.l);
    u.y = pack_bf16x2(run.acc[db][2] / run.l, run.acc[db][3] / run.l);
    *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) = u;
  }
}

// Fan the splits out when the grid would leave most CUs idle.
constexpr int kFanoutBelowWg = 512;

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int64_t sid_extend_attention_workspace_bytes(int batch, int64_t total_q,
                                                        int num_q_heads, int num_kv_heads,
                                                        int max_extend_len, int max_kv_len) {
  if (batch <= 0 || total_q <= 0 || max_extend_len <= 0 || max_kv_len <= 0) return 0;
  const int64_t mtiles = ceil_div(max_extend_len, BQ);
  if (static_cast<int64_t>(batch) * num_kv_heads * mtiles >= kFanoutBelowWg) return 0;
  const int64_t splits = ceil_div(max_kv_len, KSPLIT);
  return splits * total_q * num_q_heads * (D + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int sid_extend_attention_fwd(const void* q, const void* k_cache, const void* v_cache,
                                        const int32_t* qo_indptr, const int32_t* kv_indptr,
                                        const int32_t* kv_indices, int batch, int64_t total_q,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int64_t num_slots, int max_extend_len, int max_kv_len,
                                        float sm_scale, void* workspace, int64_t workspace_bytes,
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
  SID_REQUIRE(batch <= 65535 && num_kv_heads <= 65535, "extend_attention: grid too large");
  const int mtiles = ceil_div(max_extend_len, BQ);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t need = sid_extend_attention_workspace_bytes(batch, total_q, num_q_heads,
                                                           num_kv_heads, max_extend_len,
                                                           max_kv_len);
  const bool fanout = need > 0 && workspace != nullptr && workspace_bytes >= need;
  if (fanout) {
    const int splits = ceil_div(max_kv_len, KSPLIT);
    SID_REQUIRE(static_cast<int64_t>(mtiles) * splits <= 65535, "extend_attention: grid too large");
    float* pa = static_cast<float*>(workspace);
    float* pml = pa + static_cast<int64_t>(splits) * total_q * num_q_heads * D;
    hipLaunchKernelGGL(extend_attention_kernel, dim3(batch, num_kv_heads, mtiles * splits),
                       dim3(256), 0, s, (const bf16_t*)q, (const bf16_t*)k_cache,
                       (const bf16_t*)v_cache, qo_indptr, kv_indptr, kv_indices, num_q_heads,
                       num_kv_heads, num_slots, sm_scale, mtiles, total_q, (bf16_t*)o, pa, pml);
    int rc = check_launch("extend_attention");
    if (rc != SID_OK) return rc;
    const int64_t items = total_q * num_q_heads;
    SID_REQUIRE((items + 3) / 4 < (1ll << 31), "extend_attention: too many rows");
    hipLaunchKernelGGL(extend_merge_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s,
                       qo_indptr, kv_indptr, batch, num_q_heads, total_q, pa, pml, (bf16_t*)o);
    return check_launch("extend_attention merge");
  }
  SID_REQUIRE(mtiles <= 65535, "extend_attention: grid too large");
  hipLaunchKernelGGL(extend_attention_kernel, dim3(batch, num_kv_heads, mtiles), dim3(256), 0, s,
                     (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, qo_indptr,
                     kv_indptr, kv_indices, num_q_heads, num_kv_heads, num_slots, sm_scale, mtiles,
                     total_q, (bf16_t*)o, nullptr, nullptr);
  return check_launch("extend_attention");
}
