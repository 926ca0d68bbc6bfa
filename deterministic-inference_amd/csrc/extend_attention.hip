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
// row's position are exact no-ops for it (rescale 2^0 = 1, p = 0, fold
// weight 2^(-1e30 - m) = 0). States keep their maximum m in log2 units
// (scores times sm_scale * log2(e)). So a row's bits depend only on its q, its
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
//   softmax       : online, per query row, with a lazy reference maximum (moved
//                   only when a tile's maximum exceeds it by 2^8); reductions
//                   over the 4 lanes of a row by xor 16 / xor 32 (max is
//                   order-free, sums commute);
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
// LDS row strides (bf16) of the K and V tiles: 304 bytes each. Layout only (bit-identical);
// of 136-152 x 136-160 this measured best on the verify fan-out (~4% over 272 / 288 bytes)
// and equal on prefill.
constexpr int KS_STRIDE = D + 24;
constexpr int VS_STRIDE = D + 24;
constexpr float NEG_BIG = -1e30f;
constexpr float LOG2E = 1.4426950408889634f;
// Slack of the lazy softmax maximum, in log2 units: scores up to 2^LAZY_T above the row's
// reference maximum are taken without moving it.
constexpr float LAZY_T = 8.0f;

// 2^x by the hardware instruction (v_exp_f32): the argument is at most LAZY_T, and results
// that would be denormal may flush to zero.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over lanes l and l ^ 16 (l ^ 32): v_permlane16/32_swap hand each lane the
// values of both lanes of its pair as (lower lane's, upper lane's), so both lanes compute
// the same expression on the same operands (identical bits) without an LDS round trip.
__device__ __forceinline__ float pair16_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float pair32_max(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float pair16_sum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

typedef short s16x4_v __attribute__((ext_vector_type(4)));
typedef short s16x8_v __attribute__((ext_vector_type(8)));

// 4 bf16 of a V^T fragment through the LDS transpose read: within each 16-lane group,
// lane L receives element L % 4 of the 8-byte values addressed by lanes L / 4 + 4j
// (j = 0..3) of its group.
__device__ __forceinline__ s16x4_v ld_tr16(const bf16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_v*)(p));
}

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
// The fold's per-row scalars and its elementwise step, shared by every path that folds.
struct FoldScale {
  float mn, alpha, beta;
};
__device__ __forceinline__ FoldScale fold_scale(float run_m, float m) {
  const float mn = fmaxf(run_m, m);
  return {mn, exp2_fast(run_m - mn), exp2_fast(m - mn)};
}
// Written as one explicit fma over a separately rounded product, so the compiler has no
// contraction choice to make differently in different kernels.
__device__ __forceinline__ float fold_elem(float run, float part, const FoldScale& f) {
  return __builtin_fmaf(run, f.alpha, part * f.beta);
}

__device__ __forceinline__ void fold(RowState& run, float m, float l, const f32x4_v (&a)[8]) {
  const FoldScale f = fold_scale(run.m, m);
  run.l = fold_elem(run.l, l, f);
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) run.acc[db][i] = fold_elem(run.acc[db][i], a[db][i], f);
  run.m = f.mn;
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
  int q_min;
  bool row_ok;
  int r, g, wave, lane, tid;
};

// Global -> register staging of one 64-key tile (K row-major, V for the transposed copy).
// Loaded one tile ahead of the math, so the next tile's HBM round trip overlaps the
// current tile's MFMAs; 8 x 16 bytes per thread.
struct TileRegs {
  u32x4_v k[4];
  u32x4_v v[4];
};

// Pool slots of the split's keys, staged in LDS once per split (s_idx[j] = slot of key
// split_start + j; 0 past the sequence or out of range), so a tile's K/V loads wait on
// LDS rather than on a global index load.
__device__ __forceinline__ void stage_slots(int32_t* s_idx, const Ctx& c, int split_start) {
  const int pos = split_start + c.tid;
  int32_t slot = pos < c.kv_len ? c.idx[pos] : 0;
  if (slot < 0 || slot >= c.num_slots) slot = 0;
  s_idx[c.tid] = slot;
}

__device__ __forceinline__ void load_tile(TileRegs& r, const Ctx& c, const int32_t* s_idx,
                                          int k0) {
  // K: vector v = tid + 256*i -> key v/16, 16-byte chunk v%16 (k0: tile offset in split).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = c.tid + 256 * i;
    const int64_t slot = s_idx[k0 + (v >> 4)];
    r.k[i] = reinterpret_cast<const u32x4_v*>(c.k_cache + slot * c.row_stride + c.h_kv * D)[v & 15];
  }
  // V: the same key / chunk assignment (rows stored as they are; transposed on read).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = c.tid + 256 * i;
    const int64_t slot = s_idx[k0 + (v >> 4)];
    r.v[i] = reinterpret_cast<const u32x4_v*>(c.v_cache + slot * c.row_stride + c.h_kv * D)[v & 15];
  }
}

__device__ __forceinline__ void store_tile(const TileRegs& r, const Ctx& c, bf16_t* sK,
                                           bf16_t* sV) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = c.tid + 256 * i;
    *reinterpret_cast<u32x4_v*>(&sK[(v >> 4) * KS_STRIDE + (v & 15) * 8]) = r.k[i];
    *reinterpret_cast<u32x4_v*>(&sV[(v >> 4) * VS_STRIDE + (v & 15) * 8]) = r.v[i];
  }
}

// Softmax of one tile's scores s (in place: s becomes p), in the exp2 domain:
// p = 2^(s * sc2 - m) with sc2 = sm_scale * log2(e) and m the row's reference maximum in
// the same units. The reference maximum is lazy: it moves to the tile's maximum only when
// that exceeds it by more than LAZY_T, so p <= 2^LAZY_T and most tiles leave it (and the
// accumulator) alone. Every decision is per row (per lane group), so a row's bits depend
// on its own scores only. MASK: apply causality and row validity (keys beyond the row's
// position give p = 0). Returns the accumulator's rescale factor (exactly 1 when the
// reference maximum stays).
template <bool MASK>
__device__ __forceinline__ float softmax_tile(float (&s)[16], RowState& st, const Ctx& c, int t0,
                                              float sc2) {
  bool vis[16];
  float tmax = NEG_BIG;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if constexpr (MASK) {
      const int key = t0 + 32 * (i >> 3) + 8 * c.g + (i & 7);
      vis[i] = (key <= c.q_abs) & c.row_ok;
      tmax = fmaxf(tmax, vis[i] ? s[i] : NEG_BIG);
    } else {
      tmax = fmaxf(tmax, s[i]);
    }
  }
  tmax = pair16_max(tmax);
  tmax = pair32_max(tmax);
  const float mc = tmax * sc2;
  const float m_used = mc > st.m + LAZY_T ? mc : st.m;
  const float rescale = exp2_fast(st.m - m_used);
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = exp2_fast(__builtin_fmaf(s[i], sc2, -m_used));
    if constexpr (MASK) s[i] = vis[i] ? p : 0.0f;
    else s[i] = p;
    psum += s[i];
  }
  psum = pair16_sum(psum);
  psum = pair32_sum(psum);
  st.l = __builtin_fmaf(st.l, rescale, psum);
  st.m = m_used;
  return rescale;
}

// The 64-key tile starting at absolute key t0, already in LDS, folded into `st` (online
// softmax).
__device__ __forceinline__ void tile_math(RowState& st, const Ctx& c, int t0,
                                          const bf16x8_v (&qf)[4], float sc2,
                                          const bf16_t* sK, const bf16_t* sV) {
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

  // `full` (wave-uniform): every row of the wave sees every key of the tile, so no mask.
  const float rescale = t0 + BN - 1 <= c.q_min ? softmax_tile<false>(s, st, c, t0, sc2)
                                              : softmax_tile<true>(s, st, c, t0, sc2);

  bf16x8_v pf[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    uint4 u;  // p is finite (exp of a finite difference, or 0)
    u.x = pack_bf16x2(s[8 * kb + 0], s[8 * kb + 1]);
    u.y = pack_bf16x2(s[8 * kb + 2], s[8 * kb + 3]);
    u.z = pack_bf16x2(s[8 * kb + 4], s[8 * kb + 5]);
    u.w = pack_bf16x2(s[8 * kb + 6], s[8 * kb + 7]);
    pf[kb] = __builtin_bit_cast(bf16x8_v, u);
  }
  // x * 1 == x: the rescale is skipped (same bits) unless some row of the wave moved its
  // reference maximum.
  if (__builtin_amdgcn_ballot_w64(rescale != 1.0f) != 0) {
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      st.acc[db][0] *= rescale;
      st.acc[db][1] *= rescale;
      st.acc[db][2] *= rescale;
      st.acc[db][3] *= rescale;
    }
  }
#pragma unroll
  for (int db = 0; db < 8; ++db) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // A = V^T rows 16 db + r (dims), columns 32 kb + 8 g .. +7 (keys): lane s of a group
      // addresses key 32 kb + 8 g + s / 4 (+ 4), dims 16 db + 4 (s % 4) .. +3.
      const bf16_t* vb = &sV[(32 * kb + 8 * c.g + (c.r >> 2)) * VS_STRIDE + 16 * db + 4 * (c.r & 3)];
      const s16x4_v lo = ld_tr16(vb);
      const s16x4_v hi = ld_tr16(vb + 4 * VS_STRIDE);
      const bf16x8_v vf = __builtin_bit_cast(
          bf16x8_v, static_cast<s16x8_v>(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
      st.acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[kb], st.acc[db], 0, 0, 0);
    }
  }
}

// Keys [t_begin, t_end) of one split (t_begin = split start, at most KSPLIT keys) folded
// into `st` tile by tile, with the next tile's loads in flight during each tile's math.
// (Issuing all of the split's tile loads up front measured slower on the verify fan-out:
// 20.0 -> 21.6 us per layer.)
__device__ __forceinline__ void run_tiles(RowState& st, const Ctx& c, int t_begin, int t_end,
                                          const bf16x8_v (&qf)[4], float sc2, bf16_t* sK,
                                          bf16_t* sV, int32_t* s_idx) {
  if (t_begin >= t_end) return;
  __syncthreads();  // previous split's tiles done with s_idx
  stage_slots(s_idx, c, t_begin);
  __syncthreads();
  TileRegs r;
  load_tile(r, c, s_idx, 0);
  for (int t0 = t_begin; t0 < t_end; t0 += BN) {
    __syncthreads();  // previous tile's math done with the LDS tiles
    store_tile(r, c, sK, sV);
    __syncthreads();
    if (t0 + BN < t_end) load_tile(r, c, s_idx, t0 + BN - t_begin);
    tile_math(st, c, t0, qf, sc2, sK, sV);
  }
}

// part_* layout: [split][total_q][HQ]; part_a holds the unnormalised accumulator
// (128 dims), part_ml = (m, l). Lane holds dims 16*db + 4*g .. +3 of its row.
template <bool FANOUT>
__global__ void __launch_bounds__(256) extend_attention_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ qo_indptr,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    int num_q_heads, int num_kv_heads, int64_t num_slots, float sm_scale, int mtiles,
    int64_t total_q, bf16_t* __restrict__ o, float* __restrict__ part_a,
    float* __restrict__ part_ml, int32_t* __restrict__ part_n) {
  __shared__ __align__(16) bf16_t sK[BN * KS_STRIDE];
  __shared__ __align__(16) bf16_t sV[BN * VS_STRIDE];
  __shared__ int32_t s_idx[KSPLIT];

  const int b = blockIdx.x;
  const int h_kv = blockIdx.y;
  constexpr bool fanout = FANOUT;
  // Without fan-out a workgroup walks every split up to its tile's causal limit, so late
  // query tiles take longest: dispatch them first (blockIdx.z = 0 is the last tile).
  const int mtile = fanout ? static_cast<int>(blockIdx.z) % mtiles
                           : mtiles - 1 - static_cast<int>(blockIdx.z);
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
  c.q_min = prefix + mtile * BQ + 16 * (c.wave & 1);  // the wave's first row
  const float sc2 = sm_scale * LOG2E;
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
  if constexpr (FANOUT) {
    RowState st;
    fresh(st);
    run_tiles(st, c, split * KSPLIT, min(visible_end, (split + 1) * KSPLIT), qf, sc2, sK,
              sV, s_idx);
    if (!c.row_ok) return;
    const int64_t pr = static_cast<int64_t>(split) * total_q * num_q_heads + prow;
    float* pa = part_a + pr * D;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<f32x4_v*>(pa + 16 * db + 4 * c.g) = st.acc[db];
    if (c.g == 0) {
      part_ml[2 * pr] = st.m;
      part_ml[2 * pr + 1] = st.l;
      if (split == 0) part_n[prow] = nsplits;
    }
    return;
  } else {
  RowState run;
  fresh(run);
  for (int sp = 0; sp < nsplits; ++sp) {
    RowState st;
    fresh(st);
    run_tiles(st, c, sp * KSPLIT, min(visible_end, (sp + 1) * KSPLIT), qf, sc2, sK, sV,
              s_idx);
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
}

// Fold the fanned-out split states of every (query row, head) item in split order: one
// wave per item (global item = row * HQ + head), lane l owning dims 2l and 2l + 1. fold()
// is elementwise with per-row scalars, so any assignment of dims to lanes computes the
// same bits as the attention kernel's own layout. The item's split count (written by the
// attention kernel's split-0 workgroup) is loaded first, then up to MERGE_CHUNK of its
// splits' states together, then folded.
constexpr int MERGE_CHUNK = 16;

__global__ void __launch_bounds__(256) extend_merge_kernel(
    int64_t items, int splits, const float* __restrict__ part_a,
    const float* __restrict__ part_ml, const int32_t* __restrict__ part_n,
    bf16_t* __restrict__ o) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= items) return;  // whole waves: no barrier below
  // Only the item's own splits are loaded: the grid's split count follows the pass's
  // key-length bucket (up to twice the longest sequence), and the splits past the item's
  // own hold nothing it reads (measured: verify pass, 4 x 32 rows over 2k keys, 22.1 ->
  // 20.5 us per layer with the fan-out).
  const int nsplits = min(part_n[item], splits);
  float m = NEG_BIG, l = 0.0f;
  float2 acc = make_float2(0.0f, 0.0f);
  for (int c0 = 0; c0 < nsplits; c0 += MERGE_CHUNK) {
    const int n = min(MERGE_CHUNK, nsplits - c0);
    float2 a[MERGE_CHUNK];
    float sm[MERGE_CHUNK], sl[MERGE_CHUNK];
#pragma unroll
    for (int sp = 0; sp < MERGE_CHUNK; ++sp) {
      if (sp < n) {
        const int64_t pr = static_cast<int64_t>(c0 + sp) * items + item;
        a[sp] = reinterpret_cast<const float2*>(part_a + pr * D)[lane];
        sm[sp] = part_ml[2 * pr];
        sl[sp] = part_ml[2 * pr + 1];
      }
    }
#pragma unroll
    for (int sp = 0; sp < MERGE_CHUNK; ++sp) {
      if (sp < n) {  // fold() on two dims
        const FoldScale f = fold_scale(m, sm[sp]);
        l = fold_elem(l, sl[sp], f);
        acc.x = fold_elem(acc.x, a[sp].x, f);
        acc.y = fold_elem(acc.y, a[sp].y, f);
        m = f.mn;
      }
    }
  }
  reinterpret_cast<uint32_t*>(o + item * D)[lane] = pack_bf16x2(acc.x / l, acc.y / l);
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
  // per (split, row, head): 128 accumulator floats + (m, l); per (row, head): split count
  return (splits * (D + 2) + 1) * total_q * num_q_heads * static_cast<int64_t>(sizeof(float));
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
    const int64_t items = total_q * num_q_heads;
    float* pa = static_cast<float*>(workspace);
    float* pml = pa + static_cast<int64_t>(splits) * items * D;
    int32_t* pn = reinterpret_cast<int32_t*>(pml + static_cast<int64_t>(splits) * items * 2);
    hipLaunchKernelGGL(extend_attention_kernel<true>, dim3(batch, num_kv_heads, mtiles * splits),
                       dim3(256), 0, s, (const bf16_t*)q, (const bf16_t*)k_cache,
                       (const bf16_t*)v_cache, qo_indptr, kv_indptr, kv_indices, num_q_heads,
                       num_kv_heads, num_slots, sm_scale, mtiles, total_q, (bf16_t*)o, pa, pml,
                       pn);
    int rc = check_launch("extend_attention");
    if (rc != SID_OK) return rc;
    const int64_t groups = (items + 3) / 4;
    SID_REQUIRE(groups < (1ll << 31), "extend_attention: too many rows for the merge");
    hipLaunchKernelGGL(extend_merge_kernel, dim3((unsigned)groups), dim3(256), 0, s, items,
                       splits, pa, pml, pn, (bf16_t*)o);
    return check_launch("extend_attention merge");
  }
  SID_REQUIRE(mtiles <= 65535, "extend_attention: grid too large");
  hipLaunchKernelGGL(extend_attention_kernel<false>, dim3(batch, num_kv_heads, mtiles), dim3(256), 0, s,
                     (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, qo_indptr,
                     kv_indptr, kv_indices, num_q_heads, num_kv_heads, num_slots, sm_scale, mtiles,
                     total_q, (bf16_t*)o, nullptr, nullptr, nullptr);
  return check_launch("extend_attention");
}
