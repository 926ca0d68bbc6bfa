// Split-KV paged decode attention for gfx950 (CDNA4, wave64).
//
// Stage 1: one workgroup per (request, segment) computes the partial attention of all
// 16 query heads over the segment's tokens. A segment is a run of at most `seg` tokens
// inside one KV split; split geometry follows kv_per_split in
// sid/csrc/flash_decode.cu:56-60 exactly (it decides which tokens each split owns, so it
// must match the host-side policy of sid/kernels/decode_attention.py:56-85); seg = 0
// makes every split a single segment (the reference's partition). Stage 2 merges the
// request's segments with the log-sum-exp rescale in increasing token order.
//
// Why all heads in one workgroup: a pool row of one token is HKV x D bf16 = 2 KiB
// (8 heads x 256 B). Reading whole rows keeps every HBM access a contiguous 2 KiB run
// (measured ~6.8 TB/s for the bare gather, against ~6.0 TB/s when each workgroup reads
// one head's 256-byte slice of every row).
//
// Inside a segment the work is laid out for wave64:
//   * lane group g (8 lanes) of every wave owns kv head g and its two query heads; lane
//     `sub` owns dims 8*sub..8*sub+7 and 64+8*sub..64+8*sub+7, so one K (or V) load
//     instruction of a wave covers the first (second) 128 bytes of all 8 heads of a token
//     - eight whole 128-byte lines;
//   * q.k uses v_dot2_f32_bf16 on the packed bf16 operands, reduced over the 8 lanes of a
//     head with three DPP steps (every lane ends with the same bits because each step
//     adds a commutative pair);
//   * a wave takes TPL consecutive tokens per iteration (waves interleaved), and each lane
//     group keeps its heads' online-softmax state (running max m, running sum l, fp32
//     accumulator) over the wave's tokens; the waves are merged through LDS in wave order.
// The result is a fixed function of (request data, seq_len, num_splits, seg): no
// atomics, no dependence on batch composition or scheduling.
#include "common.h"

#include <cstdlib>
#include <mutex>

namespace sid {
namespace {

constexpr int HEAD_DIM = 128;
constexpr int HKV = 8;              // kv heads (a lane group per head)
constexpr int QPK = 2;              // query heads per kv head
constexpr int HQ = HKV * QPK;
constexpr bool kNonTemporal = true;  // K/V rows are streamed once: +9% HBM throughput
constexpr int HEUR_TILE = 32;       // granularity of the heuristic split size
constexpr float NEG_BIG = -1e30f;   // finite "minus infinity" for running maxima
constexpr int kOrderSlotBits = 12;  // wg_order entries: request << 12 | slot
constexpr int kOrderEmpty = 1 << 30;  // wg_order entry flag: the item holds no tokens

__host__ __device__ __forceinline__ int kv_per_split(int seq_len, int n_splits, int fixed_split) {
  if (fixed_split > 0) return fixed_split;
  return ceil_div(ceil_div(seq_len, n_splits), HEUR_TILE) * HEUR_TILE;
}

// The split count of a request when the caller passes no num_splits array: the reference's
// policies restated on the device (sid/kernels/decode_attention.py:65-85): fixed-size splits
// cover the sequence, the heuristic takes one split per 32 tokens up to the grid's split
// count. A request without tokens gets 0 (its output is zeros).
__device__ __forceinline__ int derived_splits(int seq_len, int max_splits, int fixed_split) {
  if (seq_len <= 0) return 0;
  if (fixed_split > 0) return ceil_div(seq_len, fixed_split);
  return min(ceil_div(seq_len, HEUR_TILE), max_splits);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a),
                                         __builtin_bit_cast(bf16x2_v, b), c, false);
}

// 16-dim partial dot product of one query head with one token row (the two
// 16-byte halves a lane owns), fixed order.
__device__ __forceinline__ float dot16(const u32x4_v (&qa)[2], const u32x4_v (&ka)[2]) {
  float s = dot2(qa[0].x, ka[0].x, 0.0f);
  s = dot2(qa[0].y, ka[0].y, s);
  s = dot2(qa[0].z, ka[0].z, s);
  s = dot2(qa[0].w, ka[0].w, s);
  s = dot2(qa[1].x, ka[1].x, s);
  s = dot2(qa[1].y, ka[1].y, s);
  s = dot2(qa[1].z, ka[1].z, s);
  s = dot2(qa[1].w, ka[1].w, s);
  return s;
}

// Sum over the 8 lanes of a token group; all 8 lanes get identical bits.
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp<DPP_QUAD_XOR1>(v);
  v += dpp<DPP_QUAD_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  return v;
}

__device__ __forceinline__ void unpack16(const u32x4_v (&va)[2], float (&out)[16]) {
  const uint32_t w[8] = {va[0].x, va[0].y, va[0].z, va[0].w, va[1].x, va[1].y, va[1].z, va[1].w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    out[2 * i] = bf16_lo(w[i]);
    out[2 * i + 1] = bf16_hi(w[i]);
  }
}

// Per-iteration register state of one lane: K and V halves of its TPL tokens.
template <int TPL>
struct TileRegs {
  u32x4_v k[TPL][2];
  u32x4_v v[TPL][2];
};

template <bool NT>
__device__ __forceinline__ u32x4_v ld16(const u32x4_v* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

// Token range [start, end) of partial slot y of a request, or false if the slot is empty.
// Slot y is segment j = y % sps of split s = y / sps, with sps = ceil(chunk / seg).
__host__ __device__ __forceinline__ bool segment_range(int seq_len, int n_splits, int fixed_split,
                                                       int seg, int y, int& start, int& end) {
  const int chunk = kv_per_split(seq_len, n_splits, fixed_split);
  const int sl = seg > 0 ? min(seg, chunk) : chunk;
  const int sps = ceil_div(chunk, sl);
  const int s = y / sps;
  if (s >= n_splits) return false;
  const int split_start = s * chunk;
  const int split_end = min(split_start + chunk, seq_len);
  start = split_start + (y % sps) * sl;
  end = min(start + sl, split_end);
  return start < end;
}

// LDS of one stage-1 workgroup: the waves' softmax states, then the merge's scales. The
// accumulators come first and the struct is 16-byte aligned, so their stores and the merge's
// reads are whole 16-byte LDS accesses (with a 4-byte-aligned struct the compiler splits
// them into 4-byte pairs: one request of 1024 tokens took 9.3 -> 10.0 us).
template <int NW>
struct alignas(16) Stage1Lds {
  float acc[NW][HQ][HEAD_DIM];
  float m[NW][HQ];
  float l[NW][HQ];
  float sc[NW][HQ];
  float den[HQ];
  float mx[HQ];
};

// The partial attention of request b over partial slot y (a segment of one split), by one
// workgroup of NW waves taking TPL tokens per wave iteration. Every exit is
// workgroup-uniform. The next iteration's slot indices load while this one's rows are in
// flight (a long segment of a small batch is a chain of iterations: fixed-256 at B = 1, ctx
// 1024 26.8 -> 23.7 us; no change on full grids). (Software-pipelined forms with the next
// iteration's rows loading during this one's math measured no faster.)
template <int NW, int TPL>
__device__ __forceinline__ void stage1_item(
    Stage1Lds<NW>& sh, int b, int y, const bf16_t* __restrict__ q,
    const bf16_t* __restrict__ k_cache, const bf16_t* __restrict__ v_cache,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ num_splits, int max_splits, int fixed_split, int seg,
    float sm_scale, int64_t num_slots, int part_stride, float* __restrict__ part_o,
    float* __restrict__ part_lse, bf16_t* __restrict__ o_direct) {
  constexpr int IT = NW * TPL;  // tokens per workgroup iteration
  const int tid = threadIdx.x;
  // Wave index as a wave-uniform value: token positions derived from it are uniform, so
  // slot indices come in through scalar loads with no per-lane branches.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int grp = lane >> 3;  // kv head
  const int sub = lane & 7;

  const int kv_base = kv_indptr[b];
  const int seq_len = kv_indptr[b + 1] - kv_base;
  const int n_splits = num_splits != nullptr ? num_splits[b]
                                             : derived_splits(seq_len, max_splits, fixed_split);

  auto& s_m = sh.m;
  auto& s_l = sh.l;
  auto& s_acc = sh.acc;

  const int64_t out_row = static_cast<int64_t>(b) * HQ;
  // A slot with no tokens marks itself empty (log-sum-exp NEG_BIG): every slot below the
  // grid's slot count is written on every call, so stage 2 can tell used slots from the
  // log-sum-exps alone.
  auto mark_empty = [&]() {
    if (o_direct == nullptr && tid < HQ) part_lse[(out_row + tid) * part_stride + y] = NEG_BIG;
  };
  if (n_splits <= 0 || seq_len <= 0) {
    // Empty request: stage 2 would write zeros (flash_decode.cu:246-249).
    if (o_direct != nullptr && y == 0) {
      for (int i = tid; i < HQ * HEAD_DIM; i += NW * 64) o_direct[out_row * HEAD_DIM + i] = 0;
    }
    mark_empty();
    return;
  }
  int start, end;
  if (!segment_range(seq_len, n_splits, fixed_split, seg, y, start, end)) {
    mark_empty();
    return;
  }

  // Query heads 2*grp and 2*grp+1, packed bf16: lane `sub` holds the dims it owns.
  u32x4_v qv[QPK][2];
  {
    const u32x4_v* qb = reinterpret_cast<const u32x4_v*>(q + (out_row + QPK * grp) * HEAD_DIM);
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
      qv[h][0] = qb[h * (HEAD_DIM / 8) + sub];
      qv[h][1] = qb[h * (HEAD_DIM / 8) + 8 + sub];
    }
  }

  float m[QPK], l[QPK], acc[QPK][16];
#pragma unroll
  for (int h = 0; h < QPK; ++h) {
    m[h] = NEG_BIG;
    l[h] = 0.0f;
#pragma unroll
    for (int d = 0; d < 16; ++d) acc[h][d] = 0.0f;
  }

  const int32_t* idx = kv_indices + kv_base;
  const bf16_t* kbase = k_cache + grp * HEAD_DIM;
  const bf16_t* vbase = v_cache + grp * HEAD_DIM;
  constexpr int64_t kRow = static_cast<int64_t>(HKV) * HEAD_DIM;  // pool row, elements

  // Rows of the TPL tokens from t0. Positions past the segment end load the segment's last
  // token instead (real, finite data) and are flagged invalid: they get weight 0 below.
  // No branch guards a load, so all index loads issue before the first is waited for.
  auto load_idx = [&](int t0, int32_t (&raw)[TPL]) {
#pragma unroll
    for (int t = 0; t < TPL; ++t) raw[t] = idx[min(t0 + t, end - 1)];
  };
  auto load_tile = [&](int t0, const int32_t (&raw)[TPL], bool (&ok)[TPL], TileRegs<TPL>& r) {
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      int64_t sv = static_cast<int64_t>(raw[t]);
      if (sv < 0 || sv >= num_slots) sv = 0;
      ok[t] = t0 + t < end;
      const u32x4_v* kp = reinterpret_cast<const u32x4_v*>(kbase + sv * kRow);
      const u32x4_v* vp = reinterpret_cast<const u32x4_v*>(vbase + sv * kRow);
      r.k[t][0] = ld16<kNonTemporal>(kp + sub);
      r.k[t][1] = ld16<kNonTemporal>(kp + 8 + sub);
      r.v[t][0] = ld16<kNonTemporal>(vp + sub);
      r.v[t][1] = ld16<kNonTemporal>(vp + 8 + sub);
    }
    // Keep the scheduler from sinking these loads into the math that consumes them (it
    // would otherwise reuse one token's registers and serialise the TPL round trips).
    __builtin_amdgcn_sched_barrier(0);
  };
  auto compute = [&](const bool (&ok)[TPL], const TileRegs<TPL>& r) {
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
      float sc[TPL];
      float tmax = NEG_BIG;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        sc[t] = group8_sum(dot16(qv[h], r.k[t])) * sm_scale;
        if (ok[t]) tmax = fmaxf(tmax, sc[t]);
      }
      const float mn = fmaxf(m[h], tmax);
      const float rs = __expf(m[h] - mn);
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        sc[t] = ok[t] ? __expf(sc[t] - mn) : 0.0f;
        psum += sc[t];
      }
      l[h] = l[h] * rs + psum;
      m[h] = mn;
      // x * 1.0f == x: once the running maxima settle, no lane of the wave rescales, and the
      // 16 multiplies are skipped with identical bits.
      if (__builtin_amdgcn_ballot_w64(rs != 1.0f) != 0) {
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[h][d] *= rs;
      }
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        float vf[16];
        unpack16(r.v[t], vf);
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[h][d] += sc[t] * vf[d];
      }
    }
  };

  int32_t raw[TPL];
  load_idx(start + wave * TPL, raw);
  for (int t0 = start + wave * TPL; t0 < end; t0 += IT) {
    bool ok[TPL];
    TileRegs<TPL> r;
    load_tile(t0, raw, ok, r);
    load_idx(t0 + IT, raw);  // the next tile's slots load during this tile's rows and math
    compute(ok, r);
  }

#pragma unroll
  for (int h = 0; h < QPK; ++h) {
    const int hq = QPK * grp + h;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s_acc[wave][hq][8 * sub + j] = acc[h][j];
      s_acc[wave][hq][64 + 8 * sub + j] = acc[h][8 + j];
    }
    if (sub == 0) {
      s_m[wave][hq] = m[h];
      s_l[wave][hq] = l[h];
    }
  }
  __syncthreads();

  // Merge the waves in increasing wave order. A wave that saw no token of the segment has
  // m = NEG_BIG and l = 0 and drops out (its scale underflows). One thread per query head
  // takes the max over the waves, every wave's scale and the denominator once; then each
  // thread folds 4 consecutive dims of one head (128-bit LDS reads), with the same
  // per-output operations in the same order as folding every dim on its own.
  auto& s_sc = sh.sc;
  auto& s_den = sh.den;
  auto& s_mx = sh.mx;
  if (tid < HQ) {
    float mx = s_m[0][tid];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_m[w][tid]);
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float sc = __expf(s_m[w][tid] - mx);
      s_sc[w][tid] = sc;
      den += s_l[w][tid] * sc;
    }
    s_den[tid] = den;
    s_mx[tid] = mx;
  }
  __syncthreads();
  constexpr int Q4 = HEAD_DIM / 4;
  for (int i = tid; i < HQ * Q4; i += NW * 64) {
    const int h = i / Q4;
    const int d0 = (i % Q4) * 4;
    float num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float sc = s_sc[w][h];
      const float4 a = *reinterpret_cast<const float4*>(&s_acc[w][h][d0]);
      num[0] += a.x * sc;
      num[1] += a.y * sc;
      num[2] += a.z * sc;
      num[3] += a.w * sc;
    }
    const float den = s_den[h];
    const float4 out = make_float4(num[0] / den, num[1] / den, num[2] / den, num[3] / den);
    if (o_direct != nullptr) {
      *reinterpret_cast<uint2*>(&o_direct[(out_row + h) * HEAD_DIM + d0]) =
          make_uint2(pack_bf16x2(out.x, out.y), pack_bf16x2(out.z, out.w));
    } else {
      const int64_t prow = (out_row + h) * part_stride + y;
      *reinterpret_cast<float4*>(&part_o[prow * HEAD_DIM + d0]) = out;
      if (d0 == 0) part_lse[prow] = s_mx[h] + __logf(den);
    }
  }
}


// Grid form: workgroup (b, y) of a batch x grid_slots grid, or the entry of wg_order at its
// linear id (a permutation of the grid, heaviest segments first; only the placement changes,
// not what is computed).
template <int NW, int TPL>
__global__ void __launch_bounds__(NW * 64) decode_stage1_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ num_splits,
    int max_splits, int fixed_split, int seg, float sm_scale, int64_t num_slots, int part_stride,
    float* __restrict__ part_o, float* __restrict__ part_lse, bf16_t* __restrict__ o_direct,
    const int32_t* __restrict__ wg_order) {
  __shared__ Stage1Lds<NW> sh;
  int b = blockIdx.x;
  int y = blockIdx.y;
  if (wg_order != nullptr) {
    const int packed = wg_order[blockIdx.x + blockIdx.y * gridDim.x] & ~kOrderEmpty;
    b = packed >> kOrderSlotBits;
    y = packed & ((1 << kOrderSlotBits) - 1);
    if (b >= static_cast<int>(gridDim.x) || y >= static_cast<int>(gridDim.y)) return;
  }
  stage1_item<NW, TPL>(sh, b, y, q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                       max_splits, fixed_split, seg, sm_scale, num_slots, part_stride, part_o,
                       part_lse, o_direct);
}

// Worker form: `workers` workgroups, worker w computing the items order[w], order[w +
// workers], order[w + 2 workers], ... of the batch x grid_slots items (order: a permutation
// of them all, empty slots included, dealt so the workers' token counts balance). Each item
// is computed exactly as the grid form computes it, so only placement differs: the same bits.
// Entries with kOrderEmpty set are items known to hold no tokens, and in a worker's sequence
// they follow all of its other entries: from its first one on, the worker marks all of its
// remaining items empty in one pass of its threads (one order load and one log-sum-exp
// store each) instead of one dependent round trip per item.
// Every worker runs a bounded loop over its share and exits.
template <int NW, int TPL>
__global__ void __launch_bounds__(NW * 64) decode_stage1_worker_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ num_splits,
    int max_splits, int fixed_split, int seg, float sm_scale, int64_t num_slots, int part_stride,
    float* __restrict__ part_o, float* __restrict__ part_lse, const int32_t* __restrict__ order,
    int batch, int grid_slots) {
  __shared__ Stage1Lds<NW> sh;
  const int n_items = batch * grid_slots;
  const int W = static_cast<int>(gridDim.x);
  int i = static_cast<int>(blockIdx.x);
  for (; i < n_items; i += W) {
    const int packed = order[i];  // workgroup-uniform
    if (packed & kOrderEmpty) break;
    const int b = packed >> kOrderSlotBits;
    const int y = packed & ((1 << kOrderSlotBits) - 1);
    if (b < batch && y < grid_slots) {
      stage1_item<NW, TPL>(sh, b, y, q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                           max_splits, fixed_split, seg, sm_scale, num_slots, part_stride,
                           part_o, part_lse, nullptr);
    }
    __syncthreads();  // the item's merge reads of the LDS are done before the next item's writes
  }
  // The worker's remaining items i, i + W, ... (flagged empty): HQ markers each, one per
  // thread.
  const int rest = i < n_items ? (n_items - i + W - 1) / W : 0;
  for (int t = threadIdx.x; t < rest * HQ; t += NW * 64) {
    const int packed = order[i + (t / HQ) * W] & ~kOrderEmpty;
    const int b = packed >> kOrderSlotBits;
    const int y = packed & ((1 << kOrderSlotBits) - 1);
    if (b < batch && y < grid_slots)
      part_lse[(static_cast<int64_t>(b) * HQ + t % HQ) * part_stride + y] = NEG_BIG;
  }
}

// Stage 2: one workgroup per (query head, request), thread = output dim. The slots'
// log-sum-exps are staged in LDS in parallel (stage 1 writes every slot below grid_slots on
// every call: a partial, or NEG_BIG for a slot without tokens, so the request's geometry is
// not needed here); every thread then merges the non-empty slots sequentially in
// increasing slot order (increasing token order), as in sid/csrc/flash_decode.cu:231-273
// with segments in place of splits. A request with no used slot gets zeros
// (flash_decode.cu:246-249). The partial loads of different slots are independent, so they
// overlap.
constexpr int kMaxGridSlots = 1024;

__global__ void __launch_bounds__(HEAD_DIM) decode_stage2_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse, int grid_slots,
    int part_stride, bf16_t* __restrict__ o) {
  __shared__ float s_lse[kMaxGridSlots];
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t row = static_cast<int64_t>(b) * HQ + hq;
  const float* lse = part_lse + row * part_stride;
  const float* po = part_o + row * part_stride * HEAD_DIM;
  for (int y = d; y < grid_slots; y += HEAD_DIM) s_lse[y] = lse[y];
  __syncthreads();
  float mx = NEG_BIG;
  for (int y = 0; y < grid_slots; ++y) mx = fmaxf(mx, s_lse[y]);
  if (mx == NEG_BIG) {
    o[row * HEAD_DIM + d] = 0;
    return;
  }
  float num = 0.0f, den = 0.0f;
#pragma unroll 8
  for (int y = 0; y < grid_slots; ++y) {
    const float ly = s_lse[y];
    const bool valid = ly != NEG_BIG;
    const float pv = valid ? po[y * HEAD_DIM + d] : 0.0f;  // empty slots hold no data
    const float w = valid ? __expf(ly - mx) : 0.0f;
    num += w * pv;
    den += w;
  }
  o[row * HEAD_DIM + d] = f32_to_bf16(num / den);
}

// Stage 2 for grids of at most CAP slots (the common case): the same merge in the same
// order as decode_stage2_kernel, with every slot's partial load issued at once, before the
// log-sum-exps are even back (unused slots' partials are loaded, in bounds as part_stride >=
// grid_slots, and dropped by a select), so the workgroup makes one memory round trip where
// the loop above makes one per 8 slots after the log-sum-exp one. Config 3's shape (9 slots):
// attention 86.9 -> 86.4 us per layer, graph-timed.
template <int CAP>
__global__ void __launch_bounds__(HEAD_DIM) decode_stage2_fixed_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse, int grid_slots,
    int part_stride, bf16_t* __restrict__ o) {
  __shared__ float s_lse[CAP];
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t row = static_cast<int64_t>(b) * HQ + hq;
  const float* lse = part_lse + row * part_stride;
  const float* po = part_o + row * part_stride * HEAD_DIM;
  float pv[CAP];
#pragma unroll
  for (int y = 0; y < CAP; ++y) pv[y] = y < grid_slots ? po[y * HEAD_DIM + d] : 0.0f;
  if (d < grid_slots) s_lse[d] = lse[d];
  __syncthreads();
  float mx = NEG_BIG;
#pragma unroll
  for (int y = 0; y < CAP; ++y)
    if (y < grid_slots) mx = fmaxf(mx, s_lse[y]);
  if (mx == NEG_BIG) {
    o[row * HEAD_DIM + d] = 0;
    return;
  }
  float num = 0.0f, den = 0.0f;
#pragma unroll
  for (int y = 0; y < CAP; ++y) {
    if (y < grid_slots) {
      const float ly = s_lse[y];
      const bool valid = ly != NEG_BIG;
      const float p = valid ? pv[y] : 0.0f;
      const float w = valid ? __expf(ly - mx) : 0.0f;
      num += w * p;
      den += w;
    }
  }
  o[row * HEAD_DIM + d] = f32_to_bf16(num / den);
}

// Stage 2 for batches of at most kLatencyBatch requests (at most 64 workgroups, so latency,
// not throughput, is the cost): the same merge in the same order, with the loads of a chunk
// of kChunk slots (log-sum-exp and partial) all issued at once and nothing loaded before
// them: stage 1 marks the slots it leaves empty (log-sum-exp NEG_BIG), so the used slots
// are known from the log-sum-exps and the kernel makes one dependent round trip, where
// decode_stage2_kernel takes one for the log-sum-exps (staged in LDS) and then one per 8
// slots. Unused slots' partials are loaded (in bounds: part_stride >= grid_slots) and
// dropped by a select. Measured: one request of 1024 tokens (32 slots) 11.5 -> 10.7 us per
// call; from 8 requests up it is slower than decode_stage2_kernel (more code per slot,
// 1 us at B = 64, 7 us at B = 256).
constexpr int kChunk = 32;
constexpr int kLatencyBatch = 4;

__global__ void __launch_bounds__(HEAD_DIM) decode_stage2_latency_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse, int grid_slots,
    int part_stride, bf16_t* __restrict__ o) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t row = static_cast<int64_t>(b) * HQ + hq;
  const float* lse = part_lse + row * part_stride;
  const float* po = part_o + row * part_stride * HEAD_DIM;
  float mx = NEG_BIG;
  float num = 0.0f, den = 0.0f;
  // Pass 1 finds the max over the used slots; when the grid fits one chunk (the common
  // case) the chunk's values stay in registers for pass 2.
  float lv[kChunk], pv[kChunk];
  for (int c0 = 0; c0 < grid_slots; c0 += kChunk) {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      lv[j] = c0 + j < grid_slots ? lse[c0 + j] : NEG_BIG;
    }
#pragma unroll
    for (int j = 0; j < kChunk; ++j) mx = fmaxf(mx, lv[j]);
  }
  if (mx == NEG_BIG) {  // empty request (flash_decode.cu:246-249)
    o[row * HEAD_DIM + d] = 0;
    return;
  }
  for (int c0 = 0; c0 < grid_slots; c0 += kChunk) {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      if (grid_slots > kChunk) lv[j] = c0 + j < grid_slots ? lse[c0 + j] : NEG_BIG;
      pv[j] = c0 + j < grid_slots ? po[(c0 + j) * HEAD_DIM + d] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const bool valid = lv[j] != NEG_BIG;
      const float w = valid ? __expf(lv[j] - mx) : 0.0f;
      num += w * (valid ? pv[j] : 0.0f);
      den += w;
    }
  }
  o[row * HEAD_DIM + d] = f32_to_bf16(num / den);
}

// Stage-1 shapes (waves per workgroup x tokens per wave iteration). They fix the in-segment
// reduction order, so the bits of a result depend on the shape; every shape is a constant of
// the call (sid_flash_decode_segments_fwd's `variant`), never of the data.
//   0: 4 x 4  the default (the reference-signature entry points, batch_invariant)
//   1: 4 x 1  fewest registers, 4 waves/SIMD: best when the grid is full and HBM-bound
//   2: 8 x 2  half the per-wave round trips of a segment: best when fewer workgroups than CUs
//   3: 4 x 2  between the two: grids of one to two workgroups per CU
// (measured on 20 batch shapes, uniform and lognormal lengths, B = 1..256).
constexpr int kNumVariants = 4;

int launch_decode(const void* q, const void* k_cache, const void* v_cache,
                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* num_splits,
                  int max_splits, int batch, int64_t num_slots, int fixed_split_size, int seg,
                  int grid_slots, float sm_scale, float* part_o, float* part_lse, int part_stride, void* o,
                  int variant, const int32_t* wg_order, int workers, hipStream_t s) {
  const bool direct = (grid_slots == 1);
  auto stage1 = [&](auto kern, int nw) {
    hipLaunchKernelGGL(kern, dim3(batch, grid_slots), dim3(nw * 64), 0, s, (const bf16_t*)q,
                       (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_indptr, kv_indices,
                       num_splits, max_splits, fixed_split_size, seg, sm_scale, num_slots, part_stride, part_o,
                       part_lse, direct ? (bf16_t*)o : nullptr, wg_order);
  };
  auto worker = [&](auto kern, int nw) {
    hipLaunchKernelGGL(kern, dim3(workers), dim3(nw * 64), 0, s, (const bf16_t*)q,
                       (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_indptr, kv_indices,
                       num_splits, max_splits, fixed_split_size, seg, sm_scale, num_slots,
                       part_stride, part_o, part_lse, wg_order, batch, grid_slots);
  };
  if (workers == 0 || direct) {
    switch (variant) {
      case 1: stage1(decode_stage1_kernel<4, 1>, 4); break;
      case 2: stage1(decode_stage1_kernel<8, 2>, 8); break;
      case 3: stage1(decode_stage1_kernel<4, 2>, 4); break;
      default: stage1(decode_stage1_kernel<4, 4>, 4); break;
    }
  } else {
    switch (variant) {
      case 1: worker(decode_stage1_worker_kernel<4, 1>, 4); break;
      case 2: worker(decode_stage1_worker_kernel<8, 2>, 8); break;
      case 3: worker(decode_stage1_worker_kernel<4, 2>, 4); break;
      default: worker(decode_stage1_worker_kernel<4, 4>, 4); break;
    }
  }
  int rc = check_launch("flash_decode_fwd stage1");
  if (rc != SID_OK || direct) return rc;
  if (batch <= kLatencyBatch) {
    hipLaunchKernelGGL(decode_stage2_latency_kernel, dim3(HQ, batch), dim3(HEAD_DIM), 0, s,
                       part_o, part_lse, grid_slots, part_stride, (bf16_t*)o);
  } else if (grid_slots <= 32) {
    auto fixed = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(HQ, batch), dim3(HEAD_DIM), 0, s, part_o, part_lse,
                         grid_slots, part_stride, (bf16_t*)o);
    };
    if (grid_slots <= 4) fixed(decode_stage2_fixed_kernel<4>);
    else if (grid_slots <= 8) fixed(decode_stage2_fixed_kernel<8>);
    else if (grid_slots <= 12) fixed(decode_stage2_fixed_kernel<12>);
    else if (grid_slots <= 16) fixed(decode_stage2_fixed_kernel<16>);
    else if (grid_slots <= 24) fixed(decode_stage2_fixed_kernel<24>);
    else fixed(decode_stage2_fixed_kernel<32>);
  } else {
    hipLaunchKernelGGL(decode_stage2_kernel, dim3(HQ, batch), dim3(HEAD_DIM), 0, s, part_o,
                       part_lse, grid_slots, part_stride, (bf16_t*)o);
  }
  return check_launch("flash_decode_fwd stage2");
}

int check_decode_args(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* kv_indptr, const int32_t* kv_indices,
                      const int32_t* num_splits, void* o, int batch, int num_q_heads,
                      int num_kv_heads, int head_dim, int64_t num_slots, int max_splits,
                      int fixed_split_size) {
  SID_REQUIRE(q && k_cache && v_cache && kv_indptr && kv_indices && o,
              "flash_decode_fwd: null pointer");
  SID_REQUIRE(head_dim == HEAD_DIM, "flash_decode_fwd: head_dim must be %d, got %d", HEAD_DIM,
              head_dim);
  SID_REQUIRE(num_kv_heads == HKV && num_q_heads == HQ,
              "flash_decode_fwd: expected %d q heads and %d kv heads (got %d q, %d kv)", HQ, HKV,
              num_q_heads, num_kv_heads);
  SID_REQUIRE(num_slots > 0, "flash_decode_fwd: empty KV pool");
  SID_REQUIRE(max_splits >= 1 && max_splits <= kMaxGridSlots,
              "flash_decode_fwd: max_splits %d out of range [1, %d]", max_splits, kMaxGridSlots);
  SID_REQUIRE(fixed_split_size >= 0, "flash_decode_fwd: negative fixed_split_size");
  SID_REQUIRE(batch <= (1 << 30), "flash_decode_fwd: batch %d too large", batch);
  return SID_OK;
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_flash_decode_workers_fwd(
    const void* q, const void* k_cache, const void* v_cache, const int32_t* kv_indptr,
    const int32_t* kv_indices, const int32_t* num_splits, int batch, int num_q_heads,
    int num_kv_heads, int head_dim, int64_t num_slots, int max_splits, int fixed_split_size,
    int segment_size, int grid_slots, int variant, const int32_t* wg_order, float sm_scale,
    float* part_o, float* part_lse, int part_batch, int part_stride, void* o, int workers,
    void* stream) {
  SID_REQUIRE(batch >= 0, "flash_decode_fwd: negative batch");
  SID_REQUIRE(variant >= 0 && variant < kNumVariants, "flash_decode_fwd: unknown variant %d",
              variant);
  if (batch == 0) return SID_OK;
  int rc = check_decode_args(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits, o, batch,
                             num_q_heads, num_kv_heads, head_dim, num_slots, max_splits,
                             fixed_split_size);
  if (rc != SID_OK) return rc;
  SID_REQUIRE(segment_size >= 0, "flash_decode_fwd: negative segment_size");
  SID_REQUIRE(grid_slots >= 1 && grid_slots <= kMaxGridSlots,
              "flash_decode_fwd: grid_slots %d out of range [1, %d]", grid_slots, kMaxGridSlots);
  SID_REQUIRE(batch < (1 << (30 - kOrderSlotBits)) && kMaxGridSlots <= (1 << kOrderSlotBits),
              "flash_decode_fwd: batch %d too large for the workgroup order", batch);
  SID_REQUIRE(workers >= 0 && workers <= (1 << 20), "flash_decode_fwd: workers %d out of range",
              workers);
  SID_REQUIRE(workers == 0 || wg_order != nullptr,
              "flash_decode_fwd: a worker launch needs the item order (wg_order)");
  if (grid_slots > 1) {
    SID_REQUIRE(part_o && part_lse, "flash_decode_fwd: null workspace");
    SID_REQUIRE(part_batch >= batch && part_stride >= grid_slots,
                "flash_decode_fwd: part_o workspace too small / wrong shape "
                "(part_batch %d, part_stride %d, batch %d, grid_slots %d)",
                part_batch, part_stride, batch, grid_slots);
  }
  return launch_decode(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits, max_splits, batch,
                       num_slots, fixed_split_size, segment_size, grid_slots, sm_scale, part_o, part_lse,
                       part_stride, o, variant, wg_order, workers,
                       static_cast<hipStream_t>(stream));
}

extern "C" int sid_flash_decode_segments_fwd(
    const void* q, const void* k_cache, const void* v_cache, const int32_t* kv_indptr,
    const int32_t* kv_indices, const int32_t* num_splits, int batch, int num_q_heads,
    int num_kv_heads, int head_dim, int64_t num_slots, int max_splits, int fixed_split_size,
    int segment_size, int grid_slots, int variant, const int32_t* wg_order, float sm_scale,
    float* part_o, float* part_lse, int part_batch, int part_stride, void* o, void* stream) {
  return sid_flash_decode_workers_fwd(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                                      batch, num_q_heads, num_kv_heads, head_dim, num_slots,
                                      max_splits, fixed_split_size, segment_size, grid_slots,
                                      variant, wg_order, sm_scale, part_o, part_lse, part_batch,
                                      part_stride, o, 0, stream);
}

extern "C" int sid_flash_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* num_splits, int batch, int num_q_heads,
                                    int num_kv_heads, int head_dim, int64_t num_slots,
                                    int max_splits, int fixed_split_size, float sm_scale,
                                    float* part_o, float* part_lse, int part_batch,
                                    int part_stride, void* o, void* stream) {
  SID_REQUIRE(batch <= 0 || num_splits != nullptr, "flash_decode_fwd: null num_splits");
  // One segment per split: the grid has exactly the reference's max_splits slots.
  return sid_flash_decode_segments_fwd(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits,
                                       batch, num_q_heads, num_kv_heads, head_dim, num_slots,
                                       max_splits, fixed_split_size, 0, max_splits, 0, nullptr,
                                       sm_scale, part_o, part_lse, part_batch, part_stride, o,
                                       stream);
}

// ---- allocation-free entry point ------------------------------------------------------
//
// Split partials in a file-scope device array instead of a caller workspace, for callers
// that cannot allocate. Each GPU the library runs on holds its own copy for the life of the
// process. Host code never passes the array's name to a kernel (on the host it is only a
// stand-in symbol): the device address comes from hipGetSymbolAddress, once per device,
// with that device current.
namespace sid {
namespace {

constexpr int64_t kScratchBytes = SID_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

int scratch_for_current_device(unsigned char** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  SID_REQUIRE(err == hipSuccess, "flash_decode_fwd_noalloc: hipGetDevice failed: %s",
              hipGetErrorString(err));
  SID_REQUIRE(dev >= 0 && dev < kMaxDevices, "flash_decode_fwd_noalloc: device %d out of range",
              dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    SID_REQUIRE(err == hipSuccess && ptr != nullptr,
                "flash_decode_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
  return SID_OK;
}

}  // namespace
}  // namespace sid

extern "C" int64_t sid_flash_decode_noalloc_scratch_bytes(void) { return sid::kScratchBytes; }

extern "C" int sid_flash_decode_segments_fwd_noalloc(
    const void* q, const void* k_cache, const void* v_cache, const int32_t* kv_indptr,
    const int32_t* kv_indices, const int32_t* num_splits, int batch, int num_q_heads,
    int num_kv_heads, int head_dim, int64_t num_slots, int max_splits, int fixed_split_size,
    int segment_size, int grid_slots, int variant, const int32_t* wg_order, float sm_scale,
    void* o, void* stream) {
  using namespace sid;
  SID_REQUIRE(batch >= 0, "flash_decode_fwd_noalloc: negative batch");
  SID_REQUIRE(variant >= 0 && variant < kNumVariants,
              "flash_decode_fwd_noalloc: unknown variant %d", variant);
  if (batch == 0) return SID_OK;
  int rc = check_decode_args(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits, o, batch,
                             num_q_heads, num_kv_heads, head_dim, num_slots, max_splits,
                             fixed_split_size);
  if (rc != SID_OK) return rc;
  SID_REQUIRE(segment_size >= 0, "flash_decode_fwd_noalloc: negative segment_size");
  SID_REQUIRE(grid_slots >= 1 && grid_slots <= kMaxGridSlots,
              "flash_decode_fwd_noalloc: grid_slots %d out of range [1, %d]", grid_slots,
              kMaxGridSlots);
  // partials: part_o [batch][HQ][grid_slots][D] fp32, then part_lse [batch][HQ][grid_slots]
  const int64_t o_bytes = (int64_t)batch * HQ * grid_slots * HEAD_DIM * 4;
  const int64_t lse_off = (o_bytes + 255) / 256 * 256;
  const int64_t need = lse_off + (int64_t)batch * HQ * grid_slots * 4;
  SID_REQUIRE(grid_slots == 1 || need <= kScratchBytes,
              "flash_decode_fwd_noalloc: %lld bytes of split partials (batch %d x %d slots) "
              "exceed the %lld-byte scratch; use sid_flash_decode_segments_fwd with a "
              "workspace", (long long)need, batch, grid_slots, (long long)kScratchBytes);
  float* part_o = nullptr;
  float* part_lse = nullptr;
  if (grid_slots > 1) {
    unsigned char* base = nullptr;
    rc = scratch_for_current_device(&base);
    if (rc != SID_OK) return rc;
    part_o = reinterpret_cast<float*>(base);
    part_lse = reinterpret_cast<float*>(base + lse_off);
  }
  // Stage 2 reads only the slots stage 1 wrote in this call, so nothing is cleared.
  return launch_decode(q, k_cache, v_cache, kv_indptr, kv_indices, num_splits, max_splits, batch,
                       num_slots, fixed_split_size, segment_size, grid_slots, sm_scale, part_o, part_lse,
                       grid_slots, o, variant, wg_order, 0, static_cast<hipStream_t>(stream));
}
