// Split-KV paged decode attention for gfx950 (CDNA4, wave64).
//
// Stage 1: one workgroup per (kv head, request, split) computes the partial
// attention of BOTH query heads of the GQA pair (HQ = 2 * HKV) over the
// split's KV range, reading every K/V row once. Stage 2 merges the splits
// with the log-sum-exp rescale in fixed split order. Split geometry follows
// kv_per_split in sid/csrc/flash_decode.cu:56-60 exactly (it decides which
// tokens each split owns, so it must match the host-side policy of
// sid/kernels/decode_attention.py:56-85).
//
// Inside a split the work is laid out for wave64 and HBM streaming:
//   * a token's K (or V) row for one kv head is 256 bytes; 8 lanes cover it
//     with two 16-byte loads each (lane `sub` owns dims 8*sub..8*sub+7 and
//     64+8*sub..64+8*sub+7), so a wave has 8 token rows in flight per load
//     instruction and every load instruction fetches whole 128-byte lines;
//   * q.k uses v_dot2_f32_bf16 on the packed bf16 operands, reduced over the
//     8 lanes of a token with three DPP steps (every lane ends with the same
//     bits because each step adds a commutative pair);
//   * each 8-lane group keeps its own online-softmax state (running max m,
//     running sum l, fp32 accumulator for its 16 dims x 2 heads) over the
//     tokens it owns, so the hot loop has no cross-lane reduction beyond the
//     dot product. Groups are merged at the end inside the wave (lane
//     exchanges xor 8/16/32), then the waves through LDS, in a fixed order.
// The result is a fixed function of (request data, seq_len, num_splits):
// no atomics, no dependence on batch composition or scheduling.
#include "common.h"

namespace sid {
namespace {

constexpr int HEAD_DIM = 128;
constexpr int QPK = 2;              // query heads per kv head
constexpr int HEUR_TILE = 32;       // granularity of the heuristic split size
constexpr float NEG_BIG = -1e30f;   // finite "minus infinity" for running maxima

__host__ __device__ __forceinline__ int kv_per_split(int seq_len, int n_splits, int fixed_split) {
  if (fixed_split > 0) return fixed_split;
  return ceil_div(ceil_div(seq_len, n_splits), HEUR_TILE) * HEUR_TILE;
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

// Exchange-and-merge of two online-softmax states (lane <-> lane ^ mask).
template <int MASK>
__device__ __forceinline__ float xchg(float v) {
  if constexpr (MASK == 8) {
    return dpp<DPP_ROW_ROR8>(v);
  } else {
    return lane_xor(v, MASK);
  }
}

template <int MASK, int NH>
__device__ __forceinline__ void merge_with_partner(float (&m)[NH], float (&l)[NH],
                                                   float (&acc)[NH][16]) {
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const float mo = xchg<MASK>(m[h]);
    const float lo = xchg<MASK>(l[h]);
    const float mn = fmaxf(m[h], mo);
    const float a = __expf(m[h] - mn);
    const float c = __expf(mo - mn);
    l[h] = l[h] * a + lo * c;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      const float other = xchg<MASK>(acc[h][d]);
      acc[h][d] = acc[h][d] * a + other * c;
    }
    m[h] = mn;
  }
}

// Per-iteration register state of one lane: the pool slots of its TPL tokens
// and their K and V halves.
template <int TPL, int HPW>
struct TileRegs {
  u32x4_v k[TPL][HPW][2];
  u32x4_v v[TPL][HPW][2];
};

template <bool NT>
__device__ __forceinline__ u32x4_v ld16(const u32x4_v* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

// NW waves per workgroup; TPL tokens per lane group per iteration, so one
// wave iteration covers IT = 8 * TPL consecutive tokens of the split.
// PF: software pipeline inside each wave (slot indices fetched two iterations
// ahead, K/V rows one iteration ahead) so the index -> row dependent loads
// are off the critical path. NT: non-temporal K/V loads (streamed once).
// RF: request-fastest grid (blockIdx.x = request, blockIdx.y = kv head group), so the
// round-robin workgroup->XCD assignment keeps all heads of a request on one XCD;
// otherwise the kv head is fastest (every workgroup of head h on the same XCD).
// HPW: kv heads per workgroup; a lane group then reads HPW adjacent 256-byte head rows
// of a token (one contiguous HPW*256-byte run). Every head is reduced exactly as with
// HPW = 1, so HPW does not change any bit of the result.
template <int NW, int TPL, bool PF, bool NT, bool RF = false, int HPW = 1>
__global__ void __launch_bounds__(NW * 64) decode_stage1_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ num_splits,
    int fixed_split, float sm_scale, int num_kv_heads, int64_t num_slots, int part_stride,
    float* __restrict__ part_o, float* __restrict__ part_lse, bf16_t* __restrict__ o_direct) {
  constexpr int IT = 8 * TPL;
  constexpr int NH = HPW * QPK;  // query heads handled by this workgroup
  const int h_kv = (RF ? blockIdx.y : blockIdx.x) * HPW;  // first kv head
  const int b = RF ? blockIdx.x : blockIdx.y;
  const int split = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int grp = lane >> 3;
  const int sub = lane & 7;
  const int num_q_heads = num_kv_heads * QPK;

  const int kv_base = kv_indptr[b];
  const int seq_len = kv_indptr[b + 1] - kv_base;
  const int n_splits = num_splits[b];

  __shared__ float s_m[NW][NH];
  __shared__ float s_l[NW][NH];
  __shared__ float s_acc[NW][NH][HEAD_DIM];

  const int64_t out_row = static_cast<int64_t>(b) * num_q_heads + h_kv * QPK;
  if (n_splits <= 0 || seq_len <= 0) {
    // Empty request: stage 2 would write zeros (flash_decode.cu:246-249).
    if (o_direct != nullptr && split == 0) {
      for (int i = tid; i < NH * HEAD_DIM; i += NW * 64) o_direct[out_row * HEAD_DIM + i] = 0;
    }
    return;
  }
  if (split >= n_splits) return;
  const int chunk = kv_per_split(seq_len, n_splits, fixed_split);
  const int start = split * chunk;
  if (start >= seq_len) return;
  const int end = min(start + chunk, seq_len);

  // Query heads, packed bf16: lane `sub` holds the dims it owns for every head
  // (query head h uses kv head h / QPK of this workgroup).
  u32x4_v qv[NH][2];
  {
    const u32x4_v* qb = reinterpret_cast<const u32x4_v*>(q + out_row * HEAD_DIM);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      qv[h][0] = qb[h * (HEAD_DIM / 8) + sub];
      qv[h][1] = qb[h * (HEAD_DIM / 8) + 8 + sub];
    }
  }

  float m[NH], l[NH], acc[NH][16];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    m[h] = NEG_BIG;
    l[h] = 0.0f;
#pragma unroll
    for (int d = 0; d < 16; ++d) acc[h][d] = 0.0f;
  }

  const int n_it = ceil_div(end - start, IT);
  const int32_t* idx = kv_indices + kv_base;
  const int64_t row_stride = static_cast<int64_t>(num_kv_heads) * HEAD_DIM;
  const bf16_t* kbase = k_cache + h_kv * HEAD_DIM;
  const bf16_t* vbase = v_cache + h_kv * HEAD_DIM;

  // Slot of token t of iteration `it` for this lane (-1 = past the split's end).
  auto load_slots = [&](int it, int64_t (&sl)[TPL]) {
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      const int pos = start + it * IT + grp + 8 * t;
      int64_t s = -1;
      if (it < n_it && pos < end) {
        s = static_cast<int64_t>(idx[pos]);
        if (s < 0 || s >= num_slots) s = 0;
      }
      sl[t] = s;
    }
  };
  auto load_rows = [&](const int64_t (&sl)[TPL], TileRegs<TPL, HPW>& r) {
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        if (sl[t] >= 0) {
          const u32x4_v* kp =
              reinterpret_cast<const u32x4_v*>(kbase + sl[t] * row_stride + hh * HEAD_DIM);
          const u32x4_v* vp =
              reinterpret_cast<const u32x4_v*>(vbase + sl[t] * row_stride + hh * HEAD_DIM);
          r.k[t][hh][0] = ld16<NT>(kp + sub);
          r.k[t][hh][1] = ld16<NT>(kp + 8 + sub);
          r.v[t][hh][0] = ld16<NT>(vp + sub);
          r.v[t][hh][1] = ld16<NT>(vp + 8 + sub);
        } else {
          r.k[t][hh][0] = r.k[t][hh][1] = r.v[t][hh][0] = r.v[t][hh][1] = u32x4_v{0u, 0u, 0u, 0u};
        }
      }
    }
  };
  auto compute = [&](const int64_t (&sl)[TPL], const TileRegs<TPL, HPW>& r) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int hh = h / QPK;
      float s[TPL];
      float tmax = NEG_BIG;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        s[t] = group8_sum(dot16(qv[h], r.k[t][hh])) * sm_scale;
        if (sl[t] >= 0) tmax = fmaxf(tmax, s[t]);
      }
      const float mn = fmaxf(m[h], tmax);
      const float rs = __expf(m[h] - mn);
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        s[t] = sl[t] >= 0 ? __expf(s[t] - mn) : 0.0f;
        psum += s[t];
      }
      l[h] = l[h] * rs + psum;
      m[h] = mn;
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[h][d] *= rs;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        float vf[16];
        unpack16(r.v[t][hh], vf);
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[h][d] += s[t] * vf[d];
      }
    }
  };

  if constexpr (!PF) {
    for (int it = wave; it < n_it; it += NW) {
      int64_t sl[TPL];
      TileRegs<TPL, HPW> r;
      load_slots(it, sl);
      load_rows(sl, r);
      compute(sl, r);
    }
  } else {
    // Two register sets A/B alternate; slots run two iterations ahead of compute.
    int64_t sa[TPL], sb[TPL], sn[TPL];
    TileRegs<TPL, HPW> ra, rb;
    int it = wave;
    load_slots(it, sa);
    load_slots(it + NW, sb);
    load_rows(sa, ra);
    while (it < n_it) {
      load_rows(sb, rb);                // rows of it + NW
      load_slots(it + 2 * NW, sn);      // slots of it + 2*NW
      compute(sa, ra);                  // it
      it += NW;
      if (it >= n_it) break;
#pragma unroll
      for (int t = 0; t < TPL; ++t) sa[t] = sn[t];
      load_rows(sa, ra);                // rows of it + NW
      load_slots(it + 2 * NW, sn);      // slots of it + 2*NW
      compute(sb, rb);                  // it
      it += NW;
#pragma unroll
      for (int t = 0; t < TPL; ++t) sb[t] = sn[t];
    }
  }

  // Merge the 8 token groups of the wave: lane ^ 8, ^ 16, ^ 32 (fixed order).
  merge_with_partner<8, NH>(m, l, acc);
  merge_with_partner<16, NH>(m, l, acc);
  merge_with_partner<32, NH>(m, l, acc);

  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s_acc[wave][h][8 * sub + j] = acc[h][j];
        s_acc[wave][h][64 + 8 * sub + j] = acc[h][8 + j];
      }
      if (sub == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();

  // Merge the waves in increasing wave order; thread -> (head, dim).
  for (int i = tid; i < NH * HEAD_DIM; i += NW * 64) {
    const int h = i / HEAD_DIM;
    const int d = i % HEAD_DIM;
    float mx = s_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_m[w][h]);
    float den = 0.0f, num = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float sc = __expf(s_m[w][h] - mx);
      den += s_l[w][h] * sc;
      num += s_acc[w][h][d] * sc;
    }
    const float out = num / den;
    if (o_direct != nullptr) {
      o_direct[(out_row + h) * HEAD_DIM + d] = f32_to_bf16(out);
    } else {
      const int64_t prow = (out_row + h) * part_stride + split;
      part_o[prow * HEAD_DIM + d] = out;
      if (d == 0) part_lse[prow] = mx + __logf(den);
    }
  }
}

// Stage 2: thread = output dim; sequential merge over the request's valid
// splits (s * chunk < seq_len), as in sid/csrc/flash_decode.cu:231-273.
__global__ void __launch_bounds__(HEAD_DIM) decode_stage2_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ num_splits,
    int fixed_split, int max_splits, int num_q_heads, int part_stride, bf16_t* __restrict__ o) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t row = static_cast<int64_t>(b) * num_q_heads + hq;
  const int seq_len = kv_indptr[b + 1] - kv_indptr[b];
  const int n_splits = min(num_splits[b], max_splits);
  if (n_splits <= 0 || seq_len <= 0) {
    o[row * HEAD_DIM + d] = 0;
    return;
  }
  const int chunk = kv_per_split(seq_len, num_splits[b], fixed_split);
  const float* lse = part_lse + row * part_stride;
  const float* po = part_o + row * part_stride * HEAD_DIM;
  float mx = NEG_BIG;
  for (int s = 0; s < n_splits && s * chunk < seq_len; ++s) mx = fmaxf(mx, lse[s]);
  float num = 0.0f, den = 0.0f;
  for (int s = 0; s < n_splits && s * chunk < seq_len; ++s) {
    const float w = __expf(lse[s] - mx);
    num += w * po[s * HEAD_DIM + d];
    den += w;
  }
  o[row * HEAD_DIM + d] = f32_to_bf16(num / den);
}

// Production configuration (the bits of a result depend on NW and TPL, which fix the
// in-split reduction order; they are constants, independent of batch and policy).
constexpr int kWaves = 4;
constexpr int kTokPerLane = 4;
constexpr bool kPipelined = false;   // measured: no gain over 2 workgroups per CU
constexpr bool kNonTemporal = true;  // K/V rows are streamed once: +9% HBM throughput
constexpr bool kRequestFastest = true;

template <int NW, int TPL, bool PF, bool NT, bool RF = false, int HPW = 1>
int launch_decode(const void* q, const void* k_cache, const void* v_cache,
                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* num_splits,
                  int batch, int num_q_heads, int num_kv_heads, int64_t num_slots, int max_splits,
                  int fixed_split_size, float sm_scale, float* part_o, float* part_lse,
                  int part_stride, void* o, hipStream_t s) {
  const bool direct = (max_splits == 1);
  if (num_kv_heads % HPW != 0) {
    set_error("flash_decode_fwd: %d kv heads not divisible by %d heads per workgroup",
              num_kv_heads, HPW);
    return SID_ERR_INVALID;
  }
  const int groups = num_kv_heads / HPW;
  const dim3 grid1 = RF ? dim3(batch, groups, max_splits) : dim3(groups, batch, max_splits);
  hipLaunchKernelGGL((decode_stage1_kernel<NW, TPL, PF, NT, RF, HPW>), grid1, dim3(NW * 64), 0, s,
                     (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_indptr,
                     kv_indices, num_splits, fixed_split_size, sm_scale, num_kv_heads, num_slots,
                     part_stride, part_o, part_lse, direct ? (bf16_t*)o : nullptr);
  int rc = check_launch("flash_decode_fwd stage1");
  if (rc != SID_OK || direct) return rc;
  const dim3 grid2(num_q_heads, batch);
  hipLaunchKernelGGL(decode_stage2_kernel, grid2, dim3(HEAD_DIM), 0, s, part_o, part_lse,
                     kv_indptr, num_splits, fixed_split_size, max_splits, num_q_heads,
                     part_stride, (bf16_t*)o);
  return check_launch("flash_decode_fwd stage2");
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_flash_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* num_splits, int batch, int num_q_heads,
                                    int num_kv_heads, int head_dim, int64_t num_slots,
                                    int max_splits, int fixed_split_size, float sm_scale,
                                    float* part_o, float* part_lse, int part_batch,
                                    int part_stride, void* o, void* stream) {
  SID_REQUIRE(batch >= 0, "flash_decode_fwd: negative batch");
  if (batch == 0) return SID_OK;
  SID_REQUIRE(q && k_cache && v_cache && kv_indptr && kv_indices && num_splits && o,
              "flash_decode_fwd: null pointer");
  SID_REQUIRE(head_dim == HEAD_DIM, "flash_decode_fwd: head_dim must be %d, got %d", HEAD_DIM,
              head_dim);
  SID_REQUIRE(num_kv_heads > 0 && num_q_heads == QPK * num_kv_heads,
              "flash_decode_fwd: expected %d q heads per kv head (got %d q, %d kv)", QPK,
              num_q_heads, num_kv_heads);
  SID_REQUIRE(num_slots > 0, "flash_decode_fwd: empty KV pool");
  SID_REQUIRE(max_splits >= 1 && max_splits <= 65535, "flash_decode_fwd: max_splits %d out of range",
              max_splits);
  SID_REQUIRE(fixed_split_size >= 0, "flash_decode_fwd: negative fixed_split_size");
  SID_REQUIRE(batch <= 65535, "flash_decode_fwd: batch %d exceeds the grid limit", batch);
  const bool direct = (max_splits == 1);
  if (!direct) {
    SID_REQUIRE(part_o && part_lse, "flash_decode_fwd: null workspace");
    SID_REQUIRE(part_batch >= batch && part_stride >= max_splits,
                "flash_decode_fwd: part_o workspace too small / wrong shape "
                "(part_batch %d, part_stride %d, batch %d, max_splits %d)",
                part_batch, part_stride, batch, max_splits);
  }
  return launch_decode<kWaves, kTokPerLane, kPipelined, kNonTemporal, kRequestFastest>(
      q, k_cache, v_cache, kv_indptr, kv_indices, num_splits, batch, num_q_heads, num_kv_heads,
      num_slots, max_splits, fixed_split_size, sm_scale, part_o, part_lse, part_stride, o,
      static_cast<hipStream_t>(stream));
}
