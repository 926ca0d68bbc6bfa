// Greedy token selection: per-row argmax over the fp32 logits with torch's
// semantics (first index among equal maxima; NaN counts as the maximum, the
// first NaN wins). The (value, index) order used below is total, so the
// result does not depend on the reduction tree.
#include "common.h"

namespace sid {
namespace {

__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v;
  const bool bn = bv != bv;
  if (vn || bn) {
    if (vn && bn) return i < bi;
    return vn;
  }
  return v > bv || (v == bv && i < bi);
}

// ---- stochastic sampling (temperature / top-k / top-p / seeded Gumbel-max) ---------------
//
// One 1024-thread workgroup per row; the reference's sample() (sid/engine/sampler.py:32-69)
// with its truncation made exact:
//   temperature <= 0: the greedy argmax (first index, NaN wins), as argmax_kernel.
//   otherwise p = softmax(logits / T) (max, then the sum of exp(x - max) in a fixed order,
//   p = exp(x - max) / sum); tokens are ranked by (p descending, index ascending); rank r is
//   kept iff r < top_k (top_k <= 0: no limit) and the probability mass of the ranks before
//   it is <= top_p (top_p >= 1: no limit); rank 0 is always kept. The draw is
//   argmax over kept tokens of log(p + 1e-10) + gumbel(seed, position, token), with the
//   reference's int64 hash (sid/engine/sampler.py:22-29) and first-index ties.
// The mass before a rank is accumulated in 64-bit fixed point (units of 2^-48, each p
// rounded down), so it is an exact integer sum: the cut does not depend on any summation
// order. (The reference sums a float cumsum in sorted order; the two differ only when the
// mass lands within rounding of top_p.) The cut is found without sorting: p >= 0, so the
// bits of p order like p, and a 4-level 8-bit radix select over those bits, with LDS
// histograms of (count, fixed-point mass), descends to the key of the last kept rank; the
// keys of the row are written once to the workspace (only when a limit applies: with no
// top-k / top-p limit every token is kept and the draw reads p straight from the logits).
// Equal keys at the cut are ranked by index with a block-wide scan.
constexpr int kSampleThreads = 1024;
constexpr int kSampleWaves = kSampleThreads / 64;
constexpr double kMassUnit = 281474976710656.0;  // 2^48
constexpr int kHistCopies = 16;

__device__ __forceinline__ uint64_t mass_of(uint32_t key) {
  return static_cast<uint64_t>(static_cast<double>(__uint_as_float(key)) * kMassUnit);
}

// Calls f(value, column) for every column of a row: 16-byte loads, UNROLL of them in flight
// per thread, when the row is 16-byte aligned (else one element per load). Which thread sees
// which column is fixed by the row's alignment and length alone.
template <int UNROLL, typename F>
__device__ __forceinline__ void for_each_col(const float* __restrict__ row, int cols, F&& f) {
  const int tid = threadIdx.x;
  int vec = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const float4* row4 = reinterpret_cast<const float4*>(row);
    const int n4 = cols >> 2;
    constexpr int kStep = kSampleThreads * UNROLL;
    int base = 0;
    for (; base + kStep <= n4; base += kStep) {
      float4 v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = row4[base + u * kSampleThreads + tid];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int c = 4 * (base + u * kSampleThreads + tid);
        f(v[u].x, c);
        f(v[u].y, c + 1);
        f(v[u].z, c + 2);
        f(v[u].w, c + 3);
      }
    }
    // The rest (fewer than kStep vectors) in one more pass with every load issued first; a
    // thread visits the same columns in the same order as a loop over them would.
    if (base < n4) {
      float4 v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int i = base + u * kSampleThreads + tid;
        if (i < n4) v[u] = row4[i];
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int i = base + u * kSampleThreads + tid;
        if (i < n4) {
          f(v[u].x, 4 * i);
          f(v[u].y, 4 * i + 1);
          f(v[u].z, 4 * i + 2);
          f(v[u].w, 4 * i + 3);
        }
      }
    }
    vec = 4 * n4;
  }
  for (int c = vec + tid; c < cols; c += kSampleThreads) f(row[c], c);
}

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int mask = 1; mask < 64; mask <<= 1) v = fmaxf(v, lane_xor(v, mask));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kSampleWaves; ++w) r = fmaxf(r, red[w]);
  return r;
}

// Fixed-order float sum: xor butterfly inside each wave, then the waves in order.
__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int mask = 1; mask < 64; mask <<= 1) v += lane_xor(v, mask);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kSampleWaves; ++w) r += red[w];
  return r;
}

// Best (value, index) of the block under better(); every thread gets the result.
__device__ __forceinline__ void block_best(float& bv, int64_t& bi, float* s_v, int64_t* s_i) {
  for (int mask = 1; mask < 64; mask <<= 1) {
    const float ov = lane_xor(bv, mask);
    const int lo = __builtin_amdgcn_ds_bpermute((__lane_id() ^ mask) << 2, static_cast<int>(bi));
    const int hi = __builtin_amdgcn_ds_bpermute((__lane_id() ^ mask) << 2, static_cast<int>(bi >> 32));
    const int64_t oi = (static_cast<int64_t>(hi) << 32) | static_cast<uint32_t>(lo);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = bv;
    s_i[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  bv = s_v[0];
  bi = s_i[0];
  for (int w = 1; w < kSampleWaves; ++w) {
    if (better(s_v[w], s_i[w], bv, bi)) {
      bv = s_v[w];
      bi = s_i[w];
    }
  }
}

// Greedy argmax of one row per workgroup.
__global__ void __launch_bounds__(kSampleThreads) argmax_kernel(const float* __restrict__ logits,
                                                                int64_t ld, int64_t* __restrict__ out,
                                                                int64_t cols) {
  __shared__ float s_bv[kSampleWaves];
  __shared__ int64_t s_bi[kSampleWaves];
  const float* row = logits + static_cast<int64_t>(blockIdx.x) * ld;
  float bv = -INFINITY;
  int64_t bi = cols;  // sentinel larger than any index
  for_each_col<8>(row, static_cast<int>(cols), [&](float v, int c) {
    if (better(v, c, bv, bi)) {
      bv = v;
      bi = c;
    }
  });
  block_best(bv, bi, s_bv, s_bi);
  if (threadIdx.x == 0) out[blockIdx.x] = bi < cols ? bi : 0;
}

__global__ void __launch_bounds__(kSampleThreads) sample_kernel(
    const float* __restrict__ logits, int64_t ld, const float* __restrict__ temps,
    const int64_t* __restrict__ top_ks, const float* __restrict__ top_ps,
    const int64_t* __restrict__ seeds, const int64_t* __restrict__ positions, int64_t cols,
    uint32_t* __restrict__ keys_ws, int64_t* __restrict__ out) {
  // Radix histograms, one copy per lane & 15 (so at most 4 lanes of a wave instruction can
  // hit one address); rows padded to 257 entries so equal bins of different copies fall in
  // different LDS banks.
  __shared__ uint32_t h_cnt[kHistCopies][257];
  __shared__ uint64_t h_mass[kHistCopies][257];
  __shared__ float s_red[kSampleWaves];
  __shared__ float s_bv[kSampleWaves];
  __shared__ int64_t s_bi[kSampleWaves];
  __shared__ int64_t s_scan[kSampleThreads];
  __shared__ uint64_t s_sel[4];  // prefix, count above, mass above, count in final bin
  __shared__ int64_t s_cut;

  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int copy = tid & (kHistCopies - 1);
  const int ncols = static_cast<int>(cols);
  const float* row = logits + r * ld;
  const float t = temps[r];

  float bv = -INFINITY;
  int64_t bi = cols;
  if (!(t > 0.0f)) {  // greedy row
    for_each_col<8>(row, ncols, [&](float v, int c) {
      if (better(v, c, bv, bi)) {
        bv = v;
        bi = c;
      }
    });
    block_best(bv, bi, s_bv, s_bi);
    if (tid == 0) out[r] = bi < cols ? bi : 0;
    return;
  }

  // softmax of logits / t. Division by t > 0 is monotone (correct rounding preserves
  // order), so max(x / t) = max(x) / t and the first pass needs no division.
  float mx = -INFINITY;
  for_each_col<8>(row, ncols, [&](float v, int) { mx = fmaxf(mx, v); });
  mx = block_max(mx, s_red) / t;
  float part = 0.0f;
  for_each_col<4>(row, ncols, [&](float v, int) { part += expf(v / t - mx); });
  const float sum = block_sum(part, s_red);
  uint32_t* keys = keys_ws + r * cols;

  const int64_t k = top_ks[r];
  const uint64_t k_lim = (k > 0 && k < cols) ? static_cast<uint64_t>(k) : static_cast<uint64_t>(cols);
  const float tp = top_ps[r];
  const bool p_lim = tp < 1.0f;
  const uint64_t mass_lim = p_lim ? (tp > 0.0f ? static_cast<uint64_t>(static_cast<double>(tp) * kMassUnit) : 0ull)
                                  : ~0ull;
  uint32_t v_cut = 0;       // key of the last kept rank
  int64_t idx_cut = cols;   // among keys == v_cut, indices <= idx_cut are kept
  const bool truncate = p_lim || k_lim < static_cast<uint64_t>(cols);
  if (truncate) {
    // keys = bits of p (p >= 0, so they order like p), written once, read by every level
    for_each_col<4>(row, ncols, [&](float v, int c) {
      keys[c] = __float_as_uint(expf(v / t - mx) / sum);
    });
    __syncthreads();  // keys visible to the block
    uint32_t prefix = 0, pmask = 0;
    uint64_t cnt_above = 0, mass_above = 0, final_cnt = 0;
    for (int level = 0; level < 4; ++level) {
      const int shift = 24 - 8 * level;
      for (int i = tid; i < kHistCopies * 257; i += kSampleThreads) {
        (&h_cnt[0][0])[i] = 0;
        (&h_mass[0][0])[i] = 0;
      }
      __syncthreads();
      for_each_col<8>(reinterpret_cast<const float*>(keys), ncols, [&](float kv, int) {
        const uint32_t key = __float_as_uint(kv);
        if ((key & pmask) == prefix) {
          const int b = (key >> shift) & 255;
          atomicAdd(&h_cnt[copy][b], 1u);
          atomicAdd(reinterpret_cast<unsigned long long*>(&h_mass[copy][b]),
                    static_cast<unsigned long long>(mass_of(key)));
        }
      });
      __syncthreads();
      if (tid < 256) {  // integer totals: exact in any order
        uint32_t cn = 0;
        uint64_t ms = 0;
        for (int w = 0; w < kHistCopies; ++w) {
          cn += h_cnt[w][tid];
          ms += h_mass[w][tid];
        }
        h_cnt[0][tid] = cn;
        h_mass[0][tid] = ms;
      }
      __syncthreads();
      if (tid == 0) {
        // Highest bin first (larger p); the bin holding the last kept rank is the last
        // non-empty bin whose first rank is kept: rank cnt_above with cnt_above ranks and
        // mass_above before it. Rank 0 is always kept, so such a bin exists.
        int chosen = -1;
        for (int b = 255; b >= 0; --b) {
          const uint64_t cn = h_cnt[0][b];
          if (cn == 0) continue;
          const uint64_t ms = h_mass[0][b];
          chosen = b;
          const bool next_kept = cnt_above + cn < k_lim && mass_above + ms <= mass_lim;
          int nb = b - 1;
          while (nb >= 0 && h_cnt[0][nb] == 0) --nb;
          if (!next_kept || nb < 0) break;
          cnt_above += cn;
          mass_above += ms;
        }
        prefix |= static_cast<uint32_t>(chosen) << shift;
        pmask |= 0xffu << shift;
        final_cnt = h_cnt[0][chosen];
        s_sel[0] = prefix;
        s_sel[1] = cnt_above;
        s_sel[2] = mass_above;
        s_sel[3] = final_cnt;
      }
      __syncthreads();
      prefix = static_cast<uint32_t>(s_sel[0]);
      pmask |= 0xffu << shift;
      cnt_above = s_sel[1];
      mass_above = s_sel[2];
      final_cnt = s_sel[3];
    }
    v_cut = prefix;
    // Ties at the cut: how many of the final_cnt equal keys are kept (>= 1).
    uint64_t n_keep = final_cnt;
    if (k_lim - cnt_above < n_keep) n_keep = k_lim - cnt_above;
    const uint64_t q = mass_of(v_cut);
    if (p_lim && q > 0) {
      const uint64_t by_mass = (mass_lim - mass_above) / q + 1;
      if (by_mass < n_keep) n_keep = by_mass;
    }
    if (n_keep < final_cnt) {
      // Index of the n_keep-th tie in index order: contiguous chunks, block scan.
      const int64_t chunk = (cols + kSampleThreads - 1) / kSampleThreads;
      const int64_t c0 = min(cols, chunk * tid);
      const int64_t c1 = min(cols, c0 + chunk);
      int64_t mine = 0;
      for (int64_t c = c0; c < c1; ++c) mine += keys[c] == v_cut;
      s_scan[tid] = mine;
      __syncthreads();
      for (int off = 1; off < kSampleThreads; off <<= 1) {  // inclusive scan
        const int64_t add = tid >= off ? s_scan[tid - off] : 0;
        __syncthreads();
        s_scan[tid] += add;
        __syncthreads();
      }
      const int64_t before = s_scan[tid] - mine;
      const int64_t want = static_cast<int64_t>(n_keep) - 1;  // 0-based tie position
      if (want >= before && want < before + mine) {
        int64_t seen = before;
        for (int64_t c = c0; c < c1; ++c) {
          if (keys[c] == v_cut) {
            if (seen == want) {
              s_cut = c;
              break;
            }
            ++seen;
          }
        }
      }
      __syncthreads();
      idx_cut = s_cut;
    }
  }

  const uint32_t row_hash = gumbel_row(seeds[r], positions[r]);
  auto draw = [&](uint32_t key, int c) {
    const float s = logf(__uint_as_float(key) + kSampleEps) + seeded_gumbel(row_hash, c);
    if (better(s, c, bv, bi)) {
      bv = s;
      bi = c;
    }
  };
  if (truncate) {
    for_each_col<4>(reinterpret_cast<const float*>(keys), ncols, [&](float kv, int c) {
      const uint32_t key = __float_as_uint(kv);
      if (key > v_cut || (key == v_cut && c <= idx_cut)) draw(key, c);
    });
  } else {  // every token kept: p straight from the logits (same bits as the keys)
    for_each_col<4>(row, ncols, [&](float v, int c) {
      draw(__float_as_uint(expf(v / t - mx) / sum), c);
    });
  }
  block_best(bv, bi, s_bv, s_bi);
  if (tid == 0) out[r] = bi < cols ? bi : 0;
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_argmax_rows(const float* logits, int64_t ld, int64_t* out, int64_t rows,
                               int64_t cols, void* stream) {
  SID_REQUIRE(rows >= 0 && cols >= 0, "argmax_rows: negative size");
  if (rows == 0) return SID_OK;
  SID_REQUIRE(logits && out, "argmax_rows: null pointer");
  SID_REQUIRE(cols > 0 && ld >= cols, "argmax_rows: bad row stride %lld for %lld columns",
              (long long)ld, (long long)cols);
  SID_REQUIRE(rows < (1ll << 31) && cols < (1ll << 31), "argmax_rows: too large");
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(kSampleThreads), 0,
                     static_cast<hipStream_t>(stream), logits, ld, out, cols);
  return check_launch("argmax_rows");
}


extern "C" int64_t sid_sample_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return rows * cols * static_cast<int64_t>(sizeof(uint32_t));
}

extern "C" int sid_sample_rows(const float* logits, int64_t ld, const float* temperatures,
                               const int64_t* top_ks, const float* top_ps, const int64_t* seeds,
                               const int64_t* positions, int64_t rows, int64_t cols,
                               void* workspace, int64_t workspace_bytes, int64_t* out,
                               void* stream) {
  SID_REQUIRE(rows >= 0 && cols >= 0, "sample_rows: negative size");
  if (rows == 0) return SID_OK;
  SID_REQUIRE(logits && temperatures && top_ks && top_ps && seeds && positions && out,
              "sample_rows: null pointer");
  SID_REQUIRE(cols > 0 && ld >= cols, "sample_rows: bad row stride %lld for %lld columns",
              (long long)ld, (long long)cols);
  SID_REQUIRE(rows < (1ll << 31) && cols < (1ll << 31), "sample_rows: too large");
  const int64_t need = sid_sample_workspace_bytes(rows, cols);
  SID_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "sample_rows: workspace %lld bytes, need %lld", (long long)workspace_bytes,
              (long long)need);
  hipLaunchKernelGGL(sample_kernel, dim3((unsigned)rows), dim3(kSampleThreads), 0,
                     static_cast<hipStream_t>(stream), logits, ld, temperatures, top_ks, top_ps,
                     seeds, positions, cols, static_cast<uint32_t*>(workspace), out);
  return check_launch("sample_rows");
}
