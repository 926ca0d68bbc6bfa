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

constexpr int kThreads = 1024;

__global__ void __launch_bounds__(kThreads) argmax_kernel(const float* __restrict__ logits,
                                                          int64_t ld, int64_t* __restrict__ out,
                                                          int64_t cols) {
  const int64_t r = blockIdx.x;
  const float* row = logits + r * ld;
  float bv = -INFINITY;
  int64_t bi = cols;  // sentinel larger than any index
  auto take = [&](float v, int64_t c) {
    if (better(v, c, bv, bi)) {
      bv = v;
      bi = c;
    }
  };
  // Vector body: 16-byte loads, UNROLL of them in flight per thread (the row start must
  // be 16-byte aligned for this; otherwise everything goes through the scalar tail).
  constexpr int UNROLL = 8;
  int64_t vec_cols = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const float4* row4 = reinterpret_cast<const float4*>(row);
    const int64_t n4 = cols / 4;
    const int64_t step = static_cast<int64_t>(kThreads) * UNROLL;
    int64_t base = 0;
    for (; base + step <= n4; base += step) {
      float4 v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = row4[base + u * kThreads + threadIdx.x];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t c = 4 * (base + u * kThreads + threadIdx.x);
        take(v[u].x, c);
        take(v[u].y, c + 1);
        take(v[u].z, c + 2);
        take(v[u].w, c + 3);
      }
    }
    vec_cols = 4 * base;
  }
  for (int64_t c = vec_cols + threadIdx.x; c < cols; c += kThreads) take(row[c], c);
  // Wave reduction, then across waves through LDS.
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
  __shared__ float s_v[kThreads / 64];
  __shared__ int64_t s_i[kThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[wave] = bv;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) {
      if (better(s_v[w], s_i[w], bv, bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    }
    out[r] = bi < cols ? bi : 0;
  }
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
  SID_REQUIRE(rows < (1ll << 31), "argmax_rows: too many rows");
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), logits, ld, out, cols);
  return check_launch("argmax_rows");
}
