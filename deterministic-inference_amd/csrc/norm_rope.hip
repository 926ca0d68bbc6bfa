// Row-wise elementwise kernels of the decode step: RMSNorm (plain and fused
// with the residual add), NeoX RoPE and the SwiGLU gate. All are tiny and
// bandwidth/launch bound; what matters is a fixed in-row reduction order
// (every row is reduced by the same lane pattern, so results are independent
// of the row's index and of how many rows are processed together).
#include "common.h"

#include <cmath>

namespace sid {
namespace {

// A row is processed by LPR consecutive lanes (LPR a power of two <= 64);
// lane j of the row owns 16-byte vectors j, j + LPR, j + 2*LPR, ...
// Sum of squares: lane-local sequential sum, then an xor butterfly across
// the LPR lanes; every lane of the row ends with identical bits.
__device__ __forceinline__ float row_sum(float v, int lpr) {
  for (int mask = 1; mask < lpr; mask <<= 1) v += lane_xor(v, mask);
  return v;
}

__device__ __forceinline__ void load8(const uint4& u, float (&f)[8]) {
  f[0] = bf16_lo(u.x); f[1] = bf16_hi(u.x);
  f[2] = bf16_lo(u.y); f[3] = bf16_hi(u.y);
  f[4] = bf16_lo(u.z); f[5] = bf16_hi(u.z);
  f[6] = bf16_lo(u.w); f[7] = bf16_hi(u.w);
}

__device__ __forceinline__ uint4 store8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// Up to MAXV vectors per lane are kept in registers between the two passes.
constexpr int MAXV = 16;

// FUSED = false: out = rmsnorm(x) * w.
// FUSED = true:  r = x + residual (fp32); residual = bf16(r); x = rmsnorm(r) * w.
template <bool FUSED>
__global__ void __launch_bounds__(256) rmsnorm_kernel(uint4* __restrict__ x,
                                                      uint4* __restrict__ residual,
                                                      const uint4* __restrict__ w,
                                                      uint4* __restrict__ out, int64_t rows,
                                                      int hidden, int lpr, float eps) {
  const int tid = threadIdx.x;
  const int rows_per_block = 256 / lpr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + tid / lpr;
  const int j = tid % lpr;
  const int nvec = hidden / 8;
  const int per_lane = nvec / lpr;  // host guarantees nvec % lpr == 0 and per_lane <= MAXV
  const bool active = row < rows;
  const int64_t base = row * nvec;

  float v[MAXV][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < per_lane && active) {
      const int c = j + i * lpr;
      load8(x[base + c], v[i]);
      if constexpr (FUSED) {
        float r[8];
        load8(residual[base + c], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = r[e] + v[i][e];
        residual[base + c] = store8(v[i]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
  }
  // Rows of a block are whole lane groups, so the butterfly never mixes rows;
  // inactive lanes contribute zeros to their own (discarded) row.
  ss = row_sum(ss, lpr);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
  if (!active) return;
  uint4* dst = FUSED ? x : out;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < per_lane) {
      const int c = j + i * lpr;
      float wf[8];
      load8(w[c], wf);
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = v[i][e] * rstd * wf[e];
      dst[base + c] = store8(y);
    }
  }
}

int pick_lpr(int hidden) {
  const int nvec = hidden / 8;
  int lpr = 64;
  while (lpr > 1 && nvec % lpr != 0) lpr >>= 1;
  while (lpr > nvec) lpr >>= 1;
  return lpr;
}

// One block per token; thread -> (head, pair of rotary indices).
__global__ void __launch_bounds__(256) rope_kernel(uint32_t* __restrict__ q, uint32_t* __restrict__ k,
                                                   const int64_t* __restrict__ positions,
                                                   const float* __restrict__ cos_sin,
                                                   int num_q_heads, int num_kv_heads, int head_dim,
                                                   int64_t max_positions) {
  const int64_t t = blockIdx.x;
  const int64_t pos = positions[t];
  if (pos < 0 || pos >= max_positions) return;
  const int half = head_dim / 2;
  const int pairs = half / 2;  // packed bf16x2 words per half
  const float* cs = cos_sin + pos * head_dim;
  const int total = (num_q_heads + num_kv_heads) * pairs;
  for (int p = threadIdx.x; p < total; p += blockDim.x) {
    const int head = p / pairs;
    const int i = p % pairs;
    uint32_t* base = head < num_q_heads
                         ? q + (t * num_q_heads + head) * (head_dim / 2)
                         : k + (t * num_kv_heads + (head - num_q_heads)) * (head_dim / 2);
    const uint32_t a = base[i];
    const uint32_t b = base[pairs + i];
    const float c0 = cs[2 * i], c1 = cs[2 * i + 1];
    const float s0 = cs[half + 2 * i], s1 = cs[half + 2 * i + 1];
    const float x1a = bf16_lo(a), x1b = bf16_hi(a);
    const float x2a = bf16_lo(b), x2b = bf16_hi(b);
    base[i] = pack_bf16x2(x1a * c0 - x2a * s0, x1b * c1 - x2b * s1);
    base[pairs + i] = pack_bf16x2(x2a * c0 + x1a * s0, x2b * c1 + x1b * s1);
  }
}

// out = bf16(bf16(silu(gate)) * up), 8 elements per thread.
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint4* __restrict__ gate_up,
                                                       uint4* __restrict__ out, int64_t rows,
                                                       int64_t inter_vec) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * inter_vec) return;
  const int64_t r = i / inter_vec;
  const int64_t c = i % inter_vec;
  float g[8], u[8], y[8];
  load8(gate_up[r * 2 * inter_vec + c], g);
  load8(gate_up[r * 2 * inter_vec + inter_vec + c], u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = round_bf16(g[e] / (1.0f + __expf(-g[e])));
    y[e] = s * u[e];
  }
  out[i] = store8(y);
}

}  // namespace
}  // namespace sid

using namespace sid;

static int launch_rmsnorm(bool fused, void* x, void* residual, const void* w, void* out,
                          int64_t rows, int hidden, float eps, void* stream, const char* name) {
  SID_REQUIRE(rows >= 0, "%s: negative rows", name);
  if (rows == 0) return SID_OK;
  SID_REQUIRE(x && w && (fused ? residual != nullptr : out != nullptr), "%s: null pointer", name);
  SID_REQUIRE(hidden >= 8 && hidden % 8 == 0, "%s: hidden %d must be a positive multiple of 8",
              name, hidden);
  const int lpr = pick_lpr(hidden);
  SID_REQUIRE(hidden / 8 / lpr <= MAXV, "%s: hidden %d too large (max %d)", name, hidden,
              MAXV * 64 * 8);
  const int rpb = 256 / lpr;
  const int64_t blocks = (rows + rpb - 1) / rpb;
  SID_REQUIRE(blocks < (1ll << 31), "%s: too many rows", name);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (fused) {
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, (uint4*)x,
                       (uint4*)residual, (const uint4*)w, nullptr, rows, hidden, lpr, eps);
  } else {
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, (uint4*)x,
                       nullptr, (const uint4*)w, (uint4*)out, rows, hidden, lpr, eps);
  }
  return check_launch(name);
}

extern "C" int sid_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int hidden,
                           float eps, void* stream) {
  return launch_rmsnorm(false, const_cast<void*>(x), nullptr, w, out, rows, hidden, eps, stream,
                        "rmsnorm");
}

extern "C" int sid_fused_add_rmsnorm(void* x, void* residual, const void* w, int64_t rows,
                                     int hidden, float eps, void* stream) {
  return launch_rmsnorm(true, x, residual, w, nullptr, rows, hidden, eps, stream,
                        "fused_add_rmsnorm");
}

extern "C" int sid_rope_apply(void* q, void* k, const int64_t* positions, const float* cos_sin,
                              int64_t num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                              int64_t max_positions, void* stream) {
  SID_REQUIRE(num_tokens >= 0, "rope: negative token count");
  if (num_tokens == 0) return SID_OK;
  SID_REQUIRE(q && k && positions && cos_sin, "rope: null pointer");
  SID_REQUIRE(head_dim > 0 && head_dim % 4 == 0, "rope: head_dim %d must be a multiple of 4",
              head_dim);
  SID_REQUIRE(num_q_heads > 0 && num_kv_heads >= 0, "rope: bad head counts");
  SID_REQUIRE(num_tokens < (1ll << 31), "rope: too many tokens");
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)num_tokens), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (uint32_t*)q, (uint32_t*)k, positions,
                     cos_sin, num_q_heads, num_kv_heads, head_dim, max_positions);
  return check_launch("rope");
}

extern "C" int sid_silu_mul(const void* gate_up, void* out, int64_t num_tokens, int64_t inter,
                            void* stream) {
  SID_REQUIRE(num_tokens >= 0, "silu_mul: negative token count");
  if (num_tokens == 0) return SID_OK;
  SID_REQUIRE(gate_up && out, "silu_mul: null pointer");
  SID_REQUIRE(inter > 0 && inter % 8 == 0, "silu_mul: intermediate size must be a multiple of 8");
  const int64_t total = num_tokens * (inter / 8);
  const int64_t blocks = (total + 255) / 256;
  SID_REQUIRE(blocks < (1ll << 31), "silu_mul: too many elements");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (const uint4*)gate_up, (uint4*)out,
                     num_tokens, inter / 8);
  return check_launch("silu_mul");
}
