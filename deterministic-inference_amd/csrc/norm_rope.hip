// Row-wise kernels of the decode step: RMSNorm (plain and fused with the
// residual add), NeoX RoPE, SwiGLU, and the fused QKV epilogue (q/k-norm +
// RoPE + KV-cache write). They are launch/bandwidth bound; what matters is a
// fixed in-row reduction order (every row is reduced by the same lane
// pattern, so results do not depend on the row's index or on how many rows
// are processed together).
//
// Inputs that come straight out of a projection can be given either as the
// bf16 matrix or as the GEMM's fp32 chunk partials (sid_linear_partials); in
// the latter case the chunks are folded here in increasing chunk order and
// rounded to bf16, which is exactly sid_linear's result, so the fused kernels
// are bit-identical to "sid_linear, then the op". All arithmetic that two
// kernels share goes through the same helpers with explicit fmaf, so the
// fused and unfused paths also agree bit for bit after the first rounding.
#include "common.h"
#include "rowmath.h"

#include <cmath>

namespace sid {
namespace {

// An activation row: a bf16 matrix [rows, ld], or GEMM chunk partials
// fp32 [nchunks][rows][ld] folded in chunk order and rounded to bf16.
struct RowSrc {
  const bf16_t* bf;
  const float* part;
  int64_t ld;
  int64_t chunk_stride;
  int nchunks;
};

// NCH > 0: exactly NCH chunks, all loads issued before the fold (fully unrolled);
// NCH == 0: s.bf; NCH < 0: s.nchunks chunks, generic loop.
template <int NCH>
__device__ __forceinline__ void load8_src(const RowSrc& s, int64_t row, int64_t col, float (&f)[8]) {
  if constexpr (NCH == 0) {
    load8(*reinterpret_cast<const uint4*>(s.bf + row * s.ld + col), f);
    return;
  } else {
    const float* p = s.part + row * s.ld + col;
    if constexpr (NCH > 0) {
      float4 a[NCH], b[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        a[c] = *reinterpret_cast<const float4*>(p + c * s.chunk_stride);
        b[c] = *reinterpret_cast<const float4*>(p + c * s.chunk_stride + 4);
      }
      f[0] = a[0].x; f[1] = a[0].y; f[2] = a[0].z; f[3] = a[0].w;
      f[4] = b[0].x; f[5] = b[0].y; f[6] = b[0].z; f[7] = b[0].w;
#pragma unroll
      for (int c = 1; c < NCH; ++c) {
        f[0] += a[c].x; f[1] += a[c].y; f[2] += a[c].z; f[3] += a[c].w;
        f[4] += b[c].x; f[5] += b[c].y; f[6] += b[c].z; f[7] += b[c].w;
      }
    } else {
      float4 a = *reinterpret_cast<const float4*>(p);
      float4 b = *reinterpret_cast<const float4*>(p + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
      for (int c = 1; c < s.nchunks; ++c) {
        p += s.chunk_stride;
        a = *reinterpret_cast<const float4*>(p);
        b = *reinterpret_cast<const float4*>(p + 4);
        f[0] += a.x; f[1] += a.y; f[2] += a.z; f[3] += a.w;
        f[4] += b.x; f[5] += b.y; f[6] += b.z; f[7] += b.w;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = round_bf16(f[e]);
  }
}

// Calls fn.template operator()<NCH>() with NCH the compile-time chunk count of src
// (0 for a bf16 source; -1 for a count without a specialised instance).
template <typename F>
__host__ void dispatch_nch(const RowSrc& src, F&& fn) {
  if (src.part == nullptr) return fn.template operator()<0>();
  switch (src.nchunks) {
    case 1: return fn.template operator()<1>();
    case 2: return fn.template operator()<2>();
    case 3: return fn.template operator()<3>();
    case 4: return fn.template operator()<4>();
    case 8: return fn.template operator()<8>();
    case 12: return fn.template operator()<12>();
    case 16: return fn.template operator()<16>();
    default: return fn.template operator()<-1>();
  }
}

// ---- RMSNorm ----------------------------------------------------------------------------

constexpr int MAXV = 16;  // vectors per lane kept in registers between the two passes

// FUSED = false: out = rmsnorm(x) * w.
// FUSED = true:  r = residual + x (fp32); residual = bf16(r); out = rmsnorm(r) * w.
template <bool FUSED, int NCH>
__global__ void __launch_bounds__(256) rmsnorm_kernel(RowSrc xs, uint4* __restrict__ residual,
                                                      const uint4* __restrict__ w,
                                                      uint4* __restrict__ out, int64_t rows,
                                                      int hidden, int lpr, float eps) {
  const int tid = threadIdx.x;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / lpr) + tid / lpr;
  const int j = tid % lpr;
  const int nvec = hidden / 8;
  const int per_lane = nvec / lpr;  // the host guarantees nvec % lpr == 0, per_lane <= MAXV
  const bool active = row < rows;
  const int64_t base = row * nvec;

  // Weights first: independent of the row, so their latency overlaps the row loads.
  uint4 wv[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < per_lane) wv[i] = w[j + i * lpr];
  }
  float v[MAXV][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < per_lane && active) {
      const int c = j + i * lpr;
      load8_src<NCH>(xs, row, static_cast<int64_t>(c) * 8, v[i]);
      if constexpr (FUSED) {
        float r[8];
        load8(residual[base + c], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = r[e] + v[i][e];
        residual[base + c] = store8(v[i]);
      }
      ss = sumsq8(v[i], ss);
    }
  }
  // Rows of a block are whole lane groups: the butterfly never mixes rows.
  ss = group_sum(ss, lpr);
  const float rstd = rms_rstd(ss, hidden, eps);
  if (!active) return;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < per_lane) {
      const int c = j + i * lpr;
      float wf[8], y[8];
      load8(wv[i], wf);
      rms_apply8(v[i], rstd, wf, y);
      out[base + c] = store8(y);
    }
  }
}

// Few rows (decode): one 256-thread workgroup per row. Pass 1 spreads the memory work
// (chunk fold, residual add) over all 256 threads, 4 columns each, into an fp32 row in
// LDS; pass 2 reduces the sum of squares with exactly the lane layout and order of
// rmsnorm_kernel (lpr lanes, lane j owning vectors j + i*lpr, sequential fmaf, then the
// xor butterfly), so both kernels produce identical bits and either may serve any row.
template <int NCH>
__device__ __forceinline__ void load4_src(const RowSrc& s, int64_t row, int64_t col, float (&f)[4]) {
  if constexpr (NCH == 0) {
    const uint2 u = *reinterpret_cast<const uint2*>(s.bf + row * s.ld + col);
    f[0] = bf16_lo(u.x); f[1] = bf16_hi(u.x); f[2] = bf16_lo(u.y); f[3] = bf16_hi(u.y);
    return;
  } else {
    const float* p = s.part + row * s.ld + col;
    if constexpr (NCH > 0) {
      float4 a[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) a[c] = *reinterpret_cast<const float4*>(p + c * s.chunk_stride);
      f[0] = a[0].x; f[1] = a[0].y; f[2] = a[0].z; f[3] = a[0].w;
#pragma unroll
      for (int c = 1; c < NCH; ++c) {
        f[0] += a[c].x; f[1] += a[c].y; f[2] += a[c].z; f[3] += a[c].w;
      }
    } else {
      float4 a = *reinterpret_cast<const float4*>(p);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      for (int c = 1; c < s.nchunks; ++c) {
        p += s.chunk_stride;
        a = *reinterpret_cast<const float4*>(p);
        f[0] += a.x; f[1] += a.y; f[2] += a.z; f[3] += a.w;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = round_bf16(f[e]);
  }
}

constexpr int ROWBLOCK_THREADS = 256;

template <bool FUSED, int NCH>
__global__ void __launch_bounds__(ROWBLOCK_THREADS) rmsnorm_rowblock_kernel(
    RowSrc xs, uint2* __restrict__ residual, const uint2* __restrict__ w, uint2* __restrict__ out,
    int hidden, int lpr, float eps) {
  extern __shared__ float srow[];  // [hidden] fp32 row, then rstd
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nq = hidden / 4;
  const int64_t base = row * nq;
  for (int u = tid; u < nq; u += ROWBLOCK_THREADS) {
    float v[4];
    load4_src<NCH>(xs, row, static_cast<int64_t>(u) * 4, v);
    if constexpr (FUSED) {
      const uint2 r = residual[base + u];
      v[0] = bf16_lo(r.x) + v[0];
      v[1] = bf16_hi(r.x) + v[1];
      v[2] = bf16_lo(r.y) + v[2];
      v[3] = bf16_hi(r.y) + v[3];
      residual[base + u] = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
    *reinterpret_cast<float4*>(&srow[4 * u]) = make_float4(v[0], v[1], v[2], v[3]);
  }
  __syncthreads();
  if (tid < 64) {
    const int per_lane = hidden / 8 / lpr;
    float ss = 0.0f;
    if (tid < lpr) {
      for (int i = 0; i < per_lane; ++i) {
        const int c = tid + i * lpr;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = srow[8 * c + e];
        ss = sumsq8(v, ss);
      }
    }
    ss = group_sum(ss, lpr);
    if (tid == 0) srow[hidden] = rms_rstd(ss, hidden, eps);
  }
  __syncthreads();
  const float rstd = srow[hidden];
  for (int u = tid; u < nq; u += ROWBLOCK_THREADS) {
    const float4 v = *reinterpret_cast<const float4*>(&srow[4 * u]);
    const uint2 wu = w[u];
    const float y0 = (v.x * rstd) * bf16_lo(wu.x);
    const float y1 = (v.y * rstd) * bf16_hi(wu.x);
    const float y2 = (v.z * rstd) * bf16_lo(wu.y);
    const float y3 = (v.w * rstd) * bf16_hi(wu.y);
    out[base + u] = make_uint2(pack_bf16x2(y0, y1), pack_bf16x2(y2, y3));
  }
}

int pick_lpr(int hidden) {
  const int nvec = hidden / 8;
  int lpr = 64;
  while (lpr > 1 && nvec % lpr != 0) lpr >>= 1;
  while (lpr > nvec) lpr >>= 1;
  return lpr;
}

// ---- RoPE -----------------------------------------------------------------------------

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
    float o1a, o2a, o1b, o2b;
    rope_pair(bf16_lo(a), bf16_lo(b), cs[2 * i], cs[half + 2 * i], o1a, o2a);
    rope_pair(bf16_hi(a), bf16_hi(b), cs[2 * i + 1], cs[half + 2 * i + 1], o1b, o2b);
    base[i] = pack_bf16x2(o1a, o1b);
    base[pairs + i] = pack_bf16x2(o2a, o2b);
  }
}

// ---- SwiGLU -------------------------------------------------------------------------------

// out = bf16(bf16(silu(gate)) * up), 4 elements per thread (many small workgroups, so a
// decode batch's few MB of chunk partials are read by every CU).
template <int NCH>
__global__ void __launch_bounds__(128) silu_mul_kernel(RowSrc gu, uint2* __restrict__ out,
                                                       int64_t rows, int64_t inter_q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * inter_q) return;
  const int64_t r = i / inter_q;
  const int64_t c = i % inter_q;
  float g[4], u[4], y[4];
  load4_src<NCH>(gu, r, c * 4, g);
  load4_src<NCH>(gu, r, (inter_q + c) * 4, u);
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = silu_mul1(g[e], u[e]);
  out[i] = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
}

// ---- fused QKV epilogue -------------------------------------------------------------------

// Row t of the projection is [q (HQ*128) | k (HKV*128) | v (HKV*128)]. A head is
// handled by 16 lanes (lane j: dims 8j..8j+7, which is rmsnorm_kernel's layout for
// hidden 128), 8 heads per 128-thread block. q/k heads: per-head RMSNorm, round, RoPE (the
// rotate-half partner of lane j is lane j ^ 8, one DPP row_ror:8 away), round;
// v heads: copied. q goes to q_out [T, HQ, 128]; k and v to the pools at slots[t].
constexpr int QD = 128;

template <int NCH>
__global__ void __launch_bounds__(128) qkv_post_kernel(
    RowSrc src, int num_q_heads, int num_kv_heads, const uint4* __restrict__ q_norm,
    const uint4* __restrict__ k_norm, float eps, const int64_t* __restrict__ positions,
    const float* __restrict__ cos_sin, int64_t max_positions, const int64_t* __restrict__ slots,
    uint4* __restrict__ q_out, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    int64_t num_slots) {
  const int64_t t = blockIdx.x;
  const int head = blockIdx.y * 8 + (threadIdx.x >> 4);
  const int j = threadIdx.x & 15;
  const int heads = num_q_heads + 2 * num_kv_heads;
  // Whole 16-lane groups are uniform; the DPP/bpermute below needs every lane of a
  // row active, so out-of-range heads compute on clamped data and skip the stores.
  const bool valid = head < heads;
  const int hh = valid ? head : heads - 1;
  float v[8];
  load8_src<NCH>(src, t, static_cast<int64_t>(hh) * QD + 8 * j, v);

  const bool is_v = hh >= num_q_heads + num_kv_heads;
  const int64_t slot = slots[t];
  const bool slot_ok = slot >= 0 && slot < num_slots;
  const int kv_row = 16 * num_kv_heads;  // uint4 per pool row
  if (is_v) {
    if (valid && slot_ok)
      v_cache[slot * kv_row + (hh - num_q_heads - num_kv_heads) * 16 + j] = store8(v);
    return;  // v heads occupy whole blocks' tail groups; no cross-lane op follows for them
  }
  const bool is_q = hh < num_q_heads;
  QkRopeIn in;
  qk_rope_load(in, j, is_q ? q_norm : k_norm, positions[t], cos_sin, max_positions);
  float o[8];
  qk_head_norm_rope(v, j, in, eps, o);
  if (!valid) return;
  if (is_q) {
    q_out[(t * num_q_heads + hh) * 16 + j] = store8(o);
  } else if (slot_ok) {
    k_cache[slot * kv_row + (hh - num_q_heads) * 16 + j] = store8(o);
  }
}

}  // namespace
}  // namespace sid

using namespace sid;

// Below this many rows the one-workgroup-per-row kernel is used.
constexpr int64_t kRowBlockBelow = 1024;

static int launch_rmsnorm(bool fused, RowSrc xs, void* residual, const void* w, void* out,
                          int64_t rows, int hidden, float eps, void* stream, const char* name) {
  SID_REQUIRE(rows >= 0, "%s: negative rows", name);
  if (rows == 0) return SID_OK;
  SID_REQUIRE((xs.bf || xs.part) && w && out && (!fused || residual), "%s: null pointer", name);
  SID_REQUIRE(hidden >= 8 && hidden % 8 == 0, "%s: hidden %d must be a positive multiple of 8",
              name, hidden);
  const int lpr = pick_lpr(hidden);
  SID_REQUIRE(hidden / 8 / lpr <= MAXV, "%s: hidden %d too large (max %d)", name, hidden,
              MAXV * 64 * 8);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows < kRowBlockBelow) {
    // Decode-sized batches: a 256-thread workgroup per row (identical bits).
    const size_t lds = (static_cast<size_t>(hidden) + 4) * sizeof(float);
    dispatch_nch(xs, [&]<int NCH>() {
      if (fused) {
        hipLaunchKernelGGL((rmsnorm_rowblock_kernel<true, NCH>), dim3((unsigned)rows),
                           dim3(ROWBLOCK_THREADS), lds, s, xs, (uint2*)residual, (const uint2*)w,
                           (uint2*)out, hidden, lpr, eps);
      } else {
        hipLaunchKernelGGL((rmsnorm_rowblock_kernel<false, NCH>), dim3((unsigned)rows),
                           dim3(ROWBLOCK_THREADS), lds, s, xs, nullptr, (const uint2*)w,
                           (uint2*)out, hidden, lpr, eps);
      }
    });
    return check_launch(name);
  }
  const int rpb = 256 / lpr;
  const int threads = rpb * lpr;
  const int64_t blocks = (rows + rpb - 1) / rpb;
  SID_REQUIRE(blocks < (1ll << 31), "%s: too many rows", name);
  dispatch_nch(xs, [&]<int NCH>() {
    if (fused) {
      hipLaunchKernelGGL((rmsnorm_kernel<true, NCH>), dim3((unsigned)blocks), dim3(threads), 0, s, xs,
                         (uint4*)residual, (const uint4*)w, (uint4*)out, rows, hidden, lpr, eps);
    } else {
      hipLaunchKernelGGL((rmsnorm_kernel<false, NCH>), dim3((unsigned)blocks), dim3(threads), 0, s,
                         xs, nullptr, (const uint4*)w, (uint4*)out, rows, hidden, lpr, eps);
    }
  });
  return check_launch(name);
}

static RowSrc bf_src(const void* x, int64_t ld) { return RowSrc{(const bf16_t*)x, nullptr, ld, 0, 0}; }

static RowSrc part_src(const float* p, int nchunks, int64_t rows, int64_t ld) {
  return RowSrc{nullptr, p, ld, rows * ld, nchunks};
}

extern "C" int sid_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int hidden,
                           float eps, void* stream) {
  return launch_rmsnorm(false, bf_src(x, hidden), nullptr, w, out, rows, hidden, eps, stream,
                        "rmsnorm");
}

extern "C" int sid_fused_add_rmsnorm(void* x, void* residual, const void* w, int64_t rows,
                                     int hidden, float eps, void* stream) {
  return launch_rmsnorm(true, bf_src(x, hidden), residual, w, x, rows, hidden, eps, stream,
                        "fused_add_rmsnorm");
}

extern "C" int sid_fused_add_rmsnorm_partials(const float* partials, int nchunks, void* residual,
                                              const void* w, void* out, int64_t rows, int hidden,
                                              float eps, void* stream) {
  SID_REQUIRE(nchunks >= 1, "fused_add_rmsnorm_partials: nchunks must be >= 1");
  return launch_rmsnorm(true, part_src(partials, nchunks, rows, hidden), residual, w, out, rows,
                        hidden, eps, stream, "fused_add_rmsnorm_partials");
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

static int launch_silu(RowSrc gu, void* out, int64_t num_tokens, int64_t inter, void* stream,
                       const char* name) {
  SID_REQUIRE(num_tokens >= 0, "%s: negative token count", name);
  if (num_tokens == 0) return SID_OK;
  SID_REQUIRE((gu.bf || gu.part) && out, "%s: null pointer", name);
  SID_REQUIRE(inter > 0 && inter % 8 == 0, "%s: intermediate size must be a multiple of 8", name);
  const int64_t total = num_tokens * (inter / 4);
  const int64_t blocks = (total + 127) / 128;
  SID_REQUIRE(blocks < (1ll << 31), "%s: too many elements", name);
  dispatch_nch(gu, [&]<int NCH>() {
    hipLaunchKernelGGL(silu_mul_kernel<NCH>, dim3((unsigned)blocks), dim3(128), 0,
                       static_cast<hipStream_t>(stream), gu, (uint2*)out, num_tokens, inter / 4);
  });
  return check_launch(name);
}

extern "C" int sid_silu_mul(const void* gate_up, void* out, int64_t num_tokens, int64_t inter,
                            void* stream) {
  return launch_silu(bf_src(gate_up, 2 * inter), out, num_tokens, inter, stream, "silu_mul");
}

extern "C" int sid_silu_mul_partials(const float* partials, int nchunks, void* out,
                                     int64_t num_tokens, int64_t inter, void* stream) {
  SID_REQUIRE(nchunks >= 1, "silu_mul_partials: nchunks must be >= 1");
  return launch_silu(part_src(partials, nchunks, num_tokens, 2 * inter), out, num_tokens, inter,
                     stream, "silu_mul_partials");
}

extern "C" int sid_qkv_post(const void* qkv, const float* partials, int nchunks,
                            int64_t num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                            const void* q_norm, const void* k_norm, float eps,
                            const int64_t* positions, const float* cos_sin,
                            int64_t max_positions, const int64_t* slots, void* q_out,
                            void* k_cache, void* v_cache, int64_t num_slots, void* stream) {
  SID_REQUIRE(num_tokens >= 0, "qkv_post: negative token count");
  if (num_tokens == 0) return SID_OK;
  SID_REQUIRE((qkv != nullptr) != (partials != nullptr),
              "qkv_post: exactly one of qkv and partials must be given");
  SID_REQUIRE(partials == nullptr || nchunks >= 1, "qkv_post: nchunks must be >= 1");
  SID_REQUIRE(head_dim == QD, "qkv_post: head_dim must be %d, got %d", QD, head_dim);
  SID_REQUIRE(num_q_heads > 0 && num_kv_heads > 0, "qkv_post: bad head counts");
  SID_REQUIRE(q_norm && k_norm && positions && cos_sin && slots && q_out && k_cache && v_cache,
              "qkv_post: null pointer");
  SID_REQUIRE(num_slots > 0, "qkv_post: empty KV pool");
  SID_REQUIRE(num_tokens < (1ll << 31), "qkv_post: too many tokens");
  const int64_t ld = static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * QD;
  const RowSrc src = partials ? part_src(partials, nchunks, num_tokens, ld) : bf_src(qkv, ld);
  const int heads = num_q_heads + 2 * num_kv_heads;
  const dim3 grid((unsigned)num_tokens, (unsigned)ceil_div(heads, 8));
  dispatch_nch(src, [&]<int NCH>() {
    hipLaunchKernelGGL(qkv_post_kernel<NCH>, grid, dim3(128), 0, static_cast<hipStream_t>(stream),
                       src, num_q_heads, num_kv_heads, (const uint4*)q_norm, (const uint4*)k_norm,
                       eps, positions, cos_sin, max_positions, slots, (uint4*)q_out,
                       (uint4*)k_cache, (uint4*)v_cache, num_slots);
  });
  return check_launch("qkv_post");
}
