// Decode-step GEMMs y = x @ w^T on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reduction order (the determinism contract of sid_linear): K is cut into
// 256-wide chunks; chunk c is accumulated from zero by 8 MFMA k-steps of 32
// in increasing k, and the output is the left fold c0 + c1 + c2 + ... in
// increasing chunk order, plus the bias. That order depends only on K, never
// on M or on the tile a row lands in, so a row's result is bitwise identical
// whether it is computed alone or inside any batch (the batch-invariance
// property of sid/kernels/matmul_persistent.py:1-9, here true in every mode).
//
// Skinny kernel (decode shapes, M <= 64 per row group): a workgroup owns 16*NB
// output columns and up to 64 rows; its waves take the K chunks in parallel
// (wave w: chunks w, w + waves, ...), stream the weight rows straight from
// HBM into MFMA B operands (16-byte loads, each weight byte read once per row
// group), take A operands from x (small, L2-resident), park each chunk's
// partial tile in LDS, and after one barrier fold the chunks in order.
#include "common.h"

namespace sid {
namespace {

constexpr int KC = 256;        // chunk width of the canonical reduction order
constexpr int KSTEP = 32;      // MFMA 16x16x32 k-step
constexpr int MROWS = 64;      // rows per row group (4 MFMA row blocks)

__device__ __forceinline__ bf16x8_v ld_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_v*>(p);
}

template <int NB>
__global__ void __launch_bounds__(1024) linear_skinny_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int out_fp32) {
  constexpr int NT = 16 * NB;
  constexpr int RS = NT + 4;  // LDS row stride (floats): spreads the 4 lane groups over banks
  extern __shared__ float red[];  // [nchunks][MROWS][RS]

  const int nchunks = static_cast<int>(K / KC);
  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MROWS;
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M - m0));
  const int mbs = (mrows + 15) >> 4;

  const bf16_t* arow[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int64_t row = min<int64_t>(m0 + 16 * mb + r, M - 1);  // clamp: rows >= M are discarded
    arow[mb] = x + row * ldx + 8 * g;
  }
  const bf16_t* brow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) brow[nb] = w + (n0 + 16 * nb + r) * K + 8 * g;

  for (int c = wave; c < nchunks; c += nw) {
    f32x4_v acc[4][NB];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};

    const int64_t kc = static_cast<int64_t>(c) * KC;
#pragma unroll
    for (int s = 0; s < KC / KSTEP; ++s) {
      const int64_t k = kc + s * KSTEP;
      bf16x8_v bf[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bf[nb] = ld_frag(brow[nb] + k);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < mbs) {
          const bf16x8_v af = ld_frag(arow[mb] + k);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[nb], acc[mb][nb], 0, 0, 0);
        }
      }
    }
    float* dst = red + static_cast<int64_t>(c) * MROWS * RS;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < mbs) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[(16 * mb + 4 * g + i) * RS + 16 * nb + r] = acc[mb][nb][i];
      }
    }
  }
  __syncthreads();

  for (int e = threadIdx.x; e < mrows * NT; e += blockDim.x) {
    const int row = e / NT;
    const int col = e % NT;
    float t = red[row * RS + col];
    for (int c = 1; c < nchunks; ++c) t += red[(static_cast<int64_t>(c) * MROWS + row) * RS + col];
    if (bias != nullptr) t += bf16_to_f32(bias[n0 + col]);
    const int64_t off = (m0 + row) * N + n0 + col;
    if (out_fp32) {
      static_cast<float*>(y)[off] = round_bf16(t);
    } else {
      static_cast<bf16_t*>(y)[off] = f32_to_bf16(t);
    }
  }
}

constexpr int kMaxLds = 160 * 1024;

template <int NB>
int launch_skinny(const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                  int64_t m, int64_t n, int64_t k, int out_fp32, hipStream_t stream) {
  constexpr int NT = 16 * NB;
  const int nchunks = static_cast<int>(k / KC);
  const int nw = nchunks < 16 ? nchunks : 16;
  const size_t lds = static_cast<size_t>(nchunks) * MROWS * (NT + 4) * sizeof(float);
  SID_REQUIRE(lds <= (size_t)kMaxLds, "linear: K=%lld needs %zu bytes of LDS (max %d)",
              (long long)k, lds, kMaxLds);
  const int64_t gy = (m + MROWS - 1) / MROWS;
  SID_REQUIRE(gy <= 65535, "linear: M=%lld too large", (long long)m);
  static bool configured = false;
  if (!configured) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_skinny_kernel<NB>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    configured = true;
  }
  hipLaunchKernelGGL(linear_skinny_kernel<NB>, dim3((unsigned)(n / NT), (unsigned)gy),
                     dim3(nw * 64), lds, stream, (const bf16_t*)x, ldx, (const bf16_t*)w,
                     (const bf16_t*)bias, y, m, n, k, out_fp32);
  return check_launch("linear");
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                          int64_t m, int64_t n, int64_t k, int out_fp32, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear: negative size");
  if (m == 0 || n == 0) return SID_OK;
  SID_REQUIRE(x && w && y, "linear: null pointer");
  SID_REQUIRE(k > 0 && k % KC == 0, "linear: K=%lld must be a positive multiple of %d",
              (long long)k, KC);
  SID_REQUIRE(n % 16 == 0, "linear: N=%lld must be a multiple of 16", (long long)n);
  SID_REQUIRE(ldx >= k && ldx % 8 == 0, "linear: row stride %lld of x must be >= K and a multiple of 8",
              (long long)ldx);
  SID_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
              "linear: x and w must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t row_groups = (m + MROWS - 1) / MROWS;
  if (n % 32 == 0 && (n / 32) * row_groups >= 1024) {
    return launch_skinny<2>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
  }
  return launch_skinny<1>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
}
