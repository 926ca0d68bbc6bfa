// Decode-step GEMMs y = x @ w^T on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reduction order (the determinism contract of sid_linear): K is cut into
// 256-wide chunks; chunk c is accumulated from zero by 8 MFMA k-steps of 32
// in increasing k, and the output is the left fold c0 + c1 + c2 + ... in
// increasing chunk order, then + bias, then one rounding to bf16. That order
// depends only on K, never on M, on the tile a row lands in, or on which
// kernel folds the chunks, so a row's bits are identical whether it is
// computed alone or inside any batch (the batch-invariance property that
// sid/kernels/matmul_persistent.py:1-9 buys with a separate slow kernel is
// here true of the one fast kernel).
//
// Tiling (decode: M <= 64 rows per row group; weights are the HBM stream):
//   * workgroup = 4 waves = 64 output columns (wave w owns MFMA column block w)
//     x one row group of up to 64 rows;
//   * the row group's x chunk (64 x 256 bf16 = 32 KiB) is staged in LDS and
//     shared by the 4 waves, and each wave streams its weight rows straight
//     into MFMA B operands (16-byte loads, every weight byte read once);
//   * direct mode (sid_linear): a workgroup walks every chunk, prefetching the
//     next chunk's weights and x into registers while the MFMAs of the current
//     one run, and folds in registers;
//   * partial mode (sid_linear_partials): one chunk per workgroup (4..12x more
//     workgroups for K = 1024..3072, which the small-N decode projections need
//     to fill 256 CUs) writing its fp32 chunk tile to partials[c][m][n]; the
//     consumer kernel folds the chunks in order (see norm_rope.hip). No
//     cross-workgroup synchronisation: the kernel boundary orders the two.
#include "common.h"

namespace sid {
namespace {

constexpr int KC = 256;      // chunk width of the canonical reduction order
constexpr int KSTEP = 32;    // MFMA 16x16x32 k-step
constexpr int NSTEP = KC / KSTEP;
constexpr int MROWS = 64;    // rows per row group (4 MFMA row blocks)
constexpr int NTILE_MIN = 64;  // column granularity (4 waves x 16); N must be a multiple
constexpr int XS = KC + 8;   // LDS row stride of the staged x chunk (bf16 elements)

__device__ __forceinline__ bf16x8_v ld_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_v*>(p);
}

// x chunk in registers: thread t holds 16-byte vector t%32 of rows t/32 + 2*NW*i. The
// row-count test is written per pass (i < rows16 / (2*NW), uniform over the workgroup
// because rows16 is a multiple of 16 and 2*NW divides 16 or is 32), which keeps the 8 vectors in registers: a per-lane test
// here, or HIP's struct-wrapped uint4 as the element type, made the compiler demote them
// to scratch and serialise every load (native vector types stay in registers).
template <int NW>
__device__ __forceinline__ void load_x(bf16x8_v (&xv)[8], const bf16_t* __restrict__ x, int64_t ldx,
                                       int64_t m0, int64_t M, int rows16, int64_t k0) {
  constexpr int RPP = NW * 2;  // rows per pass: 32 threads per row
  const int tid = threadIdx.x;
  const int vec = tid & 31;
  const int passes = rows16 / RPP;
#pragma unroll
  for (int i = 0; i < 64 / RPP; ++i) {
    if (i < passes) {
      const int row = (tid >> 5) + RPP * i;
      const int64_t gr = min<int64_t>(m0 + row, M - 1);  // rows >= M are clamped and discarded
      xv[i] = ld_frag(x + gr * ldx + k0 + vec * 8);
    }
  }
}

template <int NW>
__device__ __forceinline__ void store_x(bf16_t* sx, const bf16x8_v (&xv)[8], int rows16) {
  constexpr int RPP = NW * 2;
  const int tid = threadIdx.x;
  const int vec = tid & 31;
  const int passes = rows16 / RPP;
#pragma unroll
  for (int i = 0; i < 64 / RPP; ++i) {
    if (i < passes) {
      const int row = (tid >> 5) + RPP * i;
      *reinterpret_cast<bf16x8_v*>(&sx[row * XS + vec * 8]) = xv[i];
    }
  }
}

__device__ __forceinline__ void load_w(bf16x8_v (&wf)[NSTEP], const bf16_t* wrow, int64_t k0) {
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) wf[s] = ld_frag(wrow + k0 + KSTEP * s);
}

// One chunk of one wave's 16 columns: acc[mb] = sum over the chunk, from zero.
__device__ __forceinline__ void chunk_mfma(f32x4_v (&acc)[4], const bf16x8_v (&wf)[NSTEP],
                                           const bf16_t* sx, int mbs, int r, int g) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < mbs) {
        const bf16x8_v af =
            *reinterpret_cast<const bf16x8_v*>(&sx[(16 * mb + r) * XS + KSTEP * s + 8 * g]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc[mb], 0, 0, 0);
      }
    }
  }
}

// partials == nullptr: direct mode (all chunks, y written). Otherwise partial mode:
// chunk blockIdx.y only, fp32 tile written to partials[chunk][row][col].
// NW waves per workgroup = 16*NW columns sharing one staged x chunk.
// PF: prefetch the next chunk's weights and x during the current chunk's MFMAs (more
// registers, fewer resident workgroups) instead of loading at the top of each chunk.
template <int NW, bool PF = true>
__global__ void __launch_bounds__(NW * 64) linear_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int out_fp32, float* __restrict__ partials) {
  __shared__ __align__(16) bf16_t sx[MROWS * XS];

  const int nchunks = static_cast<int>(K / KC);
  const bool partial = partials != nullptr;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * NW);
  const int64_t m0 = static_cast<int64_t>(blockIdx.z) * MROWS;
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M - m0));
  const int mbs = (mrows + 15) >> 4;
  const int rows16 = mbs * 16;
  const bf16_t* wrow = w + (n0 + 16 * wave + r) * K + 8 * g;
  const int col = 16 * wave + r;

  const int c_begin = partial ? static_cast<int>(blockIdx.y) : 0;
  const int c_end = partial ? c_begin + 1 : nchunks;

  bf16x8_v wf[NSTEP];
  bf16x8_v xr[8];
  load_w(wf, wrow, static_cast<int64_t>(c_begin) * KC);
  load_x<NW>(xr, x, ldx, m0, M, rows16, static_cast<int64_t>(c_begin) * KC);

  f32x4_v total[4];
  for (int c = c_begin; c < c_end; ++c) {
    if (c != c_begin) {
      __syncthreads();  // previous chunk's x fully consumed
      if constexpr (!PF) {
        load_w(wf, wrow, static_cast<int64_t>(c) * KC);
        load_x<NW>(xr, x, ldx, m0, M, rows16, static_cast<int64_t>(c) * KC);
      }
    }
    store_x<NW>(sx, xr, rows16);
    __syncthreads();
    bf16x8_v wcur[NSTEP];
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) wcur[s] = wf[s];
    if (PF && c + 1 < c_end) {  // prefetch the next chunk while this one computes
      load_w(wf, wrow, static_cast<int64_t>(c + 1) * KC);
      load_x<NW>(xr, x, ldx, m0, M, rows16, static_cast<int64_t>(c + 1) * KC);
    }
    f32x4_v acc[4];
    chunk_mfma(acc, wcur, sx, mbs, r, g);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (c == c_begin) {
        total[mb] = acc[mb];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) total[mb][i] += acc[mb][i];
      }
    }
  }

  // Lane holds rows 16*mb + 4*g + i of column `col`.
  if (partial) {
    float* dst = partials + (static_cast<int64_t>(c_begin) * M + m0) * N + n0 + col;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < mbs) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * mb + 4 * g + i;
          if (row < mrows) dst[static_cast<int64_t>(row) * N] = total[mb][i];
        }
      }
    }
    return;
  }
  const float bv = bias != nullptr ? bf16_to_f32(bias[n0 + col]) : 0.0f;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < mbs) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * g + i;
        if (row < mrows) {
          float v = total[mb][i];
          if (bias != nullptr) v += bv;
          const int64_t off = (m0 + row) * N + n0 + col;
          if (out_fp32) {
            static_cast<float*>(y)[off] = round_bf16(v);
          } else {
            static_cast<bf16_t*>(y)[off] = f32_to_bf16(v);
          }
        }
      }
    }
  }
}

// Wide-N, K = 1024, M <= 64 (lm_head at decode): every weight fragment of the workgroup's
// 16*NW columns for all four chunks is requested up front (128 VGPRs), the whole x row
// group is staged once in LDS (64 x 1032 bf16), then the chunks are reduced in order.
// One workgroup per CU, 256 KiB of weights in flight per CU. Same per-element
// arithmetic as linear_kernel, so the bits are identical.
constexpr int WIDE_K = 1024;
constexpr int WIDE_NCH = WIDE_K / KC;
constexpr int WXS = WIDE_K + 8;

template <int NW>
__global__ void __launch_bounds__(NW * 64) linear_wide_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int out_fp32) {
  extern __shared__ __align__(16) bf16_t wsx[];  // [rows16][WXS]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * NW);
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M));
  const int mbs = (mrows + 15) >> 4;
  const int rows16 = mbs * 16;
  const bf16_t* wrow = w + (n0 + 16 * wave + r) * WIDE_K + 8 * g;
  const int col = 16 * wave + r;

  bf16x8_v wf[WIDE_NCH][NSTEP];
#pragma unroll
  for (int c = 0; c < WIDE_NCH; ++c) load_w(wf[c], wrow, static_cast<int64_t>(c) * KC);

  // x: 128 16-byte vectors per row; NW*64 threads -> NW/2 rows per pass.
  constexpr int VPT = MROWS * (WIDE_K / 8) / (NW * 64);  // vectors per thread for 64 rows
  bf16x8_v xv[VPT];
  const int vec = threadIdx.x & 127;
  const int row0 = threadIdx.x >> 7;
  constexpr int RPP = NW / 2;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int row = row0 + RPP * i;
    if (row < rows16) {
      const int64_t gr = min<int64_t>(row, M - 1);
      xv[i] = ld_frag(x + gr * ldx + vec * 8);
    }
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int row = row0 + RPP * i;
    if (row < rows16) *reinterpret_cast<bf16x8_v*>(&wsx[row * WXS + vec * 8]) = xv[i];
  }
  __syncthreads();

  f32x4_v total[4];
#pragma unroll
  for (int c = 0; c < WIDE_NCH; ++c) {
    f32x4_v acc[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < mbs) {
          const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(
              &wsx[(16 * mb + r) * WXS + c * KC + KSTEP * s + 8 * g]);
          acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[c][s], acc[mb], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (c == 0) {
        total[mb] = acc[mb];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) total[mb][i] += acc[mb][i];
      }
    }
  }
  const float bv = bias != nullptr ? bf16_to_f32(bias[n0 + col]) : 0.0f;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < mbs) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * g + i;
        if (row < mrows) {
          float v = total[mb][i];
          if (bias != nullptr) v += bv;
          const int64_t off = static_cast<int64_t>(row) * N + n0 + col;
          if (out_fp32) {
            static_cast<float*>(y)[off] = round_bf16(v);
          } else {
            static_cast<bf16_t*>(y)[off] = f32_to_bf16(v);
          }
        }
      }
    }
  }
}

int check_shapes(const void* x, int64_t ldx, const void* w, int64_t m, int64_t n, int64_t k,
                 const char* name) {
  SID_REQUIRE(x && w, "%s: null pointer", name);
  SID_REQUIRE(k > 0 && k % KC == 0, "%s: K=%lld must be a positive multiple of %d", name,
              (long long)k, KC);
  SID_REQUIRE(n % NTILE_MIN == 0, "%s: N=%lld must be a multiple of %d", name, (long long)n,
              NTILE_MIN);
  SID_REQUIRE(ldx >= k && ldx % 8 == 0,
              "%s: row stride %lld of x must be >= K and a multiple of 8", name, (long long)ldx);
  SID_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
              "%s: x and w must be 16-byte aligned", name);
  SID_REQUIRE((m + MROWS - 1) / MROWS <= 65535 && n / NTILE_MIN < (1ll << 31),
              "%s: problem too large", name);
  return SID_OK;
}

template <int NW, bool PF = true>
void launch_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t m,
                   int64_t n, int64_t k, int out_fp32, float* partials, hipStream_t stream) {
  const dim3 grid((unsigned)(n / (16 * NW)), partials ? (unsigned)(k / KC) : 1u,
                  (unsigned)((m + MROWS - 1) / MROWS));
  hipLaunchKernelGGL((linear_kernel<NW, PF>), grid, dim3(NW * 64), 0, stream, (const bf16_t*)x, ldx,
                     (const bf16_t*)w, (const bf16_t*)bias, y, m, n, k, out_fp32, partials);
}

// Waves per workgroup: more waves share one staged x chunk (less L2->LDS traffic per
// weight byte) but leave fewer workgroups; wide direct GEMMs (lm_head, prefill) use 8.
// (16 waves would cap the kernel at 128 VGPRs and spill.)
int pick_waves(int64_t n, int64_t m, bool partial) {
  if (partial) return 4;
  const int64_t groups = (m + MROWS - 1) / MROWS;
  if (n % 128 == 0 && (n / 128) * groups >= 512) return 8;
  return 4;
}

void launch_any(int nw, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                int64_t m, int64_t n, int64_t k, int out_fp32, float* partials, hipStream_t s) {
  switch (nw) {
    case 8: return launch_linear<8>(x, ldx, w, bias, y, m, n, k, out_fp32, partials, s);
    default: return launch_linear<4>(x, ldx, w, bias, y, m, n, k, out_fp32, partials, s);
  }
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int sid_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                          int64_t m, int64_t n, int64_t k, int out_fp32, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear: negative size");
  if (m == 0 || n == 0) return SID_OK;
  SID_REQUIRE(y != nullptr, "linear: null output");
  int rc = check_shapes(x, ldx, w, m, n, k, "linear");
  if (rc != SID_OK) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (m <= MROWS && k == WIDE_K && n % 128 == 0 && n / 128 >= 512) {
    static bool lds_ok = false;
    const size_t lds = static_cast<size_t>(MROWS) * WXS * sizeof(bf16_t);
    if (!lds_ok) {
      hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_wide_kernel<8>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
      lds_ok = true;
    }
    const size_t lds_used = static_cast<size_t>((m + 15) / 16 * 16) * WXS * sizeof(bf16_t);
    hipLaunchKernelGGL(linear_wide_kernel<8>, dim3((unsigned)(n / 128)), dim3(512), lds_used, s,
                       (const bf16_t*)x, ldx, (const bf16_t*)w, (const bf16_t*)bias, y, m, n,
                       out_fp32);
    return check_launch("linear");
  }
  launch_any(pick_waves(n, m, false), x, ldx, w, bias, y, m, n, k, out_fp32, nullptr, s);
  return check_launch("linear");
}

extern "C" int sid_linear_partials(const void* x, int64_t ldx, const void* w, float* partials,
                                   int64_t m, int64_t n, int64_t k, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear_partials: negative size");
  if (m == 0 || n == 0) return SID_OK;
  SID_REQUIRE(partials != nullptr, "linear_partials: null output");
  int rc = check_shapes(x, ldx, w, m, n, k, "linear_partials");
  if (rc != SID_OK) return rc;
  SID_REQUIRE(k / KC <= 65535, "linear_partials: too many chunks");
  launch_any(pick_waves(n, m, true), x, ldx, w, nullptr, nullptr, m, n, k, 0, partials,
             static_cast<hipStream_t>(stream));
  return check_launch("linear_partials");
}
