// Decode-step GEMMs y = x @ w^T on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Reduction order (the determinism contract of sid_linear): K is cut into
// 256-wide chunks; chunk c is accumulated from zero by 8 MFMA k-steps of 32
// in increasing k, and the output is the left fold c0 + c1 + c2 + ... in
// increasing chunk order, then + bias, then one rounding. That order depends
// only on K, never on M, on the tile a row lands in, or on how the chunks are
// spread over workgroups, so a row's bits are identical whether it is computed
// alone or inside any batch (the batch-invariance property that
// sid/kernels/matmul_persistent.py:1-9 buys with a separate slow kernel is
// here true of the one fast kernel).
//
// Tiling for decode shapes (M <= 64 rows per row group, weights streamed once):
//   * workgroup = 4 waves = 64 output columns (wave w owns MFMA column block w)
//     x one row group of up to 64 rows x one or all K chunks;
//   * the row group's x chunk (64 x 256 bf16 = 32 KiB) is staged once in LDS
//     and shared by the 4 waves; each wave issues its 8 weight fragments
//     (16-byte loads, every weight byte read exactly once) before waiting;
//   * split mode (enough workspace, M <= 64): one K chunk per workgroup, so a
//     GEMM with K = 1024..3072 runs 4..12x more workgroups. Each workgroup
//     writes its chunk tile (fp32) to the workspace and bumps the tile's
//     arrival counter; the workgroup that arrives last folds the tile's chunks
//     in chunk order, writes y and resets the counter to zero (so the
//     workspace needs zeroing only once, and graph replays need no memset);
//   * otherwise (huge N such as lm_head, or M > 64) a workgroup walks all
//     chunks itself and folds them in registers in the same order.
#include "common.h"

namespace sid {
namespace {

constexpr int KC = 256;          // chunk width of the canonical reduction order
constexpr int KSTEP = 32;        // MFMA 16x16x32 k-step
constexpr int MROWS = 64;        // rows per row group (4 MFMA row blocks)
constexpr int NTILE = 64;        // columns per workgroup (4 waves x 16)
constexpr int XS = KC + 8;       // LDS row stride of the staged x chunk (bf16 elements)
constexpr int kSplitMinWg = 1024;  // use split mode when tiles x row groups is below this

__device__ __forceinline__ bf16x8_v ld_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_v*>(p);
}

// Stage x[m0 .. m0+rows) x [k0, k0+256) into LDS (rows clamped to M-1).
__device__ __forceinline__ void stage_x(bf16_t* sx, const bf16_t* __restrict__ x, int64_t ldx,
                                        int64_t m0, int64_t M, int rows16, int64_t k0) {
  // 32 16-byte vectors per row; 256 threads -> 8 rows per pass.
  const int tid = threadIdx.x;
  const int vec = tid & 31;
  for (int row = tid >> 5; row < rows16; row += 8) {
    const int64_t gr = min<int64_t>(m0 + row, M - 1);
    *reinterpret_cast<uint4*>(&sx[row * XS + vec * 8]) =
        *reinterpret_cast<const uint4*>(x + gr * ldx + k0 + vec * 8);
  }
}

// One 256-wide chunk of one wave's 16 columns: acc[mb] = sum over the chunk.
__device__ __forceinline__ void chunk_mfma(f32x4_v (&acc)[4], const bf16x8_v (&wf)[KC / KSTEP],
                                           const bf16_t* sx, int mbs, int r, int g) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KC / KSTEP; ++s) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < mbs) {
        const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(&sx[(16 * mb + r) * XS + KSTEP * s + 8 * g]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc[mb], 0, 0, 0);
      }
    }
  }
}

__device__ __forceinline__ void store_out(void* y, int out_fp32, int64_t off, float v) {
  if (out_fp32) {
    static_cast<float*>(y)[off] = round_bf16(v);
  } else {
    static_cast<bf16_t*>(y)[off] = f32_to_bf16(v);
  }
}

__global__ void __launch_bounds__(256) linear_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int out_fp32, float* __restrict__ ws, uint32_t* __restrict__ counters) {
  __shared__ __align__(16) bf16_t sx[MROWS * XS];
  __shared__ int s_last;

  const int nchunks = static_cast<int>(K / KC);
  const bool split = ws != nullptr;
  const int tile = blockIdx.x;
  const int rg = blockIdx.z;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(tile) * NTILE;
  const int64_t m0 = static_cast<int64_t>(rg) * MROWS;
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M - m0));
  const int mbs = (mrows + 15) >> 4;
  const bf16_t* wrow = w + (n0 + 16 * wave + r) * K + 8 * g;

  const int c_begin = split ? static_cast<int>(blockIdx.y) : 0;
  const int c_end = split ? c_begin + 1 : nchunks;

  f32x4_v total[4];
  for (int c = c_begin; c < c_end; ++c) {
    const int64_t k0 = static_cast<int64_t>(c) * KC;
    bf16x8_v wf[KC / KSTEP];
#pragma unroll
    for (int s = 0; s < KC / KSTEP; ++s) wf[s] = ld_frag(wrow + k0 + KSTEP * s);
    if (c != c_begin) __syncthreads();  // previous chunk's x fully consumed
    stage_x(sx, x, ldx, m0, M, mbs * 16, k0);
    __syncthreads();
    f32x4_v acc[4];
    chunk_mfma(acc, wf, sx, mbs, r, g);
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

  // Lane holds rows 16*mb + 4*g + i of column 16*wave + r.
  const int col = 16 * wave + r;
  if (!split) {
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
            store_out(y, out_fp32, (m0 + row) * N + n0 + col, v);
          }
        }
      }
    }
    return;
  }

  // Split mode: park this chunk's tile, count arrivals, the last arrival folds.
  const int ntiles = static_cast<int>(N / NTILE);
  const int64_t tile_id = static_cast<int64_t>(rg) * ntiles + tile;
  float* tile_ws = ws + tile_id * nchunks * (MROWS * NTILE);
  float* mine = tile_ws + static_cast<int64_t>(c_begin) * (MROWS * NTILE);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < mbs) {
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[(16 * mb + 4 * g + i) * NTILE + col] = total[mb][i];
    }
  }
  __threadfence();  // release: this chunk's tile is visible device-wide
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&counters[tile_id], 1u);
    s_last = (prev == static_cast<uint32_t>(nchunks - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // acquire: see every other chunk's tile
  for (int e = threadIdx.x; e < mrows * NTILE; e += 256) {
    const int row = e / NTILE;
    const int cc = e % NTILE;
    const float* p = tile_ws + e;
    float v = __builtin_nontemporal_load(p);
    for (int c = 1; c < nchunks; ++c) v += __builtin_nontemporal_load(p + static_cast<int64_t>(c) * MROWS * NTILE);
    if (bias != nullptr) v += bf16_to_f32(bias[n0 + cc]);
    store_out(y, out_fp32, (m0 + row) * N + n0 + cc, v);
  }
  if (threadIdx.x == 0) atomicExch(&counters[tile_id], 0u);
}

// Workspace layout: [tiles * row groups] uint32 counters (rounded up to 256 bytes), then
// fp32 partial tiles [tiles * row groups][chunks][64][64].
int64_t split_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  const int64_t groups = (m + MROWS - 1) / MROWS;
  const int64_t tiles = n / NTILE;
  const int64_t chunks = k / KC;
  if (groups != 1 || chunks < 2 || tiles * groups >= kSplitMinWg) return 0;
  const int64_t counters = ((tiles * groups * 4 + 255) / 256) * 256;
  return counters + tiles * groups * chunks * MROWS * NTILE * 4;
}

}  // namespace
}  // namespace sid

using namespace sid;

extern "C" int64_t sid_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || n % NTILE != 0 || k % KC != 0) return 0;
  return split_workspace_bytes(m, n, k);
}

extern "C" int sid_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                          int64_t m, int64_t n, int64_t k, int out_fp32, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear: negative size");
  if (m == 0 || n == 0) return SID_OK;
  SID_REQUIRE(x && w && y, "linear: null pointer");
  SID_REQUIRE(k > 0 && k % KC == 0, "linear: K=%lld must be a positive multiple of %d",
              (long long)k, KC);
  SID_REQUIRE(n % NTILE == 0, "linear: N=%lld must be a multiple of %d", (long long)n, NTILE);
  SID_REQUIRE(ldx >= k && ldx % 8 == 0,
              "linear: row stride %lld of x must be >= K and a multiple of 8", (long long)ldx);
  SID_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
              "linear: x and w must be 16-byte aligned");
  const int64_t groups = (m + MROWS - 1) / MROWS;
  const int64_t tiles = n / NTILE;
  SID_REQUIRE(groups <= 65535 && tiles < (1ll << 31), "linear: problem too large");
  const int64_t need = split_workspace_bytes(m, n, k);
  const bool split = need > 0 && workspace != nullptr && workspace_bytes >= need;
  uint32_t* counters = nullptr;
  float* ws = nullptr;
  if (split) {
    SID_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                "linear: workspace must be 256-byte aligned");
    counters = static_cast<uint32_t*>(workspace);
    ws = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                  ((tiles * groups * 4 + 255) / 256) * 256);
  }
  const dim3 grid((unsigned)tiles, split ? (unsigned)(k / KC) : 1u, (unsigned)groups);
  hipLaunchKernelGGL(linear_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     (const bf16_t*)x, ldx, (const bf16_t*)w, (const bf16_t*)bias, y, m, n, k,
                     out_fp32, ws, counters);
  return check_launch("linear");
}
