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
// Kernels (all with that order):
//   * linear_chunk_kernel: split-K partials for decode-sized M (sid_linear_partials): one
//     256-wide chunk of 64 columns per 4-wave workgroup, x chunk staged in LDS, weights
//     streamed straight into MFMA B operands; writes partials[c][m][n], which the consumer
//     kernel folds in chunk order (norm_rope.hip). No cross-workgroup synchronisation.
//   * linear_kernel: direct y for M < 64 in one row group, every chunk of a column tile
//     in one workgroup with the next chunk's operands prefetched during the MFMAs;
//   * linear_tiled_kernel: direct y for M >= 64 (prefill, and decode / verify rows past the
//     split-K cuts), LDS-tiled 128 x 128 / 128 x 64; also gate_up with the SwiGLU epilogue;
//   * linear_stream_kernel: lm_head-shaped N (persistent grid, x staged once per CU), with
//     an optional fused greedy argmax.
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

// Direct y = x w^T (+ bias) for one 64-row group and 16*NW columns: every chunk in order,
// the next chunk's weights and x prefetched into registers during the current chunk's
// MFMAs. NW waves share one staged x chunk.
template <int NW>
__global__ void __launch_bounds__(NW * 64) linear_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int out_fp32) {
  __shared__ __align__(16) bf16_t sx[MROWS * XS];

  const int nchunks = static_cast<int>(K / KC);
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

  const int c_begin = 0;
  const int c_end = nchunks;

  bf16x8_v wf[NSTEP];
  bf16x8_v xr[8];
  load_w(wf, wrow, static_cast<int64_t>(c_begin) * KC);
  load_x<NW>(xr, x, ldx, m0, M, rows16, static_cast<int64_t>(c_begin) * KC);

  f32x4_v total[4];
  for (int c = c_begin; c < c_end; ++c) {
    if (c != c_begin) __syncthreads();  // previous chunk's x fully consumed
    store_x<NW>(sx, xr, rows16);
    __syncthreads();
    bf16x8_v wcur[NSTEP];
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) wcur[s] = wf[s];
    if (c + 1 < c_end) {  // prefetch the next chunk while this one computes
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

// Partial mode: one 256-wide chunk per workgroup (blockIdx.y), fp32 tile written to
// partials[chunk][row][col]. MBS (16-row blocks in the row group) is a compile-time
// constant so the 8 x MBS MFMAs and their LDS reads are straight-line code; the chunk's
// MFMA sequence is chunk_mfma's, so the partials are the bits linear_kernel folds.
template <int NW, int MBS>
__global__ void __launch_bounds__(NW * 64) linear_chunk_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w, int64_t M, int64_t N,
    int64_t K, float* __restrict__ partials) {
  __shared__ __align__(16) bf16_t sx[MBS * 16 * XS];
  constexpr int RPP = NW * 2;  // x rows per pass: 32 threads per row
  constexpr int PASSES = (MBS * 16 + RPP - 1) / RPP;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * NW);
  const int c = blockIdx.y;
  const int64_t m0 = static_cast<int64_t>(blockIdx.z) * MROWS;
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M - m0));
  const int64_t k0 = static_cast<int64_t>(c) * KC;

  bf16x8_v wf[NSTEP];
  load_w(wf, w + (n0 + 16 * wave + r) * K + 8 * g, k0);
  bf16x8_v xv[PASSES];
  const int vec = threadIdx.x & 31;
#pragma unroll
  for (int i = 0; i < PASSES; ++i) {
    const int row = (threadIdx.x >> 5) + RPP * i;
    const int64_t gr = min<int64_t>(m0 + min(row, MBS * 16 - 1), M - 1);  // clamped, discarded
    xv[i] = ld_frag(x + gr * ldx + k0 + vec * 8);
  }
#pragma unroll
  for (int i = 0; i < PASSES; ++i) {
    const int row = (threadIdx.x >> 5) + RPP * i;
    if (row < MBS * 16) *reinterpret_cast<bf16x8_v*>(&sx[row * XS + vec * 8]) = xv[i];
  }
  __syncthreads();
  f32x4_v acc[MBS];
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
      const bf16x8_v af =
          *reinterpret_cast<const bf16x8_v*>(&sx[(16 * mb + r) * XS + KSTEP * s + 8 * g]);
      acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc[mb], 0, 0, 0);
    }
  }
  float* dst = partials + (static_cast<int64_t>(c) * M + m0) * N + n0 + 16 * wave + r;
  if (mrows == MBS * 16) {  // full row group (uniform): unguarded stores
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[static_cast<int64_t>(16 * mb + 4 * g + i) * N] = acc[mb][i];
    }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * mb + 4 * g + i;
      if (row < mrows) dst[static_cast<int64_t>(row) * N] = acc[mb][i];
    }
  }
}

// Greedy argmax order over (value, column), torch's: larger value, then smaller index; NaN
// above everything, first NaN wins. A total order, so a maximum over any split of the
// columns into candidates, reduced in any order, is the same (value, column).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  const bool vn = v != v;
  const bool bn = bv != bv;
  if (vn || bn) {
    if (vn && bn) return i < bi;
    return vn;
  }
  return v > bv || (v == bv && i < bi);
}

struct SampleStats {
  float* mx;
  float* sm;
  float* a1v;
  float* a1x;
  float* a2v;
  int* a1i;
};

__device__ __forceinline__ void softmax_merge(float& m, float& s, float om, float os) {
  const float nm = fmaxf(m, om);
  const float a = m == -INFINITY ? 0.0f : s * expf(m - nm);
  const float b = om == -INFINITY ? 0.0f : os * expf(om - nm);
  m = nm;
  s = a + b;
}

// One lane's sampler statistics over the columns it has seen (see linear_sample_kernel):
// greedy rows keep only (v1, i1) = the best (logit, column) under argmax_better.
struct SState {
  float m, s, v1, x1, v2;
  int i1;
};

__device__ __forceinline__ SState sstate_empty() {
  return SState{-INFINITY, 0.0f, -INFINITY, -INFINITY, -INFINITY, 0x7fffffff};
}

// Column `col` with bf16-rounded logit vr, for a row with temperature t and noise row hash h.
__device__ __forceinline__ void sstate_add(SState& a, float vr, int col, float t, uint32_t h) {
  if (!(t > 0.0f)) {
    if (argmax_better(vr, col, a.v1, a.i1)) {
      a.v1 = vr;
      a.i1 = col;
    }
    return;
  }
  const float xv = vr / t;
  if (xv > a.m) {
    a.s = a.s * expf(a.m - xv) + 1.0f;
    a.m = xv;
  } else {
    a.s += expf(xv - a.m);
  }
  const float xg = xv + seeded_gumbel(h, col);
  if (xg > a.v1 || (xg == a.v1 && col < a.i1)) {
    a.v2 = a.v1;
    a.v1 = xg;
    a.x1 = xv;
    a.i1 = col;
  } else {
    a.v2 = fmaxf(a.v2, xg);
  }
}

// a <- a merged with b (a fixed function of the two states).
__device__ __forceinline__ void sstate_merge(SState& a, const SState& b, bool greedy) {
  if (greedy) {
    if (argmax_better(b.v1, b.i1, a.v1, a.i1)) {
      a.v1 = b.v1;
      a.i1 = b.i1;
    }
    return;
  }
  softmax_merge(a.m, a.s, b.m, b.s);
  if (b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1)) {
    a.v2 = fmaxf(a.v1, b.v2);
    a.v1 = b.v1;
    a.x1 = b.x1;
    a.i1 = b.i1;
  } else {
    a.v2 = fmaxf(a.v2, fmaxf(b.v1, b.v2));
  }
}

// Merge over the 16 lanes of a DPP row (xor butterfly; every lane ends with the same state).
__device__ __forceinline__ void sstate_merge16(SState& a, bool greedy) {
  const int lane = __lane_id();
#pragma unroll
  for (int mask = 1; mask < 16; mask <<= 1) {
    SState b;
    b.m = lane_xor(a.m, mask);
    b.s = lane_xor(a.s, mask);
    b.v1 = lane_xor(a.v1, mask);
    b.x1 = lane_xor(a.x1, mask);
    b.v2 = lane_xor(a.v2, mask);
    b.i1 = __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, a.i1);
    sstate_merge(a, b, greedy);
  }
}

__device__ __forceinline__ void sstate_store(const SampleStats& st, int64_t o, const SState& a) {
  st.mx[o] = a.m;
  st.sm[o] = a.s;
  st.a1v[o] = a.v1;
  st.a1x[o] = a.x1;
  st.a2v[o] = a.v2;
  st.a1i[o] = a.i1;
}

// Per-row inputs of a fused sampler epilogue; statistics go to st at [group][cand_rows].
struct SampleIn {
  const float* temps;
  const int64_t* seeds;
  const int64_t* positions;
  SampleStats st;
  int64_t cand_rows;
};

// ---- large-M tiled GEMM (prefill) ---------------------------------------------------------
//
// 128 x 128 output tile per 4-wave workgroup (wave (wm, wn): 64 x 64 = 4 x 4 MFMA blocks),
// K streamed in 64-deep sub-tiles through double-buffered LDS (the next sub-tile's x and w
// rows are loaded into registers while the current one's MFMAs run). Every output element
// sees the canonical order: each 256-wide chunk accumulated from zero by 8 MFMA k-steps in
// increasing k (two per sub-tile), the chunk sums left-folded c0 + c1 + ..., then + bias and
// one rounding; the operand layout per MFMA is linear_kernel's. So the bits equal
// sid_linear's for any M, while the tile reuse (each x row feeds 128 columns, each weight
// row 128 rows) makes large M MFMA-bound instead of bound by re-reading operands.
constexpr int TT_K = 64;
// LDS row stride (bf16): 160 bytes. (Layout only; measured against 144 bytes, which
// allows two workgroups per CU: 3-13% faster on prefill shapes M = 1024-8192, e.g. qkv at
// M = 8192 95.6 -> 88.4 us, o at M = 4096 33.1 -> 29.3 us; an XOR-swizzled unpadded layout
// measured the same as this padding.)
constexpr int TT_KS = TT_K + 16;
constexpr int TT_SUB_PER_CHUNK = KC / TT_K;

// WM x WN waves; wave (wm, wn) owns MB x NB MFMA blocks = (16 MB) x (16 NB) outputs.
// PF = 1: the next sub-tile is loaded into registers during the current one's MFMAs, and the
// compiler schedules the loads among them (best when the grid fills the chip: the MFMAs
// are the bound). PF = 2: a ring of two register buffers keeps two sub-tiles in flight,
// issued at fixed points (best for grids of at most one workgroup per CU, where every
// sub-tile's global-memory latency would otherwise be exposed). Same arithmetic either way.
//
// AM (greedy lm_head): the epilogue also keeps each row's best (bf16-rounded logit, column)
// over the tile's columns, in argmax_better's order, and writes it to
// best_val / best_idx [blockIdx.x][M] for argmax_finalize_kernel; y may then be null (no
// logits written).
//
// SW (gate_up + SwiGLU, weights [gate rows | up rows] of inter rows each): the tile's first
// NB/2 column blocks of each wave are gate rows and the last NB/2 the up rows of the same
// inter columns, so a lane holds both values of its outputs; the epilogue writes
// act[row][c] = silu_mul1(gate, up) of the bf16-rounded projections ([M, inter], the bits of
// sid_silu_mul over sid_linear's output) and no projection.
template <int WM, int WN, int MB, int NB, int PF, bool AM = false, bool SW = false,
          bool SP = false>
__global__ void __launch_bounds__(WM * WN * 64, (AM || SP) ? 4 : 1) linear_tiled_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int64_t M, int64_t N, int64_t K,
    int out_fp32, float* __restrict__ best_val, int* __restrict__ best_idx, SampleIn sp) {
  constexpr int TM = WM * MB * 16;
  constexpr int TN = WN * NB * 16;
  constexpr int THREADS = WM * WN * 64;
  constexpr int LA = TM * (TT_K / 8) / THREADS;  // 16-byte x vectors per thread per sub-tile
  constexpr int LB = TN * (TT_K / 8) / THREADS;
  static_assert(LA * THREADS == TM * (TT_K / 8) && LB * THREADS == TN * (TT_K / 8), "tile");
  __shared__ __align__(16) bf16_t sa[2][TM * TT_KS];
  __shared__ __align__(16) bf16_t sb[2][TN * TT_KS];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * TN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * TM;

  // Sub-tile loads (8 vectors of 16 bytes per 64-deep row). Rows past M (x) or N (w) are
  // clamped to the last valid row; their results are dropped.
  const bf16_t* xrow[LA];
  const bf16_t* wrow[LB];
  int arow[LA], avec[LA], brow[LB], bvec[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int v = tid + THREADS * i;
    arow[i] = v >> 3;
    avec[i] = v & 7;
    xrow[i] = x + min<int64_t>(m0 + arow[i], M - 1) * ldx + avec[i] * 8;
  }
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int v = tid + THREADS * i;
    brow[i] = v >> 3;
    bvec[i] = v & 7;
    int64_t wr = n0 + brow[i];
    if constexpr (SW) {  // LDS row j = wave column block's row: gate or up row of column c
      static_assert(NB % 2 == 0, "SwiGLU tiles pair gate and up column blocks");
      const int jw = brow[i] / (NB * 16);
      const int jb = (brow[i] / 16) % NB;
      const int64_t c = blockIdx.x * (TN / 2) + jw * (NB / 2) * 16 + (jb % (NB / 2)) * 16 +
                        (brow[i] % 16);
      wr = jb < NB / 2 ? c : N / 2 + c;
    }
    wrow[i] = w + min<int64_t>(wr, N - 1) * K + bvec[i] * 8;
  }
  static_assert(PF == 1 || PF == 2 || PF == 4, "PF must divide the 4 sub-tiles of a chunk");
  bf16x8_v ra[PF][LA], rb[PF][LB];
  auto load_sub = [&](int kt, bf16x8_v (&da)[LA], bf16x8_v (&db)[LB]) {
    const int64_t k0 = static_cast<int64_t>(kt) * TT_K;
#pragma unroll
    for (int i = 0; i < LA; ++i) da[i] = ld_frag(xrow[i] + k0);
#pragma unroll
    for (int i = 0; i < LB; ++i) db[i] = ld_frag(wrow[i] + k0);
  };
  auto store_sub = [&](int buf, const bf16x8_v (&da)[LA], const bf16x8_v (&db)[LB]) {
#pragma unroll
    for (int i = 0; i < LA; ++i)
      *reinterpret_cast<bf16x8_v*>(&sa[buf][arow[i] * TT_KS + avec[i] * 8]) = da[i];
#pragma unroll
    for (int i = 0; i < LB; ++i)
      *reinterpret_cast<bf16x8_v*>(&sb[buf][brow[i] * TT_KS + bvec[i] * 8]) = db[i];
  };

  f32x4_v acc[MB][NB], tot[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // One sub-tile's MFMAs out of LDS buffer `cur`, and the fold at the end of a chunk.
  auto mma_sub = [&](int cur) {
#pragma unroll
    for (int s = 0; s < TT_K / KSTEP; ++s) {
      bf16x8_v af[MB], bfv[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *reinterpret_cast<const bf16x8_v*>(
            &sa[cur][(MB * 16 * wm + 16 * mb + r) * TT_KS + KSTEP * s + 8 * g]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bfv[nb] = *reinterpret_cast<const bf16x8_v*>(
            &sb[cur][(NB * 16 * wn + 16 * nb + r) * TT_KS + KSTEP * s + 8 * g]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mb], bfv[nb], acc[mb][nb], 0, 0, 0);
      }
    }
  };
  auto fold = [&](bool first) {  // chunk complete: fold, restart
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (first) {
          tot[mb][nb] = acc[mb][nb];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) tot[mb][nb][i] += acc[mb][nb][i];
        }
        acc[mb][nb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  };

  const int nsub = static_cast<int>(K / TT_K);  // a multiple of 4 (K is a multiple of 256)
  if constexpr (PF == 1) {
    load_sub(0, ra[0], rb[0]);
    store_sub(0, ra[0], rb[0]);
    __syncthreads();
    for (int kt = 0; kt < nsub; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nsub) load_sub(kt + 1, ra[0], rb[0]);
      mma_sub(cur);
      if (kt % TT_SUB_PER_CHUNK == TT_SUB_PER_CHUNK - 1) fold(kt < TT_SUB_PER_CHUNK);
      if (kt + 1 < nsub) {
        store_sub(cur ^ 1, ra[0], rb[0]);
        __syncthreads();
      }
    }
  } else {
    // One 256-wide chunk (4 sub-tiles) per outer iteration. Sub-tile t lives in register
    // slot t % PF until it is stored to LDS buffer t & 1. The loads PF sub-tiles ahead are
    // unconditional (indices clamped to the last sub-tile, whose repeats are stored but
    // never read), so the loop is straight-line and each store waits only for its own
    // slot's loads; a scheduling barrier keeps each batch of loads where it is issued.
    load_sub(0, ra[0], rb[0]);
    store_sub(0, ra[0], rb[0]);
#pragma unroll
    for (int p = 1; p <= PF; ++p) load_sub(min(p, nsub - 1), ra[p % PF], rb[p % PF]);
    __syncthreads();
    const int nch = nsub / TT_SUB_PER_CHUNK;
    for (int c = 0; c < nch; ++c) {
#pragma unroll
      for (int j = 0; j < TT_SUB_PER_CHUNK; ++j) {
        const int kt = c * TT_SUB_PER_CHUNK + j;
        const int cur = j & 1;  // kt & 1
        mma_sub(cur);
        if (j == TT_SUB_PER_CHUNK - 1) fold(c == 0);
        const int slot = (j + 1) % PF;  // sub-tile kt + 1 (4 c is a multiple of PF)
        store_sub(cur ^ 1, ra[slot], rb[slot]);
        __syncthreads();
        load_sub(min(kt + 1 + PF, nsub - 1), ra[slot], rb[slot]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // Lane holds rows 16*mb + 4*g + i, column 16*nb + r of the wave's block.
  if constexpr (SW) {
    const int64_t inter = N / 2;
#pragma unroll
    for (int nb = 0; nb < NB / 2; ++nb) {
      const int64_t col = blockIdx.x * (TN / 2) + wn * (NB / 2) * 16 + 16 * nb + r;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t row = m0 + MB * 16 * wm + 16 * mb + 4 * g + i;
          if (row >= M) continue;
          const float gv = round_bf16(tot[mb][nb][i]);
          const float uv = round_bf16(tot[mb][nb + NB / 2][i]);
          static_cast<bf16_t*>(y)[row * inter + col] = f32_to_bf16(silu_mul1(gv, uv));
        }
      }
    }
  } else if constexpr (SP) {
    // Sampler epilogue, one row block at a time: each lane's statistics over its columns
    // (logits written as fp32 when y is given), merged over the 16 column lanes of a row,
    // then over the WN waves of a row band in wave order through LDS (the x tile buffer,
    // free once every wave is past its last MFMA); one record per (column tile, row).
    float* s_f = reinterpret_cast<float*>(&sa[0][0]);  // [5][WN][TM] floats, then [WN][TM] ints
    int* s_i = reinterpret_cast<int*>(s_f + 5 * WN * TM);
    static_assert(6 * WN * TM * 4 <= TM * TT_KS * 2, "sampler scratch exceeds the x tile");
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lr = MB * 16 * wm + 16 * mb + 4 * g + i;
        const int64_t row = m0 + lr;
        const int64_t rc = min<int64_t>(row, M - 1);
        const float t = sp.temps[rc];
        const uint32_t h = gumbel_row(sp.seeds[rc], sp.positions[rc]);
        SState a = sstate_empty();
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int64_t col = n0 + NB * 16 * wn + 16 * nb + r;
          if (col >= N || row >= M) continue;
          const float vr = round_bf16(tot[mb][nb][i]);
          if (y != nullptr) static_cast<float*>(y)[row * N + col] = vr;
          sstate_add(a, vr, static_cast<int>(col), t, h);
        }
        sstate_merge16(a, !(t > 0.0f));
        if (r == 0) {
          const int o = wn * TM + lr;
          s_f[o] = a.m;
          s_f[WN * TM + o] = a.s;
          s_f[2 * WN * TM + o] = a.v1;
          s_f[3 * WN * TM + o] = a.x1;
          s_f[4 * WN * TM + o] = a.v2;
          s_i[o] = a.i1;
        }
      }
    }
    __syncthreads();
    for (int lr = tid; lr < TM; lr += THREADS) {
      const int64_t row = m0 + lr;
      if (row >= M) continue;
      const bool greedy = !(sp.temps[row] > 0.0f);
      SState a = sstate_empty();
#pragma unroll
      for (int q = 0; q < WN; ++q) {
        const int o = q * TM + lr;
        const SState b{s_f[o], s_f[WN * TM + o], s_f[2 * WN * TM + o], s_f[3 * WN * TM + o],
                       s_f[4 * WN * TM + o], s_i[o]};
        if (q == 0) {
          a = b;
        } else {
          sstate_merge(a, b, greedy);
        }
      }
      sstate_store(sp.st, static_cast<int64_t>(blockIdx.x) * sp.cand_rows + row, a);
    }
  } else if constexpr (!AM) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int64_t col = n0 + NB * 16 * wn + 16 * nb + r;
      if (col >= N) continue;
      const float bv = bias != nullptr ? bf16_to_f32(bias[col]) : 0.0f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t row = m0 + MB * 16 * wm + 16 * mb + 4 * g + i;
          if (row >= M) continue;
          float v = tot[mb][nb][i];
          if (bias != nullptr) v += bv;
          if (out_fp32) {
            static_cast<float*>(y)[row * N + col] = round_bf16(v);
          } else {
            static_cast<bf16_t*>(y)[row * N + col] = f32_to_bf16(v);
          }
        }
      }
    }
  } else {
    // Greedy epilogue, one row block at a time (few live registers: the kernel keeps its
    // occupancy): each lane's best over its columns (logits written as fp32 when y is
    // given), then over the 16 column lanes of each row, then over the WN waves of a row
    // band through LDS (the x tile buffer, free once every wave is past its last MFMA).
    float* s_v = reinterpret_cast<float*>(&sa[0][0]);
    int* s_i = reinterpret_cast<int*>(s_v + WN * TM);
    static_assert(2 * WN * TM * 4 <= TM * TT_KS * 2, "argmax scratch exceeds the x tile");
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + MB * 16 * wm + 16 * mb + 4 * g + i;
        float v = -INFINITY;
        int ix = 0x7fffffff;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int64_t col = n0 + NB * 16 * wn + 16 * nb + r;
          if (col >= N || row >= M) continue;
          float t = tot[mb][nb][i];
          if (bias != nullptr) t += bf16_to_f32(bias[col]);
          const float vr = round_bf16(t);
          if (y != nullptr) static_cast<float*>(y)[row * N + col] = vr;
          if (argmax_better(vr, static_cast<int>(col), v, ix)) {
            v = vr;
            ix = static_cast<int>(col);
          }
        }
#pragma unroll
        for (int mask = 1; mask < 16; mask <<= 1) {
          const float ov = lane_xor(v, mask);
          const int oi = __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, ix);
          if (argmax_better(ov, oi, v, ix)) {
            v = ov;
            ix = oi;
          }
        }
        if (r == 0) {
          const int lr = MB * 16 * wm + 16 * mb + 4 * g + i;
          s_v[wn * TM + lr] = v;
          s_i[wn * TM + lr] = ix;
        }
      }
    }
    __syncthreads();
    for (int lr = tid; lr < TM; lr += THREADS) {
      float v = s_v[lr];
      int ix = s_i[lr];
#pragma unroll
      for (int q = 1; q < WN; ++q) {
        if (argmax_better(s_v[q * TM + lr], s_i[q * TM + lr], v, ix)) {
          v = s_v[q * TM + lr];
          ix = s_i[q * TM + lr];
        }
      }
      const int64_t row = m0 + lr;
      if (row < M) {
        best_val[static_cast<int64_t>(blockIdx.x) * M + row] = v;
        best_idx[static_cast<int64_t>(blockIdx.x) * M + row] = ix;
      }
    }
  }
}

template <int WM, int WN, int MB, int NB, int PF, bool AM = false, bool SW = false,
          bool SP = false>
void launch_tiled(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t m,
                  int64_t n, int64_t k, int out_fp32, hipStream_t s, float* best_val = nullptr,
                  int* best_idx = nullptr, SampleIn sp = SampleIn{}) {
  constexpr int TM = WM * MB * 16, TN = WN * NB * 16;
  const dim3 grid((unsigned)((n + TN - 1) / TN), (unsigned)((m + TM - 1) / TM));
  hipLaunchKernelGGL((linear_tiled_kernel<WM, WN, MB, NB, PF, AM, SW, SP>), grid,
                     dim3(WM * WN * 64), 0, s, (const bf16_t*)x, ldx, (const bf16_t*)w,
                     (const bf16_t*)bias, y, m, n, k, out_fp32, best_val, best_idx, sp);
}

// sid_linear takes the tiled kernel from this many rows up: 8 waves (4 x 2), each 32 x 64
// outputs (a 128 x 128 tile), or 32 x 32 (128 x 64) when 128 x 128 tiles would leave fewer
// than two workgroups per CU. (Measured on prefill shapes: 25-29% of the bf16 MFMA peak at
// M >= 2048 vs 8% for the 64-row-group kernel; 4 waves of 64 x 64 held both accumulator
// sets in AGPRs at one wave per SIMD and reached 13%. From 64 rows it also beats the 64-row-
// group kernel on the decode shapes, weights from HBM, consumer included: qkv at 128 rows
// 15.8 vs 22.1 us, o 19.3 vs 33.0, down 28.1 vs 47.3.)
constexpr int64_t kTiledMinM = 64;
constexpr int64_t kTiledWideMinTiles = 512;
// sid_linear_silu_mul takes the tiled form from this many rows up.
constexpr int64_t kLinearSiluTiledMinM = 96;

// K of the streaming kernel below, its chunk count and LDS row stride of staged x.
constexpr int WIDE_K = 1024;
constexpr int WIDE_NCH = WIDE_K / KC;
constexpr int WXS = WIDE_K + 8;

// Streaming wide-N GEMM for K = 1024, M <= 64 (lm_head at decode), optionally with the
// greedy argmax fused into its epilogue.
//
// A persistent grid of one 8-wave workgroup per CU stages the x row group in LDS once;
// every wave then owns every (number of waves)-th 16-column wave tile and streams its weights
// chunk by chunk (16 columns x 256 k = 8 KiB per chunk) through a ring of three register
// buffers, so two chunks are always in flight while the MFMAs of the third run. Each
// chunk's MFMA sequence and the left fold of the four chunks are those of linear_kernel,
// so the logits have the same bits. With ARGMAX, each lane keeps the best (value, column)
// of the rows it holds over its wave's columns (the values compared are the bf16-rounded
// logits the unfused path writes); the wave's best per row goes to a workspace
// [waves][M] that argmax_finalize_kernel reduces. The (value, index) order is total
// (torch's: larger value, then smaller index; NaN above everything, first NaN wins), so
// the result does not depend on how the columns are split.
constexpr int STREAM_WAVES = 8;

template <int MBS, bool ARGMAX, bool LEAN = false>
__global__ void __launch_bounds__(STREAM_WAVES * 64) linear_stream_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ bias, void* __restrict__ y, int M, int N, int out_fp32,
    float* __restrict__ best_val, int* __restrict__ best_idx, int cand_rows, int row0) {
  extern __shared__ __align__(16) bf16_t lx[];  // [MBS*16][WXS]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int gw = blockIdx.x * STREAM_WAVES + wave;
  const int num_waves = gridDim.x * STREAM_WAVES;
  const int tiles = N / 16;
  // Wave gw owns tiles gw, gw + num_waves, ...: at any moment the chip's waves read
  // neighbouring tiles (measured against contiguous runs per wave: M = 1 67.8 -> 65.4 us,
  // M = 64 82.2 -> 81.0). The argmax order is total, so the assignment does not matter.
  const int t_begin = gw, t_step = num_waves;
  const int units = (gw < tiles ? (tiles - gw + num_waves - 1) / num_waves : 0) * WIDE_NCH;

  // Unit u = (tile t_begin + (u/4) * t_step, chunk u%4); loads past the end are clamped to
  // the last unit (redundant, never consumed) so every issue point is unconditional.
  auto unit_ptr = [&](int u) {
    u = min(u, max(units - 1, 0));
    const int64_t col = static_cast<int64_t>(t_begin + (u >> 2) * t_step) * 16 + r;
    return w + col * WIDE_K + (u & 3) * KC + 8 * g;
  };
  bf16x8_v b0[NSTEP], b1[NSTEP], b2[NSTEP];
  if (units > 0) {
    load_w(b0, unit_ptr(0), 0);
    load_w(b1, unit_ptr(1), 0);
  }

  // Stage x (rows >= M clamped to row M-1; their outputs are discarded).
  constexpr int ROWS = MBS * 16;
  constexpr int VPR = WIDE_K / 8;  // 16-byte vectors per row
  constexpr int VPT = ROWS * VPR / (STREAM_WAVES * 64);
  {
    bf16x8_v xv[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = threadIdx.x + i * STREAM_WAVES * 64;
      const int row = v / VPR;
      xv[i] = ld_frag(x + static_cast<int64_t>(min(row, M - 1)) * ldx + (v % VPR) * 8);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = threadIdx.x + i * STREAM_WAVES * 64;
      *reinterpret_cast<bf16x8_v*>(&lx[(v / VPR) * WXS + (v % VPR) * 8]) = xv[i];
    }
  }
  __syncthreads();
  // A wave without columns (N/16 < waves) still writes its (-inf, none) candidates.
  if (!ARGMAX && units == 0) return;

  f32x4_v total[MBS];
  float bv[MBS][4];
  int bi[MBS][4];
  if constexpr (ARGMAX) {
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bv[mb][i] = -INFINITY;
        bi[mb][i] = 0x7fffffff;
      }
    }
  }

  auto consume = [&](const bf16x8_v (&wf)[NSTEP], int u) {
    const int c = u & 3;
    f32x4_v acc[MBS];
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) {
        const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(
            &lx[(16 * mb + r) * WXS + c * KC + KSTEP * s + 8 * g]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc[mb], 0, 0, 0);
      }
    }
    if (c == 0) {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) total[mb] = acc[mb];
    } else {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) total[mb][i] += acc[mb][i];
      }
    }
    if (c != 3) return;
    const int col = (t_begin + (u >> 2) * t_step) * 16 + r;
    // LEAN: no bias and no logits written (the greedy-only call), so the epilogue holds no
    // load and no store that the weight stream's waits would have to account for.
    const bool has_bias = !LEAN && bias != nullptr;
    const bool has_y = !LEAN && y != nullptr;
    const float bias_v = has_bias ? bf16_to_f32(bias[col]) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * g + i;
        float v = total[mb][i];
        if (has_bias) v += bias_v;
        const float vr = round_bf16(v);
        if (has_y && row < M) {
          const int64_t off = static_cast<int64_t>(row) * N + col;
          if (out_fp32) {
            static_cast<float*>(y)[off] = vr;
          } else {
            static_cast<bf16_t*>(y)[off] = f32_to_bf16(v);
          }
        }
        if constexpr (ARGMAX) {
          if (argmax_better(vr, col, bv[mb][i], bi[mb][i])) {
            bv[mb][i] = vr;
            bi[mb][i] = col;
          }
        }
      }
    }
  };

  for (int u = 0; u < units; u += 3) {
    load_w(b2, unit_ptr(u + 2), 0);
    consume(b0, u);
    load_w(b0, unit_ptr(u + 3), 0);
    if (u + 1 < units) consume(b1, u + 1);
    load_w(b1, unit_ptr(u + 4), 0);
    if (u + 2 < units) consume(b2, u + 2);
  }

  if constexpr (ARGMAX) {
    // Best over the 16 column lanes of each row (lanes r = 0..15 of a row group g).
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = bv[mb][i];
        int ix = bi[mb][i];
#pragma unroll
        for (int mask = 1; mask < 16; mask <<= 1) {
          const float ov = lane_xor(v, mask);
          const int oi = __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, ix);
          if (argmax_better(ov, oi, v, ix)) {
            v = ov;
            ix = oi;
          }
        }
        const int row = 16 * mb + 4 * g + i;
        if (r == 0 && row < M) {
          best_val[static_cast<int64_t>(gw) * cand_rows + row0 + row] = v;
          best_idx[static_cast<int64_t>(gw) * cand_rows + row0 + row] = ix;
        }
      }
    }
  }
}

// Per row: the best of the per-wave candidates (any order gives the same answer).
__global__ void __launch_bounds__(256) argmax_finalize_kernel(const float* __restrict__ best_val,
                                                              const int* __restrict__ best_idx,
                                                              int num_waves, int M,
                                                              int64_t* __restrict__ out) {
  const int row = blockIdx.x;
  float v = -INFINITY;
  int ix = 0x7fffffff;
  // Eight candidates per thread loaded at once (one round trip for the 2048 waves of the
  // persistent grid instead of eight); the order is total, so the visiting order is free.
  constexpr int U = 8;
  for (int base = threadIdx.x; base < num_waves; base += 256 * U) {
    float cv[U];
    int ci[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int wv = base + 256 * u;
      const bool in = wv < num_waves;
      const int64_t off = static_cast<int64_t>(in ? wv : 0) * M + row;
      cv[u] = in ? best_val[off] : -INFINITY;
      ci[u] = in ? best_idx[off] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (argmax_better(cv[u], ci[u], v, ix)) {
        v = cv[u];
        ix = ci[u];
      }
    }
  }
  for (int mask = 1; mask < 64; mask <<= 1) {
    const float ov = lane_xor(v, mask);
    const int oi = __builtin_amdgcn_ds_bpermute((__lane_id() ^ mask) << 2, ix);
    if (argmax_better(ov, oi, v, ix)) {
      v = ov;
      ix = oi;
    }
  }
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = v;
    s_i[threadIdx.x >> 6] = ix;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k) {
      if (argmax_better(s_v[k], s_i[k], v, ix)) {
        v = s_v[k];
        ix = s_i[k];
      }
    }
    out[row] = ix == 0x7fffffff ? 0 : ix;
  }
}

// ---- lm_head with the stochastic sampler fused into its epilogue ---------------------------
//
// The draw of sid/engine/sampler.py:32-69 without truncation (top_k <= 0, top_p >= 1):
// token = argmax_c log(p_c + eps) + g_c with p = softmax(l / T) and g the seeded Gumbel
// noise; greedy rows (T <= 0) take the argmax of the logits. Nothing of the logits is
// written. linear_sample_kernel is linear_stream_kernel (same grid, same per-column MFMA
// sequence and chunk fold, so the same logit bits l_c) with this epilogue: for every row it
// holds, each lane keeps over its wave's columns
//   mx, sm   online softmax state of x = l / T (sm = sum of exp(x - mx), rescaled when mx
//            grows),
//   a1       the column with the largest x + g (value a1v, its x a1x, index a1i; ties to the
//            lower index), a2v the second largest x + g;
// the 16 lanes of a row are merged in a fixed butterfly and written per (wave, row).
// sample_finalize_kernel takes one row: M = max mx, S = sum of sm exp(mx - M) in wave order,
// then the exact score log(exp(x - M) / S + eps) + g of every wave's a1 (the formula of the
// unfused sampler). Any other column c of a wave scores
//   log(exp(x_c + g_c - M) / S + eps exp(g_c)) <= log(exp(a2v - M) / S + eps exp(G)),
// increasing in x_c + g_c and in g_c (G: the largest value the noise takes, at u = 1 - 2^-24),
// so a wave whose bound stays below the best candidate
// (by a margin far above float rounding) cannot hold the winner. A wave that fails the test
// (a near-tie, or non-finite statistics: then every wave) has its logits recomputed for the
// row with the same MFMA sequence (identical bits) and every column scored exactly.
template <int MBS>
__global__ void __launch_bounds__(STREAM_WAVES * 64) linear_sample_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w, int M, int N,
    const float* __restrict__ temps, const int64_t* __restrict__ seeds,
    const int64_t* __restrict__ positions, SampleStats st, int cand_rows, int row0) {
  extern __shared__ __align__(16) bf16_t lx[];  // [MBS*16][WXS]
  __shared__ float s_t[64];
  __shared__ uint32_t s_h[64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int gw = blockIdx.x * STREAM_WAVES + wave;
  const int num_waves = gridDim.x * STREAM_WAVES;
  const int tiles = N / 16;
  const int t_begin = static_cast<int>(static_cast<int64_t>(gw) * tiles / num_waves);
  const int t_end = static_cast<int>(static_cast<int64_t>(gw + 1) * tiles / num_waves);
  const int units = (t_end - t_begin) * WIDE_NCH;

  auto unit_ptr = [&](int u) {
    u = min(u, max(units - 1, 0));
    const int64_t col = static_cast<int64_t>(t_begin + (u >> 2)) * 16 + r;
    return w + col * WIDE_K + (u & 3) * KC + 8 * g;
  };
  bf16x8_v b0[NSTEP], b1[NSTEP], b2[NSTEP];
  if (units > 0) {
    load_w(b0, unit_ptr(0), 0);
    load_w(b1, unit_ptr(1), 0);
  }
  constexpr int ROWS = MBS * 16;
  constexpr int VPR = WIDE_K / 8;
  constexpr int VPT = ROWS * VPR / (STREAM_WAVES * 64);
  {
    bf16x8_v xv[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = threadIdx.x + i * STREAM_WAVES * 64;
      const int row = v / VPR;
      xv[i] = ld_frag(x + static_cast<int64_t>(min(row, M - 1)) * ldx + (v % VPR) * 8);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = threadIdx.x + i * STREAM_WAVES * 64;
      *reinterpret_cast<bf16x8_v*>(&lx[(v / VPR) * WXS + (v % VPR) * 8]) = xv[i];
    }
  }
  if (threadIdx.x < 64) {
    const int row = min(static_cast<int>(threadIdx.x), M - 1) + row0;
    s_t[threadIdx.x] = temps[row];
    s_h[threadIdx.x] = gumbel_row(seeds[row], positions[row]);
  }
  __syncthreads();

  f32x4_v total[MBS];
  float mx[MBS][4], sm[MBS][4], a1v[MBS][4], a1x[MBS][4], a2v[MBS][4];
  int a1i[MBS][4];
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mx[mb][i] = -INFINITY;
      sm[mb][i] = 0.0f;
      a1v[mb][i] = -INFINITY;
      a1x[mb][i] = -INFINITY;
      a2v[mb][i] = -INFINITY;
      a1i[mb][i] = 0x7fffffff;
    }
  }

  auto consume = [&](const bf16x8_v (&wf)[NSTEP], int u) {
    const int c = u & 3;
    f32x4_v acc[MBS];
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) acc[mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) {
        const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(
            &lx[(16 * mb + r) * WXS + c * KC + KSTEP * s + 8 * g]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc[mb], 0, 0, 0);
      }
    }
    if (c == 0) {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) total[mb] = acc[mb];
    } else {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) total[mb][i] += acc[mb][i];
      }
    }
    if (c != 3) return;
    const int col = (t_begin + (u >> 2)) * 16 + r;
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * g + i;
        const float vr = round_bf16(total[mb][i]);
        const float t = s_t[row];
        if (!(t > 0.0f)) {  // greedy row: the logit itself
          if (argmax_better(vr, col, a1v[mb][i], a1i[mb][i])) {
            a1v[mb][i] = vr;
            a1i[mb][i] = col;
          }
          continue;
        }
        const float xv = vr / t;
        if (xv > mx[mb][i]) {
          sm[mb][i] = sm[mb][i] * expf(mx[mb][i] - xv) + 1.0f;
          mx[mb][i] = xv;
        } else {
          sm[mb][i] += expf(xv - mx[mb][i]);
        }
        const float gn = seeded_gumbel(s_h[row], col);
        const float xg = xv + gn;
        if (xg > a1v[mb][i] || (xg == a1v[mb][i] && col < a1i[mb][i])) {
          a2v[mb][i] = a1v[mb][i];
          a1v[mb][i] = xg;
          a1x[mb][i] = xv;
          a1i[mb][i] = col;
        } else {
          a2v[mb][i] = fmaxf(a2v[mb][i], xg);
        }
      }
    }
  };

  for (int u = 0; u < units; u += 3) {
    load_w(b2, unit_ptr(u + 2), 0);
    consume(b0, u);
    load_w(b0, unit_ptr(u + 3), 0);
    if (u + 1 < units) consume(b1, u + 1);
    load_w(b1, unit_ptr(u + 4), 0);
    if (u + 2 < units) consume(b2, u + 2);
  }

  // Merge the 16 column lanes of each row (fixed butterfly), lane r = 0 writes.
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * mb + 4 * g + i;
      const bool greedy = !(s_t[row] > 0.0f);
      float m = mx[mb][i], sv = sm[mb][i], v1 = a1v[mb][i], x1 = a1x[mb][i], v2 = a2v[mb][i];
      int i1 = a1i[mb][i];
#pragma unroll
      for (int mask = 1; mask < 16; mask <<= 1) {
        const int src = (lane ^ mask) << 2;
        const float om = lane_xor(m, mask);
        const float os = lane_xor(sv, mask);
        const float ov1 = lane_xor(v1, mask);
        const float ox1 = lane_xor(x1, mask);
        const float ov2 = lane_xor(v2, mask);
        const int oi1 = __builtin_amdgcn_ds_bpermute(src, i1);
        if (greedy) {
          if (argmax_better(ov1, oi1, v1, i1)) {
            v1 = ov1;
            i1 = oi1;
          }
          continue;
        }
        softmax_merge(m, sv, om, os);
        if (ov1 > v1 || (ov1 == v1 && oi1 < i1)) {
          v2 = fmaxf(v1, ov2);
          v1 = ov1;
          x1 = ox1;
          i1 = oi1;
        } else {
          v2 = fmaxf(v2, fmaxf(ov1, ov2));
        }
      }
      if (r == 0 && row < M) {
        const int64_t o = static_cast<int64_t>(gw) * cand_rows + row0 + row;
        st.mx[o] = m;
        st.sm[o] = sv;
        st.a1v[o] = v1;
        st.a1x[o] = x1;
        st.a2v[o] = v2;
        st.a1i[o] = i1;
      }
    }
  }
}

__device__ __forceinline__ bool score_better(float v, int i, float bv, int bi) {
  return argmax_better(v, i, bv, bi);
}

// Best (value, index) over the block under argmax_better; every thread gets the result.
__device__ __forceinline__ void block_best_i32(float& bv, int& bi, float* s_v, int* s_i) {
  for (int mask = 1; mask < 64; mask <<= 1) {
    const float ov = lane_xor(bv, mask);
    const int oi = __builtin_amdgcn_ds_bpermute((__lane_id() ^ mask) << 2, bi);
    if (argmax_better(ov, oi, bv, bi)) {
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
  for (int k = 1; k < static_cast<int>(blockDim.x >> 6); ++k) {
    if (argmax_better(s_v[k], s_i[k], bv, bi)) {
      bv = s_v[k];
      bi = s_i[k];
    }
  }
  __syncthreads();
}

constexpr int kFinThreads = 256;
constexpr float kCertMargin = 1e-3f;  // the certificate's slack over float rounding

__global__ void __launch_bounds__(kFinThreads) sample_finalize_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w, int N,
    SampleStats st, int num_waves, int M, const float* __restrict__ temps,
    const int64_t* __restrict__ seeds, const int64_t* __restrict__ positions,
    int* __restrict__ redo, int64_t* __restrict__ out, int recompute_all, int group_tiles) {
  __shared__ float s_v[kFinThreads / 64];
  __shared__ int s_i[kFinThreads / 64];
  __shared__ float s_red[kFinThreads / 64];
  __shared__ int s_nredo;
  __shared__ __align__(16) bf16_t s_x[WIDE_K];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float t = temps[row];
  auto at = [&](int wv) { return static_cast<int64_t>(wv) * M + row; };

  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (!(t > 0.0f)) {  // greedy row
    for (int wv = tid; wv < num_waves; wv += kFinThreads) {
      if (argmax_better(st.a1v[at(wv)], st.a1i[at(wv)], bv, bi)) {
        bv = st.a1v[at(wv)];
        bi = st.a1i[at(wv)];
      }
    }
    block_best_i32(bv, bi, s_v, s_i);
    if (tid == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
    return;
  }
  // M and S (fixed order: each thread's waves in order, then the butterfly, then waves)
  float m = -INFINITY;
  for (int wv = tid; wv < num_waves; wv += kFinThreads) m = fmaxf(m, st.mx[at(wv)]);
  for (int mask = 1; mask < 64; mask <<= 1) m = fmaxf(m, lane_xor(m, mask));
  if ((tid & 63) == 0) s_red[tid >> 6] = m;
  __syncthreads();
  m = s_red[0];
  for (int k = 1; k < kFinThreads / 64; ++k) m = fmaxf(m, s_red[k]);
  __syncthreads();
  float part = 0.0f;
  for (int wv = tid; wv < num_waves; wv += kFinThreads) {
    const float mw = st.mx[at(wv)];
    if (mw != -INFINITY) part += st.sm[at(wv)] * expf(mw - m);
  }
  for (int mask = 1; mask < 64; mask <<= 1) part += lane_xor(part, mask);
  if ((tid & 63) == 0) s_red[tid >> 6] = part;
  __syncthreads();
  float sum = s_red[0];
  for (int k = 1; k < kFinThreads / 64; ++k) sum += s_red[k];
  const bool full = recompute_all || !isfinite(m) || !isfinite(sum) || !(sum > 0.0f);
  // eps * exp(G), G = the largest noise value (u = 1 - 2^-24), rounded up a little
  const float g_max = -logf(-logf(16777215.0f / 16777216.0f + kSampleEps) + kSampleEps);
  const float eps_g = kSampleEps * expf(g_max) * 1.0001f;
  const uint32_t h = gumbel_row(seeds[row], positions[row]);
  auto score = [&](float xv, int col) {
    return logf(expf(xv - m) / sum + kSampleEps) + seeded_gumbel(h, col);
  };
  // Every wave's candidate, scored exactly.
  if (!full) {
    for (int wv = tid; wv < num_waves; wv += kFinThreads) {
      const int c = st.a1i[at(wv)];
      if (c == 0x7fffffff) continue;
      const float sc = score(st.a1x[at(wv)], c);
      if (argmax_better(sc, c, bv, bi)) {
        bv = sc;
        bi = c;
      }
    }
  }
  block_best_i32(bv, bi, s_v, s_i);
  // Waves whose other columns might beat the best candidate.
  if (tid == 0) s_nredo = 0;
  __syncthreads();
  int* list = redo + static_cast<int64_t>(row) * num_waves;
  for (int wv = tid; wv < num_waves; wv += kFinThreads) {
    bool need = full;
    if (!need && st.a1i[at(wv)] != 0x7fffffff) {
      const float bound = logf(expf(st.a2v[at(wv)] - m) / sum + eps_g);
      need = !(bound + kCertMargin < bv);
    }
    if (need) list[atomicAdd(&s_nredo, 1)] = wv;
  }
  __syncthreads();
  const int nredo = s_nredo;
  if (nredo > 0) {
    for (int i = tid; i < WIDE_K / 8; i += kFinThreads)
      *reinterpret_cast<bf16x8_v*>(&s_x[8 * i]) =
          *reinterpret_cast<const bf16x8_v*>(x + static_cast<int64_t>(row) * ldx + 8 * i);
    __syncthreads();
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int tiles = N / 16;
    // Recompute the listed waves' logits (the streaming kernel's MFMA sequence and chunk fold
    // with this row in all 16 A rows, so every lane's result is the row's logit of its
    // column) and score every column.
    for (int k = wave; k < nredo; k += kFinThreads / 64) {
      const int wv = list[k];
      // The group's 16-column tiles: a streaming wave's run, or a fixed-width column tile.
      const int tb = group_tiles > 0 ? wv * group_tiles
                                     : static_cast<int>(static_cast<int64_t>(wv) * tiles / num_waves);
      const int te = group_tiles > 0 ? min(tiles, (wv + 1) * group_tiles)
                                     : static_cast<int>(static_cast<int64_t>(wv + 1) * tiles / num_waves);
      for (int tile = tb; tile < te; ++tile) {
        const int col = tile * 16 + r;
        const bf16_t* wrow = w + static_cast<int64_t>(col) * WIDE_K + 8 * g;
        f32x4_v tot = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < WIDE_NCH; ++c) {
          bf16x8_v wf[NSTEP];
          load_w(wf, wrow, c * KC);
          f32x4_v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int s = 0; s < NSTEP; ++s) {
            const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(&s_x[c * KC + KSTEP * s + 8 * g]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[s], acc, 0, 0, 0);
          }
          if (c == 0) {
            tot = acc;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) tot[i] += acc[i];
          }
        }
        if (g == 0) {
          const float vr = round_bf16(tot[0]);
          const float sc = score(vr / t, col);
          if (argmax_better(sc, col, bv, bi)) {
            bv = sc;
            bi = col;
          }
        }
      }
    }
    block_best_i32(bv, bi, s_v, s_i);
  }
  if (tid == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
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

template <int NW>
void launch_linear(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t m,
                   int64_t n, int64_t k, int out_fp32, hipStream_t stream) {
  const dim3 grid((unsigned)(n / (16 * NW)), 1u, (unsigned)((m + MROWS - 1) / MROWS));
  hipLaunchKernelGGL((linear_kernel<NW>), grid, dim3(NW * 64), 0, stream, (const bf16_t*)x, ldx,
                     (const bf16_t*)w, (const bf16_t*)bias, y, m, n, k, out_fp32);
}

// Waves per workgroup: more waves share one staged x chunk (less L2->LDS traffic per
// weight byte) but leave fewer workgroups; wide direct GEMMs (lm_head, prefill) use 8.
// (16 waves would cap the kernel at 128 VGPRs and spill.)
int pick_waves(int64_t n, int64_t m) {
  const int64_t groups = (m + MROWS - 1) / MROWS;
  if (n % 128 == 0 && (n / 128) * groups >= 512) return 8;
  return 4;
}

void launch_any(int nw, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                int64_t m, int64_t n, int64_t k, int out_fp32, hipStream_t s) {
  switch (nw) {
    case 8: return launch_linear<8>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
    default: return launch_linear<4>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
  }
}

// The streaming kernel serves sid_linear from this many columns up (lm_head-sized N).
constexpr int64_t kStreamMinN = 32768;

// Persistent-grid size of the streaming kernel: one workgroup per CU of the current device.
int stream_grid() {
  static int count[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    count[dev] = n;
  }
  return count[dev];
}

// Row groups of up to 64 rows are streamed one after the other (the weights are re-read
// per group); up to this many rows that still beats the tiled kernel on lm_head shapes.
constexpr int64_t kStreamMaxM = 256;

bool stream_shape_ok(int64_t m, int64_t n, int64_t k) {
  return m >= 1 && m <= kStreamMaxM && k == WIDE_K && n % 16 == 0 && n < (1ll << 31);
}

template <int MBS, bool AM, bool LEAN>
void launch_stream_form(const bf16_t* x, int64_t ldx, const void* w, const void* bias, void* y,
                        int m, int n, int out_fp32, float* bv, int* bi, int cand_rows, int row0,
                        hipStream_t s) {
  const size_t lds = static_cast<size_t>(MBS * 16) * WXS * sizeof(bf16_t);
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_stream_kernel<MBS, AM, LEAN>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    attr_set = true;
  }
  hipLaunchKernelGGL((linear_stream_kernel<MBS, AM, LEAN>), dim3(stream_grid()),
                     dim3(STREAM_WAVES * 64), lds, s, x, ldx, (const bf16_t*)w,
                     (const bf16_t*)bias, y, m, n, out_fp32, bv, bi, cand_rows, row0);
}

template <int MBS, bool AM>
void launch_stream_mbs(const bf16_t* x, int64_t ldx, const void* w, const void* bias, void* y,
                       int m, int n, int out_fp32, float* bv, int* bi, int cand_rows, int row0,
                       hipStream_t s) {
  if constexpr (AM) {
    if (bias == nullptr && y == nullptr) {
      launch_stream_form<MBS, AM, true>(x, ldx, w, bias, y, m, n, out_fp32, bv, bi, cand_rows,
                                        row0, s);
      return;
    }
  }
  launch_stream_form<MBS, AM, false>(x, ldx, w, bias, y, m, n, out_fp32, bv, bi, cand_rows, row0,
                                     s);
}

// One launch per 64-row group; group g reads x rows 64g.., writes y rows 64g.. and the
// candidate rows 64g.. of the [waves][m] workspace.
template <bool AM>
void launch_stream(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int m,
                   int n, int out_fp32, float* bv, int* bi, hipStream_t s) {
  for (int r0 = 0; r0 < m; r0 += MROWS) {
    const int mg = min(MROWS, m - r0);
    const bf16_t* xg = static_cast<const bf16_t*>(x) + static_cast<int64_t>(r0) * ldx;
    void* yg = nullptr;
    if (y != nullptr) {
      const int64_t off = static_cast<int64_t>(r0) * n;
      yg = out_fp32 ? static_cast<void*>(static_cast<float*>(y) + off)
                    : static_cast<void*>(static_cast<bf16_t*>(y) + off);
    }
    switch ((mg + 15) / 16) {
      case 1: launch_stream_mbs<1, AM>(xg, ldx, w, bias, yg, mg, n, out_fp32, bv, bi, m, r0, s); break;
      case 2: launch_stream_mbs<2, AM>(xg, ldx, w, bias, yg, mg, n, out_fp32, bv, bi, m, r0, s); break;
      case 3: launch_stream_mbs<3, AM>(xg, ldx, w, bias, yg, mg, n, out_fp32, bv, bi, m, r0, s); break;
      default: launch_stream_mbs<4, AM>(xg, ldx, w, bias, yg, mg, n, out_fp32, bv, bi, m, r0, s); break;
    }
  }
}

// ---- gate_up projection with the SwiGLU epilogue (decode-sized M) -----------------------
//
// out[m, j] = bf16(bf16(silu(g)) * u), g = bf16(x w[j]^T), u = bf16(x w[I + j]^T), each a
// canonical chunk fold: the same bits as sid_linear_partials + sid_silu_mul_partials, with
// neither the fp32 partials' round trip through memory nor the second launch. A workgroup
// has one wave per 256-wide chunk (NCH waves, K = 256 NCH) and owns 8 NB output columns of
// a 64-row group; in MFMA column block nb, lanes 0-7 are gate rows j0+8nb.. and lanes 8-15
// the matching up rows I+j0+8nb.. of w. Wave c accumulates chunk c from zero with x and w
// fragments loaded straight from global memory (each wave reads a different chunk, so
// nothing is shared through LDS; the NB column blocks share the wave's x fragments); the
// chunk sums meet in LDS and are folded c0 + c1 + ... in order.
template <int NCH, int MBS, int NB>
__global__ void __launch_bounds__(NCH * 64) linear_silu_kernel(const bf16_t* __restrict__ x,
                                                               const bf16_t* __restrict__ w,
                                                               int64_t M, int64_t inter,
                                                               bf16_t* __restrict__ out) {
  constexpr int64_t K = static_cast<int64_t>(NCH) * KC;
  constexpr int SS = 16 * NB + 1;  // LDS row stride of a chunk sum tile (floats)
  __shared__ float sacc[NCH][MROWS * SS];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t j0 = static_cast<int64_t>(blockIdx.x) * (8 * NB);
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MROWS;
  const int mrows = static_cast<int>(min<int64_t>(MROWS, M - m0));
  const int64_t k0 = static_cast<int64_t>(wave) * KC;

  bf16x8_v wf[NB][NSTEP];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t wr = r < 8 ? j0 + 8 * nb + r : inter + j0 + 8 * nb + (r - 8);
    load_w(wf[nb], w + wr * K + 8 * g, k0);
  }
  bf16x8_v xf[MBS][NSTEP];
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
    const int64_t row = min<int64_t>(m0 + 16 * mb + r, M - 1);  // clamped rows are dropped
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) xf[mb][s] = ld_frag(x + row * K + k0 + KSTEP * s + 8 * g);
  }
  // Every load is issued before the first MFMA (one memory latency per workgroup; left to
  // itself the compiler interleaves loads and MFMAs and waits on each group).
  __builtin_amdgcn_sched_barrier(0);
  f32x4_v acc[NB][MBS];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) acc[nb][mb] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int mb = 0; mb < MBS; ++mb)
        acc[nb][mb] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[mb][s], wf[nb][s], acc[nb][mb], 0, 0, 0);
    }
  }
  // Lane holds rows 16 mb + 4 g + i of column block nb, column r.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sacc[wave][(16 * mb + 4 * g + i) * SS + 16 * nb + r] = acc[nb][mb][i];
    }
  }
  __syncthreads();
  // 64 rows x 8 NB outputs, two adjacent outputs per thread per pass.
  for (int o = threadIdx.x; o < MBS * 16 * 4 * NB; o += NCH * 64) {
    const int row = o / (4 * NB);
    const int q = o % (4 * NB);
    const int nb = q >> 2;
    const int col = 2 * (q & 3);  // within the block's 8 gate columns
    if (row >= mrows) continue;
    const int base = row * SS + 16 * nb + col;
    float y[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float gs = sacc[0][base + e];
      float us = sacc[0][base + 8 + e];
#pragma unroll
      for (int c = 1; c < NCH; ++c) {
        gs += sacc[c][base + e];
        us += sacc[c][base + 8 + e];
      }
      y[e] = silu_mul1(round_bf16(gs), round_bf16(us));
    }
    *reinterpret_cast<uint32_t*>(out + (m0 + row) * inter + j0 + 8 * nb + col) =
        pack_bf16x2(y[0], y[1]);
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
  // The streaming kernel reads the weights once per 64-row group; past one group the tiled
  // kernel (each weight row reused by 128 rows) is faster: M = 128 151936 x 1024 fp32
  // logits 165 -> 101 us, M = 256 327 -> 179 us (identical bits).
  if (m <= MROWS && stream_shape_ok(m, n, k) && n >= kStreamMinN) {
    launch_stream<false>(x, ldx, w, bias, y, static_cast<int>(m), static_cast<int>(n), out_fp32,
                         nullptr, nullptr, s);
    return check_launch("linear");
  }
  if (m >= kTiledMinM || (m > MROWS && n >= kStreamMinN)) {
    SID_REQUIRE((m + 63) / 64 <= 65535, "linear: too many rows");
    const int64_t wide_tiles = ((m + 127) / 128) * ((n + 127) / 128);
    if (wide_tiles >= kTiledWideMinTiles) {
      launch_tiled<4, 2, 2, 4, 1>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
    } else if (((m + 127) / 128) * ((n + 63) / 64) <= stream_grid()) {
      // At most one workgroup per CU: two sub-tiles in flight (measured, same bits: qkv
      // M = 256 13.2 -> 11.2 us, o M = 2048 23.8 -> 18.6 us, down M = 2048 33.2 -> 24.9 us)
      launch_tiled<4, 2, 2, 2, 2>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
    } else {
      launch_tiled<4, 2, 2, 2, 1>(x, ldx, w, bias, y, m, n, k, out_fp32, s);
    }
    return check_launch("linear");
  }
  launch_any(pick_waves(n, m), x, ldx, w, bias, y, m, n, k, out_fp32, s);
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
  // Row groups of 64; a single group smaller than 64 rows gets the matching MBS.
  const int mbs = m >= MROWS ? 4 : static_cast<int>((m + 15) / 16);
  const dim3 grid((unsigned)(n / 64), (unsigned)(k / KC), (unsigned)((m + MROWS - 1) / MROWS));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, (const bf16_t*)x, ldx, (const bf16_t*)w, m, n, k,
                       partials);
  };
  switch (mbs) {
    case 1: go(linear_chunk_kernel<4, 1>); break;
    case 2: go(linear_chunk_kernel<4, 2>); break;
    case 3: go(linear_chunk_kernel<4, 3>); break;
    default: go(linear_chunk_kernel<4, 4>); break;
  }
  return check_launch("linear_partials");
}

// sid_linear_argmax: up to one 64-row group streams the weights once (linear_stream_kernel,
// one candidate per wave); more rows take the tiled GEMM with the argmax epilogue (one
// candidate per 128-column tile, no logits needed: verify pass, 128 rows x 151936,
// 101 us GEMM + 32 us argmax_rows before). Both reduce with argmax_finalize_kernel. The
// workspace holds stream_grid() * STREAM_WAVES candidates per row, which bounds the tiled
// path's column tiles.
static bool argmax_streams(int64_t m, int64_t n, int64_t k) {
  return m <= MROWS && stream_shape_ok(m, n, k);
}

static int64_t argmax_candidates() { return static_cast<int64_t>(stream_grid()) * STREAM_WAVES; }

extern "C" int64_t sid_linear_argmax_workspace_bytes(int64_t m) {
  if (m < 1 || (m + MROWS - 1) / MROWS > 65535) return 0;
  return argmax_candidates() * m * static_cast<int64_t>(sizeof(float) + sizeof(int));
}

extern "C" int sid_linear_argmax(const void* x, int64_t ldx, const void* w, const void* bias,
                                 float* logits, int64_t m, int64_t n, int64_t k, void* workspace,
                                 int64_t workspace_bytes, int64_t* out_idx, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear_argmax: negative size");
  if (m == 0) return SID_OK;
  SID_REQUIRE(n > 0, "linear_argmax: no columns");
  SID_REQUIRE(out_idx != nullptr && workspace != nullptr, "linear_argmax: null pointer");
  int rc = check_shapes(x, ldx, w, m, n, k, "linear_argmax");
  if (rc != SID_OK) return rc;
  const int64_t need = sid_linear_argmax_workspace_bytes(m);
  SID_REQUIRE(need > 0 && workspace_bytes >= need, "linear_argmax: workspace %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)need);
  SID_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
              "linear_argmax: workspace must be 16-byte aligned");
  const int64_t cands = argmax_candidates();
  float* bv = static_cast<float*>(workspace);
  int* bi = reinterpret_cast<int*>(bv + cands * m);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int used;
  if (argmax_streams(m, n, k)) {
    launch_stream<true>(x, ldx, w, bias, logits, static_cast<int>(m), static_cast<int>(n), 1, bv,
                        bi, s);
    used = static_cast<int>(cands);
  } else {
    const int64_t tiles = (n + 127) / 128;
    SID_REQUIRE(tiles <= cands, "linear_argmax: N=%lld has more than %lld column tiles",
                (long long)n, (long long)cands);
    SID_REQUIRE((m + 127) / 128 <= 65535, "linear_argmax: too many rows");
    launch_tiled<4, 2, 2, 4, 1, true>(x, ldx, w, bias, logits, m, n, k, 1, s, bv, bi);
    used = static_cast<int>(tiles);
  }
  rc = check_launch("linear_argmax");
  if (rc != SID_OK) return rc;
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)m), dim3(256), 0, s, bv, bi, used,
                     static_cast<int>(m), out_idx);
  return check_launch("linear_argmax finalize");
}

// Workspace of sid_linear_sample: 6 per-(wave, row) statistics + the finalize's lists.
static int64_t sample_ws_bytes(int64_t m) {
  const int64_t waves = static_cast<int64_t>(stream_grid()) * STREAM_WAVES;
  return waves * m * 4 * 7;
}

// Rows one sid_linear_sample call takes: the streaming grouping up to kStreamMaxM, the
// 128-column tiles up to this many (prefill / verify passes of large batches).
constexpr int64_t kTiledSampleMaxM = 4096;

extern "C" int64_t sid_linear_sample_workspace_bytes(int64_t m) {
  if (m < 1 || m > kTiledSampleMaxM) return 0;
  return sample_ws_bytes(m);
}

template <int MBS>
static void launch_sample_mbs(const bf16_t* x, int64_t ldx, const void* w, int m, int n,
                              const float* temps, const int64_t* seeds, const int64_t* pos,
                              SampleStats st, int cand_rows, int row0, hipStream_t s) {
  const size_t lds = static_cast<size_t>(MBS * 16) * WXS * sizeof(bf16_t);
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_sample_kernel<MBS>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    attr_set = true;
  }
  hipLaunchKernelGGL((linear_sample_kernel<MBS>), dim3(stream_grid()), dim3(STREAM_WAVES * 64),
                     lds, s, x, ldx, (const bf16_t*)w, m, n, temps, seeds, pos, st, cand_rows,
                     row0);
}

// The streaming sampler reads the weights once per 64-row group; above this many rows (or
// when asked) the tiled GEMM with the sampler epilogue reads them once per 128-row tile
// (candidate groups: 128-column tiles instead of streaming waves). Measured at T = 0.7,
// 151936 x 1024, graph-timed (streaming vs tiled, us): 1 row 80 vs 108, 64 rows 120 vs
// 142, 128 rows 214 vs 158, 192 rows 265 vs 266, 256 rows 285 vs 284.
constexpr int64_t kStreamSampleMaxM = 64;

extern "C" int sid_linear_sample(const void* x, int64_t ldx, const void* w, int64_t m, int64_t n,
                                 int64_t k, const float* temperatures, const int64_t* seeds,
                                 const int64_t* positions, void* workspace,
                                 int64_t workspace_bytes, int64_t* out_idx, float* logits,
                                 int flags, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear_sample: negative size");
  SID_REQUIRE((flags & ~7) == 0 && (flags & 6) != 6, "linear_sample: bad flags %d", flags);
  if (m == 0) return SID_OK;
  SID_REQUIRE(n > 0, "linear_sample: no columns");
  SID_REQUIRE(out_idx && workspace && temperatures && seeds && positions,
              "linear_sample: null pointer");
  int rc = check_shapes(x, ldx, w, m, n, k, "linear_sample");
  if (rc != SID_OK) return rc;
  const bool tiled =
      (flags & 2) != 0 || ((flags & 4) == 0 && (m > kStreamSampleMaxM || logits != nullptr));
  SID_REQUIRE(stream_shape_ok(tiled ? 1 : m, n, k) && m <= kTiledSampleMaxM,
              "linear_sample: needs K == %d and 1 <= M <= %d (%d with the 128-column tiles); "
              "got M=%lld, K=%lld",
              WIDE_K, (int)kStreamMaxM, (int)kTiledSampleMaxM, (long long)m, (long long)k);
  const int64_t need = sample_ws_bytes(m);
  SID_REQUIRE(workspace_bytes >= need, "linear_sample: workspace %lld bytes, need %lld",
              (long long)workspace_bytes, (long long)need);
  SID_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
              "linear_sample: workspace must be 16-byte aligned");
  SID_REQUIRE(!(flags & 4) || logits == nullptr,
              "linear_sample: the streaming grouping writes no logits");
  const int stream_groups = stream_grid() * STREAM_WAVES;
  const int groups = tiled ? static_cast<int>((n + 127) / 128) : stream_groups;
  SID_REQUIRE(groups <= stream_groups, "linear_sample: N=%lld has more than %d column tiles",
              (long long)n, stream_groups);
  const int64_t plane = static_cast<int64_t>(stream_groups) * m;
  float* base = static_cast<float*>(workspace);
  SampleStats st{base, base + plane, base + 2 * plane, base + 3 * plane, base + 4 * plane,
                 reinterpret_cast<int*>(base + 5 * plane)};
  int* redo = reinterpret_cast<int*>(base + 6 * plane);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int mi = static_cast<int>(m);
  if (tiled) {
    SID_REQUIRE((m + 127) / 128 <= 65535, "linear_sample: too many rows");
    launch_tiled<4, 2, 2, 4, 1, false, false, true>(
        x, ldx, w, nullptr, logits, m, n, k, 1, s, nullptr, nullptr,
        SampleIn{temperatures, seeds, positions, st, m});
    rc = check_launch("linear_sample");
    if (rc != SID_OK) return rc;
  } else {
    for (int r0 = 0; r0 < mi; r0 += MROWS) {
      const int mg = min(MROWS, mi - r0);
      const bf16_t* xg = static_cast<const bf16_t*>(x) + static_cast<int64_t>(r0) * ldx;
      switch ((mg + 15) / 16) {
        case 1: launch_sample_mbs<1>(xg, ldx, w, mg, (int)n, temperatures, seeds, positions, st, mi, r0, s); break;
        case 2: launch_sample_mbs<2>(xg, ldx, w, mg, (int)n, temperatures, seeds, positions, st, mi, r0, s); break;
        case 3: launch_sample_mbs<3>(xg, ldx, w, mg, (int)n, temperatures, seeds, positions, st, mi, r0, s); break;
        default: launch_sample_mbs<4>(xg, ldx, w, mg, (int)n, temperatures, seeds, positions, st, mi, r0, s); break;
      }
      rc = check_launch("linear_sample");
      if (rc != SID_OK) return rc;
    }
  }
  hipLaunchKernelGGL(sample_finalize_kernel, dim3((unsigned)m), dim3(kFinThreads), 0, s,
                     (const bf16_t*)x, ldx, (const bf16_t*)w, (int)n, st, groups, mi,
                     temperatures, seeds, positions, redo, out_idx, flags & 1,
                     tiled ? 8 : 0);
  return check_launch("linear_sample finalize");
}

extern "C" int sid_linear_silu_mul(const void* x, const void* w, void* out, int64_t m, int64_t k,
                                   int64_t inter, void* stream) {
  SID_REQUIRE(m >= 0 && k >= 0 && inter >= 0, "linear_silu_mul: negative size");
  if (m == 0 || inter == 0) return SID_OK;
  SID_REQUIRE(x && w && out, "linear_silu_mul: null pointer");
  SID_REQUIRE(k == 4 * KC, "linear_silu_mul: K must be %d, got %lld", 4 * KC, (long long)k);
  SID_REQUIRE(inter % 8 == 0, "linear_silu_mul: intermediate size %lld not a multiple of 8",
              (long long)inter);
  SID_REQUIRE(inter / 8 <= 0x7fffffff && (m + MROWS - 1) / MROWS <= 65535,
              "linear_silu_mul: too large");
  SID_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 4 == 0,
              "linear_silu_mul: misaligned operand");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (m >= kLinearSiluTiledMinM && inter % 64 == 0) {
    // From 96 rows: the tiled GEMM with the SwiGLU epilogue, in sid_linear's tile shapes
    // (grid over the 2 * inter projection columns; the [M, 2 * inter] projection is never
    // written). Same bits as the kernel below and as sid_linear + sid_silu_mul. Measured
    // (I = 3072, weights from HBM, graph-timed): M = 64 11.9 us vs 9.8 for the kernel below,
    // M = 96 12.4 vs 13.6, M = 128 12.8 vs 15.6, M = 192 12.5 vs 20.7; against sid_linear +
    // sid_silu_mul M = 256 11.0 vs 15.1 us, M = 2048 38.4 vs 48.2, M = 8192 143 vs 171.
    SID_REQUIRE((m + 127) / 128 <= 65535, "linear_silu_mul: too many rows");
    const int64_t n = 2 * inter;
    if (((m + 127) / 128) * ((n + 127) / 128) >= kTiledWideMinTiles) {
      launch_tiled<4, 2, 2, 4, 1, false, true>(x, k, w, nullptr, out, m, n, k, 0, s);
    } else if (((m + 127) / 128) * ((n + 63) / 64) <= stream_grid()) {
      launch_tiled<4, 2, 2, 2, 2, false, true>(x, k, w, nullptr, out, m, n, k, 0, s);
    } else {
      launch_tiled<4, 2, 2, 2, 1, false, true>(x, k, w, nullptr, out, m, n, k, 0, s);
    }
    return check_launch("linear_silu_mul");
  }
  const int mbs = m >= MROWS ? 4 : static_cast<int>((m + 15) / 16);
  // Two column blocks per wave halve the x read per output (M = 64, I = 3072, weights from
  // HBM: 12.3 -> 9.3 us); an I that is not a multiple of 16 takes one block per wave.
  const int nb = inter % 16 == 0 ? 2 : 1;
  const dim3 grid((unsigned)(inter / (8 * nb)), (unsigned)((m + MROWS - 1) / MROWS));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(4 * 64), 0, s, (const bf16_t*)x, (const bf16_t*)w, m,
                       inter, (bf16_t*)out);
  };
  if (nb == 2) {
    switch (mbs) {
      case 1: go(linear_silu_kernel<4, 1, 2>); break;
      case 2: go(linear_silu_kernel<4, 2, 2>); break;
      case 3: go(linear_silu_kernel<4, 3, 2>); break;
      default: go(linear_silu_kernel<4, 4, 2>); break;
    }
  } else {
    switch (mbs) {
      case 1: go(linear_silu_kernel<4, 1, 1>); break;
      case 2: go(linear_silu_kernel<4, 2, 1>); break;
      case 3: go(linear_silu_kernel<4, 3, 1>); break;
      default: go(linear_silu_kernel<4, 4, 1>); break;
    }
  }
  return check_launch("linear_silu_mul");
}
