// The decode step's projections with their neighbours fused in (decode-sized M: a batch of
// single-token rows). Per layer the chain is
//
//   q, K/V cache  <- sid_rmsnorm_qkv_post(r)          input RMSNorm + qkv projection +
//                                                      q/k-norm + RoPE + cache write
//   o             <- decode attention(q)
//   residual, r   <- sid_linear_residual(o, W_o)       o projection + residual add
//   act           <- sid_rmsnorm_linear_silu_mul(r)    post RMSNorm + gate_up + SwiGLU
//   residual, r   <- sid_linear_residual(act, W_down)  down projection + residual add
//
// where r is the fp32 sum residual + projection (the value sid/kernels/rmsnorm.py:27-42
// normalises; the bf16 residual is its rounding). Five launches per layer instead of eight,
// and no fp32 split-K partials in memory.
//
// Bits: every projection keeps sid_linear's reduction order (256-wide chunks, each
// accumulated from zero by 8 v_mfma_f32_16x16x32_bf16 k-steps in increasing k with the same
// operand layout, chunks left-folded in increasing order, one rounding to bf16), every
// RMSNorm rmsnorm_kernel's order for a 64-lane row (lane j owns the 8-element vectors
// j + 64 i, sequential fmaf, xor butterfly), and the q/k-norm + RoPE and the SwiGLU go
// through the same helpers as qkv_post_kernel and silu_mul_kernel. So the chain's outputs
// are bit-identical to the unfused sequence sid_linear -> sid_fused_add_rmsnorm ->
// sid_linear_silu_mul -> ... (checked by the GPU tests), and M-invariant like it.
//
// Shape of the work (MI355X: every one of these kernels moves 4-13 MB, i.e. a few us at
// HBM rate, so what counts is one memory round trip per workgroup): each workgroup issues
// all of its global loads (weights straight into MFMA B fragments, activations) before its
// first MFMA, and owns a whole column tile over the whole K, so nothing but the outputs is
// written. Workgroups that share a weight tile (the row groups of one column tile) are
// numbered so they land on the same XCD (workgroups are dealt round-robin over the 8 XCDs
// in id order) and share its L2.
#include "common.h"
#include "rowmath.h"

namespace sid {
namespace {

constexpr int KC = 256;     // chunk width of the canonical reduction order
constexpr int KSTEP = 32;   // MFMA 16x16x32 k-step
constexpr int NSTEP = KC / KSTEP;

__device__ __forceinline__ bf16x8_v ld_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_v*>(p);
}

// Packed weight fragments with the non-temporal hint: each is read by the row groups of one
// column tile at about the same time and then not again in the step (chain 26.3 -> 25.3 us
// per layer at M = 64, weights from HBM; the same hint on the lm_head stream made it slower,
// 74 -> 85 us).
__device__ __forceinline__ bf16x8_v ld_frag_w(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_v,
                            __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p)));
}

// Workgroup id -> (column tile, row group) with the R row groups of a tile on one XCD
// (ids congruent mod 8) when the tile count is a multiple of 8.
__device__ __forceinline__ void xcd_tile(int id, int ntiles, int R, int& tile, int& rg) {
  if ((ntiles & 7) == 0) {
    tile = (id & 7) + 8 * ((id >> 3) / R);
    rg = (id >> 3) % R;
  } else {
    tile = id / R;
    rg = id % R;
  }
}

// ---- MFMA operands ------------------------------------------------------------------------
//
// The canonical operand layout puts row r, elements 32 s + 8 g .. +7 of a 256-wide chunk in
// lane r + 16 g of k-step register s. Read straight from a row-major matrix that is 16 rows
// x 64 bytes per instruction with neighbouring lanes in different rows, which the memory
// pipeline serves at about half the rate of whole-line reads (measured on MI355X). So:
//
// * Weights are used in a fragment-packed copy (made once at load time, see
//   sid_pack_decode_weights): for 16-row block b and chunk c, the 8 KB of its fragments are
//   stored in register order, [b][c][s][lane][8], and a wave loads its operand with eight
//   contiguous 1 KB reads straight into registers.
// * Activation tiles (16 rows x one chunk, 8 KB) are staged by each wave in a private LDS
//   region with global_load_lds (1 KB per instruction, the 16-byte pieces XOR-swizzled:
//   piece c of row r at slot c ^ (r & 15)) and read back as fragments without bank
//   conflicts.
// Same values in the same registers as the direct loads, so the same bits.
__device__ __forceinline__ void packed_load(bf16x8_v (&f)[NSTEP], const bf16_t* __restrict__ wp,
                                            int64_t block, int c, int nch, int lane) {
  const bf16_t* p = wp + ((block * nch + c) * NSTEP) * 512 + 8 * lane;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) f[s] = ld_frag_w(p + 512 * s);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Stage rows row0 .. row0 + 15 (rows past `last` clamped to it; the caller drops their
// results), elements k0 .. k0 + 255, of a row-major bf16 matrix into the wave's 8 KB region.
__device__ __forceinline__ void stage_tile(char* region, const bf16_t* __restrict__ p, int64_t ld,
                                           int row0, int last, int64_t k0, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int piece = 64 * i + lane;
    const int row = piece >> 5;
    const int c = (piece & 31) ^ (row & 15);
    const bf16_t* g = p + static_cast<int64_t>(min(row0 + row, last)) * ld + k0 + 8 * c;
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)(region + 1024 * i), 16, 0, 0);
  }
}

__device__ __forceinline__ void staged_frags(bf16x8_v (&f)[NSTEP], const char* region, int lane) {
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s)
    f[s] = *reinterpret_cast<const bf16x8_v*>(region + r * 512 + 16 * ((4 * s + g) ^ r));
}

// Waits until this wave's outstanding global loads (global_load_lds included) are done.
__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- the fp32 residual sum r32 -------------------------------------------------------------
//
// r32 rows are stored in the RMSNorm lane order so a 64-lane norm reads them with whole-line
// loads: element 8 v + e of a row (v = j + 64 i: lane j's i-th 8-element vector; e < 8) sits
// at i * 512 + (e >> 2) * 256 + 4 j + (e & 3).
__device__ __forceinline__ int r32_pos(int col) {
  const int v = col >> 3, e = col & 7;
  return (v >> 6) * 512 + (e >> 2) * 256 + 4 * (v & 63) + (e & 3);
}

// ---- RMSNorm of a row into the MFMA A tile --------------------------------------------------
//
// One wave per row, hidden = 512 PL: lane j holds the 8-element vectors j + 64 i (i < PL)
// (rmsnorm_kernel's layout for 64 lanes per row). F32: the row is an r32 row; otherwise
// bf16 in column order. Loads and arithmetic are split so a kernel can issue the loads with
// its weight loads.
template <int PL, bool F32>
__device__ __forceinline__ void norm_row_load(const void* __restrict__ src, int64_t row, int j,
                                              float (&v)[PL][8]) {
  constexpr int H = 512 * PL;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    if constexpr (F32) {
      const float* p = static_cast<const float*>(src) + row * H + 512 * i + 4 * j;
      const float4 a = *reinterpret_cast<const float4*>(p);
      const float4 b = *reinterpret_cast<const float4*>(p + 256);
      v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
      v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
    } else {
      load8(*reinterpret_cast<const uint4*>(static_cast<const bf16_t*>(src) + row * H +
                                            8 * (j + 64 * i)),
            v[i]);
    }
  }
}

// rmsnorm(v) * w rounded to bf16 (rmsnorm_kernel's bits): y[i] = lane j's 8-element vector
// j + 64 i of the output row, packed.
template <int PL>
__device__ __forceinline__ void norm_w_load(const uint4* __restrict__ w, int j, uint4 (&wv)[PL]) {
#pragma unroll
  for (int i = 0; i < PL; ++i) wv[i] = w[j + 64 * i];
}

template <int PL>
__device__ __forceinline__ void norm_row_apply(const float (&v)[PL][8], int j,
                                               const uint4 (&wv)[PL], float eps,
                                               uint4 (&y)[PL]) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PL; ++i) ss = sumsq8(v[i], ss);
  ss = group_sum64(ss);
  const float rstd = rms_rstd(ss, 512 * PL, eps);
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    float wf[8], o[8];
    load8(wv[i], wf);
    rms_apply8(v[i], rstd, wf, o);
    y[i] = store8(o);
  }
}

// The same, written to row `row` of an A tile in LDS: 16-byte piece p of the row at
// tile + row * 2 H bytes + 16 (p ^ (row & 15)), the layout a_frag reads (no padding, no bank
// conflicts).
template <int PL>
__device__ __forceinline__ void norm_row_store(const float (&v)[PL][8], int j,
                                               const uint4 (&wv)[PL], float eps,
                                               char* tile, int row) {
  uint4 y[PL];
  norm_row_apply<PL>(v, j, wv, eps, y);
#pragma unroll
  for (int i = 0; i < PL; ++i)
    *reinterpret_cast<uint4*>(tile + row * (1024 * PL) + 16 * ((j + 64 * i) ^ (row & 15))) = y[i];
}

// A fragment of k-step s of chunk c from such a tile (row r of row block mb, part g).
template <int PL>
__device__ __forceinline__ bf16x8_v a_frag(const char* tile, int row, int c, int s, int g) {
  const int p = 32 * c + 4 * s + g;
  return *reinterpret_cast<const bf16x8_v*>(tile + row * (1024 * PL) + 16 * (p ^ (row & 15)));
}

// ---- projection + residual add ------------------------------------------------------------
//
// y = x w^T for a 16-row x 16 NBW-column tile over K = 256 NCH: wave c stages chunk c of the
// x rows and loads chunk c of the NBW packed w blocks, then accumulates each block from zero;
// the chunk sums meet in LDS and are folded c0 + c1 + ... in order; then
// r = residual + bf16(y) (fp32), residual = bf16(r), r32 = r (in r32 order).
// These kernels are bound by the bytes each workgroup pulls through its CU's L2 port (time
// ~ 3 us + per-CU bytes / ~55 GB/s, measured), so from 96 rows a workgroup takes 32 columns
// (NBW = 2) and above 128 rows 64 (NBW = 4): the staged rows then serve more weight bytes,
// and the CUs pull 25% fewer bytes than with two 16-column workgroups each.
template <int NCH, int NBW>
__global__ void __launch_bounds__(NCH * 64) linear_residual_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ wpk,
    bf16_t* __restrict__ residual, float* __restrict__ r32, int M, int N, int R) {
  constexpr int COLS = 16 * NBW;
  constexpr int SS = COLS + 1;  // LDS row stride of a chunk tile (floats)
  static_assert(16 * SS * 4 <= 8192, "a chunk-sum tile must fit its wave's staging region");
  // Wave c's chunk sums overwrite its own staged rows once they are in registers.
  __shared__ __align__(16) char stage[NCH][8192];
  auto sacc = [&](int c) { return reinterpret_cast<float*>(stage[c]); };
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int tile, rg;
  xcd_tile(blockIdx.x, N / COLS, R, tile, rg);
  const int n0 = tile * COLS;
  const int m0 = rg * 16;
  // The epilogue's residual values first (thread t: outputs t, t + 64 NCH, ...), so the
  // epilogue waits for no further round trip.
  constexpr int OUTS = 16 * COLS;
  constexpr int PER = (OUTS + NCH * 64 - 1) / (NCH * 64);
  // Unconditional loads from clamped (in-bounds) positions: a guarded load would become a
  // branch that waits for it on the spot.
  bf16_t resv[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int o = min(static_cast<int>(threadIdx.x) + q * NCH * 64, OUTS - 1);
    const int erow = min(m0 + o / COLS, M - 1);
    resv[q] = residual[static_cast<int64_t>(erow) * N + n0 + o % COLS];
  }
  stage_tile(stage[wave], x, ldx, m0, M - 1, static_cast<int64_t>(wave) * KC, lane);
  bf16x8_v xf[NSTEP], wf[NBW][NSTEP];
#pragma unroll
  for (int j = 0; j < NBW; ++j) packed_load(wf[j], wpk, tile * NBW + j, wave, NCH, lane);
  wait_loads();
  staged_frags(xf, stage[wave], lane);
  const int r = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    f32x4_v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[s], wf[j][s], acc, 0, 0, 0);
    // Lane holds rows 4 g + i of column 16 j + r.
#pragma unroll
    for (int i = 0; i < 4; ++i) sacc(wave)[(4 * g + i) * SS + 16 * j + r] = acc[i];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int o = threadIdx.x + q * NCH * 64;
    const int erow = o / COLS;
    const int ecol = o % COLS;
    if (o >= OUTS || m0 + erow >= M) break;  // rows ascend with o
    const int64_t off = static_cast<int64_t>(m0 + erow) * N + n0 + ecol;
    const bf16_t res = resv[q];
    float tot = sacc(0)[erow * SS + ecol];
#pragma unroll
    for (int c = 1; c < NCH; ++c) tot += sacc(c)[erow * SS + ecol];
    const float rr = bf16_to_f32(res) + round_bf16(tot);
    residual[off] = f32_to_bf16(rr);
    r32[static_cast<int64_t>(m0 + erow) * N + r32_pos(n0 + ecol)] = rr;
  }
}

// ---- RMSNorm + gate_up projection + SwiGLU ------------------------------------------------
//
// act[m, j] = bf16(bf16(silu(g)) * u), g / u the gate / up projections of
// x = bf16(rmsnorm(src) * norm_w). A workgroup owns 16 MBS rows and 8 NB gate columns (with
// their up columns); in MFMA column block nb, rows 0-7 are gate rows j0 + 8 nb.. of w and
// rows 8-15 the matching up rows inter + j0 + 8 nb.. (linear_silu_kernel's layout). Its
// NCH x NB waves are (chunk, column block) pairs. Every wave issues its weight tile's loads
// and its rows' loads, normalises its rows into the shared A tile, transposes its weight
// tile; then every wave runs its chunk's MFMAs for all row blocks, and the chunk sums are
// folded in order in LDS (aliasing the transposition scratch, dead by then).
//
// NBW > 1: each wave owns NBW column blocks of its chunk (NB / NBW waves per chunk), so a
// workgroup covers NBW times the columns with the same wave count and each normalised row is
// shared by more weight bytes: at 128 rows (32-row workgroups, 48 gate columns each) the
// workgroups pull 30% fewer bytes through their CUs' L2 ports than with 24 columns.
template <int PL, bool F32, int MBS, int NB, int NBW = 1>
__global__ void __launch_bounds__(2 * PL * (NB / NBW) * 64) norm_silu_kernel(
    const void* __restrict__ src, const uint4* __restrict__ norm_w, float eps,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ out, int M, int inter, int R) {
  static_assert(NB % NBW == 0, "column blocks per wave must divide the workgroup's");
  constexpr int NCH = 2 * PL;
  constexpr int H = 512 * PL;
  constexpr int NW = NCH * (NB / NBW);
  constexpr int ROWS = 16 * MBS;
  constexpr int SS = 16 * NB + 1;    // LDS row stride of a chunk-sum tile (floats)
  constexpr int RPW = (ROWS + NW - 1) / NW;
  // The chunk sums reuse the A tile's LDS once every wave's MFMAs are done with it.
  constexpr int kSx = ROWS * 2 * H;
  constexpr int kSacc = NCH * ROWS * SS * 4;
  __shared__ __align__(16) char smem[kSx > kSacc ? kSx : kSacc];
  char* sx = smem;
  auto sacc = [&](int k) { return reinterpret_cast<float*>(smem) + k * ROWS * SS; };
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int c = wave % NCH;
  const int nb0 = (wave / NCH) * NBW;  // first column block of this wave
  int tile, rg;
  xcd_tile(blockIdx.x, inter / (8 * NB), R, tile, rg);
  const int j0 = tile * 8 * NB;
  const int m0 = rg * ROWS;

  // Norm weights and activation rows first: the norm waits only for them. A wave's rows are
  // held RB at a time (all of them up to 3 per wave; 64-row workgroups normalise 6 per wave
  // in two batches, the second loaded once the first is in LDS).
  constexpr int RB = RPW < 3 ? RPW : 3;
  uint4 nw[PL];
  norm_w_load<PL>(norm_w, lane, nw);
  float v[RB][PL][8];
#pragma unroll
  for (int q = 0; q < RB; ++q) {
    const int row = wave + NW * q;
    if (row < ROWS) norm_row_load<PL, F32>(src, min(m0 + row, M - 1), lane, v[q]);
  }
  bf16x8_v wf[NBW][NSTEP];
#pragma unroll
  for (int j = 0; j < NBW; ++j)
    packed_load(wf[j], w, static_cast<int64_t>(tile) * NB + nb0 + j, c, NCH, lane);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b0 = 0; b0 < RPW; b0 += RB) {
    if (b0 > 0) {
#pragma unroll
      for (int q = 0; q < RB; ++q) {
        const int row = wave + NW * (b0 + q);
        if (b0 + q < RPW && row < ROWS)
          norm_row_load<PL, F32>(src, min(m0 + row, M - 1), lane, v[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int row = wave + NW * (b0 + q);
      if (b0 + q < RPW && row < ROWS) norm_row_store<PL>(v[q], lane, nw, eps, sx, row);
    }
  }
  __syncthreads();
  f32x4_v acc[MBS][NBW];
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[mb][j] = f32x4_v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
    for (int mb = 0; mb < MBS; ++mb) {
      const bf16x8_v af = a_frag<PL>(sx, 16 * mb + r, c, s, g);
#pragma unroll
      for (int j = 0; j < NBW; ++j)
        acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[j][s], acc[mb][j], 0, 0, 0);
    }
  }
  __syncthreads();  // the A tile is dead from here on
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sacc(c)[(16 * mb + 4 * g + i) * SS + 16 * (nb0 + j) + r] = acc[mb][j][i];
    }
  }
  __syncthreads();
  // ROWS x 8 NB outputs, two adjacent gate columns per thread.
  for (int o = threadIdx.x; o < ROWS * 4 * NB; o += NW * 64) {
    const int row = o / (4 * NB);
    const int q = o % (4 * NB);
    const int b = q >> 2;
    const int col = 2 * (q & 3);
    if (m0 + row >= M) continue;
    const int base = row * SS + 16 * b + col;
    float y[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float gs = sacc(0)[base + e];
      float us = sacc(0)[base + 8 + e];
#pragma unroll
      for (int k = 1; k < NCH; ++k) {
        gs += sacc(k)[base + e];
        us += sacc(k)[base + 8 + e];
      }
      y[e] = silu_mul1(round_bf16(gs), round_bf16(us));
    }
    *reinterpret_cast<uint32_t*>(out + static_cast<int64_t>(m0 + row) * inter + j0 + 8 * b + col) =
        pack_bf16x2(y[0], y[1]);
  }
}

// ---- RMSNorm + qkv projection + q/k-norm + RoPE + KV-cache write -----------------------
//
// A workgroup owns one head (128 projection columns: a q, k or v head) of 16 rows. Its 8
// waves are the head's 16-column blocks; wave b holds its block's weights for every chunk
// (all loads issued first, with the rows the workgroup normalises into LDS), accumulates
// chunk by chunk and folds in registers. The bf16-rounded head then goes through
// qkv_post_kernel's epilogue: q / k heads per-head RMSNorm + RoPE (16 lanes per row), q to
// q_out, k and v to the pools at slots[row] (negative or out-of-range slots skipped).
constexpr int QD = 128;

// MBS = 2: 32-row workgroups (each weight fragment used for two row blocks), for batches
// whose 16-row grid would not fit the CUs in one round.
template <int PL, bool F32, int MBS>
__global__ void __launch_bounds__(512) norm_qkv_kernel(
    const void* __restrict__ src, const uint4* __restrict__ norm_w, float eps,
    const bf16_t* __restrict__ w, int M, int num_q_heads, int num_kv_heads, int R,
    const uint4* __restrict__ q_norm, const uint4* __restrict__ k_norm,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_sin,
    int64_t max_positions, const int64_t* __restrict__ slots, uint4* __restrict__ q_out,
    uint4* __restrict__ k_cache, uint4* __restrict__ v_cache, int64_t num_slots) {
  constexpr int NCH = 2 * PL;
  constexpr int H = 512 * PL;
  constexpr int YS = QD + 4;
  constexpr int ROWS = 16 * MBS;
  constexpr int RPW = ROWS / 8;  // rows each wave normalises
  __shared__ __align__(16) char sx[ROWS * 2 * H];
  __shared__ __align__(16) float sy[ROWS * YS];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int heads = num_q_heads + 2 * num_kv_heads;
  int head, rg;
  xcd_tile(blockIdx.x, heads, R, head, rg);
  const int m0 = rg * ROWS;

  // Epilogue operands first (thread t < 16 ROWS: row t / 16, head lanes t % 16), then the
  // norm weights and rows, then the weight tiles: each wait covers only what it needs.
  const int row = threadIdx.x >> 4;
  const int j = threadIdx.x & 15;
  const bool epi = threadIdx.x < 16 * ROWS;
  const int64_t t = min(m0 + row, M - 1);
  const bool valid = epi && m0 + row < M;
  const bool is_v = head >= num_q_heads + num_kv_heads;
  const bool is_q = head < num_q_heads;
  int64_t slot = -1, pos = -1;
  if (epi) {
    slot = slots[t];
    pos = positions[t];
  }
  uint4 nw[PL];
  norm_w_load<PL>(norm_w, lane, nw);
  float v[RPW][PL][8];
#pragma unroll
  for (int q = 0; q < RPW; ++q) norm_row_load<PL, F32>(src, min(m0 + wave + 8 * q, M - 1), lane, v[q]);
  bf16x8_v wf[NCH][NSTEP];
#pragma unroll
  for (int c = 0; c < NCH; ++c) packed_load(wf[c], w, static_cast<int64_t>(head) * 8 + wave, c, NCH, lane);
  __builtin_amdgcn_sched_barrier(0);
  // The rotary table row depends on the position: its loads go out once that one is back,
  // with everything issued after it still in flight.
  QkRopeIn in;
  if (epi && !is_v) qk_rope_load(in, j, is_q ? q_norm : k_norm, pos, cos_sin, max_positions);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < RPW; ++q) norm_row_store<PL>(v[q], lane, nw, eps, sx, wave + 8 * q);
  __syncthreads();
#pragma unroll
  for (int mb = 0; mb < MBS; ++mb) {
    f32x4_v tot;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      f32x4_v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < NSTEP; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_frag<PL>(sx, 16 * mb + r, c, s, g),
                                                      wf[c][s], acc, 0, 0, 0);
      if (c == 0) {
        tot = acc;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) tot[i] += acc[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sy[(16 * mb + 4 * g + i) * YS + 16 * wave + r] = round_bf16(tot[i]);
  }
  __syncthreads();
  if (!epi) return;
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = sy[row * YS + 8 * j + e];
  const bool slot_ok = valid && slot >= 0 && slot < num_slots;
  const int kv_row = 16 * num_kv_heads;  // uint4 per pool row
  if (is_v) {
    if (slot_ok) v_cache[slot * kv_row + (head - num_q_heads - num_kv_heads) * 16 + j] = store8(y);
    return;
  }
  float o[8];
  qk_head_norm_rope(y, j, in, eps, o);
  if (is_q) {
    if (valid) q_out[(t * num_q_heads + head) * 16 + j] = store8(o);
  } else if (slot_ok) {
    k_cache[slot * kv_row + (head - num_q_heads) * 16 + j] = store8(o);
  }
}

// ---- weight packing ------------------------------------------------------------------------
//
// packed[b][c][s][lane] (16 bytes each) = row(b, lane & 15), elements 256 c + 32 s + 8 (lane >> 4)
// .. +7 of w, where row(b, r) = 16 b + r, or for a gate_up weight [gate rows | up rows] of
// `inter` rows each: gate row 8 b + r for r < 8, up row inter + 8 b + r - 8 (one 16-byte piece
// per thread).
__global__ void __launch_bounds__(256) pack_weight_kernel(const uint4* __restrict__ w,
                                                          uint4* __restrict__ packed, int64_t n,
                                                          int64_t k, int64_t inter) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nch = k / KC;
  if (i >= n * k / 8) return;
  const int lane = static_cast<int>(i & 63);
  const int s = static_cast<int>((i >> 6) & 7);
  const int64_t bc = i >> 9;
  const int64_t c = bc % nch;
  const int64_t b = bc / nch;
  const int r = lane & 15;
  const int64_t row = inter > 0 ? (r < 8 ? 8 * b + r : inter + 8 * b + (r - 8)) : 16 * b + r;
  packed[i] = w[(row * k + c * KC + 32 * s + 8 * (lane >> 4)) / 8];
}

// ---- RMSNorm of fp32 rows (the final norm of the chain) ------------------------------------
template <int PL>
__global__ void __launch_bounds__(256) rmsnorm_f32_kernel(const float* __restrict__ x,
                                                          const uint4* __restrict__ w,
                                                          bf16_t* __restrict__ out, int M,
                                                          float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint4 nw[PL];
  norm_w_load<PL>(w, lane, nw);
  float v[PL][8];
  norm_row_load<PL, true>(x, min(row, M - 1), lane, v);
  if (row >= M) return;  // whole waves
  uint4 y[PL];
  norm_row_apply<PL>(v, lane, nw, eps, y);
  uint4* o = reinterpret_cast<uint4*>(out + static_cast<int64_t>(row) * 512 * PL);
#pragma unroll
  for (int i = 0; i < PL; ++i) o[lane + 64 * i] = y[i];
}

}  // namespace
}  // namespace sid

using namespace sid;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// From this many rows the o / down and gate_up workgroups take twice the columns (fewer bytes
// per CU through L2; measured per layer at 96 rows 36.8 -> 31.1 us, at 128 37.2 -> 31.0; at
// 64 rows the halved workgroup count loses, 26.7 -> 30.6).
constexpr int64_t kWideMinRows = 96;
// Above this many rows the gate_up workgroups take 64 rows (one round of workgroups where
// 32-row ones need two).
constexpr int64_t kDeepMinRows = 128;
// Above 128 rows the 16-row qkv workgroups (and the 32-column o / down ones) number more than
// the CUs hold at once, so the qkv workgroups take 32 rows and the o / down ones 64 columns:
// per layer at 192 rows qkv 14.7 -> 11.9 us, down 12.9 -> 9.8; at 256 the chain 52.9 ->
// 45.4 us.
constexpr int64_t kQkvWideAboveRows = 128;
constexpr int64_t kXWideAboveRows = 128;

extern "C" int sid_linear_residual(const void* x, int64_t ldx, const void* w, void* residual,
                                   float* r32, int64_t m, int64_t n, int64_t k, void* stream) {
  SID_REQUIRE(m >= 0 && n >= 0 && k >= 0, "linear_residual: negative size");
  if (m == 0 || n == 0) return SID_OK;
  SID_REQUIRE(x && w && residual && r32, "linear_residual: null pointer");
  SID_REQUIRE(n % 512 == 0, "linear_residual: N=%lld must be a multiple of 512", (long long)n);
  SID_REQUIRE(k == 1024 || k == 2048 || k == 3072 || k == 4096,
              "linear_residual: K=%lld must be 1024, 2048, 3072 or 4096", (long long)k);
  SID_REQUIRE(ldx >= k && ldx % 8 == 0, "linear_residual: row stride %lld must be >= K and a multiple of 8", (long long)ldx);
  SID_REQUIRE(aligned16(x) && aligned16(w), "linear_residual: operands must be 16-byte aligned");
  // 32-column workgroups from 96 rows, 64-column ones above kXWideAboveRows (K = 4096 keeps
  // 32: its 16-wave workgroups would spill with four column blocks).
  const int nbw = m > kXWideAboveRows && k <= 3072 ? 4 : m >= kWideMinRows ? 2 : 1;
  const int64_t R = (m + 15) / 16;
  SID_REQUIRE(R * (n / (16 * nbw)) < (1ll << 31), "linear_residual: too large");
  const dim3 grid((unsigned)(R * (n / (16 * nbw))));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kern, int nch) {
    hipLaunchKernelGGL(kern, grid, dim3(nch * 64), 0, s, (const bf16_t*)x, ldx, (const bf16_t*)w,
                       (bf16_t*)residual, r32, (int)m, (int)n, (int)R);
  };
#define SID_LR(NCH)                                                               \
  (nbw == 1 ? go(linear_residual_kernel<NCH, 1>, NCH)                               \
            : nbw == 2 ? go(linear_residual_kernel<NCH, 2>, NCH) : go(linear_residual_kernel<NCH, 4>, NCH))
  switch (k) {
    case 1024: SID_LR(4); break;
    case 2048: SID_LR(8); break;
    case 3072: SID_LR(12); break;
    default:
      if (nbw == 1) go(linear_residual_kernel<16, 1>, 16); else go(linear_residual_kernel<16, 2>, 16);
      break;
  }
#undef SID_LR
  return check_launch("linear_residual");
}

extern "C" int sid_rmsnorm_linear_silu_mul(const void* src, int src_fp32, const void* norm_w,
                                           float eps, const void* w, void* out, int64_t m,
                                           int64_t hidden, int64_t inter, void* stream) {
  SID_REQUIRE(m >= 0 && hidden >= 0 && inter >= 0, "rmsnorm_linear_silu_mul: negative size");
  if (m == 0 || inter == 0) return SID_OK;
  SID_REQUIRE(src && norm_w && w && out, "rmsnorm_linear_silu_mul: null pointer");
  SID_REQUIRE(hidden == 512 || hidden == 1024,
              "rmsnorm_linear_silu_mul: hidden %lld must be 512 or 1024", (long long)hidden);
  SID_REQUIRE(inter % 24 == 0, "rmsnorm_linear_silu_mul: intermediate %lld not a multiple of 24",
              (long long)inter);
  SID_REQUIRE(aligned16(src) && aligned16(norm_w) && aligned16(w) &&
                  (reinterpret_cast<uintptr_t>(out) & 3) == 0,
              "rmsnorm_linear_silu_mul: misaligned operand");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // 16-row workgroups for a handful of rows, 32 rows beyond, 64 above kDeepMinRows; from
  // kWideMinRows rows each wave takes two column blocks (48 gate columns per workgroup), when
  // they tile inter.
  const int mbs = m <= 16 ? 1 : (m > kDeepMinRows && inter % 48 == 0 ? 4 : 2);
  const bool wide = mbs >= 2 && m >= kWideMinRows && inter % 48 == 0;
  const int nb = wide ? 6 : 3;
  const int64_t R = (m + 16 * mbs - 1) / (16 * mbs);
  const int64_t tiles = inter / (8 * nb);
  SID_REQUIRE(R * tiles < (1ll << 31), "rmsnorm_linear_silu_mul: too large");
  const dim3 grid((unsigned)(R * tiles));
  auto go = [&](auto kern, int pl) {
    hipLaunchKernelGGL(kern, grid, dim3(2 * pl * 3 * 64), 0, s, src, (const uint4*)norm_w, eps,
                       (const bf16_t*)w, (bf16_t*)out, (int)m, (int)inter, (int)R);
  };
  const int pl = static_cast<int>(hidden / 512);
  const bool f = src_fp32 != 0;
#define SID_NS(PL, F)                                                            \
  (mbs == 1 ? go(norm_silu_kernel<PL, F, 1, 3>, PL)                             \
   : mbs == 4 ? go(norm_silu_kernel<PL, F, 4, 6, 2>, PL)                        \
            : (wide ? go(norm_silu_kernel<PL, F, 2, 6, 2>, PL) : go(norm_silu_kernel<PL, F, 2, 3>, PL)))
  if (pl == 1) {
    if (f) SID_NS(1, true); else SID_NS(1, false);
  } else {
    if (f) SID_NS(2, true); else SID_NS(2, false);
  }
#undef SID_NS
  return check_launch("rmsnorm_linear_silu_mul");
}

extern "C" int sid_rmsnorm_qkv_post(const void* src, int src_fp32, const void* norm_w, float eps,
                                    const void* w_qkv, int64_t m, int64_t hidden,
                                    int num_q_heads, int num_kv_heads, int head_dim,
                                    const void* q_norm, const void* k_norm,
                                    const int64_t* positions, const float* cos_sin,
                                    int64_t max_positions, const int64_t* slots, void* q_out,
                                    void* k_cache, void* v_cache, int64_t num_slots,
                                    void* stream) {
  SID_REQUIRE(m >= 0 && hidden >= 0, "rmsnorm_qkv_post: negative size");
  if (m == 0) return SID_OK;
  SID_REQUIRE(src && norm_w && w_qkv && q_norm && k_norm && positions && cos_sin && slots &&
                  q_out && k_cache && v_cache,
              "rmsnorm_qkv_post: null pointer");
  SID_REQUIRE(head_dim == QD, "rmsnorm_qkv_post: head_dim must be %d, got %d", QD, head_dim);
  SID_REQUIRE(num_q_heads > 0 && num_kv_heads > 0, "rmsnorm_qkv_post: bad head counts");
  SID_REQUIRE(hidden == 512 || hidden == 1024,
              "rmsnorm_qkv_post: hidden %lld must be 512 or 1024", (long long)hidden);
  SID_REQUIRE(num_slots > 0, "rmsnorm_qkv_post: empty KV pool");
  SID_REQUIRE(aligned16(src) && aligned16(norm_w) && aligned16(w_qkv) && aligned16(q_out) &&
                  aligned16(k_cache) && aligned16(v_cache),
              "rmsnorm_qkv_post: operands must be 16-byte aligned");
  // 32-row workgroups once 16-row ones would take more than one round of the CUs.
  const int mbs = m > kQkvWideAboveRows ? 2 : 1;
  const int64_t R = (m + 16 * mbs - 1) / (16 * mbs);
  const int heads = num_q_heads + 2 * num_kv_heads;
  SID_REQUIRE(R * heads < (1ll << 31), "rmsnorm_qkv_post: too large");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(R * heads));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(512), 0, s, src, (const uint4*)norm_w, eps,
                       (const bf16_t*)w_qkv, (int)m, num_q_heads, num_kv_heads, (int)R,
                       (const uint4*)q_norm, (const uint4*)k_norm, positions, cos_sin,
                       max_positions, slots, (uint4*)q_out, (uint4*)k_cache, (uint4*)v_cache,
                       num_slots);
  };
#define SID_NQ(PL, F) \
  (mbs == 1 ? go(norm_qkv_kernel<PL, F, 1>) : go(norm_qkv_kernel<PL, F, 2>))
  if (hidden == 512) {
    if (src_fp32) SID_NQ(1, true); else SID_NQ(1, false);
  } else {
    if (src_fp32) SID_NQ(2, true); else SID_NQ(2, false);
  }
#undef SID_NQ
  return check_launch("rmsnorm_qkv_post");
}

extern "C" int sid_pack_decode_weight(const void* w, void* packed, int64_t n, int64_t k,
                                      int gate_up, void* stream) {
  SID_REQUIRE(n >= 0 && k >= 0, "pack_decode_weight: negative size");
  if (n == 0 || k == 0) return SID_OK;
  SID_REQUIRE(w && packed && w != packed, "pack_decode_weight: null or aliased pointer");
  SID_REQUIRE(k % KC == 0, "pack_decode_weight: K=%lld must be a multiple of 256", (long long)k);
  SID_REQUIRE(n % 16 == 0, "pack_decode_weight: N=%lld must be a multiple of 16", (long long)n);
  SID_REQUIRE(aligned16(w) && aligned16(packed), "pack_decode_weight: misaligned operand");
  const int64_t pieces = n * k / 8;
  SID_REQUIRE((pieces + 255) / 256 < (1ll << 31), "pack_decode_weight: too large");
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (const uint4*)w, (uint4*)packed, n, k,
                     gate_up ? n / 2 : int64_t(0));
  return check_launch("pack_decode_weight");
}

extern "C" int sid_rmsnorm_f32(const float* x, const void* w, void* out, int64_t rows,
                               int hidden, float eps, void* stream) {
  SID_REQUIRE(rows >= 0, "rmsnorm_f32: negative rows");
  if (rows == 0) return SID_OK;
  SID_REQUIRE(x && w && out, "rmsnorm_f32: null pointer");
  SID_REQUIRE(hidden == 512 || hidden == 1024 || hidden == 2048,
              "rmsnorm_f32: hidden %d must be 512, 1024 or 2048", hidden);
  SID_REQUIRE(aligned16(x) && aligned16(w) && aligned16(out), "rmsnorm_f32: misaligned operand");
  SID_REQUIRE((rows + 3) / 4 < (1ll << 31), "rmsnorm_f32: too many rows");
  const dim3 grid((unsigned)((rows + 3) / 4));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (hidden) {
    case 512: hipLaunchKernelGGL(rmsnorm_f32_kernel<1>, grid, dim3(256), 0, s, x, (const uint4*)w, (bf16_t*)out, (int)rows, eps); break;
    case 1024: hipLaunchKernelGGL(rmsnorm_f32_kernel<2>, grid, dim3(256), 0, s, x, (const uint4*)w, (bf16_t*)out, (int)rows, eps); break;
    default: hipLaunchKernelGGL(rmsnorm_f32_kernel<4>, grid, dim3(256), 0, s, x, (const uint4*)w, (bf16_t*)out, (int)rows, eps); break;
  }
  return check_launch("rmsnorm_f32");
}
