// Shared helpers for the sid HIP kernels (gfx950 / CDNA4, wave64).
//
// Everything here is device-agnostic plumbing: bf16 <-> fp32 conversion with
// round-to-nearest-even (the rounding torch uses for bf16 tensors), wave64 DPP
// lane exchanges, the thread-local error string returned through the C-ABI,
// and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdarg>

#include "../../include/sid_hip.h"

namespace sid {

typedef uint16_t bf16_t;  // raw bf16 bits; the C-ABI passes bf16 tensors as void*

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_v;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_v;
// Native 16-byte vector (HIP's uint4 is a struct; arrays of it can defeat SROA).
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even; a NaN stays a NaN with the quiet bit set (the top
// payload bits kept). gfx950's v_cvt_pk_bf16_f32 does exactly this: it matched the integer
// formulation ((u + 0x7fff + lsb) >> 16; NaN: (u >> 16) | 0x40) on 4M random bit patterns
// including every NaN class, so the one-instruction form is used.
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_hw{lo, hi}), bf16x2_hw));
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return static_cast<bf16_t>(cvt_pk_bf16(f, 0.0f));
}

// Round an fp32 value to the nearest bf16 and return it as fp32.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// SwiGLU element on bf16-rounded inputs: bf16(silu(g)) * u (torch's F.silu(gate) * up,
// before the caller's final rounding). Shared by silu_mul_kernel and the GEMM epilogue that
// fuses it, so both give the same bits.
__device__ __forceinline__ float silu_mul1(float g, float u) {
  const float s = round_bf16(g / (1.0f + __expf(-g)));
  return s * u;
}

// Two fp32 values to packed bf16 (f32_to_bf16 of each).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return cvt_pk_bf16(lo, hi); }

// DPP lane exchanges inside a row of 16 lanes. The control words are the
// GCN/CDNA DPP encodings: quad_perm [1,0,3,2] swaps neighbours, quad_perm
// [2,3,0,1] swaps pairs, row_half_mirror reverses each group of 8 lanes,
// row_ror:8 rotates a 16-lane row by 8 (an exchange of the two halves).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;
constexpr int DPP_QUAD_XOR2 = 0x4E;
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_ROR8 = 0x128;

// Full-wave exchange for lanes farther apart than a DPP row (ds_bpermute).
__device__ __forceinline__ float lane_xor(float v, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ---- the sampler's seeded Gumbel noise (sid/engine/sampler.py:22-29) ----------------------
constexpr float kSampleEps = 1e-10f;

// The reference's noise for (seed, position, column): int64 arithmetic with wraparound,
// floor modulo 2^24 (= the low 24 bits in two's complement), u / 2^24. Only the low 24 bits
// of the hash are used, and the low bits of a product depend only on the low bits of its
// factors, so the per-column part is a 32-bit multiply and the per-row part (gumbel_row) is
// computed once.
__device__ __forceinline__ uint32_t gumbel_row(int64_t seed, int64_t pos) {
  const uint64_t step = (static_cast<uint64_t>(seed) * 19349663ull) ^
                        (static_cast<uint64_t>(pos) * 73856093ull);
  return static_cast<uint32_t>(step * 8589934591ull);
}

__device__ __forceinline__ float seeded_gumbel(uint32_t row_hash, int col) {
  const uint32_t h = row_hash ^ (static_cast<uint32_t>(col) * 479001599u);
  const float u = static_cast<float>(h & 0xffffffu) / 16777216.0f;
  return -logf(-logf(u + kSampleEps) + kSampleEps);
}

// Thread-local error message for the C-ABI (read back via sid_last_error()).
void set_error(const char* fmt, ...);
int check_launch(const char* what);

}  // namespace sid

#define SID_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::sid::set_error(__VA_ARGS__);           \
      return SID_ERR_INVALID;                  \
    }                                          \
  } while (0)
