// Row arithmetic shared by the norm / RoPE kernels and the GEMMs that fuse them
// (norm_rope.hip, decode_chain.hip): every kernel that computes an RMSNorm, a q/k-norm or a
// rotary pair goes through these helpers, so fused and unfused paths give the same bits.
#pragma once

#include "common.h"

namespace sid {

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

// ---- shared arithmetic --------------------------------------------------------------

__device__ __forceinline__ float sumsq8(const float (&v)[8], float acc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = fmaf(v[e], v[e], acc);
  return acc;
}

// Xor butterfly over an aligned group of `lpr` lanes (identical bits in every lane).
__device__ __forceinline__ float group_sum(float v, int lpr) {
  for (int mask = 1; mask < lpr; mask <<= 1) v += lane_xor(v, mask);
  return v;
}

// group_sum(v, 64) with the same bits, without LDS round trips: the xor-1 / xor-2 steps are
// DPP quad permutations; after them a quad holds one value, so the xor-4 partner can be any
// lane of the other quad (DPP half-mirror); xor-8 is DPP row_ror:8; after that each 16-lane
// row holds one value R_k, and the last two butterfly steps give (R0 + R1) + (R2 + R3) in
// every lane (IEEE addition is commutative, so every lane's sum has the same bits).
__device__ __forceinline__ float group_sum64(float v) {
  v += dpp<DPP_QUAD_XOR1>(v);
  v += dpp<DPP_QUAD_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_ROW_ROR8>(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ float rms_rstd(float sumsq, int hidden, float eps) {
  return 1.0f / sqrtf(sumsq / static_cast<float>(hidden) + eps);
}

__device__ __forceinline__ void rms_apply8(const float (&v)[8], float rstd, const float (&w)[8],
                                           float (&y)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (v[e] * rstd) * w[e];
}

// NeoX rotate-half on one (x1, x2) = (x[i], x[i + D/2]) pair.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& o1, float& o2) {
  o1 = fmaf(x1, c, -(x2 * s));
  o2 = fmaf(x2, c, x1 * s);
}

// group_sum(v, 16) with the same bits, all in DPP (see group_sum64).
__device__ __forceinline__ float group_sum16(float v) {
  v += dpp<DPP_QUAD_XOR1>(v);
  v += dpp<DPP_QUAD_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_ROW_ROR8>(v);
  return v;
}

// The per-lane operands of qk_head_norm_rope that come from memory, so a kernel can load
// them ahead of the values: the norm weights of the lane's 8 dims, and cos / sin of their
// rotary indices at the row's position (rot false: position outside the table). Loads
// only: the values are converted where they are used, so waiting for them never waits for
// loads issued after these.
struct QkRopeIn {
  uint4 w;            // 8 bf16 norm weights
  float4 c[2], s[2];  // cos / sin of the lane's 8 rotary indices
  bool rot;
};

__device__ __forceinline__ void qk_rope_load(QkRopeIn& in, int j, const uint4* __restrict__ w,
                                             int64_t pos, const float* __restrict__ cos_sin,
                                             int64_t max_positions) {
  constexpr int D = 128;
  in.w = w[j];
  in.rot = pos >= 0 && pos < max_positions;
  const float* cs = cos_sin + (in.rot ? pos : 0) * D + 8 * (j & 7);
  in.c[0] = *reinterpret_cast<const float4*>(cs);
  in.c[1] = *reinterpret_cast<const float4*>(cs + 4);
  in.s[0] = *reinterpret_cast<const float4*>(cs + D / 2);
  in.s[1] = *reinterpret_cast<const float4*>(cs + D / 2 + 4);
}

// One q or k head of the fused QKV epilogue, held by an aligned group of 16 lanes (lane j:
// dims 8j..8j+7 of the head, head_dim 128): per-head RMSNorm with weight w (rmsnorm's lane
// layout for hidden 128: sequential fmaf over the lane's 8 dims, xor butterfly over the 16
// lanes), rounded to bf16, then NeoX RoPE (the rotate-half partner of lane j is lane j ^ 8,
// one DPP row_ror:8 away) with the fp32 [cos(64) | sin(64)] table row of the position; a
// position outside the table leaves the normed values. Every lane of the 16 must be active.
__device__ __forceinline__ void qk_head_norm_rope(const float (&v)[8], int j, const QkRopeIn& in,
                                                  float eps, float (&o)[8]) {
  constexpr int D = 128;
  float wf[8], y[8];
  load8(in.w, wf);
  const float c[8] = {in.c[0].x, in.c[0].y, in.c[0].z, in.c[0].w,
                      in.c[1].x, in.c[1].y, in.c[1].z, in.c[1].w};
  const float sn[8] = {in.s[0].x, in.s[0].y, in.s[0].z, in.s[0].w,
                       in.s[1].x, in.s[1].y, in.s[1].z, in.s[1].w};
  const float ss = group_sum16(sumsq8(v, 0.0f));
  rms_apply8(v, rms_rstd(ss, D, eps), wf, y);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf16(y[e]);
  const bool first_half = j < 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float partner = dpp<DPP_ROW_ROR8>(y[e]);
    float o1, o2;
    if (first_half) {
      rope_pair(y[e], partner, c[e], sn[e], o1, o2);
      o[e] = o1;
    } else {
      rope_pair(partner, y[e], c[e], sn[e], o1, o2);
      o[e] = o2;
    }
    if (!in.rot) o[e] = y[e];
  }
}

}  // namespace sid
