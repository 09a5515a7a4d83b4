// Device helpers of the q/k-norm + RoPE + KV-store step, shared by its own
// kernel (model_ops.hip) and by the attention kernel that runs it in its
// prologue (verify_attention.hip), so both compute the same bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hs_fp8.h"

namespace hs {

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// f32 -> bf16, round to nearest even
__device__ __forceinline__ uint16_t to_bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));  // v_cvt_pk_bf16_f32 (RNE)
}
// bf16 * bf16 rounded to bf16 (the product is exact in fp32)
__device__ __forceinline__ uint16_t bf_mul(uint16_t a, uint16_t b) { return to_bf(bf(a) * bf(b)); }

// lane-exchange moves within a 16-lane row (DPP): the value of lane l ^ 1,
// l ^ 2, 7 - l within its 8 lanes, and l ^ 8
__device__ __forceinline__ float row_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_mirror8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a row with the same bits in every lane, all in
// VALU: pairwise adds over the lanes l ^ 1, l ^ 2, 7 - l and l ^ 8. Both lanes
// of a pair add the same two values, so every lane ends with the same sum.
__device__ __forceinline__ float row16_sum(float v) {
#pragma clang fp contract(off)
  v += row_xor1(v);
  v += row_xor2(v);
  v += row_mirror8(v);
  v += row_xor8(v);
  return v;
}

// RMSNorm (layernorm.py:18-25: normalise in fp32, round, multiply by the
// weight) and neox RoPE (rotary_embedding.py:8-16, cos/sin cache [pos, 64 |
// 64]) of one 128-wide head held by a 16-lane row: lane j of the row holds
// dims 8j .. 8j + 7 (x, fp32 of the bf16 inputs), their weights w, and the
// rotation c, s of frequencies (8j .. 8j + 7) mod 64; the rotation partner of
// dim d < 64 is dim d + 64, in lane j ^ 8. Returns the rotated head rounded to
// bf16. Every product and sum is rounded on its own (as torch's fp32 ops), so
// the bits do not depend on which kernel inlines it; the sum of squares is
// the lane's eight in order, then the row's tree.
__device__ __forceinline__ void norm_rope_row(const float (&x)[8], const uint16_t (&w)[8],
                                              const float (&c)[8], const float (&s)[8],
                                              float eps, int j, uint16_t (&y)[8]) {
#pragma clang fp contract(off)
  float ss = x[0] * x[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) ss += x[k] * x[k];
  ss = row16_sum(ss);
  const float inv = rsqrtf(ss / 128.0f + eps);
  float xn[8], pn[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) xn[k] = bf(bf_mul(to_bf(x[k] * inv), w[k]));
#pragma unroll
  for (int k = 0; k < 8; ++k) pn[k] = row_xor8(xn[k]);
  if (j < 8) {  // dims d < 64: x1 = xn, x2 = partner
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = to_bf(xn[k] * c[k] - pn[k] * s[k]);
  } else {      // dims d + 64: x2 = xn, x1 = partner
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = to_bf(xn[k] * c[k] + pn[k] * s[k]);
  }
}

// 8 bf16 values of a 16-byte load
__device__ __forceinline__ void unpack8(uint4 u, uint16_t (&h)[8]) {
  h[0] = (uint16_t)u.x; h[1] = (uint16_t)(u.x >> 16);
  h[2] = (uint16_t)u.y; h[3] = (uint16_t)(u.y >> 16);
  h[4] = (uint16_t)u.z; h[5] = (uint16_t)(u.z >> 16);
  h[6] = (uint16_t)u.w; h[7] = (uint16_t)(u.w >> 16);
}
__device__ __forceinline__ uint4 pack8(const uint16_t (&h)[8]) {
  return make_uint4((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                    (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16));
}

// the rotation of dims 8j .. 8j + 7 from a cos/sin row [cos 64 | sin 64]
__device__ __forceinline__ void load_rot8(const float* cs_row, int j, float (&c)[8],
                                          float (&s)[8]) {
  const int f = (8 * j) & 63;
  const float4 c0 = *reinterpret_cast<const float4*>(cs_row + f);
  const float4 c1 = *reinterpret_cast<const float4*>(cs_row + f + 4);
  const float4 s0 = *reinterpret_cast<const float4*>(cs_row + 64 + f);
  const float4 s1 = *reinterpret_cast<const float4*>(cs_row + 64 + f + 4);
  c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
  c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
  s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w;
  s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;
}

// the e4m3fn code a cache with per-tensor scale `scale` stores for bf16 value a
__device__ __forceinline__ uint8_t e4m3_of_bf16(uint16_t a, float scale) {
#pragma clang fp contract(off)
  return f32_to_e4m3fn_sat(bf(a) / scale);
}

// e4m3fn codes of 8 bf16 values, packed in two dwords
__device__ __forceinline__ uint2 e4m3x8_of_bf16(const uint16_t (&h)[8], float scale) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    lo |= (uint32_t)e4m3_of_bf16(h[k], scale) << (8 * k);
    hi |= (uint32_t)e4m3_of_bf16(h[4 + k], scale) << (8 * k);
  }
  return make_uint2(lo, hi);
}

// dims 8j .. 8j + 7 of a cache row at element offset elem: 16 bf16 bytes, or
// 8 e4m3fn codes for an FP8 cache with per-tensor scale `scale`
template <bool kFp8>
__device__ __forceinline__ void store_row8(uint8_t* base, int64_t elem, int j,
                                           const uint16_t (&h)[8], float scale) {
  if constexpr (kFp8)
    *reinterpret_cast<uint2*>(base + elem + 8 * j) = e4m3x8_of_bf16(h, scale);
  else
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + elem + 8 * j) = pack8(h);
}

}  // namespace hs
