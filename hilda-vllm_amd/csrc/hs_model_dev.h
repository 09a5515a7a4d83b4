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

// RMSNorm (layernorm.py:18-25: normalise in fp32, round, multiply by the
// weight) and neox RoPE (rotary_embedding.py:8-16, cos/sin cache [pos, 64 | 64])
// of one 128-wide head held as the pair (l, l + 64) by lane l, from the
// lane's values x1, x2, weights w1, w2 and rotation c, s; returns the rotated
// pair rounded to bf16. Every product and sum is rounded on its own (as
// torch's fp32 ops), so the bits do not depend on which kernel inlines it.
__device__ __forceinline__ void norm_rope_vals(float x1, float x2, uint16_t w1, uint16_t w2,
                                               float c, float s, float eps, uint16_t& o1,
                                               uint16_t& o2) {
#pragma clang fp contract(off)
  float ss = x1 * x1 + x2 * x2;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = rsqrtf(ss / 128.0f + eps);
  x1 = bf(bf_mul(to_bf(x1 * inv), w1));
  x2 = bf(bf_mul(to_bf(x2 * inv), w2));
  o1 = to_bf(x1 * c - x2 * s);
  o2 = to_bf(x2 * c + x1 * s);
}

// norm_rope_vals of the head at src with weights w and cos/sin row cs
__device__ __forceinline__ void norm_rope_pair(const uint16_t* src, const uint16_t* w,
                                               const float* cs, float eps, int lane,
                                               uint16_t& o1, uint16_t& o2) {
  norm_rope_vals(bf(src[lane]), bf(src[lane + 64]), w[lane], w[lane + 64], cs[lane],
                 cs[64 + lane], eps, o1, o2);
}

// the e4m3fn code a cache with per-tensor scale `scale` stores for bf16 value a
__device__ __forceinline__ uint8_t e4m3_of_bf16(uint16_t a, float scale) {
#pragma clang fp contract(off)
  return f32_to_e4m3fn_sat(bf(a) / scale);
}

template <bool kFp8>
__device__ __forceinline__ void store_pair(uint8_t* base, int64_t elem, int lane, uint16_t a,
                                           uint16_t b, float scale) {
  if constexpr (kFp8) {
    base[elem + lane] = e4m3_of_bf16(a, scale);
    base[elem + lane + 64] = e4m3_of_bf16(b, scale);
  } else {
    uint16_t* p = reinterpret_cast<uint16_t*>(base) + elem;
    p[lane] = a;
    p[lane + 64] = b;
  }
}

}  // namespace hs
