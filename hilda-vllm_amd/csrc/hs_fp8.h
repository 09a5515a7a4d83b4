// FP8 e4m3fn encoding of the KV-cache stores (kv_cache.hip, model_ops.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace hs {

// float -> fp8 e4m3fn, round to nearest even, saturating to +-448, NaN -> 0x7f
__device__ __forceinline__ uint8_t f32_to_e4m3fn_sat(float v) {
  const uint32_t bits = __float_as_uint(v);
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  float a = fabsf(v);
  if (a != a) return 0x7f;
  if (a >= 448.0f) return sign | 0x7e;
  if (a < 0x1p-6f) {  // subnormal range: multiples of 2^-9
    const int qv = (int)rintf(a * 512.0f);  // 0..8; 8 is the smallest normal (code 0x08)
    return sign | (uint8_t)qv;
  }
  int e = (int)((__float_as_uint(a) >> 23) & 0xffu) - 127;  // floor(log2 a), in [-6, 8]
  float scaled = ldexpf(a, 3 - e);                            // [8, 16)
  int qv = (int)rintf(scaled);
  if (qv == 16) {
    qv = 8;
    e += 1;
  }
  int code = ((e + 7) << 3) | (qv - 8);
  if (code > 0x7e) code = 0x7e;
  return sign | (uint8_t)code;
}

}  // namespace hs
