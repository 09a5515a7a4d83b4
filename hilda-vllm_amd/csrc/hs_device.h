// Device-side arithmetic shared by the hilda-spec kernels (gfx950 / CDNA4).
//
// Every kernel that feeds an accept/reject decision or a sampled token uses
// only the functions below, so the result of each decision is a pure function
// of the inputs:
//   * hs_exp     - exp(y) for y <= 0 by Cody-Waite range reduction (ln2 split
//                  in a 16-bit high part and a low part) and the degree-7
//                  Taylor polynomial of exp(r), |r| <= ln2/2, in Horner form
//                  with explicit fused multiply-adds; the result is flushed to
//                  0 below y = -86 so that it is never subnormal.
//   * hs_div_t   - x / T, correctly rounded (IEEE division semantics); T == 1
//                  is the identity.
//   * hs_fx44    - floor(v * 2^44) as an unsigned 64-bit integer, taken from
//                  the float's bit pattern (no float->int conversion rounding).
//   * hs_f32_of_u64 - round-to-nearest-even conversion of a u64 to float;
//                  hs_f32_rz_of_u64 rounds toward zero and is used for every
//                  softmax normaliser (sum of fixed-point exps), so that
//                  probabilities are never rounded below the fp32 value a
//                  sequential fp32 softmax gives on the reference's
//                  known-answer inputs.
//   * hs_key     - order-preserving map float -> u32 (-0.0 folded onto +0.0).
// With these, softmax normalisers and cumulative masses are exact integer sums
// and do not depend on the order in which waves or workgroups add them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace hs {

constexpr int kWave = 64;
constexpr int kChunk = 2048;          // elements per softmax chunk
constexpr int kChunkGroups = 4;       // lane holds 4 groups of 8 elements
constexpr int kGroupElems = 8;
constexpr float kTwo44 = 17592186044416.0f;        // 2^44
constexpr float kTwoM44 = 5.684341886080801e-14f;  // 2^-44
constexpr float kTwo40 = 1099511627776.0f;         // 2^40
constexpr float kTwoM40 = 9.094947017729282e-13f;  // 2^-40

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// exp(y), y <= 0 (values above 0 are clamped to y = 0 by callers' max
// subtraction; NaN maps to 0).
__device__ __forceinline__ float hs_exp(float y) {
  if (!(y >= -86.0f)) return 0.0f;
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;       // 16 significant bits
  const float kLn2Lo = 1.428606765330187e-06f;   // ln2 - kLn2Hi
  float t = y * kLog2e;
  float k = rintf(t);
  float r = fmaf(-k, kLn2Hi, y);
  r = fmaf(-k, kLn2Lo, r);
  // 1/n! for n = 7..2
  float p = 1.98412698e-04f;
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ki = (int)k;  // in [-125, 0]
  float scale = u2f((uint32_t)(ki + 127) << 23);
  return p * scale;
}

// hs_exp(y) * 2^20, equal bit for bit to that product, without a branch:
//   * every coefficient of the polynomial carries the factor 2^20; scaling by
//     a power of two commutes with each rounding while the values stay normal,
//     which they do here (p in [2^19, 2^21), result >= 2^-105);
//   * k = rint(t) by the rounding constant 1.5 * 2^23: t + 1.5 * 2^23 rounds t
//     to the nearest integer, ties to even (the constant is even), as rintf
//     does for |t| < 2^22, and the sum's low bits are 0x4B400000 + k, which
//     give 2^k without a float->int conversion. k's zero may be +0 where
//     rintf gives -0; r is then the same value, and fma(p, r, c) with r = +-0
//     returns c;
//   * for y < -86 and NaN the value is computed and then discarded.
__device__ __forceinline__ float hs_exp_2p20(float y) {
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.428606765330187e-06f;
  const float kS = 1048576.0f;       // 2^20
  const float kRound = 12582912.0f;  // 1.5 * 2^23
  const float t = y * kLog2e;
  const float kf = t + kRound;
  const float k = kf - kRound;
  float r = fmaf(-k, kLn2Hi, y);
  r = fmaf(-k, kLn2Lo, r);
  float p = 1.98412698e-04f * kS;
  p = fmaf(p, r, 1.38888889e-03f * kS);
  p = fmaf(p, r, 8.33333333e-03f * kS);
  p = fmaf(p, r, 4.16666667e-02f * kS);
  p = fmaf(p, r, 1.66666667e-01f * kS);
  p = fmaf(p, r, 0.5f * kS);
  p = fmaf(p, r, 1.0f * kS);
  p = fmaf(p, r, 1.0f * kS);
  const float scale = u2f((f2u(kf) - 0x4B400000u + 127u) << 23);
  const float v = p * scale;
  return (y >= -86.0f) ? v : 0.0f;
}

// Correctly rounded x / t. For t == 1 the division is skipped (exact).
__device__ __forceinline__ float hs_div_t(float x, float t) {
  return (t == 1.0f) ? x : x / t;
}

// Correctly rounded a / b given rb = a correctly rounded 1/b: one product and
// one remainder-correction step (Markstein). The correction is exact for
// |a| in [2^-96, 2^60] and b in [2^-10, 2^20] (checked against IEEE division
// on 7e8 operand pairs); outside that range, and for zero numerators (sign of
// zero), the IEEE division is used.
__device__ __forceinline__ float hs_div_rcp(float a, float b, float rb) {
  const float aa = fabsf(a);
  if (!(aa >= 0x1p-96f && aa <= 0x1p60f)) return a / b;
  const float q = a * rb;
  const float r = fmaf(-q, b, a);
  return fmaf(r, rb, q);
}
// The corrected product alone, for callers that have checked the range.
__device__ __forceinline__ float hs_div_rcp_in_range(float a, float b, float rb) {
  const float q = a * rb;
  const float r = fmaf(-q, b, a);
  return fmaf(r, rb, q);
}
// True when hs_div_rcp may be used with divisor b.
__device__ __forceinline__ bool hs_rcp_ok(float b) { return b >= 0x1p-10f && b <= 0x1p20f; }

// x / t for the temperature: identity for t == 1, else the corrected product
// (rt = 1/t correctly rounded, fast = hs_rcp_ok(t)).
__device__ __forceinline__ float hs_div_temp(float x, float t, float rt, bool fast) {
  if (t == 1.0f) return x;
  return fast ? hs_div_rcp(x, t, rt) : x / t;
}

// floor(v * 2^44) for v in [0, 1] split as hi * 2^24 + lo with 32-bit parts:
// hi = floor(v 2^20), lo = floor(frac(v 2^20) 2^24). Each step is exact
// (scaling by powers of two, Sterbenz subtraction, truncating conversion).
__device__ __forceinline__ void hs_fx44_split(float v, uint32_t& hi, uint32_t& lo) {
  const float t = v * 1048576.0f;
  const uint32_t h = (uint32_t)t;
  const float f = t - (float)h;
  hi += h;
  lo += (uint32_t)(f * 16777216.0f);
}
// hs_fx44_split of v given t = v * 2^20 (hs_exp_2p20's output): the same two
// parts, the fraction by v_fract (t - floor(t), exact for t in [0, 2^20]).
__device__ __forceinline__ void hs_fx44_acc(float t, uint32_t& hi, uint32_t& lo) {
  hi += (uint32_t)t;
  lo += (uint32_t)(__builtin_amdgcn_fractf(t) * 16777216.0f);
}
__device__ __forceinline__ uint64_t hs_join44(uint32_t hi, uint32_t lo) {
  return ((uint64_t)hi << 24) + (uint64_t)lo;
}

// floor(v * 2^44) for 0 <= v < 2^19 (v finite); negative or NaN -> 0.
__device__ __forceinline__ uint64_t hs_fx44(float v) {
  uint32_t b = f2u(v);
  if (b & 0x80000000u) return 0;
  int ex = (int)((b >> 23) & 0xffu);
  if (ex == 0 || ex == 0xff) return 0;
  uint64_t m = (uint64_t)((b & 0x7fffffu) | 0x800000u);
  int sh = ex - 150 + 44;
  if (sh >= 0) return m << sh;
  if (sh <= -24) return 0;
  return m >> (-sh);
}

// floor(v * 2^40), same domain rules.
__device__ __forceinline__ uint64_t hs_fx40(float v) {
  uint32_t b = f2u(v);
  if (b & 0x80000000u) return 0;
  int ex = (int)((b >> 23) & 0xffu);
  if (ex == 0 || ex == 0xff) return 0;
  uint64_t m = (uint64_t)((b & 0x7fffffu) | 0x800000u);
  int sh = ex - 150 + 40;
  if (sh >= 0) return m << sh;
  if (sh <= -24) return 0;
  return m >> (-sh);
}

// u64 -> float, round to nearest even.
__device__ __forceinline__ float hs_f32_of_u64(uint64_t n) {
  if (n == 0) return 0.0f;
  int msb = 63 - __clzll((long long)n);
  if (msb <= 23) return (float)(uint32_t)n;
  int sh = msb - 23;
  uint64_t m = n >> sh;
  uint64_t rem = n & ((1ull << sh) - 1ull);
  uint64_t half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (m & 1ull))) m++;
  if (m == (1ull << 24)) { m >>= 1; sh++; }
  // value = m * 2^sh with m in [2^23, 2^24)
  uint32_t bits = ((uint32_t)(sh + 23 + 127) << 23) | ((uint32_t)m & 0x7fffffu);
  return u2f(bits);
}

// u64 -> float, round toward zero (used for every softmax normaliser).
__device__ __forceinline__ float hs_f32_rz_of_u64(uint64_t n) {
  if (n == 0) return 0.0f;
  int msb = 63 - __clzll((long long)n);
  if (msb <= 23) return (float)(uint32_t)n;
  int sh = msb - 23;
  uint64_t m = n >> sh;
  uint32_t bits = ((uint32_t)(sh + 23 + 127) << 23) | ((uint32_t)m & 0x7fffffu);
  return u2f(bits);
}

// Order-preserving key: larger float -> larger key; -0.0 == +0.0.
__device__ __forceinline__ uint32_t hs_key(float x) {
  uint32_t b = f2u(x);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float hs_unkey(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return u2f(b);
}

// floor(u24 * w / 2^24) for u24 < 2^24, w < 2^62 (exact 86-bit product).
__device__ __forceinline__ uint64_t hs_mulshift24(uint32_t u24, uint64_t w) {
  uint64_t hi = w >> 32, lo = w & 0xffffffffull;
  return ((uint64_t)u24 * hi << 8) + (((uint64_t)u24 * lo) >> 24);
}

// Uniform in [0,1) -> 24-bit fixed point, clamped into [0, 2^24 - 1].
__device__ __forceinline__ uint32_t hs_u24(float u) {
  if (!(u > 0.0f)) return 0u;
  float s = u * 16777216.0f;
  if (s >= 16777215.0f) return 16777215u;
  return (uint32_t)s;  // truncation; s is in [0, 2^24)
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

// ---- wave-level reductions (64 lanes) ----
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, o, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = (uint64_t)__shfl_xor((unsigned long long)v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
// inclusive prefix sum across the wave (lane order)
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint64_t w = (uint64_t)__shfl_up((unsigned long long)v, o, 64);
    if (lane >= o) v += w;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t w = (uint32_t)__shfl_up((int)v, o, 64);
    if (lane >= o) v += w;
  }
  return v;
}

}  // namespace hs
