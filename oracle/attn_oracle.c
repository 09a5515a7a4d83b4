/*
 * attn_oracle.c - CPU restatement of the FP8 e4m3fn KV-cache number format.
 *
 * TEST INFRASTRUCTURE ONLY (checker for hilda-vllm_amd/csrc/kv_cache.hip and
 * the FP8 path of verify_attention.hip; never linked into the product).
 *
 * The reference imports its FP8 store/attention kernels from an external
 * package that is not in the reference tree (mini_vllm/layers/attention.py:
 * 17-56); its cache dtype is torch.float8_e4m3fn (model_runner.py:151). This
 * file defines the format the build uses: OCP E4M3FN (bias 7, no infinities,
 * S.1111.111 = NaN, max 448), dequantised as code * scale, quantised as
 * sat_e4m3fn(x / scale) with round-to-nearest-even and saturation at +-448.
 * It is written from the format definition (a value table), independently of
 * the kernel's bit manipulation.
 */
#include <math.h>
#include <stdint.h>

float or_e4m3fn_decode(uint8_t c) {
  const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + m / 8.0f, e - 7);
  return s ? -v : v;
}

/* nearest code by exhaustive search over the 127 non-negative finite codes */
uint8_t or_e4m3fn_encode_sat(float x) {
  if (isnan(x)) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  float a = fabsf(x);
  if (a > 448.0f) a = 448.0f;
  int best = 0;
  double bd = INFINITY;
  for (int c = 0; c <= 0x7e; ++c) {
    double d = fabs((double)or_e4m3fn_decode((uint8_t)c) - (double)a);
    /* ties to even code (even mantissa) */
    if (d < bd || (d == bd && (c & 1) == 0)) {
      bd = d;
      best = c;
    }
  }
  return sign | (uint8_t)best;
}

void or_e4m3fn_quantize(const float* x, int64_t n, float scale, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_e4m3fn_encode_sat(x[i] / scale);
}
