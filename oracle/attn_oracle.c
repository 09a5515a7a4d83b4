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

/* Nearest code among the 127 non-negative finite codes, whose values increase
 * with the code: a binary search over the value table brackets |x| between
 * codes c and c + 1, and the nearer one wins (ties to the even code, i.e. the
 * even mantissa). */
static float g_tab[127];
static int g_tab_ready = 0;

static void tab_init(void) {
  if (g_tab_ready) return;
  for (int c = 0; c <= 0x7e; ++c) g_tab[c] = or_e4m3fn_decode((uint8_t)c);
  g_tab_ready = 1;
}

uint8_t or_e4m3fn_encode_sat(float x) {
  if (isnan(x)) return 0x7f;
  tab_init();
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  float a = fabsf(x);
  if (a > 448.0f) a = 448.0f;
  int lo = 0, hi = 0x7e;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (g_tab[mid] <= a) lo = mid;
    else hi = mid - 1;
  }
  int best = lo;
  if (lo < 0x7e) {
    const double d0 = (double)a - (double)g_tab[lo];
    const double d1 = (double)g_tab[lo + 1] - (double)a;
    if (d1 < d0 || (d1 == d0 && ((lo + 1) & 1) == 0)) best = lo + 1;
  }
  return sign | (uint8_t)best;
}

void or_e4m3fn_quantize(const float* x, int64_t n, float scale, uint8_t* out) {
  tab_init();
  for (int64_t i = 0; i < n; ++i) out[i] = or_e4m3fn_encode_sat(x[i] / scale);
}
