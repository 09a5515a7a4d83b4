// Skinny GEMM of the decode / verify projections on gfx950:
//   Y[M, N] = X[M, K] W[N, K]^T   (bf16 in, fp32 accumulation, bf16 out), M <= 8.
//
// With M <= 8 rows (the gamma+1 verify tokens of one sequence, or the draft's
// single token) the projection streams its weight matrix once and does 2 * M
// flops per weight element: it is bound by HBM (or, for the draft's small
// matrices, by latency). An MFMA tile would be at least half empty here, so the
// products use v_dot2_f32_bf16 on the VALU, which lets every wave read its
// weights as whole contiguous 1 KB runs (lane l owns elements 8l .. 8l+7 of a
// 512-element K step).
//
// Work split: a workgroup owns kR output features (rows of W) and splits K
// evenly among its P waves. Each wave walks its K range in 512-element steps
// with the activations of the step in registers (kR weight loads per M
// activation loads), keeps kR x M fp32 partial sums, reduces them across the
// wave with butterfly shuffles and across the P waves through LDS.
// Epilogue 1 (SwiGLU, activation.py:8-16): the workgroup computes the gate rows
// n and the up rows F + n of a [2F, K] weight and writes
// bf16(bf16(silu(bf16(g))) * bf16(u)), the rounding of the unfused
// silu_mul(linear(x, gate_up)).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"

namespace hs {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x2_t as_bf2(uint32_t u) {
  union {
    uint32_t u;
    bf16x2_t v;
  } c;
  c.u = u;
  return c.v;
}

__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

constexpr int kStep = 512;  // K elements per wave step (64 lanes x 8)

constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }
constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }
constexpr int kMaxWaves = 8;

// One recursive-halving step (offset 32 >> ST) on the first NV >> ST values,
// unrolled at compile time: the lane keeps the half selected by its lane bit and
// adds the partner's copy of that half.
template <int NV, int ST, int NH>
__device__ __forceinline__ void halve(float (&v)[NV], int lane, int& idx) {
  if constexpr (ST < NH) {
    constexpr int o = 32 >> ST;
    constexpr int half = NV >> (ST + 1);
    const bool upper = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = upper ? v[i] : v[i + half];
      const float keep = upper ? v[i + half] : v[i];
      v[i] = keep + __shfl_xor(send, o, 64);
    }
    if (upper) idx += half;
    halve<NV, ST + 1, NH>(v, lane, idx);
  }
}

// Plain butterflies over the lane bits the halving did not consume.
template <int NV, int LEFT, int ST>
__device__ __forceinline__ void butterfly(float (&v)[NV], int lane) {
  (void)lane;
  if constexpr (ST < 6) {
    constexpr int o = 32 >> ST;
#pragma unroll
    for (int i = 0; i < LEFT; ++i) v[i] += __shfl_xor(v[i], o, 64);
    butterfly<NV, LEFT, ST + 1>(v, lane);
  }
}

template <int M, int R, int EPI>
__global__ __launch_bounds__(kMaxWaves * 64) void k_skinny(const uint16_t* __restrict__ X, int64_t xs,
                                                           const uint16_t* __restrict__ W, int K,
                                                           int F, uint16_t* __restrict__ Y,
                                                           int64_t ys, int steps_per_wave) {
  constexpr int RR = EPI ? 2 * R : R;  // weight rows of the workgroup
  __shared__ float s_part[kMaxWaves][RR * M];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int n0 = blockIdx.x * R;

  const uint16_t* wrow[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const int n = (EPI && r >= R) ? F + n0 + (r - R) : n0 + r;
    wrow[r] = W + (int64_t)n * K;
  }
  float acc[RR][M];
#pragma unroll
  for (int r = 0; r < RR; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  const int k0 = wid * steps_per_wave * kStep + 8 * lane;
  for (int s = 0; s < steps_per_wave; ++s) {
    const int k = k0 + s * kStep;
    uint4 xv[M], wv[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) wv[r] = *reinterpret_cast<const uint4*>(wrow[r] + k);
#pragma unroll
    for (int m = 0; m < M; ++m) xv[m] = *reinterpret_cast<const uint4*>(X + (int64_t)m * xs + k);
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float a = acc[r][m];
        a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[r].x), as_bf2(xv[m].x), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[r].y), as_bf2(xv[m].y), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[r].z), as_bf2(xv[m].z), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[r].w), as_bf2(xv[m].w), a, false);
        acc[r][m] = a;
      }
  }
  // wave sums by recursive halving: each exchange step sends half of the values
  // still held, so the NV values (RR * M padded to a power of two) cost NV - 1
  // shuffles instead of 6 NV; value i ends in lane i (NV <= 64) or lanes hold
  // NV / 64 consecutive values
  constexpr int NV = pow2_at_least(RR * M);
  float v[NV];
#pragma unroll
  for (int r = 0; r < RR; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) v[r * M + m] = acc[r][m];
#pragma unroll
  for (int i = RR * M; i < NV; ++i) v[i] = 0.0f;
  constexpr int kHalvings = NV < 64 ? ilog2(NV) : 6;
  int idx = 0;
  halve<NV, 0, kHalvings>(v, lane, idx);
  constexpr int kLeft = NV >> kHalvings;  // values per lane after halving
  butterfly<NV, kLeft, kHalvings>(v, lane);
  // lanes that differ only in the butterflied low bits hold the same values
  if ((lane & ((64 >> kHalvings) - 1)) == 0) {
#pragma unroll
    for (int i = 0; i < kLeft; ++i)
      if (idx + i < RR * M) s_part[wid][idx + i] = v[i];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= R * M) return;
  const int r = t / M, m = t % M;
  float y = 0.0f;
  for (int w = 0; w < nw; ++w) y += s_part[w][r * M + m];
  uint16_t out;
  if (EPI) {
    float u = 0.0f;
    for (int w = 0; w < nw; ++w) u += s_part[w][(R + r) * M + m];
    const float g = bfv(to_bf16(y));
    const uint16_t sl = to_bf16(g / (1.0f + __expf(-g)));
    out = to_bf16(bfv(sl) * bfv(to_bf16(u)));
  } else {
    out = to_bf16(y);
  }
  Y[(int64_t)m * ys + n0 + r] = out;
}

template <int M, int R, int EPI>
void launch_skinny(const uint16_t* X, int64_t xs, const uint16_t* W, int K, int N, int F,
                   uint16_t* Y, int64_t ys, hipStream_t stream) {
  const int steps = K / kStep;
  int waves = steps < kMaxWaves ? steps : kMaxWaves;
  while (steps % waves) --waves;
  hipLaunchKernelGGL((k_skinny<M, R, EPI>), dim3(N / R), dim3(64 * waves), 0, stream, X, xs, W, K,
                     F, Y, ys, steps / waves);
}

template <int R, int EPI>
void dispatch_m(int M, const uint16_t* X, int64_t xs, const uint16_t* W, int K, int N, int F,
                uint16_t* Y, int64_t ys, hipStream_t s) {
  switch (M) {
    case 1: launch_skinny<1, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 2: launch_skinny<2, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 3: launch_skinny<3, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 4: launch_skinny<4, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 5: launch_skinny<5, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 6: launch_skinny<6, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    case 7: launch_skinny<7, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
    default: launch_skinny<8, R, EPI>(X, xs, W, K, N, F, Y, ys, s); break;
  }
}

}  // namespace
}  // namespace hs

using namespace hs;

extern "C" {

int hs_linear(const void* x, int64_t x_stride, const void* weight, int rows, int in_features,
              int out_features, int epilogue, void* out, int64_t out_stride, void* stream) {
  if (!x || !weight || !out) return HS_ERR_INVALID;
  if (rows < 1 || in_features < 1 || out_features < 1) return HS_ERR_INVALID;
  if (epilogue != HS_LINEAR_PLAIN && epilogue != HS_LINEAR_SWIGLU) return HS_ERR_INVALID;
  if (rows > 8 || in_features % kStep) return HS_ERR_UNSUPPORTED;
  // with SwiGLU the weight is [2 * out_features, K] and the output [rows, out_features]
  const int N = out_features;
  const int R = (N % 8 == 0 && N >= 4096) ? 8 : 4;
  if (N % R) return HS_ERR_UNSUPPORTED;
  if ((x_stride % 8) || (out_stride < N) || (x_stride < in_features)) return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)x | (uintptr_t)weight) & 15) return HS_ERR_UNSUPPORTED;
  const uint16_t* X = static_cast<const uint16_t*>(x);
  const uint16_t* Wt = static_cast<const uint16_t*>(weight);
  uint16_t* Y = static_cast<uint16_t*>(out);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int F = N;  // up rows start at F (SwiGLU)
  if (epilogue == HS_LINEAR_SWIGLU) {
    if (R == 8) dispatch_m<8, 1>(rows, X, x_stride, Wt, in_features, N, F, Y, out_stride, s);
    else dispatch_m<4, 1>(rows, X, x_stride, Wt, in_features, N, F, Y, out_stride, s);
  } else {
    if (R == 8) dispatch_m<8, 0>(rows, X, x_stride, Wt, in_features, N, F, Y, out_stride, s);
    else dispatch_m<4, 0>(rows, X, x_stride, Wt, in_features, N, F, Y, out_stride, s);
  }
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

}  // extern "C"
