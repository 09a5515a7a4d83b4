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
// Work split: persistent workgroups (as many as fit on the chip at once) walk
// tiles of kR output features (rows of W), tile = blockIdx.x + i * gridDim.x.
// A workgroup splits K evenly among its P waves (S 512-element steps each);
// every wave loads its K slice of the M activation rows once, keeps it in
// registers for all of the workgroup's tiles, and per tile streams kR x S
// weight vectors (non-temporal loads: each weight is read once per call),
// keeps kR x M fp32 partial sums, reduces them across the wave with
// recursive-halving shuffles and across the P waves through LDS (two buffers,
// one barrier per tile). Weight tiles are double-buffered in registers: a
// workgroup issues its first two tiles before the activation prologue, and
// refills a buffer with the tile two ahead as soon as its products are done,
// so two tiles per wave are in flight while the sums are combined.
// Epilogue 1 (SwiGLU, activation.py:8-16): the tile holds the gate rows n and
// the up rows F + n of a [2F, K] weight and writes
// bf16(bf16(silu(bf16(g))) * bf16(u)), the rounding of the unfused
// silu_mul(linear(x, gate_up)).
// Prologue (hs_linear_rmsnorm): the activation rows are the decoder's RMSNorm
// of x (+ residual) (layernorm.py:18-36). Every wave sums the squares of its K
// slice, the workgroup combines the wave sums through LDS, and each wave
// normalises the slice it holds; workgroup 0 also writes the new residual
// bf16(x + residual). Being persistent, a workgroup does this once for all of
// its tiles, which replaces the separate norm launch in front of the qkv and
// gate_up projections at the cost of one extra barrier per workgroup.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"

namespace hs {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x2_t as_bf2(uint32_t u) { return __builtin_bit_cast(bf16x2_t, u); }

__device__ __forceinline__ float bfv(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// f32 -> bf16, round to nearest even
__device__ __forceinline__ uint16_t to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));  // v_cvt_pk_bf16_f32 (RNE)
}
// two f32 -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

constexpr int kStep = 512;  // K elements per wave step (64 lanes x 8)
constexpr int kMaxWaves = 8;
constexpr int kR = 4;       // output features per tile
constexpr int kMaxS = 3;    // K steps per wave (K <= 8 * 3 * 512 = 12288)
constexpr int kMaxNormS = 2;

// weights are streamed once per call: non-temporal, so that they do not evict
// the activation rows and the other workgroups' data from the caches
__device__ __forceinline__ uint4 load_stream(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }
constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

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

// Sums NV0 per-lane values over the wave and stores value i of the wave at
// dst[i] (dst in LDS). NV0 - 1 shuffles for NV0 <= 64 instead of 6 * NV0.
template <int NV0>
__device__ __forceinline__ void wave_sums_to(const float (&vals)[NV0], int lane, float* dst) {
  constexpr int NV = pow2_at_least(NV0);
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV0; ++i) v[i] = vals[i];
#pragma unroll
  for (int i = NV0; i < NV; ++i) v[i] = 0.0f;
  constexpr int kH = NV < 64 ? ilog2(NV) : 6;
  int idx = 0;
  halve<NV, 0, kH>(v, lane, idx);
  constexpr int kLeft = NV >> kH;  // values per lane after halving
  butterfly<NV, kLeft, kH>(v, lane);
  // lanes that differ only in the butterflied low bits hold the same values
  if ((lane & ((64 >> kH) - 1)) == 0) {
#pragma unroll
    for (int i = 0; i < kLeft; ++i)
      if (idx + i < NV0) dst[idx + i] = v[i];
  }
}

struct SkinnyArgs {
  const uint16_t* X;  // [M, K] activations (row stride xs)
  int64_t xs;
  const uint16_t* W;  // [N, K] weight ([2F, K] gate | up with SwiGLU)
  int K;
  int F;       // first up row (SwiGLU)
  int ntiles;  // N / kR
  uint16_t* Y;  // [M, N] output (row stride ys)
  int64_t ys;
  // RMSNorm prologue (NORM): X <- bf16(bf16((X + Rin) * inv_rms) * NW)
  const uint16_t* Rin;  // may be null
  int64_t rs_in;
  uint16_t* Rout;  // bf16(X + Rin), written by workgroup 0; may be null
  int64_t rs_out;
  const uint16_t* NW;
  float eps;
};

__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  f[0] = bfv((uint16_t)u.x);
  f[1] = bfv((uint16_t)(u.x >> 16));
  f[2] = bfv((uint16_t)u.y);
  f[3] = bfv((uint16_t)(u.y >> 16));
  f[4] = bfv((uint16_t)u.z);
  f[5] = bfv((uint16_t)(u.z >> 16));
  f[6] = bfv((uint16_t)u.w);
  f[7] = bfv((uint16_t)(u.w >> 16));
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint4 u;
  u.x = pk_bf16(f[0], f[1]);
  u.y = pk_bf16(f[2], f[3]);
  u.z = pk_bf16(f[4], f[5]);
  u.w = pk_bf16(f[6], f[7]);
  return u;
}

template <int S, int RR>
__device__ __forceinline__ void load_tile(uint4 (&wv)[S][RR], const SkinnyArgs& a, int tile,
                                          int k0) {
  const int n0 = tile * kR;
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const int n = r >= kR ? a.F + n0 + (r - kR) : n0 + r;
    const uint16_t* row = a.W + (int64_t)n * a.K + k0;
#pragma unroll
    for (int s = 0; s < S; ++s) wv[s][r] = load_stream(row + s * kStep);
  }
}

// Activation slice of the wave, raw: xr[s][m] = 8 bf16 of row m at k0 + s * kStep
// (and the residual rows rr with RES, the norm weights nr with NORM). Issued
// before the weight loads and fenced from them, so the prologue that consumes
// them waits for these loads only while the weights are still in flight.
template <int M, int S, bool NORM, bool RES>
__device__ __forceinline__ void issue_activations(uint4 (&xr)[S][M], uint4 (&rr)[S][M],
                                                  uint4 (&nr)[S], const SkinnyArgs& a, int k0) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int64_t k = k0 + s * kStep;
      xr[s][m] = *reinterpret_cast<const uint4*>(a.X + (int64_t)m * a.xs + k);
      if (RES) rr[s][m] = *reinterpret_cast<const uint4*>(a.Rin + (int64_t)m * a.rs_in + k);
    }
    if (NORM) nr[s] = *reinterpret_cast<const uint4*>(a.NW + k0 + s * kStep);
  }
  // keeps the compiler from interleaving these loads with the weight loads
  // issued next (loads complete in order, so a wait for the last activation
  // load would otherwise also wait for the weights issued before it)
  asm volatile("" ::: "memory");
}

// Projection input of the wave from the raw slices: the slices themselves, or
// (NORM) their RMSNorm with the workgroup-wide sum of squares.
template <int M, int S, bool NORM, bool RES>
__device__ __forceinline__ void finish_activations(uint4 (&xv)[S][M], const uint4 (&xr)[S][M],
                                                   const uint4 (&rr)[S][M], const uint4 (&nr)[S],
                                                   const SkinnyArgs& a,
                                                   int k0, int lane, int wid, int nw) {
  if constexpr (!NORM) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) xv[s][m] = xr[s][m];
  } else {
    __shared__ float s_ss[kMaxWaves][M];
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        // x (+ residual) in fp32, element by element as the unfused add + RMSNorm
        float f[8];
        unpack8(xr[s][m], f);
        if (RES) {
          float g[8];
          unpack8(rr[s][m], g);
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] += g[j];
          if (a.Rout && blockIdx.x == 0)
            *reinterpret_cast<uint4*>(a.Rout + (int64_t)m * a.rs_out + k0 + s * kStep) = pack8(f);
        } else if (a.Rout && blockIdx.x == 0) {
          *reinterpret_cast<uint4*>(a.Rout + (int64_t)m * a.rs_out + k0 + s * kStep) = xr[s][m];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss[m] += f[j] * f[j];
      }
    wave_sums_to<M>(ss, lane, s_ss[wid]);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float nwf[8];
      unpack8(nr[s], nwf);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float t = 0.0f;
        for (int w = 0; w < nw; ++w) t += s_ss[w][m];
        const float inv = rsqrtf(t / (float)a.K + a.eps);
        float f[8];
        unpack8(xr[s][m], f);
        if (RES) {
          float g[8];
          unpack8(rr[s][m], g);
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] += g[j];
        }
        // layernorm.py:18-36: normalise in fp32, round, multiply by the weight
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = bfv(to_bf16(f[j] * inv)) * nwf[j];
        xv[s][m] = pack8(f);
      }
    }
  }
}

// One tile: products of the wave's weight slice wv with the activations, the
// weight loads of tile `prefetch` issued into wv as soon as it is consumed
// (PF 1: always, PF 2: if that tile exists, PF 0: none), then the wave /
// workgroup reduction and the tile's outputs.
template <int M, int S, int EPI, int PF>
__device__ __forceinline__ void tile_step(uint4 (&wv)[S][EPI ? 2 * kR : kR],
                                          const uint4 (&xv)[S][M], const SkinnyArgs& a, int tile,
                                          int prefetch, int k0, int lane, int wid, int nw,
                                          float (*s_part)[EPI ? 2 * kR * M : kR * M]) {
  constexpr int RR = EPI ? 2 * kR : kR;
  float acc[RR * M];
#pragma unroll
  for (int i = 0; i < RR * M; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float c = acc[r * M + m];
        c = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[s][r].x), as_bf2(xv[s][m].x), c, false);
        c = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[s][r].y), as_bf2(xv[s][m].y), c, false);
        c = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[s][r].z), as_bf2(xv[s][m].z), c, false);
        c = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(wv[s][r].w), as_bf2(xv[s][m].w), c, false);
        acc[r * M + m] = c;
      }
  if (PF == 1 || (PF == 2 && prefetch < a.ntiles)) load_tile<S, RR>(wv, a, prefetch, k0);
  wave_sums_to<RR * M>(acc, lane, s_part[wid]);
  // one barrier per tile: the LDS buffer written here is read back after it,
  // and written again only two tiles later, after the next tile's barrier
  __syncthreads();
  const int t = threadIdx.x;
  if (t < kR * M) {
    const int r = t / M, m = t % M;
    float y = 0.0f;
    for (int w = 0; w < nw; ++w) y += s_part[w][r * M + m];
    uint16_t out;
    if (EPI) {
      float u = 0.0f;
      for (int w = 0; w < nw; ++w) u += s_part[w][(kR + r) * M + m];
      const float g = bfv(to_bf16(y));
      const uint16_t sl = to_bf16(g / (1.0f + __expf(-g)));
      out = to_bf16(bfv(sl) * bfv(to_bf16(u)));
    } else {
      out = to_bf16(y);
    }
    a.Y[(int64_t)m * a.ys + tile * kR + r] = out;
  }
}

template <int M, int S, int EPI, bool NORM, bool RES>
__global__ __launch_bounds__(kMaxWaves * 64) void k_skinny(SkinnyArgs a) {
  // the argument block's two 64-byte lines (the second also holds the hidden
  // launch arguments) requested together, not one miss each as fields are
  // first used: small calls are latency-bound
  asm volatile("" ::"s"(a.X), "s"(a.rs_in));
  constexpr int RR = EPI ? 2 * kR : kR;  // weight rows of a tile
  __shared__ float s_part[2][kMaxWaves][RR * M];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int k0 = wid * S * kStep + 8 * lane;
  int tile = blockIdx.x;
  if (tile >= a.ntiles) return;  // the host launches at most ntiles workgroups
  const int step = gridDim.x;

  uint4 xr[S][M], rr[S][M], nr[S];
  issue_activations<M, S, NORM, RES>(xr, rr, nr, a, k0);
  uint4 wa[S][RR];
  load_tile<S, RR>(wa, a, tile, k0);
  uint4 xv[S][M];
  // two register buffers of weights unless a tile is large (SwiGLU tiles over
  // more than one K step), where the second buffer would spill
  constexpr bool kDouble = RR * S <= 12;
  if constexpr (!kDouble) {
    // one buffer: the next tile's loads overlap the current tile's reduction
    finish_activations<M, S, NORM, RES>(xv, xr, rr, nr, a, k0, lane, wid, nw);
    for (int buf = 0;; buf ^= 1) {
      tile_step<M, S, EPI, 2>(wa, xv, a, tile, tile + step, k0, lane, wid, nw, s_part[buf]);
      tile += step;
      if (tile >= a.ntiles) break;
    }
  } else {
    // Two weight tiles in flight from the start: the activations first (the
    // prologue waits for them only), then the workgroup's first two tiles.
    // Tiles alternate between the buffers wa / wb, and a buffer is refilled
    // with the tile two ahead as soon as its products are done. Every load up
    // to the last two tiles is unconditional, so each wait before a tile's
    // products covers that tile's loads only (after a conditional load the
    // compiler has to wait for every outstanding load). A workgroup with a
    // single tile (the host sizes the grid to avoid it on large matrices)
    // loads that tile twice.
    const int T = (a.ntiles - tile + step - 1) / step;  // tiles of this workgroup
    uint4 wb[S][RR];
    load_tile<S, RR>(wb, a, T > 1 ? tile + step : tile, k0);
    finish_activations<M, S, NORM, RES>(xv, xr, rr, nr, a, k0, lane, wid, nw);
    if (T == 1) {
      tile_step<M, S, EPI, 0>(wa, xv, a, tile, 0, k0, lane, wid, nw, s_part[0]);
      return;
    }
    int j = 0;
    for (; j + 3 < T; j += 2, tile += 2 * step) {
      tile_step<M, S, EPI, 1>(wa, xv, a, tile, tile + 2 * step, k0, lane, wid, nw, s_part[0]);
      tile_step<M, S, EPI, 1>(wb, xv, a, tile + step, tile + 3 * step, k0, lane, wid, nw,
                              s_part[1]);
    }
    if (T - j == 3) {
      tile_step<M, S, EPI, 1>(wa, xv, a, tile, tile + 2 * step, k0, lane, wid, nw, s_part[0]);
      tile_step<M, S, EPI, 0>(wb, xv, a, tile + step, 0, k0, lane, wid, nw, s_part[1]);
      tile_step<M, S, EPI, 0>(wa, xv, a, tile + 2 * step, 0, k0, lane, wid, nw, s_part[0]);
    } else {
      tile_step<M, S, EPI, 0>(wa, xv, a, tile, 0, k0, lane, wid, nw, s_part[0]);
      tile_step<M, S, EPI, 0>(wb, xv, a, tile + step, 0, k0, lane, wid, nw, s_part[1]);
    }
  }
}

int g_num_cus[64];  // per device, filled on first use

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!g_num_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    g_num_cus[dev] = n;
  }
  return g_num_cus[dev];
}

template <int M, int S, int EPI, bool NORM, bool RES>
void launch_skinny(const SkinnyArgs& a, int waves, hipStream_t stream) {
  // resident workgroups per CU at this block size (queried once per size)
  static int occ[kMaxWaves + 1];
  if (!occ[waves]) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_skinny<M, S, EPI, NORM, RES>,
                                                     64 * waves, 0) != hipSuccess || n <= 0)
      n = 1;
    occ[waves] = n;
  }
  const int64_t cus = num_cus();
  int64_t grid = cus * occ[waves];
  // double-buffered kernels: at least two tiles per workgroup once the matrix
  // has enough tiles to keep every CU busy with half as many workgroups
  constexpr bool kDouble = (EPI ? 2 * kR : kR) * S <= 12;
  if (kDouble && a.ntiles >= 2 * cus && grid > a.ntiles / 2) grid = a.ntiles / 2;
  // verify-row projections with the RMSNorm prologue: at least 6 tiles per
  // workgroup once the matrix has a CU's worth of them, so that the prologue
  // (activation loads, a barrier, the norm) is paid by fewer workgroups and the
  // double buffer streams behind it (8B qkv, 4 rows: 13.3 -> 12.5 us)
  if (NORM && M >= 2 && a.ntiles >= 6 * cus && grid > a.ntiles / 6) grid = a.ntiles / 6;
  if (grid > a.ntiles) grid = a.ntiles;
  hipLaunchKernelGGL((k_skinny<M, S, EPI, NORM, RES>), dim3((unsigned)grid), dim3(64 * waves), 0,
                     stream, a);
}

template <int S, int EPI, bool NORM, bool RES>
void dispatch_m(int M, const SkinnyArgs& a, int waves, hipStream_t s) {
  switch (M) {
    case 1: launch_skinny<1, S, EPI, NORM, RES>(a, waves, s); break;
    case 2: launch_skinny<2, S, EPI, NORM, RES>(a, waves, s); break;
    case 3: launch_skinny<3, S, EPI, NORM, RES>(a, waves, s); break;
    case 4: launch_skinny<4, S, EPI, NORM, RES>(a, waves, s); break;
    case 5: launch_skinny<5, S, EPI, NORM, RES>(a, waves, s); break;
    case 6: launch_skinny<6, S, EPI, NORM, RES>(a, waves, s); break;
    case 7: launch_skinny<7, S, EPI, NORM, RES>(a, waves, s); break;
    default: launch_skinny<8, S, EPI, NORM, RES>(a, waves, s); break;
  }
}

// waves = the largest divisor of K / 512 that is at most 8; S = steps per wave
void split_k(int K, int& waves, int& S) {
  const int steps = K / kStep;
  waves = steps < kMaxWaves ? steps : kMaxWaves;
  while (steps % waves) --waves;
  S = steps / waves;
}

template <bool NORM, bool RES>
int dispatch(int rows, const SkinnyArgs& a, int epilogue, hipStream_t s) {
  int waves, S;
  split_k(a.K, waves, S);
  if (S > (NORM ? kMaxNormS : kMaxS)) return HS_ERR_UNSUPPORTED;
  if (epilogue == HS_LINEAR_SWIGLU) {
    // gate and up rows double the weight registers: at most 2 steps per wave
    if (S == 1) dispatch_m<1, 1, NORM, RES>(rows, a, waves, s);
    else if (S == 2) dispatch_m<2, 1, NORM, RES>(rows, a, waves, s);
    else return HS_ERR_UNSUPPORTED;
  } else {
    if (S == 1) dispatch_m<1, 0, NORM, RES>(rows, a, waves, s);
    else if (S == 2) dispatch_m<2, 0, NORM, RES>(rows, a, waves, s);
    else if constexpr (!NORM) dispatch_m<3, 0, NORM, RES>(rows, a, waves, s);
  }
  return HS_OK;
}

// checks shared by both entry points; fills the plain fields of `a`
int check_common(const void* x, int64_t x_stride, const void* weight, int rows, int in_features,
                 int out_features, int epilogue, void* out, int64_t out_stride, SkinnyArgs& a) {
  if (!x || !weight || !out) return HS_ERR_INVALID;
  if (rows < 1 || in_features < 1 || out_features < 1) return HS_ERR_INVALID;
  if (epilogue != HS_LINEAR_PLAIN && epilogue != HS_LINEAR_SWIGLU) return HS_ERR_INVALID;
  if (rows > 8 || in_features % kStep) return HS_ERR_UNSUPPORTED;
  const int N = out_features;
  if (N % kR) return HS_ERR_UNSUPPORTED;
  if ((x_stride % 8) || (out_stride < N) || (x_stride < in_features)) return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)x | (uintptr_t)weight) & 15) return HS_ERR_UNSUPPORTED;
  a = SkinnyArgs{};
  a.X = static_cast<const uint16_t*>(x);
  a.xs = x_stride;
  a.W = static_cast<const uint16_t*>(weight);
  a.K = in_features;
  a.F = N;
  a.ntiles = N / kR;
  a.Y = static_cast<uint16_t*>(out);
  a.ys = out_stride;
  return HS_OK;
}

// byte ranges of two row-strided bf16 matrices [rows, cols] intersect
bool overlaps(const void* p, int64_t ps, const void* q, int64_t qs, int rows, int cols) {
  if (!p || !q) return false;
  const uintptr_t a0 = (uintptr_t)p, a1 = a0 + 2 * ((uint64_t)(rows - 1) * ps + cols);
  const uintptr_t b0 = (uintptr_t)q, b1 = b0 + 2 * ((uint64_t)(rows - 1) * qs + cols);
  return a0 < b1 && b0 < a1;
}

}  // namespace
}  // namespace hs

using namespace hs;

extern "C" {

int hs_linear(const void* x, int64_t x_stride, const void* weight, int rows, int in_features,
              int out_features, int epilogue, void* out, int64_t out_stride, void* stream) {
  SkinnyArgs a;
  int rc = check_common(x, x_stride, weight, rows, in_features, out_features, epilogue, out,
                        out_stride, a);
  if (rc != HS_OK) return rc;
  rc = dispatch<false, false>(rows, a, epilogue, reinterpret_cast<hipStream_t>(stream));
  if (rc != HS_OK) return rc;
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_linear_rmsnorm(const void* x, int64_t x_stride, const void* residual_in,
                      int64_t residual_in_stride, void* residual_out, int64_t residual_out_stride,
                      const void* norm_weight, float eps, const void* weight, int rows,
                      int in_features, int out_features, int epilogue, void* out,
                      int64_t out_stride, void* stream) {
  SkinnyArgs a;
  int rc = check_common(x, x_stride, weight, rows, in_features, out_features, epilogue, out,
                        out_stride, a);
  if (rc != HS_OK) return rc;
  if (!norm_weight || !(eps >= 0.0f)) return HS_ERR_INVALID;
  const int K = in_features;
  if (residual_in && ((residual_in_stride % 8) || residual_in_stride < K)) return HS_ERR_UNSUPPORTED;
  if (residual_out && ((residual_out_stride % 8) || residual_out_stride < K))
    return HS_ERR_UNSUPPORTED;
  if (((uintptr_t)residual_in | (uintptr_t)residual_out | (uintptr_t)norm_weight) & 15)
    return HS_ERR_UNSUPPORTED;
  // workgroup 0 writes residual_out while the others still read x / residual_in
  if (overlaps(residual_out, residual_out_stride, x, x_stride, rows, K) ||
      overlaps(residual_out, residual_out_stride, residual_in, residual_in_stride, rows, K))
    return HS_ERR_INVALID;
  a.Rin = static_cast<const uint16_t*>(residual_in);
  a.rs_in = residual_in_stride;
  a.Rout = static_cast<uint16_t*>(residual_out);
  a.rs_out = residual_out_stride;
  a.NW = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  rc = residual_in ? dispatch<true, true>(rows, a, epilogue, s)
                   : dispatch<true, false>(rows, a, epilogue, s);
  if (rc != HS_OK) return rc;
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

}  // extern "C"
