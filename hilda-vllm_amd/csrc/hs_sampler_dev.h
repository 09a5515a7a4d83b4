// Device helpers shared by the sampler kernels (spec_accept.hip, spec_filter.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hs_device.h"
#include "hs_sampler.h"

namespace hs {

// ---------------------------------------------------------------------------
// loads
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float ld1(const T* p);
template <>
__device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld1<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// Loads the 8 consecutive elements [idx, idx+8) of a row as floats; elements
// at or beyond V read as 0 (callers mask them by index).
template <typename T>
__device__ __forceinline__ void load8(const T* __restrict__ rp, int64_t idx, int V, bool vec_ok,
                                      float (&v)[8]) {
  if (vec_ok && idx + 8 <= V) {
    if constexpr (sizeof(T) == 2) {
      uint4 r = *reinterpret_cast<const uint4*>(rp + idx);
      v[0] = u2f(r.x << 16); v[1] = u2f(r.x & 0xffff0000u);
      v[2] = u2f(r.y << 16); v[3] = u2f(r.y & 0xffff0000u);
      v[4] = u2f(r.z << 16); v[5] = u2f(r.z & 0xffff0000u);
      v[6] = u2f(r.w << 16); v[7] = u2f(r.w & 0xffff0000u);
    } else {
      float4 a = *reinterpret_cast<const float4*>(rp + idx);
      float4 b = *reinterpret_cast<const float4*>(rp + idx + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (idx + k < V) ? ld1<T>(rp + idx + k) : 0.0f;
  }
}

__device__ __forceinline__ void load8_f32(const float* __restrict__ rp, int64_t idx, int V,
                                          bool vec_ok, float (&v)[8]) {
  load8<float>(rp, idx, V, vec_ok, v);
}

__device__ __forceinline__ void store8_f32(float* __restrict__ rp, int64_t idx, int V, bool vec_ok,
                                           const float (&v)[8]) {
  if (vec_ok && idx + 8 <= V) {
    *reinterpret_cast<float4*>(rp + idx) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(rp + idx + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (idx + k < V) rp[idx + k] = v[k];
  }
}

// element index of (group g, lane, k) inside a chunk starting at c0
__device__ __forceinline__ int64_t elem_idx(int64_t c0, int g, int lane, int k) {
  return c0 + (int64_t)g * (kWave * kGroupElems) + lane * kGroupElems + k;
}

__device__ __forceinline__ bool desc_keep(const RowDesc& d, uint32_t key, int64_t idx) {
  return d.all || key > d.tkey || (key == d.tkey && idx <= (int64_t)d.tidx);
}

// Probability of element x (already divided by T) under a row descriptor.
__device__ __forceinline__ float desc_prob(const RowDesc& d, float x, int64_t idx) {
  return desc_keep(d, hs_key(x), idx) ? hs_exp(x - d.m) / d.s : 0.0f;
}

// Element index of (thread tid, element k) of chunk c: each of the 256
// threads owns 8 consecutive elements, so thread order is element order.
__device__ __forceinline__ int64_t chunk_elem(int c, int tid, int k) {
  return (int64_t)c * kChunk + (int64_t)tid * kGroupElems + k;
}

// Folds the chunk partials of one row into its max M and normaliser
//   S = f32rz(sum_c floor(2^40 * f32rz(E_c) 2^-44 * exp(m_c - M))) 2^-40
// (one wave; every lane returns the same descriptor, kept set = whole row).
__device__ __forceinline__ RowDesc fold_row_desc(const Problem& P, const Work& W, int row,
                                                 int lane) {
  const ChunkStat* cp = W.part + (int64_t)row * P.nchunk;
  float M = -INFINITY;
  for (int c = lane; c < P.nchunk; c += kWave) M = fmaxf(M, cp[c].m);
  M = wave_max_f32(M);
  uint64_t S = 0;
  for (int c = lane; c < P.nchunk; c += kWave) {
    const float ec = hs_f32_rz_of_u64(cp[c].e) * kTwoM44;
    S += hs_fx40(ec * hs_exp(cp[c].m - M));
  }
  S = wave_sum_u64(S);
  RowDesc d;
  d.m = M;
  d.s = hs_f32_rz_of_u64(S) * kTwoM40;
  d.tkey = 0u;
  d.tidx = 0x7fffffff;
  d.all = 1;
  d.token = -1;
  d.s_full = d.s;
  d.pad = 0;
  return d;
}

}  // namespace hs
