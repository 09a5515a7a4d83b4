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

// One wave per chunk: lane `lane` holds elements c0 + 512 s + 8 lane + k
// (group s = 0..3, k = 0..7), each group one coalesced 1 KB (bf16) or 2 KB
// (f32) wave load, kept as raw 16-byte words until used. For 16-byte aligned
// rows with V % 8 == 0 a group is wholly inside the row or wholly past its
// end; past the end, and for every group when `use` is false, the lane reads
// the row's first 16 bytes (one cache line for the wave) and the values are
// not used. No branch, so all of a chunk's loads are in flight together.
constexpr int kLaneChunkGroups = kChunk / (kWave * kGroupElems);  // 4

template <typename T>
struct LaneChunk {
  static constexpr int kWords = kLaneChunkGroups * kGroupElems * (int)sizeof(T) / 16;
  uint4 w[kWords];
};

__device__ __forceinline__ int64_t lane_chunk_idx(int64_t c0, int s, int lane, int k) {
  return c0 + (int64_t)s * (kWave * kGroupElems) + lane * kGroupElems + k;
}

template <typename T>
__device__ __forceinline__ void lane_chunk_load(const T* __restrict__ rp, int64_t c0, int V,
                                                int lane, bool use, LaneChunk<T>& r) {
#pragma unroll
  for (int s = 0; s < kLaneChunkGroups; ++s) {
    const int64_t i = lane_chunk_idx(c0, s, lane, 0);
    const T* p = rp + ((use && i < V) ? i : 0);
    if constexpr (sizeof(T) == 2) {
      r.w[s] = *reinterpret_cast<const uint4*>(p);
    } else {
      r.w[2 * s] = *reinterpret_cast<const uint4*>(p);
      r.w[2 * s + 1] = *reinterpret_cast<const uint4*>(p + 4);
    }
  }
}

__device__ __forceinline__ uint32_t u4_word(const uint4& u, int i) {
  return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w;
}

// element (s, k) of a lane's chunk as float (s, k compile-time after unrolling)
template <typename T>
__device__ __forceinline__ float lane_chunk_val(const LaneChunk<T>& r, int s, int k) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = u4_word(r.w[s], k >> 1);
    return (k & 1) ? u2f(w & 0xffff0000u) : u2f(w << 16);
  } else {
    return u2f(u4_word(r.w[2 * s + (k >> 2)], k & 3));
  }
}

// True when every value held in the lane's chunk words has |x| in
// [2^-96, 2^60], the numerator range in which hs_div_rcp's corrected product
// is exact (zeros, subnormals, infinities and NaN fail). On the bit patterns,
// with lo/hi the patterns of 2^-96 and 2^60: 2|x| - 2 lo, taken modulo 2^16
// (bf16, both halves of a word at once) or 2^32 (f32), is at most 2 (hi - lo)
// exactly for |x| in range; doubling drops the sign bit and values below lo
// wrap above the bound.
template <typename T>
__device__ __forceinline__ bool lane_chunk_rcp_ok(const LaneChunk<T>& r) {
  if constexpr (sizeof(T) == 2) {
    using u16x2 = unsigned short __attribute__((ext_vector_type(2)));
    const u16x2 two = {2, 2}, off = {0xE100, 0xE100};  // -2 * 0x0F80 mod 2^16
    u16x2 acc = {0, 0};
#pragma unroll
    for (int i = 0; i < LaneChunk<T>::kWords; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u16x2 v = __builtin_bit_cast(u16x2, u4_word(r.w[i], j));
        acc = __builtin_elementwise_max(acc, v * two + off);
      }
    return acc.x <= 0x9C00 && acc.y <= 0x9C00;  // 2 * (0x5D80 - 0x0F80)
  } else {
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < LaneChunk<T>::kWords; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t t = (u4_word(r.w[i], j) << 1) + 0xE1000000u;  // -2 * 0x0F800000
        acc = t > acc ? t : acc;
      }
    return acc <= 0x9C000000u;  // 2 * (0x5D800000 - 0x0F800000)
  }
}

// x / T (hs_div_temp) for every element of a lane's chunk, with one
// wave-uniform choice per chunk instead of per element: the identity for
// T = 1; the corrected product when hs_rcp_ok(T) and every numerator of the
// wave's chunk is in its exact range; hs_div_temp per element otherwise.
// T must be the same in every lane.
template <typename T>
__device__ __forceinline__ void lane_chunk_div_temp(const LaneChunk<T>& r, float Tt,
                                                    float (&x)[kLaneChunkGroups][kGroupElems]) {
  const float rT = 1.0f / Tt;
  const bool fast = hs_rcp_ok(Tt);
  if (Tt == 1.0f) {
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s)
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k) x[s][k] = lane_chunk_val<T>(r, s, k);
  } else if (fast && __builtin_amdgcn_ballot_w64(!lane_chunk_rcp_ok<T>(r)) == 0) {
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s)
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k)
        x[s][k] = hs_div_rcp_in_range(lane_chunk_val<T>(r, s, k), Tt, rT);
  } else {
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s)
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k)
        x[s][k] = hs_div_temp(lane_chunk_val<T>(r, s, k), Tt, rT, fast);
  }
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
