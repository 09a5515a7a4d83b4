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

// Atomic ticket: returns true in every lane of the wave that took the last
// ticket of `expected`. Release/acquire fences make the partials written by
// the other workgroups visible across XCDs.
__device__ __forceinline__ bool last_ticket(uint32_t* ctr, uint32_t expected, int lane) {
  __threadfence();
  uint32_t old = 0;
  if (lane == 0) old = atomicAdd(ctr, 1u);
  old = __shfl(old, 0, 64);
  if (old != expected - 1u) return false;
  __threadfence();
  if (lane == 0) *ctr = 0u;  // leave the counter zeroed for the next call
  return true;
}

// ---------------------------------------------------------------------------
// row statistics: chunk max + exact exp-sum, row fold, optional decision
// ---------------------------------------------------------------------------
template <typename T>
__device__ void fold_row(const Problem& P, const Work& W, int row, int lane, float* row_stats) {
  const ChunkStat* cp = W.part + (int64_t)row * P.nchunk;
  float M = -INFINITY;
  for (int c = lane; c < P.nchunk; c += kWave) M = fmaxf(M, cp[c].m);
  M = wave_max_f32(M);
  uint64_t S = 0;
  for (int c = lane; c < P.nchunk; c += kWave) {
    float ec = hs_f32_rz_of_u64(cp[c].e) * kTwoM44;
    S += hs_fx40(ec * hs_exp(cp[c].m - M));
  }
  S = wave_sum_u64(S);
  if (lane == 0) {
    RowDesc d;
    d.m = M;
    d.s = hs_f32_rz_of_u64(S) * kTwoM40;
    d.tkey = 0u;
    d.tidx = 0x7fffffff;
    d.all = 1;
    d.token = -1;
    d.s_full = d.s;
    d.pad = 0;
    W.desc[row] = d;
    if (row_stats) {
      row_stats[2 * (int64_t)row] = d.m;
      row_stats[2 * (int64_t)row + 1] = d.s;
    }
  }
}

// One wave decides how many drafts of `unit` are accepted
// (model_runner.py:403-409) and where the bonus/residual draw happens
// (:410-426).
template <typename T>
__device__ void decide_unit(const Problem& P, const AcceptArgs& A, const Work& W, int unit,
                            int lane) {
  const int g = A.gamma;
  bool rej = false;
  if (lane < g) {
    const int64_t d = A.dtok[(int64_t)unit * g + lane];
    const int64_t row = (int64_t)unit * (g + 1) + lane;
    float pt = 0.0f, pd = 0.0f;
    if (d >= 0 && d < P.V) {
      const T* rp = reinterpret_cast<const T*>(P.logits) + row * P.row_stride;
      float x = hs_div_t(ld1<T>(rp + d), P.temps[unit]);
      RowDesc D = W.desc[row];
      pt = desc_prob(D, x, d);
      pd = A.q[((int64_t)unit * g + lane) * A.q_stride + d];
    }
    float ratio = pt / fmaxf(pd, 1e-10f);
    float a = fminf(ratio, 1.0f);
    rej = !(A.u_acc[(int64_t)unit * g + lane] < a);
  }
  uint64_t mask = __ballot(rej);
  int r = mask ? (__ffsll((long long)mask) - 1) : g;
  if (lane == 0) {
    SeqState s;
    s.kind = (r < g) ? kKindResidual : kKindBonus;
    s.row = unit * (g + 1) + r;
    s.qrow = unit * g + r;
    s.nacc = r;
    s.pad[0] = s.pad[1] = s.pad[2] = s.pad[3] = 0;
    W.st[unit] = s;
  }
}

}  // namespace hs
