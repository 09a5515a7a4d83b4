// Fused acceptance sampler and row sampler for gfx950.
//
// Replaces the rejection-sampling loop of ModelRunner.run_verify
// (mini_vllm/engine/model_runner.py:387-428) and the sampling ops of
// Sampler.forward (mini_vllm/layers/sampler.py:13-49).
//
// One hs_spec_accept call (B sequences, gamma drafts, V vocab) is a short
// chain of launches with no communication between workgroups of a launch
// (on gfx950 a cross-XCD release/acquire costs an L2 write-back plus an L2
// invalidate per workgroup; kernel boundaries are cheaper):
//   1. k_chunk_stats   one 256-thread workgroup per 2048-element chunk of a
//      target row: chunk max m_c and E_c = sum floor(2^44 exp(x_i - m_c)).
//      Target logits are read from HBM exactly once here. For 16-byte
//      aligned rows with V % 8 == 0, k_chunk_stats_w does the same with one
//      wave per chunk.
//   2. (filtered mode) k_row_filter, spec_filter.hip: top-k / top-p kept set
//      and normaliser per row.
//   3. k_sample_part   grid (splits, B). Every workgroup first recomputes the
//      decision of its sequence from the chunk partials (a few hundred
//      values, deterministic, so all workgroups agree without talking), then
//      streams its share of the resample row (target row r, plus draft row r
//      for a residual) and writes exact per-chunk weight sums.
//   4. k_sample_final  one workgroup per sequence: locates the chunk holding
//      the inverse-CDF point and rescans that one chunk to find the token.
// Greedy mode: k_chunk_argmax then k_greedy_final.
// Reference-mode calls small enough for one workgroup per CU run instead as
// one launch, k_accept_small (spec_accept_small.hip), with the same arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "hs_bookkeeping.h"
#include "hs_device.h"
#include "hs_sampler.h"
#include "hs_sampler_dev.h"
#include "../../include/hilda_spec.h"

namespace hs {

constexpr int kT = kChunkThreads;  // 256 threads, 8 elements each, per chunk

// ---------------------------------------------------------------------------
// 1. chunk statistics
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kT) void k_chunk_stats(Problem P, Work W) {
  __shared__ float s_m[kT / kWave];
  __shared__ uint64_t s_e[kT / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t items = (int64_t)P.units * P.rows_per_unit * P.nchunk;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int row = (int)(it / P.nchunk);
    const int c = (int)(it % P.nchunk);
    const int unit = row / P.rows_per_unit;
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
    const int64_t i0 = chunk_elem(c, tid, 0);
    float x[8];
    load8<T>(rp, i0, P.V, vec_ok, x);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[k] = hs_div_temp(x[k], Tt, rT, fast);
      if (i0 + k < P.V) m = fmaxf(m, x[k]);
    }
    m = wave_max_f32(m);
    if (lane == 0) s_m[wid] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    uint32_t hi = 0, lo = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + k < P.V) hs_fx44_split(hs_exp(x[k] - m), hi, lo);
    uint64_t e = wave_sum_u64(hs_join44(hi, lo));
    if (lane == 0) s_e[wid] = e;
    __syncthreads();
    if (tid == 0) {
      ChunkStat cs;
      cs.m = m;
      cs.pad = 0;
      cs.e = s_e[0] + s_e[1] + s_e[2] + s_e[3];
      W.part[it] = cs;
    }
    if (P.filtered && c == 0) {
      // the filter passes accumulate into these (kernel order: this launch first)
      const int64_t hb = (int64_t)row * kCB + tid;
      W.h1m[hb] = 0ull;
      W.h1e[hb] = 0ull;
      W.h1c[hb] = 0u;
      W.h2m[hb] = 0ull;
      W.h2e[hb] = 0ull;
      W.h2c[hb] = 0u;
      if (tid == 0) W.filt[row].ncand = 0;
      if (tid == 0 && row == 0) W.flist[0] = W.flist[1] = 0;
    }
  }
}

// The same statistics with one wave per chunk (aligned rows, V % 8 == 0):
// no barrier; waves stride over the items.
template <typename T>
__device__ __forceinline__ void chunk_stats_wave(const Problem& P, const Work& W, int64_t it,
                                                 const LaneChunk<T>& r, int lane) {
  const int row = (int)(it / P.nchunk);
  const int c = (int)(it % P.nchunk);
  const int unit = row / P.rows_per_unit;
  const int64_t c0 = (int64_t)c * kChunk;
  float x[kLaneChunkGroups][kGroupElems];
  lane_chunk_div_temp<T>(r, P.temps[unit], x);
  // every group of a chunk that ends inside the row is in it (wave-uniform)
  const bool full = c0 + kChunk <= P.V;
  float m = -INFINITY;
  uint32_t hi = 0, lo = 0;
  if (full) {
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s)
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k) m = fmaxf(m, x[s][k]);
    m = wave_max_f32(m);
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s)
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k) {
        hs_fx44_acc(hs_exp_2p20(x[s][k] - m), hi, lo);
        // the running sums are taken every 4 elements: left alone, the
        // compiler regroups the 32 integer additions into one tree at the end
        // and keeps every element's two parts live (spills past 64 VGPRs)
        if (k % 4 == 3) asm volatile("" : "+v"(hi), "+v"(lo));
      }
  } else {
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s) {
      const bool in = lane_chunk_idx(c0, s, lane, 0) < P.V;
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k)
        if (in) m = fmaxf(m, x[s][k]);
    }
    m = wave_max_f32(m);
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s) {
      const bool in = lane_chunk_idx(c0, s, lane, 0) < P.V;
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k)
        if (in) hs_fx44_acc(hs_exp_2p20(x[s][k] - m), hi, lo);
    }
  }
  const uint64_t e = wave_sum_u64(hs_join44(hi, lo));
  if (lane == 0) {
    ChunkStat cs;
    cs.m = m;
    cs.pad = 0;
    cs.e = e;
    W.part[it] = cs;
  }
}

// The filter passes accumulate into these (kernel order: this launch first);
// the wave of a row's first chunk clears them, before it loads the chunk (no
// statistics registers are live then).
__device__ __forceinline__ void clear_filter_row(const Problem& P, const Work& W, int64_t it,
                                                 int lane) {
  const int row = (int)(it / P.nchunk);
  if (!P.filtered || it - (int64_t)row * P.nchunk != 0) return;
  for (int i = lane; i < kCB; i += kWave) {
    const int64_t hb = (int64_t)row * kCB + i;
    W.h1m[hb] = 0ull;
    W.h1e[hb] = 0ull;
    W.h1c[hb] = 0u;
    W.h2m[hb] = 0ull;
    W.h2e[hb] = 0ull;
    W.h2c[hb] = 0u;
  }
  if (lane == 0) W.filt[row].ncand = 0;
  if (lane == 0 && row == 0) W.flist[0] = W.flist[1] = 0;
}

template <typename T>
__global__ __launch_bounds__(kT) void k_chunk_stats_w(Problem P, Work W) {
  const int lane = threadIdx.x & 63;
  // the wave index is uniform across the wave: kept in a scalar register, the
  // chunk, row and temperature are too, and the branches on them are uniform
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t items = (int64_t)P.units * P.rows_per_unit * P.nchunk;
  const int64_t stride = (int64_t)gridDim.x * (kT / kWave);
  int64_t it = (int64_t)blockIdx.x * (kT / kWave) + wid;
  if (it >= items) return;
  const T* base = reinterpret_cast<const T*>(P.logits);
  auto load = [&](int64_t item, LaneChunk<T>& r) {
    const bool use = item < items;
    const int64_t row = use ? item / P.nchunk : 0;
    const int64_t c0 = use ? (item % P.nchunk) * (int64_t)kChunk : 0;
    lane_chunk_load<T>(base + row * P.row_stride, c0, P.V, lane, use, r);
  };
  // One chunk in registers at a time (60 VGPRs, 8 waves per SIMD): the other
  // resident waves hide a wave's load latency, which measured faster than
  // holding the next chunk in flight (80 VGPRs, 6 waves per SIMD).
  for (; it < items; it += stride) {
    clear_filter_row(P, W, it, lane);
    LaneChunk<T> a;
    load(it, a);
    chunk_stats_wave<T>(P, W, it, a, lane);
  }
}

// greedy: argmax over raw logits, lowest index on ties
template <typename T>
__global__ __launch_bounds__(kT) void k_chunk_argmax(Problem P, Work W) {
  __shared__ uint64_t s_b[kT / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t items = (int64_t)P.units * P.rows_per_unit * P.nchunk;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int row = (int)(it / P.nchunk);
    const int c = (int)(it % P.nchunk);
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
    const int64_t i0 = chunk_elem(c, tid, 0);
    float v[8];
    load8<T>(rp, i0, P.V, vec_ok, v);
    uint64_t best = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = i0 + k;
      if (i < P.V) {
        uint64_t pk = ((uint64_t)hs_key(v[k]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        best = pk > best ? pk : best;
      }
    }
    best = wave_max_u64(best);
    if (lane == 0) s_b[wid] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t b = s_b[0];
      for (int w = 1; w < kT / kWave; ++w) b = s_b[w] > b ? s_b[w] : b;
      ChunkStat cs;
      cs.m = 0.0f;
      cs.pad = 0;
      cs.e = b;
      W.part[it] = cs;
    }
    __syncthreads();
  }
}

// one wave per unit: per-row argmax, then the greedy acceptance
__global__ __launch_bounds__(kWave) void k_greedy_final(Problem P, AcceptArgs A, Work W,
                                                        int64_t* tokens_out) {
  const int unit = blockIdx.x;
  const int lane = threadIdx.x;
  const int R = P.rows_per_unit;
  __shared__ int s_tok[kMaxGamma + 1];
  for (int j = 0; j < R; ++j) {
    const ChunkStat* cp = W.part + (int64_t)(unit * R + j) * P.nchunk;
    uint64_t best = 0;
    for (int c = lane; c < P.nchunk; c += kWave) best = cp[c].e > best ? cp[c].e : best;
    best = wave_max_u64(best);
    if (lane == 0) s_tok[j] = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
  }
  __syncthreads();
  if (!A.tok_out) {  // row sampler: one row per unit
    if (lane == 0) tokens_out[unit] = s_tok[0];
    return;
  }
  const int g = A.gamma;
  bool rej = false;
  if (lane < g) rej = (A.dtok[(int64_t)unit * g + lane] != (int64_t)s_tok[lane]);
  const uint64_t mask = __ballot(rej);
  const int r = mask ? (__ffsll((long long)mask) - 1) : g;
  if (lane <= g) {
    int64_t v;
    if (lane < r) v = A.dtok[(int64_t)unit * g + lane];
    else if (lane == r) v = s_tok[r];
    else v = -1;
    A.tok_out[(int64_t)unit * (g + 1) + lane] = v;
  }
  if (lane == 0) {
    A.nacc_out[unit] = r;
    A.len_out[unit] = r + 1;
  }
}

// ---------------------------------------------------------------------------
// 3. decision + resample partial sums
// ---------------------------------------------------------------------------
// Decision of one unit from row descriptors held in LDS (one wave).
template <typename T>
__device__ void decide_from(const Problem& P, const AcceptArgs& A, const RowDesc* sd, int unit,
                            int lane, SeqState* out) {
  const int g = A.gamma;
  bool rej = false;
  if (lane < g) {
    const int64_t d = A.dtok[(int64_t)unit * g + lane];
    float pt = 0.0f, pd = 0.0f;
    if (d >= 0 && d < P.V) {
      const int64_t row = (int64_t)unit * (g + 1) + lane;
      const T* rp = reinterpret_cast<const T*>(P.logits) + row * P.row_stride;
      const float x = hs_div_t(ld1<T>(rp + d), P.temps[unit]);
      pt = desc_prob(sd[lane], x, d);
      pd = A.q[((int64_t)unit * g + lane) * A.q_stride + d];
    }
    const float ratio = pt / fmaxf(pd, 1e-10f);
    const float a = fminf(ratio, 1.0f);
    rej = !(A.u_acc[(int64_t)unit * g + lane] < a);
  }
  const uint64_t mask = __ballot(rej);
  const int r = mask ? (__ffsll((long long)mask) - 1) : g;
  if (lane == 0) {
    out->kind = (r < g) ? kKindResidual : kKindBonus;
    out->row = unit * (g + 1) + r;
    out->qrow = unit * g + r;
    out->nacc = r;
  }
}

// Start of k_sample_part: the unit's row
// descriptors (from the filter kernel, or folded here from the chunk
// statistics), the decision, and the unit's bookkeeping writes by split 0.
// Every workgroup of the unit computes the same values.
template <typename T>
__device__ __forceinline__ SeqState part_prologue(const Problem& P, const AcceptArgs& A,
                                                  const Work& W, const SampleOut& O,
                                                  int desc_ready, int unit, int split,
                                                  RowDesc* s_desc, SeqState* s_st) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int R = P.rows_per_unit;
  const bool spec = (A.tok_out != nullptr);
  if (desc_ready) {
    for (int j = tid; j < R; j += kT) s_desc[j] = W.desc[(int64_t)unit * R + j];
  } else {
    for (int j = wid; j < R; j += kT / kWave) {
      RowDesc d = fold_row_desc(P, W, unit * R + j, lane);
      if (lane == 0) s_desc[j] = d;
    }
  }
  __syncthreads();
  if (wid == 0) {
    if (spec) {
      decide_from<T>(P, A, s_desc, unit, lane, s_st);
    } else if (lane == 0) {
      s_st->kind = kKindPlain;
      s_st->row = unit;
      s_st->qrow = -1;
      s_st->nacc = 0;
    }
  }
  __syncthreads();
  const SeqState st = *s_st;
  if (split == 0 && tid == 0) W.st[unit] = st;
  if (split == 0 && O.row_stats && tid < R) {
    const int64_t row = (int64_t)unit * R + tid;
    O.row_stats[2 * row] = s_desc[tid].m;
    O.row_stats[2 * row + 1] = s_desc[tid].s;
  }
  if (split == 0 && !desc_ready && tid < R) W.desc[(int64_t)unit * R + tid] = s_desc[tid];
  return st;
}

template <typename T>
__global__ __launch_bounds__(kT) void k_sample_part(Problem P, AcceptArgs A, Work W, SampleOut O,
                                                    int mode, int desc_ready) {
  __shared__ RowDesc s_desc[kMaxGamma + 1];
  __shared__ SeqState s_st;
  __shared__ uint64_t s_w[kT / kWave], s_p[kT / kWave];
  const int unit = blockIdx.y;
  const int split = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int R = P.rows_per_unit;
  (void)mode;
  const SeqState st = part_prologue<T>(P, A, W, O, desc_ready, unit, split, s_desc, &s_st);

  const int row = st.row;
  const bool residual = (st.kind == kKindResidual);
  const RowDesc D = s_desc[row - unit * R];
  const float Tt = P.temps[unit];
  const float rT = 1.0f / Tt;
  const bool fastT = hs_rcp_ok(Tt);
  const float rS = 1.0f / D.s;
  const bool fastS = hs_rcp_ok(D.s);
  const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
  const float* qp = residual ? A.q + (int64_t)st.qrow * A.q_stride : nullptr;
  const bool q_vec = residual && ((reinterpret_cast<uintptr_t>(qp) & 15u) == 0);
  float* pout = O.probs ? O.probs + (int64_t)row * O.probs_stride : nullptr;
  const bool p_vec = pout && ((reinterpret_cast<uintptr_t>(pout) & 15u) == 0);
  const bool masked = (O.out_kind == 1);
  // out_kind 2: the row's unfiltered probabilities, exp(x - m) / s_full over
  // every element (m, the row maximum, is always kept), beside the filtered draw
  const bool full = (O.out_kind == 2);
  const float rSf = 1.0f / D.s_full;
  const bool fastSf = hs_rcp_ok(D.s_full);
  const int c_begin = (int)((int64_t)split * P.nchunk / P.nsplit);
  const int c_end = (int)((int64_t)(split + 1) * P.nchunk / P.nsplit);

  for (int c = c_begin; c < c_end; ++c) {
    const int64_t i0 = chunk_elem(c, tid, 0);
    float v[8], q[8], pr[8];
    load8<T>(rp, i0, P.V, vec_ok, v);
    if (residual) load8_f32(qp, i0, P.V, q_vec, q);
    uint32_t whi = 0, wlo = 0, phi = 0, plo = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = i0 + k;
      float p = 0.0f, xm = -INFINITY, pf = 0.0f;
      if (i < P.V) {
        const float x = hs_div_temp(v[k], Tt, rT, fastT);
        const bool kept = desc_keep(D, hs_key(x), i);
        if (kept || full) {
          const float e = hs_exp(x - D.m);
          if (kept) {
            p = fastS ? hs_div_rcp(e, D.s, rS) : e / D.s;
            xm = x;
          }
          if (full) pf = fastSf ? hs_div_rcp(e, D.s_full, rSf) : e / D.s_full;
        }
      }
      pr[k] = masked ? xm : (full ? pf : p);
      hs_fx44_split(p, phi, plo);
      if (residual) hs_fx44_split(fmaxf(p - q[k], 0.0f), whi, wlo);
    }
    if (pout) store8_f32(pout, i0, P.V, p_vec, pr);
    if (O.sample) {
      const uint64_t sw = wave_sum_u64(hs_join44(whi, wlo));
      const uint64_t sp = wave_sum_u64(hs_join44(phi, plo));
      if (lane == 0) {
        s_w[wid] = sw;
        s_p[wid] = sp;
      }
      __syncthreads();
      if (tid == 0) {
        SampPart s;
        s.w = s_w[0] + s_w[1] + s_w[2] + s_w[3];
        s.p = s_p[0] + s_p[1] + s_p[2] + s_p[3];
        W.spart[(int64_t)unit * P.nchunk + c] = s;
      }
      __syncthreads();
    }
  }
}

// The same partial sums with one wave per chunk (aligned target and draft
// rows, V % 8 == 0, no probabilities written): a workgroup's four waves take
// the chunks of its range with all of a chunk's loads in flight, and each
// wave writes its chunk's sums itself (no barrier per chunk). kPartWaveChunks
// chunks per wave: the grid then holds about nchunk / 4 workgroups per unit,
// all resident at B = 64, each paying the decision prologue once.
constexpr int kPartWaveChunks = 1;
template <typename T>
__global__ __launch_bounds__(kT) void k_sample_part_w(Problem P, AcceptArgs A, Work W, SampleOut O,
                                                      int desc_ready) {
  __shared__ RowDesc s_desc[kMaxGamma + 1];
  __shared__ SeqState s_st;
  const int unit = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: chunk choices too
  const int R = P.rows_per_unit;
  const SeqState st = part_prologue<T>(P, A, W, O, desc_ready, unit, split, s_desc, &s_st);
  const int row = st.row;
  const bool residual = (st.kind == kKindResidual);
  const RowDesc D = s_desc[row - unit * R];
  const float Tt = P.temps[unit];
  const float rT = 1.0f / Tt;
  const bool fastT = hs_rcp_ok(Tt);
  const float rS = 1.0f / D.s;
  const bool fastS = hs_rcp_ok(D.s);
  const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const float* qp = residual ? A.q + (int64_t)st.qrow * A.q_stride : nullptr;
  constexpr int kPerWg = (kT / kWave) * kPartWaveChunks;
  const int c_end = (split + 1) * kPerWg < P.nchunk ? (split + 1) * kPerWg : P.nchunk;
  for (int c = split * kPerWg + wid; c < c_end; c += kT / kWave) {
    const int64_t c0 = (int64_t)c * kChunk;
    LaneChunk<T> r;
    LaneChunk<float> qr;
    lane_chunk_load<T>(rp, c0, P.V, lane, true, r);
    if (residual) lane_chunk_load<float>(qp, c0, P.V, lane, true, qr);
    uint32_t whi, wlo, phi, plo;
    const bool full = c0 + kChunk <= P.V;  // wave-uniform
    // One pass per element: x = x / T, kept or not (p = 0 outside the kept set
    // and the row), e * 2^20 = hs_exp_2p20(x - m), p * 2^20 from it, and the
    // fixed-point sums of p and max(p - q, 0). p * 2^20 = (e * 2^20) / S by the
    // corrected product equals 2^20 hs_div_rcp(e, S) when e is 0 or in
    // [2^-96, 1] (the quotient is then normal); a chunk where some e lies in
    // (0, 2^-96), or whose S or T rule the corrected product out, is summed
    // with hs_div_temp and hs_div_rcp on e itself. max(p - q, 0) * 2^20 =
    // max(p * 2^20 - q * 2^20, 0): scaling commutes with the rounding of a
    // normal difference, and a subnormal difference is exact.
    auto sums = [&](auto x_of, auto keep_of, auto p20_of) {
      uint32_t umin = 0xffffffffu;  // min over the lane of bits(e * 2^20) - 1 (0 -> max)
      phi = plo = whi = wlo = 0;
#pragma unroll
      for (int g = 0; g < kLaneChunkGroups; ++g) {
        const bool in = full || lane_chunk_idx(c0, g, lane, 0) < P.V;
#pragma unroll
        for (int k = 0; k < kGroupElems; ++k) {
          const float x = x_of(lane_chunk_val<T>(r, g, k));
          const bool kept = in && keep_of(x, lane_chunk_idx(c0, g, lane, k));
          const float ev = hs_exp_2p20(x - D.m);  // computed for every lane: no branch
          const float e20 = kept ? ev : 0.0f;
          const uint32_t u = f2u(e20) - 1u;
          umin = u < umin ? u : umin;
          const float p20 = p20_of(e20);
          hs_fx44_acc(p20, phi, plo);
          if (residual)
            hs_fx44_acc(fmaxf(p20 - lane_chunk_val<float>(qr, g, k) * 1048576.0f, 0.0f), whi,
                        wlo);
          // running sums taken every 4 elements (see chunk_stats_wave), and
          // no more than 4 elements' work interleaved (register pressure)
          if (k % 4 == 3) {
            asm volatile("" : "+v"(phi), "+v"(plo), "+v"(whi), "+v"(wlo), "+v"(umin));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      return __builtin_amdgcn_ballot_w64(umin < f2u(0x1p-76f) - 1u) == 0;
    };
    auto p20_fast = [&](float e20) { return hs_div_rcp_in_range(e20, D.s, rS); };
    auto keep_all = [](float, int64_t) { return true; };
    auto keep_desc = [&](float x, int64_t i) { return desc_keep(D, hs_key(x), i); };
    auto x_same = [](float v) { return v; };
    auto x_rcp = [&](float v) { return hs_div_rcp_in_range(v, Tt, rT); };
    bool ok = false;
    if (fastS) {
      if (Tt == 1.0f)
        ok = D.all ? sums(x_same, keep_all, p20_fast) : sums(x_same, keep_desc, p20_fast);
      else if (fastT && __builtin_amdgcn_ballot_w64(!lane_chunk_rcp_ok<T>(r)) == 0)
        ok = D.all ? sums(x_rcp, keep_all, p20_fast) : sums(x_rcp, keep_desc, p20_fast);
    }
    if (!ok)
      sums([&](float v) { return hs_div_temp(v, Tt, rT, fastT); }, keep_desc, [&](float e20) {
        const float e = e20 * 0x1p-20f;
        return (fastS ? hs_div_rcp(e, D.s, rS) : e / D.s) * 1048576.0f;
      });
    const uint64_t sw = wave_sum_u64(hs_join44(whi, wlo));
    const uint64_t sp = wave_sum_u64(hs_join44(phi, plo));
    if (lane == 0) {
      SampPart sps;
      sps.w = sw;
      sps.p = sp;
      W.spart[(int64_t)unit * P.nchunk + c] = sps;
    }
  }
}

// ---------------------------------------------------------------------------
// 4. final inverse-CDF search
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kT) void k_sample_final(Problem P, AcceptArgs A, Work W,
                                                     SampleOut O) {
  __shared__ uint64_t s_tot[2];
  __shared__ int s_cstar;
  __shared__ uint64_t s_before;
  __shared__ uint64_t s_ws[kT / kWave];
  __shared__ long long s_tok;
  const int unit = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const SeqState st = W.st[unit];
  const int R = P.rows_per_unit;
  const int row = st.row;
  if (st.kind == kKindNone || row < unit * R || row >= (unit + 1) * R) return;
  const bool residual = (st.kind == kKindResidual);
  const SampPart* spp = W.spart + (int64_t)unit * P.nchunk;

  if (wid == 0) {
    uint64_t wt = 0, pt = 0;
    for (int c = lane; c < P.nchunk; c += kWave) {
      wt += spp[c].w;
      pt += spp[c].p;
    }
    wt = wave_sum_u64(wt);
    pt = wave_sum_u64(pt);
    // residual normalisation or fallback to P[r] (model_runner.py:419-424)
    const bool use_res = residual && (hs_f32_of_u64(wt) * kTwoM44 > 1e-10f);
    const uint64_t total = use_res ? wt : pt;
    const uint64_t t = hs_mulshift24(hs_u24(O.uniforms[unit]), total);
    int cstar = -1;
    uint64_t before = 0, running = 0;
    for (int cb = 0; cb < P.nchunk && cstar < 0; cb += kWave) {
      const int c = cb + lane;
      uint64_t val = 0;
      if (c < P.nchunk) val = use_res ? spp[c].w : spp[c].p;
      const uint64_t incl = wave_incl_scan_u64(val, lane);
      const uint64_t m = __ballot(running + incl > t);
      if (m) {
        const int l = __ffsll((long long)m) - 1;
        const uint64_t incl_l = __shfl(incl, l, 64);
        const uint64_t val_l = __shfl(val, l, 64);
        cstar = cb + l;
        before = running + incl_l - val_l;
      } else {
        running += __shfl(incl, 63, 64);
      }
    }
    if (lane == 0) {
      s_tot[0] = use_res ? 1ull : 0ull;
      s_tot[1] = t;
      s_cstar = cstar;
      s_before = before;
      s_tok = -1;
    }
  }
  __syncthreads();
  const int cstar = s_cstar;
  if (cstar >= 0) {
    const bool use_res = s_tot[0] != 0;
    const uint64_t trel = s_tot[1] - s_before;
    const RowDesc D = W.desc[row];
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fastT = hs_rcp_ok(Tt);
    const float rS = 1.0f / D.s;
    const bool fastS = hs_rcp_ok(D.s);
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
    const float* qp = residual ? A.q + (int64_t)st.qrow * A.q_stride : nullptr;
    const bool q_vec = residual && ((reinterpret_cast<uintptr_t>(qp) & 15u) == 0);
    const int64_t i0 = chunk_elem(cstar, tid, 0);
    float v[8], q[8];
    uint64_t w[8];
    load8<T>(rp, i0, P.V, vec_ok, v);
    if (residual) load8_f32(qp, i0, P.V, q_vec, q);
    uint64_t s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = i0 + k;
      float p = 0.0f;
      if (i < P.V) {
        const float x = hs_div_temp(v[k], Tt, rT, fastT);
        if (desc_keep(D, hs_key(x), i)) {
          const float e = hs_exp(x - D.m);
          p = fastS ? hs_div_rcp(e, D.s, rS) : e / D.s;
        }
      }
      const float wt = use_res ? fmaxf(p - q[k], 0.0f) : p;
      uint32_t hi = 0, lo = 0;
      hs_fx44_split(wt, hi, lo);
      w[k] = hs_join44(hi, lo);
      s += w[k];
    }
    // block-wide inclusive scan in element order (thread order)
    const uint64_t incl = wave_incl_scan_u64(s, lane);
    if (lane == 63) s_ws[wid] = incl;
    __syncthreads();
    uint64_t off = 0;
    for (int ww = 0; ww < wid; ++ww) off += s_ws[ww];
    const uint64_t lo_ = off + incl - s;
    if (lo_ <= trel && trel < off + incl) {
      uint64_t acc = lo_;
      for (int k = 0; k < 8; ++k) {
        acc += w[k];
        if (acc > trel) {
          s_tok = (long long)(i0 + k);
          break;
        }
      }
    }
    __syncthreads();
  }
  const int64_t token = (int64_t)s_tok;
  if (A.tok_out) {
    const int gm = A.gamma;
    if (tid <= gm) {
      int64_t v;
      if (tid < st.nacc) v = A.dtok[(int64_t)unit * gm + tid];
      else if (tid == st.nacc) v = token;
      else v = -1;
      A.tok_out[(int64_t)unit * (gm + 1) + tid] = v;
    }
    if (tid == 0) {
      A.nacc_out[unit] = st.nacc;
      A.len_out[unit] = st.nacc + 1;
    }
  }
  if (O.tokens && tid == 0) O.tokens[unit] = token;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

Layout make_layout(int units, int rows, int nchunk) {
  Layout L;
  size_t off = 0;
  L.sync = off; off = align_up(off + sizeof(SmallSync), 256);
  // single-launch acceptance: 3 tagged words per (row, chunk) and 4 per (unit, chunk),
  // in a region of fixed size and place for every shape
  (void)units;
  L.tags = off; off = align_up(off + kSmallTagBytes + kTopkTagBytes, 256);
  L.part = off; off = align_up(off + (size_t)rows * nchunk * sizeof(ChunkStat), 256);
  L.desc = off; off = align_up(off + (size_t)rows * sizeof(RowDesc), 256);
  L.st = off; off = align_up(off + (size_t)units * sizeof(SeqState), 256);
  L.spart = off; off = align_up(off + (size_t)units * nchunk * sizeof(SampPart), 256);
  L.filt = off; off = align_up(off + (size_t)rows * sizeof(FilterScratch), 256);
  L.cand = off; off = align_up(off + (size_t)rows * kCand * sizeof(uint64_t), 256);
  L.h1m = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint64_t), 256);
  L.h1e = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint64_t), 256);
  L.h1c = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint32_t), 256);
  L.h2m = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint64_t), 256);
  L.h2e = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint64_t), 256);
  L.h2c = off; off = align_up(off + (size_t)rows * kCB * sizeof(uint32_t), 256);
  L.flist = off; off = align_up(off + (2 + 2 * (size_t)rows) * sizeof(int32_t), 256);
  L.total = off;
  return L;
}

Work bind_work(void* ws, const Layout& L) {
  char* b = static_cast<char*>(ws);
  Work W;
  W.sync = reinterpret_cast<SmallSync*>(b + L.sync);
  W.tags = reinterpret_cast<uint64_t*>(b + L.tags);
  W.part = reinterpret_cast<ChunkStat*>(b + L.part);
  W.desc = reinterpret_cast<RowDesc*>(b + L.desc);
  W.st = reinterpret_cast<SeqState*>(b + L.st);
  W.spart = reinterpret_cast<SampPart*>(b + L.spart);
  W.filt = reinterpret_cast<FilterScratch*>(b + L.filt);
  W.cand = reinterpret_cast<uint64_t*>(b + L.cand);
  W.h1m = reinterpret_cast<uint64_t*>(b + L.h1m);
  W.h1e = reinterpret_cast<uint64_t*>(b + L.h1e);
  W.h1c = reinterpret_cast<uint32_t*>(b + L.h1c);
  W.h2m = reinterpret_cast<uint64_t*>(b + L.h2m);
  W.h2e = reinterpret_cast<uint64_t*>(b + L.h2e);
  W.h2c = reinterpret_cast<uint32_t*>(b + L.h2c);
  W.flist = reinterpret_cast<int32_t*>(b + L.flist);
  return W;
}

static inline int nchunk_of(int V) { return (V + kChunk - 1) / kChunk; }

static int grid_items(int64_t items) {
  const int64_t cap = 4096;  // 16 workgroups per CU on 256 CUs
  return (int)(items < cap ? items : cap);
}

static int pick_split(int units, int nchunk) {
  const int target = 1024;  // workgroups of k_sample_part
  int s = (target + units - 1) / units;
  if (s < 1) s = 1;
  if (s > nchunk) s = nchunk;
  return s;
}

static inline int launch_ok() { return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH; }

// the wave-per-chunk kernels need 16-byte aligned rows and V % 8 == 0
template <typename T>
static bool wave_chunks_ok(const Problem& P, const AcceptArgs& A) {
  if (P.V % kGroupElems) return false;
  if ((reinterpret_cast<uintptr_t>(P.logits) & 15u) || ((P.row_stride * (int64_t)sizeof(T)) % 16))
    return false;
  if (A.q && ((reinterpret_cast<uintptr_t>(A.q) & 15u) || ((A.q_stride * 4) % 16))) return false;
  return true;
}

template <typename T>
int run_sampler_chain(const Problem& P0, const AcceptArgs& A, const Work& W, int mode,
                      SampleOut O, hipStream_t stream) {
  Problem P = P0;
  const int rows = P.units * P.rows_per_unit;
  const int64_t items = (int64_t)rows * P.nchunk;
  if (mode == HS_ACCEPT_GREEDY) {
    hipLaunchKernelGGL(k_chunk_argmax<T>, dim3(grid_items(items)), dim3(kT), 0, stream, P, W);
    hipLaunchKernelGGL(k_greedy_final, dim3(P.units), dim3(kWave), 0, stream, P, A, W, O.tokens);
    return launch_ok();
  }
  const bool wave = wave_chunks_ok<T>(P, A);
  if (wave) {
    // one chunk per wave, at most the 8 workgroups (32 waves) per CU that fit
    // at once on 256 CUs
    const int64_t wgs = (items + kT / kWave - 1) / (kT / kWave);
    hipLaunchKernelGGL(k_chunk_stats_w<T>, dim3((int)(wgs < 2048 ? wgs : 2048)), dim3(kT), 0,
                       stream, P, W);
  } else {
    hipLaunchKernelGGL(k_chunk_stats<T>, dim3(grid_items(items)), dim3(kT), 0, stream, P, W);
  }
  const bool filtered = (mode == HS_ACCEPT_FILTERED);
  if (filtered) {
    int rc = launch_filter<T>(P, W, O.row_stats, wave, stream);
    if (rc != HS_OK) return rc;
  }
  if (!O.probs && !O.sample) {
    // statistics only: one workgroup per unit folds the rows for row_stats
    P.nsplit = P.nchunk;  // no chunk lies in split 0's range when nsplit > nchunk - 1
    hipLaunchKernelGGL(k_sample_part<T>, dim3(1, P.units), dim3(kT), 0, stream, P, A, W, O, mode,
                       filtered ? 1 : 0);
    return launch_ok();
  }
  if (wave && !O.probs) {
    // (split 0 of either kernel writes the unit's state; k_sample_final reads
    // only the per-chunk sums)
    constexpr int kPerWg = (kT / kWave) * kPartWaveChunks;
    P.nsplit = (P.nchunk + kPerWg - 1) / kPerWg;
    hipLaunchKernelGGL(k_sample_part_w<T>, dim3(P.nsplit, P.units), dim3(kT), 0, stream, P, A, W,
                       O, filtered ? 1 : 0);
  } else {
    P.nsplit = pick_split(P.units, P.nchunk);
    hipLaunchKernelGGL(k_sample_part<T>, dim3(P.nsplit, P.units), dim3(kT), 0, stream, P, A, W, O,
                       mode, filtered ? 1 : 0);
  }
  if (O.sample)
    hipLaunchKernelGGL(k_sample_final<T>, dim3(P.units), dim3(kT), 0, stream, P, A, W, O);
  return launch_ok();
}

}  // namespace hs

using namespace hs;

extern "C" {

const char* hs_status_string(int status) {
  switch (status) {
    case HS_OK: return "ok";
    case HS_ERR_INVALID: return "invalid argument";
    case HS_ERR_WORKSPACE: return "workspace too small";
    case HS_ERR_LAUNCH: return "kernel launch failed";
    case HS_ERR_UNSUPPORTED: return "unsupported configuration";
    case HS_ERR_SCRATCH_LIMIT:
      return "call needs more scratch than the allocation-free entry point holds";
    default: return "unknown status";
  }
}

int hs_version(void) { return (0 << 16) | 2; }

size_t hs_spec_accept_workspace_size(int batch, int gamma, int vocab) {
  if (batch <= 0 || gamma <= 0 || vocab <= 0) return 0;
  return make_layout(batch, batch * (gamma + 1), nchunk_of(vocab)).total;
}

// hs_spec_accept; with cn, also the step's bookkeeping: in the acceptance's
// single launch at batch 1 (*fused = 1), else left to the caller (*fused = 0)
static int accept_impl(const void* target_logits, int logits_dtype, int64_t logits_row_stride,
                       const float* draft_probs, int64_t draft_row_stride,
                       const int64_t* draft_tokens, const float* temperatures,
                       const int32_t* top_ks, const float* top_ps, const float* u_accept,
                       const float* u_resample, int batch, int gamma, int vocab, int mode,
                       int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                       float* row_stats, void* workspace, size_t workspace_bytes,
                       const CommitNext* cn, int* fused, void* stream) {
  *fused = 0;
  if (batch <= 0 || gamma <= 0 || gamma > kMaxGamma || vocab <= 0) return HS_ERR_INVALID;
  if (batch > kMaxRows) return HS_ERR_UNSUPPORTED;
  const bool topk_le64 = (mode & HS_ACCEPT_TOPK_LE64) != 0;
  const bool chain_only = (mode & HS_ACCEPT_CHAIN) != 0;
  mode &= ~(HS_ACCEPT_TOPK_LE64 | HS_ACCEPT_CHAIN);
  if (mode != HS_ACCEPT_REFERENCE && mode != HS_ACCEPT_FILTERED && mode != HS_ACCEPT_GREEDY)
    return HS_ERR_INVALID;
  if (topk_le64 && mode != HS_ACCEPT_FILTERED) return HS_ERR_INVALID;
  if (logits_dtype != HS_F32 && logits_dtype != HS_BF16) return HS_ERR_INVALID;
  if (!target_logits || !draft_tokens || !num_accepted || !out_tokens || !out_len || !workspace)
    return HS_ERR_INVALID;
  if (logits_row_stride < vocab) return HS_ERR_INVALID;
  if (mode != HS_ACCEPT_GREEDY) {
    if (!draft_probs || !temperatures || !u_accept || !u_resample) return HS_ERR_INVALID;
    if (draft_row_stride < vocab) return HS_ERR_INVALID;
  }
  if (mode == HS_ACCEPT_FILTERED && (!top_ks || !top_ps)) return HS_ERR_INVALID;
  const int nchunk = nchunk_of(vocab);
  Layout L = make_layout(batch, batch * (gamma + 1), nchunk);
  if (workspace_bytes < L.total) return HS_ERR_WORKSPACE;

  Problem P;
  P.logits = target_logits;
  P.row_stride = logits_row_stride;
  P.rows_per_unit = gamma + 1;
  P.units = batch;
  P.V = vocab;
  P.nchunk = nchunk;
  P.nsplit = 1;
  P.temps = temperatures;
  P.top_ks = top_ks;
  P.top_ps = top_ps;
  P.filtered = (mode == HS_ACCEPT_FILTERED);
  AcceptArgs A;
  A.q = draft_probs;
  A.q_stride = draft_row_stride;
  A.dtok = draft_tokens;
  A.u_acc = u_accept;
  A.gamma = gamma;
  A.nacc_out = num_accepted;
  A.tok_out = out_tokens;
  A.len_out = out_len;
  SampleOut O;
  O.probs = nullptr;
  O.probs_stride = 0;
  O.out_kind = 0;
  O.uniforms = u_resample;
  O.tokens = nullptr;
  O.sample = 1;
  O.row_stats = row_stats;
  Work W = bind_work(workspace, L);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!chain_only && small_accept_ok(P, A, mode, logits_dtype == HS_F32 ? 4 : 2)) {
    const CommitNext* c = (cn && batch == 1) ? cn : nullptr;
    *fused = c ? 1 : 0;
    if (logits_dtype == HS_F32) return launch_accept_small<float>(P, A, W, O, c, s);
    return launch_accept_small<uint16_t>(P, A, W, O, c, s);
  }
  if (!chain_only && topk_le64 && small_topk_ok(P, A, logits_dtype == HS_F32 ? 4 : 2)) {
    if (logits_dtype == HS_F32) return launch_accept_small_topk<float>(P, A, W, O, s);
    return launch_accept_small_topk<uint16_t>(P, A, W, O, s);
  }
  if (logits_dtype == HS_F32) return run_sampler_chain<float>(P, A, W, mode, O, s);
  return run_sampler_chain<uint16_t>(P, A, W, mode, O, s);
}

int hs_spec_accept(const void* target_logits, int logits_dtype, int64_t logits_row_stride,
                   const float* draft_probs, int64_t draft_row_stride,
                   const int64_t* draft_tokens, const float* temperatures,
                   const int32_t* top_ks, const float* top_ps,
                   const float* u_accept, const float* u_resample,
                   int batch, int gamma, int vocab, int mode,
                   int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                   float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  int fused = 0;
  return accept_impl(target_logits, logits_dtype, logits_row_stride, draft_probs,
                     draft_row_stride, draft_tokens, temperatures, top_ks, top_ps, u_accept,
                     u_resample, batch, gamma, vocab, mode, num_accepted, out_tokens, out_len,
                     row_stats, workspace, workspace_bytes, nullptr, &fused, stream);
}

int hs_spec_accept_commit_next(const void* target_logits, int logits_dtype,
                               int64_t logits_row_stride, const float* draft_probs,
                               int64_t draft_row_stride, const int64_t* draft_tokens,
                               const float* temperatures, const int32_t* top_ks,
                               const float* top_ps, const float* u_accept,
                               const float* u_resample, int batch, int gamma, int vocab, int mode,
                               int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                               float* row_stats, void* workspace, size_t workspace_bytes,
                               const hs_commit_next_args* next, void* stream) {
  if (!next || !next->state || next->state->B != batch) return HS_ERR_INVALID;
  const hs_commit_next_args& n = *next;
  CommitNext c;
  int rc = make_commit_next(n.state, gamma, n.eligible, n.workspace, n.workspace_bytes,
                            n.next_gamma, n.status, n.lookback, n.input_ids, n.positions,
                            n.slot_mapping, n.cu_seqlens_q, n.cu_seqlens_k, n.v_input_ids,
                            n.v_positions, n.v_slot_mapping, n.v_cu_seqlens_q, n.v_cu_seqlens_k,
                            &c);
  if (rc != HS_OK) return rc;
  int fused = 0;
  rc = accept_impl(target_logits, logits_dtype, logits_row_stride, draft_probs, draft_row_stride,
                   draft_tokens, temperatures, top_ks, top_ps, u_accept, u_resample, batch,
                   gamma, vocab, mode, num_accepted, out_tokens, out_len, row_stats, workspace,
                   workspace_bytes, &c, &fused, stream);
  if (rc != HS_OK || fused) return rc;
  return hs_spec_commit_next(n.state, gamma, out_tokens, out_len, n.eligible, n.workspace,
                             n.workspace_bytes, n.next_gamma, n.status, n.lookback, n.input_ids,
                             n.positions, n.slot_mapping, n.cu_seqlens_q, n.cu_seqlens_k,
                             n.v_input_ids, n.v_positions, n.v_slot_mapping, n.v_cu_seqlens_q,
                             n.v_cu_seqlens_k, stream);
}

size_t hs_sampler_workspace_size(int rows, int vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return make_layout(rows, rows, nchunk_of(vocab)).total;
}

int hs_sampler(const void* logits, int logits_dtype, int64_t logits_row_stride, int rows, int vocab,
               const float* temperatures, const int32_t* top_ks, const float* top_ps, int mode,
               float* probs_out, int64_t probs_row_stride, int out_kind, const float* uniforms,
               int64_t* tokens_out, float* row_stats, void* workspace, size_t workspace_bytes,
               void* stream) {
  if (rows <= 0 || vocab <= 0) return HS_ERR_INVALID;
  if (rows > kMaxRows) return HS_ERR_UNSUPPORTED;
  const bool chain_only = (mode & HS_ACCEPT_CHAIN) != 0;
  mode &= ~HS_ACCEPT_CHAIN;
  if (mode != HS_ACCEPT_REFERENCE && mode != HS_ACCEPT_FILTERED && mode != HS_ACCEPT_GREEDY)
    return HS_ERR_INVALID;
  if (logits_dtype != HS_F32 && logits_dtype != HS_BF16) return HS_ERR_INVALID;
  if (!logits || !workspace) return HS_ERR_INVALID;
  if (logits_row_stride < vocab) return HS_ERR_INVALID;
  if (mode != HS_ACCEPT_GREEDY && (uniforms == nullptr) != (tokens_out == nullptr))
    return HS_ERR_INVALID;
  if (mode == HS_ACCEPT_GREEDY) {
    if (probs_out || !tokens_out) return HS_ERR_INVALID;
  } else {
    if (!temperatures) return HS_ERR_INVALID;
    if (probs_out && probs_row_stride < vocab) return HS_ERR_INVALID;
  }
  if (out_kind < 0 || out_kind > 2) return HS_ERR_INVALID;
  if (mode == HS_ACCEPT_FILTERED && (!top_ks || !top_ps)) return HS_ERR_INVALID;
  // reference mode keeps every element: its unfiltered probabilities are out_kind 0's
  if (mode == HS_ACCEPT_REFERENCE && out_kind == 2) out_kind = 0;
  const int nchunk = nchunk_of(vocab);
  Layout L = make_layout(rows, rows, nchunk);
  if (workspace_bytes < L.total) return HS_ERR_WORKSPACE;
  Problem P;
  P.logits = logits;
  P.row_stride = logits_row_stride;
  P.rows_per_unit = 1;
  P.units = rows;
  P.V = vocab;
  P.nchunk = nchunk;
  P.nsplit = 1;
  P.temps = temperatures;
  P.top_ks = top_ks;
  P.top_ps = top_ps;
  P.filtered = (mode == HS_ACCEPT_FILTERED);
  AcceptArgs A;
  memset(&A, 0, sizeof(A));
  SampleOut O;
  O.probs = probs_out;
  O.probs_stride = probs_row_stride;
  O.out_kind = out_kind;
  O.uniforms = uniforms;
  O.tokens = tokens_out;
  O.sample = (mode != HS_ACCEPT_GREEDY && tokens_out) ? 1 : 0;
  O.row_stats = row_stats;
  Work W = bind_work(workspace, L);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int esz = logits_dtype == HS_F32 ? 4 : 2;
  // a few rows in reference mode: one launch (k_sample_small), the same bits
  if (!chain_only && mode == HS_ACCEPT_REFERENCE && small_sampler_ok(P, O, esz)) {
    if (logits_dtype == HS_F32) return launch_sample_small<float>(P, W, O, s);
    return launch_sample_small<uint16_t>(P, W, O, s);
  }
  if (logits_dtype == HS_F32) return run_sampler_chain<float>(P, A, W, mode, O, s);
  return run_sampler_chain<uint16_t>(P, A, W, mode, O, s);
}

}  // extern "C"
