// Fused acceptance sampler and row sampler for gfx950.
//
// Replaces the rejection-sampling loop of ModelRunner.run_verify
// (mini_vllm/engine/model_runner.py:387-428) and the sampling ops of
// Sampler.forward (mini_vllm/layers/sampler.py:13-49).
//
// Pipeline of one hs_spec_accept call (B sequences, gamma drafts, V vocab):
//   1. k_row_stats  grid (nsplit, B*(gamma+1)), one wave per workgroup.
//      Each wave streams 2048-element chunks of a target row once from HBM
//      and writes the chunk max m_c and the exact fixed-point sum
//      E_c = sum_i floor(2^44 * exp(x_i - m_c)). The last workgroup of a row
//      (atomic ticket) folds the chunk partials into the row max M and the
//      normaliser S; the last row of a sequence then runs the accept test
//      for all gamma drafts in one wave and records where to resample.
//   2. (filtered mode) k_row_filter: one workgroup per row finds the top-k /
//      top-p boundary (spec_filter.hip).
//   3. k_sample     grid (nsplit, B): streams only the resample row (target
//      row r, and draft row r for a residual) and writes per-chunk exact
//      weight sums; the last workgroup locates the chunk holding the
//      inverse-CDF point and rescans that one chunk to find the token.
// Greedy mode uses k_row_argmax instead of 1-3.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "hs_device.h"
#include "hs_sampler.h"
#include "hs_sampler_dev.h"
#include "../../include/hilda_spec.h"

namespace hs {

template <typename T>
__global__ __launch_bounds__(64) void k_row_stats(Problem P, AcceptArgs A, Work W, int fin,
                                                  float* row_stats) {
  const int row = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x;
  const int unit = row / P.rows_per_unit;
  const float Tt = P.temps[unit];
  const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
  const int c_begin = (int)((int64_t)split * P.nchunk / P.nsplit);
  const int c_end = (int)((int64_t)(split + 1) * P.nchunk / P.nsplit);

  for (int c = c_begin; c < c_end; ++c) {
    const int64_t c0 = (int64_t)c * kChunk;
    float x[kChunkGroups][8];
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g) load8<T>(rp, elem_idx(c0, g, lane, 0), P.V, vec_ok, x[g]);
    float m = -INFINITY;
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        x[g][k] = hs_div_t(x[g][k], Tt);
        if (elem_idx(c0, g, lane, k) < P.V) m = fmaxf(m, x[g][k]);
      }
    m = wave_max_f32(m);
    uint64_t e = 0;
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (elem_idx(c0, g, lane, k) < P.V) e += hs_fx44(hs_exp(x[g][k] - m));
    e = wave_sum_u64(e);
    if (lane == 0) {
      ChunkStat cs;
      cs.m = m;
      cs.pad = 0;
      cs.e = e;
      W.part[(int64_t)row * P.nchunk + c] = cs;
    }
  }

  if (!last_ticket(W.rowctr + row, (uint32_t)P.nsplit, lane)) return;
  fold_row<T>(P, W, row, lane, row_stats);

  if (fin == kFinDecide) {
    if (!last_ticket(W.unitctr + unit, (uint32_t)P.rows_per_unit, lane)) return;
    decide_unit<T>(P, A, W, unit, lane);
  } else if (fin == kFinPlain) {
    if (lane == 0) {
      SeqState s;
      s.kind = kKindPlain;
      s.row = row;
      s.qrow = -1;
      s.nacc = 0;
      s.pad[0] = s.pad[1] = s.pad[2] = s.pad[3] = 0;
      W.st[unit] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// greedy: argmax over raw logits (lowest index on ties)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(64) void k_row_argmax(Problem P, AcceptArgs A, Work W, int fin,
                                                   int64_t* tokens_out) {
  const int row = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x;
  const int unit = row / P.rows_per_unit;
  const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
  const int c_begin = (int)((int64_t)split * P.nchunk / P.nsplit);
  const int c_end = (int)((int64_t)(split + 1) * P.nchunk / P.nsplit);

  for (int c = c_begin; c < c_end; ++c) {
    const int64_t c0 = (int64_t)c * kChunk;
    uint64_t best = 0;
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g) {
      float v[8];
      load8<T>(rp, elem_idx(c0, g, lane, 0), P.V, vec_ok, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        int64_t i = elem_idx(c0, g, lane, k);
        if (i < P.V) {
          uint64_t pk = ((uint64_t)hs_key(v[k]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
          best = pk > best ? pk : best;
        }
      }
    }
    best = wave_max_u64(best);
    if (lane == 0) {
      ChunkStat cs;
      cs.m = 0.0f;
      cs.pad = 0;
      cs.e = best;
      W.part[(int64_t)row * P.nchunk + c] = cs;
    }
  }

  if (!last_ticket(W.rowctr + row, (uint32_t)P.nsplit, lane)) return;
  {
    const ChunkStat* cp = W.part + (int64_t)row * P.nchunk;
    uint64_t best = 0;
    for (int c = lane; c < P.nchunk; c += kWave) best = cp[c].e > best ? cp[c].e : best;
    best = wave_max_u64(best);
    int tok = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
    if (lane == 0) {
      RowDesc d;
      d.m = hs_unkey((uint32_t)(best >> 32));
      d.s = 1.0f;
      d.tkey = 0u;
      d.tidx = 0x7fffffff;
      d.all = 1;
      d.token = tok;
      d.s_full = 1.0f;
      d.pad = 0;
      W.desc[row] = d;
      if (fin == kFinPlain && tokens_out) tokens_out[row] = tok;
    }
  }
  if (fin != kFinDecide) return;
  if (!last_ticket(W.unitctr + unit, (uint32_t)P.rows_per_unit, lane)) return;

  // greedy acceptance: draft j accepted iff it equals the target argmax of row j
  const int g = A.gamma;
  bool rej = false;
  if (lane < g) {
    int64_t d = A.dtok[(int64_t)unit * g + lane];
    int t = W.desc[(int64_t)unit * (g + 1) + lane].token;
    rej = (d != (int64_t)t);
  }
  uint64_t mask = __ballot(rej);
  int r = mask ? (__ffsll((long long)mask) - 1) : g;
  if (lane <= g) {
    int64_t v;
    if (lane < r) v = A.dtok[(int64_t)unit * g + lane];
    else if (lane == r) v = W.desc[(int64_t)unit * (g + 1) + r].token;
    else v = -1;
    A.tok_out[(int64_t)unit * (g + 1) + lane] = v;
  }
  if (lane == 0) {
    A.nacc_out[unit] = r;
    A.len_out[unit] = r + 1;
  }
}

// ---------------------------------------------------------------------------
// sample: inverse-CDF draw from one row per unit (bonus/plain) or from the
// residual max(P - Q, 0) (reject)
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void unit_weights(const Problem& P, const RowDesc& D, float Tt,
                                             const float (&v)[8], const float (&q)[8],
                                             bool residual, bool masked, int64_t i0,
                                             uint64_t (&wres)[8], uint64_t (&wp)[8],
                                             float (&pr)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t i = i0 + k;
    float p = 0.0f, xm = -INFINITY;
    if (i < P.V) {
      const float x = hs_div_t(v[k], Tt);
      if (desc_keep(D, hs_key(x), i)) {
        p = hs_exp(x - D.m) / D.s;
        xm = x;
      }
    }
    pr[k] = masked ? xm : p;
    wp[k] = hs_fx44(p);
    wres[k] = residual ? hs_fx44(fmaxf(p - q[k], 0.0f)) : 0ull;
  }
}

template <typename T>
__global__ __launch_bounds__(64) void k_sample(Problem P, AcceptArgs A, Work W, SampleOut O) {
  const int unit = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x;
  const SeqState st = W.st[unit];
  const int row = st.row;
  // the state is written by the preceding kernel of this call; anything out
  // of range means there is nothing to draw for this unit
  if (st.kind == kKindNone || row < 0 || row >= P.units * P.rows_per_unit) return;
  if (st.kind == kKindResidual && (st.qrow < 0 || st.qrow >= P.units * A.gamma)) return;
  const bool residual = (st.kind == kKindResidual);
  const RowDesc D = W.desc[row];
  const float Tt = P.temps[row / P.rows_per_unit];
  const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
  const float* qp = residual ? A.q + (int64_t)st.qrow * A.q_stride : nullptr;
  const bool q_vec = residual && ((reinterpret_cast<uintptr_t>(qp) & 15u) == 0);
  float* pout = O.probs ? O.probs + (int64_t)row * O.probs_stride : nullptr;
  const bool p_vec = pout && ((reinterpret_cast<uintptr_t>(pout) & 15u) == 0);
  const bool masked = (O.out_kind == 1);
  const int c_begin = (int)((int64_t)split * P.nchunk / P.nsplit);
  const int c_end = (int)((int64_t)(split + 1) * P.nchunk / P.nsplit);

  for (int c = c_begin; c < c_end; ++c) {
    const int64_t c0 = (int64_t)c * kChunk;
    uint64_t sw = 0, sp = 0;
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g) {
      const int64_t i0 = elem_idx(c0, g, lane, 0);
      float v[8], q[8], pr[8];
      uint64_t wres[8], wp[8];
      load8<T>(rp, i0, P.V, vec_ok, v);
      if (residual) load8_f32(qp, i0, P.V, q_vec, q);
      else {
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = 0.0f;
      }
      unit_weights<T>(P, D, Tt, v, q, residual, masked, i0, wres, wp, pr);
      if (pout) store8_f32(pout, i0, P.V, p_vec, pr);
#pragma unroll
      for (int k = 0; k < 8; ++k) { sw += wres[k]; sp += wp[k]; }
    }
    sw = wave_sum_u64(sw);
    sp = wave_sum_u64(sp);
    if (lane == 0) {
      SampPart s;
      s.w = sw;
      s.p = sp;
      W.spart[(int64_t)unit * P.nchunk + c] = s;
    }
  }
  if (!O.sample) return;
  if (!last_ticket(W.sampctr + unit, (uint32_t)P.nsplit, lane)) return;

  // totals and the choice between residual and plain weights (model_runner.py:419-424)
  const SampPart* spp = W.spart + (int64_t)unit * P.nchunk;
  uint64_t wt = 0, pt = 0;
  for (int c = lane; c < P.nchunk; c += kWave) { wt += spp[c].w; pt += spp[c].p; }
  wt = wave_sum_u64(wt);
  pt = wave_sum_u64(pt);
  const bool use_res = residual && (hs_f32_of_u64(wt) * kTwoM44 > 1e-10f);
  const uint64_t total = use_res ? wt : pt;
  const float u = O.uniforms[unit];
  const uint64_t t = hs_mulshift24(hs_u24(u), total);

  // chunk holding the draw
  int cstar = -1;
  uint64_t before = 0, running = 0;
  for (int cb = 0; cb < P.nchunk && cstar < 0; cb += kWave) {
    int c = cb + lane;
    uint64_t val = 0;
    if (c < P.nchunk) val = use_res ? spp[c].w : spp[c].p;
    uint64_t incl = wave_incl_scan_u64(val, lane);
    uint64_t m = __ballot(running + incl > t);
    if (m) {
      int l = __ffsll((long long)m) - 1;
      uint64_t incl_l = __shfl(incl, l, 64);
      uint64_t val_l = __shfl(val, l, 64);
      cstar = cb + l;
      before = running + incl_l - val_l;
    } else {
      running += __shfl(incl, 63, 64);
    }
  }

  int64_t token = -1;
  if (cstar >= 0) {
    const uint64_t trel = t - before;
    const int64_t c0 = (int64_t)cstar * kChunk;
    uint64_t base = 0;
    for (int g = 0; g < kChunkGroups; ++g) {
      const int64_t i0 = elem_idx(c0, g, lane, 0);
      float v[8], q[8], pr[8];
      uint64_t wres[8], wp[8];
      load8<T>(rp, i0, P.V, vec_ok, v);
      if (residual) load8_f32(qp, i0, P.V, q_vec, q);
      else {
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = 0.0f;
      }
      unit_weights<T>(P, D, Tt, v, q, residual, masked, i0, wres, wp, pr);
      uint64_t s = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += use_res ? wres[k] : wp[k];
      uint64_t incl = wave_incl_scan_u64(s, lane);
      uint64_t m = __ballot(base + incl > trel);
      if (m) {
        int l = __ffsll((long long)m) - 1;
        int64_t found = -1;
        if (lane == l) {
          uint64_t acc = base + incl - s;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            acc += use_res ? wres[k] : wp[k];
            if (found < 0 && acc > trel) found = i0 + k;
          }
        }
        token = (int64_t)__shfl((long long)found, l, 64);
        break;
      }
      base += __shfl(incl, 63, 64);
    }
  }

  if (A.tok_out) {
    const int gm = A.gamma;
    if (lane <= gm) {
      int64_t v;
      if (lane < st.nacc) v = A.dtok[(int64_t)unit * gm + lane];
      else if (lane == st.nacc) v = token;
      else v = -1;
      A.tok_out[(int64_t)unit * (gm + 1) + lane] = v;
    }
    if (lane == 0) {
      A.nacc_out[unit] = st.nacc;
      A.len_out[unit] = st.nacc + 1;
    }
  }
  if (O.tokens && lane == 0) O.tokens[unit] = token;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// The ticket counters come first, at fixed offsets for every shape (one slot
// per possible row/unit), so the "counters are left zero" invariant holds
// across calls of different shapes that share one workspace.
Layout make_layout(int units, int rows, int nchunk) {
  Layout L;
  size_t off = 0;
  L.rowctr = off; off = align_up(off + (size_t)kMaxRows * sizeof(uint32_t), 256);
  L.unitctr = off; off = align_up(off + (size_t)kMaxRows * sizeof(uint32_t), 256);
  L.sampctr = off; off = align_up(off + (size_t)kMaxRows * sizeof(uint32_t), 256);
  L.part = off; off = align_up(off + (size_t)rows * nchunk * sizeof(ChunkStat), 256);
  L.desc = off; off = align_up(off + (size_t)rows * sizeof(RowDesc), 256);
  L.st = off; off = align_up(off + (size_t)units * sizeof(SeqState), 256);
  L.spart = off; off = align_up(off + (size_t)units * nchunk * sizeof(SampPart), 256);
  L.filt = off; off = align_up(off + (size_t)rows * sizeof(FilterScratch), 256);
  L.total = off;
  return L;
}

Work bind_work(void* ws, const Layout& L) {
  char* b = static_cast<char*>(ws);
  Work W;
  W.part = reinterpret_cast<ChunkStat*>(b + L.part);
  W.desc = reinterpret_cast<RowDesc*>(b + L.desc);
  W.st = reinterpret_cast<SeqState*>(b + L.st);
  W.spart = reinterpret_cast<SampPart*>(b + L.spart);
  W.filt = reinterpret_cast<FilterScratch*>(b + L.filt);
  W.rowctr = reinterpret_cast<uint32_t*>(b + L.rowctr);
  W.unitctr = reinterpret_cast<uint32_t*>(b + L.unitctr);
  W.sampctr = reinterpret_cast<uint32_t*>(b + L.sampctr);
  return W;
}

static inline int nchunk_of(int V) { return (V + kChunk - 1) / kChunk; }

static int pick_split(int units_or_rows, int nchunk) {
  const int target = 2048;  // waves in flight across 256 CUs
  int s = (target + units_or_rows - 1) / units_or_rows;
  if (s < 1) s = 1;
  if (s > nchunk) s = nchunk;
  return s;
}

template <typename T>
int launch_accept(const Problem& P0, const AcceptArgs& A, const Work& W, int mode, float* row_stats,
                  const float* u_res, hipStream_t stream) {
  Problem P = P0;
  const int rows = P.units * P.rows_per_unit;
  P.nsplit = pick_split(rows, P.nchunk);
  dim3 g1(P.nsplit, rows);
  if (mode == HS_ACCEPT_GREEDY) {
    hipLaunchKernelGGL(k_row_argmax<T>, g1, dim3(64), 0, stream, P, A, W, (int)kFinDecide,
                       (int64_t*)nullptr);
    return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
  }
  const int fin = (mode == HS_ACCEPT_FILTERED) ? kFinRow : kFinDecide;
  hipLaunchKernelGGL(k_row_stats<T>, g1, dim3(64), 0, stream, P, A, W, fin, row_stats);
  if (mode == HS_ACCEPT_FILTERED) {
    int rc = launch_filter<T>(P, A, W, /*decide=*/1, row_stats, stream);
    if (rc != HS_OK) return rc;
  }
  Problem P2 = P;
  P2.nsplit = pick_split(P.units, P.nchunk);
  SampleOut O;
  O.probs = nullptr;
  O.probs_stride = 0;
  O.out_kind = 0;
  O.uniforms = u_res;
  O.tokens = nullptr;
  O.sample = 1;
  hipLaunchKernelGGL(k_sample<T>, dim3(P2.nsplit, P.units), dim3(64), 0, stream, P2, A, W, O);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

template <typename T>
int launch_sampler(const Problem& P0, const Work& W, int mode, float* probs, int64_t probs_stride,
                   int out_kind, const float* uniforms, int64_t* tokens, float* row_stats,
                   hipStream_t stream) {
  Problem P = P0;
  const int rows = P.units;
  P.nsplit = pick_split(rows, P.nchunk);
  AcceptArgs A;
  memset(&A, 0, sizeof(A));
  dim3 g1(P.nsplit, rows);
  if (mode == HS_ACCEPT_GREEDY) {
    hipLaunchKernelGGL(k_row_argmax<T>, g1, dim3(64), 0, stream, P, A, W, (int)kFinPlain, tokens);
    return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(k_row_stats<T>, g1, dim3(64), 0, stream, P, A, W, (int)kFinPlain, row_stats);
  if (mode == HS_ACCEPT_FILTERED) {
    int rc = launch_filter<T>(P, A, W, /*decide=*/0, row_stats, stream);
    if (rc != HS_OK) return rc;
  }
  if (!probs && !tokens) return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
  SampleOut O;
  O.probs = probs;
  O.probs_stride = probs_stride;
  O.out_kind = out_kind;
  O.uniforms = uniforms;
  O.tokens = tokens;
  O.sample = tokens ? 1 : 0;
  hipLaunchKernelGGL(k_sample<T>, dim3(P.nsplit, rows), dim3(64), 0, stream, P, A, W, O);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
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
    default: return "unknown status";
  }
}

int hs_version(void) { return (0 << 16) | 1; }

size_t hs_spec_accept_workspace_size(int batch, int gamma, int vocab) {
  if (batch <= 0 || gamma <= 0 || vocab <= 0) return 0;
  return make_layout(batch, batch * (gamma + 1), nchunk_of(vocab)).total;
}

int hs_spec_accept(const void* target_logits, int logits_dtype, int64_t logits_row_stride,
                   const float* draft_probs, int64_t draft_row_stride,
                   const int64_t* draft_tokens, const float* temperatures,
                   const int32_t* top_ks, const float* top_ps,
                   const float* u_accept, const float* u_resample,
                   int batch, int gamma, int vocab, int mode,
                   int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                   float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  if (batch <= 0 || gamma <= 0 || gamma > kMaxGamma || vocab <= 0) return HS_ERR_INVALID;
  if ((int64_t)batch * (gamma + 1) > kMaxRows) return HS_ERR_UNSUPPORTED;
  if (mode != HS_ACCEPT_REFERENCE && mode != HS_ACCEPT_FILTERED && mode != HS_ACCEPT_GREEDY)
    return HS_ERR_INVALID;
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
  AcceptArgs A;
  A.q = draft_probs;
  A.q_stride = draft_row_stride;
  A.dtok = draft_tokens;
  A.u_acc = u_accept;
  A.gamma = gamma;
  A.nacc_out = num_accepted;
  A.tok_out = out_tokens;
  A.len_out = out_len;
  Work W = bind_work(workspace, L);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (logits_dtype == HS_F32)
    return launch_accept<float>(P, A, W, mode, row_stats, u_resample, s);
  return launch_accept<uint16_t>(P, A, W, mode, row_stats, u_resample, s);
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
  if (out_kind != 0 && out_kind != 1) return HS_ERR_INVALID;
  if (mode == HS_ACCEPT_FILTERED && (!top_ks || !top_ps)) return HS_ERR_INVALID;
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
  Work W = bind_work(workspace, L);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (logits_dtype == HS_F32)
    return launch_sampler<float>(P, W, mode, probs_out, probs_row_stride, out_kind, uniforms,
                                 tokens_out, row_stats, s);
  return launch_sampler<uint16_t>(P, W, mode, probs_out, probs_row_stride, out_kind, uniforms,
                                  tokens_out, row_stats, s);
}

}  // extern "C"
