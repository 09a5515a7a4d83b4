// Single-launch acceptance for small batches (reference mode), gfx950.
//
// Same computation as the launch chain of spec_accept.hip (k_chunk_stats ->
// k_sample_part -> k_sample_final) for ModelRunner.run_verify's rejection
// loop, mini_vllm/engine/model_runner.py:387-428, with identical arithmetic
// (exact fixed-point chunk sums over the same 2048-element chunks, the same
// row fold, decision and inverse-CDF draw), so every decision and token is the
// same bit for bit. At batch 1 the chain is bound by three launches' worth of
// dependent latency, not by its 3 MB of reads; this kernel runs the three
// phases in one grid of (chunk, sequence) workgroups:
//   A. chunk statistics of the gamma+1 target rows of chunk c (the rows stay
//      in registers, together with the draft rows' chunk), plus the target
//      logit and draft probability at each draft token;
//   B. every workgroup gathers all chunk statistics of its sequence, folds
//      the row normalisers and takes the decision (deterministic, so all
//      agree), then sums the exact weights of its own chunk of the resample
//      row (residual max(P - Q, 0) or P) from registers;
//   C. every workgroup gathers the chunk weight sums and locates the chunk
//      holding the inverse-CDF point; the workgroup that owns it finds the
//      token with a scan of its registers and writes the outputs.
// Workgroups exchange data through the workspace without barriers: every
// 32-bit payload is stored in one 64-bit word together with the launch's
// epoch (device-scope stores and loads, which write through and miss in the
// XCD's L2), and a reader re-reads a word until it carries the current epoch.
// The epoch comes from a counter every workgroup increments on entry; the
// last one to enter advances it for the next launch, so epochs never repeat
// (2^32 launches) whatever the shapes of earlier calls on the same workspace,
// and the tagged words live in a region of the workspace (kSmallTagBytes at a
// fixed offset) that no other kernel writes.
// The host launches at most one workgroup per CU, so every workgroup is
// resident while others wait for its data; the waits are still bounded (an
// error flag is set and the outputs are marked invalid if one runs out).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hs_device.h"
#include "hs_sampler.h"
#include "hs_sampler_dev.h"
#include "../../include/hilda_spec.h"

namespace hs {

namespace {

constexpr uint32_t kSpinLimit = 1u << 20;

__device__ __forceinline__ void put_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t payload) {
  return ((uint64_t)tag << 32) | payload;
}

// Reads the N tagged words at base[c * N + k] of the NC chunks
// c = lane + i * 64 (chunks past nchunk read chunk 0 and are ignored) until
// every used word carries `tag`. All loads of a round are issued before any is
// waited for. The wait is bounded: when it runs out, the workgroup's flag
// *bad (LDS) and the workspace's error flag are set.
template <int NC, int N>
__device__ __forceinline__ void read_tagged(const uint64_t* base, int nchunk, int lane,
                                            uint32_t tag, uint32_t (&out)[NC][N], SmallSync* sy,
                                            int* bad) {
  for (uint32_t spins = 0;; ++spins) {
    uint64_t v[NC][N];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + i * kWave;
      const int cc = c < nchunk ? c : 0;
#pragma unroll
      for (int k = 0; k < N; ++k) v[i][k] = get_u64(base + (int64_t)cc * N + k);
    }
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const bool used = lane + i * kWave < nchunk;
#pragma unroll
      for (int k = 0; k < N; ++k) {
        out[i][k] = used ? (uint32_t)v[i][k] : 0u;
        ok = ok && (!used || (uint32_t)(v[i][k] >> 32) == tag);
      }
    }
    if (ok) return;
    if (spins == kSpinLimit) {
      *bad = 1;
      __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// 8 consecutive elements [idx, idx + 8) of a 16-byte aligned row whose length
// is a multiple of 8, so a group is either wholly inside the row (`in`) or
// wholly past its end; past the end the load reads the row's first group and
// the values are zeroed. No branch, so the loads of every row go out together.
template <typename T>
__device__ __forceinline__ void load8_row(const T* rp, int64_t idx, bool in, float (&v)[8]) {
  const T* src = rp + (in ? idx : 0);
  if constexpr (sizeof(T) == 2) {
    const uint4 r = *reinterpret_cast<const uint4*>(src);
    v[0] = u2f(r.x << 16); v[1] = u2f(r.x & 0xffff0000u);
    v[2] = u2f(r.y << 16); v[3] = u2f(r.y & 0xffff0000u);
    v[4] = u2f(r.z << 16); v[5] = u2f(r.z & 0xffff0000u);
    v[6] = u2f(r.w << 16); v[7] = u2f(r.w & 0xffff0000u);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = in ? v[k] : 0.0f;
}

// Workgroup of one (chunk, sequence): NG groups of 256 threads; group gi holds
// target rows gi, gi + NG (and the draft rows of the same indices), each
// thread 8 consecutive elements of its rows' chunk, so the per-element work
// of the gamma + 1 rows is spread over up to 16 waves per CU.
template <int G>
struct SmallShape {
  static constexpr int R = G + 1;                 // target rows per sequence
  static constexpr int NG = R < 4 ? R : 4;        // row groups
  static constexpr int RPG = (R + NG - 1) / NG;   // rows per group (1 or 2)
  static constexpr int NW = NG * 4;               // waves
  static constexpr int kThreads = NW * kWave;
};

// Tagged words of the workspace: chunk statistics (m, E low, E high) per
// (row, chunk), then chunk weight sums (w low, w high, p low, p high) per
// (unit, chunk), each chunk's words adjacent.
__device__ __forceinline__ uint64_t* stat_words(const Work& W, int row, int nchunk) {
  return W.tags + (int64_t)row * nchunk * 3;
}
__device__ __forceinline__ uint64_t* samp_words(const Work& W, int rows, int unit, int nchunk) {
  return W.tags + (int64_t)rows * nchunk * 3 + (int64_t)unit * nchunk * 4;
}

// Row descriptor from the chunk statistics of one row (one wave): the fold of
// fold_row_desc (hs_sampler_dev.h) over the tagged copies.
__device__ __forceinline__ RowDesc fold_row_tagged(const Problem& P, const Work& W, int row,
                                                   uint32_t tag, int lane, int* bad) {
  float M = -INFINITY;
  float mc[4];
  uint64_t ec[4];
  // nchunk <= 256 (one workgroup per CU): at most 4 chunks per lane
  uint32_t w[4][3];
  read_tagged<4, 3>(stat_words(W, row, P.nchunk), P.nchunk, lane, tag, w, W.sync, bad);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mc[i] = lane + i * kWave < P.nchunk ? u2f(w[i][0]) : -INFINITY;
    ec[i] = ((uint64_t)w[i][2] << 32) | w[i][1];
    M = fmaxf(M, mc[i]);
  }
  M = wave_max_f32(M);
  uint64_t S = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (lane + i * kWave < P.nchunk)
      S += hs_fx40(hs_f32_rz_of_u64(ec[i]) * kTwoM44 * hs_exp(mc[i] - M));
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

// G: drafts per sequence (gamma), a compile-time constant so that the rows
// live in registers and every load is unconditional
template <typename T, int G>
__global__ __launch_bounds__(SmallShape<G>::kThreads) void k_accept_small(Problem P, AcceptArgs A,
                                                                          Work W, SampleOut O) {
  using S = SmallShape<G>;
  constexpr int R = S::R, NG = S::NG, RPG = S::RPG, NW = S::NW;
  __shared__ float s_m[NW][RPG];
  __shared__ uint64_t s_e[NW][RPG];
  __shared__ RowDesc s_desc[R];
  __shared__ float s_xd[G], s_qd[G];
  __shared__ int64_t s_dt[G];
  __shared__ int s_nacc, s_kind;
  __shared__ uint32_t s_tag;
  __shared__ int s_cstar;
  __shared__ uint64_t s_trel;
  __shared__ int s_use_res;
  __shared__ long long s_tok;
  __shared__ int s_bad;

  const int c = blockIdx.x;
  const int unit = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform indices (scalar registers, so branches on them are scalar)
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wid >> 2, gw = wid & 3;  // row group and wave in it
  const int gt = tid & 255;                // thread in the row group
  const uint32_t nwg = gridDim.x * gridDim.y;
  SmallSync* sy = W.sync;
  const int rows = P.units * R;
  const int64_t i0 = chunk_elem(c, gt, 0);
  const bool in = i0 < P.V;
  const T* lrow = reinterpret_cast<const T*>(P.logits) + (int64_t)unit * R * P.row_stride;
  const float* qrow = A.q + (int64_t)unit * G * A.q_stride;

  // small inputs of wave 0 (it takes the decision): draft tokens and
  // acceptance uniforms, issued first so that their waits cover only them
  int64_t d = -1;
  float u_acc = 1.0f;
  const int jl = lane < G ? lane : 0;
  if (wid == 0) {
    d = A.dtok[(int64_t)unit * G + jl];
    u_acc = A.u_acc[(int64_t)unit * G + jl];
  }
  const float u_res = O.uniforms[unit];
  const float Tt = P.temps[unit];
  const float rT = 1.0f / Tt;
  const bool fastT = hs_rcp_ok(Tt);

  // ---- phase A: this group's rows of chunk c ----
  float x[RPG][8], q[RPG][8];
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    const int j = grp + NG * s;
    // a slot past the last row (and the bonus row's absent draft row) reads
    // only its clamped row's first 8 elements, not a second copy of that row
    load8_row<T>(lrow + (j < R ? j : R - 1) * P.row_stride, i0, in && j < R, x[s]);
    load8_row<float>(qrow + (j < G ? j : G - 1) * A.q_stride, i0, in && j < G, q[s]);
  }
  // keeps the scheduler from hoisting uses of the small inputs (and their
  // waits) above the row loads
  __builtin_amdgcn_sched_barrier(0);
  // logit and draft probability at every draft token (decision inputs, wave
  // 0), then the entry count: this workgroup joins the launch, and the last
  // one to enter advances the epoch for the next launch (every workgroup of
  // this one has read it by then)
  const bool dok = lane < G && d >= 0 && d < P.V;
  T xd_raw = 0;
  float qd = 0.0f;
  uint64_t start = 0;
  if (wid == 0) {
    const int64_t dc = dok ? d : 0;
    xd_raw = lrow[jl * P.row_stride + dc];
    qd = qrow[jl * A.q_stride + dc];
    if (lane == 0) {
      start = __hip_atomic_fetch_add(&sy->start, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)start == nwg - 1)
        __hip_atomic_store(&sy->start, ((start >> 32) + 1) << 32, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // a count already at the grid size means the word was not left by a
  // completed launch (an uncleared workspace, or one shared with another
  // call): the epoch may not advance, so this call's outputs are invalid
  const bool entry_bad = wid == 0 && lane == 0 && (uint32_t)start >= nwg;
  if (entry_bad) __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  float m[RPG];
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    m[s] = -INFINITY;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[s][k] = hs_div_temp(x[s][k], Tt, rT, fastT);
      if (in) m[s] = fmaxf(m[s], x[s][k]);
    }
    m[s] = wave_max_f32(m[s]);
    if (lane == 0) s_m[wid][s] = m[s];
  }
  if (tid == 0) {
    s_tag = (uint32_t)(start >> 32) + 1u;  // tag 0 never matches a zeroed word
    s_bad = entry_bad ? 1 : 0;
  }
  __syncthreads();
  const uint32_t tag = s_tag;
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    const float* gm = &s_m[grp * 4][0];
    m[s] = fmaxf(fmaxf(gm[0 * RPG + s], gm[1 * RPG + s]), fmaxf(gm[2 * RPG + s], gm[3 * RPG + s]));
    uint32_t hi = 0, lo = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (in) hs_fx44_split(hs_exp(x[s][k] - m[s]), hi, lo);
    const uint64_t e = wave_sum_u64(hs_join44(hi, lo));
    if (lane == 0) s_e[wid][s] = e;
  }
  if (wid == 0 && lane < G) {
    s_dt[lane] = d;
    s_xd[lane] = dok ? hs_div_t(ld1<T>(&xd_raw), Tt) : 0.0f;
    s_qd[lane] = qd;
  }
  __syncthreads();
  if (gt == 0) {
#pragma unroll
    for (int s = 0; s < RPG; ++s) {
      const int j = grp + NG * s;
      if (j < R) {
        const uint64_t* ge = &s_e[grp * 4][0];
        const uint64_t es = ge[0 * RPG + s] + ge[1 * RPG + s] + ge[2 * RPG + s] + ge[3 * RPG + s];
        uint64_t* sw = stat_words(W, unit * R + j, P.nchunk) + c * 3;
        put_u64(sw, tagged(tag, f2u(m[s])));
        put_u64(sw + 1, tagged(tag, (uint32_t)es));
        put_u64(sw + 2, tagged(tag, (uint32_t)(es >> 32)));
      }
    }
  }

  // ---- phase B: row normalisers, decision, weights of this chunk ----
  if (wid < R) {
    const RowDesc dd = fold_row_tagged(P, W, unit * R + wid, tag, lane, &s_bad);
    if (lane == 0) s_desc[wid] = dd;
  }
  __syncthreads();
  if (wid == 0) {
    bool rej = false;
    if (lane < G) {
      float pt = 0.0f, pd = 0.0f;
      if (dok) {
        pt = desc_prob(s_desc[lane], s_xd[lane], d);
        pd = s_qd[lane];
      }
      const float ratio = pt / fmaxf(pd, 1e-10f);
      const float a = fminf(ratio, 1.0f);
      rej = !(u_acc < a);
    }
    const uint64_t mask = __ballot(rej);
    const int r = mask ? (__ffsll((long long)mask) - 1) : G;
    if (lane == 0) {
      s_nacc = r;
      s_kind = (r < G) ? kKindResidual : kKindBonus;
    }
  }
  if (c == 0 && O.row_stats && tid < R) {
    const int64_t row = (int64_t)unit * R + tid;
    O.row_stats[2 * row] = s_desc[tid].m;
    O.row_stats[2 * row + 1] = s_desc[tid].s;
  }
  __syncthreads();
  const int r = s_nacc;
  const bool residual = (s_kind == kKindResidual);
  const bool mine = grp == r % NG;  // this group holds row r
  uint64_t w[8], pw[8];
  if (mine) {
    const RowDesc D = s_desc[r];
    const float rS = 1.0f / D.s;
    const bool fastS = hs_rcp_ok(D.s);
    const int sr = r / NG;
    float xr[8], qr[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xr[k] = x[0][k];
      qr[k] = q[0][k];
    }
#pragma unroll
    for (int s = 1; s < RPG; ++s)
      if (s == sr) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          xr[k] = x[s][k];
          qr[k] = q[s][k];
        }
      }
    uint64_t tw = 0, tp = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float p = 0.0f;
      if (in) {
        const float ex = hs_exp(xr[k] - D.m);
        p = fastS ? hs_div_rcp(ex, D.s, rS) : ex / D.s;
      }
      uint32_t hi = 0, lo = 0;
      hs_fx44_split(p, hi, lo);
      pw[k] = hs_join44(hi, lo);
      hi = 0;
      lo = 0;
      if (residual) hs_fx44_split(fmaxf(p - qr[k], 0.0f), hi, lo);
      w[k] = hs_join44(hi, lo);
      tw += w[k];
      tp += pw[k];
    }
    tw = wave_sum_u64(tw);
    tp = wave_sum_u64(tp);
    if (lane == 0) {
      s_e[gw][0] = tw;
      s_e[4 + gw][0] = tp;  // NW >= 8 whenever R >= 2
    }
  }
  __syncthreads();
  if (tid == 0) {
    const uint64_t bw = s_e[0][0] + s_e[1][0] + s_e[2][0] + s_e[3][0];
    const uint64_t bp = s_e[4][0] + s_e[5][0] + s_e[6][0] + s_e[7][0];
    uint64_t* sw = samp_words(W, rows, unit, P.nchunk) + c * 4;
    put_u64(sw, tagged(tag, (uint32_t)bw));
    put_u64(sw + 1, tagged(tag, (uint32_t)(bw >> 32)));
    put_u64(sw + 2, tagged(tag, (uint32_t)bp));
    put_u64(sw + 3, tagged(tag, (uint32_t)(bp >> 32)));
  }

  // ---- phase C: chunk of the inverse-CDF point, token in its owner ----
  if (wid == 0) {
    uint64_t cw[4], cp[4];
    uint64_t wt = 0, pt = 0;
    uint32_t v[4][4];
    read_tagged<4, 4>(samp_words(W, rows, unit, P.nchunk), P.nchunk, lane, tag, v, sy, &s_bad);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cw[i] = ((uint64_t)v[i][1] << 32) | v[i][0];
      cp[i] = ((uint64_t)v[i][3] << 32) | v[i][2];
      wt += cw[i];
      pt += cp[i];
    }
    wt = wave_sum_u64(wt);
    pt = wave_sum_u64(pt);
    // residual normalisation or fallback to P[r] (model_runner.py:419-424)
    const bool use_res = residual && (hs_f32_of_u64(wt) * kTwoM44 > 1e-10f);
    const uint64_t total = use_res ? wt : pt;
    const uint64_t t = hs_mulshift24(hs_u24(u_res), total);
    int cstar = -1;
    uint64_t before = 0, running = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (cstar < 0) {
        const uint64_t val = use_res ? cw[i] : cp[i];
        const uint64_t incl = wave_incl_scan_u64(val, lane);
        const uint64_t mm = __ballot(running + incl > t);
        if (mm) {
          const int l = __ffsll((long long)mm) - 1;
          cstar = i * kWave + l;
          before = running + __shfl(incl, l, 64) - __shfl(val, l, 64);
        } else {
          running += __shfl(incl, 63, 64);
        }
      }
    }
    if (lane == 0) {
      s_cstar = cstar;
      s_trel = t - before;
      s_use_res = use_res ? 1 : 0;
      s_tok = -1;
    }
  }
  __syncthreads();
  const int cstar = s_cstar;
  if (cstar != c && !(cstar < 0 && c == 0)) return;  // one writer per unit
  if (cstar == c) {
    const uint64_t trel = s_trel;
    const bool use_res = s_use_res != 0;
    uint64_t sv = 0, incl = 0;
    if (mine) {
#pragma unroll
      for (int k = 0; k < 8; ++k) sv += use_res ? w[k] : pw[k];
      incl = wave_incl_scan_u64(sv, lane);
      if (lane == 63) s_e[gw][0] = incl;
    }
    __syncthreads();
    if (mine) {
      uint64_t off = 0;
      for (int ww = 0; ww < gw; ++ww) off += s_e[ww][0];
      const uint64_t lo = off + incl - sv;
      if (lo <= trel && trel < off + incl) {
        uint64_t acc = lo;
        for (int k = 0; k < 8; ++k) {
          acc += use_res ? w[k] : pw[k];
          if (acc > trel) {
            s_tok = (long long)(i0 + k);
            break;
          }
        }
      }
    }
    __syncthreads();
  }
  // the outputs depend only on data this workgroup read, so they are valid
  // unless one of its own waits ran out
  const bool bad = s_bad != 0;
  const int64_t token = (int64_t)s_tok;
  if (tid <= G) {
    int64_t v;
    if (bad) v = -1;
    else if (tid < r) v = s_dt[tid];
    else if (tid == r) v = token;
    else v = -1;
    A.tok_out[(int64_t)unit * R + tid] = v;
  }
  if (tid == 0) {
    A.nacc_out[unit] = bad ? -1 : r;
    A.len_out[unit] = bad ? 0 : r + 1;
  }
}

}  // namespace

int small_accept_ok(const Problem& P, const AcceptArgs& A, int mode, int esz) {
  if (mode != HS_ACCEPT_REFERENCE || A.gamma < 1 || A.gamma > 7) return 0;
  // 16-byte aligned rows whose length is a multiple of 8 elements
  if ((P.V % 8) || (((uintptr_t)P.logits | (uintptr_t)A.q) & 15) || ((P.row_stride * esz) % 16) ||
      ((A.q_stride * 4) % 16))
    return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  // every workgroup must be resident at once: at most one per CU (the folds
  // read at most four chunks per lane: nchunk <= 256); the tagged words must
  // fit the region reserved for them
  const size_t tag_bytes =
      ((size_t)P.units * (A.gamma + 1) * 3 + (size_t)P.units * 4) * (size_t)P.nchunk * 8;
  return (P.nchunk <= 4 * kWave && (int64_t)P.nchunk * P.units <= cus &&
          tag_bytes <= kSmallTagBytes) ? 1 : 0;
}

template <typename T>
int launch_accept_small(const Problem& P, const AcceptArgs& A, const Work& W, const SampleOut& O,
                        hipStream_t stream) {
  const dim3 grid(P.nchunk, P.units);
  switch (A.gamma) {
#define HS_SMALL_CASE(G)                                                               \
  case G:                                                                              \
    hipLaunchKernelGGL((k_accept_small<T, G>), grid, dim3(SmallShape<G>::kThreads), 0, \
                       stream, P, A, W, O);                                            \
    break;
    HS_SMALL_CASE(1)
    HS_SMALL_CASE(2)
    HS_SMALL_CASE(3)
    HS_SMALL_CASE(4)
    HS_SMALL_CASE(5)
    HS_SMALL_CASE(6)
    HS_SMALL_CASE(7)
#undef HS_SMALL_CASE
    default: return HS_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

template int launch_accept_small<float>(const Problem&, const AcceptArgs&, const Work&,
                                        const SampleOut&, hipStream_t);
template int launch_accept_small<uint16_t>(const Problem&, const AcceptArgs&, const Work&,
                                           const SampleOut&, hipStream_t);

}  // namespace hs
