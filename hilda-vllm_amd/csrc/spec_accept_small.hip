// Single-launch acceptance for small batches, gfx950: reference mode
// (k_accept_small) and filtered mode with every top-k in [1, 64]
// (k_accept_small_topk, described above its definition).
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
#include <string.h>

#include "hs_bookkeeping.h"
#include "hs_device.h"
#include "hs_sampler.h"
#include "hs_sampler_dev.h"
#include "../../include/hilda_spec.h"

// sum over the active lanes of the wave (device library; DPP lane moves)
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_add_u64(
    unsigned long long);

namespace hs {

namespace {

// polls a thread may spend waiting over all its waits of one launch (unless
// the workspace's spin_limit word sets another budget)
constexpr uint32_t kSpinLimit = 1u << 20;
// tags carry an epoch in bits 0..30; a word published by a workgroup whose
// own waits failed carries the tag with this bit set, so that its readers
// fail at once instead of taking values computed from incomplete data
constexpr uint32_t kPoison = 0x80000000u;

// the launch's tag from the entry word's epoch: never 0 (a zeroed word) and
// never with kPoison set
__device__ __forceinline__ uint32_t launch_tag(uint64_t start) {
  return (uint32_t)((start >> 32) % 0x7fffffffull) + 1u;
}

// the wait budget of this launch (SmallSync::spin_limit)
__device__ __forceinline__ uint32_t spin_budget(const SmallSync* sy) {
  const uint32_t w = __hip_atomic_load(const_cast<uint32_t*>(&sy->spin_limit), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return w ? w - 1u : kSpinLimit;
}

// marks the workgroup's outputs invalid (its LDS flag) and the workspace's
// sticky error word
__device__ __forceinline__ void fail_wait(SmallSync* sy, int* bad) {
  *bad = 1;
  __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// the workgroup's flag as other waves may have set it (no barrier between)
__device__ __forceinline__ bool is_bad(int* bad) {
  return __hip_atomic_load(bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}

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
// waited for. The wait is bounded: it gives up at once when the workgroup's
// flag *bad (LDS) is set or a word carries the poisoned tag, and when the
// thread's polls this launch (*spent) reach `limit`; giving up sets *bad and
// the workspace's error flag.
template <int NC, int N>
__device__ __forceinline__ void read_tagged(const uint64_t* base, int nchunk, int lane,
                                            uint32_t tag, uint32_t (&out)[NC][N], SmallSync* sy,
                                            int* bad, uint32_t& spent, uint32_t limit) {
  for (;;) {
    uint64_t v[NC][N];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + i * kWave;
      const int cc = c < nchunk ? c : 0;
#pragma unroll
      for (int k = 0; k < N; ++k) v[i][k] = get_u64(base + (int64_t)cc * N + k);
    }
    bool ok = true, poisoned = false;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const bool used = lane + i * kWave < nchunk;
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const uint32_t t = (uint32_t)(v[i][k] >> 32);
        out[i][k] = used ? (uint32_t)v[i][k] : 0u;
        ok = ok && (!used || t == tag);
        poisoned = poisoned || (used && t == (tag | kPoison));
      }
    }
    if (ok) return;
    if (poisoned || spent >= limit || is_bad(bad)) {
      fail_wait(sy, bad);
      return;
    }
    ++spent;
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
                                                   uint32_t tag, int lane, int* bad,
                                                   uint32_t& spent, uint32_t limit) {
  float M = -INFINITY;
  float mc[4];
  uint64_t ec[4];
  // nchunk <= 256 (one workgroup per CU): at most 4 chunks per lane
  uint32_t w[4][3];
  read_tagged<4, 3>(stat_words(W, row, P.nchunk), P.nchunk, lane, tag, w, W.sync, bad, spent,
                    limit);
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
// live in registers and every load is unconditional. kCommit (batch 1): the
// workgroup that writes the outputs then runs the step's bookkeeping C with
// them (commit_next_body).
template <typename T, int G, bool kCommit>
__global__ __launch_bounds__(SmallShape<G>::kThreads) void k_accept_small(Problem P, AcceptArgs A,
                                                                          Work W, SampleOut O,
                                                                          CommitNext C) {
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
  __shared__ int64_t s_otok[R];
  __shared__ int32_t s_olen;
  __shared__ B1Plan s_plan[kCommit ? kWave : 1];

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
  const uint32_t limit = spin_budget(sy);
  uint32_t spent = 0;
  // the unit's outputs are marked invalid first (by its chunk-0 workgroup,
  // acknowledged before that workgroup publishes anything): only a workgroup
  // whose own waits all succeeded writes them again at the end, so a unit
  // without such a writer keeps -1 / 0 rather than a partial write
  if (c == 0 && tid == 0) {
    __hip_atomic_store(&A.nacc_out[unit], -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&A.len_out[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

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
  // kCommit: the last wave (idle while the exchanges below are waited for)
  // reads the bookkeeping's state words and table row now and the second round
  // before phase B, and plans the commit of the accepted drafts and one more
  // token while phase C's exchange is waited for; the writer then stores it
  constexpr int kFW = NW - 1;
  B1Pre pre{};
  if constexpr (kCommit)
    if (wid == kFW) b1_load1(C, pre);
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
    s_tag = launch_tag(start);
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
    // the invalid marks above reach memory before this workgroup's first word
    if (c == 0 && tid == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t ptag = s_bad ? (tag | kPoison) : tag;
#pragma unroll
    for (int s = 0; s < RPG; ++s) {
      const int j = grp + NG * s;
      if (j < R) {
        const uint64_t* ge = &s_e[grp * 4][0];
        const uint64_t es = ge[0 * RPG + s] + ge[1 * RPG + s] + ge[2 * RPG + s] + ge[3 * RPG + s];
        uint64_t* sw = stat_words(W, unit * R + j, P.nchunk) + c * 3;
        put_u64(sw, tagged(ptag, f2u(m[s])));
        put_u64(sw + 1, tagged(ptag, (uint32_t)es));
        put_u64(sw + 2, tagged(ptag, (uint32_t)(es >> 32)));
      }
    }
  }

  if constexpr (kCommit)
    if (wid == kFW) b1_load2(C, pre);

  // ---- phase B: row normalisers, decision, weights of this chunk ----
  if (wid < R) {
    const RowDesc dd = fold_row_tagged(P, W, unit * R + wid, tag, lane, &s_bad, spent, limit);
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
  // this thread's residual / plain weight sums, then its first offsets within
  // the chunk (mine)
  uint64_t lo_w = 0, lo_p = 0;
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
    lo_w = tw;
    lo_p = tp;
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
    const uint32_t ptag = s_bad ? (tag | kPoison) : tag;
    put_u64(sw, tagged(ptag, (uint32_t)bw));
    put_u64(sw + 1, tagged(ptag, (uint32_t)(bw >> 32)));
    put_u64(sw + 2, tagged(ptag, (uint32_t)bp));
    put_u64(sw + 3, tagged(ptag, (uint32_t)(bp >> 32)));
  }

  // each thread's offsets within the chunk for the token search of the chunk's
  // owner (known only after the exchange below), from the wave scans and the
  // earlier waves' sums, once this chunk's sums are published
  if (mine) {
    const uint64_t iw = wave_incl_scan_u64(lo_w, lane), ip = wave_incl_scan_u64(lo_p, lane);
    uint64_t ow = iw - lo_w, op = ip - lo_p;
    for (int ww = 0; ww < gw; ++ww) {
      ow += s_e[ww][0];
      op += s_e[4 + ww][0];
    }
    lo_w = ow;
    lo_p = op;
  }
  // (the plan waits in LDS, one entry per lane of the wave)
  if constexpr (kCommit) {
    if (wid == kFW) {
      B1Plan q;
      b1_plan(C, pre, r + 1, s_dt, q);
      s_plan[lane] = q;
    }
  }

  // ---- phase C: chunk of the inverse-CDF point, token in its owner ----
  if (wid == 0) {
    uint64_t cw[4], cp[4];
    uint64_t wt = 0, pt = 0;
    uint32_t v[4][4];
    read_tagged<4, 4>(samp_words(W, rows, unit, P.nchunk), P.nchunk, lane, tag, v, sy, &s_bad,
                      spent, limit);
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
    // the element whose weight range [acc, acc + weight) holds trel (zero
    // weights hold nothing): one in the chunk
    const uint64_t trel = s_trel;
    const bool use_res = s_use_res != 0;
    if (mine) {
      uint64_t acc = use_res ? lo_w : lo_p;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint64_t v = use_res ? w[k] : pw[k];
        if (acc <= trel && trel < acc + v) s_tok = (long long)(i0 + k);
        acc += v;
      }
    }
    __syncthreads();
  }
  // the outputs depend only on data this workgroup read, so they are valid
  // unless one of its own waits failed (then they keep the invalid marks of
  // the chunk-0 workgroup, written through before any word this workgroup
  // read); stored at agent scope, after those marks
  if (s_bad != 0) return;
  const int64_t token = (int64_t)s_tok;
  if (tid <= G) {
    int64_t v;
    if (tid < r) v = s_dt[tid];
    else if (tid == r) v = token;
    else v = -1;
    __hip_atomic_store(&A.tok_out[(int64_t)unit * R + tid], v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (kCommit) s_otok[tid] = v;
  }
  if (tid == 0) {
    __hip_atomic_store(&A.len_out[unit], r + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&A.nacc_out[unit], r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (kCommit) s_olen = r + 1;
  }
  if constexpr (kCommit) {
    // the step's bookkeeping, from the outputs just written (this is the
    // only workgroup that reaches here: one unit, one writer)
    __shared__ CommitNextLds<S::kThreads> s_cn;
    __syncthreads();
    B1Plan q{};
    if (wid == kFW) q = s_plan[lane];
    commit_next_planned<S::kThreads>(C, q, kFW, s_otok, &s_olen, s_cn);
  }
}


// ---------------------------------------------------------------------------
// Single launch for filtered mode with every top-k in [1, kTopkMax].
//
// Top-k bounds the kept set of each target row to at most 64 elements, so the
// whole decision and draw of a sequence depend on its rows' top-k candidates
// only, and no third exchange is needed:
//   A. every workgroup (one per 2048-element chunk of the sequence) publishes
//      the maximum (key, index) pair of its chunk of every row;
//   B. every workgroup reads all chunk maxima of its sequence's rows; the k-th
//      largest, tau, is at or below the k-th largest element of the row (k
//      distinct chunk maxima are at or above it), so the row's top-k elements
//      are among those at or above tau. Each workgroup publishes its chunk's
//      elements at or above tau (key, index, draft probability), at most its
//      64 largest (a chunk holds at most k of the row's top k);
//   C. workgroup 0 gathers the candidates (wave j: row j), sorts them, keeps
//      the top k, applies top-p on them with the exact fixed-point masses of
//      the chain (sampler.py:27-49), takes the decision and draws the resample
//      or bonus token over the kept set of at most 64 elements, in index order.
// The arithmetic (temperature division, exp, fixed-point sums and their
// roundings, the draw) is the chain's, so decisions and tokens are the same.
// ---------------------------------------------------------------------------

// rank key of element idx with order key `key`: larger key first, lower index
// first among equal keys (0 never occurs for a real element: idx < 2^31)
__device__ __forceinline__ uint64_t rank_pair(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t pair_idx(uint64_t p) {
  return 0xffffffffu - (uint32_t)p;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort, descending, of the NPL*64 keys a wave holds as v[s] at
// position s*64 + lane, carrying one 32-bit payload per key. Equal keys keep
// their own payloads (both partners of a compare keep theirs on a tie).
template <int NPL>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&v)[NPL], uint32_t (&pl)[NPL],
                                               int lane) {
  constexpr int N = NPL * kWave;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= kWave) {
        const int ts = stride / kWave;
#pragma unroll
        for (int s = 0; s < NPL; ++s) {
          const int s2 = s ^ ts;
          if (s2 > s) {
            const bool desc = ((s * kWave + lane) & size) == 0;
            const bool sw = desc ? (v[s] < v[s2]) : (v[s] > v[s2]);
            if (sw) {
              const uint64_t t = v[s];
              v[s] = v[s2];
              v[s2] = t;
              const uint32_t u = pl[s];
              pl[s] = pl[s2];
              pl[s2] = u;
            }
          }
        }
      } else {
#pragma unroll
        for (int s = 0; s < NPL; ++s) {
          const uint64_t w = shfl_xor_u64(v[s], stride);
          const uint32_t wp = (uint32_t)__shfl_xor((int)pl[s], stride, 64);
          const bool lower = (lane & stride) == 0;
          const bool desc = ((s * kWave + lane) & size) == 0;
          const bool take = (lower == desc) ? (w > v[s]) : (w < v[s]);
          if (take) {
            v[s] = w;
            pl[s] = wp;
          }
        }
      }
    }
  }
}

// Number of entries of v[0, n) (LDS) greater than `mine`; eight reads are issued
// before their compares, so a step costs one LDS latency, not eight.
__device__ __forceinline__ int count_greater(const uint64_t* v, int n, uint64_t mine) {
  int rank = 0, x = 0;
  for (; x + 8 <= n; x += 8) {
    uint64_t t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = v[x + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) rank += t[u] > mine ? 1 : 0;
  }
  for (; x < n; ++x) rank += v[x] > mine ? 1 : 0;
  return rank;
}

// One tagged word, re-read until it carries `tag` (bounded as read_tagged).
__device__ __forceinline__ uint32_t get_tagged(const uint64_t* p, uint32_t tag, SmallSync* sy,
                                               int* bad, uint32_t& spent, uint32_t limit) {
  for (;;) {
    const uint64_t v = get_u64(p);
    const uint32_t t = (uint32_t)(v >> 32);
    if (t == tag) return (uint32_t)v;
    if (t == (tag | kPoison) || spent >= limit || is_bad(bad)) {
      fail_wait(sy, bad);
      return 0u;
    }
    ++spent;
    __builtin_amdgcn_s_sleep(1);
  }
}

// regions of the top-k words (after the reference-mode words)
struct TopkWords {
  uint64_t* base;
  int rows, nchunk;
  __device__ uint64_t* maxw(int row) const { return base + (int64_t)row * nchunk * 2; }
  __device__ uint64_t* cntw(int row) const {
    return base + (int64_t)rows * nchunk * 2 + (int64_t)row * nchunk;
  }
  __device__ uint64_t* candw(int row, int c) const {
    return base + (int64_t)rows * nchunk * 3 + ((int64_t)row * nchunk + c) * (3 * kTopkSlots);
  }
};

__device__ __forceinline__ TopkWords topk_words(const Work& W, int rows, int nchunk) {
  TopkWords t;
  t.base = W.tags + kSmallTagBytes / 8;
  t.rows = rows;
  t.nchunk = nchunk;
  return t;
}

// Candidates of one row gathered by one wave: entries [b0, b0 + 64*NPL) of the
// row's list (chunk order), written through the wave's LDS buffer into the
// sort layout (position s*64 + lane); positions past n hold key 0.
template <int NPL>
__device__ __forceinline__ void gather_cands(const TopkWords& TW, int row, const uint32_t (&cnt)[4],
                                             const uint32_t (&off)[4], int nchunk, int b0, int n,
                                             uint32_t tag, SmallSync* sy, int* bad,
                                             uint32_t& spent, uint32_t limit, int lane,
                                             uint64_t* buf_p, uint32_t* buf_q, uint64_t (&v)[NPL],
                                             uint32_t (&pl)[NPL]) {
  const int b1 = b0 + NPL * kWave;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + i * kWave;
    if (c >= nchunk) continue;
    const int lo = (int)off[i] > b0 ? (int)off[i] : b0;
    const int hi = (int)(off[i] + cnt[i]) < b1 ? (int)(off[i] + cnt[i]) : b1;
    const uint64_t* cw = TW.candw(row, c);
    for (int e = lo; e < hi; ++e) {
      const uint64_t* w = cw + 3 * (e - (int)off[i]);
      const uint32_t key = get_tagged(w, tag, sy, bad, spent, limit);
      const uint32_t idx = get_tagged(w + 1, tag, sy, bad, spent, limit);
      const uint32_t q = get_tagged(w + 2, tag, sy, bad, spent, limit);
      buf_p[e - b0] = rank_pair(key, idx);
      buf_q[e - b0] = q;
    }
  }
  // other lanes of the wave read these entries: the writes complete first
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    const int e = b0 + s * kWave + lane;
    const bool ok = e < n;
    v[s] = ok ? buf_p[s * kWave + lane] : 0ull;
    pl[s] = ok ? buf_q[s * kWave + lane] : 0u;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

template <typename T, int G>
__global__ __launch_bounds__(SmallShape<G>::kThreads) void k_accept_small_topk(Problem P,
                                                                               AcceptArgs A,
                                                                               Work W,
                                                                               SampleOut O) {
  using S = SmallShape<G>;
  constexpr int R = S::R, NG = S::NG, RPG = S::RPG, NW = S::NW, NT = S::kThreads;
  constexpr int kOv = kChunk;  // overflow sort buffer: one row's chunk
  __shared__ uint64_t s_pm[NW][RPG];
  __shared__ uint32_t s_cn[NW][RPG];
  __shared__ uint64_t s_tau[R];
  __shared__ RowDesc s_desc[R];
  __shared__ float s_xd[G], s_qd[G];
  __shared__ int64_t s_dt[G];
  __shared__ int s_nacc;
  __shared__ uint32_t s_tag;
  __shared__ int s_bad;   // outputs invalid (a broken top-k promise, inconsistent words)
  __shared__ int s_fail;  // a wait failed: this workgroup's later words are poisoned
  __shared__ long long s_tok;
  __shared__ int s_nb[R];
  __shared__ uint32_t s_kidx[R][kTopkMax];
  __shared__ float s_ke[R][kTopkMax];
  __shared__ uint32_t s_kq[R][kTopkMax];
  // overflow sort of one row's chunk (phase B), or the gather buffers of the
  // waves of workgroup 0 (phase C)
  __shared__ uint64_t s_big[kOv];
  __shared__ uint32_t s_bigq[kOv];
  // phase C: per row the exclusive candidate offsets of the chunks (and the
  // total at [nchunk]), the positions of the k largest, the draw's kept set
  __shared__ int s_off[R][4 * kWave + 1];
  __shared__ int s_sorted[R][kTopkMax];
  __shared__ uint64_t s_dw[kWave];
  __shared__ uint32_t s_didx[kWave];

  const int c = blockIdx.x;
  const int unit = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wid >> 2;
  const int gt = tid & 255;
  const uint32_t nwg = gridDim.x * gridDim.y;
  SmallSync* sy = W.sync;
  const int rows = P.units * R;
  const TopkWords TW = topk_words(W, rows, P.nchunk);
  const int64_t i0 = chunk_elem(c, gt, 0);
  const bool in = i0 < P.V;
  const uint32_t limit = spin_budget(sy);
  uint32_t spent = 0;
  const T* lrow = reinterpret_cast<const T*>(P.logits) + (int64_t)unit * R * P.row_stride;
  const float* qrow = A.q + (int64_t)unit * G * A.q_stride;

  int64_t d = -1;
  float u_acc = 1.0f;
  const int jl = lane < G ? lane : 0;
  if (wid == 0) {
    d = A.dtok[(int64_t)unit * G + jl];
    u_acc = A.u_acc[(int64_t)unit * G + jl];
  }
  const float u_res = O.uniforms[unit];
  const float Tt = P.temps[unit];
  const int topk = P.top_ks[unit];
  const float topp = P.top_ps[unit];
  const float rT = 1.0f / Tt;
  const bool fastT = hs_rcp_ok(Tt);

  // ---- phase A: rows in registers, chunk maximum pairs ----
  float x[RPG][8], q[RPG][8];
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    const int j = grp + NG * s;
    load8_row<T>(lrow + (j < R ? j : R - 1) * P.row_stride, i0, in && j < R, x[s]);
    load8_row<float>(qrow + (j < G ? j : G - 1) * A.q_stride, i0, in && j < G, q[s]);
  }
  __builtin_amdgcn_sched_barrier(0);
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
  const bool entry_bad = wid == 0 && lane == 0 && (uint32_t)start >= nwg;
  if (entry_bad) __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // a top-k outside [1, kTopkMax] (or above the chunk count) breaks the caller's promise
  const bool k_bad = topk < 1 || topk > kTopkMax || topk > P.nchunk;

  uint32_t key[RPG][8];
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    uint64_t pm = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[s][k] = hs_div_temp(x[s][k], Tt, rT, fastT);
      key[s][k] = hs_key(x[s][k]);
      const uint64_t pr = rank_pair(key[s][k], (uint32_t)(i0 + k));
      if (in && pr > pm) pm = pr;
    }
    pm = wave_max_u64(pm);
    if (lane == 0) s_pm[wid][s] = pm;
  }
  if (tid == 0) {
    s_tag = launch_tag(start);
    s_bad = k_bad ? 1 : 0;
    s_fail = entry_bad ? 1 : 0;
  }
  if (tid < R) s_tau[tid] = 0ull;
  __syncthreads();
  const uint32_t tag = s_tag;
  if (gt == 0) {
    const uint32_t ptag = s_fail ? (tag | kPoison) : tag;
#pragma unroll
    for (int s = 0; s < RPG; ++s) {
      const int j = grp + NG * s;
      if (j < R) {
        uint64_t pm = s_pm[grp * 4][s];
#pragma unroll
        for (int w = 1; w < 4; ++w) pm = s_pm[grp * 4 + w][s] > pm ? s_pm[grp * 4 + w][s] : pm;
        uint64_t* mw = TW.maxw(unit * R + j) + c * 2;
        put_u64(mw, tagged(ptag, (uint32_t)(pm >> 32)));
        put_u64(mw + 1, tagged(ptag, (uint32_t)pm));
      }
    }
  }
  if (wid == 0 && lane < G) {
    s_dt[lane] = d;
    s_xd[lane] = dok ? hs_div_t(ld1<T>(&xd_raw), Tt) : 0.0f;
    s_qd[lane] = qd;
  }

  // ---- phase B: tau per row, this chunk's candidates ----
  const int kk = k_bad ? 1 : topk;
  // the chunk maxima of every row into LDS (wave j: row j); each thread then
  // ranks one of them against the others of its row (broadcast reads) and the
  // one ranked k - 1 is tau (pairs are distinct: their indices differ)
  if (wid < R) {
    uint32_t w[4][2];
    read_tagged<4, 2>(TW.maxw(unit * R + wid), P.nchunk, lane, tag, w, sy, &s_fail, spent, limit);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cc = lane + i * kWave;
      if (cc < P.nchunk) s_big[wid * P.nchunk + cc] = ((uint64_t)w[i][0] << 32) | w[i][1];
    }
  }
  __syncthreads();
  for (int t = tid; t < R * P.nchunk; t += NT) {
    const int j = t / P.nchunk;
    const uint64_t* rp = s_big + j * P.nchunk;
    const uint64_t mine = rp[t - j * P.nchunk];
    if (count_greater(rp, P.nchunk, mine) == kk - 1) s_tau[j] = mine;
  }
  __syncthreads();
  uint32_t cmask[RPG];  // bit k: element k is a candidate of row slot s
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    const int j = grp + NG * s;
    const uint64_t tau = s_tau[j < R ? j : 0];
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (in && j < R && rank_pair(key[s][k], (uint32_t)(i0 + k)) >= tau) m |= 1u << k;
    cmask[s] = m;
    const uint32_t n = wave_sum_u32((uint32_t)__builtin_popcount(m));
    if (lane == 0) s_cn[wid][s] = n;
  }
  __syncthreads();
  // words of a workgroup whose waits failed carry the poisoned tag
  const uint32_t ptag = s_fail ? (tag | kPoison) : tag;
#pragma unroll
  for (int s = 0; s < RPG; ++s) {
    const int j = grp + NG * s;
    if (j >= R) continue;
    const uint32_t* gc = &s_cn[grp * 4][0];
    const uint32_t n = gc[0 * RPG + s] + gc[1 * RPG + s] + gc[2 * RPG + s] + gc[3 * RPG + s];
    if (n > (uint32_t)kTopkSlots) continue;  // published below, after an LDS sort
    uint32_t woff = 0;
    for (int w = 0; w < (wid & 3); ++w) woff += gc[w * RPG + s];
    const uint32_t mine = (uint32_t)__builtin_popcount(cmask[s]);
    const uint32_t before = wave_incl_scan_u32(mine, lane) - mine;
    uint64_t* cw = TW.candw(unit * R + j, c);
    uint32_t slot = woff + before;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (cmask[s] & (1u << k)) {
        put_u64(cw + 3 * slot, tagged(ptag, key[s][k]));
        put_u64(cw + 3 * slot + 1, tagged(ptag, (uint32_t)(i0 + k)));
        put_u64(cw + 3 * slot + 2, tagged(ptag, f2u(j < G ? q[s][k] : 0.0f)));
        ++slot;
      }
    }
    if (gt == 0) put_u64(TW.cntw(unit * R + j) + c, tagged(ptag, n));
  }
  // rows with more than kTopkSlots candidates in this chunk (ties, or rows whose
  // largest values crowd into one chunk): sort the chunk's candidate pairs in
  // LDS with the whole workgroup and publish the 64 largest
  for (int j = 0; j < R; ++j) {
    const int g = j % NG, s = j / NG;
    const uint32_t* gc = &s_cn[g * 4][0];
    const uint32_t n = gc[0 * RPG + s] + gc[1 * RPG + s] + gc[2 * RPG + s] + gc[3 * RPG + s];
    if (n <= (uint32_t)kTopkSlots) continue;  // workgroup-uniform
    __syncthreads();
    if (grp == g) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        s_big[gt * 8 + k] = (cmask[s] & (1u << k)) ? rank_pair(key[s][k], (uint32_t)(i0 + k))
                                                  : 0ull;
    }
    __syncthreads();
    for (int size = 2; size <= kOv; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < kOv; i += NT) {
          const int l = i ^ stride;
          if (l > i) {
            const uint64_t a = s_big[i], b = s_big[l];
            const bool desc = (i & size) == 0;
            if (desc ? (a < b) : (a > b)) {
              s_big[i] = b;
              s_big[l] = a;
            }
          }
        }
        __syncthreads();
      }
    }
    if (tid < kTopkSlots) {
      const uint64_t pr = s_big[tid];
      const uint32_t idx = pair_idx(pr);
      const float qv = j < G ? qrow[j * A.q_stride + idx] : 0.0f;
      uint64_t* cw = TW.candw(unit * R + j, c) + 3 * tid;
      put_u64(cw, tagged(ptag, (uint32_t)(pr >> 32)));
      put_u64(cw + 1, tagged(ptag, idx));
      put_u64(cw + 2, tagged(ptag, f2u(qv)));
      if (tid == 0) put_u64(TW.cntw(unit * R + j) + c, tagged(ptag, (uint32_t)kTopkSlots));
    }
  }
  __syncthreads();     // s_big is reused below
  if (c != 0) return;  // workgroup 0 of the sequence gathers and decides

  // ---- phase C (workgroup 0): kept sets, decision, draw ----
  // candidate counts of every (row, chunk) -> exclusive offsets (wave j: row j)
  if (wid < R) {
    uint32_t cnt[4][1];
    read_tagged<4, 1>(TW.cntw(unit * R + wid), P.nchunk, lane, tag, cnt, sy, &s_fail, spent,
                      limit);
    uint32_t run = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cc = lane + i * kWave;
      const uint32_t cn = cc < P.nchunk ? (cnt[i][0] <= (uint32_t)kTopkSlots ? cnt[i][0] : 0u)
                                        : 0u;
      if (cc < P.nchunk && cnt[i][0] > (uint32_t)kTopkSlots) s_bad = 1;
      const uint32_t inc = wave_incl_scan_u32(cn, lane);
      if (cc < P.nchunk) s_off[wid][cc] = (int)(run + inc - cn);
      run += (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    }
    if (lane == 0) s_off[wid][P.nchunk] = (int)run;
  }
  __syncthreads();
  int rb[R + 1];  // first entry of each row in the workgroup's list
  rb[0] = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) rb[j + 1] = rb[j] + s_off[j][P.nchunk];
  const int total = rb[R];
  const bool in_lds = total <= kOv;  // workgroup-uniform
  if (in_lds) {
    // every candidate's three words, all of a thread's loads in flight together
    constexpr int kPer = (kOv + NT - 1) / NT;
    const uint64_t* ad[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = tid + i * NT;
      ad[i] = nullptr;
      if (e < total) {
        int j = 0;
#pragma unroll
        for (int jj = 1; jj < R; ++jj) j += rb[jj] <= e ? 1 : 0;
        const int el = e - rb[j];
        int lo = 0, hi = P.nchunk;  // s_off[j][lo] <= el < s_off[j][hi]
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (s_off[j][mid] <= el) lo = mid;
          else hi = mid;
        }
        ad[i] = TW.candw(unit * R + j, lo) + 3 * (el - s_off[j][lo]);
      }
    }
    uint64_t wv[kPer][3];
    for (;;) {
#pragma unroll
      for (int i = 0; i < kPer; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k) wv[i][k] = ad[i] ? get_u64(ad[i] + k) : tagged(tag, 0u);
      bool ok = true, poisoned = false;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const uint32_t t = (uint32_t)(wv[i][k] >> 32);
          ok = ok && t == tag;
          poisoned = poisoned || t == (tag | kPoison);
        }
      if (ok) break;
      if (poisoned || spent >= limit || is_bad(&s_fail)) {
        fail_wait(sy, &s_fail);
        break;
      }
      ++spent;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = tid + i * NT;
      if (e < total) {
        s_big[e] = rank_pair((uint32_t)wv[i][0], (uint32_t)wv[i][1]);
        s_bigq[e] = (uint32_t)wv[i][2];
      }
    }
    __syncthreads();
    // rank every candidate within its row (broadcast reads); the k largest are
    // listed in rank order
    for (int e = tid; e < total; e += NT) {
      int j = 0;
#pragma unroll
      for (int jj = 1; jj < R; ++jj) j += rb[jj] <= e ? 1 : 0;
      const int rank = count_greater(s_big + rb[j], rb[j + 1] - rb[j], s_big[e]);
      if (rank < kk) s_sorted[j][rank] = e;
    }
    __syncthreads();
  }
  if (wid < R) {
    const int row = unit * R + wid;
    const int n = s_off[wid][P.nchunk];
    uint64_t top = 0ull;
    uint32_t topq = 0u;
    if (in_lds) {
      if (lane < kk && lane < n) {
        const int e = s_sorted[wid][lane];
        top = s_big[e];
        topq = s_bigq[e];
      }
    } else {
      // more than kOv candidates in all (ties, crowded chunks): each wave merges its
      // row's list 192 entries at a time into the 64 largest
      uint32_t off[4], cn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int cc = lane + i * kWave;
        off[i] = cc < P.nchunk ? (uint32_t)s_off[wid][cc] : 0u;
        cn[i] = cc < P.nchunk ? (uint32_t)(s_off[wid][cc + 1] - s_off[wid][cc]) : 0u;
      }
      uint64_t* bp = s_big + wid * 256;
      uint32_t* bq = s_bigq + wid * 256;
      uint64_t v[4];
      uint32_t pl[4];
      gather_cands<4>(TW, row, cn, off, P.nchunk, 0, n, tag, sy, &s_fail, spent, limit, lane, bp,
                      bq, v, pl);
      wave_sort_desc<4>(v, pl, lane);
      for (int b0 = 4 * kWave; b0 < n; b0 += 3 * kWave) {
        uint64_t v2[4];
        uint32_t p2[4];
        gather_cands<4>(TW, row, cn, off, P.nchunk, b0 - kWave, n, tag, sy, &s_fail, spent, limit,
                        lane, bp,
                        bq, v2, p2);
        v2[0] = v[0];
        p2[0] = pl[0];
        wave_sort_desc<4>(v2, p2, lane);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          v[s] = v2[s];
          pl[s] = p2[s];
        }
      }
      top = v[0];
      topq = pl[0];
    }
    // lane r < k holds rank r of the row's top k
    const int kn = kk;
    const bool rk = lane < kn;
    const float xr = hs_unkey((uint32_t)(top >> 32));
    const float M = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(xr), 0));
    const float er = rk ? hs_exp(xr - M) : 0.0f;
    const uint64_t fe = rk ? hs_fx44(er) : 0ull;
    const float SA = hs_f32_rz_of_u64(__ockl_wfred_add_u64(fe)) * kTwoM44;
    int nb = kn;
    float Sk = SA;
    if (topp < 1.0f) {
      const float mr = rk ? er / SA : 0.0f;
      const uint64_t cum = wave_incl_scan_u64(rk ? hs_fx44(mr) : 0ull, lane);
      const bool keep = rk && (lane == 0 || hs_f32_of_u64(cum) * kTwoM44 < topp);
      nb = __popcll(__ballot(keep));
      if (nb < kn) Sk = hs_f32_rz_of_u64(__ockl_wfred_add_u64(lane < nb ? fe : 0ull)) * kTwoM44;
    }
    // the last kept pair (both halves zero-extended: the low half has its top bit set)
    const uint64_t last =
        (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)top, nb - 1) |
        ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(top >> 32), nb - 1) << 32);
    if (lane < nb) {
      s_kidx[wid][lane] = pair_idx(top);
      s_ke[wid][lane] = er;
      s_kq[wid][lane] = topq;
    }
    if (lane == 0) {
      RowDesc dd;
      dd.m = M;
      dd.s = Sk;
      dd.tkey = (uint32_t)(last >> 32);
      dd.tidx = (int32_t)pair_idx(last);
      dd.all = 0;
      dd.token = -1;
      dd.s_full = Sk;
      dd.pad = 0;
      s_desc[wid] = dd;
      s_nb[wid] = nb;
      if (n < kn) s_bad = 1;  // fewer candidates than k: inconsistent words
      if (O.row_stats) {
        O.row_stats[2 * (int64_t)row] = M;
        O.row_stats[2 * (int64_t)row + 1] = Sk;
      }
    }
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
    // resample (residual max(P - Q, 0), or P when its sum is <= 1e-10) or bonus
    // draw over the kept set of row r, in index order
    const int nb = s_nb[r];
    const bool has = lane < nb;
    const float Sr = s_desc[r].s;
    const uint32_t idx = has ? s_kidx[r][lane] : 0xffffffffu;
    const float p = has ? s_ke[r][lane] / Sr : 0.0f;
    const float qv = has ? u2f(s_kq[r][lane]) : 0.0f;
    const uint64_t pw = hs_fx44(p);
    const uint64_t w = (r < G) ? hs_fx44(fmaxf(p - qv, 0.0f)) : 0ull;
    const uint64_t wt = __ockl_wfred_add_u64(w);
    const uint64_t pt = __ockl_wfred_add_u64(pw);
    const bool use_res = (r < G) && (hs_f32_of_u64(wt) * kTwoM44 > 1e-10f);
    const uint64_t total_w = use_res ? wt : pt;
    const uint64_t t = hs_mulshift24(hs_u24(u_res), total_w);
    // inclusive prefix of the weights in index order: each kept element sums the
    // weights of the kept elements at or below its index; the token is the one
    // element whose prefix passes t while its exclusive prefix does not
    const uint64_t mywt = use_res ? w : pw;
    s_dw[lane] = mywt;
    s_didx[lane] = idx;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    uint64_t incl = 0;
    int x = 0;
    for (; x + 8 <= nb; x += 8) {
      uint32_t ix[8];
      uint64_t wx[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        ix[u] = s_didx[x + u];
        wx[u] = s_dw[x + u];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) incl += ix[u] <= idx ? wx[u] : 0ull;
    }
    for (; x < nb; ++x) incl += s_didx[x] <= idx ? s_dw[x] : 0ull;
    const uint64_t hit = __ballot(has && incl > t && incl - mywt <= t);
    const int first = hit ? __ffsll((long long)hit) - 1 : 0;
    const uint32_t tok_idx = (uint32_t)__builtin_amdgcn_readlane((int)idx, first);
    if (lane == 0) {
      s_nacc = r;
      s_tok = hit ? (long long)tok_idx : -1ll;
    }
  }
  __syncthreads();
  const bool bad = s_bad != 0 || s_fail != 0;
  const int r = s_nacc;
  if (tid <= G) {
    int64_t v;
    if (bad) v = -1;
    else if (tid < r) v = s_dt[tid];
    else if (tid == r) v = (int64_t)s_tok;
    else v = -1;
    A.tok_out[(int64_t)unit * R + tid] = v;
  }
  if (tid == 0) {
    A.nacc_out[unit] = bad ? -1 : r;
    A.len_out[unit] = bad ? 0 : r + 1;
  }
}


// Single-launch row sampler for a few rows (the draft step's probabilities
// and token at small batch, model_runner.py:312-313 with sampler.py:13-25,
// reference mode): one 256-thread workgroup per (chunk, row), every
// workgroup resident at once (the host checks the CU count).
//   A: the chunk's maximum and exact exp-sum of x = logit / T (the chain's
//      chunk statistics), published as tagged words;
//   B: every workgroup folds the row's normaliser from all chunks' words
//      (fold_row_tagged), writes its chunk's probabilities p = e / S and
//      publishes the chunk's fixed-point weight sum (k_sample_part's
//      arithmetic);
//   C: every workgroup locates the chunk holding the inverse-CDF point
//      t = u * W from all weight sums; the workgroup owning it finds the
//      token in its registers (k_sample_final's rule).
// Waits, poisoned words and the invalid mark as in k_accept_small: the row's
// chunk-0 workgroup marks the token -1 first, and only a workgroup whose
// waits all succeeded writes it again.
template <typename T>
__global__ __launch_bounds__(kChunkThreads) void k_sample_small(Problem P, Work W, SampleOut O) {
  __shared__ float s_m[kChunkThreads / kWave];
  __shared__ uint64_t s_e[kChunkThreads / kWave];
  __shared__ RowDesc s_desc;
  __shared__ uint32_t s_tag;
  __shared__ int s_bad;
  __shared__ int s_cstar;
  __shared__ uint64_t s_trel;
  __shared__ long long s_tok;
  const int c = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nwg = gridDim.x * gridDim.y;
  SmallSync* sy = W.sync;
  const int64_t i0 = chunk_elem(c, tid, 0);
  const bool in = i0 < P.V;
  const T* lrow = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
  const uint32_t limit = spin_budget(sy);
  uint32_t spent = 0;
  if (O.sample && c == 0 && tid == 0)
    __hip_atomic_store(&O.tokens[row], (int64_t)-1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- phase A: chunk statistics ----
  float x[8];
  load8_row<T>(lrow, i0, in, x);
  const float u = O.sample ? O.uniforms[row] : 0.0f;
  const float Tt = P.temps[row];
  const float rT = 1.0f / Tt;
  const bool fastT = hs_rcp_ok(Tt);
  __builtin_amdgcn_sched_barrier(0);
  // the entry count (see k_accept_small)
  uint64_t start = 0;
  if (tid == 0) {
    start = __hip_atomic_fetch_add(&sy->start, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)start == nwg - 1)
      __hip_atomic_store(&sy->start, ((start >> 32) + 1) << 32, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  const bool entry_bad = tid == 0 && (uint32_t)start >= nwg;
  if (entry_bad) __hip_atomic_store(&sy->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    x[k] = hs_div_temp(x[k], Tt, rT, fastT);
    if (in) m = fmaxf(m, x[k]);
  }
  m = wave_max_f32(m);
  if (lane == 0) s_m[wid] = m;
  if (tid == 0) {
    s_tag = launch_tag(start);
    s_bad = entry_bad ? 1 : 0;
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
  {
    uint32_t hi = 0, lo = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (in) hs_fx44_split(hs_exp(x[k] - m), hi, lo);
    const uint64_t e = wave_sum_u64(hs_join44(hi, lo));
    if (lane == 0) s_e[wid] = e;
  }
  __syncthreads();
  if (tid == 0) {
    // the invalid mark reaches memory before this workgroup's first word
    if (c == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t ptag = s_bad ? (tag | kPoison) : tag;
    const uint64_t es = s_e[0] + s_e[1] + s_e[2] + s_e[3];
    uint64_t* sw = stat_words(W, row, P.nchunk) + c * 3;
    put_u64(sw, tagged(ptag, f2u(m)));
    put_u64(sw + 1, tagged(ptag, (uint32_t)es));
    put_u64(sw + 2, tagged(ptag, (uint32_t)(es >> 32)));
  }

  // ---- phase B: normaliser, this chunk's probabilities and weight sum ----
  if (wid == 0) {
    const RowDesc dd = fold_row_tagged(P, W, row, tag, lane, &s_bad, spent, limit);
    if (lane == 0) s_desc = dd;
  }
  __syncthreads();
  const RowDesc D = s_desc;
  if (c == 0 && O.row_stats && tid == 0) {
    O.row_stats[2 * (int64_t)row] = D.m;
    O.row_stats[2 * (int64_t)row + 1] = D.s;
  }
  const float rS = 1.0f / D.s;
  const bool fastS = hs_rcp_ok(D.s);
  uint64_t pw[8];
  float pr[8];
  uint64_t tp = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float p = 0.0f;
    if (in) {
      const float e = hs_exp(x[k] - D.m);
      p = fastS ? hs_div_rcp(e, D.s, rS) : e / D.s;
    }
    pr[k] = p;
    uint32_t hi = 0, lo = 0;
    hs_fx44_split(p, hi, lo);
    pw[k] = hs_join44(hi, lo);
    tp += pw[k];
  }
  if (O.probs && in) {
    float* pp = O.probs + (int64_t)row * O.probs_stride + i0;
    *reinterpret_cast<float4*>(pp) = make_float4(pr[0], pr[1], pr[2], pr[3]);
    *reinterpret_cast<float4*>(pp + 4) = make_float4(pr[4], pr[5], pr[6], pr[7]);
  }
  if (!O.sample) return;
  uint64_t lo = tp;  // this thread's sum, then its first offset within the chunk
  tp = wave_sum_u64(tp);
  if (lane == 0) s_e[wid] = tp;
  __syncthreads();
  if (tid == 0) {
    const uint32_t ptag = s_bad ? (tag | kPoison) : tag;
    const uint64_t bp = s_e[0] + s_e[1] + s_e[2] + s_e[3];
    uint64_t* sw = samp_words(W, P.units, row, P.nchunk) + c * 2;
    put_u64(sw, tagged(ptag, (uint32_t)bp));
    put_u64(sw + 1, tagged(ptag, (uint32_t)(bp >> 32)));
  }

  // this thread's offset within the chunk for the owner's token search (known
  // only after the exchange below), once the chunk's sum is published
  {
    const uint64_t ip = wave_incl_scan_u64(lo, lane);
    uint64_t o = ip - lo;
    for (int ww = 0; ww < wid; ++ww) o += s_e[ww];
    lo = o;
  }

  // ---- phase C: chunk of the inverse-CDF point, token in its owner ----
  if (wid == 0) {
    uint32_t v[4][2];
    read_tagged<4, 2>(samp_words(W, P.units, row, P.nchunk), P.nchunk, lane, tag, v, sy, &s_bad,
                      spent, limit);
    uint64_t cp[4], pt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cp[i] = ((uint64_t)v[i][1] << 32) | v[i][0];
      pt += cp[i];
    }
    pt = wave_sum_u64(pt);
    const uint64_t t = hs_mulshift24(hs_u24(u), pt);
    int cstar = -1;
    uint64_t before = 0, running = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (cstar < 0) {
        const uint64_t incl = wave_incl_scan_u64(cp[i], lane);
        const uint64_t mm = __ballot(running + incl > t);
        if (mm) {
          const int l = __ffsll((long long)mm) - 1;
          cstar = i * kWave + l;
          before = running + __shfl(incl, l, 64) - __shfl(cp[i], l, 64);
        } else {
          running += __shfl(incl, 63, 64);
        }
      }
    }
    if (lane == 0) {
      s_cstar = cstar;
      s_trel = t - before;
      s_tok = -1;
    }
  }
  __syncthreads();
  const int cstar = s_cstar;
  if (cstar != c && !(cstar < 0 && c == 0)) return;  // one writer per row
  if (cstar == c) {
    // the element whose weight range [acc, acc + weight) holds trel
    const uint64_t trel = s_trel;
    uint64_t acc = lo;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (acc <= trel && trel < acc + pw[k]) s_tok = (long long)(i0 + k);
      acc += pw[k];
    }
    __syncthreads();
  }
  if (s_bad != 0) return;  // the token keeps its invalid mark
  if (tid == 0)
    __hip_atomic_store(&O.tokens[row], (int64_t)s_tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
                        const CommitNext* cn, hipStream_t stream) {
  if (cn && P.units != 1) return HS_ERR_UNSUPPORTED;
  CommitNext C;
  if (cn) C = *cn;
  else memset(&C, 0, sizeof(C));
  const dim3 grid(P.nchunk, P.units);
  switch (A.gamma) {
#define HS_SMALL_CASE(G)                                                                      \
  case G:                                                                                     \
    if (cn)                                                                                   \
      hipLaunchKernelGGL((k_accept_small<T, G, true>), grid, dim3(SmallShape<G>::kThreads), 0, \
                         stream, P, A, W, O, C);                                              \
    else                                                                                      \
      hipLaunchKernelGGL((k_accept_small<T, G, false>), grid, dim3(SmallShape<G>::kThreads),  \
                         0, stream, P, A, W, O, C);                                           \
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

int small_topk_ok(const Problem& P, const AcceptArgs& A, int esz) {
  if (A.gamma < 1 || A.gamma > 7) return 0;
  if ((P.V % 8) || (((uintptr_t)P.logits | (uintptr_t)A.q) & 15) || ((P.row_stride * esz) % 16) ||
      ((A.q_stride * 4) % 16))
    return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  // every workgroup resident at once; at least kTopkMax chunk maxima per row
  // (tau needs k of them); the words fit their region
  return (P.nchunk >= kTopkMax && P.nchunk <= 4 * kWave && (int64_t)P.nchunk * P.units <= cus &&
          (int64_t)P.units * (A.gamma + 1) * P.nchunk <= kTopkPairs) ? 1 : 0;
}

template <typename T>
int launch_accept_small_topk(const Problem& P, const AcceptArgs& A, const Work& W,
                             const SampleOut& O, hipStream_t stream) {
  const dim3 grid(P.nchunk, P.units);
  switch (A.gamma) {
#define HS_TOPK_CASE(G)                                                                     \
  case G:                                                                                   \
    hipLaunchKernelGGL((k_accept_small_topk<T, G>), grid, dim3(SmallShape<G>::kThreads), 0, \
                       stream, P, A, W, O);                                                 \
    break;
    HS_TOPK_CASE(1)
    HS_TOPK_CASE(2)
    HS_TOPK_CASE(3)
    HS_TOPK_CASE(4)
    HS_TOPK_CASE(5)
    HS_TOPK_CASE(6)
    HS_TOPK_CASE(7)
#undef HS_TOPK_CASE
    default: return HS_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int small_sampler_ok(const Problem& P, const SampleOut& O, int esz) {
  if (P.V % 8 || ((uintptr_t)P.logits & 15) || ((P.row_stride * esz) % 16)) return 0;
  if (O.probs && (((uintptr_t)O.probs & 15) || ((O.probs_stride * 4) % 16))) return 0;
  if (O.out_kind != 0 || (!O.probs && !O.sample)) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  // every workgroup resident at once (one 256-thread workgroup per CU at
  // most), at most four chunks per lane in the folds, words within the region
  const size_t tag_bytes = ((size_t)P.units * 3 + (size_t)P.units * 4) * (size_t)P.nchunk * 8;
  return (P.nchunk <= 4 * kWave && (int64_t)P.nchunk * P.units <= cus &&
          tag_bytes <= kSmallTagBytes) ? 1 : 0;
}

template <typename T>
int launch_sample_small(const Problem& P, const Work& W, const SampleOut& O,
                        hipStream_t stream) {
  hipLaunchKernelGGL(k_sample_small<T>, dim3(P.nchunk, P.units), dim3(kChunkThreads), 0,
                     stream, P, W, O);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

template int launch_sample_small<float>(const Problem&, const Work&, const SampleOut&,
                                        hipStream_t);
template int launch_sample_small<uint16_t>(const Problem&, const Work&, const SampleOut&,
                                           hipStream_t);

template int launch_accept_small<float>(const Problem&, const AcceptArgs&, const Work&,
                                        const SampleOut&, const CommitNext*, hipStream_t);
template int launch_accept_small_topk<float>(const Problem&, const AcceptArgs&, const Work&,
                                             const SampleOut&, hipStream_t);
template int launch_accept_small_topk<uint16_t>(const Problem&, const AcceptArgs&, const Work&,
                                                const SampleOut&, hipStream_t);
template int launch_accept_small<uint16_t>(const Problem&, const AcceptArgs&, const Work&,
                                           const SampleOut&, const CommitNext*, hipStream_t);

}  // namespace hs
