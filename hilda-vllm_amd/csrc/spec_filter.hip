// Top-k / top-p row filter for gfx950 (filtered mode of the sampler).
//
// Semantics follow Sampler._apply_top_k / _apply_top_p,
// mini_vllm/layers/sampler.py:27-49:
//   * x = logits.float() / T (sampler.py:20);
//   * top-k keeps the first k elements of the descending order (ties: lower
//     vocabulary index first), k <= 0 or k >= V disables it (:30);
//   * top-p sorts the survivors descending, forms their softmax and cumulative
//     sum, keeps ranks whose cumulative sum is strictly below p, and always
//     keeps rank 0 (:43-47); p >= 1 disables it for that row.
// The cumulative sum is the exact fixed-point sum of floor(2^44 * p_r),
// rounded to float, so the kept set does not depend on summation order.
//
// Work split:
//   1. top-k with k <= number of 2048-element chunks: the k-th largest chunk
//      maximum is a lower bound of the k-th largest element, so a
//      chunk-parallel pass appends every element at or above it to the row's
//      candidate list (a few dozen for ordinary logits); one workgroup per row
//      sorts them in LDS and applies top-k and top-p (which only looks at the k
//      survivors). From 32 rows up (aligned rows) the pass is gather_k_body,
//      one wave per chunk, reading only the chunks whose maximum reaches the
//      bound; k_filter_plan1 lists the rows of each mode for the passes;
//   2. top-p alone: chunk-parallel passes build an exact mass histogram over
//      256 buckets of (M - x) * 8 (bucket 255 collects the zero masses), find
//      the bucket where the cumulative mass reaches p and append its elements
//      (or, when it holds more than 256, refine it into 256 sub-buckets: up to
//      4096 elements the whole bucket is still appended and the row workgroup
//      keeps the boundary sub-bucket's, above that the row workgroup lists the
//      boundary sub-bucket's elements from the row itself);
//      the row workgroup sorts them and scans
//      their masses from the histogram's prefix;
//   3. otherwise (k above the chunk count, or more than 4096 candidates): the
//      row workgroup runs 8-bit radix passes over the order key with count /
//      mass histograms, finishing in LDS as soon as the candidates fit; ties
//      at the final key are resolved in closed form (equal keys have equal
//      mass) plus one index-ordered pass when a tie is split.
// The acceptance test runs afterwards in k_sample_part (spec_accept.hip).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hs_device.h"
#include "hs_sampler.h"
#include "hs_sampler_dev.h"
#include "../../include/hilda_spec.h"

namespace hs {

constexpr int kFT = kFilterThreads;
constexpr int kFW = kFT / kWave;  // waves per workgroup

struct FilterSmem {
  uint64_t cand[kCand];
  union {
    struct {
      uint64_t scanm[kCand];
      uint64_t scane[kCand];
    } sc;
  } u;
  uint32_t hc[256];
  uint64_t hm[256];
  uint64_t he[256];
  uint64_t wsum[kFW];
  uint64_t wsum2[kFW];
  uint64_t wsum3[kFW];
  uint64_t u64v[8];
  int32_t i32v[8];
};

// exclusive block scan of one u64 per thread; also returns the block total
__device__ __forceinline__ uint64_t block_excl_scan(uint64_t v, uint64_t* wsum, uint64_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
  for (int w = 0; w < kFW; ++w) {
    uint64_t s = wsum[w];
    if (w < wid) off += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

__device__ __forceinline__ uint64_t block_sum(uint64_t v, uint64_t* wsum) {
  uint64_t tot;
  (void)block_excl_scan(v, wsum, &tot);
  return tot;
}

// Smallest X with round_to_float(X) >= p * 2^44 (so that "cumsum < p" is
// "exact fixed-point cumsum < X").
__device__ __forceinline__ uint64_t mass_threshold(float p) {
  const float t = p * kTwo44;  // exact
  if (!(t > 0.0f)) return 0ull;
  // integers below the midpoint of t and the float just below it round below t,
  // integers above it round to t or more; the midpoint itself (a tie) rounds to
  // t only when t's significand is even
  const float tm = u2f(f2u(t) - 1u);
  const double mid = 0.5 * ((double)t + (double)tm);
  uint64_t x0 = (uint64_t)ceil(mid);
  if ((double)x0 == mid && (f2u(t) & 1u)) x0 += 1;
  return x0;
}

// Last coarse bucket whose elements top-p can keep, from a bound that needs
// no pass over the row: an element in bucket b > J has x - M <= -(J+1)/8 (up
// to one rounding of M - x), so its fixed-point mass is at most
// e^-(J+1)/8 / S (1 + 1e-5) (exp within 2.5e-7 relative, one rounding of its
// argument and of the division), and all of them together at most
// U = V e^-(J+1)/8 (1 + 1e-5) / S. The masses of the whole row sum to at
// least 1 - 1e-5 (S is a rounded-toward-zero sum of the same exponentials,
// each floor loses < 2^-44), so when U <= 1 - p - 2e-5 the cumulative mass
// reaches p (the threshold of mass_threshold) inside buckets 0..J. J is the
// smallest bucket with V e^-(J+1)/8 1.001 / S <= (1 - p) - 1e-4 (wider
// margins than the bound needs); kCB - 1 (no bucket skipped) when p is too
// close to 1 or J would reach the last buckets.
__device__ __forceinline__ int mass_skip_bucket(int V, float S, float p) {
  const double room = (1.0 - (double)p) - 1e-4;
  if (!(room > 0.0) || !(S > 0.0f)) return kCB - 1;
  const double t = 8.0 * log((double)V * 1.001 / ((double)S * room));  // need J + 1 >= t
  if (!(t < (double)(kCB - 2))) return kCB - 1;
  const int j = (int)ceil(t) - 1;
  return j < 0 ? 0 : j;
}

template <typename T>
struct RowCtx {
  const T* rp;
  bool vec_ok;
  int V;
  float Tt;
  float rt;   // 1 / Tt, correctly rounded
  bool fast;  // hs_div_rcp applies to Tt
  float M;
  // membership in the kept set A of an earlier stage
  bool a_all;
  uint32_t a_key;
  int64_t a_idx;
  // x = logit / T with IEEE division semantics
  __device__ float div(float v) const { return hs_div_temp(v, Tt, rt, fast); }
  __device__ bool inA(uint32_t key, int64_t i) const {
    return a_all || key > a_key || (key == a_key && i <= a_idx);
  }
};

// Visits every element (raw value, index) of the row. Each thread takes groups
// of 8 consecutive elements kFT * 8 apart and loads kAhead groups before
// handling them, so one workgroup keeps several loads per lane in flight.
template <typename T, typename F>
__device__ __forceinline__ void stream_row(const RowCtx<T>& C, F&& f) {
  constexpr int kAhead = 4;
  const int64_t step = (int64_t)kFT * 8;
  for (int64_t b0 = (int64_t)threadIdx.x * 8; b0 < C.V; b0 += step * kAhead) {
    float v[kAhead][8];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int64_t base = b0 + u * step;
      if (base < C.V) load8<T>(C.rp, base, C.V, C.vec_ok, v[u]);
    }
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int64_t base = b0 + u * step;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (base + k < C.V) f(v[u][k], base + k);
    }
  }
}

// Histogram pass: counts (and masses when `mass`) of elements in A whose key
// prefix above `shift + 8` bits equals `prefix`, bucketed by the next 8 bits.
template <typename T, bool kMass>
__device__ void hist_pass(RowCtx<T> C, FilterSmem& sm, int lvl, uint32_t prefix,
                          float sA) {
  const int tid = threadIdx.x;
  for (int b = tid; b < 256; b += kFT) {
    sm.hc[b] = 0u;
    sm.hm[b] = 0ull;
    sm.he[b] = 0ull;
  }
  __syncthreads();
  const int shift = 24 - 8 * lvl;
  const float rsA = 1.0f / sA;
  const bool fastA = hs_rcp_ok(sA);
  stream_row(C, [&](float raw, int64_t i) {
    const float x = C.div(raw);
    const uint32_t key = hs_key(x);
    if (lvl > 0 && (key >> (shift + 8)) != prefix) return;
    if (!C.inA(key, i)) return;
    const uint32_t b = (key >> shift) & 255u;
    atomicAdd(&sm.hc[b], 1u);
    if (kMass) {
      const float e = hs_exp(x - C.M);
      const uint64_t em = hs_fx44(e);
      const uint64_t mm = hs_fx44(hs_div_temp(e, sA, rsA, fastA));
      if (mm) atomicAdd((unsigned long long*)&sm.hm[b], (unsigned long long)mm);
      if (em) atomicAdd((unsigned long long*)&sm.he[b], (unsigned long long)em);
    }
  });
  __syncthreads();
}

// Gathers every element of A with key >= lo_key into sm.cand as
// (key << 32) | (0xffffffff - index) and sorts them descending (rank order).
// Returns the padded power-of-two size; sm.i32v[0] holds the count.
template <typename T>
__device__ int gather_sort(RowCtx<T> C, FilterSmem& sm, uint32_t lo_key, int expect) {
  const int tid = threadIdx.x;
  int n2 = 1;
  while (n2 < expect) n2 <<= 1;
  if (n2 < 2) n2 = 2;
  for (int i = tid; i < n2; i += kFT) sm.cand[i] = 0ull;
  if (tid == 0) sm.i32v[0] = 0;
  __syncthreads();
  stream_row(C, [&](float raw, int64_t i) {
    const uint32_t key = hs_key(C.div(raw));
    if (key < lo_key || !C.inA(key, i)) return;
    const int slot = atomicAdd(&sm.i32v[0], 1);
    if (slot < kCand)
      sm.cand[slot] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  });
  __syncthreads();
  // bitonic sort, descending
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2; i += kFT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          uint64_t a = sm.cand[i], b = sm.cand[ixj];
          const bool desc = ((i & k) == 0);
          if (desc ? (a < b) : (a > b)) {
            sm.cand[i] = b;
            sm.cand[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  return n2;
}

__device__ __forceinline__ uint32_t cand_key(uint64_t c) { return (uint32_t)(c >> 32); }
__device__ __forceinline__ int64_t cand_idx(uint64_t c) {
  return (int64_t)(0xffffffffu - (uint32_t)(c & 0xffffffffull));
}

// Index of the n-th (1-based) element in index order with key == key0 and in A.
template <typename T>
__device__ int64_t nth_tie(RowCtx<T> C, FilterSmem& sm, uint32_t key0, uint64_t n) {
  const int tid = threadIdx.x;
  uint64_t running = 0;
  if (tid == 0) sm.u64v[0] = ~0ull;
  __syncthreads();
  for (int64_t tile = 0; tile < C.V; tile += (int64_t)kFT * 8) {
    const int64_t base = tile + (int64_t)tid * 8;
    float v[8];
    uint32_t cnt = 0;
    bool hit[8];
    if (base < C.V) load8<T>(C.rp, base, C.V, C.vec_ok, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = base + k;
      hit[k] = false;
      if (i < C.V) {
        const uint32_t key = hs_key(C.div(v[k]));
        hit[k] = (key == key0) && C.inA(key, i);
      }
      cnt += hit[k] ? 1u : 0u;
    }
    uint64_t tot;
    const uint64_t ex = block_excl_scan(cnt, sm.wsum, &tot);
    if (running + ex < n && n <= running + ex + cnt) {
      uint64_t acc = running + ex;
      for (int k = 0; k < 8; ++k) {
        if (hit[k]) {
          acc++;
          if (acc == n) {
            sm.u64v[0] = (uint64_t)(base + k);
            break;
          }
        }
      }
    }
    __syncthreads();
    if (sm.u64v[0] != ~0ull) break;
    running += tot;
  }
  const int64_t r = (int64_t)sm.u64v[0];
  __syncthreads();
  return r;
}

// Top-p over sorted candidates sm.cand[0, n) (rank order from rank 0).
// Writes kept count, boundary and S_B (e-units) to shared scalars.
__device__ __forceinline__ void lds_top_p(FilterSmem& sm, int n, float M, float sA, bool p_on, uint64_t theta,
                          int n2) {
  const int tid = threadIdx.x;
  // per-thread block of kRpt consecutive ranks
  constexpr int kRpt = kCand / kFT;
  uint64_t me[kRpt], mm[kRpt];
  uint64_t se = 0, smm = 0;
  const int r0 = tid * kRpt;
#pragma unroll
  for (int k = 0; k < kRpt; ++k) {
    const int r = r0 + k;
    me[k] = 0;
    mm[k] = 0;
    if (r < n) {
      const float x = hs_unkey(cand_key(sm.cand[r]));
      const float e = hs_exp(x - M);
      me[k] = hs_fx44(e);
      mm[k] = hs_fx44(e / sA);
    }
    se += me[k];
    smm += mm[k];
  }
  uint64_t tot_e, tot_m;
  const uint64_t exe = block_excl_scan(se, sm.wsum, &tot_e);
  const uint64_t exm = block_excl_scan(smm, sm.wsum2, &tot_m);
  (void)n2;
  {
    uint64_t ae = exe, am = exm;
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
      const int r = r0 + k;
      ae += me[k];
      am += mm[k];
      if (r < kCand) {
        sm.u.sc.scane[r] = ae;
        sm.u.sc.scanm[r] = am;
      }
    }
  }
  if (tid == 0) sm.i32v[1] = n;  // first rank with cumsum >= theta (n if none)
  __syncthreads();
  if (p_on) {
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
      const int r = r0 + k;
      if (r < n && sm.u.sc.scanm[r] >= theta) {
        atomicMin(&sm.i32v[1], r);
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    int K = sm.i32v[1];
    if (K < 1) K = 1;
    sm.i32v[2] = K;
    sm.u64v[1] = sm.u.sc.scane[K - 1];  // S_B
    sm.u64v[2] = sm.cand[K - 1];   // boundary
  }
  __syncthreads();
}

// Bitonic sort of sm.cand[0, n2) descending (n2 a power of two).
__device__ __forceinline__ void sort_desc(FilterSmem& sm, int n2) {
  const int tid = threadIdx.x;
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2; i += kFT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          uint64_t a = sm.cand[i], b = sm.cand[ixj];
          const bool desc = ((i & k) == 0);
          if (desc ? (a < b) : (a > b)) {
            sm.cand[i] = b;
            sm.cand[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Bitonic sort of n2 = 64 * E entries of sm.cand (descending) by wave 0 in
// registers: element i = lane * E + e.
template <int E>
__device__ __forceinline__ void wave_sort_desc(FilterSmem& sm) {
  const int lane = threadIdx.x;
  constexpr int n2 = 64 * E;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = sm.cand[lane * E + e];
#pragma unroll
  for (int k = 2; k <= n2; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < E) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int pe = e ^ j;
          if (pe > e) {
            const bool desc = (((lane * E + e) & k) == 0);
            const uint64_t a = v[e], b = v[pe];
            if (desc ? (a < b) : (a > b)) {
              v[e] = b;
              v[pe] = a;
            }
          }
        }
      } else {
        const int lm = j / E;  // partner lane distance
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint64_t o = __shfl_xor((unsigned long long)v[e], lm, kWave);
          const bool desc = (((lane * E + e) & k) == 0);
          const bool keep_max = (desc == ((lane & lm) == 0));
          v[e] = keep_max ? (v[e] > o ? v[e] : o) : (v[e] < o ? v[e] : o);
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) sm.cand[lane * E + e] = v[e];
}

// Sorts sm.cand[0, n) descending, padding with zeros (which sort last) up to a
// power of two; wave 0 alone sorts up to 256 entries in registers.
__device__ __forceinline__ int pad_sort(FilterSmem& sm, int n) {
  int n2 = 64;
  while (n2 < n) n2 <<= 1;
  for (int i = n + threadIdx.x; i < n2; i += kFT) sm.cand[i] = 0ull;
  __syncthreads();
  if (n2 <= 256) {
    if (threadIdx.x < kWave) {
      if (n2 == 64) wave_sort_desc<1>(sm);
      else if (n2 == 128) wave_sort_desc<2>(sm);
      else wave_sort_desc<4>(sm);
    }
    __syncthreads();
  } else {
    sort_desc(sm, n2);
  }
  return n2;
}

// Wave 0 over sorted candidates sm.cand[0, n), n <= 256 (4 ranks per lane):
//   esum_k = sum of floor(2^44 exp(x_r - M)) over the first k ranks (k <= n);
//   first  = first rank r < n whose base_m + sum_{r' <= r} floor(2^44 e_r' / sA)
//            reaches theta (n if none), with e_first = e-mass sum of ranks
//            < first (ranks 0 .. first-1).
// Results in sm.i32v[1] (first) and sm.u64v[1] (e_first), sm.u64v[3] (esum_k).
__device__ __forceinline__ void wave_scan_cands(FilterSmem& sm, int n, float M, float sA,
                                                uint64_t base_m, uint64_t theta, int k) {
  const int lane = threadIdx.x;
  if (lane < kWave) {
    uint64_t me[4], mm[4];
    uint64_t le = 0, lm = 0, lk = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = lane * 4 + q;
      me[q] = 0;
      mm[q] = 0;
      if (r < n) {
        const float e = hs_exp(hs_unkey(cand_key(sm.cand[r])) - M);
        me[q] = hs_fx44(e);
        mm[q] = hs_fx44(e / sA);
      }
      le += me[q];
      lm += mm[q];
      if (r < k) lk += me[q];
    }
    const uint64_t ie = wave_incl_scan_u64(le, lane);
    const uint64_t im = wave_incl_scan_u64(lm, lane);
    const uint64_t esk = wave_sum_u64(lk);
    uint64_t ae = ie - le, am = base_m + im - lm;
    int first = n;
    uint64_t efirst = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = lane * 4 + q;
      if (r < n && first == n && am + mm[q] >= theta) {
        first = r;
        efirst = ae;
      }
      ae += me[q];
      am += mm[q];
    }
    const uint64_t hit = __ballot(first < n);
    if (hit) {
      const int src = __ffsll((long long)hit) - 1;
      first = __shfl(first, src, kWave);
      efirst = __shfl((unsigned long long)efirst, src, kWave);
    } else {
      first = n;
      efirst = wave_sum_u64(le);
    }
    if (lane == 0) {
      sm.i32v[1] = first;
      sm.u64v[1] = efirst;
      sm.u64v[3] = esk;
    }
  }
  __syncthreads();
}

// Inclusive scans of the masses of the sorted candidates sm.cand[0, n):
// sm.i32v[1] = first rank whose scan reaches theta_rel (n if none), with the
// inclusive e-mass scan in sm.u.sc.scane.
__device__ __forceinline__ void scan_bucket(FilterSmem& sm, int n, float M, float sA, uint64_t theta_rel) {
  const int tid = threadIdx.x;
  constexpr int kRpt = kCand / kFT;
  uint64_t me[kRpt], mm[kRpt];
  uint64_t se = 0, smm = 0;
  const int r0 = tid * kRpt;
#pragma unroll
  for (int k = 0; k < kRpt; ++k) {
    const int r = r0 + k;
    me[k] = 0;
    mm[k] = 0;
    if (r < n) {
      const float e = hs_exp(hs_unkey(cand_key(sm.cand[r])) - M);
      me[k] = hs_fx44(e);
      mm[k] = hs_fx44(e / sA);
    }
    se += me[k];
    smm += mm[k];
  }
  uint64_t te, tm;
  uint64_t ae = block_excl_scan(se, sm.wsum, &te);
  uint64_t am = block_excl_scan(smm, sm.wsum2, &tm);
  if (tid == 0) sm.i32v[1] = n;
  __syncthreads();
  bool found = false;
#pragma unroll
  for (int k = 0; k < kRpt; ++k) {
    const int r = r0 + k;
    ae += me[k];
    am += mm[k];
    if (r < n) {
      sm.u.sc.scane[r] = ae;
      if (!found && am >= theta_rel) {
        atomicMin(&sm.i32v[1], r);
        found = true;
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Chunk-parallel filter passes (256-thread workgroups, 8 elements per thread
// per 2048-element chunk, the geometry of k_chunk_stats; each workgroup takes
// a segment of consecutive chunks of one row, see seg_plan).
//   mode 1 (top-k with k <= chunks): pass 1 appends every element at or above
//           the k-th largest chunk maximum to the row's candidate list;
//   mode 2 (top-p alone): pass 1 accumulates exact masses into a 256-bucket
//           histogram of (M - x) * 8 (bucket 255 collects the zero masses);
//           pass 2 finds the coarse bucket where the cumulative mass reaches p
//           and appends its elements (at most kDirect of them), or else
//           histograms them into 256 fine sub-buckets (still appending them
//           all when they fit the kCand list, for k_row_filter to pick the
//           fine boundary bucket from); above kCand elements k_row_filter
//           finds the fine boundary bucket and lists its elements itself.
// k_row_filter then finishes each row in LDS from its candidates.
// ---------------------------------------------------------------------------
constexpr int kPT = kChunkThreads;
static_assert(kPT == kCB, "one histogram bucket per thread");
// a coarse boundary bucket with more elements than this is refined into fine
// sub-buckets first (small candidate sets sort in one wave)
constexpr uint32_t kDirect = 256;
// pass 1 (wave kernel) keeps a bucket's count above bit 45 of its mass word
constexpr int kPackShift = 45;
// per-wave logit queue of the top-p first pass (a 512-element group adds at
// most 512; 12 KB per workgroup keeps 8 workgroups per CU within the LDS)
constexpr uint32_t kQ1 = 768;
// per-wave candidate buffer of k_filter_pass2_w
constexpr uint32_t kCandBuf = 128;
// per-wave element queue of k_filter_pass2_w (holds a half group: 256)
constexpr uint32_t kQueue = 256;

__device__ __forceinline__ int filter_mode(const Problem& P, int unit) {
  const int kk = P.top_ks[unit];
  const float pp = P.top_ps[unit];
  const bool k_on = (kk > 0 && kk < P.V);
  if (k_on && kk <= P.nchunk) return 1;
  if (!k_on && pp < 1.0f) return 2;
  return 0;
}

// coarse bucket of (M - x) * 8; monotone in x
__device__ __forceinline__ int coarse_bucket(float x, float M) {
  const float d = (M - x) * 8.0f;
  return (d < (float)(kCB - 1)) ? (int)d : kCB - 1;
}
// fine bucket inside coarse bucket b1 (x must lie in b1); monotone in x
__device__ __forceinline__ int fine_bucket(float x, float M, int b1) {
  const float f = ((M - x) * 8.0f - (float)b1) * 256.0f;  // exact: Sterbenz, powers of two
  const int b = (int)f;
  return b < 0 ? 0 : (b > kCB - 1 ? kCB - 1 : b);
}

// Smallest float r (in hs_key order, over [-inf, +inf]) with pred(r) true, for
// a pred that is false below some value and true from it on; NaN when pred
// holds nowhere (every comparison with it is false). Called by a whole wave
// (wave-uniform arguments): each round the 64 lanes test 63 keys spread over
// the open interval, so the 2^32 keys take at most 6 rounds of one pred each.
template <typename F>
__device__ __forceinline__ float raw_threshold(F pred) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t lo = 0x007fffffu, hi = 0xff800000u;  // keys of -inf and +inf
  if (!pred(hs_unkey(hi))) return __builtin_nanf("");
  if (pred(hs_unkey(lo))) return -INFINITY;
  // invariant: pred(lo) false, pred(hi) true
  while (hi - lo > 1u) {
    const uint32_t span = hi - lo;
    const uint32_t pt = lo + (uint32_t)(((uint64_t)span * (uint64_t)(lane + 1)) >> 6);
    const bool t = (lane == kWave - 1) || pred(hs_unkey(pt));  // lane 63 tests hi
    const uint64_t m = __ballot(t);
    const int first = __ffsll((long long)m) - 1;
    const uint32_t nhi = (uint32_t)__shfl((int)pt, first, kWave);
    const uint32_t nlo = first == 0 ? lo : (uint32_t)__shfl((int)pt, first - 1, kWave);
    lo = nlo;
    hi = nhi;
  }
  return hs_unkey(hi);
}

// exclusive scan over the kNT threads of a workgroup (kNT / 64 waves)
template <int kNT>
__device__ __forceinline__ uint64_t blk_scan(uint64_t v, uint64_t* wsum, uint64_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kNT / 64; ++w) {
    const uint64_t x = wsum[w];
    if (w < wid) off += x;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

// First bucket of a kCB-bucket histogram (thread t holds bucket t, t < kCB) whose
// inclusive cumulative mass, starting from base_m, reaches theta. Returns it (or
// -1) and the count / mass / e-mass of the buckets before it (plus the bases).
struct Crossing {
  int b;
  uint64_t c, m, e;
};
template <int kNT>
__device__ __forceinline__ Crossing find_crossing(uint64_t hc, uint64_t hm, uint64_t he, uint64_t base_m,
                                  uint64_t theta, uint64_t* wsum, int* s_b, uint64_t* s_v) {
  const int t = threadIdx.x;
  uint64_t tot;
  const uint64_t xm = blk_scan<kNT>(hm, wsum, &tot) + base_m;
  const uint64_t xe = blk_scan<kNT>(he, wsum, &tot);
  const uint64_t xc = blk_scan<kNT>(hc, wsum, &tot);
  if (t == 0) *s_b = -1;
  __syncthreads();
  if (t < kCB && xm < theta && xm + hm >= theta) {
    *s_b = t;  // unique: the cumulative mass is monotone
    s_v[0] = xc;
    s_v[1] = xm;
    s_v[2] = xe;
  }
  __syncthreads();
  Crossing r;
  r.b = *s_b;
  r.c = s_v[0];
  r.m = s_v[1];
  r.e = s_v[2];
  __syncthreads();
  return r;
}

// Slots of the flagged elements (bit k of flags) of the calling wave's lanes,
// numbered element-major (every lane's element 0 in lane order, then element
// 1, ...) from ballots and lane counts, with no LDS round trip; returns the
// wave's total (wave-uniform).
template <int N = 8>
__device__ __forceinline__ uint32_t wave_slots8(uint32_t flags, uint32_t (&slot)[8]) {
  uint32_t total = 0;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const uint64_t m = __ballot((flags >> k) & 1u);
    slot[k] = total + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    total += (uint32_t)__popcll(m);
  }
  return total;
}

// The same numbering taken straight from the comparisons: build(mask) keeps
// one lane mask per element (bit l of m[k] is set when lane l's element k is
// flagged) and the running totals before each, so a lane's slot for element k
// is off[k] plus the flagged lanes below it. Callers form each mask from
// ballots of single comparisons (a v_cmp result in scalar registers, used as
// is) combined with scalar mask operations; a ballot of a compound condition
// goes through a 0/1 register and a second comparison, and a per-lane flag
// word that the ballots are re-derived from (wave_slots8) compiles to
// per-element branches and bit-field extractions, which were most of a filter
// pass's instructions.
__device__ __forceinline__ uint64_t lanes_where(bool c) { return __builtin_amdgcn_ballot_w64(c); }
template <int N>
struct WaveMasks {
  uint64_t m[N];
  uint32_t off[N];
  template <typename F>
  __device__ __forceinline__ uint32_t build(F mask) {
    uint32_t total = 0;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      m[k] = mask(k);
      off[k] = total;
      total += (uint32_t)__popcll(m[k]);
    }
    return total;
  }
  // lane's bit of ballot k (for use after code that ends the comparisons' lifetimes)
  __device__ __forceinline__ bool has(int k, int lane) const { return (m[k] >> lane) & 1ull; }
  __device__ __forceinline__ uint32_t slot(int k) const {
    return off[k] + __builtin_amdgcn_mbcnt_hi((uint32_t)(m[k] >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)m[k], 0u));
  }
};

// Appends the (up to 8) flagged elements of every lane of the calling wave (all
// lanes active) to the row's candidate list: slots from wave_slots8 and one
// global atomic per wave, no barrier. Slots past kCand are counted but not
// written (the row filter then falls back to its radix select).
__device__ __forceinline__ void wave_append_cands(const Work& W, int row, const uint32_t (&key)[8],
                                                  uint32_t flags, int64_t i0) {
  const int lane = threadIdx.x & 63;
  uint32_t slot[8];
  const uint32_t total = wave_slots8(flags, slot);
  if (total == 0) return;  // wave-uniform
  int base = 0;
  if (lane == 0) base = atomicAdd(&W.filt[row].ncand, (int)total);
  base = __builtin_amdgcn_readlane(base, 0);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int sl = base + (int)slot[k];
    if ((flags & (1u << k)) && sl < kCand)
      W.cand[(int64_t)row * kCand + sl] =
          ((uint64_t)key[k] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(i0 + k));
  }
}

// Segments of consecutive chunks for the pass kernels: a workgroup takes one
// segment of one row, with as many segments per row as fill the grid, so a
// row's LDS histogram reaches global memory once per segment.
// With nr rows in the list, nseg = max(1, grid / nr) segments per row, so
// items = nr * nseg <= max(grid, rows) and all of the indexing is 32-bit.
struct SegPlan {
  int nseg, q, r, items;
};
__device__ __forceinline__ SegPlan seg_plan(const Problem& P, int nr, int grid) {
  int nseg = nr > 0 ? grid / nr : 1;
  nseg = nseg < 1 ? 1 : (nseg > P.nchunk ? P.nchunk : nseg);
  SegPlan sp;
  sp.nseg = nseg;
  sp.q = P.nchunk / nseg;
  sp.r = P.nchunk - sp.q * nseg;
  sp.items = nr * nseg;
  return sp;
}
// chunks [c_lo, c_hi) of segment seg: the first r segments hold q + 1 chunks,
// the others q
__device__ __forceinline__ void seg_chunks(const SegPlan& sp, int seg, int& c_lo, int& c_hi) {
  c_lo = seg * sp.q + (seg < sp.r ? seg : sp.r);
  c_hi = c_lo + sp.q + (seg < sp.r ? 1 : 0);
}

struct alignas(16) PassShared {
  uint32_t keys[kCB];  // first: read as uint4
  uint64_t wsum[kPT / 64];
  uint64_t hm[kCB], he[kCB];
  uint32_t hc[kCB];
  uint64_t v[3];
  int b;
};

// 1 when key ke (slot e of ne) ranks above key kc: greater, or equal at a
// lower chunk index
__device__ __forceinline__ int rank_vs(uint32_t ke, uint32_t kc, int e, int ne, bool lower) {
  return (e < ne && (ke > kc || (ke == kc && lower))) ? 1 : 0;
}

// Per row (one 256-thread workgroup): row max M and normaliser S (the fold of
// the chunk statistics), the top-k gather threshold (mode 1: key of the keff-th
// largest chunk maximum; its rank = greater keys + equal keys of lower chunk
// index, unique) and the top-p mass threshold (mode 2).
__global__ __launch_bounds__(kPT) void k_filter_plan1(Problem P, Work W) {
  __shared__ PassShared ps;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int unit = row / P.rows_per_unit;
  const int mode = filter_mode(P, unit);
  FilterScratch& f = W.filt[row];
  if (tid == kPT - kWave && mode) {
    // the passes below walk only the rows of their mode (counters cleared by
    // the chunk-statistics launch); the last wave appends while wave 0 folds
    const int rows = P.units * P.rows_per_unit;
    if (mode == 1) W.flist[2 + atomicAdd(&W.flist[0], 1)] = row;
    else W.flist[2 + rows + atomicAdd(&W.flist[1], 1)] = row;
  }
  if (wid == 0) {
    const RowDesc d = fold_row_desc(P, W, row, lane);
    const int jmax = (mode == 2) ? mass_skip_bucket(P.V, d.s, P.top_ps[unit]) : kCB - 1;
    // the logits pass 1 histograms; a row whose max is not finite takes none
    // and goes to the row filter's radix path (k_filter_plan2)
    float rj = 0.0f;
    if (mode == 2) {
      const float Tt = P.temps[unit], rT = 1.0f / Tt, M = d.m;
      const bool fast = hs_rcp_ok(Tt);
      rj = isfinite(M) ? raw_threshold([&](float r) {
        return coarse_bucket(hs_div_temp(r, Tt, rT, fast), M) <= jmax;
      }) : __builtin_nanf("");
    }
    if (lane == 0) {
      f.m = d.m;
      f.s = d.s;
      f.b1 = -1;
      f.ac = f.am = f.ae = 0ull;
      f.theta = (mode == 2) ? mass_threshold(P.top_ps[unit]) : 0ull;
      f.jmax = jmax;
      f.rj = rj;
    }
  }
  if (mode != 1) return;
  const int keff = P.top_ks[unit];
  const ChunkStat* cp = W.part + (int64_t)row * P.nchunk;
  for (int base = 0; base < P.nchunk; base += kCB) {
    // chunk maxima [base, base + kCB) ranked against all chunk maxima
    const int c = base + tid;
    const uint32_t kc = (c < P.nchunk) ? hs_key(cp[c].m) : 0u;
    int rank = 0;
    for (int b2 = 0; b2 < P.nchunk; b2 += kCB) {
      __syncthreads();
      ps.keys[tid] = (b2 + tid < P.nchunk) ? hs_key(cp[b2 + tid].m) : 0u;
      __syncthreads();
      const int ne = (P.nchunk - b2 < kCB) ? P.nchunk - b2 : kCB;
      // four keys per LDS read (all kCB slots are written), several in flight
      const uint4* k4 = reinterpret_cast<const uint4*>(ps.keys);
#pragma unroll 4
      for (int e = 0; e < ne; e += 4) {
        const uint4 q = k4[e >> 2];
        rank += rank_vs(q.x, kc, e, ne, b2 + e < c) + rank_vs(q.y, kc, e + 1, ne, b2 + e + 1 < c) +
                rank_vs(q.z, kc, e + 2, ne, b2 + e + 2 < c) + rank_vs(q.w, kc, e + 3, ne, b2 + e + 3 < c);
      }
    }
    if (c < P.nchunk && rank == keff - 1) f.tau = kc;
  }
}

// Per mode-2 row: the coarse bucket where the cumulative mass reaches p, its
// element count and logit range, and the sums before it. b1 is -1 when the
// row never reaches p and -2 when the row filter must stream the row (no
// crossing although pass 1 skipped buckets, which the skip bound rules out,
// or a row maximum that is not finite).
__global__ __launch_bounds__(kPT) void k_filter_plan2(Problem P, Work W) {
  __shared__ PassShared ps;
  const int row = blockIdx.x, t = threadIdx.x;
  if (filter_mode(P, row / P.rows_per_unit) != 2) return;
  FilterScratch& f = W.filt[row];
  const int64_t hb = (int64_t)row * kCB + t;
  const uint32_t hc = W.h1c[hb];
  const Crossing cr = find_crossing<kPT>(hc, W.h1m[hb], W.h1e[hb], 0ull, f.theta, ps.wsum,
                                         &ps.b, ps.v);
  if (cr.b >= 0 && t == cr.b) f.c1 = hc;
  if (t < kWave) {
    const float M = f.m;
    const int b1 = !isfinite(M) ? -2 : (cr.b < 0 && f.jmax < kCB - 1) ? -2 : cr.b;
    float rlo = 0.0f, rhi = 0.0f;
    if (b1 >= 0) {
      // logits of coarse bucket b1: [min with bucket <= b1, min with bucket < b1)
      const int unit = row / P.rows_per_unit;
      const float Tt = P.temps[unit], rT = 1.0f / Tt;
      const bool fast = hs_rcp_ok(Tt);
      rlo = raw_threshold([&](float r) {
        return coarse_bucket(hs_div_temp(r, Tt, rT, fast), M) <= b1;
      });
      rhi = b1 == 0 ? INFINITY : raw_threshold([&](float r) {
        return coarse_bucket(hs_div_temp(r, Tt, rT, fast), M) < b1;
      });
    }
    if (t == 0) {
      f.b1 = b1;
      f.rlo = rlo;
      f.rhi = rhi;
      f.ac = cr.c;
      f.am = cr.m;
      f.ae = cr.e;
    }
  }
}

// only2: walk the top-p rows only (gather_k_body takes the top-k rows).
// Workgroups take segments of chunks (seg_plan): a top-p row's histogram
// accumulates in LDS over the segment and reaches global memory once (flushes
// per chunk made the global atomics a third of the pass). Top-p rows
// histogram only buckets 0..jmax (mass_skip_bucket): a wave packs those
// elements of a chunk into its LDS queue and its lanes then take the exp,
// fixed-point masses and atomics of the queue densely.
template <typename T>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_filter_pass1(
    Problem P, Work W, int only2) {
  __shared__ PassShared ps;
  __shared__ float s_q[kPT / kWave][8 * kWave];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int rows = P.units * P.rows_per_unit;
  const SegPlan sp = seg_plan(P, only2 ? W.flist[1] : rows, (int)gridDim.x);
  for (int it = blockIdx.x; it < sp.items; it += gridDim.x) {
    const int ri = it / sp.nseg;
    const int row = only2 ? W.flist[2 + rows + ri] : ri;
    const int unit = row / P.rows_per_unit;
    const int mode = filter_mode(P, unit);
    if (mode == 0) continue;
    int c_lo, c_hi;
    seg_chunks(sp, it - ri * sp.nseg, c_lo, c_hi);
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
    const FilterScratch& f = W.filt[row];
    if (mode == 1) {
      const uint32_t tau = f.tau;
      for (int c = c_lo; c < c_hi; ++c) {
        const int64_t i0 = chunk_elem(c, tid, 0);
        float x[8];
        load8<T>(rp, i0, P.V, vec_ok, x);
        uint32_t key[8], flags = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          key[k] = hs_key(hs_div_temp(x[k], Tt, rT, fast));
          if (i0 + k < P.V && key[k] >= tau) flags |= 1u << k;
        }
        wave_append_cands(W, row, key, flags, i0);
      }
    } else {
      ps.hm[tid] = 0ull;
      ps.he[tid] = 0ull;
      ps.hc[tid] = 0u;
      __syncthreads();
      const float M = f.m, S = f.s;
      const float rS = 1.0f / S;
      const bool fastS = hs_rcp_ok(S);
      const float rj = f.rj;  // logit >= rj <=> coarse bucket <= jmax
      float* q = s_q[tid / kWave];
      for (int c = c_lo; c < c_hi; ++c) {
        const int64_t i0 = chunk_elem(c, tid, 0);
        float x[8];
        load8<T>(rp, i0, P.V, vec_ok, x);
        const bool full = i0 + 8 <= P.V;
        uint32_t flags = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (x[k] >= rj && (full || i0 + k < P.V)) flags |= 1u << k;
        uint32_t slot[8];
        const uint32_t total = wave_slots8(flags, slot);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (flags & (1u << k)) q[slot[k]] = x[k];
        // the queue is this wave's: its LDS writes land before its reads
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        for (uint32_t j = (uint32_t)lane; j < total; j += kWave) {
          const float xv = hs_div_temp(q[j], Tt, rT, fast);
          const int b = coarse_bucket(xv, M);
          atomicAdd(&ps.hc[b], 1u);
          if (b < kCB - 1) {  // the last bucket holds only zero masses
            const float e = hs_exp(xv - M);
            const uint64_t em = hs_fx44(e);
            const uint64_t mm = hs_fx44(hs_div_temp(e, S, rS, fastS));
            if (mm) atomicAdd((unsigned long long*)&ps.hm[b], (unsigned long long)mm);
            if (em) atomicAdd((unsigned long long*)&ps.he[b], (unsigned long long)em);
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
      __syncthreads();
      const int64_t hb = (int64_t)row * kCB + tid;
      if (ps.hc[tid]) {
        atomicAdd(&W.h1c[hb], ps.hc[tid]);
        if (ps.hm[tid]) atomicAdd((unsigned long long*)&W.h1m[hb], (unsigned long long)ps.hm[tid]);
        if (ps.he[tid]) atomicAdd((unsigned long long*)&W.h1e[hb], (unsigned long long)ps.he[tid]);
      }
      __syncthreads();
    }
  }
}

// Top-p rows with 16-byte aligned rows and V % 8 == 0: the work of
// hs_div_temp(v, T, 1/T, fast) for one queued element per lane: the
// corrected product for every lane, then the IEEE quotient for the lanes whose
// numerator lies outside [2^-96, 2^60] (a branch the wave takes only when one
// of its lanes has such a value). T is the same in every lane.
__device__ __forceinline__ float drain_div_temp(float v, float Tt, float rT, bool fast) {
  if (Tt == 1.0f) return v;
  if (!fast) return v / Tt;
  float x = hs_div_rcp_in_range(v, Tt, rT);
  const bool out = ((f2u(v) << 1) + 0xE1000000u) > 0x9C000000u;  // see lane_chunk_rcp_ok
  if (__builtin_amdgcn_ballot_w64(out) != 0 && out) {
    // a side effect the compiler cannot move: a division is one IR instruction,
    // which it otherwise evaluates for every lane and selects
    asm volatile("" : "+v"(v));
    x = v / Tt;
  }
  return x;
}

// (e / S) * 2^20 given e20 = e * 2^20 (hs_exp_2p20), equal to
// 2^20 hs_div_temp(e, S, 1/S, fastS): the corrected product on e20 when e is
// 0 or in [2^-96, 1] (the quotient is then normal), else hs_div_rcp on e
// (lanes of a wave taking that branch only when one of its lanes needs it).
__device__ __forceinline__ float drain_p20(float e20, float S, float rS, bool fastS) {
  if (!fastS) return (e20 * 0x1p-20f / S) * 1048576.0f;
  float p20 = hs_div_rcp_in_range(e20, S, rS);
  const bool small = f2u(e20) - 1u < f2u(0x1p-76f) - 1u;  // e20 in (0, 2^-76)
  if (__builtin_amdgcn_ballot_w64(small) != 0 && small)
    p20 = hs_div_rcp(e20 * 0x1p-20f, S, rS) * 1048576.0f;
  return p20;
}

// k_filter_pass1 for mode-2 rows with one wave per chunk of the workgroup's
// segment, so that each wave has the chunk's four 1 KB (bf16) or 2 KB (f32)
// loads in flight together (lane_chunk_load); the histogram accumulates in LDS
// over the segment as there, and the logits at or above rj are packed per
// 512-element group into the wave's LDS queue.
template <typename T>
__device__ __forceinline__ void pass1_w_body(const Problem& P, const Work& W, int blk, int nblk,
                                             PassShared& ps,
                                             float (&s_q)[kPT / kWave][kQ1]) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int rows = P.units * P.rows_per_unit;
  const SegPlan sp = seg_plan(P, W.flist[1], nblk);  // top-p rows only
  float* q = s_q[wid];
  for (int it = blk; it < sp.items; it += nblk) {
    const int ri = it / sp.nseg;
    const int row = W.flist[2 + rows + ri];
    const int unit = row / P.rows_per_unit;  // a top-p row (the list holds no others)
    int c_lo, c_hi;
    seg_chunks(sp, it - ri * sp.nseg, c_lo, c_hi);
    const FilterScratch& f = W.filt[row];
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const float M = f.m, S = f.s;
    const float rS = 1.0f / S;
    const bool fastS = hs_rcp_ok(S);
    const float rj = f.rj;  // logit >= rj <=> coarse bucket <= jmax
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    ps.hm[tid] = 0ull;
    ps.he[tid] = 0ull;
    __syncthreads();
    // the queue fills over several groups and chunks before the wave works
    // through it, so its passes over the queue run with full lanes
    uint32_t nq = 0;  // wave-uniform: logits in the queue
    auto drain = [&]() {
      // the queue is this wave's: its LDS writes land before its reads
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      for (uint32_t j = (uint32_t)lane; j < nq; j += kWave) {
        const float v = q[j];
        const float xv = drain_div_temp(v, Tt, rT, fast);
        const int b = coarse_bucket(xv, M);
        // count and mass in one word (kPackShift): the masses of a row sum to
        // at most 2^44 (1 + 1e-5), a segment holds fewer than 2^19 elements
        uint64_t cm = 1ull << kPackShift;
        if (b < kCB - 1) {  // the last bucket holds only zero masses
          const float e20 = hs_exp_2p20(xv - M);  // hs_exp * 2^20
          uint32_t eh = 0, el = 0, ph = 0, pl = 0;
          hs_fx44_acc(e20, eh, el);  // hs_fx44(e)
          hs_fx44_acc(drain_p20(e20, S, rS, fastS), ph, pl);  // hs_fx44(e / S)
          const uint64_t em = hs_join44(eh, el);
          cm += hs_join44(ph, pl);
          if (em) atomicAdd((unsigned long long*)&ps.he[b], (unsigned long long)em);
        }
        atomicAdd((unsigned long long*)&ps.hm[b], (unsigned long long)cm);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      nq = 0;
    };
    for (int c = c_lo + wid; c < c_hi; c += kPT / kWave) {
      const int64_t c0 = (int64_t)c * kChunk;
      LaneChunk<T> r;
      lane_chunk_load<T>(rp, c0, P.V, lane, true, r);
#pragma unroll
      for (int g = 0; g < kLaneChunkGroups; ++g) {
        // room for a whole group first, so the comparisons below serve as the
        // ballots and as the write masks with nothing kept across a drain
        if (nq > kQ1 - kWave * kGroupElems) drain();
        const bool in = lane_chunk_idx(c0, g, lane, 0) < P.V;
        auto hit = [&](int k) { return lane_chunk_val<T>(r, g, k) >= rj; };
        const uint64_t inm = lanes_where(in);
        WaveMasks<kGroupElems> wm;
        const uint32_t total = wm.build([&](int k) { return lanes_where(hit(k)) & inm; });
        if (total == 0) continue;  // wave-uniform
#pragma unroll
        for (int k = 0; k < kGroupElems; ++k)
          if (in && hit(k)) q[nq + wm.slot(k)] = lane_chunk_val<T>(r, g, k);
        nq += total;
      }
    }
    if (nq) drain();
    __syncthreads();
    const int64_t hb = (int64_t)row * kCB + tid;
    const uint32_t cnt = (uint32_t)(ps.hm[tid] >> kPackShift);
    const uint64_t mass = ps.hm[tid] & ((1ull << kPackShift) - 1);
    if (cnt) {
      atomicAdd(&W.h1c[hb], cnt);
      if (mass) atomicAdd((unsigned long long*)&W.h1m[hb], (unsigned long long)mass);
      if (ps.he[tid]) atomicAdd((unsigned long long*)&W.h1e[hb], (unsigned long long)ps.he[tid]);
    }
    __syncthreads();
  }
}

// Top-p rows with 16-byte aligned rows and V % 8 == 0: the work of
// k_filter_pass2 with one wave per chunk of the segment (loads as in
// pass1_w_body).
template <typename T>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_filter_pass2_w(
    Problem P, Work W) {
  __shared__ PassShared ps;
  __shared__ float s_qv[kPT / kWave][kQueue];
  __shared__ uint32_t s_qi[kPT / kWave][kQueue];
  // each wave's candidates collect here and reach the row's list in one
  // atomic per kCandBuf / 2 of them (an atomic that returns costs a memory
  // round trip, which per chunk was most of the pass)
  __shared__ uint64_t s_cb[kPT / kWave][kCandBuf];
  // the wave index in a scalar register and the thread index rebuilt from it
  // and the lane: kept whole through the segment loop, threadIdx.x was the
  // value spilled (8 bytes per lane at entry) under the 64-VGPR cap
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int tid = wid * kWave + lane;
  const int rows = P.units * P.rows_per_unit;
  const SegPlan sp = seg_plan(P, W.flist[1], (int)gridDim.x);  // top-p rows only
  float* qv = s_qv[wid];
  uint32_t* qi = s_qi[wid];
  uint64_t* cb = s_cb[wid];
  for (int it = blockIdx.x; it < sp.items; it += gridDim.x) {
    const int ri = it / sp.nseg;
    const int row = W.flist[2 + rows + ri];
    const int unit = row / P.rows_per_unit;  // a top-p row (the list holds no others)
    const FilterScratch& f = W.filt[row];
    const int seg = it - ri * sp.nseg;
    const int b1 = f.b1;
    if (b1 < 0) continue;
    const uint32_t c1 = f.c1;
    const bool fine = c1 > kDirect;                  // workgroup-uniform
    const bool listed = c1 <= (uint32_t)kCand;      // see k_filter_pass2
    if (fine) {
      ps.hm[tid] = 0ull;
      ps.he[tid] = 0ull;
      ps.hc[tid] = 0u;
      __syncthreads();
    }
    int c_lo, c_hi;
    seg_chunks(sp, seg, c_lo, c_hi);
    const float M = f.m, S = f.s;
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const float rS = 1.0f / S;
    const bool fastS = hs_rcp_ok(S);
    const float rlo = f.rlo, rhi = f.rhi;  // coarse bucket b1 <=> rlo <= logit < rhi
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    uint32_t nb = 0;  // wave-uniform: candidates in cb
    auto flush = [&]() {
      int base = 0;
      if (lane == 0) base = atomicAdd(&W.filt[row].ncand, (int)nb);
      base = __builtin_amdgcn_readlane(base, 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      for (uint32_t j = (uint32_t)lane; j < nb; j += kWave)
        if (base + (int)j < kCand) W.cand[(int64_t)row * kCand + base + (int)j] = cb[j];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      nb = 0;
    };
    // bucket-b1 elements wait in the wave's LDS queue and are handled a batch
    // at a time (a handful per segment for ordinary rows): each batch is one
    // chain of dependent latencies for the wave, where per occurrence they
    // added up to most of the pass
    uint32_t nq = 0;  // wave-uniform: elements in the queue
    auto drain = [&]() {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      for (uint32_t j0 = 0; j0 < nq; j0 += kWave) {
        const uint32_t j = j0 + (uint32_t)lane;
        const bool have = j < nq;
        const float xv = have ? drain_div_temp(qv[j], Tt, rT, fast) : 0.0f;
        const uint32_t idx = have ? qi[j] : 0u;
        if (listed) {
          if (nb > kCandBuf - kWave) flush();
          const uint64_t m = __ballot(have);
          const uint32_t sl = nb + __builtin_amdgcn_mbcnt_hi(
                                       (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          if (have) cb[sl] = ((uint64_t)hs_key(xv) << 32) | (uint64_t)(0xffffffffu - idx);
          nb += (uint32_t)__popcll(m);
        }
        if (fine && have) {
          const int b = fine_bucket(xv, M, b1);
          const float e20 = hs_exp_2p20(xv - M);  // hs_exp * 2^20
          atomicAdd(&ps.hc[b], 1u);
          uint32_t eh = 0, el = 0, ph = 0, pl = 0;
          hs_fx44_acc(e20, eh, el);                           // hs_fx44(e)
          hs_fx44_acc(drain_p20(e20, S, rS, fastS), ph, pl);  // hs_fx44(e / S)
          const uint64_t mm = hs_join44(ph, pl);
          const uint64_t em = hs_join44(eh, el);
          if (mm) atomicAdd((unsigned long long*)&ps.hm[b], (unsigned long long)mm);
          if (em) atomicAdd((unsigned long long*)&ps.he[b], (unsigned long long)em);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      nq = 0;
    };
    for (int c = c_lo + wid; c < c_hi; c += kPT / kWave) {
      const int64_t c0 = (int64_t)c * kChunk;
      LaneChunk<T> r;
      lane_chunk_load<T>(rp, c0, P.V, lane, true, r);
#pragma unroll
      for (int h = 0; h < 2 * kLaneChunkGroups; ++h) {
        // half h of the lane's chunk: group h / 2, elements 4 (h % 2) .. + 4
        // (at most 256 per wave, what the queue takes at once)
        const int g = h >> 1, k0 = 4 * (h & 1);
        const int64_t i0 = lane_chunk_idx(c0, g, lane, k0);
        const bool in = i0 < P.V;
        // rlo <= v < rhi as (v >= rlo) and not (v >= rhi): the same set for every
        // v (a NaN fails the first comparison)
        const uint64_t inm = lanes_where(in);
        WaveMasks<4> wm;
        const uint32_t total = wm.build([&](int k) {
          const float v = lane_chunk_val<T>(r, g, k0 + k);
          return lanes_where(v >= rlo) & ~lanes_where(v >= rhi) & inm;
        });
        if (total == 0) continue;  // wave-uniform; the common case
        if (nq + total > kQueue) drain();
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (wm.has(k, lane)) {
            qv[nq + wm.slot(k)] = lane_chunk_val<T>(r, g, k0 + k);
            qi[nq + wm.slot(k)] = (uint32_t)(i0 + k);
          }
        nq += total;
      }
    }
    if (nq) drain();
    if (nb) flush();
    if (fine) {
      __syncthreads();
      const int64_t hb = (int64_t)row * kCB + tid;
      if (ps.hc[tid]) {
        atomicAdd(&W.h2c[hb], ps.hc[tid]);
        if (ps.hm[tid]) atomicAdd((unsigned long long*)&W.h2m[hb], (unsigned long long)ps.hm[tid]);
        if (ps.he[tid]) atomicAdd((unsigned long long*)&W.h2e[hb], (unsigned long long)ps.he[tid]);
      }
      __syncthreads();
    }
  }
}

// Top-k rows (mode 1) with 16-byte aligned rows and V % 8 == 0, one wave per
// (row, chunk): a chunk whose maximum lies below the gather threshold holds no
// candidate and is not read; the others append every element at or above it
// (the same candidates as k_filter_pass1), placed by a wave scan of the
// lanes' counts and one atomic per wave, with no barrier. Capped at 64 VGPRs
// (8 waves per SIMD, no spills): resident waves hide the load latency.
template <typename T>
__device__ __forceinline__ void gather_k_body(const Problem& P, const Work& W, int blk, int nblk) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t items = (int64_t)W.flist[0] * P.nchunk;
  const int64_t stride = (int64_t)nblk * (kPT / kWave);
  const T* base = reinterpret_cast<const T*>(P.logits);
  for (int64_t it = (int64_t)blk * (kPT / kWave) + wid; it < items; it += stride) {
    const int row = W.flist[2 + (int)(it / P.nchunk)];
    const int c = (int)(it % P.nchunk);
    const uint32_t tau = W.filt[row].tau;
    if (hs_key(W.part[(int64_t)row * P.nchunk + c].m) < tau) continue;
    const int unit = row / P.rows_per_unit;
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const int64_t c0 = (int64_t)c * kChunk;
    LaneChunk<T> r;
    lane_chunk_load<T>(base + (int64_t)row * P.row_stride, c0, P.V, lane, true, r);
    uint32_t flags = 0;
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s) {
      const bool in = lane_chunk_idx(c0, s, lane, 0) < P.V;
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k) {
        const float x = hs_div_temp(lane_chunk_val<T>(r, s, k), Tt, rT, fast);
        if (in && hs_key(x) >= tau) flags |= 1u << (s * kGroupElems + k);
      }
    }
    const int n = __popc(flags);
    int incl = n;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, kWave - 1, kWave);
    if (total == 0) continue;
    int slot0 = 0;
    if (lane == 0) slot0 = atomicAdd(&W.filt[row].ncand, total);
    int slot = __shfl(slot0, 0, kWave) + incl - n;
    uint64_t* cand = W.cand + (int64_t)row * kCand;
#pragma unroll
    for (int s = 0; s < kLaneChunkGroups; ++s) {
#pragma unroll
      for (int k = 0; k < kGroupElems; ++k) {
        if (flags & (1u << (s * kGroupElems + k))) {
          const float x = hs_div_temp(lane_chunk_val<T>(r, s, k), Tt, rT, fast);
          const uint32_t i = (uint32_t)lane_chunk_idx(c0, s, lane, k);
          if (slot < kCand) cand[slot] = ((uint64_t)hs_key(x) << 32) | (uint64_t)(0xffffffffu - i);
          ++slot;
        }
      }
    }
  }
}

// First pass of aligned rows, one launch for both lists: every workgroup takes
// its share of the top-k rows' chunks (gather_k_body), then its share of the
// top-p rows' segments (pass1_w_body), so the two kinds need no second launch
// and a workgroup done with one kind goes straight on to the other.
template <typename T>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_filter_pass1_kp(
    Problem P, Work W) {
  __shared__ PassShared ps;
  __shared__ float s_q[kPT / kWave][kQ1];
  gather_k_body<T>(P, W, (int)blockIdx.x, (int)gridDim.x);
  pass1_w_body<T>(P, W, (int)blockIdx.x, (int)gridDim.x, ps, s_q);
}

// Top-p rows, segments of chunks: the elements of the coarse boundary bucket
// b1 are appended to the candidates, and, when b1 holds more than kDirect
// elements, histogrammed into fine sub-buckets (LDS over the segment, one
// flush per segment); above kCand elements they are only histogrammed.
template <typename T>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_filter_pass2(
    Problem P, Work W) {
  __shared__ PassShared ps;
  const int tid = threadIdx.x;
  const int rows = P.units * P.rows_per_unit;
  const SegPlan sp = seg_plan(P, W.flist[1], (int)gridDim.x);  // top-p rows only
  for (int it = blockIdx.x; it < sp.items; it += gridDim.x) {
    const int ri = it / sp.nseg;
    const int row = W.flist[2 + rows + ri];
    const int unit = row / P.rows_per_unit;
    if (filter_mode(P, unit) != 2) continue;
    const FilterScratch& f = W.filt[row];
    const int seg = it - ri * sp.nseg;
    const int b1 = f.b1;
    if (b1 < 0) continue;
    const uint32_t c1 = f.c1;
    const bool fine = c1 > kDirect;  // workgroup-uniform
    // a refined bucket that fits the candidate list is also listed whole: the
    // row filter then picks the fine boundary sub-bucket out of the list
    const bool listed = c1 <= (uint32_t)kCand;
    if (fine) {
      ps.hm[tid] = 0ull;
      ps.he[tid] = 0ull;
      ps.hc[tid] = 0u;
      __syncthreads();
    }
    int c_lo, c_hi;
    seg_chunks(sp, seg, c_lo, c_hi);
    const float M = f.m, S = f.s;
    const float Tt = P.temps[unit];
    const float rT = 1.0f / Tt;
    const bool fast = hs_rcp_ok(Tt);
    const T* rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(rp) & 15u) == 0);
    const float rS = 1.0f / S;
    const bool fastS = hs_rcp_ok(S);
    const float rlo = f.rlo, rhi = f.rhi;  // coarse bucket b1 <=> rlo <= logit < rhi
    for (int c = c_lo; c < c_hi; ++c) {
      const int64_t i0 = chunk_elem(c, tid, 0);
      float x[8];
      load8<T>(rp, i0, P.V, vec_ok, x);
      const bool full = i0 + 8 <= P.V;
      uint32_t key[8], flags = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        key[k] = 0;
        if (!(x[k] >= rlo && x[k] < rhi) || !(full || i0 + k < P.V)) continue;
        const float xv = hs_div_temp(x[k], Tt, rT, fast);
        if (listed) {
          key[k] = hs_key(xv);
          flags |= 1u << k;
        }
        if (fine) {
          const int b = fine_bucket(xv, M, b1);
          const float e = hs_exp(xv - M);
          atomicAdd(&ps.hc[b], 1u);
          const uint64_t mm = hs_fx44(hs_div_temp(e, S, rS, fastS));
          const uint64_t em = hs_fx44(e);
          if (mm) atomicAdd((unsigned long long*)&ps.hm[b], (unsigned long long)mm);
          if (em) atomicAdd((unsigned long long*)&ps.he[b], (unsigned long long)em);
        }
      }
      if (listed) wave_append_cands(W, row, key, flags, i0);
    }
    if (fine) {
      __syncthreads();
      const int64_t hb = (int64_t)row * kCB + tid;
      if (ps.hc[tid]) {
        atomicAdd(&W.h2c[hb], ps.hc[tid]);
        if (ps.hm[tid]) atomicAdd((unsigned long long*)&W.h2m[hb], (unsigned long long)ps.hm[tid]);
        if (ps.he[tid]) atomicAdd((unsigned long long*)&W.h2e[hb], (unsigned long long)ps.he[tid]);
      }
      __syncthreads();
    }
  }
}

// Refined top-p rows, segments of chunks: appends the elements of fine
// sub-bucket b2 of coarse bucket b1 (no LDS, no barrier).
// Copies the row's n candidates from the workspace into sm.cand.
__device__ __forceinline__ void load_cands(const Work& W, int row, int n, FilterSmem& sm) {
  const uint64_t* src = W.cand + (int64_t)row * kCand;
  for (int i = threadIdx.x; i < n; i += kFT) sm.cand[i] = src[i];
  __syncthreads();
}

// Keeps the n candidates in LDS whose value lies in fine sub-bucket b2 of
// coarse bucket b1 (kFT threads; order not kept, the list is sorted next).
// The key -> value map is exact, so this selects the elements of fine bucket
// b2, as listing them from the row would.
__device__ __forceinline__ int keep_fine_bucket(FilterSmem& sm, int n, float M, int b1, int b2) {
  constexpr int kPer = kCand / kFT;
  uint64_t c[kPer];
  uint32_t flags = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = threadIdx.x + k * kFT;
    c[k] = i < n ? sm.cand[i] : 0ull;
    if (i < n && fine_bucket(hs_unkey(cand_key(c[k])), M, b1) == b2) flags |= 1u << k;
  }
  uint64_t total;
  const uint64_t off = block_excl_scan((uint64_t)__popc(flags), sm.wsum, &total);
  __syncthreads();  // every read of the list precedes the writes below
  int slot = (int)off;
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (flags & (1u << k)) sm.cand[slot++] = c[k];
  __syncthreads();
  return (int)total;
}

// Top-p boundary of a mode-2 row from its histograms and candidates (kFT
// threads). Returns false when the candidates overflowed (radix fallback).
struct TopP {
  bool all;
  int64_t kept;
  uint32_t bkey;
  int64_t bidx;
  uint64_t sb_fx;
};

// What the histogram passes leave for a mode-2 row: the coarse boundary
// bucket b1 (-1: the row never reaches p, -2: the row filter streams the row)
// and its element count c1, the fine boundary bucket b2 (-1: not refined),
// the count / mass / e-mass of the elements before the boundary, and the
// number of candidates listed. Workgroup-uniform.
struct TopPState {
  int b1;
  uint32_t c1;
  int b2;
  uint64_t ac, am, ae;
  int n;
};

// The state the chunk-parallel passes left in the workspace.
__device__ __forceinline__ TopPState top_p_state_of(const Work& W, int row) {
  const FilterScratch& f = W.filt[row];
  TopPState h;
  h.b1 = f.b1;
  h.c1 = h.b1 >= 0 ? W.h1c[(int64_t)row * kCB + h.b1] : 0u;
  h.b2 = -1;  // the row filter resolves the fine boundary bucket
  h.ac = f.ac;
  h.am = f.am;
  h.ae = f.ae;
  h.n = f.ncand;
  return h;
}

// 1: the boundary is found from the candidates, 0: the whole row is kept,
// -1: the row filter's radix path must decide.
__device__ __forceinline__ int top_p_usable(const TopPState& h) {
  if (h.b1 == -2) return -1;
  if (h.b1 < 0) return 0;
  if (h.c1 > kDirect && h.b2 < 0) return -1;
  if (h.n > kCand || h.n <= 0) return -1;
  return 1;
}

// top_p_usable(h) == 1 and the h.n candidates in sm.cand (unsorted).
__device__ __forceinline__ bool top_p_from_cands(FilterSmem& sm, float M, float sA, uint64_t theta,
                                                 const TopPState& h, TopP& out) {
  const int b1 = h.b1;
  const uint32_t c1 = h.c1;
  const uint64_t ac = h.ac, am = h.am, ae = h.ae;
  int n = h.n;
  if (c1 > kDirect && c1 <= (uint32_t)kCand) {
    // pass 2 listed the whole coarse bucket: keep its fine boundary sub-bucket
    n = keep_fine_bucket(sm, n, M, b1, h.b2);
    if (n <= 0) return false;
  }
  (void)pad_sort(sm, n);
  int j;
  uint64_t ej;  // e-mass of the bucket's ranks before j
  if (n <= 256) {
    wave_scan_cands(sm, n, M, sA, am, theta, 0);
    j = sm.i32v[1];
    ej = sm.u64v[1];
  } else {
    scan_bucket(sm, n, M, sA, theta - am);
    j = sm.i32v[1];
    ej = j > 0 ? sm.u.sc.scane[j - 1] : 0ull;
  }
  if (ac == 0 && j == 0) {  // rank 0 is always kept
    j = 1;
    ej = hs_fx44(hs_exp(hs_unkey(cand_key(sm.cand[0])) - M));
  }
  out.all = false;
  out.kept = (int64_t)(ac + j);
  out.sb_fx = ae + ej;
  if (j > 0) {
    out.bkey = cand_key(sm.cand[j - 1]);
    out.bidx = cand_idx(sm.cand[j - 1]);
  } else {
    out.bkey = cand_key(sm.cand[0]);  // keep exactly the keys above the bucket
    out.bidx = -1;
  }
  __syncthreads();
  return true;
}

// The row filter proper (kFT threads, one row): the kept set of the row's
// top-k / top-p and its normaliser, written to W.desc[row] (and row_stats),
// from the candidates and histograms the chunk-parallel passes left in the
// workspace. D0 is the row fold (max and normaliser over the whole row).
template <typename T>
__device__ __forceinline__ void row_filter_body(const Problem& P, const Work& W, int row,
                                                float* row_stats, FilterSmem& sm,
                                                const RowDesc& D0) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int unit = row / P.rows_per_unit;
  const int V = P.V;
  const int kk = P.top_ks[unit];
  const float pp = P.top_ps[unit];
  const int64_t keff = (kk > 0 && kk < V) ? (int64_t)kk : (int64_t)V;
  const bool k_on = keff < V;
  const bool p_on = pp < 1.0f;

  if (!(k_on || p_on) && tid == 0) {
    W.desc[row] = D0;
    if (row_stats) {
      row_stats[2 * (int64_t)row] = D0.m;
      row_stats[2 * (int64_t)row + 1] = D0.s;
    }
  }
  if (k_on || p_on) {
    RowDesc D = D0;
    RowCtx<T> C;
    C.rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    C.vec_ok = ((reinterpret_cast<uintptr_t>(C.rp) & 15u) == 0);
    C.V = V;
    C.Tt = P.temps[unit];
    C.rt = 1.0f / C.Tt;
    C.fast = hs_rcp_ok(C.Tt);
    C.M = D.m;
    C.a_all = true;
    C.a_key = 0u;
    C.a_idx = 0x7fffffff;

    // ---- stage 1: top-k boundary ------------------------------------------
    bool cand_ready = false;  // sm.cand holds the sorted A (first nA entries)
    int64_t nA = V;
    int n2 = 0;
    int path = 0;
    const int mode = filter_mode(P, unit);
    if (mode == 1) {
      // candidates at or above the keff-th largest chunk maximum (k_filter_pass1)
      const int n = W.filt[row].ncand;
      if (n <= kCand) {
        load_cands(W, row, n, sm);
        n2 = pad_sort(sm, n);
        const uint64_t bnd = sm.cand[keff - 1];
        C.a_all = false;
        C.a_key = cand_key(bnd);
        C.a_idx = cand_idx(bnd);
        cand_ready = true;
        path = 1;
      }
    }
    if (k_on && !cand_ready) {
      uint32_t prefix = 0;
      uint64_t above = 0, cnt_b = 0;
      bool done = false;
      for (int lvl = 0; lvl < 4 && !done; ++lvl) {
        hist_pass<T, false>(C, sm, lvl, prefix, 1.0f);
        if (wid == 0) {
          int b;
          uint64_t ab;
          {
            uint64_t wv[4];
            uint64_t s = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              wv[j] = sm.hc[255 - 4 * lane - j];
              s += wv[j];
            }
            uint64_t incl = wave_incl_scan_u64(s, lane);
            uint64_t m = __ballot(above + incl >= (uint64_t)keff);
            b = -1;
            ab = 0;
            if (m) {
              int l = __ffsll((long long)m) - 1;
              if (lane == l) {
                uint64_t acc = above + incl - s;
                for (int j = 0; j < 4; ++j) {
                  if (acc + wv[j] >= (uint64_t)keff) {
                    b = 255 - 4 * lane - j;
                    ab = acc;
                    break;
                  }
                  acc += wv[j];
                }
              }
              b = __shfl(b, l, 64);
              ab = __shfl((unsigned long long)ab, l, 64);
            }
          }
          if (lane == 0) {
            sm.i32v[3] = b;
            sm.u64v[3] = ab;
          }
        }
        __syncthreads();
        const int b = sm.i32v[3];
        above = sm.u64v[3];
        cnt_b = sm.hc[b < 0 ? 0 : b];
        const int shift = 24 - 8 * lvl;
        prefix = (prefix << 8) | (uint32_t)(b < 0 ? 0 : b);
        __syncthreads();
        if (above + cnt_b <= (uint64_t)kCand) {
          // finish in LDS: all elements with key >= prefix << shift
          n2 = gather_sort<T>(C, sm, prefix << shift, (int)(above + cnt_b));
          const uint64_t bnd = sm.cand[keff - 1];
          C.a_all = false;
          C.a_key = cand_key(bnd);
          C.a_idx = cand_idx(bnd);
          cand_ready = true;
          done = true;
        } else if (above + cnt_b == (uint64_t)keff) {
          C.a_all = false;
          C.a_key = prefix << shift;
          C.a_idx = 0x7fffffff;
          done = true;
        } else if (lvl == 3) {
          // full key known; split the tie by index order
          const uint64_t need_t = (uint64_t)keff - above;
          C.a_all = false;
          C.a_key = prefix;
          C.a_idx = (need_t == cnt_b) ? 0x7fffffff : nth_tie<T>(C, sm, prefix, need_t);
          done = true;
        }
      }
      nA = keff;
    }

    // ---- normaliser over A --------------------------------------------------
    float sA = D.s_full;
    uint64_t sA_fx = 0;
    const bool wave_k = k_on && cand_ready && keff <= 256;
    if (wave_k) {
      // from the sorted candidates (first keff), one wave
      wave_scan_cands(sm, (int)keff, C.M, 1.0f, 0ull, ~0ull, (int)keff);
      sA_fx = sm.u64v[3];
      sA = hs_f32_rz_of_u64(sA_fx) * kTwoM44;
    } else if (k_on && cand_ready) {
      // from the sorted candidates (first keff)
      uint64_t s = 0;
      for (int r = tid; r < (int)keff; r += kFT)
        s += hs_fx44(hs_exp(hs_unkey(cand_key(sm.cand[r])) - C.M));
      sA_fx = block_sum(s, sm.wsum);
      sA = hs_f32_rz_of_u64(sA_fx) * kTwoM44;
    } else if (k_on) {
      uint64_t s = 0;
      stream_row(C, [&](float raw, int64_t i) {
        const float x = C.div(raw);
        if (C.inA(hs_key(x), i)) s += hs_fx44(hs_exp(x - C.M));
      });
      sA_fx = block_sum(s, sm.wsum);
      sA = hs_f32_rz_of_u64(sA_fx) * kTwoM44;
    }

    // ---- stage 2: top-p -----------------------------------------------------
    uint32_t bkey = C.a_key;
    int64_t bidx = C.a_idx;
    bool ball = C.a_all;
    float sB = sA;
    int64_t kept = nA;
    if (p_on) {
      if (tid == 0) sm.u64v[4] = mass_threshold(pp);
      __syncthreads();
      const uint64_t theta = sm.u64v[4];
      if (wave_k) {
        wave_scan_cands(sm, (int)keff, C.M, sA, 0ull, theta, 0);
        int K = sm.i32v[1];  // first rank whose cumulative sum reaches p: not kept
        uint64_t eK = sm.u64v[1];
        if (K == 0) {  // rank 0 is always kept
          K = 1;
          eK = hs_fx44(hs_exp(hs_unkey(cand_key(sm.cand[0])) - C.M));
        }
        kept = K;
        sB = (K == keff) ? sA : hs_f32_rz_of_u64(eK) * kTwoM44;
        ball = false;
        bkey = cand_key(sm.cand[K - 1]);
        bidx = cand_idx(sm.cand[K - 1]);
      } else if (cand_ready) {
        lds_top_p(sm, (int)nA, C.M, sA, true, theta, n2);
        kept = sm.i32v[2];
        sB = hs_f32_rz_of_u64(sm.u64v[1]) * kTwoM44;
        ball = false;
        bkey = cand_key(sm.u64v[2]);
        bidx = cand_idx(sm.u64v[2]);
      } else {
        bool done = false;
        if (mode == 2) {
          // top-p alone: boundary from the chunk-parallel histograms + candidates
          TopPState h = top_p_state_of(W, row);
          bool in_lds = false;
          if (h.b1 >= 0 && h.c1 > kDirect) {
            // the fine sub-bucket of b1 where the cumulative mass reaches p, from
            // the second pass's fine histogram (threads >= kCB hold nothing)
            const int64_t hb = (int64_t)row * kCB + tid;
            uint64_t fc = 0, fm = 0, fe = 0;
            if (tid < kCB) {
              fc = W.h2c[hb];
              fm = W.h2m[hb];
              fe = W.h2e[hb];
            }
            const Crossing cf =
                find_crossing<kFT>(fc, fm, fe, h.am, theta, sm.wsum, &sm.i32v[4], &sm.u64v[5]);
            h.b2 = cf.b;
            if (cf.b >= 0) {
              h.ac += cf.c;
              h.am = cf.m;  // includes the base
              h.ae += cf.e;
            }
            if (cf.b >= 0 && h.c1 > (uint32_t)kCand) {
              // more elements in b1 than the list holds (the second pass listed
              // none): this workgroup lists those of the fine bucket b2 itself
              const int b1 = h.b1, b2 = cf.b;
              if (wid == 0) {
                auto at_most = [&](float r, int fb) {
                  const float x = C.div(r);
                  const int cb = coarse_bucket(x, C.M);
                  return cb < b1 || (cb == b1 && fine_bucket(x, C.M, b1) <= fb);
                };
                // logits of fine bucket b2 of b1: [flo, fhi)
                const float flo = raw_threshold([&](float r) { return at_most(r, b2); });
                const float fhi = raw_threshold([&](float r) { return at_most(r, b2 - 1); });
                if (lane == 0) {
                  sm.i32v[5] = __float_as_int(flo);
                  sm.i32v[6] = __float_as_int(fhi);
                  sm.i32v[0] = 0;
                }
              }
              __syncthreads();
              const float flo = __int_as_float(sm.i32v[5]), fhi = __int_as_float(sm.i32v[6]);
              stream_row(C, [&](float raw, int64_t i) {
                if (raw >= flo && raw < fhi) {
                  const int slot = atomicAdd(&sm.i32v[0], 1);
                  if (slot < kCand)
                    sm.cand[slot] = ((uint64_t)hs_key(C.div(raw)) << 32) |
                                    (uint64_t)(0xffffffffu - (uint32_t)i);
                }
              });
              __syncthreads();
              h.n = sm.i32v[0];
              in_lds = true;
            }
          }
          const int use = top_p_usable(h);
          if (use > 0 && !in_lds) load_cands(W, row, h.n, sm);
          TopP tpr;
          if (use == 0) tpr.all = true;
          if (use == 0 || (use > 0 && top_p_from_cands(sm, C.M, sA, theta, h, tpr))) {
            const TopP& tp = tpr;
            if (tp.all) {
              ball = true;
              kept = V;
              sB = sA;
            } else {
              kept = tp.kept;
              bkey = tp.bkey;
              bidx = tp.bidx;
              ball = (kept == V);
              sB = ball ? sA : hs_f32_rz_of_u64(tp.sb_fx) * kTwoM44;
            }
            done = true;
            path = 2;
          }
        }
        uint32_t prefix = 0;
        uint64_t above_m = 0, above_e = 0, above_c = 0;
        for (int lvl = 0; lvl < 4 && !done; ++lvl) {
          hist_pass<T, true>(C, sm, lvl, prefix, sA);
          if (wid == 0) {
            int b = -1;
            uint64_t ab = 0;
            uint64_t wv[4];
            uint64_t s = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              wv[j] = sm.hm[255 - 4 * lane - j];
              s += wv[j];
            }
            uint64_t incl = wave_incl_scan_u64(s, lane);
            uint64_t m = __ballot(above_m + incl >= theta);
            if (m) {
              int l = __ffsll((long long)m) - 1;
              if (lane == l) {
                uint64_t acc = above_m + incl - s;
                for (int j = 0; j < 4; ++j) {
                  if (acc + wv[j] >= theta) {
                    b = 255 - 4 * lane - j;
                    ab = acc;
                    break;
                  }
                  acc += wv[j];
                }
              }
              b = __shfl(b, l, 64);
              ab = __shfl((unsigned long long)ab, l, 64);
            }
            // counts and e-mass of the buckets above b
            uint64_t ce = 0, cc = 0;
            if (b >= 0) {
              for (int bb = b + 1 + lane; bb < 256; bb += 64) {
                ce += sm.he[bb];
                cc += sm.hc[bb];
              }
            }
            ce = wave_sum_u64(ce);
            cc = wave_sum_u64(cc);
            if (lane == 0) {
              sm.i32v[3] = b;
              sm.u64v[3] = ab;
              sm.u64v[5] = ce;
              sm.u64v[6] = cc;
            }
          }
          __syncthreads();
          const int b = sm.i32v[3];
          if (b < 0) {
            // the whole of A stays below the threshold: keep A
            done = true;
            __syncthreads();
            break;
          }
          above_m = sm.u64v[3];
          above_e += sm.u64v[5];
          above_c += sm.u64v[6];
          const uint64_t cnt_b = sm.hc[b];
          const int shift = 24 - 8 * lvl;
          prefix = (prefix << 8) | (uint32_t)b;
          __syncthreads();
          if (above_c + cnt_b <= (uint64_t)kCand) {
            n2 = gather_sort<T>(C, sm, prefix << shift, (int)(above_c + cnt_b));
            lds_top_p(sm, (int)(above_c + cnt_b), C.M, sA, true, theta, n2);
            kept = sm.i32v[2];
            sB = hs_f32_rz_of_u64(sm.u64v[1]) * kTwoM44;
            ball = false;
            bkey = cand_key(sm.u64v[2]);
            bidx = cand_idx(sm.u64v[2]);
            done = true;
          } else if (lvl == 3) {
            // all ties at key `prefix` share one mass
            const float xs = hs_unkey(prefix);
            const float es = hs_exp(xs - C.M);
            const uint64_t ms = hs_fx44(es / sA);
            const uint64_t need = theta - above_m;
            uint64_t t = (ms > 0) ? (need + ms - 1) / ms : cnt_b;
            if (t < 1) t = 1;
            uint64_t kt = t - 1;
            if (above_c == 0 && kt == 0) kt = 1;
            if (kt > cnt_b) kt = cnt_b;
            ball = false;
            bkey = prefix;
            if (kt == 0) bidx = -1;
            else if (kt == cnt_b) bidx = (!C.a_all && C.a_key == prefix) ? C.a_idx : 0x7fffffff;
            else bidx = nth_tie<T>(C, sm, prefix, kt);
            kept = (int64_t)(above_c + kt);
            sB = hs_f32_rz_of_u64(above_e + kt * hs_fx44(es)) * kTwoM44;
            done = true;
          }
        }
      }
    }

    if (tid == 0) {
      RowDesc d = D;
      d.all = ball ? 1 : 0;
      d.tkey = bkey;
      d.tidx = (int32_t)bidx;
      d.s = sB;
      W.desc[row] = d;
      W.filt[row].kept = (int32_t)kept;
      W.filt[row].path = path;
      if (row_stats) {
        row_stats[2 * (int64_t)row] = d.m;
        row_stats[2 * (int64_t)row + 1] = sB;
      }
    }
  }
}

// One workgroup per row, after the chunk-parallel passes: the row fold of
// k_filter_plan1 from the workspace, then the row filter proper.
template <typename T>
__global__ __launch_bounds__(kFT) void k_row_filter(Problem P, Work W, float* row_stats) {
  __shared__ FilterSmem sm;
  const int row = blockIdx.x;
  RowDesc d;
  d.m = W.filt[row].m;
  d.s = W.filt[row].s;
  d.tkey = 0u;
  d.tidx = 0x7fffffff;
  d.all = 1;
  d.token = -1;
  d.s_full = d.s;
  d.pad = 0;
  row_filter_body<T>(P, W, row, row_stats, sm, d);
}

template <typename T>
int launch_filter(const Problem& P, const Work& W, float* row_stats, bool wave,
                  hipStream_t stream) {
  const int rows = P.units * P.rows_per_unit;
  const int64_t items = (int64_t)rows * P.nchunk;
  // passes 1-3: the 8 workgroups per CU that fit at once on 256 CUs, each
  // taking a segment of chunks of one row
  const int grid1 = (int)(items < 2048 ? items : 2048);
  hipLaunchKernelGGL(k_filter_plan1, dim3(rows), dim3(kPT), 0, stream, P, W);
  if (wave && rows >= 32) {
    // top-k rows by the wave-per-chunk gather (at most the 8 workgroups per CU
    // that fit at once on 256 CUs), top-p rows by the histogram pass; below 32
    // rows one launch with a workgroup per chunk is shorter
    hipLaunchKernelGGL(k_filter_pass1_kp<T>, dim3(grid1), dim3(kPT), 0, stream, P, W);
  } else {
    hipLaunchKernelGGL(k_filter_pass1<T>, dim3(grid1), dim3(kPT), 0, stream, P, W, 0);
  }
  hipLaunchKernelGGL(k_filter_plan2, dim3(rows), dim3(kPT), 0, stream, P, W);
  if (wave)
    hipLaunchKernelGGL(k_filter_pass2_w<T>, dim3(grid1), dim3(kPT), 0, stream, P, W);
  else
    hipLaunchKernelGGL(k_filter_pass2<T>, dim3(grid1), dim3(kPT), 0, stream, P, W);
  hipLaunchKernelGGL(k_row_filter<T>, dim3(rows), dim3(kFT), 0, stream, P, W, row_stats);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

template int launch_filter<float>(const Problem&, const Work&, float*, bool, hipStream_t);
template int launch_filter<uint16_t>(const Problem&, const Work&, float*, bool, hipStream_t);


}  // namespace hs
