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
// One 512-thread workgroup owns one row (re-reads hit L2/MALL):
//   1. top-k: 8-bit radix passes over the order key, histogramming counts in
//      LDS; as soon as the candidates above the current bucket fit in LDS
//      (<= 4096) they are gathered and bitonic-sorted, which finishes the
//      selection in LDS (typically after one pass).
//   2. top-p: the same scheme with exact mass histograms (u64 LDS atomics);
//      ties at the final key are resolved in closed form (equal keys have
//      equal mass) plus one index-ordered pass when a tie is split.
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
  uint64_t scanm[kCand];
  uint64_t scane[kCand];
  uint32_t hc[256];
  uint64_t hm[256];
  uint64_t he[256];
  uint64_t wsum[kFW];
  uint64_t wsum2[kFW];
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
__device__ uint64_t mass_threshold(float p) {
  const float target = p * kTwo44;
  if (!(target > 0.0f)) return 0ull;
  uint64_t lo = 0, hi = (1ull << 62);
  while (lo < hi) {
    uint64_t mid = lo + ((hi - lo) >> 1);
    if (hs_f32_of_u64(mid) >= target) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

template <typename T>
struct RowCtx {
  const T* rp;
  bool vec_ok;
  int V;
  float Tt;
  float M;
  // membership in the kept set A of an earlier stage
  bool a_all;
  uint32_t a_key;
  int64_t a_idx;
  __device__ bool inA(uint32_t key, int64_t i) const {
    return a_all || key > a_key || (key == a_key && i <= a_idx);
  }
};

// Histogram pass: counts (and masses when `mass`) of elements in A whose key
// prefix above `shift + 8` bits equals `prefix`, bucketed by the next 8 bits.
template <typename T, bool kMass>
__device__ void hist_pass(const RowCtx<T>& C, FilterSmem& sm, int lvl, uint32_t prefix,
                          float sA) {
  const int tid = threadIdx.x;
  for (int b = tid; b < 256; b += kFT) {
    sm.hc[b] = 0u;
    sm.hm[b] = 0ull;
    sm.he[b] = 0ull;
  }
  __syncthreads();
  const int shift = 24 - 8 * lvl;
  for (int64_t base = (int64_t)tid * 8; base < C.V; base += (int64_t)kFT * 8) {
    float v[8];
    load8<T>(C.rp, base, C.V, C.vec_ok, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = base + k;
      if (i >= C.V) continue;
      const float x = hs_div_t(v[k], C.Tt);
      const uint32_t key = hs_key(x);
      if (lvl > 0 && (key >> (shift + 8)) != prefix) continue;
      if (!C.inA(key, i)) continue;
      const uint32_t b = (key >> shift) & 255u;
      atomicAdd(&sm.hc[b], 1u);
      if (kMass) {
        const float e = hs_exp(x - C.M);
        const uint64_t em = hs_fx44(e);
        const uint64_t mm = hs_fx44(e / sA);
        if (mm) atomicAdd((unsigned long long*)&sm.hm[b], (unsigned long long)mm);
        if (em) atomicAdd((unsigned long long*)&sm.he[b], (unsigned long long)em);
      }
    }
  }
  __syncthreads();
}

// Gathers every element of A with key >= lo_key into sm.cand as
// (key << 32) | (0xffffffff - index) and sorts them descending (rank order).
// Returns the padded power-of-two size; sm.i32v[0] holds the count.
template <typename T>
__device__ int gather_sort(const RowCtx<T>& C, FilterSmem& sm, uint32_t lo_key, int expect) {
  const int tid = threadIdx.x;
  int n2 = 1;
  while (n2 < expect) n2 <<= 1;
  if (n2 < 2) n2 = 2;
  for (int i = tid; i < n2; i += kFT) sm.cand[i] = 0ull;
  if (tid == 0) sm.i32v[0] = 0;
  __syncthreads();
  for (int64_t base = (int64_t)tid * 8; base < C.V; base += (int64_t)kFT * 8) {
    float v[8];
    load8<T>(C.rp, base, C.V, C.vec_ok, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = base + k;
      if (i >= C.V) continue;
      const uint32_t key = hs_key(hs_div_t(v[k], C.Tt));
      if (key < lo_key || !C.inA(key, i)) continue;
      const int slot = atomicAdd(&sm.i32v[0], 1);
      if (slot < kCand)
        sm.cand[slot] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
    }
  }
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
__device__ int64_t nth_tie(const RowCtx<T>& C, FilterSmem& sm, uint32_t key0, uint64_t n) {
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
        const uint32_t key = hs_key(hs_div_t(v[k], C.Tt));
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
__device__ void lds_top_p(FilterSmem& sm, int n, float M, float sA, bool p_on, uint64_t theta,
                          int n2) {
  const int tid = threadIdx.x;
  // per-thread block of 8 consecutive ranks
  uint64_t me[8], mm[8];
  uint64_t se = 0, smm = 0;
  const int r0 = tid * 8;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
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
    for (int k = 0; k < 8; ++k) {
      const int r = r0 + k;
      ae += me[k];
      am += mm[k];
      if (r < kCand) {
        sm.scane[r] = ae;
        sm.scanm[r] = am;
      }
    }
  }
  if (tid == 0) sm.i32v[1] = n;  // first rank with cumsum >= theta (n if none)
  __syncthreads();
  if (p_on) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r = r0 + k;
      if (r < n && sm.scanm[r] >= theta) {
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
    sm.u64v[1] = sm.scane[K - 1];  // S_B
    sm.u64v[2] = sm.cand[K - 1];   // boundary
  }
  __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(kFT) void k_row_filter(Problem P, Work W, float* row_stats) {
  __shared__ FilterSmem sm;
  __shared__ RowDesc s_fold;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int unit = row / P.rows_per_unit;
  const int V = P.V;
  const int kk = P.top_ks[unit];
  const float pp = P.top_ps[unit];
  const int64_t keff = (kk > 0 && kk < V) ? (int64_t)kk : (int64_t)V;
  const bool k_on = keff < V;
  const bool p_on = pp < 1.0f;

  if (wid == 0) {
    const RowDesc d = fold_row_desc(P, W, row, lane);
    if (lane == 0) s_fold = d;
  }
  __syncthreads();
  if (!(k_on || p_on) && tid == 0) {
    W.desc[row] = s_fold;
    if (row_stats) {
      row_stats[2 * (int64_t)row] = s_fold.m;
      row_stats[2 * (int64_t)row + 1] = s_fold.s;
    }
  }
  if (k_on || p_on) {
    RowDesc D = s_fold;
    RowCtx<T> C;
    C.rp = reinterpret_cast<const T*>(P.logits) + (int64_t)row * P.row_stride;
    C.vec_ok = ((reinterpret_cast<uintptr_t>(C.rp) & 15u) == 0);
    C.V = V;
    C.Tt = P.temps[unit];
    C.M = D.m;
    C.a_all = true;
    C.a_key = 0u;
    C.a_idx = 0x7fffffff;

    // ---- stage 1: top-k boundary ------------------------------------------
    bool cand_ready = false;  // sm.cand holds the sorted A (first nA entries)
    int64_t nA = V;
    int n2 = 0;
    if (k_on) {
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
    if (k_on && cand_ready) {
      // from the sorted candidates (first keff)
      uint64_t s = 0;
      for (int r = tid; r < (int)keff; r += kFT)
        s += hs_fx44(hs_exp(hs_unkey(cand_key(sm.cand[r])) - C.M));
      sA_fx = block_sum(s, sm.wsum);
      sA = hs_f32_rz_of_u64(sA_fx) * kTwoM44;
    } else if (k_on) {
      uint64_t s = 0;
      for (int64_t base = (int64_t)tid * 8; base < V; base += (int64_t)kFT * 8) {
        float v[8];
        load8<T>(C.rp, base, V, C.vec_ok, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int64_t i = base + k;
          if (i >= V) continue;
          const float x = hs_div_t(v[k], C.Tt);
          if (C.inA(hs_key(x), i)) s += hs_fx44(hs_exp(x - C.M));
        }
      }
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
      if (cand_ready) {
        lds_top_p(sm, (int)nA, C.M, sA, true, theta, n2);
        kept = sm.i32v[2];
        sB = hs_f32_rz_of_u64(sm.u64v[1]) * kTwoM44;
        ball = false;
        bkey = cand_key(sm.u64v[2]);
        bidx = cand_idx(sm.u64v[2]);
      } else {
        uint32_t prefix = 0;
        uint64_t above_m = 0, above_e = 0, above_c = 0;
        bool done = false;
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
      FilterScratch fs;
      fs.kept = (int32_t)kept;
      fs.path = cand_ready ? 1 : 0;
      fs.pad[0] = fs.pad[1] = 0;
      W.filt[row] = fs;
      if (row_stats) {
        row_stats[2 * (int64_t)row] = d.m;
        row_stats[2 * (int64_t)row + 1] = sB;
      }
    }
  }
}

template <typename T>
int launch_filter(const Problem& P, const Work& W, float* row_stats, hipStream_t stream) {
  const int rows = P.units * P.rows_per_unit;
  hipLaunchKernelGGL(k_row_filter<T>, dim3(rows), dim3(kFT), 0, stream, P, W, row_stats);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

template int launch_filter<float>(const Problem&, const Work&, float*, hipStream_t);
template int launch_filter<uint16_t>(const Problem&, const Work&, float*, hipStream_t);

}  // namespace hs
