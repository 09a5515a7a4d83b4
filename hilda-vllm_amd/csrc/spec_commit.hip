// Accept/rollback bookkeeping of a speculative step on the device (gfx950).
//
// Replaces the host-side bookkeeping of LLMEngine.step's spec block,
// mini_vllm/engine/llm_engine.py:104-195, the BlockManager operations it uses
// (block_manager.py:20-115), the verify staging of run_verify
// (model_runner.py:339-362) and the rejected-slot cleanup
// (model_runner.py:439-481). The state (lengths, block tables, token history,
// FIFO free list, reference counts) stays resident in HBM.
//
// Every kernel here is a single workgroup of 1024 threads: the work is a few
// integers per sequence, and the FIFO order of freed blocks depends on
// sequence order, which one workgroup resolves with block-wide scans instead
// of atomics whose outcome would depend on timing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"

namespace hs {

constexpr int kCT = 1024;  // threads of every bookkeeping kernel
constexpr int kCW = kCT / 64;

// exclusive scan over the workgroup of one int per thread; returns the total
__device__ int cscan_excl(int v, int* s_w, int* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int w = __shfl_up(incl, o, 64);
    if (lane >= o) incl += w;
  }
  if (lane == 63) s_w[wid] = incl;
  __syncthreads();
  int off = 0, tot = 0;
  for (int w = 0; w < kCW; ++w) {
    const int x = s_w[w];
    if (w < wid) off += x;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

__device__ __forceinline__ int ring_at(const hs_spec_state& s, int pos) {
  return s.free_ring[pos % s.num_blocks];
}

// ---------------------------------------------------------------------------
// pre-allocation: llm_engine.py:111-128
// ---------------------------------------------------------------------------
struct PreallocLds {
  int need[kCT], off[kCT], ok[kCT];
  int take;
};

__device__ void prealloc_body(const hs_spec_state& s, int gamma, int32_t* eligible,
                              int32_t* status, PreallocLds& L) {
  int* s_need = L.need;
  int* s_off = L.off;
  int* s_ok = L.ok;
  int& s_take = L.take;
  const int tid = threadIdx.x;
  for (int base = 0; base < s.B; base += kCT) {
    const int b = base + tid;
    int need = 0;
    if (b < s.B) {
      const int len = s.context_lens[b];
      const int cur = s.num_seq_blocks[b];
      const int needed = (len + gamma + 1 + s.block_size - 1) / s.block_size;
      need = s.finished[b] ? -1 : needed - cur;  // -1: not a candidate
      if (need > 0 && needed > s.W) need = -2;    // would overflow the table row
    }
    s_need[tid] = need;
    __syncthreads();
    // the free-count test depends on the blocks taken by earlier sequences
    if (tid == 0) {
      int avail = s.free_hdr[1];
      int taken = 0;
      const int cnt = (s.B - base < kCT) ? s.B - base : kCT;
      for (int i = 0; i < cnt; ++i) {
        const int nd = s_need[i];
        int ok = 0;
        if (nd == -2) ok = 0;
        else if (nd < 0) ok = 0;
        else if (nd > 0 && avail < nd) ok = 0;
        else {
          ok = 1;
          if (nd > 0) {
            s_off[i] = taken;
            taken += nd;
            avail -= nd;
          }
        }
        s_ok[i] = ok;
      }
      s_take = taken;
    }
    __syncthreads();
    if (b < s.B) {
      if (eligible) eligible[b] = s_ok[tid];
      if (s_ok[tid] && need > 0) {
        const int head = s.free_hdr[0];
        const int cur = s.num_seq_blocks[b];
        for (int k = 0; k < need; ++k) {
          const int blk = ring_at(s, head + s_off[tid] + k);
          s.block_tables[(int64_t)b * s.W + cur + k] = blk;
          s.ref_count[blk] = 1;
        }
        s.num_seq_blocks[b] = cur + need;
      }
      if (need == -2 && status) *status = 1;
    }
    __syncthreads();
    if (tid == 0) {
      s.free_hdr[0] = (s.free_hdr[0] + s_take) % s.num_blocks;
      s.free_hdr[1] -= s_take;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kCT) void k_prealloc(hs_spec_state s, int gamma, int32_t* eligible,
                                                  int32_t* status) {
  __shared__ PreallocLds L;
  prealloc_body(s, gamma, eligible, status, L);
}

// ---------------------------------------------------------------------------
// verify staging: model_runner.py:339-362
// ---------------------------------------------------------------------------
// draft NULL: the draft tokens' ids (rows 1 .. gamma of each sequence) are
// left as they are (written in place by the draft steps' sampler)
__device__ void verify_prepare_body(const hs_spec_state& s, const int64_t* draft, int gamma,
                                    int64_t* input_ids, int64_t* positions,
                                    int32_t* slot_mapping, int32_t* cu_q, int32_t* cu_k,
                                    int* s_w) {
  const int tid = threadIdx.x;
  const int R = gamma + 1;
  int carry = 0;
  for (int base = 0; base < s.B; base += kCT) {
    const int b = base + tid;
    int lk = 0;
    if (b < s.B) {
      const int len = s.context_lens[b];
      lk = len + gamma;
      const int nblk = s.num_seq_blocks[b];
      for (int j = 0; j < R; ++j) {
        const int pos = len - 1 + j;
        const int bi = pos / s.block_size;
        const int slot = (bi < nblk) ? s.block_tables[(int64_t)b * s.W + bi] * s.block_size +
                                           pos % s.block_size
                                     : -1;
        const int64_t o = (int64_t)b * R + j;
        if (j == 0) input_ids[o] = s.tokens[(int64_t)b * s.T + len - 1];
        else if (draft) input_ids[o] = draft[(int64_t)b * gamma + j - 1];
        positions[o] = pos;
        slot_mapping[o] = slot;
      }
      cu_q[b] = b * R;
    }
    int total;
    const int ex = cscan_excl(lk, s_w, &total);
    if (b < s.B) cu_k[b] = carry + ex;
    carry += total;
  }
  if (tid == 0) {
    cu_q[s.B] = s.B * R;
    cu_k[s.B] = carry;
  }
}

__global__ __launch_bounds__(kCT) void k_prepare(hs_spec_state s, const int64_t* draft, int gamma,
                                                 int64_t* input_ids, int64_t* positions,
                                                 int32_t* slot_mapping, int32_t* cu_q,
                                                 int32_t* cu_k) {
  __shared__ int s_w[kCW];
  verify_prepare_body(s, draft, gamma, input_ids, positions, slot_mapping, cu_q, cu_k, s_w);
}

// draft step staging: model_runner.py:294-310 (step j feeds the previous draft
// token, or last_token for j = 0, at position len - 1 + j). With lookback, step
// 0 feeds the two last tokens (positions len-2, len-1): after a step that
// accepted every draft, the draft model never saw the last accepted draft,
// and this fills that KV slot.
__device__ void draft_prepare_body(const hs_spec_state& s, const int64_t* draft, int draft_stride,
                                   int step, int lookback, int64_t* input_ids, int64_t* positions,
                                   int32_t* slot_mapping, int32_t* cu_q, int32_t* cu_k,
                                   int* s_w) {
  const int tid = threadIdx.x;
  const int R = (step == 0 && lookback) ? 2 : 1;
  int carry = 0;
  for (int base = 0; base < s.B; base += kCT) {
    const int b = base + tid;
    int lk = 0;
    if (b < s.B) {
      const int len = s.context_lens[b];
      const int cur = len + step;
      lk = cur;
      const int nblk = s.num_seq_blocks[b];
      for (int r = 0; r < R; ++r) {
        const int back = R - 1 - r;  // 1 for the look-back row
        int64_t tok;
        if (step == 0) tok = s.tokens[(int64_t)b * s.T + (len - 1 - back >= 0 ? len - 1 - back : 0)];
        else tok = draft[(int64_t)b * draft_stride + step - 1];
        const int pos = cur - 1 - back;
        const int bi = pos / s.block_size;
        const int o = b * R + r;
        input_ids[o] = tok;
        positions[o] = pos;
        slot_mapping[o] = (pos >= 0 && bi < nblk)
                              ? s.block_tables[(int64_t)b * s.W + bi] * s.block_size +
                                    pos % s.block_size
                              : -1;
      }
      cu_q[b] = b * R;
    }
    int total;
    const int ex = cscan_excl(lk, s_w, &total);
    if (b < s.B) cu_k[b] = carry + ex;
    carry += total;
  }
  if (tid == 0) {
    cu_q[s.B] = s.B * R;
    cu_k[s.B] = carry;
  }
}

__global__ __launch_bounds__(kCT) void k_draft_prepare(hs_spec_state s, const int64_t* draft,
                                                       int draft_stride, int step, int lookback,
                                                       int64_t* input_ids, int64_t* positions,
                                                       int32_t* slot_mapping, int32_t* cu_q,
                                                       int32_t* cu_k) {
  __shared__ int s_w[kCW];
  draft_prepare_body(s, draft, draft_stride, step, lookback, input_ids, positions, slot_mapping,
                     cu_q, cu_k, s_w);
}

// ---------------------------------------------------------------------------
// commit + rollback: llm_engine.py:146-195, block_manager.py:84-92
// ---------------------------------------------------------------------------
struct CommitWs {
  int32_t* dec;     // [num_blocks] decrements in this call
  int32_t* last;    // [num_blocks] 1 + index of the last event on the block
  int32_t* ev_blk;  // [B * W] block of each release event
  int32_t* ev_free; // [B * W] 1 if the event frees its block
  int32_t* seq;     // [5 * B] per-sequence scratch
};

__device__ void commit_body(const hs_spec_state& s, int gamma, const int64_t* out_tokens,
                            const int32_t* out_len, const int32_t* eligible, int32_t* appended,
                            int32_t* dirty, int dirty_mode, const CommitWs& w, int* s_w,
                            int* s_tot) {
  const int tid = threadIdx.x;
  const int R = gamma + 1;
  int32_t* s_nblk = w.seq;             // table length at entry
  int32_t* s_ndeal = w.seq + s.B;      // blocks released by a finish in this call
  int32_t* s_ntrim = w.seq + 2 * s.B;  // blocks trimmed from the tail
  int32_t* s_odeal = w.seq + 3 * s.B;  // first event of the sequence's releases
  int32_t* s_otrim = w.seq + 4 * s.B;

  // phase 1: append tokens, stop at EOS / max_tokens, count release events
  for (int b = tid; b < s.B; b += kCT) {
    const int len0 = s.context_lens[b];
    const int nblk = s.num_seq_blocks[b];
    int len = len0, fin = s.finished[b], app = 0;
    const int n = (fin || (eligible && !eligible[b])) ? 0 : out_len[b];
    for (int j = 0; j < n && !fin; ++j) {
      const int64_t tok = out_tokens[(int64_t)b * R + j];
      if (len < s.T) s.tokens[(int64_t)b * s.T + len] = tok;
      ++len;
      ++app;
      if ((!s.ignore_eos[b] && tok == s.eos) || (len - s.num_prompt[b] == s.max_tokens[b]))
        fin = 1;
    }
    // dirty slots of rejected drafts, before the table is trimmed
    if (dirty) {
      for (int j = 0; j < R; ++j) dirty[(int64_t)b * R + j] = -1;
      if (!fin && !s.finished[b] && n > 0) {
        const int lo = dirty_mode ? len - 1 : len;
        const int hi = dirty_mode ? len0 + gamma : len0 + gamma + 1;
        int k = 0;
        for (int pos = lo; pos < hi && k < R; ++pos) {
          const int bi = pos / s.block_size;
          if (pos >= 0 && bi < nblk)
            dirty[(int64_t)b * R + k++] =
                s.block_tables[(int64_t)b * s.W + bi] * s.block_size + pos % s.block_size;
        }
      }
    }
    const int newly_finished = fin && !s.finished[b];
    s_nblk[b] = nblk;
    s_ndeal[b] = newly_finished ? nblk : 0;
    const int needed = (len + s.block_size - 1) / s.block_size;
    s_ntrim[b] = (!fin && nblk > needed) ? nblk - needed : 0;
    s.context_lens[b] = len;
    s.finished[b] = fin;
    if (appended) appended[b] = app;
  }
  __syncthreads();

  // phase 2: event offsets (deallocations first, then trims, each in sequence order)
  int carry_d = 0, carry_t = 0;
  for (int base = 0; base < s.B; base += kCT) {
    const int b = base + tid;
    const int nd = b < s.B ? s_ndeal[b] : 0;
    const int nt = b < s.B ? s_ntrim[b] : 0;
    int td, tt;
    const int od = cscan_excl(nd, s_w, &td);
    const int ot = cscan_excl(nt, s_w, &tt);
    if (b < s.B) {
      s_odeal[b] = carry_d + od;
      s_otrim[b] = carry_t + ot;
    }
    carry_d += td;
    carry_t += tt;
  }
  if (tid == 0) {
    s_tot[0] = carry_d;
    s_tot[1] = carry_t;
  }
  __syncthreads();
  const int D = s_tot[0], E = s_tot[0] + s_tot[1];

  // phase 3: enumerate events (block taken from the end of the table)
  for (int b = tid; b < s.B; b += kCT) {
    const int nblk = s_nblk[b];
    int cnt, off;
    if (s_ndeal[b] > 0) {
      cnt = s_ndeal[b];  // whole table, last block first (block_manager.py:85)
      off = s_odeal[b];
    } else {
      cnt = s_ntrim[b];  // tail blocks, popped last first (llm_engine.py:175-181)
      off = D + s_otrim[b];
    }
    for (int k = 0; k < cnt; ++k) {
      const int blk = s.block_tables[(int64_t)b * s.W + nblk - 1 - k];
      w.ev_blk[off + k] = blk;
      atomicAdd(&w.dec[blk], 1);
      atomicMax(&w.last[blk], off + k + 1);
    }
  }
  __syncthreads();
  // phase 4: the last event on a block applies all decrements of this call
  for (int e = tid; e < E; e += kCT) {
    const int blk = w.ev_blk[e];
    int fr = 0;
    if (atomicAdd(&w.last[blk], 0) == e + 1) {
      const int r = s.ref_count[blk] - atomicAdd(&w.dec[blk], 0);
      s.ref_count[blk] = r;
      fr = (r == 0);
    }
    w.ev_free[e] = fr;
  }
  __syncthreads();
  // phase 5: append freed blocks to the back of the FIFO in event order
  const int head = s.free_hdr[0];
  const int count0 = s.free_hdr[1];
  int carry = 0;
  for (int base = 0; base < E; base += kCT) {
    const int e = base + tid;
    const int f = e < E ? w.ev_free[e] : 0;
    int tot;
    const int ex = cscan_excl(f, s_w, &tot);
    if (f) s.free_ring[(head + count0 + carry + ex) % s.num_blocks] = w.ev_blk[e];
    carry += tot;
  }
  __syncthreads();
  for (int e = tid; e < E; e += kCT) {
    const int blk = w.ev_blk[e];
    w.dec[blk] = 0;
    w.last[blk] = 0;
  }
  // phase 6: shrink the tables
  for (int b = tid; b < s.B; b += kCT) {
    const int nblk = s_nblk[b];
    const int keep = s.finished[b] ? 0 : (s.context_lens[b] + s.block_size - 1) / s.block_size;
    if (keep < nblk) {
      for (int k = keep; k < nblk; ++k) s.block_tables[(int64_t)b * s.W + k] = -1;
      s.num_seq_blocks[b] = keep;
    }
  }
  if (tid == 0) s.free_hdr[1] = count0 + carry;
}

__global__ __launch_bounds__(kCT) void k_commit(hs_spec_state s, int gamma, const int64_t* out_tokens,
                                                const int32_t* out_len, const int32_t* eligible,
                                                int32_t* appended, int32_t* dirty, int dirty_mode,
                                                CommitWs w) {
  __shared__ int s_w[kCW];
  __shared__ int s_tot[2];
  commit_body(s, gamma, out_tokens, out_len, eligible, appended, dirty, dirty_mode, w, s_w,
              s_tot);
}

// The commit of a step, then the next step's pre-allocation (into eligible,
// which the commit has read), its first draft step's staging and, when v_ids
// is given, its verify staging without the draft tokens' ids, in one
// workgroup: the state each part reads is the one the previous part left
// (their writes are ordered by the workgroup barriers between them).
struct VerifyStage {
  int64_t* ids;
  int64_t* pos;
  int32_t* slots;
  int32_t* cu_q;
  int32_t* cu_k;
};
__global__ __launch_bounds__(kCT) void k_commit_next(hs_spec_state s, int gamma,
                                                     const int64_t* out_tokens,
                                                     const int32_t* out_len, int32_t* eligible,
                                                     CommitWs w, int next_gamma, int32_t* status,
                                                     int lookback, int64_t* input_ids,
                                                     int64_t* positions, int32_t* slot_mapping,
                                                     int32_t* cu_q, int32_t* cu_k, VerifyStage v) {
  __shared__ int s_w[kCW];
  __shared__ int s_tot[2];
  __shared__ PreallocLds L;
  commit_body(s, gamma, out_tokens, out_len, eligible, nullptr, nullptr, 0, w, s_w, s_tot);
  __syncthreads();
  prealloc_body(s, next_gamma, eligible, status, L);
  __syncthreads();
  draft_prepare_body(s, nullptr, 0, 0, lookback, input_ids, positions, slot_mapping, cu_q, cu_k,
                     s_w);
  if (v.ids) {
    __syncthreads();  // s_w is reused
    verify_prepare_body(s, nullptr, next_gamma, v.ids, v.pos, v.slots, v.cu_q, v.cu_k, s_w);
  }
}

// zero the K/V rows of the given slots in every (kv, layer) plane
__global__ __launch_bounds__(256) void k_zero_slots(uint8_t* cache, int64_t plane_bytes,
                                                    int planes, int64_t slot_bytes,
                                                    int64_t row_bytes, const int32_t* slots,
                                                    int nslots, int64_t plane_capacity) {
  const int64_t item = blockIdx.x;  // (plane, slot)
  const int p = (int)(item / nslots), i = (int)(item % nslots);
  if (p >= planes) return;
  const int slot = slots[i];
  if (slot < 0 || (int64_t)slot >= plane_capacity) return;
  uint8_t* row = cache + p * plane_bytes + (int64_t)slot * slot_bytes;
  for (int64_t o = threadIdx.x * 4; o < row_bytes; o += 256 * 4)
    *reinterpret_cast<uint32_t*>(row + o) = 0u;
}

}  // namespace hs

using namespace hs;

extern "C" {

static int state_ok(const hs_spec_state* s) {
  if (!s || !s->context_lens || !s->num_prompt || !s->max_tokens || !s->ignore_eos ||
      !s->finished || !s->block_tables || !s->num_seq_blocks || !s->tokens || !s->free_ring ||
      !s->free_hdr || !s->ref_count)
    return 0;
  return s->B > 0 && s->W > 0 && s->T > 0 && s->num_blocks > 0 && s->block_size > 0;
}

int hs_spec_prealloc(const hs_spec_state* state, int gamma, int32_t* eligible, int32_t* status,
                     void* stream) {
  if (!state_ok(state) || gamma < 0) return HS_ERR_INVALID;
  hipLaunchKernelGGL(k_prealloc, dim3(1), dim3(kCT), 0, reinterpret_cast<hipStream_t>(stream),
                     *state, gamma, eligible, status);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_verify_prepare(const hs_spec_state* state, const int64_t* draft_tokens, int gamma,
                      int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                      int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, void* stream) {
  if (!state_ok(state) || gamma < 0 || (gamma > 0 && !draft_tokens) || !input_ids ||
      !positions || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k)
    return HS_ERR_INVALID;
  hipLaunchKernelGGL(k_prepare, dim3(1), dim3(kCT), 0, reinterpret_cast<hipStream_t>(stream),
                     *state, draft_tokens, gamma, input_ids, positions, slot_mapping,
                     cu_seqlens_q, cu_seqlens_k);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_draft_prepare(const hs_spec_state* state, const int64_t* draft_tokens, int draft_stride,
                     int step, int lookback, int64_t* input_ids, int64_t* positions,
                     int32_t* slot_mapping, int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                     void* stream) {
  if (!state_ok(state) || step < 0 || (step > 0 && (!draft_tokens || draft_stride < step)) ||
      !input_ids || !positions || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k ||
      (lookback != 0 && lookback != 1))
    return HS_ERR_INVALID;
  hipLaunchKernelGGL(k_draft_prepare, dim3(1), dim3(kCT), 0,
                     reinterpret_cast<hipStream_t>(stream), *state, draft_tokens, draft_stride,
                     step, lookback, input_ids, positions, slot_mapping, cu_seqlens_q,
                     cu_seqlens_k);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

size_t hs_spec_commit_workspace_size(int batch, int table_width, int num_blocks) {
  if (batch <= 0 || table_width <= 0 || num_blocks <= 0) return 0;
  return sizeof(int32_t) * ((size_t)2 * num_blocks + (size_t)2 * batch * table_width +
                            (size_t)5 * batch);
}

int hs_spec_commit(const hs_spec_state* state, int gamma, const int32_t* num_accepted,
                   const int64_t* out_tokens, const int32_t* out_len, const int32_t* eligible,
                   int32_t* appended, int32_t* dirty_slots, int dirty_mode, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (!state_ok(state) || gamma < 0 || !out_tokens || !out_len || !workspace)
    return HS_ERR_INVALID;
  if (dirty_mode != 0 && dirty_mode != 1) return HS_ERR_INVALID;
  if (workspace_bytes < hs_spec_commit_workspace_size(state->B, state->W, state->num_blocks))
    return HS_ERR_WORKSPACE;
  int32_t* p = static_cast<int32_t*>(workspace);
  CommitWs w;
  w.dec = p;
  w.last = p + state->num_blocks;
  w.ev_blk = p + 2 * (size_t)state->num_blocks;
  w.ev_free = w.ev_blk + (size_t)state->B * state->W;
  w.seq = w.ev_free + (size_t)state->B * state->W;
  (void)num_accepted;
  hipLaunchKernelGGL(k_commit, dim3(1), dim3(kCT), 0, reinterpret_cast<hipStream_t>(stream),
                     *state, gamma, out_tokens, out_len, eligible, appended, dirty_slots,
                     dirty_mode, w);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_spec_commit_next(const hs_spec_state* state, int gamma, const int64_t* out_tokens,
                        const int32_t* out_len, int32_t* eligible, void* workspace,
                        size_t workspace_bytes, int next_gamma, int32_t* status, int lookback,
                        int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                        int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* v_input_ids,
                        int64_t* v_positions, int32_t* v_slot_mapping, int32_t* v_cu_seqlens_q,
                        int32_t* v_cu_seqlens_k, void* stream) {
  if (!state_ok(state) || gamma < 0 || next_gamma < 0 || !out_tokens || !out_len ||
      !eligible || !workspace || !input_ids || !positions || !slot_mapping || !cu_seqlens_q ||
      !cu_seqlens_k || (lookback != 0 && lookback != 1))
    return HS_ERR_INVALID;
  // the verify staging outputs: all or none
  const int nv = (v_input_ids != nullptr) + (v_positions != nullptr) +
                 (v_slot_mapping != nullptr) + (v_cu_seqlens_q != nullptr) +
                 (v_cu_seqlens_k != nullptr);
  if (nv != 0 && nv != 5) return HS_ERR_INVALID;
  VerifyStage v{v_input_ids, v_positions, v_slot_mapping, v_cu_seqlens_q, v_cu_seqlens_k};
  if (workspace_bytes < hs_spec_commit_workspace_size(state->B, state->W, state->num_blocks))
    return HS_ERR_WORKSPACE;
  int32_t* p = static_cast<int32_t*>(workspace);
  CommitWs w;
  w.dec = p;
  w.last = p + state->num_blocks;
  w.ev_blk = p + 2 * (size_t)state->num_blocks;
  w.ev_free = w.ev_blk + (size_t)state->B * state->W;
  w.seq = w.ev_free + (size_t)state->B * state->W;
  hipLaunchKernelGGL(k_commit_next, dim3(1), dim3(kCT), 0, reinterpret_cast<hipStream_t>(stream),
                     *state, gamma, out_tokens, out_len, eligible, w, next_gamma, status,
                     lookback, input_ids, positions, slot_mapping, cu_seqlens_q, cu_seqlens_k, v);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

int hs_zero_kv_slots(void* cache, int64_t plane_bytes, int num_planes, int64_t slot_bytes,
                     int64_t row_bytes, int64_t slots_per_plane, const int32_t* slots,
                     int num_slots, void* stream) {
  if (num_slots == 0 || num_planes == 0) return HS_OK;
  if (!cache || !slots || num_slots < 0 || num_planes < 0 || row_bytes <= 0 ||
      slot_bytes < row_bytes || plane_bytes < slot_bytes * slots_per_plane)
    return HS_ERR_INVALID;
  if ((row_bytes | slot_bytes | plane_bytes) & 3) return HS_ERR_UNSUPPORTED;
  if ((uintptr_t)cache & 3) return HS_ERR_UNSUPPORTED;
  const int64_t items = (int64_t)num_planes * num_slots;
  if (items > 0x7fffffff) return HS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(k_zero_slots, dim3((unsigned)items), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<uint8_t*>(cache),
                     plane_bytes, num_planes, slot_bytes, row_bytes, slots, num_slots,
                     slots_per_plane);
  return hipGetLastError() == hipSuccess ? HS_OK : HS_ERR_LAUNCH;
}

}  // extern "C"
