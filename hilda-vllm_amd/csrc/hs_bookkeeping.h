// Device bodies of the speculative step's bookkeeping (gfx950), shared by the
// bookkeeping kernels and the acceptance kernel that commits a batch-1 step
// in the same launch.
//
// Replaces the host-side bookkeeping of LLMEngine.step's spec block,
// mini_vllm/engine/llm_engine.py:104-195, the BlockManager operations it uses
// (block_manager.py:20-115) and the staging of run_draft_decode / run_verify
// (model_runner.py:294-310, :339-362). Each body runs in one workgroup of NT
// threads (a multiple of 64, at most 1024): the work is a few integers per
// sequence, and the FIFO order of freed blocks depends on sequence order,
// which one workgroup resolves with block-wide scans instead of atomics whose
// outcome would depend on timing. Bodies that follow one another are
// separated by a workgroup barrier.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"

namespace hs {

// exclusive scan over the workgroup of one int per thread; returns the total
template <int NT>
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
  for (int w = 0; w < NT / 64; ++w) {
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
// block hash: BlockManager.compute_hash, block_manager.py:36-41
// ---------------------------------------------------------------------------
// xxh64 with seed 0 (the xxHash specification, XXH64) of the previous block's
// hash as 8 little-endian bytes, when there is one (prefix != -1), then n
// tokens as int64: whole 8-byte words, so no 4-byte or 1-byte tail round.
constexpr uint64_t kXP1 = 11400714785074694791ull, kXP2 = 14029467366897019727ull;
constexpr uint64_t kXP3 = 1609587929392839161ull, kXP4 = 9650029242287828579ull;
constexpr uint64_t kXP5 = 2870177450012600261ull;
__device__ __forceinline__ uint64_t xxh_rotl(uint64_t x, int r) {
  return (x << r) | (x >> (64 - r));
}
__device__ __forceinline__ uint64_t xxh_round(uint64_t acc, uint64_t in) {
  return xxh_rotl(acc + in * kXP2, 31) * kXP1;
}
__device__ uint64_t block_hash_of(int64_t prefix, const int64_t* toks, int n) {
  const bool pre = prefix != -1;
  const int total = n + (pre ? 1 : 0);
  auto word = [&](int i) -> uint64_t {
    return pre ? (i == 0 ? (uint64_t)prefix : (uint64_t)toks[i - 1]) : (uint64_t)toks[i];
  };
  uint64_t h;
  int i = 0;
  if (total >= 4) {
    uint64_t v1 = kXP1 + kXP2, v2 = kXP2, v3 = 0, v4 = 0ull - kXP1;
    for (; i + 4 <= total; i += 4) {
      v1 = xxh_round(v1, word(i));
      v2 = xxh_round(v2, word(i + 1));
      v3 = xxh_round(v3, word(i + 2));
      v4 = xxh_round(v4, word(i + 3));
    }
    h = xxh_rotl(v1, 1) + xxh_rotl(v2, 7) + xxh_rotl(v3, 12) + xxh_rotl(v4, 18);
    h = (h ^ xxh_round(0, v1)) * kXP1 + kXP4;
    h = (h ^ xxh_round(0, v2)) * kXP1 + kXP4;
    h = (h ^ xxh_round(0, v3)) * kXP1 + kXP4;
    h = (h ^ xxh_round(0, v4)) * kXP1 + kXP4;
  } else {
    h = kXP5;
  }
  h += (uint64_t)total * 8;
  for (; i < total; ++i) h = xxh_rotl(h ^ xxh_round(0, word(i)), 27) * kXP1 + kXP4;
  h ^= h >> 33;
  h *= kXP2;
  h ^= h >> 29;
  h *= kXP3;
  h ^= h >> 32;
  return h;
}

// ---------------------------------------------------------------------------
// pre-allocation: llm_engine.py:111-128
// ---------------------------------------------------------------------------
template <int NT>
struct PreallocLds {
  int need[NT], off[NT], ok[NT];
  int take;
};

template <int NT>
__device__ void prealloc_body(const hs_spec_state& s, int gamma, int32_t* eligible,
                              int32_t* status, PreallocLds<NT>& L) {
  int* s_need = L.need;
  int* s_off = L.off;
  int* s_ok = L.ok;
  int& s_take = L.take;
  const int tid = threadIdx.x;
  for (int base = 0; base < s.B; base += NT) {
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
      const int cnt = (s.B - base < NT) ? s.B - base : NT;
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
          if (s.block_hash) s.block_hash[blk] = -1;  // Block.reset
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

// ---------------------------------------------------------------------------
// verify staging: model_runner.py:339-362
// ---------------------------------------------------------------------------
// draft NULL: the draft tokens' ids (rows 1 .. gamma of each sequence) are
// left as they are (written in place by the draft steps' sampler)
template <int NT>
__device__ void verify_prepare_body(const hs_spec_state& s, const int64_t* draft, int gamma,
                                    int64_t* input_ids, int64_t* positions,
                                    int32_t* slot_mapping, int32_t* cu_q, int32_t* cu_k,
                                    int* s_w) {
  const int tid = threadIdx.x;
  const int R = gamma + 1;
  int carry = 0;
  for (int base = 0; base < s.B; base += NT) {
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
    const int ex = cscan_excl<NT>(lk, s_w, &total);
    if (b < s.B) cu_k[b] = carry + ex;
    carry += total;
  }
  if (tid == 0) {
    cu_q[s.B] = s.B * R;
    cu_k[s.B] = carry;
  }
}

// draft step staging: model_runner.py:294-310 (step j feeds the previous draft
// token, or last_token for j = 0, at position len - 1 + j). With lookback, step
// 0 feeds the two last tokens (positions len-2, len-1): after a step that
// accepted every draft, the draft model never saw the last accepted draft,
// and this fills that KV slot.
template <int NT>
__device__ void draft_prepare_body(const hs_spec_state& s, const int64_t* draft, int draft_stride,
                                   int step, int lookback, int64_t* input_ids, int64_t* positions,
                                   int32_t* slot_mapping, int32_t* cu_q, int32_t* cu_k,
                                   int* s_w) {
  const int tid = threadIdx.x;
  const int R = (step == 0 && lookback) ? 2 : 1;
  int carry = 0;
  for (int base = 0; base < s.B; base += NT) {
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
    const int ex = cscan_excl<NT>(lk, s_w, &total);
    if (b < s.B) cu_k[b] = carry + ex;
    carry += total;
  }
  if (tid == 0) {
    cu_q[s.B] = s.B * R;
    cu_k[s.B] = carry;
  }
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

template <int NT>
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
  for (int b = tid; b < s.B; b += NT) {
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
  for (int base = 0; base < s.B; base += NT) {
    const int b = base + tid;
    const int nd = b < s.B ? s_ndeal[b] : 0;
    const int nt = b < s.B ? s_ntrim[b] : 0;
    int td, tt;
    const int od = cscan_excl<NT>(nd, s_w, &td);
    const int ot = cscan_excl<NT>(nt, s_w, &tt);
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
  for (int b = tid; b < s.B; b += NT) {
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
  for (int e = tid; e < E; e += NT) {
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
  for (int base = 0; base < E; base += NT) {
    const int e = base + tid;
    const int f = e < E ? w.ev_free[e] : 0;
    int tot;
    const int ex = cscan_excl<NT>(f, s_w, &tot);
    if (f) s.free_ring[(head + count0 + carry + ex) % s.num_blocks] = w.ev_blk[e];
    carry += tot;
  }
  __syncthreads();
  for (int e = tid; e < E; e += NT) {
    const int blk = w.ev_blk[e];
    w.dec[blk] = 0;
    w.last[blk] = 0;
  }
  // phase 6: shrink the tables
  for (int b = tid; b < s.B; b += NT) {
    const int nblk = s_nblk[b];
    const int keep = s.finished[b] ? 0 : (s.context_lens[b] + s.block_size - 1) / s.block_size;
    if (keep < nblk) {
      for (int k = keep; k < nblk; ++k) s.block_tables[(int64_t)b * s.W + k] = -1;
      s.num_seq_blocks[b] = keep;
    }
  }
  if (tid == 0) s.free_hdr[1] = count0 + carry;
  if (!s.block_hash) return;

  // phase 7: rehash (llm_engine.py:182-194) the tables of the sequences that
  // took part and did not finish: a full block without a hash gets one (the
  // previous block's hash as prefix), a partial block loses its hash. 7a: one
  // thread per (sequence, entry) clears and finds each sequence's first full
  // block without a hash (s_first, over s_nblk's words); 7b: the sequence's
  // thread hashes from there on, in table order (each hash is the next one's
  // prefix).
  int32_t* s_first = w.seq;
  __syncthreads();
  for (int b = tid; b < s.B; b += NT) s_first[b] = 0x7fffffff;
  __syncthreads();
  const int bs = s.block_size;
  auto rehashed = [&](int b) {
    return !(eligible && !eligible[b]) && !s.finished[b];
  };
  for (int64_t p = tid; p < (int64_t)s.B * s.W; p += NT) {
    const int b = (int)(p / s.W), bi = (int)(p % s.W);
    const int nblk = s.num_seq_blocks[b];
    if (bi >= nblk || !rehashed(b)) continue;
    const int blk = s.block_tables[(int64_t)b * s.W + bi];
    if (blk < 0 || blk >= s.num_blocks) continue;
    const bool full = bi < nblk - 1 || s.context_lens[b] % bs == 0;
    const int64_t h = s.block_hash[blk];
    if (!full && h != -1) s.block_hash[blk] = -1;
    if (full && h == -1) atomicMin(&s_first[b], bi);
  }
  __syncthreads();
  for (int b = tid; b < s.B; b += NT) {
    const int f = s_first[b];
    if (f == 0x7fffffff) continue;
    const int nblk = s.num_seq_blocks[b];
    const int len = s.context_lens[b];
    const int32_t* row = s.block_tables + (int64_t)b * s.W;
    int64_t prev = f > 0 ? s.block_hash[row[f - 1]] : -1;
    for (int bi = f; bi < nblk; ++bi) {
      if (!(bi < nblk - 1 || len % bs == 0)) break;  // the partial last block
      const int blk = row[bi];
      int64_t h = s.block_hash[blk];
      if (h == -1) {
        if ((int64_t)(bi + 1) * bs > s.T) break;  // tokens past the history
        h = (int64_t)block_hash_of(prev, s.tokens + (int64_t)b * s.T + (int64_t)bi * bs, bs);
        s.block_hash[blk] = h;
      }
      prev = h;
    }
  }
}

// The commit of a step, then the next step's pre-allocation (into eligible,
// which the commit has read), its first draft step's staging and, when v.ids
// is given, its verify staging without the draft tokens' ids: the end of one
// speculative step and the start of the next. The state each part reads is
// the one the previous part left (their writes are ordered by the workgroup
// barriers between them).
struct VerifyStage {
  int64_t* ids;
  int64_t* pos;
  int32_t* slots;
  int32_t* cu_q;
  int32_t* cu_k;
};
struct CommitNext {
  hs_spec_state s;
  int gamma, next_gamma, lookback;
  int32_t* eligible;
  int32_t* status;
  CommitWs w;
  // the first draft step's staging
  int64_t* ids;
  int64_t* pos;
  int32_t* slots;
  int32_t* cu_q;
  int32_t* cu_k;
  VerifyStage v;
};
template <int NT>
struct CommitNextLds {
  int w[NT / 64];
  int tot[2];
  int fast;
  PreallocLds<NT> pre;
};
template <int NT>
__device__ void commit_next_body(const CommitNext& c, const int64_t* out_tokens,
                                 const int32_t* out_len, CommitNextLds<NT>& L) {
  commit_body<NT>(c.s, c.gamma, out_tokens, out_len, c.eligible, nullptr, nullptr, 0, c.w, L.w,
                  L.tot);
  __syncthreads();
  prealloc_body<NT>(c.s, c.next_gamma, c.eligible, c.status, L.pre);
  __syncthreads();
  draft_prepare_body<NT>(c.s, nullptr, 0, 0, c.lookback, c.ids, c.pos, c.slots, c.cu_q, c.cu_k,
                         L.w);
  if (c.v.ids) {
    __syncthreads();  // L.w is reused
    verify_prepare_body<NT>(c.s, nullptr, c.next_gamma, c.v.ids, c.v.pos, c.v.slots, c.v.cu_q,
                            c.v.cu_k, L.w);
  }
}

// ---------------------------------------------------------------------------
// commit_next_body for one sequence, in one wave
// ---------------------------------------------------------------------------
// The common step of a one-sequence state: not finished, eligible, not ending
// in this step, no rehash work (with block hashes: no block that has just
// become full, no partial block with a hash), a table row of at most 256
// entries, at most kB1Take blocks to take, staging rows within a wave. The results equal commit_next_body's; the
// wave reads the state in two rounds of loads (the state words and the table
// row; the free-list front, the history token and the reference counts of the
// tail blocks the commit may release) instead of commit_next_body's chain of
// dependent rounds, computes the results (b1_plan) and writes every address
// once, with its final value (b1_store). For any other state it stores nothing
// (commit_next_body then runs). Every lane of the wave takes part.
constexpr int kB1Take = 16;

// table entry bi of the row held as entries lane + 64 q in tb[q]
__device__ __forceinline__ int b1_row_at(const int (&tb)[4], int bi) {
  const int l = bi & 63;
  const int v0 = __shfl(tb[0], l, 64), v1 = __shfl(tb[1], l, 64);
  const int v2 = __shfl(tb[2], l, 64), v3 = __shfl(tb[3], l, 64);
  const int q = bi >> 6;
  return q == 0 ? v0 : q == 1 ? v1 : q == 2 ? v2 : v3;
}

// What the one-wave path reads, one round per load function: b1_load1 reads
// the state words (lane k < 9: word k) and the table row (lane i: entries
// i + 64 q, clamped into the row: only entries below the row length are used);
// b1_load2, from those, the free-list front (lane k: entry head + k), the tail
// blocks a commit of at least one token may release, last first (lane e: table
// entry nblk0 - 1 - e), their reference counts, the history token before the
// appended ones and (with block hashes) the low words of the table entries'
// hashes. Every load is unconditional, from a clamped in-range
// index where its own one is not needed or not valid, so that nothing waits
// for it before its use in b1_plan (a conditional load would be waited for
// where its branch joins). Nothing changes the state between the loads and
// b1_store (the step's kernels run one after another).
struct B1Pre {
  int word;
  int tb[4];
  int ring, tblk, ref;
  int64_t hist;
  int bad;    // lane with an entry out of range
  int bh[4];  // low words of the table entries' block hashes (state with hashes)
};

__device__ __forceinline__ void b1_load1(const CommitNext& c, B1Pre& P) {
  const hs_spec_state& s = c.s;
  const int lane = threadIdx.x & 63;
  const int32_t* wp = s.context_lens;
  switch (lane) {
    case 1: wp = s.num_seq_blocks; break;
    case 2: wp = s.finished; break;
    case 3: wp = c.eligible; break;
    case 4: wp = s.num_prompt; break;
    case 5: wp = s.max_tokens; break;
    case 6: wp = s.ignore_eos; break;
    case 7: wp = s.free_hdr; break;
    case 8: wp = s.free_hdr + 1; break;
    default: break;
  }
  P.word = *wp;  // lanes 9 and up: context_lens[0], unused
  const int w = s.W < 256 ? s.W : 256;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = lane + 64 * q;
    P.tb[q] = s.block_tables[i < w ? i : w - 1];
  }
}

__device__ __forceinline__ void b1_load2(const CommitNext& c, B1Pre& P) {
  const hs_spec_state& s = c.s;
  const int lane = threadIdx.x & 63;
  const int len0 = __builtin_amdgcn_readlane(P.word, 0);
  const int nblk0 = __builtin_amdgcn_readlane(P.word, 1);
  const int head = __builtin_amdgcn_readlane(P.word, 7);
  const int count0 = __builtin_amdgcn_readlane(P.word, 8);
  const int N = s.num_blocks, bs = s.block_size;
  const bool hdr_ok = head >= 0 && head < N && count0 >= 0 && count0 <= N;
  P.ring = s.free_ring[hdr_ok ? (head + lane) % N : 0];  // used for lanes below count0
  // blocks kept by any commit of at least one token: ceil((len0 + 1) / bs)
  const int nmin = len0 >= 0 ? (len0 + bs) / bs : 0;
  const bool row_ok = nblk0 >= 0 && nblk0 <= s.W && s.W <= 256;
  const bool t = row_ok && lane < nblk0 - nmin;
  P.tblk = b1_row_at(P.tb, t ? nblk0 - 1 - lane : 0);
  const bool in = P.tblk >= 0 && P.tblk < N;
  P.bad = t && !in;
  P.ref = s.ref_count[in ? P.tblk : 0];  // used for lanes below the trim count
  P.hist = s.tokens[(len0 >= 1 && len0 <= s.T) ? len0 - 1 : 0];
  // the low word of each table entry's hash: -1 has 0xffffffff there, so a hash
  // whose low word is that reads as none (the rehash then takes the workgroup
  // path, which reads whole hashes)
  if (s.block_hash) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int blk = P.tb[q];
      P.bh[q] = reinterpret_cast<const int32_t*>(
          s.block_hash)[2 * (int64_t)(blk >= 0 && blk < N ? blk : 0)];
    }
  }
}

// The one-wave path's results for a commit of n tokens, all but the last of
// which (toks[0 .. n-2]) are known: b1_plan computes everything from the loads
// and n, so that it can run before the last token is drawn; b1_store checks the
// last token and stores. ok false: the path does not apply (nothing stored).
struct B1Plan {
  int ok;
  int n, len0, len, nblk, nblk0, needed, take, head, count0, avail, elig, igeos;
  int N, ntrim;
  // lane e < ntrim: the released block (entry nblk0 - 1 - e), its count, its
  // order among the freed ones; lane k < take: the block taken
  int tblk, ref, freed, fidx, tk;
  // lane r < R0: first draft step row r (position, slot, token unless it is
  // the last one); lane j < next_gamma + 1: next verify row j
  int dpos, dsl, dlast, vpos, vsl;
  int64_t dtok;
};

__device__ void b1_plan(const CommitNext& c, const B1Pre& P, int n, const int64_t* toks,
                        B1Plan& Q) {
  const hs_spec_state& s = c.s;
  const int lane = threadIdx.x & 63;
  Q.ok = 0;
  if (s.B != 1 || s.W > 256 || c.next_gamma + 1 > 64) return;
  const int len0 = __builtin_amdgcn_readlane(P.word, 0);
  const int nblk0 = __builtin_amdgcn_readlane(P.word, 1);
  const int fin0 = __builtin_amdgcn_readlane(P.word, 2);
  const int elig0 = __builtin_amdgcn_readlane(P.word, 3);
  const int nprompt = __builtin_amdgcn_readlane(P.word, 4);
  const int maxtok = __builtin_amdgcn_readlane(P.word, 5);
  const int igeos = __builtin_amdgcn_readlane(P.word, 6);
  const int head = __builtin_amdgcn_readlane(P.word, 7);
  const int count0 = __builtin_amdgcn_readlane(P.word, 8);
  const int N = s.num_blocks, bs = s.block_size;
  if (fin0 || !elig0 || n < 1 || n > c.gamma + 1 || len0 < 1) return;
  if (head < 0 || head >= N || count0 < 0 || count0 > N) return;
  const int len = len0 + n;
  if (len > s.T) return;
  // a token that ends the sequence (EOS or max_tokens) releases its blocks;
  // the last token's EOS test is b1_store's
  bool ends = false;
  for (int j = 0; j < n; ++j) {
    if (j < n - 1 && !igeos && toks[j] == s.eos) ends = true;
    if (len0 + j + 1 - nprompt == maxtok) ends = true;
  }
  if (ends) return;
  const int needed = (len + bs - 1) / bs;  // blocks kept by the commit
  if (nblk0 < needed || nblk0 > s.W) return;
  const int ntrim = nblk0 - needed;  // at most nblk0 - ceil((len0 + 1) / bs)
  if (ntrim > 64) return;
  // the next step's pre-allocation (from the trimmed table)
  const int needed2 = (len + c.next_gamma + 1 + bs - 1) / bs;
  const int need = needed2 - needed;
  if (need > kB1Take || (need > 0 && needed2 > s.W)) return;
  // a rehash with work to do (a full block without a hash, a partial one with a
  // hash: llm_engine.py:182-194) takes the workgroup path
  if (s.block_hash) {
    bool work = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int bi = lane + 64 * q;
      const bool full = bi < needed - 1 || len % bs == 0;
      const bool none = P.bh[q] == -1;
      if (bi < needed && (full == none)) work = true;
    }
    if (__ballot(work) != 0) return;
  }
  // the tail blocks released (lane e: entry nblk0 - 1 - e)
  const bool trims = lane < ntrim;
  const int tblk = P.tblk, ref = P.ref;
  if (__ballot(trims && P.bad) != 0) return;
  // a block released twice: the generic commit folds its decrements
  bool dup = false;
  for (int k = 0; k < ntrim; ++k) {
    const int o = __shfl(tblk, k, 64);
    if (trims && k != lane && o == tblk) dup = true;
  }
  if (__ballot(dup) != 0) return;
  const bool freed = trims && ref - 1 == 0;
  const uint64_t fmask = __ballot(freed);
  const int nfreed = __popcll(fmask);
  const int avail = count0 + nfreed;
  const int ok = (need <= 0 || avail >= need) ? 1 : 0;
  const int take = (ok && need > 0) ? need : 0;
  // block taken by lane k < take: the free-list front, then the blocks freed here
  int src = 0;
  if (lane >= count0 && lane < take) {
    uint64_t m = fmask;
    for (int t = 0; t < lane - count0; ++t) m &= m - 1;
    src = __ffsll((long long)m) - 1;
  }
  const int fb = __shfl(tblk, src, 64);
  const int tk = lane < take ? (lane < count0 ? P.ring : fb) : -1;
  const int nblk = needed + take;
  // slot of position pos in the final table (-1 past it)
  auto slot_of = [&](int pos) -> int {
    const int bi = pos >= 0 ? pos / bs : 0;
    const bool valid = pos >= 0 && bi < nblk;
    const int old = b1_row_at(P.tb, bi < 256 ? bi : 0);
    const int nb = __shfl(tk, (bi - needed) & 63, 64);
    return valid ? (bi < needed ? old : nb) * bs + pos % bs : -1;
  };
  // first draft step: row r feeds the token at position len - 1 - back
  const int R0 = c.lookback ? 2 : 1;
  const int dpos = len - 1 - (R0 - 1 - lane);
  const int h = dpos >= 0 ? dpos : 0;  // at least len0 - 1 for lanes below R0
  const int jt = h - len0;             // index among the appended tokens
  Q.dlast = jt >= n - 1;
  Q.dtok = jt < 0 ? P.hist : toks[(jt >= 0 && jt < n - 1) ? jt : 0];
  Q.dpos = dpos;
  Q.dsl = slot_of(dpos);
  Q.vpos = len - 1 + lane;
  Q.vsl = slot_of(Q.vpos);
  Q.n = n;
  Q.len0 = len0;
  Q.len = len;
  Q.nblk = nblk;
  Q.nblk0 = nblk0;
  Q.needed = needed;
  Q.take = take;
  Q.head = head;
  Q.count0 = count0;
  Q.avail = avail;
  Q.elig = ok;
  Q.igeos = igeos;
  Q.N = N;
  Q.ntrim = ntrim;
  Q.tblk = tblk;
  Q.ref = ref;
  Q.freed = freed;
  Q.fidx = __popcll(fmask & ((1ull << lane) - 1));  // order among the freed
  Q.tk = tk;
  Q.ok = 1;
}

// toks[0 .. n-2] as given to b1_plan, last: the last token
__device__ bool b1_store(const CommitNext& c, const B1Plan& Q, const int64_t* toks,
                         int64_t last) {
  const hs_spec_state& s = c.s;
  const int lane = threadIdx.x & 63;
  if (!Q.ok || (!Q.igeos && last == s.eos)) return false;
  const int n = Q.n, len0 = Q.len0, len = Q.len, N = Q.N;
  // every address written once, with its final value
  if (lane < n) s.tokens[len0 + lane] = lane == n - 1 ? last : toks[lane];
  if (lane < Q.ntrim) {
    if (Q.freed) s.free_ring[(Q.head + Q.count0 + Q.fidx) % N] = Q.tblk;
    // a freed block taken again ends with reference count 1 (stored below)
    if (!(Q.freed && Q.count0 + Q.fidx < Q.take)) s.ref_count[Q.tblk] = Q.ref - 1;
  }
  if (lane < Q.take) {
    s.block_tables[Q.needed + lane] = Q.tk;
    s.ref_count[Q.tk] = 1;
    if (s.block_hash) s.block_hash[Q.tk] = -1;  // Block.reset
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = lane + 64 * q;
    if (i >= Q.nblk && i < Q.nblk0) s.block_tables[i] = -1;
  }
  if (lane == 0) {
    s.context_lens[0] = len;
    s.num_seq_blocks[0] = Q.nblk;
    s.free_hdr[0] = (Q.head + Q.take) % N;
    s.free_hdr[1] = Q.avail - Q.take;
    c.eligible[0] = Q.elig;
  }
  const int R0 = c.lookback ? 2 : 1;
  if (lane < R0) {
    c.ids[lane] = Q.dlast ? last : Q.dtok;
    c.pos[lane] = Q.dpos;
    c.slots[lane] = Q.dsl;
  }
  if (lane == 0) {
    c.cu_q[0] = 0;
    c.cu_q[1] = R0;
    c.cu_k[0] = 0;
    c.cu_k[1] = len;
  }
  // the next verify step's rows, except the draft tokens' ids
  if (c.v.ids) {
    const int R = c.next_gamma + 1;
    if (lane < R) {
      if (lane == 0) c.v.ids[0] = last;
      c.v.pos[lane] = Q.vpos;
      c.v.slots[lane] = Q.vsl;
    }
    if (lane == 0) {
      c.v.cu_q[0] = 0;
      c.v.cu_q[1] = R;
      c.v.cu_k[0] = 0;
      c.v.cu_k[1] = len + c.next_gamma;
    }
  }
  return true;
}

// commit_next_body, through the one-wave path where it applies: wave fw
// stores plan Q (its own b1_plan for this commit) if it applies, else every
// thread runs commit_next_body.
template <int NT>
__device__ void commit_next_planned(const CommitNext& c, const B1Plan& Q, int fw,
                                    const int64_t* out_tokens, const int32_t* out_len,
                                    CommitNextLds<NT>& L) {
  if ((int)(threadIdx.x >> 6) == fw) {
    const int n = out_len[0];
    const bool done = Q.ok && Q.n == n && b1_store(c, Q, out_tokens, out_tokens[n - 1]);
    if ((threadIdx.x & 63) == 0) L.fast = done ? 1 : 0;
  }
  __syncthreads();
  if (!L.fast) commit_next_body<NT>(c, out_tokens, out_len, L);
}

// the same, wave 0 loading and planning first
template <int NT>
__device__ void commit_next_any(const CommitNext& c, const int64_t* out_tokens,
                                const int32_t* out_len, CommitNextLds<NT>& L) {
  B1Plan Q{};
  if (threadIdx.x < 64) {
    B1Pre P;
    b1_load1(c, P);
    b1_load2(c, P);
    b1_plan(c, P, out_len[0], out_tokens, Q);
  }
  commit_next_planned<NT>(c, Q, 0, out_tokens, out_len, L);
}

// Builds the device arguments of commit_next_body from hs_spec_commit_next's
// (validated as that entry point does); HS_OK or the error status.
int make_commit_next(const hs_spec_state* state, int gamma, int32_t* eligible, void* workspace,
                     size_t workspace_bytes, int next_gamma, int32_t* status, int lookback,
                     int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                     int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* v_input_ids,
                     int64_t* v_positions, int32_t* v_slot_mapping, int32_t* v_cu_seqlens_q,
                     int32_t* v_cu_seqlens_k, CommitNext* out);

}  // namespace hs
