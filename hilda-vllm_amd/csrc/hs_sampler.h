// Shared types of the sampler kernels (spec_accept.hip, spec_filter.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hs {

constexpr int kMaxGamma = 32;     // drafts per sequence handled by one wave
constexpr int kFilterThreads = 512;
constexpr int kCand = 4096;       // LDS candidate capacity of the filter kernel
constexpr int kMaxRows = 65535;   // units per call (grid.y of k_sample_part)
constexpr int kChunkThreads = 256;  // one workgroup streams one 2048-element chunk
constexpr int kCB = 256;          // buckets of the top-p coarse and fine histograms

enum : int { kFinRow = 0, kFinDecide = 1, kFinPlain = 2 };
enum : int { kKindNone = 0, kKindResidual = 1, kKindBonus = 2, kKindPlain = 3 };

// per (row, chunk): chunk max and exact fixed-point exp-sum relative to it
// (greedy reuses `e` for the packed (key, ~index) maximum)
struct ChunkStat {
  float m;
  uint32_t pad;
  uint64_t e;
};

// Per-row distribution descriptor. Element i (x_i = logit_i / T) belongs to
// the kept set iff all || key(x_i) > tkey || (key(x_i) == tkey && i <= tidx);
// its probability is exp(x_i - m) / s when kept, 0 otherwise.
struct RowDesc {
  float m;
  float s;
  uint32_t tkey;
  int32_t tidx;
  int32_t all;
  int32_t token;   // greedy argmax
  float s_full;    // normaliser over the whole row
  int32_t pad;
};

// per unit (sequence in hs_spec_accept, row in hs_sampler): where to draw
struct SeqState {
  int32_t kind;
  int32_t row;    // global target row to draw from
  int32_t qrow;   // draft row for the residual
  int32_t nacc;   // accepted drafts
  int32_t pad[4];
};

struct SampPart {
  uint64_t w;  // residual weight sum of the chunk
  uint64_t p;  // probability weight sum of the chunk
};

// Per-row state of the filter passes (k_filter_plan1/2 write it, the passes and
// k_row_filter read it).
struct FilterScratch {
  int32_t kept;
  int32_t path;
  int32_t ncand;   // candidates appended by the filter passes
  int32_t b1;      // coarse boundary bucket (-1: the row never reaches p; -2: not
                   // within buckets 0..jmax, the row filter streams the row)
  int32_t jmax;    // pass 1 histograms buckets 0..jmax only (see mass_skip_bucket)
  uint32_t c1;     // elements in coarse bucket b1 (k_filter_plan2)
  float m;         // row max and normaliser (x = logit / T)
  float s;
  uint32_t tau;    // top-k gather threshold (order key)
  uint32_t pad;
  uint64_t theta;  // top-p mass threshold (fixed point)
  uint64_t ac;     // count, mass and e-mass of the elements before the boundary bucket
  uint64_t am;
  uint64_t ae;
  // raw-value (logit) thresholds of the top-p passes, exact images of their
  // bucket tests (x = logit / T is monotone in the logit): pass 1 takes
  // logit >= rj (coarse bucket <= jmax), pass 2 rlo <= logit < rhi (coarse
  // bucket b1)
  float rj, rlo, rhi, pad2;
};

struct Problem {
  const void* logits;
  int64_t row_stride;
  int rows_per_unit;
  int units;
  int V;
  int nchunk;
  int nsplit;
  const float* temps;     // per unit
  const int32_t* top_ks;  // per unit
  const float* top_ps;    // per unit
  int filtered;           // the chunk pass clears the filter scratch
};

struct AcceptArgs {
  const float* q;
  int64_t q_stride;
  const int64_t* dtok;
  const float* u_acc;
  int gamma;
  int32_t* nacc_out;
  int64_t* tok_out;
  int32_t* len_out;
};

// Launch epoch of the single-launch acceptance (spec_accept_small.hip), at the
// start of the workspace: `start` must be zero before the first call and every
// completed call leaves its count half zero; `err` is set if a wait for
// another workgroup's data ever ran out (the outputs of that call are invalid).
struct SmallSync {
  uint64_t start;  // epoch << 32 | workgroups of the current launch that started
  uint32_t err;
  // polls a thread of a single-launch acceptance may spend waiting, over all
  // its waits of one launch: 0 (a zero-filled workspace) the default budget,
  // n > 0 a budget of n - 1 (set from the host to test the failure path)
  uint32_t spin_limit;
  uint32_t pad[60];
};

struct Work {
  SmallSync* sync;
  uint64_t* tags;  // epoch-tagged partials of the single-launch acceptance
  ChunkStat* part;
  RowDesc* desc;
  SeqState* st;
  SampPart* spart;
  FilterScratch* filt;
  uint64_t* cand;  // [rows, kCand] candidates (key << 32 | ~index)
  uint64_t* h1m;   // [rows, kCB] coarse top-p histogram: masses, e-masses, counts
  uint64_t* h1e;
  uint32_t* h1c;
  uint64_t* h2m;   // [rows, kCB] fine histogram inside the coarse boundary bucket
  uint64_t* h2e;
  uint32_t* h2c;
  int32_t* flist;  // filtered mode: [2] row counts, then [rows] top-k rows, [rows] top-p rows
};

struct SampleOut {
  float* probs;
  int64_t probs_stride;
  int out_kind;  // 0: probabilities, 1: logits/T inside the kept set, -inf outside,
                 // 2: the unfiltered probabilities (the draw stays filtered)
  const float* uniforms;
  int64_t* tokens;
  int sample;
  float* row_stats;
};

// Bytes reserved for the single-launch acceptance's tagged words, right after
// the SmallSync word, in every layout: the same fixed region whatever the
// call's shape, so the chain kernels of calls of other shapes sharing the
// workspace never write there (their chunk sums, read as tagged words, could
// carry a later epoch in their high half). Eligible calls need at most
// (rows*3 + units*4) * nchunk * 8 <= 28 * 8 * 256 = 57344 bytes.
constexpr size_t kSmallTagBytes = 65536;

// Tagged words of the single-launch top-k acceptance (filtered mode with every
// top-k in [1, kTopkMax]), in a second fixed region right after the first:
// per (row, chunk) the chunk's maximum (key, index) pair (2 words) and its
// candidate count (1 word), then per (row, chunk) kTopkSlots candidates of 3
// words (key, index, draft probability). Eligible calls have at most
// kTopkPairs (row, chunk) pairs.
constexpr int kTopkMax = 64;
constexpr int kTopkSlots = 64;
constexpr int kTopkPairs = 2048;
constexpr size_t kTopkTagBytes = (size_t)kTopkPairs * (3 + 3 * kTopkSlots) * 8;

struct Layout {
  size_t sync, tags, part, desc, st, spart, filt, cand, h1m, h1e, h1c, h2m, h2e, h2c, flist, total;
};

template <typename T>
int launch_filter(const Problem& P, const Work& W, float* row_stats, bool wave,
                  hipStream_t stream);

// single-launch acceptance (reference mode) for grids that fit one workgroup
// per CU (spec_accept_small.hip); cn (batch 1 only, else NULL): the step's
// bookkeeping (hs_bookkeeping.h) run by the workgroup that writes the outputs
struct CommitNext;
int small_accept_ok(const Problem& P, const AcceptArgs& A, int mode, int esz);
template <typename T>
int launch_accept_small(const Problem& P, const AcceptArgs& A, const Work& W, const SampleOut& O,
                        const CommitNext* cn, hipStream_t stream);
// the same for filtered mode when every sequence's top-k is in [1, kTopkMax]
int small_topk_ok(const Problem& P, const AcceptArgs& A, int esz);
// single-launch row sampler (reference mode, a few rows; spec_accept_small.hip)
int small_sampler_ok(const Problem& P, const SampleOut& O, int esz);
template <typename T>
int launch_sample_small(const Problem& P, const Work& W, const SampleOut& O, hipStream_t stream);
template <typename T>
int launch_accept_small_topk(const Problem& P, const AcceptArgs& A, const Work& W,
                             const SampleOut& O, hipStream_t stream);

}  // namespace hs
