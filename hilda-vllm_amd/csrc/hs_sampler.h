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

struct FilterScratch {
  int32_t kept;
  int32_t path;
  int32_t pad[2];
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

struct Work {
  ChunkStat* part;
  RowDesc* desc;
  SeqState* st;
  SampPart* spart;
  FilterScratch* filt;
};

struct SampleOut {
  float* probs;
  int64_t probs_stride;
  int out_kind;  // 0: probabilities, 1: logits/T inside the kept set, -inf outside
  const float* uniforms;
  int64_t* tokens;
  int sample;
  float* row_stats;
};

struct Layout {
  size_t part, desc, st, spart, filt, total;
};

template <typename T>
int launch_filter(const Problem& P, const Work& W, float* row_stats, hipStream_t stream);

}  // namespace hs
