// Accept/rollback bookkeeping kernels of a speculative step (gfx950): one
// workgroup of 1024 threads each, running the bodies of hs_bookkeeping.h
// (llm_engine.py:104-195, block_manager.py:20-115, model_runner.py:294-310,
// :339-362, and the rejected-slot cleanup of model_runner.py:439-481). The
// state (lengths, block tables, token history, FIFO free list, reference
// counts) stays resident in HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hilda_spec.h"
#include "hs_bookkeeping.h"

namespace hs {

constexpr int kCT = 1024;  // threads of every bookkeeping kernel
constexpr int kCW = kCT / 64;

__global__ __launch_bounds__(kCT) void k_prealloc(hs_spec_state s, int gamma, int32_t* eligible,
                                                  int32_t* status) {
  __shared__ PreallocLds<kCT> L;
  prealloc_body<kCT>(s, gamma, eligible, status, L);
}

__global__ __launch_bounds__(kCT) void k_prepare(hs_spec_state s, const int64_t* draft, int gamma,
                                                 int64_t* input_ids, int64_t* positions,
                                                 int32_t* slot_mapping, int32_t* cu_q,
                                                 int32_t* cu_k) {
  __shared__ int s_w[kCW];
  verify_prepare_body<kCT>(s, draft, gamma, input_ids, positions, slot_mapping, cu_q, cu_k, s_w);
}

__global__ __launch_bounds__(kCT) void k_draft_prepare(hs_spec_state s, const int64_t* draft,
                                                       int draft_stride, int step, int lookback,
                                                       int64_t* input_ids, int64_t* positions,
                                                       int32_t* slot_mapping, int32_t* cu_q,
                                                       int32_t* cu_k) {
  __shared__ int s_w[kCW];
  draft_prepare_body<kCT>(s, draft, draft_stride, step, lookback, input_ids, positions,
                          slot_mapping, cu_q, cu_k, s_w);
}

__global__ __launch_bounds__(kCT) void k_commit(hs_spec_state s, int gamma, const int64_t* out_tokens,
                                                const int32_t* out_len, const int32_t* eligible,
                                                int32_t* appended, int32_t* dirty, int dirty_mode,
                                                CommitWs w) {
  __shared__ int s_w[kCW];
  __shared__ int s_tot[2];
  commit_body<kCT>(s, gamma, out_tokens, out_len, eligible, appended, dirty, dirty_mode, w, s_w,
                   s_tot);
}

__global__ __launch_bounds__(kCT) void k_commit_next(CommitNext c, const int64_t* out_tokens,
                                                     const int32_t* out_len) {
  __shared__ CommitNextLds<kCT> L;
  commit_next_any<kCT>(c, out_tokens, out_len, L);
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

static int state_ok(const hs_spec_state* s) {
  if (!s || !s->context_lens || !s->num_prompt || !s->max_tokens || !s->ignore_eos ||
      !s->finished || !s->block_tables || !s->num_seq_blocks || !s->tokens || !s->free_ring ||
      !s->free_hdr || !s->ref_count)
    return 0;
  return s->B > 0 && s->W > 0 && s->T > 0 && s->num_blocks > 0 && s->block_size > 0;
}

namespace hs {

static CommitWs bind_commit_ws(const hs_spec_state* state, void* workspace) {
  int32_t* p = static_cast<int32_t*>(workspace);
  CommitWs w;
  w.dec = p;
  w.last = p + state->num_blocks;
  w.ev_blk = p + 2 * (size_t)state->num_blocks;
  w.ev_free = w.ev_blk + (size_t)state->B * state->W;
  w.seq = w.ev_free + (size_t)state->B * state->W;
  return w;
}

int make_commit_next(const hs_spec_state* state, int gamma, int32_t* eligible, void* workspace,
                     size_t workspace_bytes, int next_gamma, int32_t* status, int lookback,
                     int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                     int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* v_input_ids,
                     int64_t* v_positions, int32_t* v_slot_mapping, int32_t* v_cu_seqlens_q,
                     int32_t* v_cu_seqlens_k, CommitNext* out) {
  if (!state_ok(state) || gamma < 0 || next_gamma < 0 || !eligible || !workspace || !input_ids ||
      !positions || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k ||
      (lookback != 0 && lookback != 1))
    return HS_ERR_INVALID;
  // the verify staging outputs: all or none
  const int nv = (v_input_ids != nullptr) + (v_positions != nullptr) +
                 (v_slot_mapping != nullptr) + (v_cu_seqlens_q != nullptr) +
                 (v_cu_seqlens_k != nullptr);
  if (nv != 0 && nv != 5) return HS_ERR_INVALID;
  if (workspace_bytes < hs_spec_commit_workspace_size(state->B, state->W, state->num_blocks))
    return HS_ERR_WORKSPACE;
  out->s = *state;
  out->gamma = gamma;
  out->next_gamma = next_gamma;
  out->lookback = lookback;
  out->eligible = eligible;
  out->status = status;
  out->w = bind_commit_ws(state, workspace);
  out->ids = input_ids;
  out->pos = positions;
  out->slots = slot_mapping;
  out->cu_q = cu_seqlens_q;
  out->cu_k = cu_seqlens_k;
  out->v = VerifyStage{v_input_ids, v_positions, v_slot_mapping, v_cu_seqlens_q, v_cu_seqlens_k};
  return HS_OK;
}

}  // namespace hs

extern "C" {


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
  const CommitWs w = bind_commit_ws(state, workspace);
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
  if (!out_tokens || !out_len) return HS_ERR_INVALID;
  CommitNext c;
  const int rc = make_commit_next(state, gamma, eligible, workspace, workspace_bytes, next_gamma,
                                  status, lookback, input_ids, positions, slot_mapping,
                                  cu_seqlens_q, cu_seqlens_k, v_input_ids, v_positions,
                                  v_slot_mapping, v_cu_seqlens_q, v_cu_seqlens_k, &c);
  if (rc != HS_OK) return rc;
  hipLaunchKernelGGL(k_commit_next, dim3(1), dim3(kCT), 0, reinterpret_cast<hipStream_t>(stream),
                     c, out_tokens, out_len);
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
