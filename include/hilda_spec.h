/*
 * hilda_spec.h - C ABI of the MI355X (gfx950) speculative-decoding verify path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, a
 * caller-owned workspace and a HIP stream (passed as void*, it is a
 * hipStream_t). Each returns 0 on success or a negative HS_ERR_* code; none of
 * them synchronises the stream or allocates device memory.
 *
 * Workspaces: query the size with the matching *_workspace_size() function
 * and pass a buffer at least that large. Two calls that share one workspace
 * must not overlap in time. A workspace is zero-filled before its first use
 * and every call leaves it ready for the next (so the calls can be recorded
 * into a HIP graph without a clearing step). Each entry point's workspace is
 * its own, except that hs_verify_attention and hs_qk_norm_rope_attend may
 * share one:
 *  - hs_spec_accept, hs_sampler and hs_spec_commit carry state from one call
 *    to the next (launch counters, the free-list scratch);
 *  - hs_verify_attention / hs_qk_norm_rope_attend hold partial results of a
 *    call after 16 KiB of merge counters that every call leaves zero.
 */
#ifndef HILDA_SPEC_H
#define HILDA_SPEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define HS_OK 0
#define HS_ERR_INVALID (-1)     /* bad size, null pointer or enum value      */
#define HS_ERR_WORKSPACE (-2)   /* workspace too small                        */
#define HS_ERR_LAUNCH (-3)      /* kernel launch failed (hipGetLastError)     */
#define HS_ERR_UNSUPPORTED (-4) /* valid request this build does not support */
#define HS_ERR_SCRATCH_LIMIT (-5) /* beyond the fixed scratch of a *_noalloc call */

/* element types */
#define HS_F32 0
#define HS_BF16 1
#define HS_FP8_E4M3 2

/* acceptance modes */
#define HS_ACCEPT_REFERENCE 0 /* temperature-only softmax (model_runner.py:398) */
#define HS_ACCEPT_FILTERED 1  /* temperature, top-k, top-p (sampler.py:20-49)   */
#define HS_ACCEPT_GREEDY 2    /* argmax match; temperature ignored             */
/* Flag OR-ed into HS_ACCEPT_FILTERED by a caller that knows every sequence's */
/* top-k is in [1, 64] (top-p any): small batches then run as a single launch */
/* (a sequence whose top-k breaks the promise gets num_accepted -1).          */
#define HS_ACCEPT_TOPK_LE64 0x100
/* Flag OR-ed into any mode of hs_spec_accept: run the launch chain (chunk    */
/* statistics, filter passes, row filter, decision and draw) even where a     */
/* single-launch kernel would serve the call. The results are the same bits;  */
/* this is for testing and timing the paths. OR-ed into the mode of          */
/* hs_sampler it likewise forces that call's launch chain.                    */
#define HS_ACCEPT_CHAIN 0x200

/* Human-readable text for a status code (static storage). */
const char* hs_status_string(int status);

/* Library version, (major << 16) | minor. */
int hs_version(void);

/* ------------------------------------------------------------------------ */
/* Fused acceptance sampler.                                                 */
/*                                                                          */
/* Replaces the per-sequence rejection-sampling loop of                      */
/* ModelRunner.run_verify, mini_vllm/engine/model_runner.py:387-428, with    */
/* the torch RNG calls (torch.rand at :407, torch.multinomial at :412,:425)  */
/* replaced by the explicit uniforms u_accept and u_resample.               */
/*                                                                          */
/* target_logits : [batch, gamma+1, vocab] rows of dtype HS_F32 or HS_BF16;  */
/*                 row (b, j) starts at element (b*(gamma+1)+j)*row_stride.  */
/* draft_probs   : [batch, gamma, vocab] f32; row (b, j) at                 */
/*                 (b*gamma+j)*draft_row_stride. Unused (may be NULL) in     */
/*                 greedy mode. In filtered mode it must hold the filtered   */
/*                 draft distribution the draft tokens were drawn from.     */
/* draft_tokens  : [batch, gamma] int64.                                     */
/* temperatures  : [batch] f32 (> 0 unless greedy); top_ks [batch] int32     */
/*                 (<= 0 or >= vocab: off); top_ps [batch] f32 (>= 1: off).  */
/*                 top_ks/top_ps are read in filtered mode only.            */
/* u_accept      : [batch, gamma] f32 in [0,1); u_resample [batch] f32.     */
/* outputs       : num_accepted [batch] int32, out_tokens [batch, gamma+1]   */
/*                 int64 (-1 after the last emitted token), out_len [batch]. */
/* row_stats     : optional [batch*(gamma+1), 2] f32: per target row the     */
/*                 softmax max and normaliser over the kept set.            */
/* workspace     : hs_spec_accept_workspace_size bytes, zero-filled before   */
/*                 its first use; calls leave it ready for the next one, of  */
/*                 any shape. Calls that share a workspace must not overlap. */
/*                 Small batches (batch x ceil(vocab/2048) workgroups fit one */
/*                 per CU, gamma <= 7, aligned rows, vocab a multiple of 8)  */
/*                 run as a single launch whose workgroups exchange data     */
/*                 through the workspace: in reference mode, and in filtered */
/*                 mode with HS_ACCEPT_TOPK_LE64 when vocab >= 64 * 2048.    */
/*                 Its waits are bounded: a thread polls at most a budget    */
/*                 (2^20 polls, over all its waits of the launch; the 32-bit */
/*                 word at byte offset 12 of the workspace, when nonzero,    */
/*                 sets it to that value minus 1, for tests of this path),   */
/*                 and a workgroup stops waiting at once when one of its     */
/*                 waits has failed or its data came from one that failed.   */
/*                 If a wait ran out, or the launch counter was not left by  */
/*                 a completed call, the sequences concerned get             */
/*                 num_accepted -1 and out_len 0 (a sequence's outputs are   */
/*                 either all valid or marked so), and the 32-bit word at    */
/*                 byte offset 8 of the workspace is set to 1 (sticky until  */
/*                 the caller clears it). Callers must check num_accepted    */
/*                 >= 0 at their next synchronisation.                       */
/* ------------------------------------------------------------------------ */
size_t hs_spec_accept_workspace_size(int batch, int gamma, int vocab);

int hs_spec_accept(const void* target_logits, int logits_dtype, int64_t logits_row_stride,
                   const float* draft_probs, int64_t draft_row_stride,
                   const int64_t* draft_tokens, const float* temperatures,
                   const int32_t* top_ks, const float* top_ps,
                   const float* u_accept, const float* u_resample,
                   int batch, int gamma, int vocab, int mode,
                   int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                   float* row_stats, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Row sampler: Sampler.forward, mini_vllm/layers/sampler.py:13-25, and the  */
/* draft-probability producer softmax(logits/T) of run_draft_decode,         */
/* mini_vllm/engine/model_runner.py:312-313.                                 */
/*                                                                          */
/* mode: HS_ACCEPT_REFERENCE (temperature only), HS_ACCEPT_FILTERED          */
/* (temperature, top-k, top-p) or HS_ACCEPT_GREEDY (argmax, lowest index on  */
/* ties; probs_out must be NULL).                                            */
/* probs_out (optional): [rows, vocab] f32. out_kind 0 writes the           */
/* probabilities of the (filtered) distribution; out_kind 1 writes logits/T  */
/* inside the kept set and -inf outside it, i.e. the masked logits of        */
/* Sampler._apply_top_k/_apply_top_p (sampler.py:27-49); out_kind 2 writes  */
/* the unfiltered softmax(logits/T) (bit-identical to a reference-mode      */
/* call's probabilities) while the draw stays filtered: the draft step of   */
/* reference-mode acceptance with top-k / top-p, which samples from Sampler  */
/* but keeps torch.softmax(logits/T) as the draft probabilities             */
/* (model_runner.py:312-313). In reference mode out_kind 2 is out_kind 0.   */
/* uniforms + tokens_out (optional, both or neither): one                    */
/* uniform per row drives an inverse-CDF draw that replaces the exponential- */
/* race draw of sampler.py:24.                                               */
/* workspace: hs_sampler_workspace_size bytes, zero-filled before its first */
/* use (every call leaves it ready for the next); not shared with other     */
/* entry points. Reference-mode calls whose rows x ceil(vocab/2048)         */
/* workgroups fit one per CU (vocab a multiple of 8, 16-byte aligned rows   */
/* and probability rows, out_kind 0) run as a single launch whose           */
/* workgroups exchange data through the workspace, with the bounded waits   */
/* of hs_spec_accept's single launch (same budget word at byte offset 12,  */
/* same sticky error word at byte offset 8); a row whose draw could not be  */
/* completed gets token -1 (its probabilities are then unspecified).        */
/* ------------------------------------------------------------------------ */
size_t hs_sampler_workspace_size(int rows, int vocab);

int hs_sampler(const void* logits, int logits_dtype, int64_t logits_row_stride,
               int rows, int vocab, const float* temperatures, const int32_t* top_ks,
               const float* top_ps, int mode, float* probs_out, int64_t probs_row_stride,
               int out_kind, const float* uniforms, int64_t* tokens_out, float* row_stats,
               void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* gamma+1-query paged-attention verify.                                     */
/*                                                                          */
/* Replaces the verify branch of Attention.forward,                          */
/* mini_vllm/layers/attention.py:145-160: flash_attn_varlen_func(q, k_cache, */
/* v_cache, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,          */
/* softmax_scale, causal=True, block_table) with bottom-right causal         */
/* alignment (query i of a sequence sees keys 0 .. Lk - Lq + i). Also serves */
/* decode (q_len 1) and prefill.                                             */
/*                                                                          */
/* q, out      : [tokens, num_q_heads, 128] bf16 with element strides        */
/*               (token, head); head elements contiguous, 16-byte aligned.   */
/* k/v cache   : [num_blocks, block_size, num_kv_heads, 128] bf16 or fp8      */
/*               e4m3fn (kv_dtype HS_BF16 / HS_FP8_E4M3), element strides    */
/*               (block, token, head); fp8 values dequantise as code*scale.  */
/* block_tables: int32 [num_seqs, block_table_width] (row stride given, at  */
/*               most INT32_MAX elements); entries outside [0, num_blocks)  */
/*               are treated as empty. NULL: the keys are the call's own    */
/*               unpaged rows (flash_attn_varlen_func without block_table,   */
/*               a prefill with no cached prefix): k_cache / v_cache are     */
/*               [tokens, num_kv_heads, 128] with element strides (token,    */
/*               head), sequence b's keys at rows cu_seqlens_k[b] ..         */
/*               cu_seqlens_k[b + 1] - 1; block arguments are ignored.       */
/* cu_seqlens_q/k: int32 [num_seqs + 1] prefix sums of query/key lengths.    */
/* The workspace (size from hs_verify_attention_workspace_size) holds, after */
/* 16 KiB of merge counters (zero-filled before the first call, left zero),  */
/* the partial results of key splits (or of the pieces of the one-workgroup- */
/* per-CU launch used for large calls). With none, or a smaller one, the     */
/* call uses the per-tile grid and returns HS_ERR_WORKSPACE if that grid     */
/* splits the keys.                                                          */
/* ------------------------------------------------------------------------ */
size_t hs_verify_attention_workspace_size(int num_seqs, int num_q_heads, int num_kv_heads,
                                          int max_seqlen_q, int max_seqlen_k);

int hs_verify_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        int64_t cache_stride_block, int64_t cache_stride_tok,
                        int64_t cache_stride_head, float k_scale, float v_scale,
                        const int32_t* block_tables, int64_t block_table_stride,
                        int block_table_width, int num_blocks, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int num_seqs, int max_seqlen_q,
                        int max_seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                        int block_size, float softmax_scale, void* out, int64_t out_stride_tok,
                        int64_t out_stride_head, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Allocation-free variant of hs_verify_attention. No counterpart in the     */
/* reference: it is for callers that cannot allocate device memory (code     */
/* under HIP graph capture, tight serving loops, harnesses that forbid       */
/* hipMalloc). Same arguments, kernels and results as hs_verify_attention    */
/* minus the workspace: the partial results live in a fixed scratch array of */
/* the library (hs_verify_attention_noalloc_scratch_bytes(), 34 MiB, one per */
/* GPU, held until the process ends). A call whose partials would not fit    */
/* returns HS_ERR_SCRATCH_LIMIT. Every call on one GPU shares that GPU's     */
/* scratch: calls that overlap in time on one GPU (two streams) race.        */
/* The scratch needs no clearing: each call writes the partials it reads.    */
/* (It starts zero-filled, as a workspace of hs_verify_attention must.)     */
int hs_verify_attention_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache, int kv_dtype,
                                int64_t cache_stride_block, int64_t cache_stride_tok,
                                int64_t cache_stride_head, float k_scale, float v_scale,
                                const int32_t* block_tables, int64_t block_table_stride,
                                int block_table_width, int num_blocks,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int num_seqs, int max_seqlen_q, int max_seqlen_k,
                                int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                float softmax_scale, void* out, int64_t out_stride_tok,
                                int64_t out_stride_head, void* stream);
size_t hs_verify_attention_noalloc_scratch_bytes(void);

/* ------------------------------------------------------------------------ */
/* KV-cache store: store_kvcache, mini_vllm/layers/attention.py:59-90, and   */
/* the FP8 store the reference imports from an external package             */
/* (attention.py:17-56, absent from the reference tree).                    */
/* key/value [num_tokens, num_kv_heads, 128] bf16; token i goes to cache slot */
/* slot_mapping[i] = block * block_size + offset; slots < 0 (the reference's */
/* -1) and blocks >= num_blocks are skipped. FP8 stores                      */
/* sat_e4m3fn(x / scale): round to nearest even, saturated to +-448.         */
/* ------------------------------------------------------------------------ */
int hs_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                     const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                     void* k_cache, void* v_cache, int kv_dtype, int64_t cache_stride_block,
                     int64_t cache_stride_tok, int64_t cache_stride_head, float k_scale,
                     float v_scale, const int32_t* slot_mapping, int num_tokens,
                     int num_kv_heads, int head_dim, int block_size, int num_blocks,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* Device-resident bookkeeping of the speculative step.                      */
/*                                                                          */
/* The state mirrors Sequence (mini_vllm/engine/sequence.py:14-132) and      */
/* BlockManager (block_manager.py:26-115) for a batch of B sequences:        */
/* context_lens = len(seq), num_prompt, max_tokens, ignore_eos (0/1),        */
/* finished (0/1), block_tables [B, W] (-1 padded) with num_seq_blocks, the  */
/* token history tokens [B, T] (T must exceed the longest sequence), the     */
/* free-block deque as a ring free_ring[num_blocks] with free_hdr = {head,    */
/* count} (pop at head, append at head+count), and ref_count[num_blocks].    */
/* block_hash (optional, NULL: no hashing): [num_blocks] int64, a block's    */
/* prefix hash (BlockManager.compute_hash, block_manager.py:36-41: xxh64,    */
/* seed 0, of the previous block's hash as 8 little-endian bytes, when there */
/* is one, then the block's tokens as int64) or -1. Pre-allocation resets    */
/* the blocks it takes to -1 (Block.reset); the commit then rehashes the     */
/* tables of the sequences that took part and did not finish, as            */
/* llm_engine.py:182-194 does (full blocks without a hash get one, partial   */
/* blocks lose theirs). The registry hash_to_block_id stays the host's.      */
/* All pointers are device pointers; the struct itself lives on the host.    */
/* ------------------------------------------------------------------------ */
typedef struct hs_spec_state {
  int32_t* context_lens;
  int32_t* num_prompt;
  int32_t* max_tokens;
  int32_t* ignore_eos;
  int32_t* finished;
  int32_t* block_tables;
  int32_t* num_seq_blocks;
  int64_t* tokens;
  int32_t* free_ring;
  int32_t* free_hdr;
  int32_t* ref_count;
  int32_t B, W, T, num_blocks, block_size;
  int32_t pad;
  int64_t eos;
  int64_t* block_hash;
} hs_spec_state;

/* Pre-allocation of blocks for len + gamma + 1 tokens,                      */
/* mini_vllm/engine/llm_engine.py:111-128: sequences in order, blocks popped */
/* from the front of the free deque with ref_count 1; a sequence is skipped  */
/* (eligible[b] = 0) when the free count is short or it is finished.         */
/* *status is set to 1 if a table row is too narrow (optional pointer).      */
int hs_spec_prealloc(const hs_spec_state* state, int gamma, int32_t* eligible, int32_t* status,
                     void* stream);

/* Verify staging, mini_vllm/engine/model_runner.py:339-362: per sequence the */
/* gamma+1 tokens [last_token, drafts], positions len-1+j, slot_mapping       */
/* (block*block_size + pos%block_size, or -1 past the table),                */
/* cu_seqlens_q (steps of gamma+1) and cu_seqlens_k (len + gamma each).       */
int hs_verify_prepare(const hs_spec_state* state, const int64_t* draft_tokens, int gamma,
                      int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                      int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, void* stream);

/* Draft-step staging, mini_vllm/engine/model_runner.py:294-310: step j of   */
/* the draft loop feeds draft_tokens[b, j-1] (last_token for j = 0) at        */
/* position len - 1 + j with context length len + j; one query per sequence.  */
/* lookback = 1 makes step 0 feed the last two tokens (positions len-2 and    */
/* len-1, two queries per sequence; outputs sized 2*B): after a step that     */
/* accepted all drafts, the reference's draft cache has no K/V for the last   */
/* accepted draft (it is never fed, :294-305) and this fills it.              */
int hs_draft_prepare(const hs_spec_state* state, const int64_t* draft_tokens, int draft_stride,
                     int step, int lookback, int64_t* input_ids, int64_t* positions,
                     int32_t* slot_mapping, int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                     void* stream);

/* Commit and rollback after acceptance, mini_vllm/engine/llm_engine.py:     */
/* 146-195: append out_tokens[b, :out_len[b]] one by one, stopping at EOS    */
/* (unless ignore_eos) or max_tokens (sequence finished: all blocks released */
/* last-first, block_manager.py:84-92); then unfinished sequences drop tail  */
/* blocks beyond ceil(len / block_size). Released blocks whose reference     */
/* count reaches 0 are appended to the free deque in the reference's order   */
/* (all finishes in sequence order, then all trims in sequence order).       */
/* appended[b] (optional) = tokens appended. dirty_slots (optional,          */
/* [B, gamma+1], -1 padded) lists the KV slots of rejected drafts            */
/* (model_runner.py:439-464): dirty_mode 0 uses the reference range          */
/* [len, old_len + gamma + 1), dirty_mode 1 the exact range                  */
/* [len - 1, old_len + gamma). num_accepted is not needed (may be NULL).     */
/* eligible (optional, [B] int32, the status of hs_spec_prealloc): rows with */
/* 0 sat out the step (llm_engine.py:120-121) and take no tokens; NULL means */
/* every row took part.                                                      */
/* The workspace must be zero-filled before its first use; every call leaves */
/* the counters it reads zero-filled again (its other words are scratch,     */
/* written before they are read), so it is ready for the next call.          */
size_t hs_spec_commit_workspace_size(int batch, int table_width, int num_blocks);
int hs_spec_commit(const hs_spec_state* state, int gamma, const int32_t* num_accepted,
                   const int64_t* out_tokens, const int32_t* out_len, const int32_t* eligible,
                   int32_t* appended, int32_t* dirty_slots, int dirty_mode, void* workspace,
                   size_t workspace_bytes, void* stream);

/* hs_spec_commit (without appended / dirty slots) followed, in the same     */
/* launch, by the next step's hs_spec_prealloc(next_gamma) into eligible     */
/* (read by the commit first) and hs_draft_prepare(step 0, lookback) into    */
/* the given staging buffers: the end of one speculative step and the        */
/* start of the next, llm_engine.py:146-195 then :111-128 and                */
/* model_runner.py:294-310, for callers that know the next step's gamma.     */
/* v_*: optional (all five or none), the next step's hs_verify_prepare       */
/* (model_runner.py:339-362) outputs except the ids of the draft tokens      */
/* (rows 1 .. next_gamma of each sequence, left unwritten for the draft      */
/* steps to fill in place).                                                  */
/* No reference counterpart: the reference runs these as separate host       */
/* steps; here they are one graph node instead of four.                      */
int hs_spec_commit_next(const hs_spec_state* state, int gamma, const int64_t* out_tokens,
                        const int32_t* out_len, int32_t* eligible, void* workspace,
                        size_t workspace_bytes, int next_gamma, int32_t* status, int lookback,
                        int64_t* input_ids, int64_t* positions, int32_t* slot_mapping,
                        int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* v_input_ids,
                        int64_t* v_positions, int32_t* v_slot_mapping, int32_t* v_cu_seqlens_q,
                        int32_t* v_cu_seqlens_k, void* stream);

/* The bookkeeping half of hs_spec_accept_commit_next: hs_spec_commit_next's  */
/* arguments after out_len, with the same meaning (state->B = batch).         */
typedef struct hs_commit_next_args {
  const hs_spec_state* state;
  int32_t* eligible;
  void* workspace;
  size_t workspace_bytes;
  int32_t next_gamma;
  int32_t lookback;
  int32_t* status;
  int64_t* input_ids;
  int64_t* positions;
  int32_t* slot_mapping;
  int32_t* cu_seqlens_q;
  int32_t* cu_seqlens_k;
  int64_t* v_input_ids;
  int64_t* v_positions;
  int32_t* v_slot_mapping;
  int32_t* v_cu_seqlens_q;
  int32_t* v_cu_seqlens_k;
} hs_commit_next_args;

/* hs_spec_accept, then hs_spec_commit_next(next->state, gamma, out_tokens,  */
/* out_len, next->...) on the same stream: a speculative step's acceptance   */
/* (model_runner.py:387-428), commit and rollback (llm_engine.py:146-195),   */
/* the next step's pre-allocation (:111-128) and its staging                 */
/* (model_runner.py:294-310, :339-362). With batch 1 and the acceptance's    */
/* single launch (reference mode, the conditions under hs_spec_accept), the  */
/* workgroup that writes the acceptance outputs runs the bookkeeping after   */
/* them: one launch in all. If that launch's bounded waits fail, the         */
/* sequence gets num_accepted -1 as in hs_spec_accept and the bookkeeping    */
/* does not run (state, eligible and staging keep their values; the two      */
/* launches would commit no token and stage the next step). Otherwise the    */
/* results are those of the two calls.                                       */
/* No reference counterpart: the reference runs acceptance and bookkeeping   */
/* as separate host steps; here a batch-1 step's are one graph node.         */
int hs_spec_accept_commit_next(const void* target_logits, int logits_dtype,
                               int64_t logits_row_stride, const float* draft_probs,
                               int64_t draft_row_stride, const int64_t* draft_tokens,
                               const float* temperatures, const int32_t* top_ks,
                               const float* top_ps, const float* u_accept,
                               const float* u_resample, int batch, int gamma, int vocab, int mode,
                               int32_t* num_accepted, int64_t* out_tokens, int32_t* out_len,
                               float* row_stats, void* workspace, size_t workspace_bytes,
                               const hs_commit_next_args* next, void* stream);

/* Zeroes row_bytes at every slot of slots[] (entries < 0 skipped) in each of */
/* num_planes planes (e.g. the 2*L (K|V, layer) planes of a                  */
/* [2, L, num_blocks, block_size, H, D] cache): byte offset                  */
/* plane * plane_bytes + slot * slot_bytes. Replaces the per-layer index     */
/* assignments of cleanup_rejected_kv_slots, model_runner.py:467-481.        */
int hs_zero_kv_slots(void* cache, int64_t plane_bytes, int num_planes, int64_t slot_bytes,
                     int64_t row_bytes, int64_t slots_per_plane, const int32_t* slots,
                     int num_slots, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused elementwise kernels of the decoder layer (bf16 in/out). They stand  */
/* in for the torch.compile-fused ops of the reference around the verify    */
/* path: RMSNorm / fused add + RMSNorm (mini_vllm/layers/layernorm.py:18-36),*/
/* q/k RMSNorm + neox RoPE (qwen3.py:82-85, rotary_embedding.py:8-50) and    */
/* SiLU-and-mul (activation.py:8-16).                                        */
/* ------------------------------------------------------------------------ */
/* Skinny projection for decode / verify rows: out[r, n] = sum_k x[r, k] *    */
/* weight[n, k] (bf16 in, fp32 accumulation, bf16 out), nn.Linear's          */
/* F.linear(x, weight) of the model's qkv / o / gate_up / down / lm_head       */
/* layers (mini_vllm/layers/linear.py) at rows <= 8. HS_LINEAR_SWIGLU takes a */
/* [2 * out_features, in_features] gate|up weight and writes                   */
/* silu(gate) * up (activation.py:8-16) with the rounding of the unfused ops.  */
/* in_features must be a multiple of 512, out_features of 4; strides in        */
/* elements. Larger row counts are plain library GEMMs.                        */
#define HS_LINEAR_PLAIN 0
#define HS_LINEAR_SWIGLU 1
int hs_linear(const void* x, int64_t x_stride, const void* weight, int rows, int in_features,
              int out_features, int epilogue, void* out, int64_t out_stride, void* stream);

/* hs_linear whose input is the decoder's RMSNorm (the input_layernorm /     */
/* post_attention_layernorm in front of qkv_proj / gate_up_proj,             */
/* qwen3.py:148-161, layernorm.py:18-36): row r of the projection input is    */
/* bf16(bf16(h * rsqrt(mean(h^2) + eps)) * norm_weight) with the fp32 sum      */
/* h = x[r] (+ residual_in[r]). residual_in may be NULL (plain RMSNorm). When  */
/* residual_out != NULL it receives bf16(h) (the add_rms_norm residual); it   */
/* must not overlap x or residual_in (HS_ERR_INVALID). Same shape limits as   */
/* hs_linear; residual strides multiples of 8 elements.                       */
int hs_linear_rmsnorm(const void* x, int64_t x_stride, const void* residual_in,
                      int64_t residual_in_stride, void* residual_out, int64_t residual_out_stride,
                      const void* norm_weight, float eps, const void* weight, int rows,
                      int in_features, int out_features, int epilogue, void* out,
                      int64_t out_stride, void* stream);

/* out = RMSNorm(x (+ residual)) * weight; with residual != NULL the residual  */
/* row is replaced by bf16(x + residual) (strides in elements).              */
int hs_rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
               const void* weight, void* out, int64_t out_stride, int rows, int hidden,
               float eps, void* stream);

/* qkv [tokens, (Hq + 2*Hkv) * 128] (row stride token_stride): q and k heads are */
/* RMS-normalised with q_weight / k_weight [128], rotated with cos_sin          */
/* [max_pos, 128] (cos | sin) at positions[tokens], and written to q_out        */
/* [tokens, Hq, 128] and k_out [tokens, Hkv, 128]. head_dim must be 128.        */
int hs_qk_norm_rope(const void* qkv, int64_t token_stride, int num_q_heads, int num_kv_heads,
                    int head_dim, const void* q_weight, const void* k_weight,
                    const float* cos_sin, const int64_t* positions, float eps, void* q_out,
                    void* k_out, int num_tokens, void* stream);

/* hs_qk_norm_rope fused with the KV store of the same tokens (the           */
/* store_kvcache call at the top of Attention.forward, attention.py:59-90 and */
/* :145): q heads go to q_out [tokens, Hq, 128]; the normalised, rotated k    */
/* heads and the v heads (columns (Hq + Hkv) * 128 .. of qkv) are written to   */
/* their slot_mapping slots of k_cache / v_cache with the layout, dtype and    */
/* scales of hs_store_kvcache (slots < 0 skipped).                            */
int hs_qk_norm_rope_store(const void* qkv, int64_t token_stride, int num_q_heads,
                          int num_kv_heads, int head_dim, const void* q_weight,
                          const void* k_weight, const float* cos_sin, const int64_t* positions,
                          float eps, void* q_out, void* k_cache, void* v_cache, int kv_dtype,
                          int64_t cache_stride_block, int64_t cache_stride_tok,
                          int64_t cache_stride_head, float k_scale, float v_scale,
                          const int32_t* slot_mapping, int block_size, int num_blocks,
                          int num_tokens, void* stream);

/* hs_qk_norm_rope_store followed by hs_verify_attention on the stored cache */
/* (Qwen3Attention.forward, mini_vllm/models/qwen3.py:83-86: q_norm, k_norm,  */
/* rotary_emb, then Attention.forward's store_kvcache and paged attention,    */
/* mini_vllm/layers/attention.py:59-90, :145-160), as one launch where one   */
/* 16-row query tile holds every query row of a (sequence, kv head) (decode */
/* and verify steps): each workgroup normalises and rotates its q rows in   */
/* LDS and stores its kv head's k/v rows of the sequence's query tokens     */
/* before reading them; keys past one split of the launch plan are spread   */
/* over several workgroups whose partial results the last of them merges    */
/* (the workspace's merge counters). Other calls run the two launches (and  */
/* the split combine), with q_out receiving q. Same outputs and cache        */
/* contents either way.                                                      */
/* qkv: [num_tokens, (Hq + 2 Hkv) * 128] bf16 holding the query tokens of    */
/* the sequences in cu_seqlens_q order (num_tokens = cu_seqlens_q[num_seqs]), */
/* cos_sin: [cos_sin_rows, 128] f32 (cos | sin), every position below       */
/* cos_sin_rows; positions / slot_mapping one entry per token (slots < 0    */
/* store nothing);                                                           */
/* q_out: [num_tokens, Hq, 128] bf16 (contents unspecified after a fused     */
/* call); the cache, table, length, scale and output arguments are those of  */
/* hs_verify_attention (k_scale / v_scale also scale the fp8 stores).        */
int hs_qk_norm_rope_attend(const void* qkv, int64_t token_stride, int num_tokens,
                           const void* q_weight, const void* k_weight, const float* cos_sin,
                           int cos_sin_rows, const int64_t* positions, float eps,
                           const int32_t* slot_mapping,
                           void* q_out, void* k_cache, void* v_cache, int kv_dtype,
                           int64_t cache_stride_block, int64_t cache_stride_tok,
                           int64_t cache_stride_head, float k_scale, float v_scale,
                           const int32_t* block_tables, int64_t block_table_stride,
                           int block_table_width, int num_blocks, const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int num_seqs, int max_seqlen_q,
                           int max_seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                           int block_size, float softmax_scale, void* out,
                           int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                           size_t workspace_bytes, void* stream);

/* out[r, :ffn] = silu(gate_up[r, :ffn]) * gate_up[r, ffn:2*ffn]. */
int hs_silu_mul(const void* gate_up, int64_t gate_up_stride, int ffn, void* out,
                int64_t out_stride, int rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HILDA_SPEC_H */
