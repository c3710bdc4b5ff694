/*
 * longspark_amd -- C ABI of the MI355X (gfx950) verify-and-refresh kernels.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * plus the hipStream_t to launch on (passed as void*), validates its
 * arguments on the host before launching anything, and returns an int status
 * (LS_OK = 0).  On failure, ls_last_error() returns a message for the calling
 * thread.  No entry point allocates device memory or synchronises the host.
 * Scratch space is caller-owned and comes in two buffers whose sizes the
 * matching *_workspace() function reports:
 *   counters -- zero-filled before first use; every call returns every
 *               counter it touched to zero, so one zeroed counter buffer can
 *               be shared by all entry points issued on one stream;
 *   scratch  -- no initialisation required.
 * Calls that share a counter or scratch buffer must not overlap (issue them
 * on one stream).
 *
 * Reference paths below are relative to the LongSpark repository root;
 * SRT = vendor/sglang/python/sglang/srt.
 */
#ifndef LONGSPARK_AMD_H_
#define LONGSPARK_AMD_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define LS_API __attribute__((visibility("default")))
#else
#define LS_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  LS_OK = 0,
  LS_ERR_SHAPE = 1,     /* sizes or strides inconsistent */
  LS_ERR_DTYPE = 2,     /* unsupported element type */
  LS_ERR_ALIGN = 3,     /* pointer alignment not supported */
  LS_ERR_LAUNCH = 4,    /* HIP launch error */
  LS_ERR_WORKSPACE = 5, /* workspace missing or too small */
  LS_ERR_VALUE = 6      /* invalid scalar parameter */
};

/* Element type codes. */
enum {
  LS_F32 = 0,
  LS_BF16 = 1,
  LS_F16 = 2,
  LS_I32 = 3,
  LS_I64 = 4
};

/* Message describing the last failure on the calling thread ("" if none). */
LS_API const char* ls_last_error(void);
/* Library version string. */
LS_API const char* ls_version(void);

/* ---------------------------------------------------------------------------
 * Greedy chain verification (fused argmax + accept length + bonus).
 *
 * Replaces the argmax / cumprod / gather sequence of
 *   src/longspark/engine/target.py:474-477 (split engine),
 *   SRT/speculative/dflash_utils.py:564-602
 *     (compute_dflash_correct_drafts_and_bonus),
 *   SRT/speculative/draft_free_kv_utils.py:360-383
 *     (compute_greedy_accept_len_and_bonus),
 *   SRT/speculative/dspark_components/kernels/accept_greedy.py:62-135
 *     (AcceptGreedy.torch / .triton, no cutoff layout).
 *
 * logits: [batch*width, vocab] rows (row r = request r / width, position
 *   r % width), element type logits_dtype (LS_BF16, LS_F16 or LS_F32), row
 *   stride logits_row_stride elements.
 * candidates: integer tokens (LS_I32 or LS_I64); drafted token j of request b
 *   (j = 0 .. width-2) is candidates[b*cand_stride_b + (cand_first_col+j)*cand_stride_k].
 *   cand_first_col = 1 for the [B, K] layout whose column 0 is the current
 *   token; 0 for the split engine's [B, K-1] drafted-only layout.
 * cutoff_verify_lens (int32 [batch], may be NULL): per-request verify window;
 *   the accepted length is capped at cutoff_verify_lens[b] - 1 and the number
 *   of tokens cut is written to cap_trim[b] (int32, may be NULL), as
 *   SRT/speculative/dspark_components/kernels/cap_correct_len.py:39-47 does
 *   (the capped length is clamped to [0, width-1] for memory safety).
 * Outputs: accept_lens[b] (int32) = number of accepted drafted tokens,
 *   bonus[b] (int64) = argmax of row accept_lens[b],
 *   truth (int32 [batch*width], may be NULL) = every row's argmax.
 * Ties resolve to the lowest index (torch.argmax).  NaN logits are not
 * supported.
 * ------------------------------------------------------------------------- */
LS_API int ls_verify_greedy_workspace(int64_t batch, int32_t width, int64_t vocab,
                                      uint64_t* counter_bytes, uint64_t* scratch_bytes);
LS_API int ls_verify_greedy(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                     const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                     int64_t cand_stride_k, int32_t cand_first_col, int64_t batch, int32_t width,
                     int64_t vocab, const int32_t* cutoff_verify_lens, int32_t* accept_lens,
                     int64_t* bonus, int32_t* truth, int32_t* cap_trim, void* counters,
                     uint64_t counter_bytes, void* scratch, uint64_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Penalty tables from each request's output-token history.
 *
 * Compact form of the accumulated [B, V] penalty tensors the reference keeps
 * (SRT/sampling/penaltylib/frequency_penalty.py:35-43,
 * presence_penalty.py:35-43, repetition_penalty.py:48-57,
 * orchestrator.py:87-104; consumed at SRT/sampling/sampling_batch_info.py:
 * 269-286):
 *   bits[b, w]  presence bitmap of history b (token v -> bit v&31 of word v>>5),
 *   rank[b, w]  number of present tokens below token 32*w,
 *   add[b, r]   additive penalty of the r-th present token in ascending token
 *               order: (0 - F) - P, F = fp32 sum of frequency[b] repeated
 *               count times, P = presence[b] (null frequency/presence = 0).
 * history: [batch, >= history_cap] int32 with row stride history_stride;
 *   history_lens (int32 [batch], may be NULL = history_cap) entries per row.
 *   Ids outside [0, vocab) are ignored.
 * words_stride >= ceil(vocab/32); add_stride >= history_cap.
 * distinct (int32 [batch], may be NULL) receives the number of present tokens;
 * nonpositive (int32 [batch], may be NULL) receives 1 where every additive
 * value is <= 0 (frequency and presence >= 0), else 0.
 * Limit: 8*ceil(vocab/32) + 4*history_cap <= 64 KiB.
 * ------------------------------------------------------------------------- */
LS_API int ls_penalty_tables(const int32_t* history, int64_t history_stride, const int32_t* history_lens,
                             int64_t batch, int32_t history_cap, int64_t vocab, const float* frequency,
                             const float* presence, uint32_t* bits, uint32_t* rank, int64_t words_stride,
                             float* add, int64_t add_stride, int32_t* distinct, int32_t* nonpositive,
                             void* stream);

/* ---------------------------------------------------------------------------
 * In-place logit adjustment of [rows, vocab] logits: penalties (tables from
 * ls_penalty_tables, repetition[b] scaling of present tokens) and the packed
 * vocabulary bitmask (bit 0 -> -inf, LSB first; only the first
 * min(vocab, 32*mask_words) columns are masked).
 *
 * Replaces SRT/speculative/dflash_utils.py:127-213
 * (apply_dflash_verify_logits_adjustments: verify_quirk = 1 builds the bias
 * on a zero tensor as that function does, verify_quirk = 0 applies the
 * penalties to the logits themselves in the order of
 * SRT/sampling/sampling_batch_info.py:269-286) and, with no penalty tables,
 * SRT/constrained/triton_ops/bitmask_ops.py:84-141
 * (apply_token_bitmask_inplace_triton).
 * rows_per_request: rows of one request (penalty table b = row / rows_per_request);
 * mask_rows_per_request: 1 (one mask row per logits row) or rows_per_request
 * (one mask row per request).  Arithmetic is fp32; bf16/fp16 rows are rounded
 * once per changed element.
 * ------------------------------------------------------------------------- */
LS_API int ls_adjust_logits(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t rows, int64_t vocab,
                            int32_t rows_per_request, const uint32_t* pen_bits, const uint32_t* pen_rank,
                            int64_t pen_words_stride, const float* pen_add, int64_t pen_add_stride,
                            const float* repetition, int32_t verify_quirk, const int32_t* vocab_mask,
                            int64_t mask_stride, int32_t mask_rows_per_request, int64_t mask_words, void* stream);

/* ---------------------------------------------------------------------------
 * Fused stochastic chain verification of a drafted block.
 *
 * Replaces, in one call, the sequence
 *   SRT/speculative/dflash_utils.py:127-213   logit adjustments (penalties, mask),
 *   SRT/speculative/dflash_utils.py:743-810   target distribution (T, top-k, top-p)
 *                                               + min-p (SRT/layers/sampler.py:238-242),
 *   SRT/speculative/dspark_components/kernels/accept_sampling.py:259-567
 *                                               single-q acceptance, residual, bonus
 *                                               (q_mode 0), or
 *   SRT/speculative/reject_sampling.py:5-204   dense-q chain sampling (q_mode 1),
 *   src/longspark/engine/sampling.py:19-57     decide_acceptance + finish_sampling,
 * with host-supplied uniforms.
 *
 * Target: logits [batch*width, vocab] (bf16/fp16/fp32), row r = request
 *   r / width, position r % width; row j < width-1 verifies drafted token j at
 *   candidates[b*cand_stride_b + (cand_first_col + j)*cand_stride_k].
 * Sampling parameters per request ([batch]): temperatures (> 0, required),
 *   top_ks (int32, >= vocab disables; NULL = disabled), top_ps (>= 1 disables),
 *   min_ps (<= 0 disables).  max_top_k: host upper bound of top_ks (0 = 1024);
 *   top-k above 1024 is not supported.
 * Penalties (optional): tables from ls_penalty_tables (pen_add NULL = no
 *   additive penalties), pen_repetition [batch] (NULL = 1); pen_verify_quirk
 *   as in ls_adjust_logits; pen_nonpositive [batch] (may be NULL) lets top-k
 *   rows whose penalties never raise a logit (repetition >= 1, additive <= 0)
 *   filter on raw logits and transform only their candidates.
 * vocab_mask (optional): int32 words, mask_row_stride >= ceil(vocab/32);
 *   mask_per_request = 1: row b, else row r.
 * Draft: q_mode 0 -- draft_token_probs [batch, width-1] fp32 (q of each drafted
 *   token) and draft rows [batch, width-1, vocab] (fp32 or bf16 logits; the q
 *   row at the rejection is softmax(row / T_d) after the draft_* top-k / top-p
 *   / min-p, each NULL = disabled, draft_temperatures NULL = temperatures);
 *   q_mode 1 -- draft rows are fp32 probabilities [batch, width-1, vocab].
 * Uniforms: uniforms [batch, width-1] (row stride uniform_stride_b),
 *   final_uniforms [batch].
 * Outputs: accept_lens[b] (int32) accepted drafted tokens, bonus[b] (int64)
 *   the token drawn from the residual (rejection) or from the last row (all
 *   accepted); p_cand_out [batch, width-1] (may be NULL) the target
 *   probability of each drafted token.  A request whose support exceeds the
 *   kernel's candidate capacity gets accept = bonus = -1 and ORs 1 into
 *   *status (may be NULL).
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* logits;
  int32_t logits_dtype;
  int64_t logits_row_stride;
  const void* candidates;
  int32_t candidates_dtype;
  int64_t cand_stride_b;
  int64_t cand_stride_k;
  int32_t cand_first_col;
  int64_t batch;
  int32_t width;
  int64_t vocab;
  const float* temperatures;
  const int32_t* top_ks;
  const float* top_ps;
  const float* min_ps;
  int32_t max_top_k;
  const uint32_t* pen_bits;
  const uint32_t* pen_rank;
  int64_t pen_words_stride;
  const float* pen_add;
  int64_t pen_add_stride;
  const float* pen_repetition;
  int32_t pen_verify_quirk;
  const int32_t* pen_nonpositive; /* [batch] from ls_penalty_tables, may be NULL */
  const int32_t* vocab_mask;
  int64_t mask_row_stride;
  int32_t mask_per_request;
  int32_t q_mode;
  const float* draft_token_probs;
  int64_t dtp_stride_b;
  const void* draft;
  int32_t draft_dtype;
  int64_t draft_stride_b;
  int64_t draft_stride_k;
  const float* draft_temperatures;
  const int32_t* draft_top_ks;
  const float* draft_top_ps;
  const float* draft_min_ps;
  const float* uniforms;
  int64_t uniform_stride_b;
  const float* final_uniforms;
  int32_t* accept_lens;
  int64_t* bonus;
  float* p_cand_out;
  int32_t* status;
  /* Optional timing: NULL, or 4 hipEvent_t handles recorded on the stream
   * before the target scan, after it, before the resolve kernel and after it
   * (the middle interval holds the fallback and draft-scan kernels). */
  void* const* timing_events;
  /* Which row-scan kernels to launch: 0 = both (each row runs in the one for
   * its path), 1 = only the raw-logit top-k scan (for callers that know every
   * row is top-k with repetition >= 1 and additive penalties <= 0; other rows
   * are still resolved exactly, more slowly), 2 = only the exact scan. */
  int32_t scan_hint;
} ls_verify_sample_args;

LS_API int ls_verify_sample_workspace(int64_t batch, int32_t width, int64_t vocab, int32_t max_top_k,
                                      uint64_t* counter_bytes, uint64_t* scratch_bytes);
LS_API int ls_verify_sample(const ls_verify_sample_args* args, void* counters, uint64_t counter_bytes,
                            void* scratch, uint64_t scratch_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LONGSPARK_AMD_H_ */
