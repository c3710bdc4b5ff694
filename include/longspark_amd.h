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
 *   SRT/speculative/dspark_components/kernels/cap_correct_len.py:44-52 does
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
 * ls_verify_greedy without a workspace argument: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory or pass
 * a workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  The counters live in a 1 MiB device array built
 * into the library; each GPU the library runs on holds its own copy until
 * the process ends (its address is looked up, and the array cleared, on the
 * first call on that device).  Limit: 8*batch*width + 4*batch bytes (each
 * part rounded up to 256) <= 1 MiB, e.g. batch 4096 x width 16; larger calls
 * return LS_ERR_WORKSPACE.  All calls on one GPU share the array: calls that
 * overlap on one GPU (different streams, or different threads' streams)
 * race and must not be issued.  Arguments and outputs as ls_verify_greedy.
 * ------------------------------------------------------------------------- */
LS_API int ls_verify_greedy_noalloc(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                    const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                    int64_t cand_stride_k, int32_t cand_first_col, int64_t batch, int32_t width,
                                    int64_t vocab, const int32_t* cutoff_verify_lens, int32_t* accept_lens,
                                    int64_t* bonus, int32_t* truth, int32_t* cap_trim, void* stream);

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
 * SRT/sampling/sampling_batch_info.py:269-286).  The bitmask alone, with
 * row indices, is ls_apply_token_bitmask below.
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
 * Per-request bias vectors added in place to every row of the request:
 * replaces the additions of SRT/speculative/dflash_utils.py:176-213
 * (apply_dflash_verify_logits_adjustments with the caller's dense [B, V]
 * penalty, mask and logit-bias tensors).
 * logits [rows, vocab] (fp32/bf16/fp16; row r belongs to request
 * r / rows_per_request); bias, bias2: fp32 [rows / rows_per_request, vocab]
 * (row strides bias_stride, bias2_stride; either may be NULL);
 * vocab_mask: packed int32 [rows / rows_per_request, mask_words] (may be NULL).
 *   separate = 0 (:176-191): z = bias (0 when NULL), columns v < 32*mask_words
 *     whose mask bit (LSB first) is 0 become -inf, then z += bias2; every row
 *     of the request gets l = T(l + T(z)), T = rounding to the logits' dtype.
 *   separate = 1 (:193-213, no mask): l = T(l + T(bias)), then
 *     l = T(l + T(bias2)); a NULL tensor is not added.
 * ------------------------------------------------------------------------- */
LS_API int ls_add_request_bias(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t rows, int64_t vocab,
                               int32_t rows_per_request, const float* bias, int64_t bias_stride,
                               const int32_t* vocab_mask, int64_t mask_stride, int64_t mask_words,
                               const float* bias2, int64_t bias2_stride, int32_t separate, void* stream);

/* ---------------------------------------------------------------------------
 * Vocabulary (grammar) bitmask applied in place: replaces
 * SRT/constrained/triton_ops/bitmask_ops.py:84-141
 * (apply_token_bitmask_inplace_triton(logits, bitmask, indices)) and the
 * ROCm binding the grammar backend calls instead,
 * sgl_kernel.apply_token_bitmask_inplace_cuda (SRT/constrained/
 * xgrammar_backend.py:43-48,112-117,239-244).
 * logits [logits_rows, vocab] (fp32/bf16/fp16, row stride row_stride);
 * bitmask int32 [mask_rows, mask_words] (row stride mask_stride), LSB first:
 * bit (v & 31) of word v >> 5 equal to 0 sets logits[row, v] = -inf, for
 * v < min(vocab, 32 * mask_words); other columns are untouched.
 * mask_words <= ceil(vocab / 32) (the reference's width check).
 * indices (int32 or int64 [num_rows], may be NULL): the rows to mask; index i
 * selects both logits row i and bitmask row i (bitmask_ops.py:61-64).  An
 * index outside either tensor is skipped.  Without indices rows 0 ..
 * num_rows-1 are masked.
 * ------------------------------------------------------------------------- */
LS_API int ls_apply_token_bitmask(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t logits_rows,
                                  int64_t vocab, const int32_t* bitmask, int64_t mask_stride, int64_t mask_rows,
                                  int64_t mask_words, const void* indices, int32_t indices_dtype, int64_t num_rows,
                                  void* stream);

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
 *   kernel's candidate capacity gets accept = bonus = -1 and sets *status
 *   (may be NULL) to 1; the call clears *status first (on the stream).
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
   * (the middle interval holds the fallback and draft-scan kernels); a NULL
   * handle is not recorded. */
  void* const* timing_events;
  /* Which row-scan kernels to launch: 0 = both (each row runs in the one for
   * its path), 1 = only the raw-logit top-k scan (for callers that know every
   * row is top-k with repetition >= 1 and additive penalties <= 0; other rows
   * are still resolved exactly, more slowly), 2 = only the exact scan. */
  int32_t scan_hint;
  /* Optional verify-length cutoff (SRT/speculative/dspark_components/kernels/
   * cap_correct_len.py:44-52 applied as accept_sampling.py:151-157,185-186 does):
   * cutoff_verify_lens [batch] int32 or NULL; accept_lens[b] becomes
   * min(accepted, max(cutoff - 1, 0)), cap_trim[b] (int32, may be NULL) the
   * drafted tokens removed, and a capped request's bonus is its drafted
   * token at the cap. */
  const int32_t* cutoff_verify_lens;
  int32_t* cap_trim;
} ls_verify_sample_args;

LS_API int ls_verify_sample_workspace(int64_t batch, int32_t width, int64_t vocab, int32_t max_top_k,
                                      uint64_t* counter_bytes, uint64_t* scratch_bytes);
LS_API int ls_verify_sample(const ls_verify_sample_args* args, void* counters, uint64_t counter_bytes,
                            void* scratch, uint64_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Dense target distributions.
 *
 * ls_softmax_temp replaces SoftmaxTemp.execute
 * (SRT/speculative/dspark_components/kernels/softmax_temp.py:17-175):
 *   out[r, v] = softmax_v(logits[r, v] / temperatures[r / rows_per_request])
 *   as fp32, rows = batch * rows_per_request, out row stride out_row_stride.
 *
 * ls_target_probs replaces build_dflash_verify_target_probs
 * (SRT/speculative/dflash_utils.py:743-810): each row's distribution after
 * temperature, top-k (ties at the k-th value to the lowest index) and top-p,
 * written dense as fp32 [rows, vocab] with zeros outside the support.
 * top_ks / top_ps / min_ps as in ls_verify_sample (min-p, applied after
 * top-p, is not part of the reference function: pass NULL to match it).
 * Workspace from ls_target_probs_workspace.  A row whose support exceeds the
 * kernel's capacity is written as zeros and sets *status (may be NULL) to 1.
 * ------------------------------------------------------------------------- */
LS_API int ls_softmax_temp(const void* logits, int32_t logits_dtype, int64_t logits_row_stride, int64_t rows,
                           int64_t vocab, const float* temperatures, int32_t rows_per_request, float* out,
                           int64_t out_row_stride, void* stream);

typedef struct {
  const void* logits;
  int32_t logits_dtype;
  int64_t logits_row_stride;
  int64_t batch;
  int32_t rows_per_request;
  int64_t vocab;
  const float* temperatures;
  const int32_t* top_ks;
  const float* top_ps;
  const float* min_ps;
  int32_t max_top_k; /* host upper bound of top_ks (0 = 1024) */
  float* out;
  int64_t out_row_stride;
  int32_t* status;
  int32_t scan_hint; /* as in ls_verify_sample */
} ls_target_probs_args;

LS_API int ls_target_probs_workspace(int64_t batch, int32_t rows_per_request, int64_t vocab, int32_t max_top_k,
                                     uint64_t* counter_bytes, uint64_t* scratch_bytes);
LS_API int ls_target_probs(const ls_target_probs_args* args, void* counters, uint64_t counter_bytes, void* scratch,
                           uint64_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Split-engine verification on dense target probabilities.
 *
 * ls_decide_acceptance replaces src/longspark/engine/sampling.py:19-35
 * (decide_acceptance): lengths[b] = number of leading positions j < gamma
 * with uniforms[b,j] * sampled_q[b,j] < target_probs[b, j, candidates[b,j]]
 * (strict); target_rows[b, :] = target_probs[b, lengths[b], :] when
 * target_rows is not NULL.  target_probs rows are contiguous; element strides
 * are given for the other dimensions.
 *
 * ls_finish_sampling replaces src/longspark/engine/sampling.py:38-57
 * (finish_sampling with uniforms): per request, probs = target_rows[b], or
 * for a rejected request (b == rejected_rows[r]) the residual
 * max(target - rejected_q_rows[r], 0) normalised by its mass when the mass
 * exceeds 1e-8; tokens[b] = #{v : uniforms[b] >= cumsum(probs)[v]}, clamped
 * to vocab - 1.
 * ------------------------------------------------------------------------- */
LS_API int ls_decide_acceptance(const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                int64_t cand_stride_k, const float* sampled_q, int64_t q_stride_b,
                                const float* uniforms, int64_t uniform_stride_b, const float* target_probs,
                                int64_t probs_stride_b, int64_t probs_stride_k, int64_t batch, int32_t gamma,
                                int64_t vocab, int64_t* lengths, float* target_rows, int64_t rows_stride_b,
                                void* stream);
LS_API int ls_finish_sampling(const float* target_rows, int64_t rows_stride_b, const int64_t* rejected_rows,
                              int64_t n_rejected, const float* rejected_q_rows, int64_t q_stride_b,
                              const float* uniforms, int64_t batch, int64_t vocab, int64_t* tokens, void* stream);

/* ---------------------------------------------------------------------------
 * Dense-q chain rejection sampling: replaces
 * SRT/speculative/reject_sampling.py:159-204 (chain_speculative_sampling_triton
 * and its kernel :5-156) for the chain layout of
 * SRT/speculative/dflash_utils.py:216-272.
 * target_probs [batch, width, vocab] and draft_probs [batch, width-1, vocab]
 * fp32 with unit vocabulary stride; candidates and retrive_index
 * [batch, width] int32/int64; uniforms [batch, width-1] (unit column stride),
 * final_uniforms [batch].
 * Drafted token j = candidates[b, j+1] is accepted while
 * uniforms[b, j] * draft_probs[b, j, tok] < target_probs[b, j, tok]; with L
 * accepted, the bonus is drawn from max(p - q, 0) at row L (p at row L when
 * L = width-1): the first token whose running sum exceeds
 * final_uniforms[b] * total, vocab-1 when none does.
 * Outputs: accept_token_num[b] = L; for n <= L, accept_index[b, n] =
 * retrive_index[b, n] and predicts[retrive_index[b, n]] = candidates[b, n+1]
 * (n < L) or the bonus (n = L); other entries are left as they are.
 * predicts must hold every retrive_index value.  Running sums are fp64.
 * Workspace sizes from ls_chain_sampling_workspace; the counters must be zero
 * on entry and are zero again when the call's work ends.
 * ------------------------------------------------------------------------- */
typedef struct {
  const float* target_probs;
  int64_t tp_stride_b;
  int64_t tp_stride_k;
  const float* draft_probs;
  int64_t dp_stride_b;
  int64_t dp_stride_k;
  const void* candidates;
  int32_t candidates_dtype;
  int64_t cand_stride_b;
  int64_t cand_stride_k;
  const void* retrive_index;
  int32_t retrive_index_dtype;
  int64_t ri_stride_b;
  int64_t ri_stride_k;
  const float* uniforms;
  int64_t uniform_stride_b;
  const float* final_uniforms;
  int64_t batch;
  int32_t width;
  int64_t vocab;
  int32_t* predicts;
  int32_t* accept_index;
  int64_t ai_stride_b;
  int64_t ai_stride_k;
  int32_t* accept_token_num;
} ls_chain_sampling_args;

LS_API int ls_chain_sampling_workspace(int64_t batch, int64_t vocab, uint64_t* counter_bytes,
                                       uint64_t* scratch_bytes);
LS_API int ls_chain_speculative_sampling(const ls_chain_sampling_args* args, void* counters, uint64_t counter_bytes,
                                         void* scratch, uint64_t scratch_bytes, void* stream);

/* Fixed-width verify outputs: out_tokens[b, c] = bonus[b] if c == accept_lens[b],
 * else candidates[b, c+1] (0 in the last column); committed[b] = accept_lens[b] + 1
 * and next_lengths[b] = prefix_lens[b] + accept_lens[b] + 1 (both may be NULL;
 * next_lengths has prefix_dtype).  Replaces
 * SRT/speculative/draft_free_kv_dispatch.py:8-57 (finalize_verify_outputs) and
 * SRT/speculative/draft_free_kv_utils.py:386-408 (build_greedy_verify_out_tokens). */
LS_API int ls_finalize_verify_outputs(const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                      int64_t cand_stride_k, const void* accept_lens, int32_t lens_dtype,
                                      int64_t lens_stride, const void* bonus, int32_t bonus_dtype,
                                      int64_t bonus_stride, const void* prefix_lens, int32_t prefix_dtype,
                                      int64_t prefix_stride, int64_t batch, int32_t width, int64_t* out_tokens,
                                      int32_t* committed, void* next_lengths, void* stream);

/* Committed verify rows into the request-to-token map: replaces
 * SRT/speculative/draft_free_kv_info.py:32-82 (_assign_fixed_verify_cache_locs).
 * For request b and i < commit_lens[b] (clamped to [0, width]):
 * req_to_token[req_pool_indices[b] * rtt_stride + start_offset[b] + i] =
 * verify_cache_locs[b * locs_stride_b + i]; positions outside [0, pool_len)
 * are skipped.  Index tensors int32/int64; req_to_token int32. */
LS_API int ls_assign_verify_cache_locs(const void* req_pool_indices, int32_t slots_dtype, const void* start_offset,
                                       int32_t start_dtype, const void* commit_lens, int32_t commit_dtype,
                                       const void* verify_cache_locs, int32_t locs_dtype, int64_t locs_stride_b,
                                       int32_t* req_to_token, int64_t rtt_stride, int64_t pool_len, int64_t batch,
                                       int32_t width, void* stream);

/* ---------------------------------------------------------------------------
 * Drafter proposal step: replaces
 * SRT/speculative/dspark_components/kernels/sample_step_tokens_with_q.py:72-382
 * (sample_step_tokens_with_q: the exponential race with the sampled q).
 * logits [rows, vocab] (fp32/bf16/fp16, unit column stride), temperatures
 * [rows] fp32, exp_noise [rows, vocab] fp32 (E ~ Exp(1), row stride
 * noise_row_stride).  Per row: s = l / T for finite l (else -inf),
 * p = softmax(s); next_tokens[r] = argmax p / E (lowest index on ties),
 * sampled_q[r] = p at that token.  A row with a NaN or +inf logit, an invalid
 * l / T, noise outside (0, inf) at a finite entry, T outside (0, inf), or no
 * finite entry gets token 0 and q = NaN and sets *status to 1 (status may be
 * NULL; the caller clears it).  Workspace sizes from ls_sample_step_workspace;
 * the counters must be zero on entry and are zero again when the call's work
 * ends.
 * ------------------------------------------------------------------------- */
LS_API int ls_sample_step_workspace(int64_t rows, int64_t vocab, uint64_t* counter_bytes, uint64_t* scratch_bytes);
LS_API int ls_sample_step(const void* logits, int32_t logits_dtype, int64_t logits_row_stride, int64_t rows,
                          int64_t vocab, const float* temperatures, const float* exp_noise, int64_t noise_row_stride,
                          int64_t* next_tokens, float* sampled_q, int32_t* status, void* counters,
                          uint64_t counter_bytes, void* scratch, uint64_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Recent-window page tables, window gather and ring append.
 * ------------------------------------------------------------------------- */

/* Raw256 page table: page_table[b, i] = req_to_token[slot_b, seq_b - raw_b + i]
 * for i < raw_b = min(seq_b, window), 0 for i >= raw_b; raw_lengths[b] = raw_b
 * (may be NULL).  req_to_token is int32 [slots, T] with element strides.
 * Replaces SRT/speculative/global16_raw256_draft_fused.py:372-413
 * (build_raw256_page_table, kernel :35-65) and the torch path
 * SRT/speculative/global16_raw256.py:1343-1361. */
LS_API int ls_raw_page_table(const int32_t* req_to_token, int64_t rtt_stride_b, int64_t rtt_stride_t,
                             const void* req_pool_indices, int32_t slots_dtype, const void* seq_lens,
                             int32_t seq_lens_dtype, int64_t batch, int32_t window, int32_t* page_table,
                             int64_t page_table_stride, int32_t* raw_lengths, void* stream);

/* Ring page table: pages[b, i] = slot_b * window + (len_b - raw_b + i) mod window,
 * raw_b = min(len_b, window).  Replaces src/longspark/engine/draft.py:14-21
 * (ring_page_table). */
LS_API int ls_ring_page_table(const void* slots, int32_t slots_dtype, const void* lengths, int32_t lengths_dtype,
                              int64_t batch, int32_t window, int32_t* pages, int64_t pages_stride,
                              int32_t* raw_lengths, void* stream);

/* Recent-window gather from a paged KV pool into a dense head-major view:
 *   out[b, l, kv, h, i, :] = pool_kv[l][loc(b, seq_b - raw_b + i), h, :]  for i < raw_b,
 *   zero for raw_b <= i < window,
 * raw_b = min(seq_b, window), loc(b, t) = page_table[row_b, t / page_size] *
 * page_size + t % page_size, row_b = table_rows[b] (NULL: b).  k_layers /
 * v_layers are device arrays [n_layers] of per-layer base addresses; a
 * token row is token_stride elements, heads head_stride apart (head rows,
 * strides and output 16-byte aligned).  With page_size 1 and table_rows =
 * req_pool_indices this reads req_to_token directly.
 * Replaces the per-layer k[locations] export of src/longspark/engine/
 * target.py:213-228 and the gather the page table of
 * SRT/speculative/global16_raw256.py:1307-1361 feeds. */
LS_API int ls_kv_window_gather(const uint64_t* k_layers, const uint64_t* v_layers, int32_t n_layers,
                               int32_t dtype, int64_t token_stride, int64_t head_stride, int32_t heads,
                               int32_t head_dim, const int32_t* page_table, int64_t page_table_stride,
                               const void* table_rows, int32_t table_rows_dtype, int32_t page_size,
                               const void* seq_lens, int32_t seq_lens_dtype, int64_t batch, int32_t window,
                               void* out, int64_t out_stride_b, int64_t out_stride_l, int64_t out_stride_kv,
                               int64_t out_stride_h, int64_t out_stride_w, int32_t* raw_lengths, void* stream);

/* Ring append: for each request b, rows j < counts[b] of the packed source
 * (row off_b + j, off_b = sum of earlier counts; or src_locs[off_b + j] when
 * src_locs is given) are written to ring row
 * slots[b] * window + (prev_lengths[b] + j) mod window of every layer, K and V.
 * Layer bases are device arrays; row_bytes and both strides multiples of 16.
 * Replaces src/longspark/engine/draft.py:207-212, 255-259 (self.keys[:,
 * ring_locs] = keys) fused with the target-side row export of
 * src/longspark/engine/target.py:213-228 (src_locs = the export locations). */
LS_API int ls_ring_append(const uint64_t* src_k_layers, const uint64_t* src_v_layers, const uint64_t* dst_k_layers,
                          const uint64_t* dst_v_layers, int32_t n_layers, int64_t row_bytes,
                          int64_t src_row_stride_bytes, int64_t dst_row_stride_bytes, const void* src_locs,
                          int32_t src_locs_dtype, const int32_t* slots, const int32_t* prev_lengths,
                          const int32_t* counts, int64_t batch, int32_t window, void* stream);

/* ---------------------------------------------------------------------------
 * Summary (Global16) state: cached position scores and the online-softmax
 * merge of accepted rows.
 *
 * Geometry: Hq query heads over Hkv KV heads (query head h uses KV head
 * h / (Hq / Hkv)), S summary rows per query head, W new rows per request
 * (W <= 32), head_dim D in {64, 128, 256}; queries, keys and values bf16 or
 * fp16 (one dtype), scores / state / LSE fp32.  All element strides; the
 * last (D) dimension is contiguous and rows of queries, keys and values are
 * 16-byte aligned.
 *
 *   scores  s[b,h,r,w] = scale * sum_d q[b,h,r,d] k[b,w,h/g,d]
 *           (softcap > 0: softcap * tanh(s / softcap)), fp32 accumulation;
 *   merge   over w < len_b = accept_lens[b]:
 *           d = logsumexp_w s, m = M + log(exp(lse - M) + exp(d - M)), M = max(lse, d),
 *           out <- out * exp(lse - m) + sum_w exp(s_w - m) v[w], lse <- m,
 *           on state row state_slots[b] (NULL: b); len_b <= 0 leaves the row unchanged.
 *
 * Replaces SRT/speculative/global16_raw256_incremental.py:400-456
 * (cache_position_scores), :459-584 (merge_accepted_positions_) and the
 * GQA-5 adapter src/longspark/patches/gqa5_attention.py:43-106; the fused
 * update covers the per-layer score+merge loop of
 * src/longspark/engine/draft.py:243-253 for all layers in one launch.
 * ------------------------------------------------------------------------- */
enum { LS_SUMMARY_SCORES = 1, LS_SUMMARY_MERGE = 2, LS_SUMMARY_UPDATE = 3 };

/* Rows of a key or value source.  Layer l starts at layers[l] (device array)
 * or, when layers is NULL, at base + l * stride_layer elements.  Row (b, w)
 * of KV head h is at  loc * stride_loc + h * stride_h  when located (loc from
 * the accepted-location table), else  b * stride_b + w * stride_w + h * stride_h. */
typedef struct ls_kv_rows {
  const void* base;
  const uint64_t* layers;
  int64_t stride_layer;
  int64_t stride_b, stride_w;
  int64_t stride_loc;
  int64_t stride_h;
  int32_t located;
} ls_kv_rows;

typedef struct ls_summary_args {
  int64_t batch;
  int32_t layers, q_heads, kv_heads, rows, width, head_dim;
  int32_t dtype;                       /* LS_BF16 or LS_F16 */
  float softmax_scale, softcap;
  /* queries [L][B][Hq][S][D] (stride 0 over requests for a shared query) */
  const void* query;
  int64_t q_stride_l, q_stride_b, q_stride_h, q_stride_s;
  ls_kv_rows keys, values;
  /* scores [L][B][Hq][S][W] fp32: written by SCORES, read by MERGE, unused by UPDATE */
  float* scores;
  int64_t sc_stride_l, sc_stride_b, sc_stride_h, sc_stride_s, sc_stride_w;
  /* state [C][L][Hq][S][D] and LSE [C][L][Hq][S] fp32, updated in place */
  float* state_output;
  int64_t so_stride_c, so_stride_l, so_stride_h, so_stride_s;
  float* state_lse;
  int64_t sl_stride_c, sl_stride_l, sl_stride_h, sl_stride_s;
  const int32_t* state_slots;          /* [B] or NULL */
  /* accepted cache locations: fixed [B][W] (element strides), or compact
   * (flat; request b's rows at locs[off_b + w], off_b = sum of earlier
   * accept_lens, written to accept_offsets[b] when accept_offsets is given) */
  const void* locs;
  int32_t locs_dtype;                  /* LS_I32 or LS_I64 */
  int64_t locs_stride_b, locs_stride_w;
  int32_t compact_locs;
  int32_t* accept_offsets;
  const int32_t* accept_lens;          /* [B] int32 */
} ls_summary_args;

LS_API int ls_summary_scores(const ls_summary_args* args, void* stream);
LS_API int ls_summary_merge(const ls_summary_args* args, void* stream);
LS_API int ls_summary_update(const ls_summary_args* args, void* stream);

/* ---- Global16 prefill initialisation ------------------------------------
 * Replaces Global16Raw256VerifyContext.run_prefill_global_attention
 * (SRT/speculative/global16_raw256.py:668-784) as driven by
 * TargetClient._prefill_summaries (src/longspark/engine/target.py:230-253):
 * one non-causal attention of the summary query rows over each request's
 * whole prefix, read through its location table (req_to_token rows,
 * page size 1), returning the output and the natural-log LSE that seed the
 * incrementally merged state.  The reference runs FA3 once per selected
 * layer; here every selected layer goes in one launch, split along the prefix.
 *   output[l][b][h][s][:] = sum_t softmax_t(score) * V[l][loc(b,t)][h/G]
 *   lse[l][b][h][s]       = logsumexp_t(score),  t < seq_lens[b]
 *   score = softcap > 0 ? softcap * tanh(q.k * scale / softcap) : q.k * scale
 * The attention weights enter the weighted sum of values as 16-bit values of
 * the key type (FA3 rounds P to the element type before its P.V product;
 * the row sums use the fp32 weights), and the output is rounded to
 * round_output's type when that is set (FA3 returns the query dtype).  An
 * empty prefix gives a zero output and LSE -inf. */
typedef struct ls_prefill_args {
  int64_t batch;
  int32_t layers, q_heads, kv_heads, rows, head_dim;
  int32_t dtype;                       /* LS_BF16 or LS_F16 (queries, keys, values) */
  float softmax_scale, softcap;
  /* queries [L][B][Hq][S][D] (stride 0 over requests for a shared query) */
  const void* query;
  int64_t q_stride_l, q_stride_b, q_stride_h, q_stride_s;
  ls_kv_rows keys, values;             /* located rows (located = 1) */
  /* location table [B][>= max_len] (req_to_token rows), int32 or int64 */
  const void* page_table;
  int32_t pt_dtype;
  int64_t pt_stride_b;
  int64_t max_len;                     /* table columns; every seq_lens[b] <= max_len */
  const int32_t* seq_lens;             /* [B] */
  /* output [L][B][Hq][S][D] and LSE [L][B][Hq][S] fp32 (element strides) */
  float* output;
  int64_t o_stride_l, o_stride_b, o_stride_h, o_stride_s;
  float* lse;
  int64_t l_stride_l, l_stride_b, l_stride_h, l_stride_s;
  int32_t round_output;                /* LS_F32 (no rounding), LS_BF16 or LS_F16 */
  int32_t chunk;                       /* prefix tokens per workgroup, a multiple of 64; 0 = from the sizes */
} ls_prefill_args;

/* Scratch bytes ls_global16_prefill needs for these arguments (0 when the
 * prefix is not split). */
LS_API int ls_global16_prefill_workspace(const ls_prefill_args* args, int64_t* scratch_bytes);
LS_API int ls_global16_prefill(const ls_prefill_args* args, void* scratch, int64_t scratch_bytes, void* stream);

/* ---- Drafter attention over the refreshed views ----------------------------
 * Replaces fused_global_local_raw_attention
 * (SRT/speculative/global16_raw256_draft_all_attention.py:52-281,348-416):
 * for each request and query head, 7 query rows attend over
 *   Raw256  rows page_table[b, t] (t < raw_lengths[b]) of the page-size-1
 *           key/value cache, scores (q.k) * scale;
 *   Global16 16 rows per query head: keys global_keys[b][h], values the fp32
 *           summary state global_values[state_slots[b]][h] rounded to bf16,
 *           scores bf16(q.k) * scale;
 *   Local7  7 rows per KV head with visibility local_mask[b][row][src],
 *           scores bf16(q.k) * scale;
 * folded as online-softmax steps in that order (raw in blocks of 64 rows),
 * each step's weights entering the weighted sum of values as bf16.  Output
 * bf16.  head_dim 128, bf16 tensors with a contiguous head dimension; every
 * stride in elements.  At most 16 query heads per KV head. */
typedef struct ls_draft_attention_args {
  int64_t batch;
  int32_t q_heads, kv_heads;
  float softmax_scale;
  const void* query;                   /* [B][Hq][7][128] bf16 */
  int64_t q_stride_b, q_stride_h, q_stride_r;
  const void* global_keys;             /* [B][Hq][16][128] bf16 */
  int64_t gk_stride_b, gk_stride_h, gk_stride_g;
  const float* global_values;          /* [C][Hq][16][128] fp32 (state pool) */
  int64_t gv_stride_b, gv_stride_h, gv_stride_g;
  const int32_t* state_slots;          /* [B] */
  const void* local_keys;              /* [B][Hkv][7][128] bf16 */
  int64_t lk_stride_b, lk_stride_h, lk_stride_l;
  const void* local_values;            /* [B][Hkv][7][128] bf16 */
  int64_t lv_stride_b, lv_stride_h, lv_stride_l;
  const uint8_t* local_mask;           /* [B][7][7] bool */
  int64_t lm_stride_b, lm_stride_r, lm_stride_l;
  const void* key_cache;               /* [S][1][Hkv][128] bf16 */
  int64_t kc_stride_s, kc_stride_h;
  const void* value_cache;
  int64_t vc_stride_s, vc_stride_h;
  const int32_t* page_table;           /* [B][256] */
  int64_t pt_stride_b;
  const int32_t* raw_lengths;          /* [B], clamped to [0, 256] */
  void* output;                        /* [B][Hq][7][128] bf16 */
  int64_t o_stride_b, o_stride_h, o_stride_r;
  /* ls_draft_merge only: the window attention computed elsewhere (FA3 in the
   * reference) as output [B*7][Hq][128] bf16 and natural-log LSE [B*7][Hq]
   * fp32 (token row b*7 + r), and the softcap of the summary/local scores */
  const void* raw_output;
  int64_t ro_stride_t, ro_stride_h;
  const float* raw_lse;
  int64_t rl_stride_t, rl_stride_h;
  float softcap;
} ls_draft_attention_args;

LS_API int ls_draft_attention(const ls_draft_attention_args* args, void* stream);

/* Replaces fused_global_local_raw_merge
 * (SRT/speculative/global16_raw256_draft_fused.py:72-312,417-479), the
 * reference's default drafter path after its FA3 window attention: the
 * Global16 and Local7 sources are each normalised on their own (weighted sum
 * of bf16 weights and values rounded to bf16, divided by the fp32 sum; scores
 * bf16(q.k) * scale, then softcap * tanh(s / softcap) when softcap > 0), and
 * the three outputs are merged by their LSEs:
 *   out = (raw * e^(lse_r - M) + global * e^(lse_g - M) + local * e^(lse_l - M)) / sum,
 * M the largest LSE, a row with no visible local row leaving that term out.
 * Uses every field of ls_draft_attention_args except key_cache, value_cache,
 * page_table and raw_lengths. */
LS_API int ls_draft_merge(const ls_draft_attention_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LONGSPARK_AMD_H_ */
