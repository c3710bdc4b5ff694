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

#ifdef __cplusplus
}
#endif

#endif /* LONGSPARK_AMD_H_ */
