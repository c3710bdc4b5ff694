// Greedy chain verification in one launch: every row's argmax, then the
// accepted prefix and the bonus token of each request.
//
// Grid: rows * slices workgroups of 256 threads.  A workgroup streams one
// slice of one row with 16-byte loads and reduces it to (max, first index).
// The last workgroup to finish a row merges the row's slices; the last row to
// finish a request compares its drafted tokens with the row argmaxes.
//
// Reference semantics: src/longspark/engine/target.py:474-477 and
// vendor/sglang/python/sglang/srt/speculative/dflash_utils.py:564-602.
#include "common.h"

namespace ls {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte loads in flight per thread per step

// Slices per row: enough workgroups to cover 256 CUs several times over,
// without cutting a row into pieces smaller than ~8K elements.
int greedy_slices(int64_t rows, int64_t vocab) {
  int64_t want = (2048 + rows - 1) / rows;
  int64_t max_by_len = vocab / 8192;
  if (max_by_len < 1) max_by_len = 1;
  if (want > max_by_len) want = max_by_len;
  if (want > 64) want = 64;
  if (want < 1) want = 1;
  return static_cast<int>(want);
}

struct GreedyWs {
  ArgMax* partials;    // [rows * slices]
  int32_t* truth;      // [rows]
  uint32_t* row_cnt;   // [rows]
  uint32_t* req_cnt;   // [batch]
};

uint64_t greedy_ws_bytes(int64_t batch, int64_t rows, int slices) {
  auto up = [](uint64_t x) { return (x + 255) & ~uint64_t(255); };
  return up(sizeof(ArgMax) * rows * slices) + up(4 * rows) + up(4 * rows) + up(4 * batch);
}

GreedyWs greedy_ws(void* base, int64_t batch, int64_t rows, int slices) {
  auto up = [](uint64_t x) { return (x + 255) & ~uint64_t(255); };
  char* p = static_cast<char*>(base);
  GreedyWs w;
  w.partials = reinterpret_cast<ArgMax*>(p);
  p += up(sizeof(ArgMax) * rows * slices);
  w.truth = reinterpret_cast<int32_t*>(p);
  p += up(4 * rows);
  w.row_cnt = reinterpret_cast<uint32_t*>(p);
  p += up(4 * rows);
  w.req_cnt = reinterpret_cast<uint32_t*>(p);
  (void)batch;
  return w;
}

template <typename Tag, bool kVec>
__device__ __forceinline__ ArgMax scan_slice(const typename Tag::storage* row, int64_t b, int64_t e) {
  using S = typename Tag::storage;
  constexpr int P = Tag::kPerVec;
  ArgMax best{-INFINITY, 0x7fffffff};
  const int tid = threadIdx.x;
  if constexpr (kVec) {
    // [b, e) starts on a vector boundary; the last slice may end mid-vector.
    const int64_t nvec = (e - b) / P;
    const uint4* vp = reinterpret_cast<const uint4*>(row + b);
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kThreads < nvec; i += kUnroll * kThreads) {
      uint4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = load16_stream(vp + i + u * kThreads);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float f[P];
        unpack16<Tag>(v[u], f);
        const int base = static_cast<int>(b + (i + u * kThreads) * P);
#pragma unroll
        for (int k = 0; k < P; ++k) {
          if (f[k] > best.v) { best.v = f[k]; best.i = base + k; }
        }
      }
    }
    for (; i < nvec; i += kThreads) {
      float f[P];
      unpack16<Tag>(load16_stream(vp + i), f);
      const int base = static_cast<int>(b + i * P);
#pragma unroll
      for (int k = 0; k < P; ++k) {
        if (f[k] > best.v) { best.v = f[k]; best.i = base + k; }
      }
    }
    for (int64_t j = b + nvec * P + tid; j < e; j += kThreads) {
      float f = to_f32<S>(row[j]);
      if (f > best.v) { best.v = f; best.i = static_cast<int>(j); }
    }
  } else {
    // Unaligned rows: element-wise, each thread walking increasing indices.
    for (int64_t j = b + tid; j < e; j += kThreads) {
      float f = to_f32<S>(row[j]);
      if (f > best.v) { best.v = f; best.i = static_cast<int>(j); }
    }
  }
  // A thread that saw only -inf keeps index INT_MAX; give it its first
  // element's index so an all -inf row still returns the first index.
  if (best.v == -INFINITY) {
    int64_t first = b + (kVec ? static_cast<int64_t>(tid) * P : tid);
    best.i = first < e ? static_cast<int>(first) : 0x7fffffff;
  }
  return best;
}

template <typename Tag, bool kVec, typename CandT>
__global__ __launch_bounds__(kThreads) void greedy_verify_kernel(
    const typename Tag::storage* __restrict__ logits, int64_t row_stride,
    const CandT* __restrict__ cand, int64_t csb, int64_t csk, int first_col, int width,
    int64_t vocab, int slices, GreedyWs ws, const int32_t* __restrict__ cutoff,
    int32_t* __restrict__ accept_out, int64_t* __restrict__ bonus_out, int32_t* __restrict__ truth_out,
    int32_t* __restrict__ trim_out) {
  __shared__ ArgMax red[kThreads / kWave];
  __shared__ int is_last;
  const int64_t row = blockIdx.x / slices;
  const int slice = blockIdx.x % slices;
  const SliceRange r = slice_range(vocab, slices, slice, Tag::kPerVec);
  const typename Tag::storage* rp = logits + row * row_stride;

  ArgMax best = scan_slice<Tag, kVec>(rp, r.v_begin, r.v_end);
  best = wave_argmax(best);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  if (lane == 0) red[wid] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgMax m = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) m = argmax_merge(m, red[w]);
    ws.partials[row * slices + slice] = m;
    is_last = (arrive(&ws.row_cnt[row]) == static_cast<uint32_t>(slices - 1));
  }
  __syncthreads();
  if (!is_last) return;

  // Last slice of this row: merge the row's partials in wave 0.
  if (threadIdx.x < kWave) {
    __threadfence();
    ArgMax m{-INFINITY, 0x7fffffff};
    for (int s = threadIdx.x; s < slices; s += kWave) m = argmax_merge(m, ws.partials[row * slices + s]);
    m = wave_argmax(m);
    if (threadIdx.x == 0) {
      reset_counter(&ws.row_cnt[row]);
      ws.truth[row] = m.i;
      if (truth_out) truth_out[row] = m.i;
      const int64_t req = row / width;
      if (arrive(&ws.req_cnt[req]) == static_cast<uint32_t>(width - 1)) {
        // Last row of this request: accepted prefix and bonus.
        __threadfence();
        reset_counter(&ws.req_cnt[req]);
        const int32_t* t = ws.truth + req * width;
        int len = 0;
        while (len < width - 1 &&
               static_cast<int64_t>(cand[req * csb + static_cast<int64_t>(first_col + len) * csk]) ==
                   static_cast<int64_t>(__hip_atomic_load(t + len, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)))
          ++len;
        int trim = 0;
        if (cutoff) {
          int cap = cutoff[req] - 1;
          cap = cap < 0 ? 0 : (cap > width - 1 ? width - 1 : cap);
          if (len > cap) { trim = len - cap; len = cap; }
        }
        if (trim_out) trim_out[req] = trim;
        accept_out[req] = len;
        bonus_out[req] = __hip_atomic_load(t + len, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <typename Tag, typename CandT>
int launch_greedy(const void* logits, int64_t row_stride, const void* cand, int64_t csb, int64_t csk,
                  int first_col, int64_t batch, int width, int64_t vocab, const int32_t* cutoff,
                  int32_t* accept, int64_t* bonus, int32_t* truth, int32_t* trim, void* workspace,
                  hipStream_t stream) {
  const int64_t rows = batch * width;
  const int slices = greedy_slices(rows, vocab);
  GreedyWs ws = greedy_ws(workspace, batch, rows, slices);
  using S = typename Tag::storage;
  const bool vec = aligned16(logits) && ((row_stride * sizeof(S)) % 16 == 0);
  dim3 grid(static_cast<unsigned>(rows * slices));
  if (vec)
    greedy_verify_kernel<Tag, true, CandT><<<grid, kThreads, 0, stream>>>(
        static_cast<const S*>(logits), row_stride, static_cast<const CandT*>(cand), csb, csk, first_col,
        width, vocab, slices, ws, cutoff, accept, bonus, truth, trim);
  else
    greedy_verify_kernel<Tag, false, CandT><<<grid, kThreads, 0, stream>>>(
        static_cast<const S*>(logits), row_stride, static_cast<const CandT*>(cand), csb, csk, first_col,
        width, vocab, slices, ws, cutoff, accept, bonus, truth, trim);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

}  // namespace
}  // namespace ls

extern "C" uint64_t ls_verify_greedy_workspace_bytes(int64_t batch, int32_t width, int64_t vocab) {
  if (batch <= 0 || width <= 0 || vocab <= 0) return 0;
  const int64_t rows = batch * width;
  return ls::greedy_ws_bytes(batch, rows, ls::greedy_slices(rows, vocab));
}

extern "C" int ls_verify_greedy(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                int64_t cand_stride_k, int32_t cand_first_col, int64_t batch, int32_t width,
                                int64_t vocab, const int32_t* cutoff_verify_lens, int32_t* accept_lens,
                                int64_t* bonus, int32_t* truth, int32_t* cap_trim, void* workspace,
                                uint64_t workspace_bytes, void* stream) {
  using namespace ls;
  LS_CHECK(batch > 0 && width >= 2 && vocab > 0, LS_ERR_SHAPE,
           "ls_verify_greedy: need batch > 0, width >= 2, vocab > 0 (got %lld, %d, %lld)",
           (long long)batch, width, (long long)vocab);
  LS_CHECK(vocab < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_verify_greedy: vocab must fit int32");
  LS_CHECK(logits_row_stride >= vocab, LS_ERR_SHAPE, "ls_verify_greedy: row stride %lld < vocab %lld",
           (long long)logits_row_stride, (long long)vocab);
  LS_CHECK(cand_first_col == 0 || cand_first_col == 1, LS_ERR_VALUE,
           "ls_verify_greedy: cand_first_col must be 0 or 1");
  LS_CHECK(logits && candidates && accept_lens && bonus, LS_ERR_VALUE, "ls_verify_greedy: null pointer");
  const uint64_t need = ls_verify_greedy_workspace_bytes(batch, width, vocab);
  LS_CHECK(workspace && workspace_bytes >= need, LS_ERR_WORKSPACE,
           "ls_verify_greedy: workspace of %llu bytes required", (unsigned long long)need);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LS_GREEDY_CAND(TAG)                                                                          \
  if (candidates_dtype == LS_I32)                                                                    \
    return launch_greedy<TAG, int32_t>(logits, logits_row_stride, candidates, cand_stride_b,         \
                                       cand_stride_k, cand_first_col, batch, width, vocab,           \
                                       cutoff_verify_lens, accept_lens, bonus, truth, cap_trim,     \
                                       workspace, s);                     \
  if (candidates_dtype == LS_I64)                                                                    \
    return launch_greedy<TAG, int64_t>(logits, logits_row_stride, candidates, cand_stride_b,         \
                                       cand_stride_k, cand_first_col, batch, width, vocab,           \
                                       cutoff_verify_lens, accept_lens, bonus, truth, cap_trim,     \
                                       workspace, s);                     \
  return fail(LS_ERR_DTYPE, "ls_verify_greedy: candidates must be int32 or int64");
  if (logits_dtype == LS_BF16) { LS_GREEDY_CAND(BF16) }
  if (logits_dtype == LS_F16) { LS_GREEDY_CAND(F16) }
  if (logits_dtype == LS_F32) { LS_GREEDY_CAND(F32) }
#undef LS_GREEDY_CAND
  return fail(LS_ERR_DTYPE, "ls_verify_greedy: logits must be bf16, fp16 or fp32");
}
