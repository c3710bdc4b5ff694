// Greedy chain verification in one launch: every row's argmax, then the
// accepted prefix and the bonus token of each request.
//
// Grid: rows * slices workgroups of 256 threads.  A workgroup streams one
// slice of one row with 16-byte loads and reduces it to (max, first index),
// which it folds into the row's packed argmax key with one atomic max.  The
// last workgroup to finish a request (counted on a per-request counter) takes
// the request's row keys -- returning them to zero -- and compares the drafted
// tokens with the row argmaxes.
//
// Reference semantics: src/longspark/engine/target.py:474-477 and
// vendor/sglang/python/sglang/srt/speculative/dflash_utils.py:564-602.
#include "common.h"

#include <mutex>

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
  uint64_t* row_key;   // counters: [rows] packed argmax keys, zero at rest
  uint32_t* req_cnt;   // counters: [batch] finished workgroups per request
};

inline uint64_t up256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

void greedy_ws_sizes(int64_t batch, int64_t rows, uint64_t* counters, uint64_t* scratch) {
  *counters = up256(8 * rows) + up256(4 * batch);
  *scratch = 0;
}

GreedyWs greedy_ws(void* counters, int64_t rows) {
  GreedyWs w;
  char* c = static_cast<char*>(counters);
  w.row_key = reinterpret_cast<uint64_t*>(c);
  w.req_cnt = reinterpret_cast<uint32_t*>(c + up256(8 * rows));
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
  __shared__ int t[64];  // row argmaxes of the request (last workgroup only)
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
  if (threadIdx.x != 0) return;

  ArgMax m = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / kWave; ++w) m = argmax_merge(m, red[w]);
  if (m.i != 0x7fffffff) atomic_max_u64(&ws.row_key[row], argmax_key(m.v, m.i));
  const int64_t req = row / width;
  const uint32_t per_req = static_cast<uint32_t>(width) * static_cast<uint32_t>(slices);
  if (arrive(&ws.req_cnt[req]) != per_req - 1) return;

  // Last workgroup of this request: take the row keys (resetting them), then
  // the accepted prefix and the bonus token.
  atomic_take_u32(&ws.req_cnt[req]);
  int len = 0;
  bool matching = true;
  for (int j = 0; j < width; ++j) {
    const int idx = argmax_key_index(atomic_take_u64(&ws.row_key[req * width + j]));
    t[j] = idx;
    if (truth_out) truth_out[req * width + j] = idx;
    if (matching && j < width - 1) {
      if (static_cast<int64_t>(cand[req * csb + static_cast<int64_t>(first_col + j) * csk]) == idx)
        ++len;
      else
        matching = false;
    }
  }
  int trim = 0;
  if (cutoff) {
    int cap = cutoff[req] - 1;
    cap = cap < 0 ? 0 : (cap > width - 1 ? width - 1 : cap);
    if (len > cap) { trim = len - cap; len = cap; }
  }
  if (trim_out) trim_out[req] = trim;
  accept_out[req] = len;
  bonus_out[req] = t[len];
}

template <typename Tag, typename CandT>
int launch_greedy(const void* logits, int64_t row_stride, const void* cand, int64_t csb, int64_t csk,
                  int first_col, int64_t batch, int width, int64_t vocab, const int32_t* cutoff,
                  int32_t* accept, int64_t* bonus, int32_t* truth, int32_t* trim, void* counters,
                  void* scratch, hipStream_t stream) {
  const int64_t rows = batch * width;
  const int slices = greedy_slices(rows, vocab);
  GreedyWs ws = greedy_ws(counters, rows);
  (void)scratch;
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

// ------------------------------------------------- allocation-free entry ---
//
// ls_verify_greedy_noalloc keeps its counters in this file-scope device
// array instead of a caller workspace.  Every GPU the library runs on holds
// its own copy until the process ends.  In host code the array's name is
// only a host-side stand-in: its device address comes from
// hipGetSymbolAddress, looked up once per device (with that device current)
// and kept in noalloc_ptr[], and only that address is passed to kernels.
constexpr uint64_t kNoAllocBytes = uint64_t(1) << 20;  // 1 MiB: rows*8 + batch*4 (256-byte aligned parts)
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char noalloc_scratch[kNoAllocBytes];
void* noalloc_ptr[kMaxDevices] = {};
std::mutex noalloc_mutex;

__global__ __launch_bounds__(256) void zero_kernel(uint4* p, uint64_t n16) {
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<uint64_t>(gridDim.x) * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's copy of the array, set up on the first call on that
// device: its address from hipGetSymbolAddress, then cleared with a kernel on
// `stream` (the counters must start at zero; every call leaves them zero).
int noalloc_counters(hipStream_t stream, void** out) {
  int dev = 0;
  LS_CHECK(hipGetDevice(&dev) == hipSuccess, LS_ERR_LAUNCH, "ls_verify_greedy_noalloc: hipGetDevice failed");
  LS_CHECK(dev >= 0 && dev < kMaxDevices, LS_ERR_VALUE, "ls_verify_greedy_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(noalloc_mutex);
  if (!noalloc_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(noalloc_scratch));
    LS_CHECK(e == hipSuccess && ptr, LS_ERR_LAUNCH, "ls_verify_greedy_noalloc: hipGetSymbolAddress failed: %s",
             hipGetErrorString(e));
    zero_kernel<<<dim3(256), 256, 0, stream>>>(static_cast<uint4*>(ptr), kNoAllocBytes / 16);
    LS_LAUNCH_CHECK();
    noalloc_ptr[dev] = ptr;
  }
  *out = noalloc_ptr[dev];
  return LS_OK;
}

}  // namespace
}  // namespace ls

extern "C" int ls_verify_greedy_workspace(int64_t batch, int32_t width, int64_t vocab,
                                         uint64_t* counter_bytes, uint64_t* scratch_bytes) {
  LS_CHECK(batch > 0 && width > 0 && vocab > 0 && counter_bytes && scratch_bytes, LS_ERR_SHAPE,
           "ls_verify_greedy_workspace: need positive sizes and output pointers");
  const int64_t rows = batch * width;
  ls::greedy_ws_sizes(batch, rows, counter_bytes, scratch_bytes);
  return LS_OK;
}

extern "C" int ls_verify_greedy(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                int64_t cand_stride_k, int32_t cand_first_col, int64_t batch, int32_t width,
                                int64_t vocab, const int32_t* cutoff_verify_lens, int32_t* accept_lens,
                                int64_t* bonus, int32_t* truth, int32_t* cap_trim, void* counters,
                                uint64_t counter_bytes, void* scratch, uint64_t scratch_bytes,
                                void* stream) {
  using namespace ls;
  LS_CHECK(batch > 0 && width >= 2 && width <= 64 && vocab > 0, LS_ERR_SHAPE,
           "ls_verify_greedy: need batch > 0, 2 <= width <= 64, vocab > 0 (got %lld, %d, %lld)",
           (long long)batch, width, (long long)vocab);
  LS_CHECK(vocab < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_verify_greedy: vocab must fit int32");
  LS_CHECK(logits_row_stride >= vocab, LS_ERR_SHAPE, "ls_verify_greedy: row stride %lld < vocab %lld",
           (long long)logits_row_stride, (long long)vocab);
  LS_CHECK(cand_first_col == 0 || cand_first_col == 1, LS_ERR_VALUE,
           "ls_verify_greedy: cand_first_col must be 0 or 1");
  LS_CHECK(logits && candidates && accept_lens && bonus, LS_ERR_VALUE, "ls_verify_greedy: null pointer");
  uint64_t need_c = 0, need_s = 0;
  ls_verify_greedy_workspace(batch, width, vocab, &need_c, &need_s);
  LS_CHECK(counters && counter_bytes >= need_c && (need_s == 0 || (scratch && scratch_bytes >= need_s)),
           LS_ERR_WORKSPACE,
           "ls_verify_greedy: needs %llu counter bytes and %llu scratch bytes",
           (unsigned long long)need_c, (unsigned long long)need_s);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LS_GREEDY_CAND(TAG)                                                                          \
  if (candidates_dtype == LS_I32)                                                                    \
    return launch_greedy<TAG, int32_t>(logits, logits_row_stride, candidates, cand_stride_b,         \
                                       cand_stride_k, cand_first_col, batch, width, vocab,           \
                                       cutoff_verify_lens, accept_lens, bonus, truth, cap_trim,     \
                                       counters, scratch, s);                     \
  if (candidates_dtype == LS_I64)                                                                    \
    return launch_greedy<TAG, int64_t>(logits, logits_row_stride, candidates, cand_stride_b,         \
                                       cand_stride_k, cand_first_col, batch, width, vocab,           \
                                       cutoff_verify_lens, accept_lens, bonus, truth, cap_trim,     \
                                       counters, scratch, s);                     \
  return fail(LS_ERR_DTYPE, "ls_verify_greedy: candidates must be int32 or int64");
  if (logits_dtype == LS_BF16) { LS_GREEDY_CAND(BF16) }
  if (logits_dtype == LS_F16) { LS_GREEDY_CAND(F16) }
  if (logits_dtype == LS_F32) { LS_GREEDY_CAND(F32) }
#undef LS_GREEDY_CAND
  return fail(LS_ERR_DTYPE, "ls_verify_greedy: logits must be bf16, fp16 or fp32");
}

extern "C" int ls_verify_greedy_noalloc(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                        const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                        int64_t cand_stride_k, int32_t cand_first_col, int64_t batch,
                                        int32_t width, int64_t vocab, const int32_t* cutoff_verify_lens,
                                        int32_t* accept_lens, int64_t* bonus, int32_t* truth, int32_t* cap_trim,
                                        void* stream) {
  using namespace ls;
  LS_CHECK(batch > 0 && width >= 2 && width <= 64 && vocab > 0, LS_ERR_SHAPE,
           "ls_verify_greedy_noalloc: need batch > 0, 2 <= width <= 64, vocab > 0 (got %lld, %d, %lld)",
           (long long)batch, width, (long long)vocab);
  uint64_t need_c = 0, need_s = 0;
  ls_verify_greedy_workspace(batch, width, vocab, &need_c, &need_s);
  LS_CHECK(need_c <= kNoAllocBytes && need_s == 0, LS_ERR_WORKSPACE,
           "ls_verify_greedy_noalloc: batch %lld x width %d needs %llu bytes of counters; the built-in buffer "
           "holds %llu (use ls_verify_greedy with a workspace)",
           (long long)batch, width, (unsigned long long)need_c, (unsigned long long)kNoAllocBytes);
  void* counters = nullptr;
  const int rc = noalloc_counters(static_cast<hipStream_t>(stream), &counters);
  if (rc != LS_OK) return rc;
  return ls_verify_greedy(logits, logits_dtype, logits_row_stride, candidates, candidates_dtype, cand_stride_b,
                          cand_stride_k, cand_first_col, batch, width, vocab, cutoff_verify_lens, accept_lens,
                          bonus, truth, cap_trim, counters, kNoAllocBytes, nullptr, 0, stream);
}
