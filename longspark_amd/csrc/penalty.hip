// Penalty tables from an output-token history, and the standalone in-place
// logit adjustment (penalties + vocabulary bitmask).
//
// The tables describe, per request, the accumulated penalties the reference
// penalisers hold as dense [B, V] tensors
// (vendor/sglang/python/sglang/srt/sampling/penaltylib/{frequency,presence,
// repetition}_penalty.py, orchestrator.py:87-104), in a compact form:
//   bits[b, w]  presence bitmap of the history (bit v & 31 of word v >> 5);
//   rank[b, w]  number of present tokens below token 32*w;
//   add[b, r]   additive penalty of the r-th present token (ascending token
//               order): (0 - F) - P with F the fp32 sum of `frequency`
//               repeated count times (scatter_add_ of identical values) and P
//               the presence value, exactly as the reference accumulates it.
// A token v is present iff its bit is set; its table entry is
// add[b, rank[b, v>>5] + popcount(bits[b, v>>5] & ((1 << (v&31)) - 1))].
#include "rowscan.h"

namespace ls {
namespace {

constexpr int kPT = 256;

constexpr int kPTT = 1024;  // threads of the table builder (one workgroup per request)

__global__ __launch_bounds__(kPTT) void penalty_tables_kernel(
    const int32_t* __restrict__ hist, int64_t hist_stride, const int32_t* __restrict__ hist_lens, int hist_cap,
    int64_t vocab, int words, const float* __restrict__ freq, const float* __restrict__ pres,
    uint32_t* __restrict__ bits_out, uint32_t* __restrict__ rank_out, int64_t words_stride,
    float* __restrict__ add_out, int64_t add_stride, int32_t* __restrict__ distinct_out,
    int32_t* __restrict__ nonpos_out) {
  extern __shared__ uint32_t lds[];
  uint32_t* bits = lds;              // [words]
  uint32_t* rank = lds + words;      // [words]
  uint32_t* cnt = lds + 2 * words;   // [hist_cap]
  __shared__ uint32_t wave_tot[kPTT / kWave];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const int32_t* h = hist + static_cast<int64_t>(b) * hist_stride;
  // The first kPre history tokens of each thread are requested before the
  // table is cleared (their addresses do not depend on the history length).
  constexpr int kPre = 2;
  int pre[kPre];
#pragma unroll
  for (int u = 0; u < kPre; ++u) pre[u] = tid + u * kPTT < hist_cap ? h[tid + u * kPTT] : -1;
  const int n = hist_lens ? min(max(hist_lens[b], 0), hist_cap) : hist_cap;

  for (int w = tid; w < words; w += kPTT) bits[w] = 0;
  if (freq)
    for (int r = tid; r < hist_cap; r += kPTT) cnt[r] = 0;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPre; ++u) {
    const int t = pre[u];
    if (tid + u * kPTT < n && t >= 0 && t < vocab) atomicOr(&bits[t >> 5], 1u << (t & 31));
  }
  for (int i = tid + kPre * kPTT; i < n; i += kPTT) {
    const int t = h[i];
    if (t >= 0 && t < vocab) atomicOr(&bits[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  // Exclusive prefix popcount over words: each thread owns a contiguous run
  // of words, one block-wide scan of the run totals.
  const int per = (words + kPTT - 1) / kPTT;
  const int w0 = tid * per;
  const int w1 = min(words, w0 + per);
  uint32_t c = 0;
  for (int w = w0; w < w1; ++w) c += __popc(bits[w]);
  const uint32_t inc = wave_incl_scan_u32(c);
  if (lane == kWave - 1) wave_tot[wid] = inc;
  __syncthreads();
  uint32_t before = 0, distinct = 0;
  for (int k = 0; k < kPTT / kWave; ++k) {
    if (k < wid) before += wave_tot[k];
    distinct += wave_tot[k];
  }
  uint32_t run = before + inc - c;
  for (int w = w0; w < w1; ++w) {
    rank[w] = run;
    run += __popc(bits[w]);
  }
  __syncthreads();
  // Occurrences per present token (only needed for the frequency penalty).
  if (freq) {
    for (int i = tid; i < n; i += kPTT) {
      const int t = h[i];
      if (t >= 0 && t < vocab) {
        const uint32_t bit = 1u << (t & 31);
        atomicAdd(&cnt[rank[t >> 5] + __popc(bits[t >> 5] & (bit - 1u))], 1u);
      }
    }
    __syncthreads();
  }
  uint32_t* bo = bits_out + static_cast<int64_t>(b) * words_stride;
  uint32_t* ro = rank_out + static_cast<int64_t>(b) * words_stride;
  for (int w = tid; w < words; w += kPTT) {
    bo[w] = bits[w];
    ro[w] = rank[w];
  }
  const float f = freq ? freq[b] : 0.f;
  const float p = pres ? pres[b] : 0.f;
  float* ao = add_out + static_cast<int64_t>(b) * add_stride;
  for (uint32_t r = tid; r < distinct; r += kPTT) {
    float acc = 0.f;  // scatter_add_ of `f`, once per occurrence
    if (freq)
      for (uint32_t i = 0; i < cnt[r]; ++i) acc += f;
    float a = 0.f - acc;  // additive tensor starts at zero, then sub_ frequency
    a = a - p;            // then sub_ presence
    ao[r] = a;
  }
  if (tid == 0 && distinct_out) distinct_out[b] = static_cast<int32_t>(distinct);
  // Every additive value is <= 0 exactly when frequency and presence are >= 0.
  if (tid == 0 && nonpos_out) nonpos_out[b] = (f >= 0.f && p >= 0.f) ? 1 : 0;
}

// In-place adjustment of [rows, V] logits: penalties then mask (true order),
// or the verify-path quirk (penalty built on zeros, then added).
template <typename T>
__global__ __launch_bounds__(kPT) void adjust_logits_kernel(
    T* __restrict__ logits, int64_t row_stride, int64_t vocab, int rows_per_request,
    const uint32_t* __restrict__ pbits, const uint32_t* __restrict__ prank, int64_t pwords_stride,
    const float* __restrict__ padd, int64_t padd_stride, const float* __restrict__ rep, int quirk,
    const int32_t* __restrict__ mask, int64_t mask_stride, int mask_rows_per_request, int64_t mask_vocab) {
  const int64_t row = blockIdx.y;
  const int64_t b = row / rows_per_request;
  rs::XForm f;
  f.pbits = pbits ? pbits + b * pwords_stride : nullptr;
  f.prank = pbits ? prank + b * pwords_stride : nullptr;
  f.padd = (pbits && padd) ? padd + b * padd_stride : nullptr;
  f.rep = rep ? rep[b] : 1.f;
  f.quirk = quirk;
  const int64_t mrow = mask_rows_per_request > 1 ? b : row;
  f.mbits = mask ? reinterpret_cast<const uint32_t*>(mask) + mrow * mask_stride : nullptr;
  T* rp = logits + row * row_stride;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kPT + threadIdx.x; v < vocab; v += static_cast<int64_t>(gridDim.x) * kPT) {
    float x = to_f32<T>(rp[v]);
    rs::XForm g = f;
    if (v >= mask_vocab) g.mbits = nullptr;  // columns beyond the mask width stay untouched
    float y = rs::transform1(g, x, v);
    if (y != x) rp[v] = from_f32<T>(y);
  }
}

// Per-request bias vectors added to every row of the request, in the logits'
// dtype (SRT/speculative/dflash_utils.py:176-213):
//   separate == 0 (the dense path, :176-191): z = bias (0 when absent), then
//     columns whose mask bit is 0 become -inf (the grammar mask fills the bias
//     tensor), then z += bias2; each row gets l = T(l + T(z)).
//   separate == 1 (:193-213): l = T(l + T(bias)), then l = T(l + T(bias2)).
// T(x) is the rounding to the logits' dtype (the reference converts the fp32
// tensor with .to(dtype) and adds in that dtype: fp32 sum, one rounding).
// One thread owns 4 columns of one request: it reads the bias columns once
// and applies them to all rows_per_request rows.
constexpr int kRB = 256;

template <typename T, bool kVec>
__global__ __launch_bounds__(kRB) void request_bias_kernel(
    T* __restrict__ logits, int64_t row_stride, int64_t vocab, int rows_per_request,
    const float* __restrict__ bias, int64_t bias_stride, const uint32_t* __restrict__ mask, int64_t mask_stride,
    int64_t mask_vocab, const float* __restrict__ bias2, int64_t bias2_stride, int separate) {
  const int64_t b = blockIdx.y;
  const int64_t v0 = (static_cast<int64_t>(blockIdx.x) * kRB + threadIdx.x) * 4;
  if (v0 >= vocab) return;
  const int n = static_cast<int>(min<int64_t>(4, vocab - v0));
  float z1[4], z2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t v = v0 + e;
    float a = 0.f, c = 0.f;
    if (e < n) {
      if (bias) a = bias[b * bias_stride + v];
      if (bias2) c = bias2[b * bias2_stride + v];
      if (!separate && mask && v < mask_vocab && !((mask[b * mask_stride + (v >> 5)] >> (v & 31)) & 1u))
        a = -INFINITY;
    }
    if (separate) {
      z1[e] = to_f32<T>(from_f32<T>(a));
      z2[e] = to_f32<T>(from_f32<T>(c));
    } else {
      z1[e] = to_f32<T>(from_f32<T>(a + c));
    }
  }
  T* rp = logits + b * rows_per_request * row_stride + v0;
  for (int j = 0; j < rows_per_request; ++j, rp += row_stride) {
    T x[4];
    if (kVec && n == 4) {
      if constexpr (sizeof(T) == 4) {
        const float4 t = *reinterpret_cast<const float4*>(rp);
        x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
      } else {
        const uint2 t = *reinterpret_cast<const uint2*>(rp);
        __builtin_memcpy(x, &t, 8);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < n) x[e] = rp[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!separate) {
        x[e] = from_f32<T>(to_f32<T>(x[e]) + z1[e]);
      } else {  // an absent tensor is not added (it would turn -0 into +0)
        if (bias) x[e] = from_f32<T>(to_f32<T>(x[e]) + z1[e]);
        if (bias2) x[e] = from_f32<T>(to_f32<T>(x[e]) + z2[e]);
      }
    }
    if (kVec && n == 4) {
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(rp) = make_float4(x[0], x[1], x[2], x[3]);
      } else {
        uint2 t;
        __builtin_memcpy(&t, x, 8);
        *reinterpret_cast<uint2*>(rp) = t;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < n) rp[e] = x[e];
    }
  }
}

// Vocabulary bitmask in place (the grammar mask): bit (v & 31) of word
// v >> 5 of the row's mask, LSB first; a 0 bit sets the logit to -inf.  One
// thread owns one mask word, i.e. 32 consecutive columns.  A word with every
// bit set changes nothing and is skipped without touching the logits; any
// other word's columns are read as 16-byte vectors, the masked ones replaced,
// and written back whole (4 vectors for 16-bit logits, 8 for fp32), so a
// wavefront moves 4 or 8 KiB of contiguous logits per access.  Rows come
// from `indices` when given (the same index selects the logits row and the
// mask row); an index outside either tensor is skipped.
template <typename T>
__device__ __forceinline__ T neg_inf_bits();
template <>
__device__ __forceinline__ float neg_inf_bits<float>() { return -INFINITY; }
template <>
__device__ __forceinline__ uint16_t neg_inf_bits<uint16_t>() { return 0xff80u; }
template <>
__device__ __forceinline__ __half neg_inf_bits<__half>() { return __ushort_as_half(0xfc00u); }

constexpr int kBM = 256;

template <typename T, bool kVec>
__global__ __launch_bounds__(kBM) void token_bitmask_kernel(T* __restrict__ logits, int64_t row_stride,
                                                            int64_t logits_rows, int64_t mvocab,
                                                            const uint32_t* __restrict__ mask, int64_t mask_stride,
                                                            int64_t mask_rows, const void* __restrict__ indices,
                                                            int idx_i64, int64_t num_rows) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kBM + threadIdx.x;
  const int64_t words = (mvocab + 31) >> 5;
  if (w >= words) return;
  for (int64_t r = blockIdx.y; r < num_rows; r += gridDim.y) {
    const int64_t row = !indices ? r
                        : idx_i64 ? static_cast<const int64_t*>(indices)[r]
                                  : static_cast<int64_t>(static_cast<const int32_t*>(indices)[r]);
    if (row < 0 || row >= logits_rows || row >= mask_rows) continue;
    const uint32_t bits = mask[row * mask_stride + w];
    if (bits == 0xffffffffu) continue;
    T* p = logits + row * row_stride + w * 32;
    const int64_t n = mvocab - w * 32 < 32 ? mvocab - w * 32 : 32;
    if (kVec && n == 32) {
      constexpr int kPer = 16 / sizeof(T);  // elements per 16-byte vector
      constexpr int kN = 32 / kPer;
      union U {
        uint4 v;
        T e[kPer];
      } u[kN];
      uint4* vp = reinterpret_cast<uint4*>(p);
#pragma unroll
      for (int i = 0; i < kN; ++i) u[i].v = vp[i];
#pragma unroll
      for (int i = 0; i < kN; ++i)
#pragma unroll
        for (int e = 0; e < kPer; ++e)
          if (!((bits >> (i * kPer + e)) & 1u)) u[i].e[e] = neg_inf_bits<T>();
#pragma unroll
      for (int i = 0; i < kN; ++i) vp[i] = u[i].v;
    } else {
      for (int e = 0; e < n; ++e)
        if (!((bits >> e) & 1u)) p[e] = neg_inf_bits<T>();
    }
  }
}

}  // namespace
}  // namespace ls

extern "C" int ls_penalty_tables(const int32_t* history, int64_t history_stride, const int32_t* history_lens,
                                 int64_t batch, int32_t history_cap, int64_t vocab, const float* frequency,
                                 const float* presence, uint32_t* bits, uint32_t* rank, int64_t words_stride,
                                 float* add, int64_t add_stride, int32_t* distinct, int32_t* nonpositive,
                                 void* stream) {
  using namespace ls;
  LS_CHECK(batch > 0 && vocab > 0 && history_cap >= 0, LS_ERR_SHAPE, "ls_penalty_tables: bad sizes");
  const int64_t words = (vocab + 31) / 32;
  LS_CHECK(words_stride >= words && add_stride >= history_cap, LS_ERR_SHAPE,
           "ls_penalty_tables: table strides too small (words %lld, history %d)", (long long)words, history_cap);
  LS_CHECK(history || history_cap == 0, LS_ERR_VALUE, "ls_penalty_tables: null history");
  LS_CHECK(bits && rank && add, LS_ERR_VALUE, "ls_penalty_tables: null output");
  const size_t lds = (2 * static_cast<size_t>(words) + static_cast<size_t>(history_cap)) * 4;
  LS_CHECK(lds <= 64 * 1024, LS_ERR_SHAPE,
           "ls_penalty_tables: vocab %lld with history %d exceeds the 64 KiB LDS budget",
           (long long)vocab, history_cap);
  penalty_tables_kernel<<<dim3(static_cast<unsigned>(batch)), kPTT, lds, static_cast<hipStream_t>(stream)>>>(
      history, history_stride, history_lens, history_cap, vocab, static_cast<int>(words), frequency, presence,
      bits, rank, words_stride, add, add_stride, distinct, nonpositive);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_adjust_logits(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t rows,
                                int64_t vocab, int32_t rows_per_request, const uint32_t* pen_bits,
                                const uint32_t* pen_rank, int64_t pen_words_stride, const float* pen_add,
                                int64_t pen_add_stride, const float* repetition, int32_t verify_quirk,
                                const int32_t* vocab_mask, int64_t mask_stride, int32_t mask_rows_per_request,
                                int64_t mask_words, void* stream) {
  using namespace ls;
  LS_CHECK(rows > 0 && vocab > 0 && rows_per_request > 0 && rows % rows_per_request == 0, LS_ERR_SHAPE,
           "ls_adjust_logits: rows must be a positive multiple of rows_per_request");
  LS_CHECK(row_stride >= vocab, LS_ERR_SHAPE, "ls_adjust_logits: row stride < vocab");
  LS_CHECK(rows <= 65535, LS_ERR_SHAPE, "ls_adjust_logits: at most 65535 rows per call");
  LS_CHECK(!pen_bits || pen_rank, LS_ERR_VALUE, "ls_adjust_logits: penalty bitmap without ranks");
  LS_CHECK(!vocab_mask || (mask_rows_per_request == 1 || mask_rows_per_request == rows_per_request),
           LS_ERR_VALUE, "ls_adjust_logits: mask must be per row or per request");
  LS_CHECK(!vocab_mask || (mask_words > 0 && mask_words * 32 >= 1 && mask_stride >= mask_words), LS_ERR_SHAPE,
           "ls_adjust_logits: bad mask shape");
  const int64_t mask_vocab = vocab_mask ? (mask_words * 32 < vocab ? mask_words * 32 : vocab) : vocab;
  dim3 grid(static_cast<unsigned>((vocab + kPT * 8 - 1) / (kPT * 8)), static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LS_ADJ(T)                                                                                         \
  adjust_logits_kernel<T><<<grid, kPT, 0, s>>>(static_cast<T*>(logits), row_stride, vocab, rows_per_request, \
                                                pen_bits, pen_rank, pen_words_stride, pen_add, pen_add_stride, \
                                                repetition, verify_quirk, vocab_mask, mask_stride,             \
                                                mask_rows_per_request, mask_vocab)
  if (logits_dtype == LS_F32) LS_ADJ(float);
  else if (logits_dtype == LS_BF16) LS_ADJ(uint16_t);
  else if (logits_dtype == LS_F16) LS_ADJ(__half);
  else return fail(LS_ERR_DTYPE, "ls_adjust_logits: logits must be fp32, bf16 or fp16");
#undef LS_ADJ
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_add_request_bias(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t rows,
                                   int64_t vocab, int32_t rows_per_request, const float* bias, int64_t bias_stride,
                                   const int32_t* vocab_mask, int64_t mask_stride, int64_t mask_words,
                                   const float* bias2, int64_t bias2_stride, int32_t separate, void* stream) {
  using namespace ls;
  LS_CHECK(logits, LS_ERR_VALUE, "ls_add_request_bias: null logits");
  LS_CHECK(rows > 0 && vocab > 0 && rows_per_request > 0 && rows % rows_per_request == 0, LS_ERR_SHAPE,
           "ls_add_request_bias: rows must be a positive multiple of rows_per_request");
  LS_CHECK(row_stride >= vocab, LS_ERR_SHAPE, "ls_add_request_bias: row stride < vocab");
  const int64_t batch = rows / rows_per_request;
  LS_CHECK(batch <= 65535, LS_ERR_SHAPE, "ls_add_request_bias: at most 65535 requests per call");
  LS_CHECK((!bias || bias_stride >= vocab) && (!bias2 || bias2_stride >= vocab), LS_ERR_SHAPE,
           "ls_add_request_bias: bias stride < vocab");
  LS_CHECK(!vocab_mask || (mask_words > 0 && mask_stride >= mask_words), LS_ERR_SHAPE,
           "ls_add_request_bias: bad mask shape");
  LS_CHECK(!(separate && vocab_mask), LS_ERR_VALUE, "ls_add_request_bias: the mask belongs to the combined form");
  if (!bias && !bias2 && !vocab_mask) return LS_OK;
  const int64_t mask_vocab = vocab_mask ? (mask_words * 32 < vocab ? mask_words * 32 : vocab) : 0;
  const dim3 grid(static_cast<unsigned>((vocab + kRB * 4 - 1) / (kRB * 4)), static_cast<unsigned>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t* m = reinterpret_cast<const uint32_t*>(vocab_mask);
#define LS_RB(T)                                                                                               \
  do {                                                                                                         \
    T* lp = static_cast<T*>(logits);                                                                           \
    const bool vec = ((reinterpret_cast<uintptr_t>(lp) % (4 * sizeof(T))) == 0) && row_stride % 4 == 0;       \
    if (vec)                                                                                                   \
      request_bias_kernel<T, true><<<grid, kRB, 0, s>>>(lp, row_stride, vocab, rows_per_request, bias,         \
                                                         bias_stride, m, mask_stride, mask_vocab, bias2,       \
                                                         bias2_stride, separate);                              \
    else                                                                                                       \
      request_bias_kernel<T, false><<<grid, kRB, 0, s>>>(lp, row_stride, vocab, rows_per_request, bias,        \
                                                          bias_stride, m, mask_stride, mask_vocab, bias2,      \
                                                          bias2_stride, separate);                             \
  } while (0)
  if (logits_dtype == LS_F32) LS_RB(float);
  else if (logits_dtype == LS_BF16) LS_RB(uint16_t);
  else if (logits_dtype == LS_F16) LS_RB(__half);
  else return fail(LS_ERR_DTYPE, "ls_add_request_bias: logits must be fp32, bf16 or fp16");
#undef LS_RB
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_apply_token_bitmask(void* logits, int32_t logits_dtype, int64_t row_stride, int64_t logits_rows,
                                      int64_t vocab, const int32_t* bitmask, int64_t mask_stride, int64_t mask_rows,
                                      int64_t mask_words, const void* indices, int32_t indices_dtype,
                                      int64_t num_rows, void* stream) {
  using namespace ls;
  LS_CHECK(logits && bitmask, LS_ERR_VALUE, "ls_apply_token_bitmask: null logits or bitmask");
  LS_CHECK(logits_rows > 0 && vocab > 0 && row_stride >= vocab, LS_ERR_SHAPE,
           "ls_apply_token_bitmask: need logits_rows > 0, vocab > 0, row_stride >= vocab");
  LS_CHECK(mask_rows > 0 && mask_words > 0 && mask_stride >= mask_words, LS_ERR_SHAPE,
           "ls_apply_token_bitmask: bad bitmask shape");
  LS_CHECK(mask_words <= (vocab + 31) / 32, LS_ERR_SHAPE,
           "ls_apply_token_bitmask: bitmask width %lld exceeds ceil(vocab / 32) = %lld", (long long)mask_words,
           (long long)((vocab + 31) / 32));
  LS_CHECK(!indices || indices_dtype == LS_I32 || indices_dtype == LS_I64, LS_ERR_DTYPE,
           "ls_apply_token_bitmask: indices must be int32 or int64");
  LS_CHECK(num_rows >= 0, LS_ERR_SHAPE, "ls_apply_token_bitmask: negative row count");
  LS_CHECK(indices || (num_rows <= logits_rows && num_rows <= mask_rows), LS_ERR_SHAPE,
           "ls_apply_token_bitmask: more rows than the logits or the bitmask hold");
  if (num_rows == 0) return LS_OK;
  const int64_t mvocab = mask_words * 32 < vocab ? mask_words * 32 : vocab;
  const int64_t words = (mvocab + 31) / 32;
  const dim3 grid(static_cast<unsigned>((words + kBM - 1) / kBM),
                  static_cast<unsigned>(num_rows < 65535 ? num_rows : 65535));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t* m = reinterpret_cast<const uint32_t*>(bitmask);
  const int i64 = indices_dtype == LS_I64 ? 1 : 0;
#define LS_BM(T)                                                                                              \
  do {                                                                                                        \
    T* lp = static_cast<T*>(logits);                                                                          \
    const bool vec = aligned16(lp) && (row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0;                \
    if (vec)                                                                                                  \
      token_bitmask_kernel<T, true><<<grid, kBM, 0, s>>>(lp, row_stride, logits_rows, mvocab, m, mask_stride,  \
                                                          mask_rows, indices, i64, num_rows);                   \
    else                                                                                                      \
      token_bitmask_kernel<T, false><<<grid, kBM, 0, s>>>(lp, row_stride, logits_rows, mvocab, m, mask_stride, \
                                                           mask_rows, indices, i64, num_rows);                  \
  } while (0)
  if (logits_dtype == LS_F32) LS_BM(float);
  else if (logits_dtype == LS_BF16) LS_BM(uint16_t);
  else if (logits_dtype == LS_F16) LS_BM(__half);
  else return fail(LS_ERR_DTYPE, "ls_apply_token_bitmask: logits must be fp32, bf16 or fp16");
#undef LS_BM
  LS_LAUNCH_CHECK();
  return LS_OK;
}
