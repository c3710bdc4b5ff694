// Split-engine verification on dense target probabilities, and the
// fixed-width verify outputs.
//
//   decide    L_b = #leading j < gamma with u[b,j] * q[b,j] < p[b, j, cand[b,j]]
//             (strict), target_rows[b] = p[b, L_b, :]
//             (src/longspark/engine/sampling.py:19-35)
//   finish    probs = p row, or for a rejected request the normalised residual
//             max(p - q, 0) / mass when mass > 1e-8; token = #{v : u >= CDF(v)}
//             clamped to V-1 (src/longspark/engine/sampling.py:38-57)
//   finalize  out[b, c] = bonus if c == L_b else cand[b, c+1] (0 in the last
//             column), committed = L+1, next = prefix + L + 1
//             (SRT/speculative/draft_free_kv_dispatch.py:8-57,
//              SRT/speculative/draft_free_kv_utils.py:386-408)
// SRT = vendor/sglang/python/sglang/srt.
#include "common.h"

namespace ls {
namespace {

constexpr int kST = 256;
constexpr int kChunk = kST * 4;  // elements per block-wide scan step

__device__ __forceinline__ int64_t ld_idx(const void* p, int dtype, int64_t i) {
  return dtype == LS_I64 ? static_cast<const int64_t*>(p)[i] : static_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ float block_sum_f(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kST / kWave; ++w) t += red[w];
  return t;
}

struct DecideArgs {
  const void* cand;
  int cand_dtype;
  int64_t csb, csk;
  const float* q;
  int64_t qsb;
  const float* u;
  int64_t usb;
  const float* p;
  int64_t psb, psk;
  int gamma;
  int64_t vocab;
  int64_t* lengths;
  float* rows;
  int64_t rsb;
};

__global__ __launch_bounds__(kST) void decide_kernel(DecideArgs a) {
  __shared__ int s_len;
  const int64_t b = blockIdx.x;
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    int len = a.gamma;
    for (int base = 0; base < a.gamma; base += kWave) {
      const int j = base + lane;
      bool ok = false;
      if (j < a.gamma) {
        const int64_t c = ld_idx(a.cand, a.cand_dtype, b * a.csb + j * a.csk);
        const float pj = (c >= 0 && c < a.vocab) ? a.p[b * a.psb + j * a.psk + c] : 0.f;
        ok = a.u[b * a.usb + j] * a.q[b * a.qsb + j] < pj;
      }
      const uint64_t fail = __ballot(j < a.gamma && !ok);
      if (fail) {
        len = base + __ffsll(static_cast<long long>(fail)) - 1;
        break;
      }
    }
    if (lane == 0) {
      s_len = len;
      a.lengths[b] = len;
    }
  }
  __syncthreads();
  if (!a.rows) return;
  const float* src = a.p + b * a.psb + static_cast<int64_t>(s_len) * a.psk;
  float* dst = a.rows + b * a.rsb;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0) {
    const int64_t nv = a.vocab / 4;
    for (int64_t i = threadIdx.x; i < nv; i += kST)
      reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(src)[i];
    for (int64_t i = nv * 4 + threadIdx.x; i < a.vocab; i += kST) dst[i] = src[i];
  } else {
    for (int64_t i = threadIdx.x; i < a.vocab; i += kST) dst[i] = src[i];
  }
}

struct FinishArgs {
  const float* t;
  int64_t tsb;
  const int64_t* rejected;
  int64_t n_rejected;
  const float* q;
  int64_t qsb;
  const float* u;
  int64_t vocab;
  int64_t* out;
};

// One workgroup per request.  The probability of element v is computed the
// same way in every pass: t[v] for an accepted request, otherwise
// max(t[v] - q[v], 0) / max(mass, 1e-30) (or t[v] when mass <= 1e-8).
// The CDF is walked in chunks of kChunk elements: each wave sums whole
// chunks, one thread accumulates the chunk sums in order until the total
// passes u, and wave 0 scans inside that chunk.
__global__ __launch_bounds__(kST) void finish_kernel(FinishArgs a) {
  __shared__ float red[kST / kWave];
  __shared__ int s_r;
  __shared__ float s_chunk[kST];
  __shared__ int s_hit;
  __shared__ float s_base;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  if (tid == 0) s_r = -1;
  __syncthreads();
  for (int64_t i = tid; i < a.n_rejected; i += kST)
    if (a.rejected[i] == b) atomicMax(&s_r, static_cast<int>(i));
  __syncthreads();
  const int r = s_r;
  const float* t = a.t + b * a.tsb;
  const float* q = r >= 0 ? a.q + r * a.qsb : nullptr;
  float den = 1.f;
  bool residual = false;
  if (r >= 0) {
    float acc = 0.f;
    for (int64_t v = tid; v < a.vocab; v += kST) acc += fmaxf(t[v] - q[v], 0.f);
    const float mass = block_sum_f(acc, red);
    residual = mass > 1e-8f;
    den = fmaxf(mass, 1e-30f);
  }
  auto prob = [&](int64_t v) -> float { return residual ? fmaxf(t[v] - q[v], 0.f) / den : t[v]; };
  const float u = a.u[b];
  const int64_t nchunks = (a.vocab + kChunk - 1) / kChunk;
  float base = 0.f;
  int64_t hit = -1;
  for (int64_t c0 = 0; c0 < nchunks && hit < 0; c0 += kST) {
    const int nc = static_cast<int>(min<int64_t>(kST, nchunks - c0));
    for (int c = wid; c < nc; c += kST / kWave) {
      const int64_t v0 = (c0 + c) * kChunk;
      float s = 0.f;
      for (int e = 0; e < kChunk / kWave; ++e) {
        const int64_t v = v0 + e * kWave + lane;
        if (v < a.vocab) s += prob(v);
      }
      s = wave_sum(s);
      if (lane == 0) s_chunk[c] = s;
    }
    __syncthreads();
    if (tid == 0) {
      int found = -1;
      float run = base;
      for (int c = 0; c < nc; ++c) {
        if (run + s_chunk[c] > u) { found = c; break; }
        run += s_chunk[c];
      }
      s_hit = found;
      s_base = run;
    }
    __syncthreads();
    if (s_hit >= 0) hit = c0 + s_hit;
    base = s_base;
    __syncthreads();
  }
  if (wid != 0) return;
  int64_t tok = a.vocab - 1;
  if (hit >= 0) {
    float run = base;
    const int64_t v0 = hit * kChunk;
    for (int e = 0; e < kChunk / kWave; ++e) {
      const int64_t v = v0 + e * kWave + lane;
      float x = v < a.vocab ? prob(v) : 0.f;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const float y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
      }
      const uint64_t m = __ballot(v < a.vocab && run + x > u);
      if (m) {
        tok = v0 + e * kWave + __ffsll(static_cast<long long>(m)) - 1;
        break;
      }
      run += __shfl(x, kWave - 1, kWave);
    }
  }
  if (lane == 0) a.out[b] = tok;
}

struct FinalizeArgs {
  const void* cand;
  int cand_dtype;
  int64_t csb, csk;
  const void* lens;
  int lens_dtype;
  int64_t lsb;
  const void* bonus;
  int bonus_dtype;
  int64_t bsb;
  const void* prefix;
  int prefix_dtype;
  int64_t psb;
  int64_t batch;
  int width;
  int64_t* out;
  int32_t* committed;
  void* next;
};

__global__ __launch_bounds__(kST) void finalize_kernel(FinalizeArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kST + threadIdx.x;
  if (i >= a.batch * a.width) return;
  const int64_t row = i / a.width;
  const int col = static_cast<int>(i % a.width);
  const int64_t len = ld_idx(a.lens, a.lens_dtype, row * a.lsb);
  const int64_t bon = ld_idx(a.bonus, a.bonus_dtype, row * a.bsb);
  const int64_t draft = col < a.width - 1 ? ld_idx(a.cand, a.cand_dtype, row * a.csb + (col + 1) * a.csk) : 0;
  a.out[i] = col == len ? bon : draft;
  if (col == 0) {
    if (a.committed) a.committed[row] = static_cast<int32_t>(len + 1);
    if (a.next) {
      const int64_t prev = ld_idx(a.prefix, a.prefix_dtype, row * a.psb);
      if (a.prefix_dtype == LS_I64) static_cast<int64_t*>(a.next)[row] = prev + len + 1;
      else static_cast<int32_t*>(a.next)[row] = static_cast<int32_t>(prev + len + 1);
    }
  }
}

inline bool is_index(int d) { return d == LS_I32 || d == LS_I64; }

}  // namespace
}  // namespace ls

extern "C" int ls_decide_acceptance(const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                    int64_t cand_stride_k, const float* sampled_q, int64_t q_stride_b,
                                    const float* uniforms, int64_t uniform_stride_b, const float* target_probs,
                                    int64_t probs_stride_b, int64_t probs_stride_k, int64_t batch, int32_t gamma,
                                    int64_t vocab, int64_t* lengths, float* target_rows, int64_t rows_stride_b,
                                    void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && gamma >= 1 && vocab >= 1, LS_ERR_SHAPE, "ls_decide_acceptance: bad sizes");
  LS_CHECK(is_index(candidates_dtype), LS_ERR_DTYPE, "ls_decide_acceptance: candidates must be int32/int64");
  LS_CHECK(candidates && sampled_q && uniforms && target_probs && lengths, LS_ERR_VALUE,
           "ls_decide_acceptance: null pointer");
  if (batch == 0) return LS_OK;
  DecideArgs a{candidates, candidates_dtype, cand_stride_b, cand_stride_k, sampled_q, q_stride_b, uniforms,
               uniform_stride_b, target_probs, probs_stride_b, probs_stride_k, gamma, vocab, lengths, target_rows,
               rows_stride_b};
  decide_kernel<<<dim3(static_cast<unsigned>(batch)), kST, 0, static_cast<hipStream_t>(stream)>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_finish_sampling(const float* target_rows, int64_t rows_stride_b, const int64_t* rejected_rows,
                                  int64_t n_rejected, const float* rejected_q_rows, int64_t q_stride_b,
                                  const float* uniforms, int64_t batch, int64_t vocab, int64_t* tokens,
                                  void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && vocab >= 1 && n_rejected >= 0 && n_rejected <= batch, LS_ERR_SHAPE,
           "ls_finish_sampling: bad sizes");
  LS_CHECK(target_rows && uniforms && tokens && (n_rejected == 0 || (rejected_rows && rejected_q_rows)),
           LS_ERR_VALUE, "ls_finish_sampling: null pointer");
  if (batch == 0) return LS_OK;
  FinishArgs a{target_rows, rows_stride_b, rejected_rows, n_rejected, rejected_q_rows, q_stride_b, uniforms, vocab,
               tokens};
  finish_kernel<<<dim3(static_cast<unsigned>(batch)), kST, 0, static_cast<hipStream_t>(stream)>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_finalize_verify_outputs(const void* candidates, int32_t candidates_dtype, int64_t cand_stride_b,
                                          int64_t cand_stride_k, const void* accept_lens, int32_t lens_dtype,
                                          int64_t lens_stride, const void* bonus, int32_t bonus_dtype,
                                          int64_t bonus_stride, const void* prefix_lens, int32_t prefix_dtype,
                                          int64_t prefix_stride, int64_t batch, int32_t width, int64_t* out_tokens,
                                          int32_t* committed, void* next_lengths, void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && width >= 2, LS_ERR_SHAPE, "ls_finalize_verify_outputs: need width >= 2");
  LS_CHECK(is_index(candidates_dtype) && is_index(lens_dtype) && is_index(bonus_dtype) &&
               (!next_lengths || is_index(prefix_dtype)),
           LS_ERR_DTYPE, "ls_finalize_verify_outputs: integer tensors must be int32/int64");
  LS_CHECK(candidates && accept_lens && bonus && out_tokens && (!next_lengths || prefix_lens), LS_ERR_VALUE,
           "ls_finalize_verify_outputs: null pointer");
  if (batch == 0) return LS_OK;
  FinalizeArgs a{candidates, candidates_dtype, cand_stride_b, cand_stride_k, accept_lens, lens_dtype, lens_stride,
                 bonus, bonus_dtype, bonus_stride, prefix_lens, prefix_dtype, prefix_stride, batch, width,
                 out_tokens, committed, next_lengths};
  const int64_t n = batch * width;
  finalize_kernel<<<dim3(static_cast<unsigned>((n + kST - 1) / kST)), kST, 0, static_cast<hipStream_t>(stream)>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}
