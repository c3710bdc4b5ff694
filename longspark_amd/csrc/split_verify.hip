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
//   chain     dense-q chain rejection sampling: accept drafted token j while
//             u[b,j] * q[b,j,c] < p[b,j,c] (c = cand[b, j+1]); the bonus is the
//             first v whose running sum of max(p - q, 0) at the first
//             rejection (p itself when all are accepted) exceeds
//             u_final * total, V-1 when none does; outputs in the
//             predicts / accept_index / accept_token_num layout
//             (SRT/speculative/reject_sampling.py:5-204)
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

// ------------------------------------------------------------ chain sampling
//
// Several workgroups per request: each sums the bonus row's values over its
// share of 1024-element chunks (one wave per chunk, fp64 sums) and publishes
// the chunk sums; the last workgroup to arrive for the request walks the
// chunk sums to the chunk where the running sum passes u * total and scans
// that chunk element by element.  The values are fp32 (max(p - q, 0) as the
// reference forms them); the running sums are fp64.

constexpr int kCT = 256;        // threads per chain workgroup
constexpr int kCChunk = 1024;   // elements per chunk: 16 per lane of one wave
constexpr int kCWaves = kCT / kWave;
constexpr int kChainRegGroups = 4;  // chunk sums held in registers by the last workgroup: up to 256 chunks

struct ChainArgs {
  const float* p;
  int64_t psb, psk;
  const float* q;
  int64_t qsb, qsk;
  const void* cand;
  int cand_dtype;
  int64_t csb, csk;
  const void* ridx;
  int ridx_dtype;
  int64_t rsb, rsk;
  const float* u;
  int64_t usb;
  const float* uf;
  int64_t batch;
  int width;
  int64_t vocab;
  int32_t* predicts;
  int32_t* aidx;
  int64_t aisb, aisk;
  int32_t* anum;
  uint64_t* part;     // [batch, nchunks] chunk sums (fp64 bit patterns)
  uint32_t* arrive;   // [batch] arrivals (zero between calls)
  int64_t nchunks;
  int slices, cps;    // workgroups per request, chunks per workgroup
};

// Accepted drafts of request b (every lane returns it): drafted token j
// (candidates column j + 1) is accepted while u[b, j] * q[b, j, c] < p[b, j, c]
// (reject_sampling.py:53-88); a token outside [0, vocab) is a rejection.
__device__ int chain_accept_len(const ChainArgs& a, int64_t b) {
  const int lane = threadIdx.x & (kWave - 1);
  const int g = a.width - 1;
  for (int base = 0; base < g; base += kWave) {
    const int j = base + lane;
    bool ok = false;
    if (j < g) {
      const int64_t c = ld_idx(a.cand, a.cand_dtype, b * a.csb + static_cast<int64_t>(j + 1) * a.csk);
      if (c >= 0 && c < a.vocab) {
        const float pj = a.p[b * a.psb + static_cast<int64_t>(j) * a.psk + c];
        const float qj = a.q[b * a.qsb + static_cast<int64_t>(j) * a.qsk + c];
        ok = a.u[b * a.usb + j] * qj < pj;
      }
    }
    const uint64_t fail = __ballot(j < g && !ok);
    if (fail) return base + __ffsll(static_cast<long long>(fail)) - 1;
  }
  return g;
}

// Lane's 16 values of chunk c: x[4 * i + e] is element c * 1024 + i * 256 +
// lane * 4 + e (0 beyond the vocabulary).  q == nullptr: the values are p;
// otherwise max(p - q, 0) (NaN differences count as 0, reject_sampling.py:103-107).
template <bool kVec>
__device__ __forceinline__ void chain_chunk(const float* __restrict__ p, const float* __restrict__ q, int64_t vocab,
                                            int64_t c, float* x) {
  const int lane = threadIdx.x & (kWave - 1);
  if constexpr (kVec) {
    // All eight 16-byte loads go out unconditionally (a clamped address; q
    // absent: p again) before any is used; the lanes of a vector that
    // crosses the end of the row read it element by element.
    const int64_t vlast = (vocab / 4 - 1) * 4;  // the last whole vector (vocab >= 4)
    const float* qs = q ? q : p;
    float4 tp[4], tq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t v0 = c * kCChunk + i * (kWave * 4) + lane * 4;
      tp[i] = *reinterpret_cast<const float4*>(p + min(v0, vlast));
      tq[i] = *reinterpret_cast<const float4*>(qs + min(v0, vlast));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t v0 = c * kCChunk + i * (kWave * 4) + lane * 4;
      float pv[4] = {tp[i].x, tp[i].y, tp[i].z, tp[i].w};
      float qv[4] = {tq[i].x, tq[i].y, tq[i].z, tq[i].w};
      if (v0 + 3 >= vocab) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pv[e] = v0 + e < vocab ? p[v0 + e] : 0.f;
          qv[e] = v0 + e < vocab ? qs[v0 + e] : 0.f;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = pv[e] - qv[e];
        x[4 * i + e] = q ? (d > 0.f ? d : 0.f) : pv[e];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t v0 = c * kCChunk + i * (kWave * 4) + lane * 4;
      float pv[4], qv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = v0 + e < vocab ? p[v0 + e] : 0.f;
        if (q) qv[e] = v0 + e < vocab ? q[v0 + e] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = pv[e] - qv[e];
        x[4 * i + e] = q ? (d > 0.f ? d : 0.f) : pv[e];
      }
    }
  }
}

template <bool kVec>
__global__ __launch_bounds__(kCT) void chain_kernel(ChainArgs a) {
  __shared__ int s_last;
  const int64_t b = static_cast<int64_t>(blockIdx.x) % a.batch;
  const int slice = static_cast<int>(static_cast<int64_t>(blockIdx.x) / a.batch);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const int len = chain_accept_len(a, b);
  const bool rejected = len < a.width - 1;
  const float* prow = a.p + b * a.psb + static_cast<int64_t>(len) * a.psk;
  const float* qrow = rejected ? a.q + b * a.qsb + static_cast<int64_t>(len) * a.qsk : nullptr;
  uint64_t* part = a.part + b * a.nchunks;

  // chunk sums of this workgroup's share
  const int64_t c_end = min<int64_t>(a.nchunks, static_cast<int64_t>(slice + 1) * a.cps);
  for (int64_t c = static_cast<int64_t>(slice) * a.cps + wid; c < c_end; c += kCWaves) {
    float x[16];
    chain_chunk<kVec>(prow, qrow, a.vocab, c, x);
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += static_cast<double>(x[k]);
    t = wave_sum_d_dpp(t);
    if (lane == 0) atomic_put_u64(part + c, static_cast<uint64_t>(__double_as_longlong(t)));
  }
  __syncthreads();
  if (tid == 0) s_last = arrive(a.arrive + b) == static_cast<uint32_t>(a.slices - 1) ? 1 : 0;
  __syncthreads();
  if (!s_last || wid != 0) return;
  if (lane == 0) atomic_take_u32(a.arrive + b);  // back to zero for the next call

  // The last workgroup: total, then the chunk where the running sum passes
  // u * total (both walks use the same group-wise scans, so they agree).  Up
  // to kChainRegGroups groups of 64 chunk sums sit in registers, loaded in one
  // round beside the indices the final writes need.
  auto chunk_sum = [&](int64_t c) -> double {
    return c < a.nchunks ? __longlong_as_double(static_cast<long long>(atomic_peek_u64(part + c))) : 0.0;
  };
  const bool one_pass = len < kWave;
  int64_t my_slot = 0, my_tok = 0;
  if (one_pass && lane <= len) {
    my_slot = ld_idx(a.ridx, a.ridx_dtype, b * a.rsb + static_cast<int64_t>(lane) * a.rsk);
    if (lane < len) my_tok = ld_idx(a.cand, a.cand_dtype, b * a.csb + static_cast<int64_t>(lane + 1) * a.csk);
  }
  int64_t hit_chunk = -1;
  double base = 0.0, target;
  if (a.nchunks <= kWave * kChainRegGroups) {
    double xs[kChainRegGroups], inc[kChainRegGroups];
#pragma unroll
    for (int g = 0; g < kChainRegGroups; ++g) xs[g] = chunk_sum(g * kWave + lane);
    double total = 0.0;
#pragma unroll
    for (int g = 0; g < kChainRegGroups; ++g) {
      inc[g] = wave_incl_scan_d_dpp(xs[g]);
      if (g * kWave < a.nchunks) total += __shfl(inc[g], kWave - 1, kWave);
    }
    target = static_cast<double>(a.uf[b]) * total;
#pragma unroll
    for (int g = 0; g < kChainRegGroups; ++g) {
      const uint64_t m = __ballot(g * kWave + lane < a.nchunks && base + inc[g] > target);
      if (hit_chunk < 0 && m) {
        const int l = __ffsll(static_cast<long long>(m)) - 1;
        hit_chunk = g * kWave + l;
        base += __shfl(inc[g] - xs[g], l, kWave);
      }
      if (hit_chunk < 0) base += __shfl(inc[g], kWave - 1, kWave);
    }
  } else {
    double total = 0.0;
    for (int64_t c0 = 0; c0 < a.nchunks; c0 += kWave) {
      const double inc = wave_incl_scan_d_dpp(chunk_sum(c0 + lane));
      total += __shfl(inc, kWave - 1, kWave);
    }
    target = static_cast<double>(a.uf[b]) * total;
    for (int64_t c0 = 0; c0 < a.nchunks; c0 += kWave) {
      const double x = chunk_sum(c0 + lane);
      const double inc = wave_incl_scan_d_dpp(x);
      const uint64_t m = __ballot(c0 + lane < a.nchunks && base + inc > target);
      if (m) {
        const int l = __ffsll(static_cast<long long>(m)) - 1;
        hit_chunk = c0 + l;
        base += __shfl(inc - x, l, kWave);
        break;
      }
      base += __shfl(inc, kWave - 1, kWave);
    }
  }
  int64_t tok = a.vocab - 1;
  if (hit_chunk >= 0) {
    float x[16];
    chain_chunk<kVec>(prow, qrow, a.vocab, hit_chunk, x);
    int64_t found = -1, last_pos = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double ls = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) ls += static_cast<double>(x[4 * i + e]);
      const double inc = wave_incl_scan_d_dpp(ls);
      double run = base + (inc - ls);
      int first = -1, lastpos = -1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        run += static_cast<double>(x[4 * i + e]);
        if (first < 0 && run > target) first = e;
        if (x[4 * i + e] > 0.f) lastpos = e;
      }
      const int64_t v0 = hit_chunk * kCChunk + i * (kWave * 4) + lane * 4;
      const uint64_t m = __ballot(found < 0 && first >= 0);
      if (found < 0 && m) {
        const int l = __ffsll(static_cast<long long>(m)) - 1;
        found = __shfl(v0 + first, l, kWave);
      }
      const uint64_t mp = __ballot(lastpos >= 0);
      if (mp) {
        const int l = 63 - __clzll(static_cast<long long>(mp));
        last_pos = __shfl(v0 + lastpos, l, kWave);
      }
      base += __shfl(inc, kWave - 1, kWave);
    }
    // the running sum passed the target inside this chunk up to rounding:
    // without an element past it, the chunk's last positive element
    tok = found >= 0 ? found : (last_pos >= 0 ? last_pos : a.vocab - 1);
  }
  if (one_pass) {
    if (lane <= len) {
      a.aidx[b * a.aisb + static_cast<int64_t>(lane) * a.aisk] = static_cast<int32_t>(my_slot);
      a.predicts[my_slot] = static_cast<int32_t>(lane < len ? my_tok : tok);
    }
  } else {
    for (int n = lane; n <= len; n += kWave) {
      const int64_t slot = ld_idx(a.ridx, a.ridx_dtype, b * a.rsb + static_cast<int64_t>(n) * a.rsk);
      a.aidx[b * a.aisb + static_cast<int64_t>(n) * a.aisk] = static_cast<int32_t>(slot);
      const int64_t t = n < len ? ld_idx(a.cand, a.cand_dtype, b * a.csb + static_cast<int64_t>(n + 1) * a.csk) : tok;
      a.predicts[slot] = static_cast<int32_t>(t);
    }
  }
  if (lane == 0) a.anum[b] = len;
}

// Committed cache rows into the request-to-token map: for request b and
// i < commit_lens[b] (clamped to [0, width]), req_to_token[slot_b, start_b + i]
// = cache_locs[b, i] (positions past pool_len are skipped).
struct AssignArgs {
  const void* slots;
  int slots_dtype;
  const void* start;
  int start_dtype;
  const void* commit;
  int commit_dtype;
  const void* locs;
  int locs_dtype;
  int64_t locs_stride_b;
  int32_t* rtt;
  int64_t rtt_stride;
  int64_t pool_len;
  int64_t batch;
  int width;
};

__global__ __launch_bounds__(kST) void assign_cache_locs_kernel(AssignArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kST + threadIdx.x;
  if (i >= a.batch * a.width) return;
  const int64_t b = i / a.width;
  const int j = static_cast<int>(i - b * a.width);
  const int64_t n = ld_idx(a.commit, a.commit_dtype, b);
  if (j >= n) return;
  const int64_t pos = ld_idx(a.start, a.start_dtype, b) + j;
  if (pos < 0 || pos >= a.pool_len) return;
  const int64_t slot = ld_idx(a.slots, a.slots_dtype, b);
  a.rtt[slot * a.rtt_stride + pos] = static_cast<int32_t>(ld_idx(a.locs, a.locs_dtype, b * a.locs_stride_b + j));
}

inline bool is_index(int d) { return d == LS_I32 || d == LS_I64; }

inline uint64_t chain_up256(uint64_t x) { return (x + 255) & ~uint64_t(255); }
inline int64_t chain_chunks(int64_t vocab) { return (vocab + kCChunk - 1) / kCChunk; }

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

extern "C" int ls_chain_sampling_workspace(int64_t batch, int64_t vocab, uint64_t* counter_bytes,
                                           uint64_t* scratch_bytes) {
  using namespace ls;
  LS_CHECK(batch >= 0 && vocab >= 1, LS_ERR_SHAPE, "ls_chain_sampling_workspace: bad sizes");
  LS_CHECK(counter_bytes && scratch_bytes, LS_ERR_VALUE, "ls_chain_sampling_workspace: null output");
  *counter_bytes = chain_up256(4 * static_cast<uint64_t>(batch));
  *scratch_bytes = chain_up256(8 * static_cast<uint64_t>(batch) * static_cast<uint64_t>(chain_chunks(vocab)));
  return LS_OK;
}

extern "C" int ls_chain_speculative_sampling(const ls_chain_sampling_args* args, void* counters,
                                             uint64_t counter_bytes, void* scratch, uint64_t scratch_bytes,
                                             void* stream) {
  using namespace ls;
  LS_CHECK(args, LS_ERR_VALUE, "ls_chain_speculative_sampling: null args");
  const ls_chain_sampling_args& x = *args;
  LS_CHECK(x.batch >= 0 && x.width >= 2 && x.vocab >= 1, LS_ERR_SHAPE,
           "ls_chain_speculative_sampling: need batch >= 0, width >= 2, vocab >= 1");
  LS_CHECK(x.batch < (int64_t(1) << 24), LS_ERR_SHAPE, "ls_chain_speculative_sampling: batch too large");
  LS_CHECK(is_index(x.candidates_dtype) && is_index(x.retrive_index_dtype), LS_ERR_DTYPE,
           "ls_chain_speculative_sampling: candidates and retrive_index must be int32/int64");
  if (x.batch == 0) return LS_OK;
  LS_CHECK(x.target_probs && x.draft_probs && x.candidates && x.retrive_index && x.uniforms &&
               x.final_uniforms && x.predicts && x.accept_index && x.accept_token_num,
           LS_ERR_VALUE, "ls_chain_speculative_sampling: null pointer");
  uint64_t need_c = 0, need_s = 0;
  ls_chain_sampling_workspace(x.batch, x.vocab, &need_c, &need_s);
  LS_CHECK(counters && scratch && counter_bytes >= need_c && scratch_bytes >= need_s, LS_ERR_SHAPE,
           "ls_chain_speculative_sampling: needs %llu counter and %llu scratch bytes",
           (unsigned long long)need_c, (unsigned long long)need_s);
  ChainArgs a{};
  a.p = x.target_probs; a.psb = x.tp_stride_b; a.psk = x.tp_stride_k;
  a.q = x.draft_probs; a.qsb = x.dp_stride_b; a.qsk = x.dp_stride_k;
  a.cand = x.candidates; a.cand_dtype = x.candidates_dtype; a.csb = x.cand_stride_b; a.csk = x.cand_stride_k;
  a.ridx = x.retrive_index; a.ridx_dtype = x.retrive_index_dtype; a.rsb = x.ri_stride_b; a.rsk = x.ri_stride_k;
  a.u = x.uniforms; a.usb = x.uniform_stride_b; a.uf = x.final_uniforms;
  a.batch = x.batch; a.width = x.width; a.vocab = x.vocab;
  a.predicts = x.predicts; a.aidx = x.accept_index; a.aisb = x.ai_stride_b; a.aisk = x.ai_stride_k;
  a.anum = x.accept_token_num;
  a.arrive = static_cast<uint32_t*>(counters);
  a.part = static_cast<uint64_t*>(scratch);
  a.nchunks = chain_chunks(x.vocab);
  // about 3072 workgroups in all, each with at least one chunk (of 1024,
  // 1536, 2048, 2560, 3072 and 4096 at B = 128, 3072 measured fastest)
  int64_t slices = (3072 + x.batch - 1) / x.batch;
  if (slices > a.nchunks) slices = a.nchunks;
  a.cps = static_cast<int>((a.nchunks + slices - 1) / slices);
  a.slices = static_cast<int>((a.nchunks + a.cps - 1) / a.cps);
  const bool vec = x.vocab >= 4 && aligned16(x.target_probs) && aligned16(x.draft_probs) && x.tp_stride_b % 4 == 0 &&
                   x.tp_stride_k % 4 == 0 && x.dp_stride_b % 4 == 0 && x.dp_stride_k % 4 == 0;
  const dim3 grid(static_cast<unsigned>(x.batch * a.slices));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec) chain_kernel<true><<<grid, kCT, 0, st>>>(a);
  else chain_kernel<false><<<grid, kCT, 0, st>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_assign_verify_cache_locs(const void* req_pool_indices, int32_t slots_dtype, const void* start_offset,
                                           int32_t start_dtype, const void* commit_lens, int32_t commit_dtype,
                                           const void* verify_cache_locs, int32_t locs_dtype, int64_t locs_stride_b,
                                           int32_t* req_to_token, int64_t rtt_stride, int64_t pool_len,
                                           int64_t batch, int32_t width, void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && width >= 1 && pool_len >= 0 && rtt_stride >= pool_len && locs_stride_b >= width,
           LS_ERR_SHAPE, "ls_assign_verify_cache_locs: bad sizes");
  LS_CHECK(is_index(slots_dtype) && is_index(start_dtype) && is_index(commit_dtype) && is_index(locs_dtype),
           LS_ERR_DTYPE, "ls_assign_verify_cache_locs: index tensors must be int32/int64");
  if (batch == 0) return LS_OK;
  LS_CHECK(req_pool_indices && start_offset && commit_lens && verify_cache_locs && req_to_token, LS_ERR_VALUE,
           "ls_assign_verify_cache_locs: null pointer");
  AssignArgs a{req_pool_indices, slots_dtype, start_offset, start_dtype, commit_lens, commit_dtype,
               verify_cache_locs, locs_dtype, locs_stride_b, req_to_token, rtt_stride, pool_len, batch, width};
  const int64_t n = batch * width;
  assign_cache_locs_kernel<<<dim3(static_cast<unsigned>((n + kST - 1) / kST)), kST, 0,
                             static_cast<hipStream_t>(stream)>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}
