// Drafter proposal step: one token per row by the exponential race, with its
// probability (SRT/speculative/dspark_components/kernels/sample_step_tokens_with_q.py:72-187):
//   s_v = l_v / T for finite l_v (-inf otherwise), p = softmax(s),
//   token = argmax_v p_v / E_v with E_v > 0 the given exponential noise (ties
//   to the lowest index), q = p_token.
// A row is invalid when a logit is NaN or +inf, when l / T is NaN or +inf,
// when a finite entry's noise is not in (0, inf), when T is not in (0, inf),
// or when no entry is finite; an invalid row gets token 0 and q = NaN and
// sets *status (the reference writes the same values, then asserts on the
// device).
//
// Each wave streams a contiguous range of 1024-element tiles of one row and
// keeps, per lane, a running maximum and sum of exponentials (rescaled when
// the maximum rises, as the reference's tile combine rescales by
// exp(m_t - m)) and the best race key.  The key p / E is ranked as
// s * log2(e) - log2(E), which orders entries exactly as p / E does and needs
// no rescaling.  About 1,792 workgroups of 4 waves cover all rows in one
// resident round; each wave publishes its part with agent-scope atomic
// exchanges and the last workgroup to arrive for a row combines the parts.
// The sum across parts is fp64.
#include "common.h"

namespace ls {
namespace {

constexpr int kSS = 256;       // threads per workgroup (4 waves)
constexpr int kTile = 1024;    // elements per tile: 16 per lane of one wave
constexpr int kSSWaves = kSS / kWave;
constexpr float kLog2e = 1.4426950408889634f;

struct SampleArgs {
  const void* logits;
  int64_t lrs;
  int64_t rows, vocab;
  const float* temps;
  const float* noise;
  int64_t nrs;
  int64_t* tokens;
  float* q;
  int32_t* status;
  uint64_t* part;     // [rows, slices * 4, 3] per-wave results
  uint32_t* arrive;   // [rows] (zero between calls)
  int64_t ntiles;
  int slices, tps;    // workgroups per row, tiles per wave
};

__device__ __forceinline__ bool finite_f(float x) { return fabsf(x) < INFINITY; }

// Logits e0..e0+3 (in range) as fp32: one 8-byte load for 16-bit types, one
// 16-byte load for fp32.
template <typename Tag>
__device__ __forceinline__ void load4(const typename Tag::storage* p, float* x) {
  if constexpr (sizeof(typename Tag::storage) == 2) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
    uint4 v;
    v.x = __builtin_nontemporal_load(w);
    v.y = __builtin_nontemporal_load(w + 1);
    v.z = 0u;
    v.w = 0u;
    float t[8];
    unpack16<Tag>(v, t);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = t[e];
  } else {
    unpack16<Tag>(load16_stream(p), x);
  }
}

// Per-lane running state over a range of tiles, in the log2 domain:
// s2 = (l / T) * log2(e); m = running max of s2, sum = sum of exp2(s2 - m);
// the race key p / E is ranked by lk = s2 - log2(E), which orders entries
// exactly as p / E does; bi / bs = index and s2 of the best key.
struct Race {
  float m, sum, bl, bs;
  int bi, ok;
};

// Fold one tile of 16 entries per lane (x: logits, sq: l / T, n: noise)
// into the lane's race state, for a tile whose entries are all known finite
// with valid noise: every validity term is true and left out.
__device__ __forceinline__ void race_fold_plain(float (&x)[16], const float (&sq)[16], const float (&n)[16],
                                                int64_t tile, Race& r) {
  const int lane = threadIdx.x & (kWave - 1);
  float lm = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    x[k] = sq[k] * kLog2e;
    lm = fmaxf(lm, x[k]);
  }
  if (lm > r.m) {  // rescale the running sum to the new maximum
    r.sum = r.m == -INFINITY ? 0.f : r.sum * __builtin_amdgcn_exp2f(r.m - lm);
    r.m = lm;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    r.sum += __builtin_amdgcn_exp2f(x[k] - r.m);
    // log2 of the noise (hardware log2; the noise is clamped to the smallest
    // normal value, below which the instruction does not resolve it)
    const float lk = x[k] - __builtin_amdgcn_logf(fmaxf(n[k], 1.17549435e-38f));
    // entries visit in increasing index order within the lane: strict > keeps the lowest
    if (lk > r.bl) {
      r.bl = lk;
      r.bs = x[k];
      r.bi = static_cast<int>(tile * kTile + (k >> 2) * (kWave * 4) + lane * 4 + (k & 3));
    }
  }
}

// The same fold with every validity rule (the reference's :97-106): a NaN or
// +inf logit, a NaN or +inf l / T of a finite logit, or invalid noise at an
// entry with a finite scaled logit clears ok; entries without a finite
// scaled logit take no part.  Runs only for tiles with such entries.
__device__ __forceinline__ void race_fold_general(float (&x)[16], float (&sq)[16], float (&n)[16], int64_t tile,
                                               Race& r) {
  const int lane = threadIdx.x & (kWave - 1);
  float lm = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float raw = x[k], s = sq[k];
    const bool lvalid = raw == raw && raw != INFINITY;
    const bool sfin = finite_f(raw) && finite_f(s);
    const bool svalid = !finite_f(raw) || (s == s && s != INFINITY);
    const bool nvalid = n[k] > 0.f && n[k] < INFINITY;
    r.ok &= (lvalid && svalid && (sfin ? nvalid : true)) ? 1 : 0;
    x[k] = sfin ? s * kLog2e : -INFINITY;
    lm = fmaxf(lm, x[k]);
    __builtin_amdgcn_sched_barrier(0);  // one entry's lane masks at a time
  }
  if (lm > r.m) {
    r.sum = r.m == -INFINITY ? 0.f : r.sum * __builtin_amdgcn_exp2f(r.m - lm);
    r.m = lm;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const bool fin = finite_f(x[k]);
    r.sum += fin ? __builtin_amdgcn_exp2f(x[k] - r.m) : 0.f;
    const bool nvalid = n[k] > 0.f && n[k] < INFINITY;
    const float lk = (fin && nvalid) ? x[k] - __builtin_amdgcn_logf(fmaxf(n[k], 1.17549435e-38f)) : -INFINITY;
    if (lk > r.bl) {
      r.bl = lk;
      r.bs = x[k];
      r.bi = static_cast<int>(tile * kTile + (k >> 2) * (kWave * 4) + lane * 4 + (k & 3));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <typename Tag, bool kVec>
__device__ __forceinline__ void race_tile(const typename Tag::storage* rp, const float* np, int64_t vocab, float t,
                                          float inv_t, int64_t tile, Race& r) {
  using S = typename Tag::storage;
  const int lane = threadIdx.x & (kWave - 1);
  float x[16], n[16];
  auto load_vec = [&](int i, int64_t e0) __attribute__((always_inline)) {
    load4<Tag>(rp + e0, x + 4 * i);
    const uint4 v = load16_stream(np + e0);
    n[4 * i + 0] = __uint_as_float(v.x);
    n[4 * i + 1] = __uint_as_float(v.y);
    n[4 * i + 2] = __uint_as_float(v.z);
    n[4 * i + 3] = __uint_as_float(v.w);
  };
  if (kVec && (tile + 1) * kTile <= vocab) {
    // a whole tile inside the row: no per-vector bounds checks
#pragma unroll
    for (int i = 0; i < 4; ++i) load_vec(i, tile * kTile + i * (kWave * 4) + lane * 4);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e0 = tile * kTile + i * (kWave * 4) + lane * 4;
      if (kVec && e0 + 3 < vocab) {
        load_vec(i, e0);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool in = e0 + j < vocab;
          x[4 * i + j] = in ? to_f32<S>(rp[e0 + j]) : -INFINITY;
          n[4 * i + j] = in ? np[e0 + j] : 1.f;
        }
      }
    }
  }
  // l * (1/T) is within 1.5 ulp of the quotient l / T; the exact quotient is
  // taken where the product may overflow (or is NaN), so that validity is
  // decided as the reference decides it (:97-106).  That is rare: the
  // divisions run only in a wave with such an entry.
  float sq[16];
  bool slow = false;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    sq[k] = x[k] * inv_t;
    slow |= !(fabsf(sq[k]) < 1e37f);
  }
  if (__builtin_expect(__ballot(slow) != 0, 0)) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (!(fabsf(sq[k]) < 1e37f)) sq[k] = x[k] / t;
  }
  // A tile whose entries all have a finite logit, a finite product l * (1/T)
  // and noise in (0, inf) takes the fold without validity selects: x * 0 is
  // exactly 0 for finite x, so one fused sum per entry finds an infinity or a
  // NaN among logit, scaled logit and noise (a sum that overflows only sends
  // the tile to the general fold).
  float chk = 0.f, nmin = INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    chk = fmaf(x[k] + sq[k] + n[k], 0.f, chk);
    nmin = fminf(nmin, n[k]);
  }
  const bool plain = !slow && chk == 0.f && nmin > 0.f;
  if (__builtin_expect(__ballot(!plain) == 0, 1)) race_fold_plain(x, sq, n, tile, r);
  else race_fold_general(x, sq, n, tile, r);
}

// Merge (m, sum, best) of two parts: the larger maximum, both sums rescaled
// to it, the larger key (lower index on equal keys).
__device__ __forceinline__ void race_merge(Race& a, float m2, float sum2, float bl2, float bs2, int bi2, int ok2) {
  const float m = fmaxf(a.m, m2);
  const float s1 = a.m == -INFINITY ? 0.f : a.sum * __builtin_amdgcn_exp2f(a.m - m);
  const float s2 = m2 == -INFINITY ? 0.f : sum2 * __builtin_amdgcn_exp2f(m2 - m);
  a.m = m;
  a.sum = s1 + s2;
  if (bl2 > a.bl || (bl2 == a.bl && bi2 < a.bi)) {
    a.bl = bl2;
    a.bs = bs2;
    a.bi = bi2;
  }
  a.ok &= ok2;
}

template <typename Tag, bool kVec>
__global__ __launch_bounds__(kSS) void sample_step_kernel(SampleArgs a) {
  using S = typename Tag::storage;
  __shared__ int s_last;
  const int64_t row = static_cast<int64_t>(blockIdx.x) % a.rows;
  const int slice = static_cast<int>(static_cast<int64_t>(blockIdx.x) / a.rows);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const float t = a.temps[row];
  const bool t_valid = t > 0.f && t < INFINITY;
  const float inv_t = 1.f / t;
  const S* rp = static_cast<const S*>(a.logits) + row * a.lrs;
  const float* np = a.noise + row * a.nrs;
  const int nw = a.slices * kSSWaves;  // published parts per row
  uint64_t* part = a.part + row * static_cast<int64_t>(nw) * 3;

  // this wave's tiles: [w * tpw, (w + 1) * tpw) of the row
  const int w = slice * kSSWaves + wid;
  Race r{-INFINITY, 0.f, -INFINITY, -INFINITY, 0x7fffffff, 1};
  const int64_t t_end = min<int64_t>(a.ntiles, static_cast<int64_t>(w + 1) * a.tps);
  for (int64_t tile = static_cast<int64_t>(w) * a.tps; tile < t_end; ++tile)
    race_tile<Tag, kVec>(rp, np, a.vocab, t, inv_t, tile, r);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1)
    race_merge(r, __shfl_xor(r.m, off, kWave), __shfl_xor(r.sum, off, kWave), __shfl_xor(r.bl, off, kWave),
               __shfl_xor(r.bs, off, kWave), __shfl_xor(r.bi, off, kWave), __shfl_xor(r.ok, off, kWave));
  if (lane == 0) {
    atomic_put_u64(part + 3 * w, (static_cast<uint64_t>(__float_as_uint(r.sum)) << 32) | __float_as_uint(r.m));
    atomic_put_u64(part + 3 * w + 1, (static_cast<uint64_t>(static_cast<uint32_t>(r.bi)) << 32) | __float_as_uint(r.bl));
    atomic_put_u64(part + 3 * w + 2, (static_cast<uint64_t>(r.ok) << 32) | __float_as_uint(r.bs));
  }
  __syncthreads();
  if (tid == 0) s_last = arrive(a.arrive + row) == static_cast<uint32_t>(a.slices - 1) ? 1 : 0;
  __syncthreads();
  if (!s_last || wid != 0) return;
  if (lane == 0) atomic_take_u32(a.arrive + row);  // back to zero for the next call

  // combine the row's parts (one wave); the sum across parts is fp64
  Race c{-INFINITY, 0.f, -INFINITY, -INFINITY, 0x7fffffff, 1};
  for (int p0 = 0; p0 < nw; p0 += kWave) {
    const int pi = min(p0 + lane, nw - 1);
    const uint64_t w0 = atomic_peek_u64(part + 3 * pi);
    const uint64_t w1 = atomic_peek_u64(part + 3 * pi + 1);
    const uint64_t w2 = atomic_peek_u64(part + 3 * pi + 2);
    if (p0 + lane < nw)
      race_merge(c, __uint_as_float(static_cast<uint32_t>(w0)), 0.f, __uint_as_float(static_cast<uint32_t>(w1)),
                 __uint_as_float(static_cast<uint32_t>(w2)), static_cast<int>(static_cast<uint32_t>(w1 >> 32)),
                 static_cast<int>(w2 >> 32));
  }
  // lane state now holds the maximum and the best key of its parts; the sums
  // are added in a second pass against the row maximum
  float gm = wave_max(c.m);
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float bl2 = __shfl_xor(c.bl, off, kWave), bs2 = __shfl_xor(c.bs, off, kWave);
    const int bi2 = __shfl_xor(c.bi, off, kWave), ok2 = __shfl_xor(c.ok, off, kWave);
    if (bl2 > c.bl || (bl2 == c.bl && bi2 < c.bi)) {
      c.bl = bl2;
      c.bs = bs2;
      c.bi = bi2;
    }
    c.ok &= ok2;
  }
  double den = 0.0;
  if (finite_f(gm)) {
    for (int p0 = lane; p0 < nw; p0 += kWave) {
      const uint64_t w0 = atomic_peek_u64(part + 3 * p0);
      const float pm = __uint_as_float(static_cast<uint32_t>(w0));
      if (pm != -INFINITY)
        den += static_cast<double>(__uint_as_float(static_cast<uint32_t>(w0 >> 32))) *
               static_cast<double>(__builtin_amdgcn_exp2f(pm - gm));
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) den += __shfl_xor(den, off, kWave);
  const bool valid = t_valid && c.ok && finite_f(gm) && den < static_cast<double>(INFINITY) && den > 0.0;
  if (lane == 0) {
    a.tokens[row] = valid ? static_cast<int64_t>(c.bi) : 0;
    a.q[row] = valid ? static_cast<float>(static_cast<double>(__builtin_amdgcn_exp2f(c.bs - gm)) / den) : NAN;
    if (!valid && a.status) atomicOr(a.status, 1);
  }
}

inline uint64_t ss_up256(uint64_t x) { return (x + 255) & ~uint64_t(255); }
inline int64_t ss_tiles(int64_t vocab) { return (vocab + kTile - 1) / kTile; }

// Workgroups of a sample-step kernel resident on the current device at once:
// CUs x the per-CU count its compiled registers and LDS allow (queried once
// per kernel).
int64_t resident_workgroups(void (*kern)(SampleArgs)) {
  static void (*seen[8])(SampleArgs) = {};
  static int64_t count[8] = {};
  for (int i = 0; i < 8; ++i)
    if (seen[i] == kern) return count[i];
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kSS, 0) != hipSuccess || per_cu <= 0) per_cu = 4;
  (void)hipGetLastError();
  const int64_t n = static_cast<int64_t>(cus) * per_cu;
  for (int i = 0; i < 8; ++i)
    if (!seen[i]) {
      seen[i] = kern;
      count[i] = n;
      break;
    }
  return n;
}

}  // namespace
}  // namespace ls

extern "C" int ls_sample_step_workspace(int64_t rows, int64_t vocab, uint64_t* counter_bytes,
                                        uint64_t* scratch_bytes) {
  using namespace ls;
  LS_CHECK(rows >= 0 && vocab >= 1, LS_ERR_SHAPE, "ls_sample_step_workspace: bad sizes");
  LS_CHECK(counter_bytes && scratch_bytes, LS_ERR_VALUE, "ls_sample_step_workspace: null output");
  *counter_bytes = ss_up256(4 * static_cast<uint64_t>(rows));
  // at most one part per tile (one per wave, each wave taking at least one tile)
  *scratch_bytes = ss_up256(24 * static_cast<uint64_t>(rows) * static_cast<uint64_t>(ss_tiles(vocab) + kSSWaves));
  return LS_OK;
}

extern "C" int ls_sample_step(const void* logits, int32_t logits_dtype, int64_t logits_row_stride, int64_t rows,
                              int64_t vocab, const float* temperatures, const float* exp_noise,
                              int64_t noise_row_stride, int64_t* next_tokens, float* sampled_q, int32_t* status,
                              void* counters, uint64_t counter_bytes, void* scratch, uint64_t scratch_bytes,
                              void* stream) {
  using namespace ls;
  LS_CHECK(rows >= 0 && vocab >= 1 && vocab < (int64_t(1) << 31), LS_ERR_SHAPE,
           "ls_sample_step: need rows >= 0 and 1 <= vocab < 2^31");
  LS_CHECK(rows < (int64_t(1) << 24), LS_ERR_SHAPE, "ls_sample_step: too many rows");
  if (rows == 0) return LS_OK;
  LS_CHECK(logits && temperatures && exp_noise && next_tokens && sampled_q, LS_ERR_VALUE,
           "ls_sample_step: null pointer");
  LS_CHECK(logits_row_stride >= vocab && noise_row_stride >= vocab, LS_ERR_SHAPE,
           "ls_sample_step: row stride < vocab");
  uint64_t need_c = 0, need_s = 0;
  ls_sample_step_workspace(rows, vocab, &need_c, &need_s);
  LS_CHECK(counters && scratch && counter_bytes >= need_c && scratch_bytes >= need_s, LS_ERR_SHAPE,
           "ls_sample_step: needs %llu counter and %llu scratch bytes", (unsigned long long)need_c,
           (unsigned long long)need_s);
  SampleArgs a{};
  a.logits = logits; a.lrs = logits_row_stride; a.rows = rows; a.vocab = vocab;
  a.temps = temperatures; a.noise = exp_noise; a.nrs = noise_row_stride;
  a.tokens = next_tokens; a.q = sampled_q; a.status = status;
  a.arrive = static_cast<uint32_t*>(counters);
  a.part = static_cast<uint64_t*>(scratch);
  a.ntiles = ss_tiles(vocab);
  // the kernel for this dtype and alignment
  const bool nvec = aligned16(exp_noise) && noise_row_stride % 4 == 0;
  void (*kern)(SampleArgs) = nullptr;
#define LS_SS(TAG)                                                                                            \
  do {                                                                                                        \
    using S = typename TAG::storage;                                                                          \
    const bool vec = nvec && (reinterpret_cast<uintptr_t>(logits) % (4 * sizeof(S))) == 0 &&                  \
                     logits_row_stride % 4 == 0;                                                              \
    kern = vec ? sample_step_kernel<TAG, true> : sample_step_kernel<TAG, false>;                              \
  } while (0)
  if (logits_dtype == LS_F32) LS_SS(F32);
  else if (logits_dtype == LS_BF16) LS_SS(BF16);
  else if (logits_dtype == LS_F16) LS_SS(F16);
  else return fail(LS_ERR_DTYPE, "ls_sample_step: logits must be fp32, bf16 or fp16");
#undef LS_SS
  // tps = tiles per wave: as many workgroups as are resident at once (one
  // round), each wave streaming a contiguous range
  const int64_t want_waves = resident_workgroups(kern) * kSSWaves;
  int64_t tpw = (rows * a.ntiles + want_waves - 1) / want_waves;
  if (tpw < 1) tpw = 1;
  a.tps = static_cast<int>(tpw);
  a.slices = static_cast<int>((a.ntiles + kSSWaves * tpw - 1) / (kSSWaves * tpw));
  LS_CHECK(rows * a.slices < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_sample_step: rows x vocab too large for one launch");
  const dim3 grid(static_cast<unsigned>(rows * a.slices));
  hipLaunchKernelGGL(kern, grid, dim3(kSS), 0, static_cast<hipStream_t>(stream), a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}
