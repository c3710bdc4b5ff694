// Row-scan machinery shared by the stochastic-verify kernels.
//
// A "row" is one vocabulary-wide vector of logits (one target position or one
// draft position).  A workgroup of kT threads streams it once with 16-byte
// loads and, per element, applies the logit transform (penalties, vocabulary
// mask), tracks the running maximum, optionally the softmax normaliser, and
// appends elements that can still belong to the sampling support to an LDS
// candidate buffer.  The buffer is compacted with an LDS radix select whenever
// it fills, so its threshold rises as the scan proceeds.  At the end the
// exact support (top-k with ties to the lowest index, then top-p, then min-p)
// is determined from the buffer alone.
//
// Semantics follow the reference torch forms:
//   penalties   vendor/sglang/python/sglang/srt/sampling/sampling_batch_info.py:269-286
//               (additive, then repetition scaling), penaltylib/*_penalty.py
//   bitmask     .../srt/constrained/triton_ops/bitmask_ops.py:60-81
//   top-k/top-p .../srt/speculative/dflash_utils.py:743-810 and
//               .../srt/layers/sampler.py:497-510, 666-675
//   min-p       .../srt/layers/sampler.py:238-242
#pragma once

#include "common.h"

namespace ls {
namespace rs {

constexpr int kT = 256;                // threads per workgroup
constexpr int kNBHi = 1024;            // compaction trigger (entries)
constexpr int kNBuf = kNBHi + 2048;    // LDS candidate capacity (entries)
constexpr int kCap = 1024;             // max support entries per row record
constexpr float kDeltaTopP = 20.0f;    // top-p-only candidates: s >= max - 20

enum Mode : int { kModeTopK = 0, kModeFilter = 1, kModeDense = 2 };

enum RowFlags : int {
  kFlagOverflow = 1,  // support could not be determined from the candidate buffer
  kFlagDense = 2,     // support is the whole vocabulary
  kFlagSkip = 4,      // row not processed (draft row of an all-accepted request)
  kFlagUnscanned = 8, // row statistics not computed (fallback computes them)
};

// Per-request sampling parameters of one row.
struct Params {
  float temperature;
  int top_k;
  float top_p;
  float min_p;
};

__device__ __forceinline__ int row_mode(const Params& p, int64_t vocab) {
  if (p.top_k < vocab) return kModeTopK;
  if (p.top_p < 1.0f || p.min_p > 0.0f) return kModeFilter;
  return kModeDense;
}

// Logit transform context of one row (all pointers may be null).
struct XForm {
  const uint32_t* pbits;  // presence bitmap of the request's history [W32]
  const uint32_t* prank;  // exclusive popcount prefix per bitmap word [W32]
  const float* padd;      // additive penalty per present token, by rank (null: all zero)
  float rep;              // repetition scaling of present tokens
  int quirk;              // 1: verify-path quirk (penalty built on zeros)
  const uint32_t* mbits;  // vocabulary mask row [W32] (bit 0 -> -inf)
};

__device__ __forceinline__ float penalise(float x, float a, float r, int quirk) {
  if (!quirk) {
    x = x + a;
    return x < 0.f ? x * r : x / r;
  }
  float p = a < 0.f ? a * r : a / r;
  return x + p;
}

// Transform one element at vocabulary index v (scalar path).
__device__ __forceinline__ float transform1(const XForm& f, float x, int64_t v) {
  const int64_t w = v >> 5;
  const uint32_t bit = 1u << (v & 31);
  if (f.pbits) {
    const uint32_t word = f.pbits[w];
    if (word & bit) {
      const float a = f.padd ? f.padd[f.prank[w] + __popc(word & (bit - 1u))] : 0.f;
      x = penalise(x, a, f.rep, f.quirk);
    }
  }
  if (f.mbits && !(f.mbits[w] & bit)) x = -INFINITY;
  return x;
}

// Transform P consecutive elements starting at e0 (P in {4, 8}, e0 % P == 0).
template <int P>
__device__ __forceinline__ void transform_vec(const XForm& f, float* x, int64_t e0) {
  const int64_t w = e0 >> 5;
  const int sh = static_cast<int>(e0 & 31);
  constexpr uint32_t lanes = (1u << P) - 1u;
  if (f.pbits) {
    const uint32_t word = f.pbits[w];
    uint32_t hit = (word >> sh) & lanes;
    if (hit) {
      if (f.padd) {
        uint32_t rank = f.prank[w] + __popc(word & ((1u << sh) - 1u));
#pragma unroll
        for (int k = 0; k < P; ++k) {
          if ((hit >> k) & 1u) {
            x[k] = penalise(x[k], f.padd[rank], f.rep, f.quirk);
            ++rank;
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < P; ++k)
          if ((hit >> k) & 1u) x[k] = penalise(x[k], 0.f, f.rep, f.quirk);
      }
    }
  }
  if (f.mbits) {
    const uint32_t m = (f.mbits[w] >> sh) & lanes;
    if (m != lanes) {
#pragma unroll
      for (int k = 0; k < P; ++k)
        if (!((m >> k) & 1u)) x[k] = -INFINITY;
    }
  }
}

// Candidate key: larger scaled logit first, then the lower index.
__device__ __forceinline__ uint64_t cand_key(float s, int idx) { return argmax_key(s, idx); }
__device__ __forceinline__ float key_s(uint64_t k) { return unordered_f32(static_cast<uint32_t>(k >> 32)); }
__device__ __forceinline__ int key_idx(uint64_t k) { return argmax_key_index(k); }

// Conservative x-domain threshold for "x / T >= s_thr": every x whose
// correctly rounded quotient reaches s_thr is >= the returned value.
__device__ __forceinline__ float x_threshold(float s_thr, float t) {
  if (s_thr == -INFINITY) return -FLT_MAX;
  float x = s_thr * t;
  return x - fabsf(x) * 9.5367431640625e-07f /* 2^-20 */ - 1e-30f;
}

// LDS state of one row scan.
struct Shared {
  uint64_t buf[kNBuf];
  uint32_t hist[256];
  float red_f[kT / kWave * 2];
  double red_d[kT / kWave];
  int red_i[kT / kWave];
  int count;
  int sel_digit;
  int sel_above;
  float tau_x;      // current x-domain append threshold
  float wg_max_x;   // workgroup running maximum of x (filter mode)
  int overflow;
  int ntrans;       // raw-filter scan: entries [0, ntrans) hold transformed values
};

// Wave-aggregated append of the elements of x[0..P) that are >= tau.
template <int P>
__device__ __forceinline__ void append_vec(Shared& sh, const float* x, float tau, int64_t e0, float t) {
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const bool pass = x[k] >= tau;
    const uint64_t m = __ballot(pass);
    if (m == 0) continue;
    const int n = __popcll(m);
    const int leader = __ffsll(static_cast<long long>(m)) - 1;
    int base = 0;
    if ((threadIdx.x & (kWave - 1)) == leader) base = atomicAdd(&sh.count, n);
    base = __shfl(base, leader, kWave);
    if (pass) {
      const int off = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
      const int pos = base + off;
      if (pos < kNBuf) sh.buf[pos] = cand_key(x[k] / t, static_cast<int>(e0 + k));
    }
  }
}

// Ordered-s (high 32 bits of a key) of the k-th largest entry among buf[0..n)
// (ties counted), by a 4 x 8-bit MSB-first radix select.  k in [1, n].
// Must be called by all threads of the workgroup.
__device__ __forceinline__ uint32_t select_kth_s(Shared& sh, int n, int k) {
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
  const int tid = threadIdx.x;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    sh.hist[tid] = 0;  // kT == 256 buckets
    __syncthreads();
    for (int i = tid; i < n; i += kT) {
      const uint32_t h = static_cast<uint32_t>(sh.buf[i] >> 32);
      if ((h & pmask) == prefix) atomicAdd(&sh.hist[(h >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < kWave) {
      // Suffix counts from the top digit down: lane l owns digits 4l..4l+3.
      uint32_t c[4];
      uint32_t local = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = sh.hist[4 * tid + j];
        local += c[j];
      }
      // inclusive suffix sum over lanes (lanes above hold larger digits)
      uint32_t suf = local;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        uint32_t v = __shfl_down(suf, o, kWave);
        if (tid + o < kWave) suf += v;
      }
      uint32_t above = suf - local;  // entries in digits owned by higher lanes
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        if (above < static_cast<uint32_t>(remaining) && above + c[j] >= static_cast<uint32_t>(remaining)) {
          sh.sel_digit = 4 * tid + j;
          sh.sel_above = static_cast<int>(above);
        }
        above += c[j];
      }
    }
    __syncthreads();
    const uint32_t d = static_cast<uint32_t>(sh.sel_digit);
    remaining -= sh.sel_above;
    prefix |= d << shift;
    pmask |= 255u << shift;
    __syncthreads();
  }
  return prefix;
}

// Keep only entries whose ordered-s is >= thr (stable).  All threads.
__device__ __forceinline__ void compact_ge(Shared& sh, uint32_t thr) {
  const int n = min(sh.count, kNBuf);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  __syncthreads();
  int out = 0;
  for (int r = 0; r < n; r += kT) {
    const int i = r + tid;
    uint64_t key = 0;
    bool keep = false;
    if (i < n) {
      key = sh.buf[i];
      keep = static_cast<uint32_t>(key >> 32) >= thr;
    }
    const uint64_t m = __ballot(keep);
    if (lane == 0) sh.red_i[wid] = __popcll(m);
    __syncthreads();
    int before = out;
    for (int w = 0; w < wid; ++w) before += sh.red_i[w];
    int total = 0;
    for (int w = 0; w < kT / kWave; ++w) total += sh.red_i[w];
    if (keep) {
      const int off = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
      sh.buf[before + off] = key;  // before + off <= i: never overwrites an unread entry
    }
    out += total;
    __syncthreads();
  }
  if (tid == 0) sh.count = out;
  __syncthreads();
}

// Sort buf[0..n) descending (bitonic, padded with zeros to a power of two).
__device__ __forceinline__ void sort_desc(Shared& sh, int n) {
  int np = 1;
  while (np < n) np <<= 1;
  const int tid = threadIdx.x;
  for (int i = n + tid; i < np; i += kT) sh.buf[i] = 0;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < np / 2; i += kT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const uint64_t a = sh.buf[lo], b = sh.buf[hi];
        if ((a < b) == desc) {
          sh.buf[lo] = b;
          sh.buf[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ float block_sum(Shared& sh, float v) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sh.red_f[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < kT / kWave; ++w) t += sh.red_f[w];
  __syncthreads();
  return t;
}

// fp64 block sum (masses that decide a top-p / min-p boundary).
__device__ __forceinline__ double block_sum_d(Shared& sh, double v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sh.red_d[wid] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kT / kWave; ++w) t += sh.red_d[w];
  __syncthreads();
  return t;
}

__device__ __forceinline__ float block_max(Shared& sh, float v) {
  v = wave_max(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sh.red_f[wid] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int w = 0; w < kT / kWave; ++w) t = fmaxf(t, sh.red_f[w]);
  __syncthreads();
  return t;
}

// Result of finalising one row.
struct Support {
  float m;       // maximum scaled logit
  float z;       // normaliser: p(v) = exp(s_v - m) / z on the support
  int n;         // support size (entries buf[0..n) sorted by key), -1 = dense
  int flags;
  uint64_t last; // key of the last support entry (membership: key >= last)
};

}  // namespace rs
}  // namespace ls
