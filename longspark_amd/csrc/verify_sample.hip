// Stochastic (rejection-sampling) chain verification, fused over the whole
// target block:
//
//   target_scan  grid (B*K rows) x S slices.  Streams every target row once
//                (bf16 / fp16 / fp32, 16-byte loads), applies penalties and the
//                vocabulary mask in registers, and determines the row's
//                sampling support exactly: temperature, top-k (ties to the
//                lowest index), top-p, min-p.  Writes a row record with the
//                probability of the verified drafted token.
//   draft_scan   grid B x S.  Computes the first rejection L of its request
//                and, for rejected requests only, scans draft row L the same
//                way to rebuild the draft distribution q there.
//   resolve      grid B.  Residual max(p - q, 0) over the target support,
//                1e-8 degenerate-mass fallback to p, inverse-CDF draw.
//
// Semantics follow vendor/sglang/python/sglang/srt/speculative/
// dspark_components/kernels/accept_sampling.py:259-343 (single-q acceptance
// with the q row rebuilt from the draft logits; unnormalised CDF
// "first v with cumsum > u * total"), with the target distribution of
// .../speculative/dflash_utils.py:743-810 plus min-p, and the draft-probs
// ("dense q") acceptance of .../speculative/reject_sampling.py:5-156.
#include "rowscan.h"
#include <stdlib.h>

namespace ls {
namespace {
using namespace rs;

struct RowRec {
  float m;        // max scaled logit of the row
  float z;        // normaliser of the support
  float p_cand;   // probability of the drafted token this row verifies
  int n;          // support entries (-1: dense support)
  int flags;
  int why;        // diagnostics: Why bits of a row resolved by the fallback
  uint64_t last;  // key of the last support entry
};

struct Args {
  // target
  const void* logits;
  int64_t lrs;
  const void* cand;
  int64_t csb, csk;
  int cfirst;
  int64_t batch;
  int width;
  int64_t vocab;
  const float* temps;
  const int32_t* top_ks;
  const float* top_ps;
  const float* min_ps;
  // penalties / mask
  const uint32_t* pbits;
  const uint32_t* prank;
  int64_t pws;
  const float* padd;
  int64_t pas;
  const float* prep;
  int quirk;
  const int32_t* pnonpos;
  const uint32_t* mask;
  int64_t mrs;
  int mask_per_request;
  // draft
  int q_mode;  // 0: sampled q + draft logits; 1: dense draft probabilities
  const float* dtp;
  int64_t dtp_sb;
  const void* draft;
  int64_t dsb, dsk;
  const float* d_temps;
  const int32_t* d_top_ks;
  const float* d_top_ps;
  const float* d_min_ps;
  // randomness
  const float* uni;
  int64_t usb;
  const float* funi;
  // outputs
  int32_t* accept;
  int64_t* bonus;
  float* p_cand_out;  // [B, K-1] or null
  int32_t* status;    // [1] or null: OR of row flags that blocked a request
  const int32_t* cutoff;  // [B] verify lengths or null: accepted length capped at cutoff - 1
  int32_t* trim;          // [B] or null: accepted drafts removed by the cap
  int cand_i64;           // candidates are int64 (else int32)
  // workspace
  uint32_t* cnt_t;    // [B*K]
  uint32_t* cnt_d;    // [B]
  RowRec* rec_t;      // [B*K]
  int32_t* sidx_t;    // [B*K, kCap]
  float* sp_t;        // [B*K, kCap]
  RowRec* rec_d;      // [B]
  int32_t* sidx_d;    // [B, kCap]
  float* sp_d;        // [B, kCap]
  uint64_t* pub_t;    // [B*K, kNBuf] slice hand-off (S_t > 1)
  uint64_t* pubs_t;   // [B*K, S_t, 2]
  uint64_t* pub_d;    // [B, kNBuf]
  uint64_t* pubs_d;   // [B, S_d, 2]
  int clear_status;    // 1 in the call's first launch: its first workgroup zeroes *status
  int hint;            // which scan kernels the launcher runs (Hint)
  int wave;            // 1: target_wave_kernel runs (takes raw rows with k <= kWaveMaxK)
  int wave_only;       // 1: no workgroup raw scan follows (the wave kernel lists every other raw row)
  int dwave;           // 1: draft_wave_kernel runs (takes draft rows that are top-k with k <= kWaveMaxK)
  int dwave_only;      // 1: no workgroup draft scan follows
  int fuse_draft;      // 1: verify_wave_kernel's grid also carries the draft slices (after the target rows)
  int inline_fb;       // 1: no target fallback launch; resolve runs the exact pass on the rows it needs
  int dslices;         // wavefront draft slices per request (<= kDraftSlices)
  uint64_t* acc_t;     // [B*K] acceptance word of each target row (fused launch; zero when not published)
  uint32_t* list_cnt;  // counters [2]: rows waiting for the exact fallback (target, draft)
  int32_t* list_t;     // [B*K]
  int32_t* list_d;     // [B]
  int s_t, s_d;
};

// Drafted token of a target row and its transformed logit (tok < 0: none).
struct CandRec {
  float x;
  int tok;
};

// ------------------------------------------------------------------ scan ---

struct ScanOut {
  float mx;   // running max of x (thread)
  float mz;   // reference max of z (thread)
  double z;   // sum exp((x - mz) / T) (thread), accumulated in fp64: it
              // decides top-p / min-p boundaries over the whole row
};

constexpr int kMaint = 4;  // steps between maintenance points

// Why a row went to the exact fallback (kept in RowRec::why for diagnostics).
enum Why : int {
  kWhyLost = 1,       // more appends than the buffer holds between maintenance points
  kWhyTies = 2,       // top-k compaction left more than the trigger (ties)
  kWhyFilter = 4,     // min-p / top-p candidates exceed the buffer
  kWhyMerge = 8,      // slice hand-off could not hold the candidates
  kWhySort = 16,      // more than 2048 candidates at finalisation
  kWhyNucleus = 32,   // top-p nucleus extends past the candidates
  kWhyCap = 64,       // support larger than a record holds
  kWhyHint = 128,     // raw-only launch: row needs the exact path, never scanned
  kWhyExact = 256,    // record written by the fallback
  kWhyDefer = 512,    // draft row: acceptance not known when its slices ran (resolve takes it)
};

// A lower bound of the k-th largest (ties counted) of the kT values v (one
// per thread), k <= kT: each wave sorts its 64 values with a bitonic network
// of lane shuffles and takes its ceil(k / waves)-th largest; at least k of
// the values are >= the smallest of those, so it is a valid lower bound.
__device__ __forceinline__ float kth_largest_of_block(Shared& sh, float v, int k) {
  constexpr int kWaves = kT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float o = __shfl_xor(v, stride, kWave);
      // descending blocks keep the maximum in the lower lane of each pair
      const bool desc = (lane & size) == 0 || size == kWave;
      const bool lower = (lane & stride) == 0;
      v = (lower == desc) ? fmaxf(v, o) : fminf(v, o);
    }
  }
  const int j = (k + kWaves - 1) / kWaves;  // 1 <= j <= 64
  const float wj = __shfl(v, j - 1, kWave);
  __syncthreads();
  if (lane == 0) sh.red_f[wid] = wj;
  __syncthreads();
  float r = sh.red_f[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fminf(r, sh.red_f[w]);
  __syncthreads();
  return r;
}

// Compaction of an over-full candidate buffer (all threads; rare).
__device__ __forceinline__ void compact_slow(Shared& sh, int mode, int k, float t, float off_s) {
  const int count = sh.count;
  if (count > kNBuf) {
    __syncthreads();
    if (threadIdx.x == 0) { sh.overflow |= kWhyLost; sh.tau_x = INFINITY; }
    __syncthreads();
    return;
  }
  if (mode == kModeTopK) {
    const uint32_t thr = select_kth_s(sh, count, k);
    compact_ge(sh, thr);
    if (threadIdx.x == 0) {
      if (sh.count > kNBHi) { sh.overflow |= kWhyTies; sh.tau_x = INFINITY; }
      else sh.tau_x = x_threshold(unordered_f32(thr), t);
    }
  } else {
    const float wmx = unordered_f32(*reinterpret_cast<unsigned*>(&sh.wg_max_x));
    compact_ge(sh, ordered_f32(wmx / t + off_s));
    if (threadIdx.x == 0 && sh.count > kNBHi) { sh.overflow |= kWhyFilter; sh.tau_x = INFINITY; }
  }
  __syncthreads();
}

// One maintenance point (all threads, once per step): publish the running
// maximum (filter mode), compact the buffer when over the trigger, and return
// the append threshold to use until the next step.
__device__ __forceinline__ float maintain(Shared& sh, int mode, int k, float t, float off_s, float mx_thread) {
  if (mode == kModeFilter) {
    const float wm = wave_max(mx_thread);
    if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(reinterpret_cast<unsigned*>(&sh.wg_max_x), ordered_f32(wm));
  }
  __syncthreads();
  // Every thread reads the decision inputs before any thread appends again
  // (second barrier), so all threads take the same branch below.
  const int count = sh.count;
  const int ovf = sh.overflow;
  const float wmx = unordered_f32(*reinterpret_cast<unsigned*>(&sh.wg_max_x));
  __syncthreads();
  if (count > kNBHi && !ovf) compact_slow(sh, mode, k, t, off_s);
  float tau = sh.tau_x;
  if (mode == kModeFilter && !sh.overflow) tau = x_threshold(wmx / t + off_s, t);
  return tau;
}

// Ring slot: one 16-byte logits vector plus the 32-token words that cover it
// (presence bitmap, its popcount rank base, vocabulary mask), all prefetched
// four steps ahead so the per-element transform never waits on a load.
struct Slot {
  uint4 v;
  uint32_t pb, pr, mb;
};

template <int P>
__device__ __forceinline__ void load_slot(Slot& s, const uint4* vp, int64_t i, int64_t nfull, const XForm& f,
                                          int64_t b) {
  if (i < nfull) {
    s.v = load16_stream(vp + i);
    const int64_t w = (b + i * P) >> 5;
    if (f.pbits) {
      s.pb = f.pbits[w];
      if (f.padd) s.pr = f.prank[w];  // ranks only index additive values
    }
    if (f.mbits) s.mb = f.mbits[w];
  }
}

// Transform P consecutive elements starting at e0 given their prefetched words.
template <int P>
__device__ __forceinline__ void transform_words(const XForm& f, float* x, int64_t e0, const Slot& s) {
  const int sh = static_cast<int>(e0 & 31);
  constexpr uint32_t lanes = (1u << P) - 1u;
  if (f.pbits) {
    const uint32_t hit = (s.pb >> sh) & lanes;
    if (hit) {
      uint32_t rank = s.pr + __popc(s.pb & ((1u << sh) - 1u));
#pragma unroll
      for (int k = 0; k < P; ++k) {
        if ((hit >> k) & 1u) {
          const float a = f.padd ? f.padd[rank] : 0.f;
          x[k] = penalise(x[k], a, f.rep, f.quirk);
          ++rank;
        }
      }
    }
  }
  if (f.mbits) {
    const uint32_t m = (s.mb >> sh) & lanes;
    if (m != lanes) {
#pragma unroll
      for (int k = 0; k < P; ++k)
        if (!((m >> k) & 1u)) x[k] = -INFINITY;
    }
  }
}

template <typename Tag, bool kVec>
__device__ ScanOut scan_range(Shared& sh, const typename Tag::storage* row, int64_t b, int64_t e,
                              const XForm& f, float t, int mode, int k, float off_s) {
  using S = typename Tag::storage;
  constexpr int P = Tag::kPerVec;
  const bool need_z = mode != kModeTopK;
  const bool xform = f.pbits || f.mbits;
  const float c2 = 1.4426950408889634f / t;
  const float off_x = (mode == kModeFilter) ? off_s * t : -INFINITY;
  const int tid = threadIdx.x;
  ScanOut o{-FLT_MAX, -FLT_MAX, 0.f};
  float tau = sh.tau_x;
  const int64_t nvv = (e - b + P - 1) / P;        // virtual vectors in [b, e)
  const int64_t nfull = kVec ? (e - b) / P : 0;    // vectors loadable with 16-byte loads
  const int64_t steps = (nvv + kT - 1) / kT;
  const uint4* vp = reinterpret_cast<const uint4*>(row + b);
  // Four slots in flight per thread, rotated through a ring.
  Slot r0 = {}, r1 = {}, r2 = {}, r3 = {};
  load_slot<P>(r0, vp, tid, nfull, f, b);
  load_slot<P>(r1, vp, kT + tid, nfull, f, b);
  load_slot<P>(r2, vp, 2 * kT + tid, nfull, f, b);
  load_slot<P>(r3, vp, 3 * kT + tid, nfull, f, b);
  int64_t st = 0;
  if (mode == kModeTopK && k <= kT && nfull >= 8 * kT) {
    // Prologue: the first four vectors of every thread give kT per-thread
    // maxima; their k-th largest is a lower bound of the row's k-th largest
    // value (k distinct elements reach it), so it can start the threshold.
    float lm = -INFINITY;
#pragma unroll 1
    for (int d = 0; d < 4; ++d) {
      const Slot& s = d == 0 ? r0 : d == 1 ? r1 : d == 2 ? r2 : r3;
      float x[P];
      unpack16<Tag>(s.v, x);
      if (xform) transform_words<P>(f, x, b + (static_cast<int64_t>(d) * kT + tid) * P, s);
#pragma unroll
      for (int q = 0; q < P; ++q) lm = fmaxf(lm, x[q]);
    }
    float t0 = kth_largest_of_block(sh, lm, k);
    t0 = t0 - fabsf(t0) * 9.5367431640625e-07f - 1e-30f;
    tau = fmaxf(tau, t0);
    if (tid == 0) sh.tau_x = tau;  // read again at the next maintenance point
    o.mx = lm;
#pragma unroll 1
    for (int d = 0; d < 4; ++d) {
      const Slot& s = d == 0 ? r0 : d == 1 ? r1 : d == 2 ? r2 : r3;
      float x[P];
      unpack16<Tag>(s.v, x);
      const int64_t e0 = b + (static_cast<int64_t>(d) * kT + tid) * P;
      if (xform) transform_words<P>(f, x, e0, s);
      float vm = x[0];
#pragma unroll
      for (int q = 1; q < P; ++q) vm = fmaxf(vm, x[q]);
      if (__ballot(vm >= tau)) append_vec<P>(sh, x, tau, e0, t);
    }
    load_slot<P>(r0, vp, 4 * kT + tid, nfull, f, b);
    load_slot<P>(r1, vp, 5 * kT + tid, nfull, f, b);
    load_slot<P>(r2, vp, 6 * kT + tid, nfull, f, b);
    load_slot<P>(r3, vp, 7 * kT + tid, nfull, f, b);
    st = 4;
  }
  for (; st < steps; ++st) {
    const int64_t i = st * kT + tid;
    const Slot cur = r0;
    r0 = r1;
    r1 = r2;
    r2 = r3;
    load_slot<P>(r3, vp, i + 4 * kT, nfull, f, b);
    float x[P];
    const int64_t e0 = b + i * P;
    if (i < nfull) {
      unpack16<Tag>(cur.v, x);
      if (xform) transform_words<P>(f, x, e0, cur);
    } else {
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int64_t v = e0 + q;
        x[q] = (i < nvv && v < e) ? transform1(f, to_f32<S>(row[v]), v) : -INFINITY;
      }
    }
    float vmax = x[0];
#pragma unroll
    for (int q = 1; q < P; ++q) vmax = fmaxf(vmax, x[q]);
    if (need_z) {
      if (vmax > o.mz) {
        o.z *= static_cast<double>(__builtin_amdgcn_exp2f((o.mz - vmax) * c2));
        o.mz = vmax;
      }
      float vs = 0.f;
#pragma unroll
      for (int q = 0; q < P; ++q) vs += __builtin_amdgcn_exp2f((x[q] - o.mz) * c2);
      o.z += static_cast<double>(vs);
    }
    o.mx = fmaxf(o.mx, vmax);
    const float tau_eff = fmaxf(tau, o.mx + off_x);
    if (__ballot(vmax >= tau_eff)) append_vec<P>(sh, x, tau_eff, e0, t);
    // Maintenance every kMaint steps (and at the last): between two points at
    // most kMaint * kT * P entries arrive; any beyond the buffer are dropped and
    // flagged, which sends the row to the exact fallback.
    if ((st & (kMaint - 1)) == kMaint - 1 || st + 1 == steps) tau = maintain(sh, mode, k, t, off_s, o.mx);
  }
  return o;
}

// ----------------------------------------------------- raw-filter top-k ---
//
// Top-k rows whose transform never raises a logit (no penalties, or
// repetition >= 1 with additive penalties <= 0; the mask only lowers values to
// -inf) are scanned on the raw logits: every element whose transformed value
// can reach the threshold has a raw value that does, so filtering raw values
// keeps every candidate.  Candidates are buffered with raw keys and
// transformed in bulk when the buffer is compacted and at the end; thresholds
// always come from transformed values.  Keys here are in the logit (x) domain
// and become scaled-logit (x / T) keys at the end of the slice.

constexpr int kRawMaint = 16;  // steps between maintenance points

__device__ __forceinline__ float x_lower(float x) {
  return x - fabsf(x) * 9.5367431640625e-07f /* 2^-20 */ - 1e-30f;
}

// Wave-aggregated append of raw keys (one LDS atomic per wave).  All 64
// lanes of the wave must call it.
template <int P>
__device__ __forceinline__ void append_raw(Shared& sh, const float* x, float tau, int64_t e0) {
  uint32_t pm = 0;
#pragma unroll
  for (int q = 0; q < P; ++q) pm |= (x[q] >= tau ? 1u : 0u) << q;
  const int cnt = __popc(pm);
  const int lane = threadIdx.x & (kWave - 1);
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  const int total = __shfl(incl, kWave - 1, kWave);
  int base = 0;
  if (lane == 0) base = atomicAdd(&sh.count, total);
  base = __shfl(base, 0, kWave);
  int pos = base + incl - cnt;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    if ((pm >> q) & 1u) {
      if (pos < kNBuf) sh.buf[pos] = cand_key(x[q], static_cast<int>(e0 + q));
      ++pos;
    }
  }
}

// Transform the buffered entries appended since the last transform (all threads).
__device__ __forceinline__ void transform_pending(Shared& sh, const XForm& f) {
  const int n = min(sh.count, kNBuf);
  if (f.pbits || f.mbits) {
    for (int i = sh.ntrans + static_cast<int>(threadIdx.x); i < n; i += kT) {
      const uint64_t key = sh.buf[i];
      const int idx = key_idx(key);
      sh.buf[i] = cand_key(transform1(f, key_s(key), idx), idx);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) sh.ntrans = n;
  __syncthreads();
}

// Transform, select the k-th largest transformed value and keep the entries
// within the rounding margin of it (all threads).  Returns the new raw
// threshold.
__device__ __forceinline__ float compact_raw(Shared& sh, const XForm& f, int k) {
  transform_pending(sh, f);
  const int n = min(sh.count, kNBuf);
  if (n <= k) return -FLT_MAX;
  const float xk = unordered_f32(select_kth_s(sh, n, k));
  const float thr = x_lower(xk);
  compact_ge(sh, ordered_f32(thr));
  if (threadIdx.x == 0) sh.ntrans = sh.count;
  __syncthreads();
  return thr;
}

__device__ __forceinline__ float maintain_raw(Shared& sh, const XForm& f, int k, int trigger) {
  __syncthreads();
  const int count = sh.count;
  const int ovf = sh.overflow;
  __syncthreads();
  if (ovf) return INFINITY;
  if (count > kNBuf) {
    if (threadIdx.x == 0) { sh.overflow |= kWhyLost; sh.tau_x = INFINITY; }
    __syncthreads();
    return INFINITY;
  }
  if (count > trigger) {
    const float thr = compact_raw(sh, f, k);
    if (threadIdx.x == 0) {
      if (sh.count > kNBHi) { sh.overflow |= kWhyTies; sh.tau_x = INFINITY; }
      else sh.tau_x = fmaxf(sh.tau_x, thr);
    }
    __syncthreads();
  }
  return sh.tau_x;
}

template <typename Tag, bool kVec>
__device__ ScanOut scan_topk_raw(Shared& sh, const typename Tag::storage* row, int64_t b, int64_t e,
                                 const XForm& f, int k) {
  using S = typename Tag::storage;
  constexpr int P = Tag::kPerVec;
  const int tid = threadIdx.x;
  const int trigger = min(kNBHi, max(2 * k + 64, 256));
  // Larger k admits more candidates per step: compact more often.
  const int maint_mask = k <= 64 ? kRawMaint - 1 : (k <= 256 ? 3 : 0);
  ScanOut o{-FLT_MAX, -FLT_MAX, 0.f};
  float tau = sh.tau_x;
  const int64_t nvv = (e - b + P - 1) / P;
  const int64_t nfull = kVec ? (e - b) / P : 0;
  const int64_t steps = (nvv + kT - 1) / kT;
  const uint4* vp = reinterpret_cast<const uint4*>(row + b);
  uint4 r0 = {}, r1 = {}, r2 = {}, r3 = {};
  if (tid < nfull) r0 = load16_stream(vp + tid);
  if (kT + tid < nfull) r1 = load16_stream(vp + kT + tid);
  if (2 * kT + tid < nfull) r2 = load16_stream(vp + 2 * kT + tid);
  if (3 * kT + tid < nfull) r3 = load16_stream(vp + 3 * kT + tid);
  int64_t st = 0;
  if (k <= kT && nfull >= 8 * kT) {
    // Prologue: the k-th largest of the kT per-thread maxima of the first
    // four transformed vectors is a lower bound of the row's k-th largest
    // transformed value.
    float lm = -INFINITY, rm = -INFINITY;
    // Penalty and mask words of the four vectors, all requested at once.
    Slot w4[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int64_t w = (b + (static_cast<int64_t>(d) * kT + tid) * P) >> 5;
      w4[d].pb = f.pbits ? f.pbits[w] : 0u;
      w4[d].pr = (f.pbits && f.padd) ? f.prank[w] : 0u;
      w4[d].mb = f.mbits ? f.mbits[w] : ~0u;
    }
#pragma unroll 1
    for (int d = 0; d < 4; ++d) {
      const uint4 v = d == 0 ? r0 : d == 1 ? r1 : d == 2 ? r2 : r3;
      const Slot& wd = d == 0 ? w4[0] : d == 1 ? w4[1] : d == 2 ? w4[2] : w4[3];
      float x[P];
      unpack16<Tag>(v, x);
#pragma unroll
      for (int q = 0; q < P; ++q) rm = fmaxf(rm, x[q]);
      if (f.pbits || f.mbits) transform_words<P>(f, x, b + (static_cast<int64_t>(d) * kT + tid) * P, wd);
#pragma unroll
      for (int q = 0; q < P; ++q) lm = fmaxf(lm, x[q]);
    }
    tau = fmaxf(tau, x_lower(kth_largest_of_block(sh, lm, k)));
    if (tid == 0) sh.tau_x = tau;
    o.mx = rm;
#pragma unroll 1
    for (int d = 0; d < 4; ++d) {
      const uint4 v = d == 0 ? r0 : d == 1 ? r1 : d == 2 ? r2 : r3;
      float x[P];
      unpack16<Tag>(v, x);
      float vm = x[0];
#pragma unroll
      for (int q = 1; q < P; ++q) vm = fmaxf(vm, x[q]);
      if (__ballot(vm >= tau)) append_raw<P>(sh, x, tau, b + (static_cast<int64_t>(d) * kT + tid) * P);
    }
    r0 = load16_stream(vp + 4 * kT + tid);
    r1 = load16_stream(vp + 5 * kT + tid);
    r2 = load16_stream(vp + 6 * kT + tid);
    r3 = load16_stream(vp + 7 * kT + tid);
    st = 4;
  }
  for (; st < steps; ++st) {
    const int64_t i = st * kT + tid;
    const uint4 cur = r0;
    r0 = r1;
    r1 = r2;
    r2 = r3;
    if (i + 4 * kT < nfull) r3 = load16_stream(vp + i + 4 * kT);
    float x[P];
    const int64_t e0 = b + i * P;
    if (i < nfull) {
      unpack16<Tag>(cur, x);
    } else {
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int64_t v = e0 + q;
        x[q] = (i < nvv && v < e) ? to_f32<S>(row[v]) : -INFINITY;
      }
    }
    float vmax = x[0];
#pragma unroll
    for (int q = 1; q < P; ++q) vmax = fmaxf(vmax, x[q]);
    o.mx = fmaxf(o.mx, vmax);
    if (__ballot(vmax >= tau)) append_raw<P>(sh, x, tau, e0);
    if ((st & maint_mask) == maint_mask || st + 1 == steps) tau = maintain_raw(sh, f, k, trigger);
  }
  return o;
}

// End of a raw-filter slice: transform what is pending, keep the top k within
// the rounding margin, and re-key the survivors by scaled logit x / T.
__device__ __forceinline__ ScanOut finish_topk_raw(Shared& sh, const ScanOut& o, const XForm& f, int k, float t) {
  ScanOut r;
  r.mx = block_max(sh, o.mx);  // raw maximum: an upper bound of the transformed one
  r.mz = r.mx;
  r.z = 0.f;
  if (!sh.overflow) {
    transform_pending(sh, f);
    const int n = min(sh.count, kNBuf);
    if (n > k) compact_raw(sh, f, k);
    const int m = min(sh.count, kNBuf);
    for (int i = threadIdx.x; i < m; i += kT) {
      const uint64_t key = sh.buf[i];
      const int idx = key_idx(key);
      sh.buf[i] = cand_key(key_s(key) / t, idx);
    }
  }
  __syncthreads();
  return r;
}

__device__ __forceinline__ bool raw_filter_ok(const XForm& f, const int32_t* nonpos, int64_t b) {
  if (!f.pbits) return true;
  return f.rep >= 1.0f && (!f.padd || (nonpos && nonpos[b]));
}

// After the scan of a slice: final compaction of the slice's candidates and
// workgroup-wide statistics.  Returns (max x, reference max, z).
__device__ __forceinline__ ScanOut finish_slice(Shared& sh, const ScanOut& o, int mode, int k, float t, float off_s) {
  ScanOut r;
  r.mx = block_max(sh, o.mx);
  if (mode != kModeTopK) {
    const float gm = r.mx;
    const double zt = (o.mz == -FLT_MAX)
                          ? 0.0
                          : o.z * static_cast<double>(__builtin_amdgcn_exp2f((o.mz - gm) * (1.4426950408889634f / t)));
    r.z = block_sum_d(sh, zt);
    r.mz = gm;
  } else {
    r.z = 0.f;
    r.mz = r.mx;
  }
  if (!sh.overflow) {
    const int count = sh.count;
    if (mode == kModeTopK && count > k) {
      const uint32_t thr = select_kth_s(sh, count, k);
      compact_ge(sh, thr);
    } else if (mode == kModeFilter && count > 0) {
      compact_ge(sh, ordered_f32(r.mx / t + off_s));
    }
  }
  __syncthreads();
  return r;
}

// --------------------------------------------------------------- finalise ---

// Index of the first entry i < n (entries sorted by key, e_i = exp(s_i - m))
// at which the running sum before i, divided by `denom`, exceeds `limit`;
// n if none.  Also returns the full sum of e_i / denom through *total.  The
// running sum is kept in fp64 (it decides the top-p boundary).
__device__ __forceinline__ int first_excl_exceeds(Shared& sh, int n, float m, double denom, float limit,
                                                  float* total) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  __shared__ int found;
  __shared__ double wsum[kT / kWave];
  if (tid == 0) found = n;
  const double lim = static_cast<double>(limit) * denom;
  double carry = 0.0;
  __syncthreads();
  for (int r = 0; r < n; r += kT) {
    const int i = r + tid;
    const double e = i < n ? static_cast<double>(__expf(key_s(sh.buf[i]) - m)) : 0.0;
    double inc = e;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const double v = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += v;
    }
    if (lane == kWave - 1) wsum[wid] = inc;
    __syncthreads();
    double before = carry;
    for (int w = 0; w < wid; ++w) before += wsum[w];
    const double excl = before + inc - e;
    if (i < n && excl > lim) atomicMin(&found, i);
    double tot = 0.0;
    for (int w = 0; w < kT / kWave; ++w) tot += wsum[w];
    carry += tot;
    __syncthreads();
    const int f = found;
    __syncthreads();  // all threads have read `found` before any thread updates it again
    if (f < n) break;
  }
  if (total) *total = static_cast<float>(carry / denom);
  const int res = found;
  __syncthreads();
  return res;
}

// ------------------------------------------------------- exact fallback ---
//
// Used when the candidate buffer cannot hold a row's support (heavy ties at
// the top-k value, top-k above the buffer capacity, a top-p nucleus that is
// not closed by the candidates).  One workgroup re-reads the row from global
// memory several times and selects the exact cut keys by MSB-first radix
// select over the 64-bit candidate keys (8-bit digits): by count for top-k,
// by mass exp(s - m) for top-p, and by value for min-p.

struct Hist {
  uint32_t cnt[256];
  double mass[256];  // fp64: the masses decide top-p boundaries
};

// One pass over the row: histogram of digit (key >> shift) & 255 of every key
// >= kmin whose bits under pmask equal prefix (counts and masses).
template <typename Tag>
__device__ __noinline__ void hist_pass(Hist& h, const typename Tag::storage* row, int64_t vocab, const XForm& f,
                                       float t, float m, uint64_t kmin, uint64_t prefix, uint64_t pmask, int shift) {
  const int tid = threadIdx.x;
  h.cnt[tid] = 0;
  h.mass[tid] = 0.0;
  __syncthreads();
  for (int64_t v = tid; v < vocab; v += kT) {
    const float s = transform1(f, to_f32<typename Tag::storage>(row[v]), v) / t;
    const uint64_t key = cand_key(s, static_cast<int>(v));
    if (key >= kmin && (key & pmask) == prefix) {
      const int d = static_cast<int>((key >> shift) & 255u);
      atomicAdd(&h.cnt[d], 1u);
      atomicAdd(&h.mass[d], static_cast<double>(__expf(s - m)));
    }
  }
  __syncthreads();
}

// k-th largest key of the row (k >= 1).
template <typename Tag>
__device__ __noinline__ uint64_t select_key_by_count(Hist& h, const typename Tag::storage* row, int64_t vocab,
                                                     const XForm& f, float t, float m, int k) {
  __shared__ int s_d, s_above;
  uint64_t prefix = 0, pmask = 0;
  int remaining = k;
  for (int shift = 56; shift >= 0; shift -= 8) {
    hist_pass<Tag>(h, row, vocab, f, t, m, 0, prefix, pmask, shift);
    if (threadIdx.x == 0) {
      int above = 0, d = 0;
      for (d = 255; d > 0; --d) {
        if (above + static_cast<int>(h.cnt[d]) >= remaining) break;
        above += static_cast<int>(h.cnt[d]);
      }
      s_d = d;
      s_above = above;
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(s_d) << shift;
    pmask |= uint64_t(255) << shift;
    remaining -= s_above;
    __syncthreads();
  }
  return prefix;
}

// Smallest key K >= kmin whose excluded mass (sum of exp(s - m) over keys
// > K and >= kmin) is <= limit: the last entry a top-p cut keeps.
template <typename Tag>
__device__ __noinline__ uint64_t select_key_by_mass(Hist& h, const typename Tag::storage* row, int64_t vocab,
                                                    const XForm& f, float t, float m, uint64_t kmin, double limit) {
  __shared__ int s_d;
  __shared__ double s_above;
  uint64_t prefix = 0, pmask = 0;
  double above = 0.0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    hist_pass<Tag>(h, row, vocab, f, t, m, kmin, prefix, pmask, shift);
    if (threadIdx.x == 0) {
      double cum = above, sel_above = above;
      int sel = -1;
      for (int d = 255; d >= 0; --d) {
        if (h.cnt[d] == 0) continue;
        if (cum <= limit) {
          sel = d;
          sel_above = cum;
        } else {
          break;
        }
        cum += h.mass[d];
      }
      s_d = sel < 0 ? 0 : sel;
      s_above = sel_above;
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(s_d) << shift;
    pmask |= uint64_t(255) << shift;
    above = s_above;
    __syncthreads();
  }
  return prefix;
}

// Count and mass of keys >= kmin; optionally the smallest s among keys >=
// kmin with exp(s - m) >= emin (as an ordered value, 0xffffffff if none).
template <typename Tag>
__device__ __noinline__ void tally(Shared& sh, const typename Tag::storage* row, int64_t vocab, const XForm& f, float t,
                                   float m, uint64_t kmin, float emin, int* count, double* mass, uint32_t* smin_ord) {
  __shared__ unsigned s_cnt, s_min;
  const int tid = threadIdx.x;
  if (tid == 0) { s_cnt = 0; s_min = 0xffffffffu; }
  __syncthreads();
  double acc = 0.0;
  unsigned c = 0, mn = 0xffffffffu;
  for (int64_t v = tid; v < vocab; v += kT) {
    const float s = transform1(f, to_f32<typename Tag::storage>(row[v]), v) / t;
    const uint64_t key = cand_key(s, static_cast<int>(v));
    if (key >= kmin) {
      const float e = __expf(s - m);
      acc += static_cast<double>(e);
      ++c;
      if (e >= emin) mn = min(mn, static_cast<unsigned>(key >> 32));
    }
  }
  atomicAdd(&s_cnt, c);
  atomicMin(&s_min, mn);
  const double tot = block_sum_d(sh, acc);
  *count = static_cast<int>(s_cnt);
  *mass = tot;
  *smin_ord = s_min;
  __syncthreads();
}

// Collect every key >= kmin into sh.buf (at most kNBuf entries), sorted descending.
template <typename Tag>
__device__ __noinline__ int collect(Shared& sh, const typename Tag::storage* row, int64_t vocab, const XForm& f,
                                    float t, uint64_t kmin) {
  if (threadIdx.x == 0) sh.count = 0;
  __syncthreads();
  for (int64_t v = threadIdx.x; v < vocab; v += kT) {
    const float s = transform1(f, to_f32<typename Tag::storage>(row[v]), v) / t;
    const uint64_t key = cand_key(s, static_cast<int>(v));
    if (key >= kmin) {
      const int pos = atomicAdd(&sh.count, 1);
      if (pos < kNBuf) sh.buf[pos] = key;
    }
  }
  __syncthreads();
  const int n = min(sh.count, 2048);
  sort_desc(sh, n);
  return n;
}

// Maximum transformed logit and the dense normaliser sum exp((x - max) / T)
// of a row that was never scanned (two passes; fallback only).
template <typename Tag>
__device__ __noinline__ void row_stats(Shared& sh, const typename Tag::storage* row, int64_t vocab, const XForm& f,
                                       float t, float* m_x, double* z) {
  float mx = -FLT_MAX;
  for (int64_t v = threadIdx.x; v < vocab; v += kT)
    mx = fmaxf(mx, transform1(f, to_f32<typename Tag::storage>(row[v]), v));
  mx = block_max(sh, mx);
  double acc = 0.0;
  for (int64_t v = threadIdx.x; v < vocab; v += kT)
    acc += static_cast<double>(__expf((transform1(f, to_f32<typename Tag::storage>(row[v]), v) - mx) / t));
  *m_x = mx;
  *z = block_sum_d(sh, acc);
}

struct Exact {
  float m, z;
  uint64_t kcut;  // support = keys >= kcut
  int n;          // support size
};

// Exact support of a row from global memory.  m_x: row max of x; z_dense:
// sum over the row of exp(s - m) (filter / dense modes).
template <typename Tag>
__device__ __noinline__ Exact exact_support(Shared& sh, const typename Tag::storage* row, int64_t vocab,
                                            const XForm& f, const Params& p, int mode, float m_x, double z_dense) {
  __shared__ Hist h;
  const float t = p.temperature;
  Exact r;
  r.m = m_x / t;
  uint64_t kmin = 0;
  double z1 = z_dense;
  int cnt;
  double mass;
  uint32_t smin;
  if (mode == kModeTopK && p.top_k < vocab) {
    kmin = select_key_by_count<Tag>(h, row, vocab, f, t, r.m, p.top_k);
    tally<Tag>(sh, row, vocab, f, t, r.m, kmin, INFINITY, &cnt, &z1, &smin);
  }
  uint64_t kcut = kmin;
  if (p.top_p < 1.0f) kcut = select_key_by_mass<Tag>(h, row, vocab, f, t, r.m, kmin, p.top_p * z1);
  if (p.min_p > 0.f) {
    // Over the top-p set: p2 = (e / z1) / P with P its mass; drop p2 < p2_max * min_p.
    tally<Tag>(sh, row, vocab, f, t, r.m, kcut, INFINITY, &cnt, &mass, &smin);
    const float pp = static_cast<float>(mass / z1);
    const float z1f = static_cast<float>(z1);
    const float thr = ((1.0f / z1f) / pp) * p.min_p;
    // keep e with (e / z1) / pp >= thr: find the smallest such s
    float emin = thr * pp * z1f;
    tally<Tag>(sh, row, vocab, f, t, r.m, kcut, emin, &cnt, &mass, &smin);
    if (smin != 0xffffffffu) {
      const uint64_t kmp = static_cast<uint64_t>(smin) << 32;
      if (kmp > kcut) kcut = kmp;
    }
  }
  tally<Tag>(sh, row, vocab, f, t, r.m, kcut, INFINITY, &cnt, &mass, &smin);
  r.z = static_cast<float>(mass);
  r.kcut = kcut;
  r.n = cnt;
  return r;
}

// Determine the exact support from the candidate buffer (or, if it could not
// hold the support, from the row itself) and write the row record.  `cand_x`
// is the transformed logit of the drafted token this row verifies.  All
// threads.
__device__ __forceinline__ void finalize_row(Shared& sh, const ScanOut& st, const Params& p, int mode, int64_t vocab,
                                          RowRec* rec, int32_t* sidx, float* sp, int cand_tok, float cand_x,
                                          uint32_t* list_cnt, int32_t* list, int32_t list_id) {
  const int tid = threadIdx.x;
  __shared__ float s_m, s_z;
  __shared__ int s_n, s_flags, s_why;
  __shared__ uint64_t s_last;
  const float t = p.temperature;
  if (tid == 0) {
    s_flags = sh.overflow ? kFlagOverflow : 0;
    s_why = sh.overflow;
    s_last = 0;
  }
  __syncthreads();
  int n = sh.count;
  if (mode == kModeDense) {
    if (tid == 0) {
      s_m = st.mx / t;
      s_z = static_cast<float>(st.z);
      s_n = -1;
      s_flags |= kFlagDense;
    }
  } else if (!s_flags) {
    if (n > 2048) {
      if (tid == 0) { s_flags |= kFlagOverflow; s_why |= kWhySort; }
    } else {
      sort_desc(sh, n);
      if (mode == kModeTopK && n > p.top_k) n = p.top_k;
      const float m = n > 0 ? key_s(sh.buf[0]) : -INFINITY;
      double z1d;
      if (mode == kModeTopK) {
        float acc = 0.f;
        for (int i = tid; i < n; i += kT) acc += __expf(key_s(sh.buf[i]) - m);
        z1d = block_sum_d(sh, static_cast<double>(acc));
      } else {
        z1d = st.z;  // dense normaliser relative to the row maximum
      }
      const float z1 = static_cast<float>(z1d);
      int n_f = n;
      float mass_all = 0.f;
      if (p.top_p < 1.0f && n > 0) {
        n_f = first_excl_exceeds(sh, n, m, z1d, p.top_p, &mass_all);
        if (mode == kModeFilter && p.min_p <= 0.f && n_f == n && mass_all <= p.top_p) {
          if (tid == 0) { s_flags |= kFlagOverflow; s_why |= kWhyNucleus; }  // nucleus open
        }
      }
      if (p.min_p > 0.f && n_f > 0) {
        // Renormalise over the top-p prefix, then drop p < p_max * min_p.
        float acc = 0.f;
        for (int i = tid; i < n_f; i += kT) acc += __expf(key_s(sh.buf[i]) - m) / z1;
        const float pp = block_sum(sh, acc);
        const float p0 = (__expf(key_s(sh.buf[0]) - m) / z1) / pp;
        const float thr = p0 * p.min_p;
        __shared__ int cut;
        if (tid == 0) cut = n_f;
        __syncthreads();
        for (int i = tid; i < n_f; i += kT) {
          const float pi = (__expf(key_s(sh.buf[i]) - m) / z1) / pp;
          if (pi < thr) atomicMin(&cut, i);
        }
        __syncthreads();
        n_f = cut;
        __syncthreads();
      }
      if (n_f > kCap && tid == 0) { s_flags |= kFlagOverflow; s_why |= kWhyCap; }
      float acc = 0.f;
      for (int i = tid; i < n_f; i += kT) acc += __expf(key_s(sh.buf[i]) - m);
      const float zf = block_sum(sh, acc);
      if (tid == 0) {
        s_m = m;
        s_z = zf;
        s_n = n_f;
        s_last = n_f > 0 ? sh.buf[n_f - 1] : ~uint64_t(0);
      }
      __syncthreads();
    }
  }
  __syncthreads();
  if (s_flags & kFlagOverflow) {
    // Resolved exactly by the fallback kernel; keep the row statistics.
    if (tid == 0) {
      RowRec r{};
      r.m = st.mx;  // x-domain maximum
      r.z = static_cast<float>(st.z);   // dense normaliser (filter / dense modes)
      r.flags = kFlagOverflow;
      r.why = s_why;
      *rec = r;
      const uint32_t slot = atomic_add_u32(list_cnt, 1u);
      list[slot] = list_id;
    }
    __syncthreads();
    return;
  }
  if (s_n > 0) {
    for (int i = tid; i < s_n; i += kT) {
      const uint64_t kk = sh.buf[i];
      sidx[i] = key_idx(kk);
      sp[i] = __expf(key_s(kk) - s_m) / s_z;
    }
  }
  __syncthreads();
  if (tid == 0) {
    RowRec r;
    r.m = s_m;
    r.z = s_z;
    r.n = s_n;
    r.flags = s_flags;
    r.why = 0;
    r.last = s_last;
    r.p_cand = 0.f;
    if (cand_tok >= 0) {
      const float sc = cand_x / t;
      const uint64_t kc = cand_key(sc, cand_tok);
      r.p_cand = (kc >= r.last && (r.n != 0 || (r.flags & kFlagDense))) ? __expf(sc - r.m) / r.z : 0.f;
    }
    *rec = r;
  }
  __syncthreads();
}

// ------------------------------------------------------- slice hand-off ---

// Publish this slice's candidates and statistics, arrive on the row counter,
// and, in the last slice to arrive, gather all slices into LDS.  Returns true
// in the workgroup that continues with the row.
__device__ __forceinline__ bool merge_slices(Shared& sh, ScanOut& st, int mode, int slices, int slice, uint64_t* pub,
                             uint64_t* pubs, uint32_t* counter, float t) {
  const int tid = threadIdx.x;
  __shared__ int is_last;
  const int cap = kNBuf / slices;
  const int n = sh.count;
  const bool ovf = sh.overflow || n > cap;
  uint64_t* my = pub + static_cast<int64_t>(slice) * cap;
  if (!ovf)
    for (int i = tid; i < n; i += kT) atomic_put_u64(my + i, sh.buf[i]);
  if (tid == 0) {
    atomic_put_u64(pubs + 2 * slice, ovf ? ~uint64_t(0) : static_cast<uint64_t>(n));
    atomic_put_u64(pubs + 2 * slice + 1,
                   (static_cast<uint64_t>(ordered_f32(st.mx)) << 32) | __float_as_uint(static_cast<float>(st.z)));
  }
  __syncthreads();  // every thread's publishes have completed
  if (tid == 0) is_last = (arrive(counter) == static_cast<uint32_t>(slices - 1));
  __syncthreads();
  if (!is_last) return false;
  __shared__ int offs[17];
  __shared__ float smx[16], sz[16];
  __shared__ double s_zm;
  if (tid == 0) {
    atomic_take_u32(counter);
    int total = 0, bad = 0;
    for (int s = 0; s < slices; ++s) {
      const uint64_t c = atomic_take_u64(pubs + 2 * s);
      const uint64_t mz = atomic_take_u64(pubs + 2 * s + 1);
      offs[s] = total;
      if (c == ~uint64_t(0)) bad = 1;
      else total += static_cast<int>(c);
      smx[s] = unordered_f32(static_cast<uint32_t>(mz >> 32));
      sz[s] = __uint_as_float(static_cast<uint32_t>(mz));
    }
    offs[slices] = total;
    sh.overflow = (bad || total > kNBuf) ? kWhyMerge : 0;
    sh.count = sh.overflow ? 0 : total;
    float gm = -FLT_MAX;
    double z = 0.0;
    for (int s = 0; s < slices; ++s) gm = fmaxf(gm, smx[s]);
    if (mode != kModeTopK) {
      const float c2 = 1.4426950408889634f / t;
      for (int s = 0; s < slices; ++s)
        if (smx[s] != -FLT_MAX)
          z += static_cast<double>(sz[s]) * static_cast<double>(__builtin_amdgcn_exp2f((smx[s] - gm) * c2));
    }
    smx[0] = gm;
    s_zm = z;
  }
  __syncthreads();
  st.mx = smx[0];
  st.mz = smx[0];
  st.z = s_zm;
  if (!sh.overflow) {
    for (int s = 0; s < slices; ++s) {
      const int base = offs[s], cnt = offs[s + 1] - offs[s];
      for (int i = tid; i < cnt; i += kT) sh.buf[base + i] = atomic_take_u64(pub + static_cast<int64_t>(s) * cap + i);
    }
  }
  __syncthreads();
  return true;
}

__device__ void init_shared(Shared& sh, int mode) {
  if (threadIdx.x == 0) {
    sh.count = 0;
    sh.ntrans = 0;
    sh.overflow = 0;
    sh.tau_x = (mode == kModeDense) ? INFINITY : -FLT_MAX;
    *reinterpret_cast<unsigned*>(&sh.wg_max_x) = ordered_f32(-FLT_MAX);
  }
  __syncthreads();
}

__device__ __forceinline__ float filter_offset(const Params& p) {
  // scaled-logit offset below the running max that can still be in the support
  if (p.min_p > 0.f) return __logf(p.min_p) - 1e-3f;
  return -kDeltaTopP;
}

__device__ __forceinline__ int slices_clamped(int s, int64_t vocab) { return s; }

// kPath: kPathRaw scans only rows eligible for the raw-logit top-k filter,
// kPathExact only the others (or every row when the launcher runs the exact
// kernel alone).  With the raw kernel alone (hint), an ineligible row is
// handed to the exact fallback unscanned.
enum Path : int { kPathRaw = 0, kPathExact = 1 };
constexpr int kWaveMaxRowK = kWave;  // top-k rows the one-wave kernel takes (k <= 64)
enum Hint : int { kHintBoth = 0, kHintRawOnly = 1, kHintExactOnly = 2 };

template <typename Tag, bool kVec, int kPath>
__device__ void process_row(Shared& sh, const typename Tag::storage* row, int64_t vocab, const Params& p,
                            const XForm& f, int slices, int slice, uint64_t* pub, uint64_t* pubs, uint32_t* cnt,
                            RowRec* rec, int32_t* sidx, float* sp, int cand_tok, float cand_x, uint32_t* list_cnt,
                            int32_t* list, int32_t list_id, bool raw_ok, int hint, int wave) {
  const int mode = row_mode(p, vocab);
  const bool raw = mode == kModeTopK && raw_ok;
  if constexpr (kPath == kPathRaw) {
    if (wave && raw && p.top_k <= kWaveMaxRowK) return;  // scanned by the one-wave kernel
    if (!raw) {
      if (hint == kHintRawOnly && !wave && slice == 0 && threadIdx.x == 0) {
        RowRec rr{};
        rr.flags = kFlagOverflow | kFlagUnscanned;
        rr.why = kWhyHint;
        *rec = rr;
        list[atomic_add_u32(list_cnt, 1u)] = list_id;
      }
      return;
    }
  } else {
    if (raw && hint != kHintExactOnly) return;
  }
  init_shared(sh, mode);
  const int k = mode == kModeTopK ? max(p.top_k, 1) : 0;
  const float off_s = mode == kModeFilter ? filter_offset(p) : 0.f;
  const SliceRange r = slice_range(vocab, slices, slice, Tag::kPerVec);
  ScanOut st;
  if constexpr (kPath == kPathRaw) {
    const ScanOut o = scan_topk_raw<Tag, kVec>(sh, row, r.v_begin, r.v_end, f, k);
    st = finish_topk_raw(sh, o, f, k, p.temperature);
  } else {
    const ScanOut o = scan_range<Tag, kVec>(sh, row, r.v_begin, r.v_end, f, p.temperature, mode, k, off_s);
    st = finish_slice(sh, o, mode, k, p.temperature, off_s);
  }
  if (slices > 1) {
    if (!merge_slices(sh, st, mode, slices, slice, pub, pubs, cnt, p.temperature)) return;
    if (!sh.overflow) {
      // re-apply the row-wide thresholds to the merged candidates
      if (mode == kModeTopK && sh.count > k) compact_ge(sh, select_kth_s(sh, sh.count, k));
      else if (mode == kModeFilter) compact_ge(sh, ordered_f32(st.mx / p.temperature + off_s));
    }
  }
  finalize_row(sh, st, p, mode, vocab, rec, sidx, sp, cand_tok, cand_x, list_cnt, list, list_id);
}

template <typename CandT>
__device__ __forceinline__ int64_t cand_at(const Args& a, int64_t b, int j) {
  return static_cast<int64_t>(static_cast<const CandT*>(a.cand)[b * a.csb + static_cast<int64_t>(a.cfirst + j) * a.csk]);
}

// (rep: the request's repetition penalty, already loaded)
__device__ __forceinline__ XForm target_xform(const Args& a, int64_t b, int64_t row, float rep) {
  XForm f;
  f.pbits = a.pbits ? a.pbits + b * a.pws : nullptr;
  f.prank = a.pbits ? a.prank + b * a.pws : nullptr;
  f.padd = (a.pbits && a.padd) ? a.padd + b * a.pas : nullptr;
  f.rep = rep;
  f.quirk = a.quirk;
  f.mbits = a.mask ? a.mask + (a.mask_per_request ? b : row) * a.mrs : nullptr;
  return f;
}

__device__ __forceinline__ XForm target_xform(const Args& a, int64_t b, int64_t row) {
  return target_xform(a, b, row, a.prep ? a.prep[b] : 1.f);
}

// --------------------------------------------------------------- kernels ---

// The drafted token a target row checks and its logit after penalties and
// mask (tok < 0: none), for the workgroup scans and the exact fallback.
template <typename TagT, typename CandT>
__device__ __forceinline__ CandRec cand_rec_of(const Args& a, int64_t row) {
  const int64_t b = row / a.width;
  const int j = static_cast<int>(row % a.width);
  CandRec cr{NAN, -1};
  if (a.cand && j < a.width - 1) {
    const int64_t c = cand_at<CandT>(a, b, j);
    if (c >= 0 && c < a.vocab) {
      using S = typename TagT::storage;
      const S* rp = static_cast<const S*>(a.logits) + row * a.lrs;
      cr.tok = static_cast<int>(c);
      cr.x = transform1(target_xform(a, b, row), to_f32<S>(rp[c]), c);
    }
  }
  return cr;
}

// The drafted token a target row checks (-1: none), for the wavefront path,
// which takes its probability from the row's support by index.
template <typename CandT>
__device__ __forceinline__ int cand_tok_of(const Args& a, int64_t row) {
  const int64_t b = row / a.width;
  const int j = static_cast<int>(row % a.width);
  if (!a.cand || j >= a.width - 1) return -1;
  const int64_t c = cand_at<CandT>(a, b, j);
  return (c >= 0 && c < a.vocab) ? static_cast<int>(c) : -1;
}

// ------------------------------------------- one wavefront per target row ---
//
// Top-k rows eligible for the raw-logit filter with k <= kWaveMaxK are
// scanned by a single wavefront each, so a row needs no workgroup barrier
// and one row's selection and finalisation overlap other rows' streaming on
// the same CU.  Every row of a batch is resident at once (2048 rows = 8
// waves per CU).  Each lane keeps kWaveDepth 16-byte loads in flight (16 KB
// per wave); the candidate buffer, its radix-select histogram and the
// support sort live in the wave's own LDS.  Semantics are those of the
// workgroup raw path: raw values are filtered against a threshold that only
// rises, candidates are transformed when the buffer is compacted and at the
// end, and the support is cut by top-k (ties to the lowest index), top-p and
// min-p.

constexpr int kWaveBuf = 2304;                    // candidate entries per wave (19 KB of LDS with the histogram: at most 8 waves per CU, so 2048 rows spread evenly)
constexpr int kWaveDepth = 16;                    // 16-byte loads in flight per lane
constexpr int kWaveMaxK = kWaveMaxRowK;           // prologue threshold from 64 lane maxima
constexpr int kWaveTrigger = kWaveBuf - kWave * 8;  // room for one step of appends

struct WaveShared {
  uint64_t buf[kWaveBuf];
  uint32_t hist[256];
};

// Orders the wave's own LDS accesses (no instruction on gfx950: a wave's LDS
// operations complete in order); keeps the compiler from moving them across.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int wave_excl_scan(int v, int* total) {
  const int inc = static_cast<int>(wave_incl_scan_u32(static_cast<uint32_t>(v)));
  *total = lane_read(inc, kWave - 1);
  return inc - v;
}

// Inclusive prefix sum over the wave: at step o (1, 2, ..., 32) lane i adds
// the value of lane i - o (i >= o), the additions of the shuffle scan in its
// order, so the sums are bit-identical to it.  Lane i - o is found without LDS
// permutes: within a row of 16 a row rotation by o, and for the first o lanes
// of a row the same rotation read from the row before (the lane swaps bring
// row 0 to row 1 and row 2 to row 3, and row 1 to row 2 by way of rows 0 and 3).
__device__ __forceinline__ float wave_incl_scan_f(float v) {
  const int lane = threadIdx.x & (kWave - 1);
  const int j = lane & 15;
  const bool row2 = (lane >> 4) == 2;
  auto prev_row = [&](uint32_t x) __attribute__((always_inline)) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);  // r[0]: even row, r[1]: odd row
    const auto s = __builtin_amdgcn_permlane32_swap(r[1], r[1], false, false);  // s[0]: the lower half's
    return row2 ? s[0] : r[0];
  };
  // (every cross-lane operation runs in all lanes; selects pick the results)
  auto step = [&](auto ror_tag, int o) __attribute__((always_inline)) {
    const uint32_t u = dpp_mov<decltype(ror_tag)::value>(__float_as_uint(v));  // lane (j - o) mod 16 of the row
    const uint32_t pu = prev_row(u);
    const float t = __uint_as_float(j >= o ? u : pu);
    v = lane >= o ? v + t : v;
  };
  step(std::integral_constant<int, 0x121>{}, 1);  // row_ror:1
  step(std::integral_constant<int, 0x122>{}, 2);  // row_ror:2
  step(std::integral_constant<int, 0x124>{}, 4);  // row_ror:4
  step(std::integral_constant<int, 0x128>{}, 8);  // row_ror:8
  const float t16 = __uint_as_float(prev_row(__float_as_uint(v)));
  v = lane >= 16 ? v + t16 : v;
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = lane >= 32 ? v + __uint_as_float(r[0]) : v;
  return v;
}

// Append the raw elements x[0..P) >= tau (all lanes call; count is uniform):
// one ballot per element position and the lane's rank among the passing
// lanes from mbcnt, so no cross-lane permute sits on the path.
template <int P>
__device__ __forceinline__ void wave_append(WaveShared& ws, int& count, const float* x, float tau, int64_t e0) {
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const bool pass = x[q] >= tau;
    const uint64_t m = __ballot(pass);
    if (m) {
      if (pass) {
        const int pos = count + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
        if (pos < kWaveBuf) ws.buf[pos] = cand_key(x[q], static_cast<int>(e0 + q));
      }
      count += __popcll(m);
    }
  }
}

__device__ __forceinline__ void wave_transform(WaveShared& ws, const XForm& f, int from, int to) {
  if (!(f.pbits || f.mbits)) return;
  to = min(to, kWaveBuf);
  for (int i = from + static_cast<int>(threadIdx.x & (kWave - 1)); i < to; i += kWave) {
    const uint64_t key = ws.buf[i];
    const int idx = key_idx(key);
    ws.buf[i] = cand_key(transform1(f, key_s(key), idx), idx);
  }
  wave_sync();
}

// k-th largest (ties counted) of the R*64 ordered values o held R per lane,
// 1 <= k <= R*64, decided bit by bit from the top: the largest t with at
// least k values >= t.  Bits below low_bit are left 0 (the result is then the
// k-th largest's high bits, a value no larger).  Counting uses ballots only.
template <int R>
__device__ __forceinline__ uint32_t wave_kth_ballot(const uint32_t (&o)[R], int k, int low_bit) {
  uint32_t t = 0;
  for (int bit = 31; bit >= low_bit; --bit) {
    const uint32_t cand = t | (1u << bit);
    int c = 0;
#pragma unroll
    for (int j = 0; j < R; ++j) c += __popcll(__ballot(o[j] >= cand));
    if (c >= k) t = cand;
  }
  return t;
}

// Ordered-s of the k-th largest of buf[0..n) (ties counted), 1 <= k <= n:
// up to 256 entries by ballot counting in registers, more by an MSB-first
// radix select over 8-bit digits.  With bf16_keys every key holds a bf16
// value, whose ordered form has its low 16 bits all 0 (positive) or all 1
// (negative): the top 16 bits then fix the whole value.  With prefix16 (fp32
// keys) only the k-th largest's top 16 bits are found, returned with the low
// 16 bits cleared: an ordered value no larger than the k-th largest.
__device__ uint32_t wave_select_kth(WaveShared& ws, int n, int k, bool bf16_keys = false, bool prefix16 = false) {
  const int lane = threadIdx.x & (kWave - 1);
  if (n <= 4 * kWave) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = j * kWave + lane;
      o[j] = i < n ? static_cast<uint32_t>(ws.buf[i] >> 32) : 0u;  // 0: below every value (a NaN's form)
    }
    uint32_t t = wave_kth_ballot<4>(o, k, (bf16_keys || prefix16) ? 16 : 0);
    if (bf16_keys) t |= (t & 0x80000000u) ? 0u : 0xFFFFu;
    return t;
  }
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
  const int passes = (bf16_keys || prefix16) ? 2 : 4;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = 24 - 8 * pass;
#pragma unroll
    for (int j = 0; j < 4; ++j) ws.hist[4 * lane + j] = 0;
    wave_sync();
    for (int i = lane; i < n; i += kWave) {
      const uint32_t h = static_cast<uint32_t>(ws.buf[i] >> 32);
      if ((h & pmask) == prefix) atomicAdd(&ws.hist[(h >> shift) & 255u], 1u);
    }
    wave_sync();
    uint32_t c[4], local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = ws.hist[4 * lane + j];
      local += c[j];
    }
    // lanes above own larger digits: the counts of the lanes past this one
    const uint32_t pre = wave_incl_scan_u32(local);
    uint32_t above = lane_read(pre, kWave - 1) - pre;
    int sel = -1, sel_above = 0;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      if (above < static_cast<uint32_t>(remaining) && above + c[j] >= static_cast<uint32_t>(remaining)) {
        sel = 4 * lane + j;
        sel_above = static_cast<int>(above);
      }
      above += c[j];
    }
    const uint64_t who = __ballot(sel >= 0);
    const int src = __ffsll(static_cast<long long>(who)) - 1;
    const uint32_t d = static_cast<uint32_t>(lane_read(sel, src));
    remaining -= lane_read(sel_above, src);
    prefix |= d << shift;
    pmask |= 255u << shift;
    wave_sync();
  }
  if (bf16_keys) prefix |= (prefix & 0x80000000u) ? 0u : 0xFFFFu;
  return prefix;
}

// Keep entries of buf[0..n) whose ordered-s is >= thr (stable); returns the count.
__device__ int wave_compact_ge(WaveShared& ws, int n, uint32_t thr) {
  const int lane = threadIdx.x & (kWave - 1);
  int out = 0;
  for (int r = 0; r < n; r += kWave) {
    const int i = r + lane;
    const uint64_t key = i < n ? ws.buf[i] : 0;
    const bool keep = i < n && static_cast<uint32_t>(key >> 32) >= thr;
    const uint64_t m = __ballot(keep);
    const int off = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                              __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
    wave_sync();
    if (keep) ws.buf[out + off] = key;  // out + off <= i: never ahead of an unread entry
    out += __popcll(m);
  }
  wave_sync();
  return out;
}

// Sort buf[0..n) descending (bitonic, zero-padded to a power of two).
__device__ void wave_sort_desc(WaveShared& ws, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  int np = 2;
  while (np < n) np <<= 1;
  for (int i = n + lane; i < np; i += kWave) ws.buf[i] = 0;
  wave_sync();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = lane; i < np / 2; i += kWave) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = ws.buf[lo], b = ws.buf[hi];
        if ((a < b) == desc) {
          ws.buf[lo] = b;
          ws.buf[hi] = a;
        }
      }
      wave_sync();
    }
  }
}

// Transform what is pending, then keep the k largest (within the rounding
// margin); returns the new raw threshold (or -FLT_MAX if n <= k).  kth (if
// given) gets, when n > k, the k-th largest value (ties counted) for bf16
// keys and its top 16 bits for other keys: never above the k-th largest.
__device__ __forceinline__ float wave_compact_topk(WaveShared& ws, const XForm& f, int& count, int& ntrans, int k,
                                                  bool bf16_raw, float* kth = nullptr) {
  wave_transform(ws, f, ntrans, count);
  ntrans = count;
  if (count <= k) return -FLT_MAX;
  // penalties change values; the mask only sets -inf (a bf16 value).  Other
  // keys get the k-th largest's top 16 bits (a value no larger): the margin
  // below keeps every candidate of the k largest either way.
  const bool bf16_keys = bf16_raw && !f.pbits;
  const float xk = unordered_f32(wave_select_kth(ws, count, k, bf16_keys, !bf16_keys));
  if (kth) *kth = xk;
  const float thr = x_lower(xk);
  count = wave_compact_ge(ws, count, ordered_f32(thr));
  ntrans = count;
  return thr;
}

// Streams the elements [e_off, e_off + nelem) of a row (rp points at element
// e_off, 16-byte aligned; e_off a multiple of P) and leaves in ws.buf[0..count)
// every element that can be among the row range's k largest transformed
// values: x-domain keys, transformed, compacted to the k largest within the
// rounding margin.  r and q hold the loads of the first two chunks, issued by
// the caller.  raw_max is the range's raw maximum (wave-reduced); kth the
// range's k-th largest transformed value when more than k candidates were
// left (else -inf); ovf gets the Why bits of a range that the buffer could
// not resolve.
template <typename TagT>
__device__ __forceinline__ void wave_scan_candidates(WaveShared& ws, const typename TagT::storage* rp, int64_t nelem,
                                                     int64_t e_off, const XForm& f, int k, uint4 (&r)[kWaveDepth],
                                                     uint4 (&q)[kWaveDepth], int& count, float& raw_max, float& kth,
                                                     int& ovf, const uint32_t* pre_pw = nullptr,
                                                     const uint32_t* pre_mw = nullptr) {
  using S = typename TagT::storage;
  constexpr int P = TagT::kPerVec;
  constexpr bool kBf16 = __is_same(TagT, BF16);
  const int lane = threadIdx.x & (kWave - 1);
  const uint4* vp = reinterpret_cast<const uint4*>(rp);
  const int64_t nfull = nelem / P;
  const int64_t steps = (nfull + kWave - 1) / kWave;
  const int64_t last = nfull - 1;

  float tau = -FLT_MAX;
  if (steps >= kWaveDepth) {
    // Prologue threshold.  Each lane keeps its 4 largest elements of the first
    // chunk among those the transform leaves unchanged (bit clear in the
    // penalty bitmap, set in the mask); the k-th largest of those 256 values
    // (ties counted) is a transformed value of k distinct elements, so it
    // bounds the range's k-th largest from below.  The penalty and mask words
    // are fetched 16 vectors at a time.
    float t0 = -INFINITY, t1 = -INFINITY, t2 = -INFINITY, t3 = -INFINITY;
    constexpr int kHalf = 16;
    static_assert(kWaveDepth % kHalf == 0, "the prologue walks the first chunk in halves of kHalf vectors");
#pragma unroll
    for (int h = 0; h < kWaveDepth / kHalf; ++h) {
      uint32_t pw[kHalf], mw[kHalf];
#pragma unroll
      for (int u = 0; u < kHalf; ++u) {
        pw[u] = 0u;
        mw[u] = ~0u;
      }
      if (pre_pw) {
        // the caller loaded the first chunk's words (e_off 0) ahead of the
        // chunks, word i*64 + l in lane l of pre_*[i]: lane l needs word
        // ((v*64 + l)*P) >> 5 of its vector v, i.e. register v*P/32, lane
        // (v*2P) % 64 + (l*P) >> 5
#pragma unroll
        for (int u = 0; u < kHalf; ++u) {
          constexpr int kRegs = kWaveDepth * 2 * P / kWave;
          static_assert(kRegs >= 1 && kWave % (2 * P) == 0, "staged word layout");
          const int v = h * kHalf + u;
          const int src = (v * 2 * P) % kWave + ((lane * P) >> 5);
          if (f.pbits) pw[u] = __shfl(pre_pw[(v * P) >> 5], src, kWave);
          if (f.mbits) mw[u] = __shfl(pre_mw[(v * P) >> 5], src, kWave);
        }
      } else {
        if (f.pbits) {
#pragma unroll
          for (int u = 0; u < kHalf; ++u)
            pw[u] = f.pbits[(e_off + static_cast<int64_t>((h * kHalf + u) * kWave + lane) * P) >> 5];
        }
        if (f.mbits) {
#pragma unroll
          for (int u = 0; u < kHalf; ++u)
            mw[u] = f.mbits[(e_off + static_cast<int64_t>((h * kHalf + u) * kWave + lane) * P) >> 5];
        }
      }
#pragma unroll
      for (int u = 0; u < kHalf; ++u) {
        float x[P];
        unpack16<TagT>(r[h * kHalf + u], x);
        const int sh = static_cast<int>((e_off + static_cast<int64_t>((h * kHalf + u) * kWave + lane) * P) & 31);
        const uint32_t ok = (~pw[u] & mw[u]) >> sh;
#pragma unroll
        for (int qq = 0; qq < P; ++qq) {
          // branch-free insertion into the sorted top 4 (t0 >= t1 >= t2 >= t3):
          // each new rank is the median of its old value, the one above and v
          const float v = ((ok >> qq) & 1u) ? x[qq] : -INFINITY;
          t3 = __builtin_amdgcn_fmed3f(t2, t3, v);
          t2 = __builtin_amdgcn_fmed3f(t1, t2, v);
          t1 = __builtin_amdgcn_fmed3f(t0, t1, v);
          t0 = fmaxf(t0, v);
        }
      }
    }
    const uint32_t o[4] = {ordered_f32(t0), ordered_f32(t1), ordered_f32(t2), ordered_f32(t3)};
    // top 16 bits of the k-th largest (a value no larger, so still a bound)
    const float tk = unordered_f32(wave_kth_ballot<4>(o, k, 16));
    if (tk > -INFINITY) tau = x_lower(tk);
  }

  count = 0;
  ovf = 0;
  raw_max = -INFINITY;
  int ntrans = 0;
  auto step = [&](float* x, int64_t st) __attribute__((always_inline)) {
    const int64_t idx = st * kWave + lane;
    if (idx >= nfull) {
#pragma unroll
      for (int qq = 0; qq < P; ++qq) x[qq] = -INFINITY;
    }
    float vmax = x[0];
#pragma unroll
    for (int qq = 1; qq < P; ++qq) vmax = fmaxf(vmax, x[qq]);
    raw_max = fmaxf(raw_max, vmax);
    // Appends past the buffer are dropped and counted; the chunk boundary
    // turns that into an overflow (the row is resolved by the exact fallback).
    if (__ballot(vmax >= tau)) wave_append<P>(ws, count, x, tau, e_off + idx * P);
  };
  // Chunks of kWaveDepth steps in two buffers: while one chunk is consumed the
  // next one is in flight.  No load stays in flight across the loop's back
  // edge (a loop-carried register with a pending load makes the compiler
  // drain every load, or copy the register, at each iteration); refills are
  // unconditional (clamped to the last vector past the end) so the buffers
  // need no merge copies.  Between chunks, compact once the buffer holds more
  // than 2k entries, so the threshold follows the running k-th largest.
  const int soft = max(2 * k, 64);
#define LS_WAVE_BOUNDARY()                                                 \
  do {                                                                      \
    if (count > kWaveBuf && !ovf) {                                         \
      ovf = kWhyLost;                                                       \
      tau = INFINITY;                                                       \
    } else if (count > soft && !ovf) {                                      \
      wave_sync();                                                          \
      tau = fmaxf(tau, wave_compact_topk(ws, f, count, ntrans, k, kBf16));  \
      if (count > kWaveTrigger) { ovf = kWhyTies; tau = INFINITY; }         \
    }                                                                       \
  } while (0)
#define LS_WAVE_CONSUME(BUF, S0)                                            \
  do {                                                                      \
    _Pragma("unroll") for (int u = 0; u < kWaveDepth; ++u) {                \
      if ((S0) + u < steps) {                                               \
        float x[P];                                                         \
        unpack16<TagT>(BUF[u], x);                                          \
        step(x, (S0) + u);                                                  \
      }                                                                     \
    }                                                                       \
  } while (0)
// A chunk whose every vector lies inside the range: no bounds checks.
#define LS_WAVE_CONSUME_FULL(BUF, S0)                                       \
  do {                                                                      \
    _Pragma("unroll") for (int u = 0; u < kWaveDepth; ++u) {                \
      float x[P];                                                           \
      unpack16<TagT>(BUF[u], x);                                            \
      float vmax = x[0];                                                    \
      _Pragma("unroll") for (int qq = 1; qq < P; ++qq) vmax = fmaxf(vmax, x[qq]); \
      raw_max = fmaxf(raw_max, vmax);                                       \
      if (__ballot(vmax >= tau))                                            \
        wave_append<P>(ws, count, x, tau, e_off + (((S0) + u) * kWave + lane) * P); \
    }                                                                       \
  } while (0)
#define LS_WAVE_CONSUME_ANY(BUF, S0)                                        \
  do {                                                                      \
    if (((S0) + kWaveDepth) * kWave <= nfull) LS_WAVE_CONSUME_FULL(BUF, S0); \
    else LS_WAVE_CONSUME(BUF, S0);                                          \
  } while (0)
#define LS_WAVE_ISSUE(BUF, S0)                                              \
  do {                                                                      \
    _Pragma("unroll") for (int u = 0; u < kWaveDepth; ++u)                  \
      BUF[u] = load16_stream(vp + min<int64_t>(((S0) + u) * kWave + lane, last)); \
  } while (0)
  LS_WAVE_CONSUME_ANY(r, 0);  // chunk 0 (read by the prologue); chunk 1 is in q
  for (int64_t s0 = kWaveDepth; s0 < steps; s0 += 2 * kWaveDepth) {
    LS_WAVE_ISSUE(r, s0 + kWaveDepth);
    LS_WAVE_BOUNDARY();
    LS_WAVE_CONSUME_ANY(q, s0);
    if (s0 + kWaveDepth >= steps) break;
    LS_WAVE_ISSUE(q, s0 + 2 * kWaveDepth);
    LS_WAVE_BOUNDARY();
    LS_WAVE_CONSUME_ANY(r, s0 + kWaveDepth);
  }
#undef LS_WAVE_ISSUE
#undef LS_WAVE_CONSUME_ANY
#undef LS_WAVE_CONSUME_FULL
#undef LS_WAVE_CONSUME
#undef LS_WAVE_BOUNDARY
  // Elements past the last whole vector (range length not a multiple of P).
  {
    const int64_t v = nfull * P + lane;
    float x[1] = {v < nelem ? to_f32<S>(rp[v]) : -INFINITY};
    raw_max = fmaxf(raw_max, x[0]);
    if (__ballot(x[0] >= tau)) wave_append<1>(ws, count, x, tau, e_off + v);
  }
  raw_max = wave_max(raw_max);
  if (count > kWaveBuf) ovf |= kWhyLost;
  wave_sync();
  kth = -INFINITY;
  if (!ovf) wave_compact_topk(ws, f, count, ntrans, k, kBf16, &kth);
}

// Support of a top-k row from its candidates ws.buf[0..count) (x-domain,
// transformed, at least the k largest within the margin): re-key by x / T,
// sort, cut by top-k (ties to the lowest index), top-p and min-p, and write
// the row record and support.  A row the candidates cannot resolve (ovf) is
// listed for the exact fallback with its raw maximum.  Returns the record
// (the same in every lane).
// With cand_by_match the drafted token's probability is that of its support
// entry, found by index (0 when it is not in the support): the support holds
// exactly the keys at or above the record's last key, so this is the value
// the cand_x form gives, without reading the token's logit.
__device__ RowRec wave_finalize_topk(WaveShared& ws, int count, const Params& p, float raw_max, int ovf, RowRec* rec,
                                   int32_t* sidx, float* sp, int cand_tok, float cand_x, uint32_t* list_cnt,
                                   int32_t* list, int32_t list_id, bool cand_by_match = false) {
  const int lane = threadIdx.x & (kWave - 1);
  const int k = p.top_k;
  const float t = p.temperature;
  int n = count;
  if (!ovf && n <= kWave) {
    // One key per lane, kept in registers: the arithmetic (and its order) of
    // the general path below, without its LDS round trips.
    uint64_t key = 0;
    if (lane < n) {
      const uint64_t k0 = ws.buf[lane];
      key = cand_key(key_s(k0) / t, key_idx(k0));
    }
    key = wave_bitonic_sort<false>(key);
    wave_sync();
    ws.buf[lane] = key;  // the sorted support keys stay in LDS for the caller
    wave_sync();
    if (n > k) n = k;
    const float m = n > 0 ? key_s(lane_read(key, 0)) : -INFINITY;
    const float e = lane < n ? __expf(key_s(key) - m) : 0.f;
    const float z1 = wave_sum(e);
    const float pi = lane < n ? e / z1 : 0.f;
    int n_f = n;
    if (p.top_p < 1.0f && n > 0) {
      const float inc = wave_incl_scan_f(pi);
      const uint64_t hit = __ballot(lane < n && 0.f + inc - pi > p.top_p);
      if (hit) n_f = __ffsll(static_cast<long long>(hit)) - 1;
    }
    if (p.min_p > 0.f && n_f > 0) {
      const float pp = wave_sum(lane < n_f ? pi : 0.f);
      const float thr = (lane_read(pi, 0) / pp) * p.min_p;
      const uint64_t hit = __ballot(lane < n_f && pi / pp < thr);
      if (hit) n_f = __ffsll(static_cast<long long>(hit)) - 1;
    }
    const float zf = wave_sum(lane < n_f ? e : 0.f);
    if (lane < n_f) {
      sidx[lane] = key_idx(key);
      sp[lane] = e / zf;
    }
    RowRec rr{};
    rr.m = m;
    rr.z = zf;
    rr.n = n_f;
    rr.flags = 0;
    rr.why = 0;
    const uint64_t lastk = lane_read(key, n_f > 0 ? n_f - 1 : 0);
    rr.last = n_f > 0 ? lastk : ~uint64_t(0);
    rr.p_cand = 0.f;
    if (cand_tok >= 0 && cand_by_match) {
      const uint64_t hit = __ballot(lane < n_f && key_idx(key) == cand_tok);
      const float pv = lane_read(e / zf, hit ? __ffsll(static_cast<long long>(hit)) - 1 : 0);
      rr.p_cand = hit ? pv : 0.f;
    } else if (cand_tok >= 0) {
      const float sc = cand_x / t;
      const uint64_t kc = cand_key(sc, cand_tok);
      rr.p_cand = (kc >= rr.last && rr.n != 0) ? __expf(sc - rr.m) / rr.z : 0.f;
    }
    if (lane == 0) *rec = rr;
    return rr;
  }
  float m = 0.f, zf = 0.f;
  int n_f = 0;
  if (!ovf) {
    for (int i = lane; i < n; i += kWave) {
      const uint64_t key = ws.buf[i];
      ws.buf[i] = cand_key(key_s(key) / t, key_idx(key));
    }
    wave_sync();
    if (n <= kWave) {
      // one key per lane: bitonic sort across the wave, descending
      const uint64_t key = wave_bitonic_sort<false>(lane < n ? ws.buf[lane] : 0);
      wave_sync();
      ws.buf[lane] = key;
      wave_sync();
    } else {
      wave_sort_desc(ws, n);
    }
    if (n > k) n = k;
    m = n > 0 ? key_s(ws.buf[0]) : -INFINITY;
    float acc = 0.f;
    for (int i = lane; i < n; i += kWave) acc += __expf(key_s(ws.buf[i]) - m);
    const float z1 = wave_sum(acc);
    n_f = n;
    if (p.top_p < 1.0f && n > 0) {
      // first entry whose exclusive prefix of probabilities exceeds top_p
      float carry = 0.f;
      for (int r0 = 0; r0 < n; r0 += kWave) {
        const int i = r0 + lane;
        const float pi = i < n ? __expf(key_s(ws.buf[i]) - m) / z1 : 0.f;
        const float inc = wave_incl_scan_f(pi);
        const uint64_t hit = __ballot(i < n && carry + inc - pi > p.top_p);
        if (hit) {
          n_f = r0 + __ffsll(static_cast<long long>(hit)) - 1;
          break;
        }
        carry += lane_read(inc, kWave - 1);
      }
    }
    if (p.min_p > 0.f && n_f > 0) {
      float a2 = 0.f;
      for (int i = lane; i < n_f; i += kWave) a2 += __expf(key_s(ws.buf[i]) - m) / z1;
      const float pp = wave_sum(a2);
      const float thr = ((__expf(key_s(ws.buf[0]) - m) / z1) / pp) * p.min_p;
      int cut = n_f;
      for (int r0 = 0; r0 < n_f; r0 += kWave) {
        const int i = r0 + lane;
        const uint64_t hit = __ballot(i < n_f && (__expf(key_s(ws.buf[i]) - m) / z1) / pp < thr);
        if (hit) {
          cut = r0 + __ffsll(static_cast<long long>(hit)) - 1;
          break;
        }
      }
      n_f = cut;
    }
    if (n_f > kCap) ovf |= kWhyCap;
    float a3 = 0.f;
    for (int i = lane; i < n_f; i += kWave) a3 += __expf(key_s(ws.buf[i]) - m);
    zf = wave_sum(a3);
  }
  RowRec rr{};
  if (ovf) {
    rr.m = raw_max;  // x-domain upper bound of the row maximum
    rr.z = 0.f;
    rr.flags = kFlagOverflow;
    rr.why = ovf;
    if (lane == 0) {
      *rec = rr;
      list[atomic_add_u32(list_cnt, 1u)] = list_id;
    }
    return rr;
  }
  for (int i = lane; i < n_f; i += kWave) {
    const uint64_t kk = ws.buf[i];
    sidx[i] = key_idx(kk);
    sp[i] = __expf(key_s(kk) - m) / zf;
  }
  rr.m = m;
  rr.z = zf;
  rr.n = n_f;
  rr.flags = 0;
  rr.why = 0;
  rr.last = n_f > 0 ? ws.buf[n_f - 1] : ~uint64_t(0);
  rr.p_cand = 0.f;
  if (cand_tok >= 0 && cand_by_match) {
    float pv = 0.f;
    for (int i = lane; i < n_f; i += kWave) {
      const uint64_t kk = ws.buf[i];
      if (key_idx(kk) == cand_tok) pv = __expf(key_s(kk) - m) / zf;
    }
    rr.p_cand = wave_max(pv);  // at most one entry matches; probabilities are >= 0
  } else if (cand_tok >= 0) {
    const float sc = cand_x / t;
    const uint64_t kc = cand_key(sc, cand_tok);
    rr.p_cand = (kc >= rr.last && rr.n != 0) ? __expf(sc - rr.m) / rr.z : 0.f;
  }
  if (lane == 0) *rec = rr;
  return rr;
}

template <typename TagT, bool kVec, typename CandT, int kPath>
__global__ __launch_bounds__(kT) void target_scan_kernel(Args a) {
  __shared__ Shared sh;
  const int64_t row = blockIdx.x / a.s_t;
  const int slice = blockIdx.x % a.s_t;
  const int64_t b = row / a.width;
  const int j = static_cast<int>(row % a.width);
  Params p{a.temps[b], a.top_ks ? max(a.top_ks[b], 1) : static_cast<int>(a.vocab), a.top_ps ? a.top_ps[b] : 1.f,
           a.min_ps ? a.min_ps[b] : 0.f};
  using S = typename TagT::storage;
  const S* rp = static_cast<const S*>(a.logits) + row * a.lrs;
  const XForm f = target_xform(a, b, row);
  if (a.clear_status && blockIdx.x == 0 && threadIdx.x == 0 && a.status) *a.status = 0;
  const CandRec cr = cand_rec_of<TagT, CandT>(a, row);
  process_row<TagT, kVec, kPath>(sh, rp, a.vocab, p, f, a.s_t, slice, a.pub_t + row * kNBuf,
                                 a.pubs_t + row * a.s_t * 2, a.cnt_t + row, a.rec_t + row,
                                 a.sidx_t + row * kCap, a.sp_t + row * kCap, cr.tok, cr.x, a.list_cnt,
                                 a.list_t, static_cast<int32_t>(row), raw_filter_ok(f, a.pnonpos, b), a.hint, a.wave);
}

// Sampling parameters of request b's draft row (the target's temperature
// when no draft temperature is given; no filter when a value is absent).
__device__ __forceinline__ Params draft_params(const Args& a, int64_t b) {
  Params p;
  p.temperature = a.d_temps ? a.d_temps[b] : a.temps[b];
  p.top_k = a.d_top_ks ? max(a.d_top_ks[b], 1) : static_cast<int>(a.vocab);
  p.top_p = a.d_top_ps ? a.d_top_ps[b] : 1.f;
  p.min_p = a.d_min_ps ? a.d_min_ps[b] : 0.f;
  return p;
}

// The same as scalar loads, all issued at once (an absent tensor reads
// temps[b] in its place).
__device__ __forceinline__ Params draft_params_uniform(const Args& a, int64_t b) {
  const uint32_t* def = reinterpret_cast<const uint32_t*>(a.temps + b);
  const uint32_t t = load_uniform(a.d_temps ? reinterpret_cast<const uint32_t*>(a.d_temps + b) : def);
  const uint32_t k = load_uniform(a.d_top_ks ? reinterpret_cast<const uint32_t*>(a.d_top_ks + b) : def);
  const uint32_t tp = load_uniform(a.d_top_ps ? reinterpret_cast<const uint32_t*>(a.d_top_ps + b) : def);
  const uint32_t mp = load_uniform(a.d_min_ps ? reinterpret_cast<const uint32_t*>(a.d_min_ps + b) : def);
  Params p;
  p.temperature = __uint_as_float(t);
  p.top_k = a.d_top_ks ? max(static_cast<int>(k), 1) : static_cast<int>(a.vocab);
  p.top_p = a.d_top_ps ? __uint_as_float(tp) : 1.f;
  p.min_p = a.d_min_ps ? __uint_as_float(mp) : 0.f;
  return p;
}

// First rejected position of request b (width-1 when every drafted token is
// accepted) and blocking flags, from the target row records.  Called by all
// 64 lanes of one wave (lane j tests position j); every lane gets the result.
template <typename CandT>
__device__ __forceinline__ int accept_length_wave(const Args& a, int64_t b, int* flags) {
  const int g = a.width - 1;
  const int lane = threadIdx.x & (kWave - 1);
  for (int base = 0; base < g; base += kWave) {
    const int j = base + lane;
    bool ok = false;
    int fl = 0;
    if (j < g) {
      const RowRec& r = a.rec_t[b * a.width + j];
      fl = r.flags;
      if (!(fl & kFlagOverflow)) {
        float q;
        if (a.q_mode == 0) {
          q = a.dtp[b * a.dtp_sb + j];
        } else {
          const int64_t c = cand_at<CandT>(a, b, j);
          q = (c >= 0 && c < a.vocab)
                  ? static_cast<const float*>(a.draft)[b * a.dsb + static_cast<int64_t>(j) * a.dsk + c]
                  : 0.f;
        }
        ok = a.uni[b * a.usb + j] * q < r.p_cand;
      }
    }
    const uint64_t fail = __ballot(j < g && !ok);
    if (fail) {
      const int first = __ffsll(static_cast<long long>(fail)) - 1;
      const int ff = lane_read(fl, first);
      *flags = (ff & kFlagOverflow) ? ff : 0;
      return base + first;
    }
  }
  *flags = (a.rec_t[b * a.width + g].flags & kFlagOverflow) ? kFlagOverflow : 0;
  return g;
}

// Wave 0 computes the accepted length into s_len / s_flags (all threads call).
template <typename CandT>
__device__ __forceinline__ void accept_length_block(const Args& a, int64_t b, int* s_len, int* s_flags) {
  if (threadIdx.x < kWave) {
    int fl;
    const int len = accept_length_wave<CandT>(a, b, &fl);
    if (threadIdx.x == 0) {
      *s_len = len;
      *s_flags = fl;
    }
  }
}

template <typename TagD, bool kVec, typename CandT, int kPath>
__global__ __launch_bounds__(kT) void draft_scan_kernel(Args a) {
  __shared__ Shared sh;
  __shared__ int s_len, s_flags;
  const int64_t b = blockIdx.x / a.s_d;
  const int slice = blockIdx.x % a.s_d;
  accept_length_block<CandT>(a, b, &s_len, &s_flags);
  __syncthreads();
  const int len = s_len;
  if (len >= a.width - 1 || s_flags) {
    const bool writer = (kPath == kPathExact) == (a.hint != kHintRawOnly);
    if (writer && slice == 0 && threadIdx.x == 0) {
      RowRec r{};
      r.flags = kFlagSkip;
      a.rec_d[b] = r;
    }
    return;
  }
  const Params p = draft_params(a, b);
  using S = typename TagD::storage;
  if (a.dwave && row_mode(p, a.vocab) == kModeTopK && p.top_k <= kWaveMaxK) return;  // draft_wave_kernel's row
  const S* rp = static_cast<const S*>(a.draft) + b * a.dsb + static_cast<int64_t>(len) * a.dsk;
  XForm f{nullptr, nullptr, nullptr, 1.f, 0, nullptr};
  process_row<TagD, kVec, kPath>(sh, rp, a.vocab, p, f, a.s_d, slice, a.pub_d + b * kNBuf,
                                 a.pubs_d + b * a.s_d * 2, a.cnt_d + b, a.rec_d + b, a.sidx_d + b * kCap,
                                 a.sp_d + b * kCap, -1, NAN, a.list_cnt + 1, a.list_d, static_cast<int32_t>(b), true,
                                 a.hint, 0);
}

// Draft rows: kDraftSlices wavefronts per rejected request each scan one
// slice of the draft row at the rejection position, keep the slice's k
// largest (within the margin) and publish them to caller workspace; the
// resolve kernel gathers the slices, keeps the row's k largest and finalises
// the row.
constexpr int kDraftSlices = 32;                  // most slices per request (a.dslices: this launch's)
// Slices launched per request (at most one per 16 KB chunk of the row):
// fewer, larger slices leave fewer waves to dispatch after the target rows;
// of 16, 18, 20, 24, 28 and 32 per fp32 row at V = 151,936, 20 measured
// fastest.
constexpr int kDraftSlicesUsed = 20;
constexpr int kDraftMinSlices = 16;               // fewest for the wavefront draft path
constexpr int kDraftCap = kNBuf / kDraftSlices;  // published candidates per slice (a hand-off row each request)

// Codes a draft slice publishes in place of its candidate count.
constexpr uint64_t kPubBad = ~uint64_t(0);        // candidates did not fit the hand-off
constexpr uint64_t kPubDefer = ~uint64_t(0) - 1;  // acceptance not known here: resolve takes the row
constexpr uint64_t kPubSkip = ~uint64_t(0) - 2;   // every drafted token accepted: no draft row needed

// Acceptance word of a target row in a fused launch: kAccPublished |
// flags << 32 | bits(p_cand).  The words start at zero (caller-zeroed
// counter workspace) and the resolve kernel returns them to zero.
constexpr uint64_t kAccPublished = uint64_t(1) << 63;

// Polls of a fused draft slice waiting for one target row (each poll sleeps
// about 512 cycles after a load): the wait ends within about a second, and
// the request's draft row then goes to the exact pass in resolve.
constexpr int kPollLimit = 1 << 19;

// Accepted length of request b for a draft slice of the fused launch: the
// first rejection among the drafted positions (width-1: none), waiting only
// for the target rows up to it, so a request that rejects early waits only
// for the rows up to the rejection.  -1: not decided
// here (a row up to the rejection went to the exact fallback, or the wait
// limit passed).  qv / uv: lane j's draft probability and uniform of
// position j (width <= 64, so one position per lane).
// w0: lane k's first read of position k's word (0 past the drafts).
__device__ __forceinline__ int fused_accept_length(const Args& a, int64_t b, float qv, float uv, uint64_t w0) {
  const int g = a.width - 1;
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t* acc = a.acc_t + b * a.width;
  // Positions below j are accepted.  The words of positions j.. are read at
  // once (lane k: position k), so a request whose rows are done is decided in
  // one round trip; while the first undecided position is unpublished only
  // its word is polled, then the rest are read at once again.
  int j = 0;
  bool all = true;
  for (int it = 0; it < kPollLimit; ++it) {
    const bool mine = all ? (lane >= j && lane < g) : lane == j;
    const uint64_t w = mine ? (it == 0 ? w0 : atomic_peek_u64(acc + lane)) : 0;
    const bool pub = (w & kAccPublished) != 0;
    const bool ovf = pub && (static_cast<uint32_t>(w >> 32) & kFlagOverflow);
    const bool rej = pub && !ovf && !(uv * qv < __uint_as_float(static_cast<uint32_t>(w)));
    const uint64_t stop = __ballot(mine && (!pub || ovf || rej));
    if (!stop) {
      if (all) return g;
      if (++j >= g) return g;  // the polled position was accepted
      all = true;
      continue;
    }
    const int k = __ffsll(static_cast<long long>(stop)) - 1;
    if (!lane_read(static_cast<int>(pub), k)) {
      j = k;
      all = false;
      __builtin_amdgcn_s_sleep(8);
      continue;
    }
    return lane_read(static_cast<int>(ovf), k) ? -1 : k;
  }
  return -1;
}

// One draft slice (one wavefront) of request b.  kFused: the slice runs in
// the target launch and takes the accepted length from the published
// acceptance words; otherwise from the final target records.
template <typename TagD, typename CandT, bool kFused>
__device__ __forceinline__ void draft_wave_slice(const Args& a, WaveShared& ws, int64_t b, int slice) {
  using S = typename TagD::storage;
  constexpr int P = TagD::kPerVec;
  const int lane = threadIdx.x;
  const int g = a.width - 1;
  // The drafted tokens' probabilities and uniforms, and the first read of
  // the acceptance words, go out together; the parameters are scalar loads.
  float qv = 0.f, uv = 0.f;
  uint64_t w0 = 0;
  if (kFused && lane < g) {
    w0 = atomic_peek_u64(a.acc_t + b * a.width + lane);
    qv = a.dtp[b * a.dtp_sb + lane];
    uv = a.uni[b * a.usb + lane];
  }
  const Params p = kFused ? draft_params_uniform(a, b) : draft_params(a, b);
  const bool topk = row_mode(p, a.vocab) == kModeTopK;
  if (!(topk && p.top_k <= kWaveMaxK)) {
    // A draft row of another path: the workgroup draft scan takes it, or,
    // when none follows, the exact pass in resolve does.
    if (a.dwave_only && slice == 0 && lane == 0) {
      RowRec rr{};
      rr.flags = kFlagOverflow | kFlagUnscanned;
      rr.why = kWhyHint;
      a.rec_d[b] = rr;
      a.list_d[atomic_add_u32(a.list_cnt + 1, 1u)] = static_cast<int32_t>(b);
    }
    return;
  }
  uint64_t code;  // candidate count, or a kPub code
  int count = 0, ovf = 0;
  float raw_max = -FLT_MAX, kth = -INFINITY;
  const XForm f{nullptr, nullptr, nullptr, 1.f, 0, nullptr};
  int len;
  if constexpr (kFused) {
    len = fused_accept_length(a, b, qv, uv, w0);
  } else {
    int fl;
    len = accept_length_wave<CandT>(a, b, &fl);
    if (len >= g || fl) {
      // the same outcome in every slice: slice 0 writes it
      if (slice == 0 && lane == 0) {
        RowRec rr{};
        rr.flags = kFlagSkip;
        a.rec_d[b] = rr;
      }
      return;
    }
  }
  if (len < 0) {
    code = kPubDefer;
  } else if (len >= g) {
    code = kPubSkip;
  } else {
    const S* row = static_cast<const S*>(a.draft) + b * a.dsb + static_cast<int64_t>(len) * a.dsk;
    const SliceRange sr = slice_range(a.vocab, a.dslices, slice, P);
    const S* rp = row + sr.v_begin;
    const int64_t nelem = sr.v_end - sr.v_begin;
    const uint4* vp = reinterpret_cast<const uint4*>(rp);
    const int64_t last = max<int64_t>(nelem / P - 1, 0);
    uint4 r[kWaveDepth], q[kWaveDepth];
#pragma unroll
    for (int u = 0; u < kWaveDepth; ++u) r[u] = load16_stream(vp + min<int64_t>(u * kWave + lane, last));
#pragma unroll
    for (int u = 0; u < kWaveDepth; ++u) q[u] = load16_stream(vp + min<int64_t>((kWaveDepth + u) * kWave + lane, last));
    // every chunk load is issued before any of them is waited for
    __builtin_amdgcn_sched_barrier(0);
    wave_scan_candidates<TagD>(ws, rp, nelem, sr.v_begin, f, p.top_k, r, q, count, raw_max, kth, ovf);
    code = (ovf || count > kDraftCap) ? kPubBad : static_cast<uint64_t>(count);
  }

  // Publish this slice (plain stores: the resolve kernel, a later launch,
  // merges the slices of the request).
  uint64_t* pub = a.pub_d + b * kNBuf + static_cast<int64_t>(slice) * kDraftCap;
  uint64_t* pubs = a.pubs_d + b * 2 * kDraftSlices;
  if (code < kPubSkip)
    for (int i = lane; i < count; i += kWave) pub[i] = ws.buf[i];
  if (lane == 0) {
    pubs[2 * slice] = code;
    pubs[2 * slice + 1] = (static_cast<uint64_t>(ordered_f32(raw_max)) << 32) | ordered_f32(kth);
  }
}

// Draft slice hand-off state of the resolve workgroup.
struct MergeShared {
  int cnt[kDraftSlices];        // candidates of each slice (0 past the launch's slices)
  float bound;                  // lower bound of the row's k-th largest
  int wave_base[kT / kWave];    // each wave's first slot in the merged list
  int count;                    // merged list length
};

// Draft row of request b from its published slices (every thread of the
// resolve workgroup): eight lanes per slice read its candidates (all at
// once); the k-th largest of the threads' 2 largest candidates (entries of
// the row, so no larger than the row's k-th largest; only its top 16 bits
// are found, which lowers it further) bounds the row's k-th largest from
// below, and the candidates within the rounding margin of that bound (or of
// the slices' own k-th values) are kept.  Wave 0 then keeps the row's k
// largest and writes the row record and support; the record is returned in
// wave 0.
constexpr int kMergeLanes = kT / kDraftSlices;         // threads per slice in the merge
constexpr int kMergePer = kDraftCap / kMergeLanes;     // hand-off entries per thread

// The thread's share of request b's slice hand-offs (entries part + kMergeLanes
// * u of slice tid / kMergeLanes), requested before the acceptance is known:
// the addresses do not depend on it, and entries past a slice's count are
// ignored by the merge.
__device__ __forceinline__ void draft_merge_prefetch(const Args& a, int64_t b, uint64_t (&v)[kMergePer]) {
  const int sl = threadIdx.x / kMergeLanes, part = threadIdx.x % kMergeLanes;
  const uint64_t* src = a.pub_d + b * kNBuf + static_cast<int64_t>(sl) * kDraftCap + part;
#pragma unroll
  for (int u = 0; u < kMergePer; ++u) v[u] = src[kMergeLanes * u];
}

__device__ __forceinline__ RowRec draft_merge_block(const Args& a, WaveShared& ws, MergeShared& ms, int64_t b,
                                                    const Params& p, float slice_bound, float raw_max,
                                                    const uint64_t (&v)[kMergePer]) {
  constexpr int kLanes = kMergeLanes;
  constexpr int kPer = kMergePer;
  static_assert(kLanes * kDraftSlices == kT && kPer * kLanes == kDraftCap, "merge lane layout");
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int sl = tid / kLanes, part = tid % kLanes;
  const int my_n = (ms.cnt[sl] - part + kLanes - 1) / kLanes;  // entries part + kLanes * t
  float t0 = -INFINITY, t1 = -INFINITY;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const float x = u < my_n ? key_s(v[u]) : -INFINITY;
    t1 = __builtin_amdgcn_fmed3f(t0, t1, x);
    t0 = fmaxf(t0, x);
  }
  ws.buf[2 * tid] = ordered_f32(t0);
  ws.buf[2 * tid + 1] = ordered_f32(t1);
  __syncthreads();
  if (wid == 0) {
    constexpr int kVals = 2 * kT / kWave;
    uint32_t o[kVals];
#pragma unroll
    for (int j = 0; j < kVals; ++j) o[j] = static_cast<uint32_t>(ws.buf[j * kWave + lane]);
    // (-inf values among them give a NaN prefix: no bound from them)
    float lb = unordered_f32(wave_kth_ballot<kVals>(o, p.top_k, 16));
    if (!(lb == lb)) lb = -INFINITY;
    if (lane == 0) ms.bound = lb;
  }
  __syncthreads();
  const float bound = fmaxf(slice_bound, ms.bound);
  const uint32_t keep_from = bound > -INFINITY ? ordered_f32(x_lower(bound)) : 0u;
  int kept = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    kept += __popcll(__ballot(u < my_n && static_cast<uint32_t>(v[u] >> 32) >= keep_from));
  if (lane == 0) ms.wave_base[wid] = kept;
  __syncthreads();
  int base = 0, count = 0;
#pragma unroll
  for (int w = 0; w < kT / kWave; ++w) {
    base += w < wid ? ms.wave_base[w] : 0;
    count += ms.wave_base[w];
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const bool keep = u < my_n && static_cast<uint32_t>(v[u] >> 32) >= keep_from;
    const uint64_t m = __ballot(keep);
    const int pos = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
    if (keep && pos < kWaveBuf) ws.buf[pos] = v[u];
    base += __popcll(m);
  }
  __syncthreads();
  RowRec rr{};
  if (wid == 0) {
    const int ovf = count > kWaveBuf ? kWhyMerge : 0;
    if (!ovf && count > kWave) {
      // more than a register sort holds: keep the k largest first
      const XForm f{nullptr, nullptr, nullptr, 1.f, 0, nullptr};
      int ntrans = count;
      wave_compact_topk(ws, f, count, ntrans, p.top_k, false);
    }
    rr = wave_finalize_topk(ws, count, p, raw_max, ovf, a.rec_d + b, a.sidx_d + b * kCap, a.sp_d + b * kCap, -1,
                            NAN, a.list_cnt + 1, a.list_d, static_cast<int32_t>(b));
  }
  return rr;
}

// Draft slices of a launch that runs after the target fallback.
template <typename TagD, typename CandT>
__global__ __launch_bounds__(kWave, 2) void draft_wave_kernel(Args a) {
  __shared__ WaveShared ws;
  draft_wave_slice<TagD, CandT, false>(a, ws, blockIdx.x / a.dslices, blockIdx.x % a.dslices);
}

// One wavefront per target row that is top-k with k <= kWaveMaxK: stream the
// row, keep its k largest transformed logits (within the margin) and write
// the row record and support.  With a.fuse_draft the grid carries, after the
// B*K target rows, a.dslices draft slices per request; each target row
// then publishes its acceptance word, and the draft slices of a request start
// as soon as the words up to the first rejection are published (workgroups
// are dispatched in order on each XCD, so every target row is resident or
// done before a draft slice of the same XCD waits).
template <typename TagT, typename TagD, typename CandT>
__global__ __launch_bounds__(kWave, 2) void verify_wave_kernel(Args a) {
  __shared__ WaveShared ws;
  using S = typename TagT::storage;
  constexpr int P = TagT::kPerVec;
  const int64_t rows = a.batch * a.width;
  if (a.clear_status && blockIdx.x == 0 && threadIdx.x == 0 && a.status) *a.status = 0;
  if (static_cast<int64_t>(blockIdx.x) >= rows) {
    const int64_t d = blockIdx.x - rows;
    draft_wave_slice<TagD, CandT, true>(a, ws, d / a.dslices, static_cast<int>(d % a.dslices));
    return;
  }
  // Rows in position-major order: the first positions, which decide most
  // requests' acceptance (and so when their draft rows can be scanned), are
  // dispatched first.
  const int64_t row = (blockIdx.x % a.batch) * a.width + blockIdx.x / a.batch;
  const int64_t b = row / a.width;
  const int lane = threadIdx.x;
  const S* rp = static_cast<const S*>(a.logits) + row * a.lrs;
  const uint4* vp = reinterpret_cast<const uint4*>(rp);
  const int64_t last = a.vocab / P - 1;
  // The row's parameters are scalar loads, all issued before the first two
  // chunks are requested: their latency overlaps the chunks', and waiting
  // for them does not wait for the chunks (a row of another path discards
  // the chunks).  An absent tensor reads temps[b] in its place.
  const int j = static_cast<int>(row - b * a.width);
  const bool has_cand = a.cand && j < a.width - 1;
  const uint32_t* w_def = reinterpret_cast<const uint32_t*>(a.temps + b);
  const uint32_t w_temp = load_uniform(w_def);
  const uint32_t w_k = load_uniform(a.top_ks ? reinterpret_cast<const uint32_t*>(a.top_ks + b) : w_def);
  const uint32_t w_p = load_uniform(a.top_ps ? reinterpret_cast<const uint32_t*>(a.top_ps + b) : w_def);
  const uint32_t w_mp = load_uniform(a.min_ps ? reinterpret_cast<const uint32_t*>(a.min_ps + b) : w_def);
  const uint32_t w_rep = load_uniform(a.prep ? reinterpret_cast<const uint32_t*>(a.prep + b) : w_def);
  const uint32_t w_np = load_uniform(a.pnonpos ? reinterpret_cast<const uint32_t*>(a.pnonpos + b) : w_def);
  // (the row's first 16 bytes stand in for an absent drafted token)
  const CandT w_c = load_uniform(has_cand ? static_cast<const CandT*>(a.cand) + b * a.csb +
                                                static_cast<int64_t>(a.cfirst + j) * a.csk
                                          : reinterpret_cast<const CandT*>(rp));
  // The penalty and mask words of the first chunk's elements (what the
  // threshold prologue reads) are loaded ahead of the chunks, so the
  // prologue waits for the first chunk only.
  constexpr int kPreRegs = kWaveDepth * 2 * P / kWave;  // words of the first chunk / 64
  static_assert((kWaveDepth * 2 * P) % kWave == 0, "the first chunk's words fill whole registers");
  const uint32_t* pre_p = a.pbits ? a.pbits + b * a.pws : nullptr;
  const uint32_t* pre_m = a.mask ? a.mask + (a.mask_per_request ? b : row) * a.mrs : nullptr;
  // (an absent bitmap reads the row's first bytes in its place: no branch)
  const uint32_t* pre_pa = pre_p ? pre_p : reinterpret_cast<const uint32_t*>(rp);
  const uint32_t* pre_ma = pre_m ? pre_m : reinterpret_cast<const uint32_t*>(rp);
  uint32_t pre_pw[kPreRegs], pre_mw[kPreRegs];
#pragma unroll
  for (int i = 0; i < kPreRegs; ++i) {
    pre_pw[i] = pre_pa[i * kWave + lane];
    pre_mw[i] = pre_ma[i * kWave + lane];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 r[kWaveDepth], q[kWaveDepth];
#pragma unroll
  for (int u = 0; u < kWaveDepth; ++u) r[u] = load16_stream(vp + min<int64_t>(u * kWave + lane, last));
#pragma unroll
  for (int u = 0; u < kWaveDepth; ++u) q[u] = load16_stream(vp + min<int64_t>((kWaveDepth + u) * kWave + lane, last));
  // every chunk load is issued before any of them is waited for
  __builtin_amdgcn_sched_barrier(0);
  Params p{__uint_as_float(w_temp), a.top_ks ? max(static_cast<int>(w_k), 1) : static_cast<int>(a.vocab),
           a.top_ps ? __uint_as_float(w_p) : 1.f, a.min_ps ? __uint_as_float(w_mp) : 0.f};
  const XForm f = target_xform(a, b, row, a.prep ? __uint_as_float(w_rep) : 1.f);
  const int mode = row_mode(p, a.vocab);
  const bool raw = mode == kModeTopK && (!f.pbits || (f.rep >= 1.0f && (!f.padd || (a.pnonpos && w_np != 0u))));
  uint64_t word = static_cast<uint64_t>(kFlagOverflow) << 32;  // acceptance not known in this launch
  if (!(raw && p.top_k <= kWaveMaxK)) {
    // Rows of the other paths.  In a raw-only launch the rows that are not raw
    // go to the exact fallback unscanned; raw rows with larger k go there too
    // when no workgroup raw scan follows.
    if (((!raw && a.hint == kHintRawOnly) || (raw && a.wave_only)) && lane == 0) {
      RowRec rr{};
      rr.flags = kFlagOverflow | kFlagUnscanned;
      rr.why = kWhyHint;
      a.rec_t[row] = rr;
      a.list_t[atomic_add_u32(a.list_cnt, 1u)] = static_cast<int32_t>(row);
    }
  } else {
    const int64_t c = static_cast<int64_t>(w_c);
    const int cand_tok = (has_cand && c >= 0 && c < a.vocab) ? static_cast<int>(c) : -1;
    int count, ovf;
    float raw_max;
    float kth;
    wave_scan_candidates<TagT>(ws, rp, a.vocab, 0, f, p.top_k, r, q, count, raw_max, kth, ovf, pre_pw, pre_mw);
    const RowRec rr = wave_finalize_topk(ws, count, p, raw_max, ovf, a.rec_t + row, a.sidx_t + row * kCap,
                                         a.sp_t + row * kCap, cand_tok, NAN, a.list_cnt, a.list_t,
                                         static_cast<int32_t>(row), true);
    word = (static_cast<uint64_t>(static_cast<uint32_t>(rr.flags)) << 32) | __float_as_uint(rr.p_cand);
  }
  if (a.fuse_draft && lane == 0) atomic_put_u64(a.acc_t + row, word | kAccPublished);
}

// Exact support of the rows the scan kernels could not resolve from their
// candidate buffers (listed on a worklist); writes their records.
__device__ __noinline__ void write_exact_record(Shared& sh, const Exact& ex, int n_f, RowRec* rec, int32_t* sidx,
                                                float* sp, int cand_tok, float cand_x, float t, int why) {
  const int tid = threadIdx.x;
  const bool sparse = ex.n <= kCap && n_f == ex.n;
  if (sparse)
    for (int i = tid; i < n_f; i += kT) {
      const uint64_t kk = sh.buf[i];
      sidx[i] = key_idx(kk);
      sp[i] = __expf(key_s(kk) - ex.m) / ex.z;
    }
  if (tid == 0) {
    RowRec r{};
    r.m = ex.m;
    r.z = ex.z;
    r.n = sparse ? n_f : -1;
    r.flags = sparse ? 0 : kFlagDense;
    r.why = why | kWhyExact;
    r.last = sparse ? (n_f > 0 ? sh.buf[n_f - 1] : ~uint64_t(0)) : ex.kcut;
    if (cand_tok >= 0) {
      const float sc = cand_x / t;
      const uint64_t kc = cand_key(sc, cand_tok);
      r.p_cand = (kc >= r.last && (r.n != 0 || !sparse)) ? __expf(sc - r.m) / r.z : 0.f;
    }
    *rec = r;
  }
  __syncthreads();
}

// Exact support of one target row the scans could not resolve; rewrites its
// record and support.  Called by the whole workgroup.
template <typename TagT, typename CandT>
__device__ __forceinline__ void target_exact_row(Shared& sh, const Args& a, int64_t row) {
  const int64_t b = row / a.width;
  const RowRec prev = a.rec_t[row];
  Params p{a.temps[b], a.top_ks ? max(a.top_ks[b], 1) : static_cast<int>(a.vocab),
           a.top_ps ? a.top_ps[b] : 1.f, a.min_ps ? a.min_ps[b] : 0.f};
  using S = typename TagT::storage;
  const S* rp = static_cast<const S*>(a.logits) + row * a.lrs;
  const XForm f = target_xform(a, b, row);
  const CandRec cr = cand_rec_of<TagT, CandT>(a, row);
  const int mode = row_mode(p, a.vocab);
  float m_x = prev.m;
  double z = prev.z;
  if (prev.flags & kFlagUnscanned) row_stats<TagT>(sh, rp, a.vocab, f, p.temperature, &m_x, &z);
  const Exact ex = exact_support<TagT>(sh, rp, a.vocab, f, p, mode, m_x, z);
  const int n_f = ex.n <= kCap ? collect<TagT>(sh, rp, a.vocab, f, p.temperature, ex.kcut) : 0;
  write_exact_record(sh, ex, n_f, a.rec_t + row, a.sidx_t + row * kCap, a.sp_t + row * kCap, cr.tok, cr.x,
                     p.temperature, prev.why);
}

template <typename TagT, typename CandT>
__global__ __launch_bounds__(kT) void target_fallback_kernel(Args a) {
  __shared__ Shared sh;
  const uint32_t n = *a.list_cnt;
  for (uint32_t li = blockIdx.x; li < n; li += gridDim.x) target_exact_row<TagT, CandT>(sh, a, a.list_t[li]);
}

// Exact support of request b's draft row at position len (a row the draft
// scans could not resolve); rewrites its record and support.  Called by the
// whole workgroup.
template <typename TagD>
__device__ __forceinline__ void draft_exact_pass(Shared& sh, const Args& a, int64_t b, int len, const RowRec prev) {
  const Params p = draft_params(a, b);
  using S = typename TagD::storage;
  const S* rp = static_cast<const S*>(a.draft) + b * a.dsb + static_cast<int64_t>(len) * a.dsk;
  XForm f{nullptr, nullptr, nullptr, 1.f, 0, nullptr};
  const int mode = row_mode(p, a.vocab);
  float m_x = prev.m;
  double z = prev.z;
  if (prev.flags & kFlagUnscanned) row_stats<TagD>(sh, rp, a.vocab, f, p.temperature, &m_x, &z);
  const Exact ex = exact_support<TagD>(sh, rp, a.vocab, f, p, mode, m_x, z);
  const int n_f = ex.n <= kCap ? collect<TagD>(sh, rp, a.vocab, f, p.temperature, ex.kcut) : 0;
  write_exact_record(sh, ex, n_f, a.rec_d + b, a.sidx_d + b * kCap, a.sp_d + b * kCap, -1, NAN, p.temperature,
                     prev.why);
}

// Probability of token v under the target row record (dense supports only).
template <typename TagT>
__device__ __forceinline__ float target_p_dense(const Args& a, const RowRec& r, int64_t b, int64_t row, int64_t v,
                                                const XForm& f, float t) {
  using S = typename TagT::storage;
  const float s = transform1(f, to_f32<S>(static_cast<const S*>(a.logits)[row * a.lrs + v]), v) / t;
  if (r.last != 0 && cand_key(s, static_cast<int>(v)) < r.last) return 0.f;
  return __expf(s - r.m) / r.z;
}

// Dense fp32 distribution of target row blockIdx.x from its record (one
// workgroup per row): zeros, then the support entries; a dense support (no
// top-k) is evaluated element by element from the logits.  A row the
// fallback could not resolve (capacity) is left zero and flags *status.
template <typename TagT>
__global__ __launch_bounds__(kT) void densify_kernel(Args a, float* out, int64_t ors) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / a.width;
  const int tid = threadIdx.x;
  if (row == 0 && tid == 0) {  // the fallback worklists return to zero (the call's last kernel)
    atomic_take_u32(a.list_cnt);
    atomic_take_u32(a.list_cnt + 1);
  }
  const RowRec r = a.rec_t[row];
  float* op = out + row * ors;
  if (r.n < 0 && !(r.flags & kFlagOverflow)) {
    const XForm f = target_xform(a, b, row);
    const float t = a.temps[b];
    for (int64_t v = tid; v < a.vocab; v += kT) op[v] = target_p_dense<TagT>(a, r, b, row, v, f, t);
    return;
  }
  int64_t done = 0;
  if ((reinterpret_cast<uintptr_t>(op) & 15u) == 0) {
    const int64_t nv = a.vocab / 4;
    float4* o4 = reinterpret_cast<float4*>(op);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t v = tid; v < nv; v += kT) store16_stream(o4 + v, z);
    done = nv * 4;
  }
  for (int64_t v = done + tid; v < a.vocab; v += kT) op[v] = 0.f;
  if (r.flags & kFlagOverflow) {
    if (tid == 0 && a.status) atomicOr(a.status, kFlagOverflow);
    return;
  }
  __syncthreads();  // the zeros are written before the support entries
  for (int i = tid; i < r.n; i += kT) op[a.sidx_t[row * kCap + i]] = a.sp_t[row * kCap + i];
}

template <typename TagD>
__device__ __forceinline__ float draft_q(const Args& a, const RowRec& d, const uint64_t* dsorted, int dn, int64_t b,
                                         int len, int64_t v, float td) {
  if (a.q_mode == 1) return static_cast<const float*>(a.draft)[b * a.dsb + static_cast<int64_t>(len) * a.dsk + v];
  if (d.flags & kFlagDense) {
    using S = typename TagD::storage;
    const float s = to_f32<S>(static_cast<const S*>(a.draft)[b * a.dsb + static_cast<int64_t>(len) * a.dsk + v]) / td;
    if (d.last != 0 && cand_key(s, static_cast<int>(v)) < d.last) return 0.f;
    return __expf(s - d.m) / d.z;
  }
  // binary search in the draft support sorted by ascending index
  int lo = 0, hi = dn - 1;
  const uint32_t want = 0xffffffffu - static_cast<uint32_t>(v);
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const uint32_t kidx = static_cast<uint32_t>(dsorted[mid] >> 32);
    if (kidx == want) return __uint_as_float(static_cast<uint32_t>(dsorted[mid]));
    if (kidx > want) lo = mid + 1;  // larger (0xffffffff - idx) = smaller idx: entries are descending
    else hi = mid - 1;
  }
  return 0.f;
}

// Sort (idx, p) pairs by ascending index into sh.buf[base ..): key =
// (0xffffffff - idx) << 32 | bits(p), sorted descending.
__device__ void load_sorted_by_index(Shared& sh, uint64_t* dst, const int32_t* idx, const float* pv, int n) {
  for (int i = threadIdx.x; i < n; i += kT)
    dst[i] = (static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(idx[i])) << 32) | __float_as_uint(pv[i]);
  __syncthreads();
  // bitonic sort of dst[0..n) (n <= kCap), padded with zeros
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = n + threadIdx.x; i < np; i += kT) dst[i] = 0;
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < np / 2; i += kT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const uint64_t x = dst[lo], y = dst[hi];
        if ((x < y) == desc) { dst[lo] = y; dst[hi] = x; }
      }
      __syncthreads();
    }
  }
}

// Inverse-CDF draw over values val(i), i < n, in order: first i whose running
// sum exceeds u * total (total = full running sum); returns i or -1.
template <typename F>
__device__ int cdf_find(Shared& sh, int n, float u, F val, float total) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  __shared__ int found;
  __shared__ float wsum[kT / kWave];
  if (tid == 0) found = -1;
  const float thr = u * total;
  float carry = 0.f;
  __syncthreads();
  for (int r = 0; r < n; r += kT) {
    const int i = r + tid;
    const float v = i < n ? val(i) : 0.f;
    float inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      float w = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += w;
    }
    if (lane == kWave - 1) wsum[wid] = inc;
    __syncthreads();
    float before = carry;
    for (int w = 0; w < wid; ++w) before += wsum[w];
    if (i < n && before + inc > thr) atomicMin(reinterpret_cast<unsigned*>(&found), static_cast<unsigned>(i));
    float tot = 0.f;
    for (int w = 0; w < kT / kWave; ++w) tot += wsum[w];
    carry += tot;
    __syncthreads();
    const int f = found;
    __syncthreads();  // all threads have read `found` before any thread updates it again
    if (f >= 0) break;
  }
  const int res = found;
  __syncthreads();
  return res;
}

// Accepted length of request b (one wave; width <= 64, so lane j holds
// position j's record): lane 0 writes it and its blocking flag (the overflow
// flag of the record at the accepted length), and the lane holding the
// record at the accepted length writes it to *s_tr.
template <typename CandT>
__device__ __forceinline__ int resolve_accept_wave(const Args& a, int64_t b, int* s_len, int* s_flags,
                                                   RowRec* s_tr, int* flags) {
  const int g = a.width - 1;
  const int lane = threadIdx.x & (kWave - 1);
  RowRec r{};
  float q = 0.f, uv = 0.f;
  if (lane <= g) r = a.rec_t[b * a.width + lane];
  if (lane < g) {
    uv = a.uni[b * a.usb + lane];
    if (a.q_mode == 0) {
      q = a.dtp[b * a.dtp_sb + lane];
    } else {
      const int64_t c = cand_at<CandT>(a, b, lane);
      q = (c >= 0 && c < a.vocab)
              ? static_cast<const float*>(a.draft)[b * a.dsb + static_cast<int64_t>(lane) * a.dsk + c]
              : 0.f;
    }
  }
  const bool ok = lane < g && !(r.flags & kFlagOverflow) && uv * q < r.p_cand;
  const uint64_t fail = __ballot(lane < g && !ok);
  const int len = fail ? __ffsll(static_cast<long long>(fail)) - 1 : g;
  const int fl = lane_read(r.flags, len) & kFlagOverflow;
  if (lane == len) *s_tr = r;
  if (lane == 0) {
    *s_len = len;
    *s_flags = fl;
  }
  *flags = fl;
  return len;
}

// Outputs of request b (len = -1: blocked).  With a cutoff the accepted
// length is capped at cutoff[b] - 1 (at least 0) and a capped request's
// bonus is its drafted token at the cap, which the target accepted
// (cap_correct_len.py:44-52 and accept_sampling.py:151-157,185-186: the bonus is read
// back from the chain's accepted slots).
__device__ __forceinline__ void write_result(const Args& a, int64_t b, int len, int64_t tok) {
  int trim = 0;
  if (a.cutoff && len >= 0) {
    const int cap = max(a.cutoff[b] - 1, 0);
    if (cap < len) {
      trim = len - cap;
      len = cap;
      const int64_t at = b * a.csb + static_cast<int64_t>(a.cfirst + cap) * a.csk;
      tok = a.cand_i64 ? static_cast<const int64_t*>(a.cand)[at]
                       : static_cast<int64_t>(static_cast<const int32_t*>(a.cand)[at]);
    }
  }
  a.accept[b] = len;
  a.bonus[b] = tok;
  if (a.trim) a.trim[b] = trim;
}

// Final draw of request b when the target support at the accepted length and
// the draft support (if a residual is needed) have at most 64 entries each
// (one wave, one entry per lane): q of each target entry by matching indices,
// the residual max(p - q, 0) when a draft token was rejected (p itself below
// the residual-mass floor), then the first entry in index order whose running
// sum exceeds u times the total (vocab - 1 when the total is zero).
// ti / tp: lane i's target support entry (i < tr.n), loaded by the caller.
template <typename TagD>
__device__ __forceinline__ void resolve_wave(const Args& a, int64_t b, int len, bool rejected, const RowRec& tr,
                                             const RowRec& dr, const uint64_t* dkeys, int ti, float tp) {
  const int lane = threadIdx.x & (kWave - 1);
  const int n = tr.n;
  const float u = a.funi[b];
  float val = tp;
  if (rejected) {
    float q = 0.f;
    if (a.q_mode == 1) {
      if (lane < n) q = static_cast<const float*>(a.draft)[b * a.dsb + static_cast<int64_t>(len) * a.dsk + ti];
    } else {
      const int dn = dr.n;
      int di = -1;
      float dp = 0.f;
      if (lane < dn) {
        if (dkeys) {
          // the support keys the merge left in LDS (x / T, descending), with
          // the probabilities it wrote recomputed the same way
          const uint64_t kk = dkeys[lane];
          di = key_idx(kk);
          dp = __expf(key_s(kk) - dr.m) / dr.z;
        } else {
          di = a.sidx_d[b * kCap + lane];
          dp = a.sp_d[b * kCap + lane];
        }
      }
      for (int j = 0; j < dn; ++j) {
        const int dj = __builtin_amdgcn_readlane(di, j);
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dp), j));
        if (dj == ti) q = pj;
      }
    }
    const float res = lane < n ? fmaxf(tp - q, 0.f) : 0.f;
    // single-q acceptance falls back to p below 1e-8 (accept_sampling.py:332-340);
    // dense-q chain sampling always uses the residual (reject_sampling.py:101-121)
    if (a.q_mode == 1 || wave_sum(res) > 1e-8f) val = res;
  }
  // entries in ascending index order (bitonic sort across the wave)
  const uint64_t key = wave_bitonic_sort<true>(
      lane < n ? (static_cast<uint64_t>(static_cast<uint32_t>(ti)) << 32) | __float_as_uint(val) : ~uint64_t(0));
  const float v = lane < n ? __uint_as_float(static_cast<uint32_t>(key)) : 0.f;
  const float inc = wave_incl_scan_f(v);
  const float total = lane_read(inc, kWave - 1);
  const uint64_t hit = __ballot(lane < n && inc > u * total);
  const int idx = static_cast<int>(key >> 32);
  const int first = hit ? __ffsll(static_cast<long long>(hit)) - 1 : 0;
  const int at = lane_read(idx, first);
  if (lane == 0) write_result(a, b, len, (total > 0.f && hit) ? at : a.vocab - 1);
}

// Wave 0 of the resolve kernel, after the accepted length and the draft
// row's merge (merged: its record, or null when no merge ran): blocked
// requests, and the final draw when both supports are small.  Returns true
// when the request is finished (outputs written); the workgroup path takes
// the rest.
template <typename TagD>
__device__ __forceinline__ bool resolve_finish(const Args& a, const WaveShared& ws, int64_t b, int len, int fl,
                                               const RowRec& tr, const RowRec* merged, int ti, float tp) {
  const int lane = threadIdx.x & (kWave - 1);
  const bool rejected = len < a.width - 1;
  RowRec dr{};
  const uint64_t* dkeys = nullptr;
  if (rejected && a.q_mode == 0 && !fl && !(tr.flags & kFlagOverflow)) {
    if (merged) {
      dr = *merged;
      dkeys = ws.buf;
    } else {
      dr = a.rec_d[b];
    }
    if (dr.flags & kFlagOverflow) return false;  // the exact pass
  } else if (rejected && a.q_mode == 0) {
    dr = a.rec_d[b];
  }
  const bool blocked = fl || (tr.flags & kFlagOverflow) ||
                       (rejected && a.q_mode == 0 && (dr.flags & (kFlagOverflow | kFlagSkip)));
  if (blocked) {
    if (lane == 0) {
      write_result(a, b, -1, -1);
      if (a.status) atomicOr(a.status, kFlagOverflow);
    }
    return true;
  }
  if (!(tr.n >= 0 && tr.n <= kWave &&
        (!rejected || a.q_mode == 1 || (!(dr.flags & kFlagDense) && dr.n <= kWave))))
    return false;
  resolve_wave<TagD>(a, b, len, rejected, tr, dr, dkeys, ti, tp);
  return true;
}

template <typename TagT, typename TagD, typename CandT>
__global__ __launch_bounds__(kT) void resolve_kernel(Args a) {
  __shared__ Shared sh;
  __shared__ WaveShared ws;
  __shared__ MergeShared ms;
  __shared__ int s_len, s_flags, s_merge, s_done;
  __shared__ float s_sbound, s_rawmax;
  __shared__ RowRec s_tr;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int g = a.width - 1;
  // scalar loads, requested first
  const Params dpar = draft_params_uniform(a, b);
  const float u_final = load_uniform(a.funi + b);
  if (tid == 0 && b == 0) {
    atomic_take_u32(a.list_cnt);
    atomic_take_u32(a.list_cnt + 1);
  }
  if (a.fuse_draft && tid < a.width) atomic_take_u64(a.acc_t + b * a.width + tid);
  if (a.p_cand_out)
    for (int j = tid; j < g; j += kT) a.p_cand_out[b * g + j] = a.rec_t[b * a.width + j].p_cand;
  // The slices' hand-offs, requested first (see draft_merge_prefetch).
  uint64_t pre[kMergePer];
  if (a.q_mode == 0 && a.dwave) draft_merge_prefetch(a, b, pre);
  // Wave 0: the accepted length, and whether the draft row at the rejection
  // is merged from wavefront slices (1), listed bad by a slice (2), or not;
  // the target support at the accepted length is requested meanwhile.
  int ti = 0;
  float tp = 0.f;
  int64_t tried = -1;  // the target row given an exact pass here
  for (;;) {
    if (tid < kWave) {
      const int lane = tid;
      const int ns = a.dslices;
      uint64_t c = 0, mw = 0;  // the slices' codes do not depend on the acceptance: requested first
      if (a.q_mode == 0 && a.dwave && lane < ns) {
        const uint64_t* pubs = a.pubs_d + b * 2 * kDraftSlices;
        c = pubs[2 * lane];
        mw = pubs[2 * lane + 1];
      }
      int fl;
      const int len = resolve_accept_wave<CandT>(a, b, &s_len, &s_flags, &s_tr, &fl);
      wave_sync();
      const RowRec tr = s_tr;
      if (lane < tr.n) {
        const int64_t trow = b * a.width + len;
        ti = a.sidx_t[trow * kCap + lane];
        tp = a.sp_t[trow * kCap + lane];
      }
      int merge = 0;
      if (len < g && a.q_mode == 0 && !fl && !(tr.flags & kFlagOverflow) && a.dwave) {
        const Params& pd = dpar;
        if (row_mode(pd, a.vocab) == kModeTopK && pd.top_k <= kWaveMaxK) {
          if (__ballot(lane < ns && c >= kPubSkip && c != kPubBad)) {
            // a slice could not decide the acceptance: the exact pass, unscanned
            if (lane == 0) {
              RowRec rr{};
              rr.flags = kFlagOverflow | kFlagUnscanned;
              rr.why = kWhyDefer;
              a.rec_d[b] = rr;
            }
          } else {
            merge = __ballot(lane < ns && c == kPubBad) ? 2 : 1;
            if (lane < kDraftSlices) ms.cnt[lane] = (lane < ns && c != kPubBad) ? static_cast<int>(c) : 0;
            const float rmx = wave_max(lane < ns ? unordered_f32(static_cast<uint32_t>(mw >> 32)) : -FLT_MAX);
            const float sb = wave_max(lane < ns ? unordered_f32(static_cast<uint32_t>(mw)) : -INFINITY);
            if (lane == 0) {
              s_rawmax = rmx;
              s_sbound = sb;
            }
          }
        }
      }
      if (lane == 0) s_merge = merge;
    }
    __syncthreads();
    // Without a fallback launch, the target row at the accepted length that
    // the scans could not resolve gets its exact pass here and the acceptance
    // is walked again (rows past the first rejection are never needed).
    if (!(a.inline_fb && s_flags)) break;
    const int64_t trow = b * a.width + s_len;
    if (trow == tried) break;  // still unresolved (capacity): the request is blocked
    tried = trow;
    target_exact_row<TagT, CandT>(sh, a, trow);
    __syncthreads();
  }
  RowRec dm{};  // the merged draft record (wave 0)
  const int merge = s_merge;
  if (merge == 1) {
    dm = draft_merge_block(a, ws, ms, b, dpar, s_sbound, s_rawmax, pre);
  } else if (merge == 2 && tid < kWave) {
    dm = wave_finalize_topk(ws, 0, dpar, s_rawmax, kWhyMerge, a.rec_d + b, a.sidx_d + b * kCap,
                            a.sp_d + b * kCap, -1, NAN, a.list_cnt + 1, a.list_d, static_cast<int32_t>(b));
  }
  if (tid < kWave) {
    const bool done = resolve_finish<TagD>(a, ws, b, s_len, s_flags, s_tr, merge ? &dm : nullptr, ti, tp);
    if (tid == 0) s_done = done ? 1 : 0;
  }
  __syncthreads();
  if (s_done) return;
  // Workgroup path: large or dense supports and rows for the exact pass.
  const int len = s_len;
  const int64_t trow = b * a.width + len;
  const RowRec tr = s_tr;
  const bool rejected = len < g;
  RowRec dr{};
  if (rejected && a.q_mode == 0) {
    dr = a.rec_d[b];
    if ((dr.flags & kFlagOverflow) && !s_flags && !(tr.flags & kFlagOverflow)) {
      // a draft row the scans left to the exact pass
      draft_exact_pass<TagD>(sh, a, b, len, dr);
      dr = a.rec_d[b];
    }
  }
  const bool blocked = s_flags || (tr.flags & kFlagOverflow) ||
                       (rejected && a.q_mode == 0 && (dr.flags & (kFlagOverflow | kFlagSkip)));
  if (blocked) {
    if (tid == 0) {
      write_result(a, b, -1, -1);
      if (a.status) atomicOr(a.status, kFlagOverflow);
    }
    return;
  }
  const float td = dpar.temperature;
  // Draft support sorted by index (sparse q rows only) in the upper LDS half.
  uint64_t* dsorted = sh.buf + 2048;
  int dn = 0;
  if (rejected && a.q_mode == 0 && !(dr.flags & kFlagDense)) {
    dn = dr.n;
    load_sorted_by_index(sh, dsorted, a.sidx_d + b * kCap, a.sp_d + b * kCap, dn);
  }
  const float u = u_final;
  int tok;
  if (tr.n >= 0) {
    // Sparse target support, sorted by index into the lower LDS half.
    const int n = tr.n;
    load_sorted_by_index(sh, sh.buf, a.sidx_t + trow * kCap, a.sp_t + trow * kCap, n);
    // residual of entry i (target probability p_i minus q at its index)
    auto pval = [&](int i) { return __uint_as_float(static_cast<uint32_t>(sh.buf[i])); };
    auto tidx = [&](int i) { return static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(sh.buf[i] >> 32)); };
    bool use_res = false;
    if (rejected) {
      float acc = 0.f;
      for (int i = tid; i < n; i += kT) acc += fmaxf(pval(i) - draft_q<TagD>(a, dr, dsorted, dn, b, len, tidx(i), td), 0.f);
      const float mass = block_sum(sh, acc);
      // single-q acceptance falls back to p below 1e-8 (accept_sampling.py:332-340);
      // dense-q chain sampling always uses the residual (reject_sampling.py:101-121)
      use_res = a.q_mode == 1 || mass > 1e-8f;
    }
    auto val = [&](int i) {
      const float pi = pval(i);
      return use_res ? fmaxf(pi - draft_q<TagD>(a, dr, dsorted, dn, b, len, tidx(i), td), 0.f) : pi;
    };
    float acc = 0.f;
    for (int i = tid; i < n; i += kT) acc += val(i);
    const float total = block_sum(sh, acc);
    const int hit = total > 0.f ? cdf_find(sh, n, u, val, total) : -1;
    tok = hit >= 0 ? static_cast<int>(tidx(hit)) : static_cast<int>(a.vocab - 1);
  } else {
    // Dense target support: stream the row (and the q source) twice.
    const XForm f = target_xform(a, b, trow);
    const float t = a.temps[b];
    bool use_res = false;
    if (rejected) {
      float acc = 0.f;
      for (int64_t v = tid; v < a.vocab; v += kT)
        acc += fmaxf(target_p_dense<TagT>(a, tr, b, trow, v, f, t) - draft_q<TagD>(a, dr, dsorted, dn, b, len, v, td), 0.f);
      use_res = a.q_mode == 1 || block_sum(sh, acc) > 1e-8f;
    }
    auto val = [&](int64_t v) {
      const float pv = target_p_dense<TagT>(a, tr, b, trow, v, f, t);
      return use_res ? fmaxf(pv - draft_q<TagD>(a, dr, dsorted, dn, b, len, v, td), 0.f) : pv;
    };
    float acc = 0.f;
    for (int64_t v = tid; v < a.vocab; v += kT) acc += val(v);
    const float total = block_sum(sh, acc);
    const int hit = total > 0.f ? cdf_find(sh, static_cast<int>(a.vocab), u, [&](int i) { return val(i); }, total) : -1;
    tok = hit >= 0 ? hit : static_cast<int>(a.vocab - 1);
  }
  if (tid == 0) write_result(a, b, len, tok);
}

inline uint64_t up256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

int pick_slices(int64_t rows, int64_t vocab, int want_wgs, int max_top_k) {
  int64_t s = (want_wgs + rows - 1) / rows;
  int64_t by_len = vocab / 8192;
  if (by_len < 1) by_len = 1;
  if (s > by_len) s = by_len;
  if (s > 16) s = 16;
  // every slice must be able to hand over top-k plus ties
  const int64_t need = static_cast<int64_t>(max_top_k) + 64;
  while (s > 1 && kNBuf / s < need) --s;
  return static_cast<int>(s < 1 ? 1 : s);
}

struct Layout {
  uint64_t counters, scratch;
  uint64_t off_rec_t, off_sidx_t, off_sp_t, off_rec_d, off_sidx_d, off_sp_d, off_pub_t, off_pubs_t, off_pub_d,
      off_pubs_d, off_list_t, off_list_d;
  int s_t, s_d;
};

Layout layout(int64_t batch, int width, int64_t vocab, int max_top_k) {
  Layout l{};
  const int64_t rows = batch * width;
  l.s_t = pick_slices(rows, vocab, 2048, max_top_k);
  l.s_d = pick_slices(batch, vocab, 1024, max_top_k);
  l.counters = up256(4 * rows) + up256(4 * batch) + 256 + up256(8 * rows);
  uint64_t o = 0;
  l.off_rec_t = o; o += up256(sizeof(RowRec) * rows);
  l.off_sidx_t = o; o += up256(4ull * rows * kCap);
  l.off_sp_t = o; o += up256(4ull * rows * kCap);
  l.off_rec_d = o; o += up256(sizeof(RowRec) * batch);
  l.off_sidx_d = o; o += up256(4ull * batch * kCap);
  l.off_sp_d = o; o += up256(4ull * batch * kCap);
  l.off_pub_t = o; o += l.s_t > 1 ? up256(8ull * rows * kNBuf) : 0;
  l.off_pubs_t = o; o += up256(16ull * rows * l.s_t);
  l.off_pub_d = o; o += up256(8ull * batch * kNBuf);  // workgroup and wavefront slice hand-off
  l.off_pubs_d = o; o += up256(16ull * batch * (l.s_d > kDraftSlices ? l.s_d : kDraftSlices));
  l.off_list_t = o; o += up256(4ull * rows);
  l.off_list_d = o; o += up256(4ull * batch);
  l.scratch = o;
  return l;
}

}  // namespace
}  // namespace ls

extern "C" int ls_verify_sample_workspace(int64_t batch, int32_t width, int64_t vocab, int32_t max_top_k,
                                          uint64_t* counter_bytes, uint64_t* scratch_bytes) {
  LS_CHECK(batch > 0 && width >= 2 && vocab > 0 && counter_bytes && scratch_bytes, LS_ERR_SHAPE,
           "ls_verify_sample_workspace: bad sizes");
  const int mk = (max_top_k <= 0 || max_top_k > ls::rs::kCap) ? ls::rs::kCap : max_top_k;
  const ls::Layout l = ls::layout(batch, width, vocab, mk);
  *counter_bytes = l.counters;
  *scratch_bytes = l.scratch;
  return LS_OK;
}

extern "C" int ls_verify_sample(const ls_verify_sample_args* in, void* counters, uint64_t counter_bytes, void* scratch,
                                uint64_t scratch_bytes, void* stream) {
  using namespace ls;
  LS_CHECK(in, LS_ERR_VALUE, "ls_verify_sample: null args");
  const ls_verify_sample_args& x = *in;
  LS_CHECK(x.batch > 0 && x.width >= 2 && x.width <= 64 && x.vocab > 0 && x.vocab < (int64_t(1) << 31),
           LS_ERR_SHAPE, "ls_verify_sample: need batch > 0, 2 <= width <= 64, 0 < vocab < 2^31");
  LS_CHECK(x.logits_row_stride >= x.vocab, LS_ERR_SHAPE, "ls_verify_sample: logits row stride < vocab");
  LS_CHECK(x.cand_first_col == 0 || x.cand_first_col == 1, LS_ERR_VALUE, "ls_verify_sample: cand_first_col");
  LS_CHECK(x.logits && x.candidates && x.temperatures && x.uniforms && x.final_uniforms && x.accept_lens && x.bonus,
           LS_ERR_VALUE, "ls_verify_sample: null required pointer");
  LS_CHECK(x.q_mode == 0 || x.q_mode == 1, LS_ERR_VALUE, "ls_verify_sample: q_mode must be 0 or 1");
  LS_CHECK(x.scan_hint >= 0 && x.scan_hint <= 2, LS_ERR_VALUE, "ls_verify_sample: scan_hint must be 0, 1 or 2");
  LS_CHECK(x.draft, LS_ERR_VALUE, "ls_verify_sample: draft rows required");
  LS_CHECK(x.q_mode == 1 || x.draft_token_probs, LS_ERR_VALUE, "ls_verify_sample: q_mode 0 needs draft_token_probs");
  LS_CHECK(x.q_mode == 0 || x.draft_dtype == LS_F32, LS_ERR_DTYPE, "ls_verify_sample: dense q must be fp32");
  LS_CHECK(!x.pen_bits || x.pen_rank, LS_ERR_VALUE, "ls_verify_sample: penalty bitmap without ranks");
  LS_CHECK(!x.pen_bits || x.pen_words_stride >= (x.vocab + 31) / 32, LS_ERR_SHAPE,
           "ls_verify_sample: penalty bitmap stride too small");
  LS_CHECK(!x.vocab_mask || x.mask_row_stride >= (x.vocab + 31) / 32, LS_ERR_SHAPE,
           "ls_verify_sample: mask must cover the vocabulary ((V+31)/32 words per row)");
  const int mk = (x.max_top_k <= 0 || x.max_top_k > rs::kCap) ? rs::kCap : x.max_top_k;
  const Layout l = layout(x.batch, x.width, x.vocab, mk);
  LS_CHECK(counters && counter_bytes >= l.counters && scratch && scratch_bytes >= l.scratch, LS_ERR_WORKSPACE,
           "ls_verify_sample: needs %llu counter and %llu scratch bytes", (unsigned long long)l.counters,
           (unsigned long long)l.scratch);

  Args a{};
  a.logits = x.logits; a.lrs = x.logits_row_stride;
  a.cand = x.candidates; a.csb = x.cand_stride_b; a.csk = x.cand_stride_k; a.cfirst = x.cand_first_col;
  a.batch = x.batch; a.width = x.width; a.vocab = x.vocab;
  a.temps = x.temperatures; a.top_ks = x.top_ks; a.top_ps = x.top_ps; a.min_ps = x.min_ps;
  a.pbits = x.pen_bits; a.prank = x.pen_rank; a.pws = x.pen_words_stride; a.padd = x.pen_add;
  a.pas = x.pen_add_stride; a.prep = x.pen_repetition; a.quirk = x.pen_verify_quirk;
  a.pnonpos = x.pen_nonpositive;
  a.mask = reinterpret_cast<const uint32_t*>(x.vocab_mask); a.mrs = x.mask_row_stride;
  a.mask_per_request = x.mask_per_request;
  a.q_mode = x.q_mode; a.dtp = x.draft_token_probs; a.dtp_sb = x.dtp_stride_b;
  a.draft = x.draft; a.dsb = x.draft_stride_b; a.dsk = x.draft_stride_k;
  a.d_temps = x.draft_temperatures; a.d_top_ks = x.draft_top_ks; a.d_top_ps = x.draft_top_ps;
  a.d_min_ps = x.draft_min_ps;
  a.uni = x.uniforms; a.usb = x.uniform_stride_b; a.funi = x.final_uniforms;
  a.accept = x.accept_lens; a.bonus = x.bonus; a.p_cand_out = x.p_cand_out; a.status = x.status;
  a.cutoff = x.cutoff_verify_lens; a.trim = x.cap_trim; a.cand_i64 = x.candidates_dtype == LS_I64;
  char* c = static_cast<char*>(counters);
  const int64_t rows = x.batch * x.width;
  a.cnt_t = reinterpret_cast<uint32_t*>(c);
  a.cnt_d = reinterpret_cast<uint32_t*>(c + up256(4 * rows));
  a.list_cnt = reinterpret_cast<uint32_t*>(c + up256(4 * rows) + up256(4 * x.batch));
  a.acc_t = reinterpret_cast<uint64_t*>(c + up256(4 * rows) + up256(4 * x.batch) + 256);
  char* s = static_cast<char*>(scratch);
  a.rec_t = reinterpret_cast<RowRec*>(s + l.off_rec_t);
  a.sidx_t = reinterpret_cast<int32_t*>(s + l.off_sidx_t);
  a.sp_t = reinterpret_cast<float*>(s + l.off_sp_t);
  a.rec_d = reinterpret_cast<RowRec*>(s + l.off_rec_d);
  a.sidx_d = reinterpret_cast<int32_t*>(s + l.off_sidx_d);
  a.sp_d = reinterpret_cast<float*>(s + l.off_sp_d);
  a.pub_t = reinterpret_cast<uint64_t*>(s + l.off_pub_t);
  a.pubs_t = reinterpret_cast<uint64_t*>(s + l.off_pubs_t);
  a.pub_d = reinterpret_cast<uint64_t*>(s + l.off_pub_d);
  a.pubs_d = reinterpret_cast<uint64_t*>(s + l.off_pubs_d);
  a.list_t = reinterpret_cast<int32_t*>(s + l.off_list_t);
  a.list_d = reinterpret_cast<int32_t*>(s + l.off_list_d);
  a.s_t = l.s_t;
  a.s_d = l.s_d;
  a.hint = x.scan_hint;
  a.wave = a.wave_only = a.dwave = a.dwave_only = a.fuse_draft = a.inline_fb = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);

  const dim3 g_t(static_cast<unsigned>(rows * l.s_t)), g_d(static_cast<unsigned>(x.batch * l.s_d)),
      g_r(static_cast<unsigned>(x.batch)), g_f(static_cast<unsigned>(rows < 256 ? rows : 256));
  void* const* ev = x.timing_events;
#define LS_EVENT(i)                                                                              \
  do {                                                                                           \
    if (ev[i] && hipEventRecord(static_cast<hipEvent_t>(ev[i]), st) != hipSuccess)               \
      return fail(LS_ERR_LAUNCH, "ls_verify_sample: hipEventRecord failed");                     \
  } while (0)
  const bool tvec_ok = aligned16(x.logits);
  const bool dvec_ok = aligned16(x.draft);
#define LS_RUN(TT, TD, CT)                                                                                    \
  do {                                                                                                        \
    using TS = typename TT::storage;                                                                          \
    using DS = typename TD::storage;                                                                          \
    const bool tv = tvec_ok && (x.logits_row_stride * sizeof(TS)) % 16 == 0;                                  \
    const bool dv = dvec_ok && (x.draft_stride_b * sizeof(DS)) % 16 == 0 && (x.draft_stride_k * sizeof(DS)) % 16 == 0; \
    a.clear_status = 1; /* the first launch below zeroes the status word */                                   \
    a.wave = (a.hint != kHintExactOnly && tv && x.vocab / TT::kPerVec >= int64_t(kWave) * kWaveDepth) ? 1 : 0; \
    a.wave_only = (a.wave && x.max_top_k > 0 && x.max_top_k <= kWaveMaxRowK) ? 1 : 0;                          \
    a.dslices = static_cast<int>(x.vocab / (TD::kPerVec * kWave * kWaveDepth) < kDraftSlicesUsed              \
                                     ? x.vocab / (TD::kPerVec * kWave * kWaveDepth) : kDraftSlicesUsed);      \
    a.dwave = (x.q_mode == 0 && a.hint != kHintExactOnly && dv && a.dslices >= kDraftMinSlices) ? 1 : 0;      \
    a.dwave_only = (a.dwave && x.max_top_k > 0 && x.max_top_k <= kWaveMaxRowK) ? 1 : 0;                       \
    a.fuse_draft = (a.wave && a.dwave) ? 1 : 0;                                                               \
    /* every row on the wavefront paths and no per-row output: resolve takes the exact passes it needs */     \
    a.inline_fb = (a.fuse_draft && a.wave_only && a.dwave_only && !x.p_cand_out) ? 1 : 0;                     \
    if (ev) LS_EVENT(0);                                                                                      \
    if (a.wave) {                                                                                             \
      const int64_t nwg = rows + (a.fuse_draft ? x.batch * a.dslices : 0);                                    \
      verify_wave_kernel<TT, TD, CT><<<dim3(static_cast<unsigned>(nwg)), kWave, 0, st>>>(a);                 \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    if (a.hint != kHintExactOnly && !a.wave_only) {                                                           \
      if (tv) target_scan_kernel<TT, true, CT, kPathRaw><<<g_t, rs::kT, 0, st>>>(a);                         \
      else target_scan_kernel<TT, false, CT, kPathRaw><<<g_t, rs::kT, 0, st>>>(a);                           \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    if (a.hint != kHintRawOnly) {                                                                             \
      if (tv) target_scan_kernel<TT, true, CT, kPathExact><<<g_t, rs::kT, 0, st>>>(a);                       \
      else target_scan_kernel<TT, false, CT, kPathExact><<<g_t, rs::kT, 0, st>>>(a);                         \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    if (ev) LS_EVENT(1);                                                                                      \
    if (!a.inline_fb) {                                                                                       \
      target_fallback_kernel<TT, CT><<<g_f, rs::kT, 0, st>>>(a);                                              \
      LS_LAUNCH_CHECK();                                                                                      \
    }                                                                                                         \
    if (x.q_mode == 0) {                                                                                      \
      if (a.dwave && !a.fuse_draft) {                                                                         \
        draft_wave_kernel<TD, CT><<<dim3(static_cast<unsigned>(x.batch * a.dslices)), kWave, 0, st>>>(a);     \
        LS_LAUNCH_CHECK();                                                                                    \
      }                                                                                                       \
      if (a.hint != kHintExactOnly && !a.dwave_only) {                                                        \
        if (dv) draft_scan_kernel<TD, true, CT, kPathRaw><<<g_d, rs::kT, 0, st>>>(a);                        \
        else draft_scan_kernel<TD, false, CT, kPathRaw><<<g_d, rs::kT, 0, st>>>(a);                          \
        LS_LAUNCH_CHECK();                                                                                    \
      }                                                                                                       \
      if (a.hint != kHintRawOnly && !a.dwave_only) {                                                          \
        if (dv) draft_scan_kernel<TD, true, CT, kPathExact><<<g_d, rs::kT, 0, st>>>(a);                      \
        else draft_scan_kernel<TD, false, CT, kPathExact><<<g_d, rs::kT, 0, st>>>(a);                        \
        LS_LAUNCH_CHECK();                                                                                    \
      }                                                                                                       \
    }                                                                                                         \
    if (ev) LS_EVENT(2);                                                                                      \
    resolve_kernel<TT, TD, CT><<<g_r, rs::kT, 0, st>>>(a);                                                    \
    LS_LAUNCH_CHECK();                                                                                        \
    if (ev) LS_EVENT(3);                                                                                      \
    return LS_OK;                                                                                             \
  } while (0)
#define LS_CAND(TT, TD)                                             \
  if (x.candidates_dtype == LS_I32) LS_RUN(TT, TD, int32_t);        \
  else if (x.candidates_dtype == LS_I64) LS_RUN(TT, TD, int64_t);   \
  else return fail(LS_ERR_DTYPE, "ls_verify_sample: candidates must be int32 or int64");
#define LS_DRAFT(TT)                                                 \
  if (x.draft_dtype == LS_F32) { LS_CAND(TT, F32) }                  \
  else if (x.draft_dtype == LS_BF16) { LS_CAND(TT, BF16) }           \
  else return fail(LS_ERR_DTYPE, "ls_verify_sample: draft rows must be fp32 or bf16");
  if (x.logits_dtype == LS_BF16) { LS_DRAFT(BF16) }
  if (x.logits_dtype == LS_F32) { LS_DRAFT(F32) }
  if (x.logits_dtype == LS_F16) { LS_DRAFT(F16) }
#undef LS_DRAFT
#undef LS_CAND
#undef LS_RUN
#undef LS_EVENT
  return fail(LS_ERR_DTYPE, "ls_verify_sample: logits must be bf16, fp16 or fp32");
}

extern "C" int ls_target_probs_workspace(int64_t batch, int32_t rows_per_request, int64_t vocab, int32_t max_top_k,
                                         uint64_t* counter_bytes, uint64_t* scratch_bytes) {
  LS_CHECK(batch > 0 && rows_per_request > 0 && vocab > 0 && counter_bytes && scratch_bytes, LS_ERR_SHAPE,
           "ls_target_probs_workspace: bad sizes");
  const int mk = (max_top_k <= 0 || max_top_k > ls::rs::kCap) ? ls::rs::kCap : max_top_k;
  const ls::Layout l = ls::layout(batch, rows_per_request, vocab, mk);
  *counter_bytes = l.counters;
  *scratch_bytes = l.scratch;
  return LS_OK;
}

extern "C" int ls_target_probs(const ls_target_probs_args* in, void* counters, uint64_t counter_bytes, void* scratch,
                               uint64_t scratch_bytes, void* stream) {
  using namespace ls;
  LS_CHECK(in, LS_ERR_VALUE, "ls_target_probs: null args");
  const ls_target_probs_args& x = *in;
  LS_CHECK(x.batch > 0 && x.rows_per_request > 0 && x.vocab > 0 && x.vocab < (int64_t(1) << 31), LS_ERR_SHAPE,
           "ls_target_probs: need batch > 0, rows_per_request > 0, 0 < vocab < 2^31");
  LS_CHECK(x.batch * x.rows_per_request < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_target_probs: too many rows");
  LS_CHECK(x.logits_row_stride >= x.vocab && x.out_row_stride >= x.vocab, LS_ERR_SHAPE,
           "ls_target_probs: row stride < vocab");
  LS_CHECK(x.logits && x.temperatures && x.out, LS_ERR_VALUE, "ls_target_probs: null required pointer");
  LS_CHECK(x.scan_hint >= 0 && x.scan_hint <= 2, LS_ERR_VALUE, "ls_target_probs: scan_hint must be 0, 1 or 2");
  const int mk = (x.max_top_k <= 0 || x.max_top_k > rs::kCap) ? rs::kCap : x.max_top_k;
  const Layout l = layout(x.batch, x.rows_per_request, x.vocab, mk);
  LS_CHECK(counters && counter_bytes >= l.counters && scratch && scratch_bytes >= l.scratch, LS_ERR_WORKSPACE,
           "ls_target_probs: needs %llu counter and %llu scratch bytes", (unsigned long long)l.counters,
           (unsigned long long)l.scratch);

  Args a{};
  a.logits = x.logits; a.lrs = x.logits_row_stride;
  a.batch = x.batch; a.width = x.rows_per_request; a.vocab = x.vocab;
  a.temps = x.temperatures; a.top_ks = x.top_ks; a.top_ps = x.top_ps; a.min_ps = x.min_ps;
  a.status = x.status;
  char* c = static_cast<char*>(counters);
  const int64_t rows = x.batch * x.rows_per_request;
  a.cnt_t = reinterpret_cast<uint32_t*>(c);
  a.cnt_d = reinterpret_cast<uint32_t*>(c + up256(4 * rows));
  a.list_cnt = reinterpret_cast<uint32_t*>(c + up256(4 * rows) + up256(4 * x.batch));
  a.acc_t = reinterpret_cast<uint64_t*>(c + up256(4 * rows) + up256(4 * x.batch) + 256);
  char* s = static_cast<char*>(scratch);
  a.rec_t = reinterpret_cast<RowRec*>(s + l.off_rec_t);
  a.sidx_t = reinterpret_cast<int32_t*>(s + l.off_sidx_t);
  a.sp_t = reinterpret_cast<float*>(s + l.off_sp_t);
  a.rec_d = reinterpret_cast<RowRec*>(s + l.off_rec_d);
  a.sidx_d = reinterpret_cast<int32_t*>(s + l.off_sidx_d);
  a.sp_d = reinterpret_cast<float*>(s + l.off_sp_d);
  a.pub_t = reinterpret_cast<uint64_t*>(s + l.off_pub_t);
  a.pubs_t = reinterpret_cast<uint64_t*>(s + l.off_pubs_t);
  a.pub_d = reinterpret_cast<uint64_t*>(s + l.off_pub_d);
  a.pubs_d = reinterpret_cast<uint64_t*>(s + l.off_pubs_d);
  a.list_t = reinterpret_cast<int32_t*>(s + l.off_list_t);
  a.list_d = reinterpret_cast<int32_t*>(s + l.off_list_d);
  a.s_t = l.s_t;
  a.s_d = l.s_d;
  a.hint = x.scan_hint;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g_t(static_cast<unsigned>(rows * l.s_t)), g_f(static_cast<unsigned>(rows < 256 ? rows : 256)), g_r(static_cast<unsigned>(rows));
  const bool tvec_ok = aligned16(x.logits);
#define LS_TP(TT)                                                                                             \
  do {                                                                                                        \
    using TS = typename TT::storage;                                                                          \
    const bool tv = tvec_ok && (x.logits_row_stride * sizeof(TS)) % 16 == 0;                                  \
    a.clear_status = 1; /* the first launch below zeroes the status word */                                   \
    a.wave = (a.hint != kHintExactOnly && tv && x.vocab / TT::kPerVec >= int64_t(kWave) * kWaveDepth) ? 1 : 0; \
    a.wave_only = (a.wave && x.max_top_k > 0 && x.max_top_k <= kWaveMaxRowK) ? 1 : 0;                          \
    if (a.wave) {                                                                                             \
      verify_wave_kernel<TT, F32, int32_t><<<dim3(static_cast<unsigned>(rows)), kWave, 0, st>>>(a);          \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    if (a.hint != kHintExactOnly && !a.wave_only) {                                                           \
      if (tv) target_scan_kernel<TT, true, int32_t, kPathRaw><<<g_t, rs::kT, 0, st>>>(a);                    \
      else target_scan_kernel<TT, false, int32_t, kPathRaw><<<g_t, rs::kT, 0, st>>>(a);                      \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    if (a.hint != kHintRawOnly) {                                                                             \
      if (tv) target_scan_kernel<TT, true, int32_t, kPathExact><<<g_t, rs::kT, 0, st>>>(a);                  \
      else target_scan_kernel<TT, false, int32_t, kPathExact><<<g_t, rs::kT, 0, st>>>(a);                    \
      LS_LAUNCH_CHECK(); a.clear_status = 0;                                                                  \
    }                                                                                                         \
    target_fallback_kernel<TT, int32_t><<<g_f, rs::kT, 0, st>>>(a);                                           \
    LS_LAUNCH_CHECK();                                                                                        \
    densify_kernel<TT><<<g_r, rs::kT, 0, st>>>(a, x.out, x.out_row_stride);                                   \
    LS_LAUNCH_CHECK();                                                                                        \
    return LS_OK;                                                                                             \
  } while (0)
  if (x.logits_dtype == LS_BF16) LS_TP(BF16);
  if (x.logits_dtype == LS_F32) LS_TP(F32);
  if (x.logits_dtype == LS_F16) LS_TP(F16);
#undef LS_TP
  return fail(LS_ERR_DTYPE, "ls_target_probs: logits must be bf16, fp16 or fp32");
}
