// Dense temperature softmax: out[r, v] = softmax_v(logits[r, v] / T[r / rows_per_request])
// (SRT/speculative/dspark_components/kernels/softmax_temp.py:69-175; the
// torch form :69-86 defines the values, x = logit / T then softmax).
//
// One workgroup of 1024 threads per row.  A 16-bit row of up to 163,840
// entries (kSRU 4-element units per thread) is read once into registers
// (softmax_temp_resident_kernel): the maximum, then the sum of exponentials,
// are taken from the registers, each combined across the workgroup, and the
// probabilities are written from them, so every logit is read from HBM once
// (the row, 297 KiB at 151,936 entries, fills most of a CU's registers: one
// row per CU at a time).  Other rows (fp32, wider vocabularies) take two
// passes (softmax_temp_kernel): the first reads the row and keeps, per
// thread, an online maximum and the sum of exponentials rescaled whenever the
// maximum rises; the second reads the row again.  Either way the output is
// written in 4-element units, one whole 16-byte fp32 vector per lane, so that
// every store instruction covers whole cache lines (two 16-byte stores 32
// bytes apart per lane half-fill each line they touch and cost 1.5x the write
// traffic).  Rows 16-byte aligned (start and stride) move as vectors; others
// element by element.
#include "rowscan.h"

namespace ls {
namespace {

constexpr int kST = 1024;   // threads per row
constexpr int kSTU = 4;     // vectors per thread in flight
constexpr int kSRU = 40;    // 4-element units per thread a register-resident row holds

// Values: p = exp2((l - l_max) * c2) / sum, c2 = log2(e) / T, which is the
// reference's exp(l / T - max(l / T)) / sum up to the rounding of its fp32
// quotient (a relative difference of about |l - l_max| / T * 2^-24 in p).
// The per-thread sums are kept in fp64 (one fp32 partial per vector).

// Four consecutive elements as fp32: one 8-byte load for 16-bit types, one
// 16-byte load for fp32 (p: 4-element aligned).  The second pass reads its
// input in these units so that each lane writes one 16-byte output vector and
// a wavefront's store covers 1 KiB contiguously (whole cache lines).
template <typename Tag>
__device__ __forceinline__ void load4_stream(const typename Tag::storage* p, float* x) {
  if constexpr (sizeof(typename Tag::storage) == 2) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    const uint32_t a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
    uint4 v;
    v.x = a; v.y = b; v.z = 0u; v.w = 0u;
    float t[8];
    unpack16<Tag>(v, t);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = t[e];
  } else {
    unpack16<Tag>(load16_stream(p), x);
  }
}

template <typename Tag, bool kVec>
__global__ __launch_bounds__(kST) void softmax_temp_kernel(const typename Tag::storage* __restrict__ logits,
                                                           int64_t lrs, int64_t vocab,
                                                           const float* __restrict__ temps, int rpr,
                                                           float* __restrict__ out, int64_t ors) {
  using S = typename Tag::storage;
  constexpr int P = Tag::kPerVec;
  __shared__ float wm[kST / kWave];
  __shared__ double wsum[kST / kWave];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const float c2 = 1.4426950408889634f / temps[row / rpr];
  const S* rp = logits + row * lrs;
  float* op = out + row * ors;
  const int64_t nvec = kVec ? vocab / P : 0;
  const uint4* vp = reinterpret_cast<const uint4*>(rp);

  // pass 1: per-thread maximum of l and sum of exp2((l - max) * c2)
  float m = -INFINITY;
  double s = 0.0;
  auto add = [&](const float* x, int n) __attribute__((always_inline)) {
    float vm = x[0];
#pragma unroll
    for (int q = 1; q < P; ++q)
      if (q < n) vm = fmaxf(vm, x[q]);
    if (vm > m) {
      if (m != -INFINITY) s *= static_cast<double>(__builtin_amdgcn_exp2f((m - vm) * c2));
      m = vm;
    }
    if (m != -INFINITY) {
      float vs = 0.f;
#pragma unroll
      for (int q = 0; q < P; ++q)
        if (q < n) vs += __builtin_amdgcn_exp2f((x[q] - m) * c2);
      s += static_cast<double>(vs);
    }
  };
  if constexpr (kVec) {
    for (int64_t v0 = tid; v0 < nvec; v0 += kSTU * kST) {
      uint4 buf[kSTU];  // ordinary loads: the row stays cached for the second pass
#pragma unroll
      for (int u = 0; u < kSTU; ++u) buf[u] = load16(vp + min<int64_t>(v0 + u * kST, nvec - 1));
#pragma unroll
      for (int u = 0; u < kSTU; ++u) {
        if (v0 + u * kST < nvec) {
          float x[P];
          unpack16<Tag>(buf[u], x);
          add(x, P);
        }
      }
    }
  }
  for (int64_t e = nvec * P + tid; e < vocab; e += kST) {
    float x[P];
    x[0] = to_f32<S>(rp[e]);
    add(x, 1);
  }

  // combine the (max, sum) pairs: within the wave, then across waves
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, kWave);
    const double s2 = __shfl_xor(s, o, kWave);
    const float mm = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0 : s * static_cast<double>(__builtin_amdgcn_exp2f((m - mm) * c2))) +
        (m2 == -INFINITY ? 0.0 : s2 * static_cast<double>(__builtin_amdgcn_exp2f((m2 - mm) * c2)));
    m = mm;
  }
  if (lane == 0) {
    wm[wid] = m;
    wsum[wid] = s;
  }
  __syncthreads();
  float rm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kST / kWave; ++w) rm = fmaxf(rm, wm[w]);
  double z = 0.0;
#pragma unroll
  for (int w = 0; w < kST / kWave; ++w)
    if (wm[w] != -INFINITY) z += wsum[w] * static_cast<double>(__builtin_amdgcn_exp2f((wm[w] - rm) * c2));
  const float inv = static_cast<float>(1.0 / z);

  // pass 2: p = exp2((l - max) * c2) / sum, in units of 4 elements
  int64_t tail = 0;
  if constexpr (kVec) {
    constexpr int kU = sizeof(S) == 2 ? 2 * kSTU : kSTU;  // 8-byte loads: twice as many in flight
    const int64_t n4 = vocab / 4;
    // last chunk first: the end of the row was read last in the first pass,
    // so more of it is still in the L2
    const int64_t steps = (n4 + kU * kST - 1) / (kU * kST);
    for (int64_t it = steps - 1; it >= 0; --it) {
      const int64_t v0 = it * (kU * kST) + tid;
      float x[kU][4];
#pragma unroll
      for (int u = 0; u < kU; ++u) load4_stream<Tag>(rp + min<int64_t>(v0 + u * kST, n4 - 1) * 4, x[u]);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t v = v0 + u * kST;
        if (v < n4) {
          float4 y;
          y.x = __builtin_amdgcn_exp2f((x[u][0] - rm) * c2) * inv;
          y.y = __builtin_amdgcn_exp2f((x[u][1] - rm) * c2) * inv;
          y.z = __builtin_amdgcn_exp2f((x[u][2] - rm) * c2) * inv;
          y.w = __builtin_amdgcn_exp2f((x[u][3] - rm) * c2) * inv;
          store16_stream(op + v * 4, y);
        }
      }
    }
    tail = n4 * 4;
  }
  for (int64_t e = tail + tid; e < vocab; e += kST)
    op[e] = __builtin_amdgcn_exp2f((to_f32<S>(rp[e]) - rm) * c2) * inv;
}

// Register-resident form for 16-bit rows with vocab / 4 <= kSRU * kST units
// (start and stride 16-byte aligned): unit v (4 consecutive entries, one
// 8-byte load) lives in thread v % kST, slot v / kST.  The row and output are
// addressed as raw buffers: one offset register per thread and the slot's
// offset as a scalar, so the kSRU loads cost no address registers and all of
// them are in flight at once.  The statistics are softmax_temp_kernel's
// first pass over the registers (the same arithmetic, taken as the loads
// arrive), and the values its second pass.
constexpr int kRawBufferWord3 = 0x00020000;  // gfx9 buffer descriptor word 3: 32-bit data format, untyped access
constexpr int kNonTemporal = 2;              // buffer access cache policy: streaming (nt)

template <typename Tag>
__global__ __launch_bounds__(kST) void softmax_temp_resident_kernel(const typename Tag::storage* __restrict__ logits,
                                                                    int64_t lrs, int64_t vocab,
                                                                    const float* __restrict__ temps, int rpr,
                                                                    float* __restrict__ out, int64_t ors) {
  using S = typename Tag::storage;
  static_assert(sizeof(S) == 2, "16-bit rows only");
  __shared__ float wm[kST / kWave];
  __shared__ double wsum[kST / kWave];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const S* rp = logits + row * lrs;
  float* op = out + row * ors;
  const int n4 = static_cast<int>(vocab / 4);
  const int rem = static_cast<int>(vocab - static_cast<int64_t>(n4) * 4);  // 0..3 trailing entries
  const int nk = tid < n4 ? (n4 - 1 - tid) / kST + 1 : 0;                  // this thread's units
  const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<S*>(rp), 0, static_cast<int>(vocab * sizeof(S)), kRawBufferWord3);
  const __amdgpu_buffer_rsrc_t dst =
      __builtin_amdgcn_make_buffer_rsrc(op, 0, static_cast<int>(vocab * sizeof(float)), kRawBufferWord3);
  const float xt = tid < rem ? to_f32<S>(rp[static_cast<int64_t>(n4) * 4 + tid]) : -INFINITY;
  // Every load of the row is issued before any is used (a slot past the
  // row's end reads zeros, outside the buffer, and is never used).
  uint32_t u[kSRU][2];
#pragma unroll
  for (int k = 0; k < kSRU; ++k) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(src, tid * 8, k * kST * 8, kNonTemporal);
    u[k][0] = v[0];
    u[k][1] = v[1];
  }
  const float c2 = 1.4426950408889634f / temps[row / rpr];
  // The packed units are the only copy of the row kept across the phases:
  // the compiler is told they may change at each phase boundary, so it
  // unpacks them again instead of keeping 4x as many fp32 values live.
  auto repack = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kSRU; ++k) asm volatile("" : "+v"(u[k][0]), "+v"(u[k][1]));
  };
  auto unit = [&](int k, float* x) __attribute__((always_inline)) {
    uint4 w;
    w.x = u[k][0]; w.y = u[k][1]; w.z = 0u; w.w = 0u;
    float t[8];
    unpack16<Tag>(w, t);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = t[e];
  };

  // Per thread, an online maximum and the sum of exp2((l - max) * c2)
  // rescaled whenever the maximum rises (one fp32 partial per unit, fp64
  // across units), taken as the units arrive; then combined across the
  // workgroup.
  float m = -INFINITY;
  double s = 0.0;
  auto add = [&](const float* x, int n) __attribute__((always_inline)) {
    float vm = x[0];
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q < n) vm = fmaxf(vm, x[q]);
    if (vm > m) {
      if (m != -INFINITY) s *= static_cast<double>(__builtin_amdgcn_exp2f((m - vm) * c2));
      m = vm;
    }
    if (m != -INFINITY) {
      float vs = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < n) vs += __builtin_amdgcn_exp2f((x[q] - m) * c2);
      s += static_cast<double>(vs);
    }
  };
#pragma unroll
  for (int k = 0; k < kSRU; ++k) {
    if (k < nk) {
      float x[4];
      unit(k, x);
      add(x, 4);
    }
  }
  if (tid < rem) add(&xt, 1);
  repack();
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, kWave);
    const double s2 = __shfl_xor(s, o, kWave);
    const float mm = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0 : s * static_cast<double>(__builtin_amdgcn_exp2f((m - mm) * c2))) +
        (m2 == -INFINITY ? 0.0 : s2 * static_cast<double>(__builtin_amdgcn_exp2f((m2 - mm) * c2)));
    m = mm;
  }
  if (lane == 0) {
    wm[wid] = m;
    wsum[wid] = s;
  }
  __syncthreads();
  float rm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kST / kWave; ++w) rm = fmaxf(rm, wm[w]);
  double z = 0.0;
#pragma unroll
  for (int w = 0; w < kST / kWave; ++w)
    if (wm[w] != -INFINITY) z += wsum[w] * static_cast<double>(__builtin_amdgcn_exp2f((wm[w] - rm) * c2));
  const float inv = static_cast<float>(1.0 / z);

  // probabilities, one 16-byte fp32 vector per unit
#pragma unroll
  for (int k = 0; k < kSRU; ++k) {
    if (k < nk) {
      float x[4];
      unit(k, x);
      unsigned int y __attribute__((ext_vector_type(4)));
      y[0] = __float_as_uint(__builtin_amdgcn_exp2f((x[0] - rm) * c2) * inv);
      y[1] = __float_as_uint(__builtin_amdgcn_exp2f((x[1] - rm) * c2) * inv);
      y[2] = __float_as_uint(__builtin_amdgcn_exp2f((x[2] - rm) * c2) * inv);
      y[3] = __float_as_uint(__builtin_amdgcn_exp2f((x[3] - rm) * c2) * inv);
      __builtin_amdgcn_raw_buffer_store_b128(y, dst, tid * 16, k * kST * 16, kNonTemporal);
    }
  }
  if (tid < rem) op[static_cast<int64_t>(n4) * 4 + tid] = __builtin_amdgcn_exp2f((xt - rm) * c2) * inv;
}

}  // namespace
}  // namespace ls

extern "C" int ls_softmax_temp(const void* logits, int32_t logits_dtype, int64_t logits_row_stride, int64_t rows,
                               int64_t vocab, const float* temperatures, int32_t rows_per_request, float* out,
                               int64_t out_row_stride, void* stream) {
  using namespace ls;
  LS_CHECK(logits && temperatures && out, LS_ERR_VALUE, "ls_softmax_temp: null pointer");
  LS_CHECK(rows > 0 && vocab > 0 && rows_per_request > 0 && rows % rows_per_request == 0, LS_ERR_SHAPE,
           "ls_softmax_temp: rows must be a positive multiple of rows_per_request");
  LS_CHECK(rows < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_softmax_temp: too many rows");
  LS_CHECK(logits_row_stride >= vocab && out_row_stride >= vocab, LS_ERR_SHAPE, "ls_softmax_temp: row stride < vocab");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
  const bool out_vec = aligned16(out) && (out_row_stride * 4) % 16 == 0;
#define LS_ST(TAG)                                                                                              \
  do {                                                                                                          \
    using S = typename TAG::storage;                                                                            \
    const S* lp = static_cast<const S*>(logits);                                                                \
    const bool vec = out_vec && aligned16(logits) && (logits_row_stride * int64_t(sizeof(S))) % 16 == 0;       \
    if constexpr (sizeof(S) == 2) {                                                                             \
      if (vec && vocab / 4 <= int64_t(kSRU) * kST) {                                                            \
        softmax_temp_resident_kernel<TAG><<<grid, kST, 0, st>>>(lp, logits_row_stride, vocab, temperatures,     \
                                                               rows_per_request, out, out_row_stride);          \
        break;                                                                                                  \
      }                                                                                                         \
    }                                                                                                           \
    if (vec)                                                                                                    \
      softmax_temp_kernel<TAG, true><<<grid, kST, 0, st>>>(lp, logits_row_stride, vocab, temperatures,         \
                                                          rows_per_request, out, out_row_stride);              \
    else                                                                                                        \
      softmax_temp_kernel<TAG, false><<<grid, kST, 0, st>>>(lp, logits_row_stride, vocab, temperatures,        \
                                                           rows_per_request, out, out_row_stride);             \
  } while (0)
  if (logits_dtype == LS_BF16) LS_ST(BF16);
  else if (logits_dtype == LS_F32) LS_ST(F32);
  else if (logits_dtype == LS_F16) LS_ST(F16);
  else return fail(LS_ERR_DTYPE, "ls_softmax_temp: logits must be bf16, fp16 or fp32");
#undef LS_ST
  LS_LAUNCH_CHECK();
  return LS_OK;
}
