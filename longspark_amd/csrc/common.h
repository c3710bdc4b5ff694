// Shared device helpers for the LongSpark verify-and-refresh kernels (gfx950).
//
// Conventions used by every kernel in this library:
//  * wave64: reductions are written for 64-lane wavefronts;
//  * rows are streamed with 16-byte global loads (8 bf16 / 4 fp32 values);
//  * cross-workgroup hand-off uses agent-scope atomics on caller-owned
//    workspace counters that every launch returns to zero (the last arriving
//    workgroup resets them), so no memset precedes a launch and a launch can
//    be captured in a graph.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/longspark_amd.h"

namespace ls {

constexpr int kWave = 64;

// ---------------------------------------------------------------- status ---

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define LS_CHECK(cond, code, ...)                 \
  do {                                            \
    if (!(cond)) return ::ls::fail((code), __VA_ARGS__); \
  } while (0)

#define LS_LAUNCH_CHECK()                                                        \
  do {                                                                           \
    hipError_t e_ = hipGetLastError();                                           \
    if (e_ != hipSuccess)                                                        \
      return ::ls::fail(LS_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e_)); \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------ conversions ---

__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {  // bf16 bit pattern
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
template <>
__device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }

// Storage tags: the element type a kernel template is instantiated for.
struct BF16 { using storage = uint16_t; static constexpr int kPerVec = 8; };
struct F16  { using storage = __half;   static constexpr int kPerVec = 8; };
struct F32  { using storage = float;    static constexpr int kPerVec = 4; };

// Unpack one 16-byte vector into kPerVec fp32 values.
template <typename Tag>
__device__ __forceinline__ void unpack16(const uint4& v, float* out);
template <>
__device__ __forceinline__ void unpack16<BF16>(const uint4& v, float* out) {
  out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x);
  out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
  out[4] = bf16_lo(v.z); out[5] = bf16_hi(v.z);
  out[6] = bf16_lo(v.w); out[7] = bf16_hi(v.w);
}
template <>
__device__ __forceinline__ void unpack16<F16>(const uint4& v, float* out) {
  const __half2* h = reinterpret_cast<const __half2*>(&v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float2 f = __half22float2(h[i]);
    out[2 * i] = f.x; out[2 * i + 1] = f.y;
  }
}
template <>
__device__ __forceinline__ void unpack16<F32>(const uint4& v, float* out) {
  out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
  out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// Streaming read that should not displace reusable lines (logits are read once).
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  uint4 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  r.z = __builtin_nontemporal_load(&q->z);
  r.w = __builtin_nontemporal_load(&q->w);
  return r;
}

// ------------------------------------------------------ wave reductions ---

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// (value, index) argmax with torch semantics: larger value wins, equal values
// keep the lower index.
struct ArgMax {
  float v;
  int i;
};
__device__ __forceinline__ ArgMax argmax_merge(ArgMax a, ArgMax b) {
  bool take_b = (b.v > a.v) || (b.v == a.v && b.i < a.i);
  return take_b ? b : a;
}
__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    ArgMax b;
    b.v = __shfl_xor(a.v, o, kWave);
    b.i = __shfl_xor(a.i, o, kWave);
    a = argmax_merge(a, b);
  }
  return a;
}

// Online-softmax pair (running max m, sum s of exp(x - m)).
struct MaxSum {
  float m;
  float s;
};
__device__ __forceinline__ MaxSum maxsum_merge(MaxSum a, MaxSum b) {
  float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return MaxSum{m, 0.f};
  float s = a.s * __expf(a.m - m) + b.s * __expf(b.m - m);
  return MaxSum{m, s};
}

// -------------------------------------------------- cross-workgroup sync ---

// Agent-scope counter increment with acquire-release ordering.  Returns the
// previous value.  Writes made by the calling thread before the call are
// visible to whichever thread observes the incremented value.
__device__ __forceinline__ uint32_t arrive(uint32_t* counter) {
  __threadfence();
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_counter(uint32_t* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Index of the current 16-byte vector range owned by one slice of a row.
struct SliceRange {
  int64_t v_begin;  // first element (inclusive)
  int64_t v_end;    // last element (exclusive)
};
// Split [0, n) into `parts` ranges whose boundaries are multiples of `gran`.
__host__ __device__ __forceinline__ SliceRange slice_range(int64_t n, int parts, int part, int gran) {
  int64_t units = (n + gran - 1) / gran;
  int64_t per = (units + parts - 1) / parts;
  int64_t b = per * part * gran;
  int64_t e = per * (part + 1) * gran;
  if (b > n) b = n;
  if (e > n) e = n;
  return SliceRange{b, e};
}

}  // namespace ls
