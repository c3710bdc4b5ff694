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
#include <type_traits>
#include <hip/hip_fp16.h>
#include <float.h>
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

// fp32 -> storage type with round-to-nearest-even.
template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((b >> 16) | 0x40u);  // quiet NaN
  b += 0x7fffu + ((b >> 16) & 1u);
  return static_cast<uint16_t>(b >> 16);
}
template <>
__device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half(v); }

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
// A read-only value at a wave-uniform address, loaded through the constant
// address space: a scalar load, counted apart from the wave's vector loads,
// so waiting for it never waits for them.  Only for memory that nothing
// writes while the kernel runs.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  uint4 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  r.z = __builtin_nontemporal_load(&q->z);
  r.w = __builtin_nontemporal_load(&q->w);
  return r;
}

// 16-byte non-temporal store (the data is consumed by another kernel).
__device__ __forceinline__ void store16_stream(void* p, const uint4& v) {
  uint4* q = reinterpret_cast<uint4*>(p);
  __builtin_nontemporal_store(v.x, &q->x);
  __builtin_nontemporal_store(v.y, &q->y);
  __builtin_nontemporal_store(v.z, &q->z);
  __builtin_nontemporal_store(v.w, &q->w);
}
__device__ __forceinline__ void store16_stream(void* p, const float4& v) {
  float4* q = reinterpret_cast<float4*>(p);
  __builtin_nontemporal_store(v.x, &q->x);
  __builtin_nontemporal_store(v.y, &q->y);
  __builtin_nontemporal_store(v.z, &q->z);
  __builtin_nontemporal_store(v.w, &q->w);
}

// ------------------------------------------------------ cross-lane ops ---
//
// Lane exchanges on VALU operations (DPP and gfx950's lane swaps) rather than
// LDS permutes (ds_bpermute), so a chain of them waits on no LDS round trip.
// Like the shuffles they replace, they expect every lane of the wave active.

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, 0xf, 0xf, false));
}

// The value lane i ^ kMask holds (kMask = 1, 2, 4, ..., 32): quad permutes for
// 1 and 2; for 4 the quad reverse (i ^ 3) then the half-row mirror (i ^ 7);
// for 8 the half-row mirror then the row mirror (i ^ 15); the lane swaps for
// 16 and 32 (each lane gets both rows of its pair and keeps the other one).
template <int kMask>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (kMask == 1) {
    return dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (kMask == 2) {
    return dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (kMask == 4) {
    return dpp_mov<0x141>(dpp_mov<0x1B>(v));  // quad_perm [3,2,1,0], row_half_mirror
  } else if constexpr (kMask == 8) {
    return dpp_mov<0x140>(dpp_mov<0x141>(v));  // row_half_mirror, row_mirror
  } else if constexpr (kMask == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
  } else {
    static_assert(kMask == 32, "lane_xor: the mask is a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
  }
}
template <int kMask, typename T>
__device__ __forceinline__ T lane_xor_as(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, lane_xor<kMask>(__builtin_bit_cast(uint32_t, v)));
  } else {
    static_assert(sizeof(T) == 8, "lane_xor_as: 4- or 8-byte values");
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = lane_xor<kMask>(static_cast<uint32_t>(b));
    const uint64_t hi = lane_xor<kMask>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

// The value of a lane every lane names alike (a wave-uniform lane index).
template <typename T>
__device__ __forceinline__ T lane_read(T v, int lane) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
  } else {
    static_assert(sizeof(T) == 8, "lane_read: 4- or 8-byte values");
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), lane));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

// Butterfly over the wave pairing lanes i ^ 32, then i ^ 16, ..., i ^ 1, each
// step op(own, partner): the operands and order of the shuffle butterfly, so
// floating-point results are bit-identical to it.  Every lane ends with it.
template <typename T, typename Op>
__device__ __forceinline__ T wave_butterfly(T v, Op op) {
  v = op(v, lane_xor_as<32>(v));
  v = op(v, lane_xor_as<16>(v));
  v = op(v, lane_xor_as<8>(v));
  v = op(v, lane_xor_as<4>(v));
  v = op(v, lane_xor_as<2>(v));
  return op(v, lane_xor_as<1>(v));
}

// Bitonic sort of one 64-bit key per lane across the wave (lane 0 first):
// descending, or ascending with kAscending.
template <bool kAscending, int kSize, int kStride>
__device__ __forceinline__ uint64_t wave_bitonic_steps(uint64_t key) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t o = lane_xor_as<kStride>(key);
  const bool dir = (lane & kSize) == 0 || kSize == kWave;
  const bool lower = (lane & kStride) == 0;
  const uint64_t hi = key > o ? key : o, lo = key < o ? key : o;
  key = (lower == dir) == kAscending ? lo : hi;
  if constexpr (kStride > 1) {
    return wave_bitonic_steps<kAscending, kSize, kStride / 2>(key);
  } else if constexpr (kSize < kWave) {
    return wave_bitonic_steps<kAscending, kSize * 2, kSize>(key);
  } else {
    return key;
  }
}
template <bool kAscending>
__device__ __forceinline__ uint64_t wave_bitonic_sort(uint64_t key) {
  return wave_bitonic_steps<kAscending, 2, 1>(key);
}

// Inclusive prefix sum of 32-bit integers over the wave on DPP steps: row
// shifts by 1, 2, 4 and 8 scan each row of 16 lanes, then the broadcasts of
// lane 15 into rows 1 and 3 and of lane 31 into rows 2 and 3 carry the row
// totals (lanes a step does not write add 0).
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true));
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true));
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true));
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, true));
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, true));
  v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, true));
  return v;
}

// ------------------------------------------------------ wave reductions ---

__device__ __forceinline__ float wave_max(float v) {
  return wave_butterfly(v, [](float x, float y) __attribute__((always_inline)) { return fmaxf(x, y); });
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_butterfly(v, [](float x, float y) __attribute__((always_inline)) { return x + y; });
}
__device__ __forceinline__ int wave_max_i(int v) {
  return wave_butterfly(v, [](int x, int y) __attribute__((always_inline)) { return max(x, y); });
}
__device__ __forceinline__ int wave_sum_i(int v) {
  return wave_butterfly(v, [](int x, int y) __attribute__((always_inline)) { return x + y; });
}

// Reductions over the 4 lanes i, i ^ 16, i ^ 32, i ^ 48 (one column of a
// 16x16 MFMA result, held 4 rows per lane) with gfx950's VALU lane swaps
// instead of LDS permutes: v_permlane16_swap leaves every lane with the
// value of its row pair's even row and of its odd row, v_permlane32_swap
// with the value of its lower-half and its upper-half lane.  The sums pair
// the same operands as the xor-16 then xor-32 butterfly, so they are
// bit-identical to it.
__device__ __forceinline__ float row_pair16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_pair16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float row_pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float col4_sum(float v) { return row_pair32_sum(row_pair16_sum(v)); }
__device__ __forceinline__ float col4_max(float v) { return row_pair32_max(row_pair16_max(v)); }

// Sum over the 64 lanes on VALU cross-lane steps only: DPP quad permutes pair
// lanes i ^ 1 and i ^ 2; once every group of 4 (then 8) holds one value, the
// row half-mirror (row mirror) pairs it with group i ^ 4 (i ^ 8); the lane
// swaps pair rows.  Every lane ends with the total.
__device__ __forceinline__ double wave_sum_d_dpp(double v) {
  auto step_dpp = [](double x, auto ctrl_tag) __attribute__((always_inline)) {
    constexpr int kCtrl = decltype(ctrl_tag)::value;
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(b), kCtrl, 0xf, 0xf, true));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(b >> 32), kCtrl, 0xf, 0xf, true));
    return x + __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
  };
  v = step_dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]: lane i ^ 1
  v = step_dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]: lane i ^ 2
  v = step_dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror: group of 4 i ^ 4
  v = step_dpp(v, std::integral_constant<int, 0x140>{});  // row_mirror: group of 8 i ^ 8
  auto swap = [](double x, bool rows32) __attribute__((always_inline)) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
    const uint32_t lo = static_cast<uint32_t>(b), hi = static_cast<uint32_t>(b >> 32);
    const auto l = rows32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                          : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = rows32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                          : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double a = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(h[0]) << 32) | l[0]));
    const double c = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(h[1]) << 32) | l[1]));
    return a + c;
  };
  v = swap(v, false);
  return swap(v, true);
}

// Inclusive prefix sum over the 64 lanes on DPP steps only: row shifts by 1, 2,
// 4 and 8 scan each row of 16 lanes, then the broadcast of lane 15 into rows 1
// and 3 and of lane 31 into rows 2 and 3 carry the row totals.  Lanes a step
// does not write, and shifts past a row's start, add 0.
__device__ __forceinline__ double wave_incl_scan_d_dpp(double v) {
  auto step = [](double x, auto ctrl_tag, auto row_mask_tag) __attribute__((always_inline)) {
    constexpr int kCtrl = decltype(ctrl_tag)::value, kRows = decltype(row_mask_tag)::value;
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
    const uint32_t lo =
        static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(b), kCtrl, kRows, 0xf, true));
    const uint32_t hi =
        static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), kCtrl, kRows, 0xf, true));
    return x + __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
  };
  using R = std::integral_constant<int, 0xf>;
  v = step(v, std::integral_constant<int, 0x111>{}, R{});  // row_shr:1
  v = step(v, std::integral_constant<int, 0x112>{}, R{});  // row_shr:2
  v = step(v, std::integral_constant<int, 0x114>{}, R{});  // row_shr:4
  v = step(v, std::integral_constant<int, 0x118>{}, R{});  // row_shr:8
  v = step(v, std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});  // row_bcast:15
  return step(v, std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});  // row_bcast:31
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
//
// gfx950 has one L2 per XCD and the L2s are not coherent with each other, so
// a device-scope fence (__threadfence) writes back and invalidates the whole
// L2 of the issuing XCD -- far too expensive to do once per workgroup.  The
// kernels here therefore pass every cross-workgroup value through agent-scope
// atomic read-modify-write operations, which are performed at the single
// coherence point of their address:
//   * producers publish with an atomic RMW (max / add / exchange) and wait for
//     it to complete (its return value) before arriving on a counter;
//   * the last arriver reads the published words with atomic RMWs too
//     (exchange with 0, which also returns them to zero for the next launch).
// Completion of the producer's RMW precedes its counter increment, which
// precedes the last arriver's increment and therefore its reads, so the reads
// observe every published value.  No L2 maintenance is needed.

__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup"); }

__device__ __forceinline__ uint32_t atomic_add_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t atomic_max_u64(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t atomic_take_u64(uint64_t* p) {
  return __hip_atomic_exchange(p, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t atomic_take_u32(uint32_t* p) {
  return __hip_atomic_exchange(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Publish a word with an atomic exchange; the returned old value is kept
// live so that a later wait for outstanding loads covers the exchange.
__device__ __forceinline__ void atomic_put_u64(uint64_t* p, uint64_t v) {
  uint64_t old = __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(old));
}
// Current value of a word published by atomic RMWs: an agent-scope atomic
// load (a coherent load, served from the coherence point and not from a
// stale line of the reader's L2), which leaves the word unchanged.
__device__ __forceinline__ uint64_t atomic_peek_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrive on a counter after this thread's prior atomics completed; returns
// the previous count.  LS_STRICT_ORDER=1 builds the increment as an
// agent-scope acquire-release RMW instead (ordering in the terms of the HIP
// memory model, at the cost of an L2 write-back and invalidate per arrival).
#ifndef LS_STRICT_ORDER
#define LS_STRICT_ORDER 0
#endif
__device__ __forceinline__ uint32_t arrive(uint32_t* counter) {
#if LS_STRICT_ORDER
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
#else
  wait_vm();
  return atomic_add_u32(counter, 1u);
#endif
}

// Order-preserving map of fp32 to uint32 (larger float -> larger integer;
// -0 is canonicalised to +0 so that the two compare equal, as floats do).
__device__ __forceinline__ uint32_t ordered_f32(float x) {
  uint32_t b = __float_as_uint(x + 0.0f);
  return b ^ (static_cast<uint32_t>(static_cast<int32_t>(b) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float unordered_f32(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
  return __uint_as_float(b);
}
// Packed argmax key: larger value wins, then the lower index.  Every real key
// is non-zero, so 0 is the neutral "nothing published" value.
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  return (static_cast<uint64_t>(ordered_f32(v)) << 32) | (0xffffffffu - static_cast<uint32_t>(idx));
}
__device__ __forceinline__ int argmax_key_index(uint64_t key) {
  return static_cast<int>(0xffffffffu - static_cast<uint32_t>(key));
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
