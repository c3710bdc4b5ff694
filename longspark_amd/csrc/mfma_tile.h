// Matrix-core tile helpers shared by the attention-shaped kernels (summary
// refresh, prefill summary initialisation): MFMA operand types, the 16x16x32
// 16-bit products, an LDS-only workgroup barrier and layer-table addressing.
#pragma once

#include "common.h"

namespace ls {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

template <typename Tag>
struct Mma;
template <>
struct Mma<BF16> {
  static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
};
template <>
struct Mma<F16> {
  static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
};

// Four 16-bit values of one column from four consecutive rows of a row-major
// LDS tile, through gfx950's transposing LDS read (ds_read_b64_tr_b16).  In
// each group of 16 lanes, lane L passes the address of the 8 bytes at (row0 +
// L / 4, col0 + 4 * (L % 4)); lane i of the group receives column col0 + i of
// rows row0 .. row0 + 3 (row0 first).  This is the operand layout of a
// 16x16x32 product's A rows read from a [rows][cols] tile, with no transposed
// copy in LDS.
__device__ __forceinline__ uint2 lds_read_col4(const uint16_t* piece) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(piece));
  return __builtin_bit_cast(uint2, r);
}

__device__ __forceinline__ const char* layer_base(const ls_kv_rows& r, int layer) {
  return r.layers ? reinterpret_cast<const char*>(r.layers[layer])
                  : static_cast<const char*>(r.base) + static_cast<int64_t>(layer) * r.stride_layer * 2;
}

// Workgroup barrier that orders LDS only: outstanding global loads stay in
// flight across it (a full __syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16-byte load through a pointer read from memory (layer tables), marked as
// global so the compiler emits a global (not flat) load.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16_global(const char* p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace ls
