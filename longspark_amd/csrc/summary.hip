// Summary (Global16) state refresh: cached position scores and the
// online-softmax merge of accepted rows, on the matrix cores.
//
// One workgroup = 4 waves = one 64-row tile of the query rows that share a
// KV head (rows r = g * S + s for the g-th query head of the group), for one
// (layer, KV head, request).  The request index varies fastest and the
// block -> unit mapping keeps consecutive units on one XCD, so the requests
// that share a query tile (queries are shared across requests) read it from
// the same L2.
//
//   scores  S[16 x 16] = Q[16 x D] . K^T[D x 16]   v_mfma_f32_16x16x32_{bf16,f16}
//           (bf16/fp16 products are exact in fp32; fp32 accumulation);
//   merge   O[16 x 16] = O * alpha + P[16 x W] . V[W x 16]   v_mfma_f32_16x16x4_f32
//           (P stays fp32: weights are not rounded to 16 bits).
// Reference math: SRT/speculative/global16_raw256_incremental.py:50-166 and
// the kernel forms :172-238 (scores) and :258-392 (merge, including its
// M + log(exp(lse - M) + exp(d - M)) LSE update);
// SRT = vendor/sglang/python/sglang/srt.
#include "common.h"

namespace ls {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kSumThreads = 256;
constexpr int kWaves = 4;
constexpr int kTileRows = 64;
constexpr int kMaxWidth = 32;

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

__device__ __forceinline__ const char* layer_base(const ls_kv_rows& r, int layer) {
  return r.layers ? reinterpret_cast<const char*>(r.layers[layer])
                  : static_cast<const char*>(r.base) + static_cast<int64_t>(layer) * r.stride_layer * 2;
}

__device__ __forceinline__ int64_t row_offset(const ls_kv_rows& r, int64_t b, int w, int64_t loc, int h) {
  return (r.located ? loc * r.stride_loc : b * r.stride_b + w * r.stride_w) + h * r.stride_h;
}

__device__ __forceinline__ int64_t load_loc(const ls_summary_args& a, int64_t b, int w, int64_t off) {
  const int64_t i = a.compact_locs ? off + w : b * a.locs_stride_b + w * a.locs_stride_w;
  return a.locs_dtype == LS_I64 ? static_cast<const int64_t*>(a.locs)[i]
                                : static_cast<int64_t>(static_cast<const int32_t*>(a.locs)[i]);
}

// max / sum over the 16 lanes that hold one row of a 16x16 MFMA result
__device__ __forceinline__ float max16(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Stage rows w < nrows of a key/value source into LDS; rows nrows..wpad-1 are zero.
// Keys keep their 16-bit pattern (pitch kp elements), values are widened to fp32.
template <int D, typename Tag, bool kWiden>
__device__ __forceinline__ void stage_rows(const ls_summary_args& a, const ls_kv_rows& src, int layer, int64_t b,
                                           int kvh, int nrows, int wpad, int64_t loc_off, void* lds, int pitch) {
  constexpr int kVecs = D / 8;
  const char* base = layer_base(src, layer);
  for (int j = threadIdx.x; j < wpad * kVecs; j += kSumThreads) {
    const int w = j / kVecs, c = j - w * kVecs;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (w < nrows) {
      const int64_t loc = src.located ? load_loc(a, b, w, loc_off) : 0;
      v = load16(base + (row_offset(src, b, w, loc, kvh) + c * 8) * 2);
    }
    if constexpr (kWiden) {
      float f[8];
      unpack16<Tag>(v, f);
      float4* dst = reinterpret_cast<float4*>(static_cast<float*>(lds) + w * pitch + c * 8);
      dst[0] = make_float4(f[0], f[1], f[2], f[3]);
      dst[1] = make_float4(f[4], f[5], f[6], f[7]);
    } else {
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(lds) + w * pitch + c * 8) = v;
    }
  }
}

template <int D, int kMode, typename Tag>
__global__ __launch_bounds__(kSumThreads) void summary_kernel(const ls_summary_args a, int tiles, int wpad) {
  constexpr bool kScore = kMode != LS_SUMMARY_MERGE;   // computes scores from queries and keys
  constexpr bool kMerge = kMode != LS_SUMMARY_SCORES;  // folds accepted rows into the state
  constexpr int kKB = D / 32;      // 32-deep steps of the score product
  constexpr int kDB = D / 16;      // 16-column blocks of the state
  constexpr int kKPitch = D + 8;   // 16-bit elements per LDS key row
  constexpr int kVPitch = D + 16;  // fp32 per LDS value row (conflict-free B reads)
  extern __shared__ __align__(16) char smem[];
  __shared__ int s_len;
  __shared__ int64_t s_off;
  uint16_t* kls = reinterpret_cast<uint16_t*>(smem);
  float* vls = reinterpret_cast<float*>(smem + (kScore ? wpad * kKPitch * 2 : 0));
  float* pls = vls + (kMerge ? wpad * kVPitch : 0);
  const int ppitch = wpad + 1;

  // XCD-aware unit: blocks are dispatched round-robin over 8 XCDs; give each
  // XCD a contiguous range of units.
  const unsigned nb = gridDim.x, bi = blockIdx.x;
  const unsigned per = nb / 8, rem = nb % 8, xcd = bi % 8;
  int64_t u = static_cast<int64_t>(xcd) * per + min(xcd, rem) + bi / 8;
  const int64_t b = u % a.batch;
  u /= a.batch;
  const int tile = static_cast<int>(u % tiles);
  u /= tiles;
  const int kvh = static_cast<int>(u % a.kv_heads);
  const int layer = static_cast<int>(u / a.kv_heads);
  const int groups = a.q_heads / a.kv_heads;
  const int nrows_total = groups * a.rows;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int g16 = lane >> 4, c16 = lane & 15;
  const int r0 = tile * kTileRows + wave * 16;

  int len = a.width;
  int64_t loc_off = 0;
  if (kMerge || a.keys.located) {
    if (threadIdx.x < kWave) {
      int64_t off = 0;
      if (a.compact_locs) {
        for (int64_t j = lane; j < b; j += kWave) off += a.accept_lens[j];
#pragma unroll
        for (int o = kWave / 2; o > 0; o >>= 1) off += __shfl_xor(off, o, kWave);
      }
      if (lane == 0) {
        int l = kMerge ? a.accept_lens[b] : a.width;
        s_len = l < 0 ? 0 : (l > a.width ? a.width : l);
        s_off = off;
        if (a.compact_locs && a.accept_offsets && layer == 0 && kvh == 0 && tile == 0)
          a.accept_offsets[b] = static_cast<int32_t>(off);
      }
    }
    __syncthreads();
    len = s_len;
    loc_off = s_off;
    if (kMerge && len <= 0) return;  // uniform over the workgroup
  }
  const int wl = kMerge ? len : a.width;  // key/value rows that take part

  // Rows this lane holds in the MFMA result layout: r0 + 4*g16 + i.
  int head_i[4], srow_i[4];
  bool valid_i[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + 4 * g16 + i;
    valid_i[i] = r < nrows_total;
    const int rr = valid_i[i] ? r : 0;
    head_i[i] = kvh * groups + rr / a.rows;
    srow_i[i] = rr % a.rows;
  }

  // State and prior LSE (issued first: they are the bulk of the traffic).
  f32x4_t acc[kDB];
  float prior[4];
  float* so_row[4];
  float* sl_ptr[4];
  if constexpr (kMerge) {
    const int64_t slot = a.state_slots ? a.state_slots[b] : b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      so_row[i] = a.state_output + slot * a.so_stride_c + layer * a.so_stride_l + head_i[i] * a.so_stride_h +
                  srow_i[i] * a.so_stride_s;
      sl_ptr[i] = a.state_lse + slot * a.sl_stride_c + layer * a.sl_stride_l + head_i[i] * a.sl_stride_h +
                  srow_i[i] * a.sl_stride_s;
      prior[i] = valid_i[i] ? *sl_ptr[i] : 0.f;
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[db][i] = valid_i[i] ? so_row[i][db * 16 + c16] : 0.f;
  }

  // Query rows in the MFMA A layout: row r0 + c16, depth 8*g16.. of each 32-step.
  uint4 qa[kScore ? kKB : 1];
  if constexpr (kScore) {
    const int r = r0 + c16;
    if (r < nrows_total) {
      const int h = kvh * groups + r / a.rows, s = r % a.rows;
      const char* q = static_cast<const char*>(a.query) +
                      (layer * a.q_stride_l + b * a.q_stride_b + h * a.q_stride_h + s * a.q_stride_s) * 2;
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) qa[kb] = load16(q + (kb * 32 + g16 * 8) * 2);
    } else {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) qa[kb] = make_uint4(0, 0, 0, 0);
    }
    stage_rows<D, Tag, false>(a, a.keys, layer, b, kvh, wl, wpad, loc_off, kls, kKPitch);
  }
  if constexpr (kMerge) stage_rows<D, Tag, true>(a, a.values, layer, b, kvh, wl, wpad, loc_off, vls, kVPitch);
  __syncthreads();

  // Scores: sc[nt][i] = S[r0 + 4*g16 + i][nt*16 + c16].
  const int wtiles = wpad / 16;
  f32x4_t sc[kMaxWidth / 16];
#pragma unroll
  for (int nt = 0; nt < kMaxWidth / 16; ++nt) {
    if (nt >= wtiles) break;
    const int w = nt * 16 + c16;
    if constexpr (kScore) {
      f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kls + w * kKPitch + kb * 32 + g16 * 8);
        t = Mma<Tag>::run(qa[kb], kv, t);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s = t[i] * a.softmax_scale;
        if (a.softcap > 0.f) s = tanhf(s / a.softcap) * a.softcap;
        t[i] = s;
      }
      sc[nt] = t;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[nt][i] = (valid_i[i] && w < len)
                        ? a.scores[layer * a.sc_stride_l + b * a.sc_stride_b + head_i[i] * a.sc_stride_h +
                                   srow_i[i] * a.sc_stride_s + w * a.sc_stride_w]
                        : -__builtin_inff();
    }
    if constexpr (kMode == LS_SUMMARY_SCORES) {
      if (w < a.width) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (valid_i[i])
            a.scores[layer * a.sc_stride_l + b * a.sc_stride_b + head_i[i] * a.sc_stride_h +
                     srow_i[i] * a.sc_stride_s + w * a.sc_stride_w] = sc[nt][i];
      }
    }
  }
  if constexpr (!kMerge) return;

  // Online-softmax merge of the rows w < len.
  float alpha[4], merged[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float m = -__builtin_inff();
#pragma unroll
    for (int nt = 0; nt < kMaxWidth / 16; ++nt)
      if (nt < wtiles && nt * 16 + c16 < len) m = fmaxf(m, sc[nt][i]);
    m = max16(m);
    float z = 0.f;
#pragma unroll
    for (int nt = 0; nt < kMaxWidth / 16; ++nt)
      if (nt < wtiles && nt * 16 + c16 < len) z += expf(sc[nt][i] - m);
    z = sum16(z);
    const float delta = m + logf(z);
    const float big = fmaxf(prior[i], delta);
    merged[i] = big + logf(expf(prior[i] - big) + expf(delta - big));
    alpha[i] = expf(prior[i] - merged[i]);
#pragma unroll
    for (int nt = 0; nt < kMaxWidth / 16; ++nt) {
      if (nt >= wtiles) break;
      const int w = nt * 16 + c16;
      const float p = (valid_i[i] && w < len) ? expf(sc[nt][i] - merged[i]) : 0.f;
      pls[(wave * 16 + 4 * g16 + i) * ppitch + w] = p;
    }
  }
  __syncthreads();
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[db][i] *= alpha[i];
  const int ksteps = (len + 3) / 4;
  for (int ks = 0; ks < ksteps; ++ks) {
    const float pa = pls[(wave * 16 + c16) * ppitch + 4 * ks + g16];
    const float* vrow = vls + (4 * ks + g16) * kVPitch + c16;
#pragma unroll
    for (int db = 0; db < kDB; ++db) acc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vrow[db * 16], acc[db], 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!valid_i[i]) continue;
#pragma unroll
    for (int db = 0; db < kDB; ++db) so_row[i][db * 16 + c16] = acc[db][i];
    if (c16 == 0) *sl_ptr[i] = merged[i];
  }
}

template <int D, int kMode>
int launch_d(const ls_summary_args& a, int tiles, int wpad, size_t lds, int64_t grid, hipStream_t st) {
  if (a.dtype == LS_BF16)
    summary_kernel<D, kMode, BF16><<<dim3(static_cast<unsigned>(grid)), kSumThreads, lds, st>>>(a, tiles, wpad);
  else
    summary_kernel<D, kMode, F16><<<dim3(static_cast<unsigned>(grid)), kSumThreads, lds, st>>>(a, tiles, wpad);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

bool rows_aligned(const ls_kv_rows& r) {
  const bool strides = ((r.located ? r.stride_loc : (r.stride_b | r.stride_w)) * 2) % 16 == 0 &&
                       (r.stride_h * 2) % 16 == 0 && (r.layers || (r.stride_layer * 2) % 16 == 0);
  return strides && (r.layers || aligned16(r.base));
}

template <int kMode>
int summary_entry(const ls_summary_args* ap, void* stream, const char* what) {
  LS_CHECK(ap != nullptr, LS_ERR_VALUE, "%s: null argument block", what);
  const ls_summary_args& a = *ap;
  constexpr bool kScore = kMode != LS_SUMMARY_MERGE;
  constexpr bool kMerge = kMode != LS_SUMMARY_SCORES;
  LS_CHECK(a.batch >= 0 && a.layers >= 1 && a.q_heads >= 1 && a.kv_heads >= 1 && a.rows >= 1, LS_ERR_SHAPE,
           "%s: sizes must be positive", what);
  LS_CHECK(a.q_heads % a.kv_heads == 0, LS_ERR_SHAPE, "%s: query heads (%d) must be a multiple of KV heads (%d)",
           what, a.q_heads, a.kv_heads);
  LS_CHECK(a.width >= 1 && a.width <= kMaxWidth, LS_ERR_SHAPE, "%s: width must be in [1, %d]", what, kMaxWidth);
  LS_CHECK(a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256, LS_ERR_SHAPE,
           "%s: head_dim must be 64, 128 or 256", what);
  LS_CHECK(a.dtype == LS_BF16 || a.dtype == LS_F16, LS_ERR_DTYPE, "%s: queries/keys/values must be bf16 or fp16",
           what);
  if (kScore) {
    LS_CHECK(a.query && (a.keys.base || a.keys.layers), LS_ERR_VALUE, "%s: query and keys are required", what);
    LS_CHECK(aligned16(a.query) && (a.q_stride_l * 2) % 16 == 0 && (a.q_stride_b * 2) % 16 == 0 &&
                 (a.q_stride_h * 2) % 16 == 0 && (a.q_stride_s * 2) % 16 == 0 && rows_aligned(a.keys),
             LS_ERR_ALIGN, "%s: query and key rows must be 16-byte aligned", what);
  }
  if (kMode != LS_SUMMARY_UPDATE) LS_CHECK(a.scores != nullptr, LS_ERR_VALUE, "%s: scores buffer required", what);
  if (kMerge) {
    LS_CHECK(a.state_output && a.state_lse && a.accept_lens && (a.values.base || a.values.layers), LS_ERR_VALUE,
             "%s: state, LSE, accept_lens and values are required", what);
    LS_CHECK(rows_aligned(a.values), LS_ERR_ALIGN, "%s: value rows must be 16-byte aligned", what);
  }
  const bool need_locs = (kMerge && a.values.located) || (kScore && a.keys.located);
  if (need_locs) {
    LS_CHECK(a.locs != nullptr, LS_ERR_VALUE, "%s: located rows need the location table", what);
    LS_CHECK(a.locs_dtype == LS_I32 || a.locs_dtype == LS_I64, LS_ERR_DTYPE, "%s: locations must be int32/int64",
             what);
    LS_CHECK(!a.compact_locs || a.accept_lens, LS_ERR_VALUE, "%s: compact locations need accept_lens", what);
  }
  if (a.batch == 0) return LS_OK;
  const int nrows = (a.q_heads / a.kv_heads) * a.rows;
  const int tiles = (nrows + kTileRows - 1) / kTileRows;
  const int wpad = (a.width + 15) / 16 * 16;
  const int64_t grid = a.batch * a.layers * a.kv_heads * tiles;
  LS_CHECK(grid < (int64_t(1) << 31), LS_ERR_SHAPE, "%s: grid too large", what);
  const int d = a.head_dim;
  const size_t lds = (kScore ? static_cast<size_t>(wpad) * (d + 8) * 2 : 0) +
                     (kMerge ? static_cast<size_t>(wpad) * (d + 16) * 4 + kTileRows * (wpad + 1) * 4 : 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (d) {
    case 64: return launch_d<64, kMode>(a, tiles, wpad, lds, grid, st);
    case 128: return launch_d<128, kMode>(a, tiles, wpad, lds, grid, st);
    default: return launch_d<256, kMode>(a, tiles, wpad, lds, grid, st);
  }
}

}  // namespace
}  // namespace ls

extern "C" int ls_summary_scores(const ls_summary_args* args, void* stream) {
  return ls::summary_entry<LS_SUMMARY_SCORES>(args, stream, "ls_summary_scores");
}
extern "C" int ls_summary_merge(const ls_summary_args* args, void* stream) {
  return ls::summary_entry<LS_SUMMARY_MERGE>(args, stream, "ls_summary_merge");
}
extern "C" int ls_summary_update(const ls_summary_args* args, void* stream) {
  return ls::summary_entry<LS_SUMMARY_UPDATE>(args, stream, "ls_summary_update");
}
