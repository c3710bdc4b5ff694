// Summary (Global16) state refresh: cached position scores and the
// online-softmax merge of accepted rows, on the matrix cores.
//
// One workgroup = 4 waves = one 64-row tile of the query rows that share a
// KV head (rows r = g * S + s for the g-th query head of the group), for one
// (layer, KV head, request); each lane owns one row.  The request index varies fastest and the
// block -> unit mapping keeps consecutive units on one XCD, so the requests
// that share a query tile (queries are shared across requests) read it from
// the same L2.
//
//   scores  S^T[16 x 16] = K[16 x D] . Q^T[D x 16]   v_mfma_f32_16x16x32_{bf16,f16}
//           (bf16/fp16 products are exact in fp32; fp32 accumulation);
//   merge   O^T[16 x 16] = O^T * alpha + V^T[16 x W] . P^T[W x 16]   v_mfma_f32_16x16x4_f32
//           (P stays fp32: weights are not rounded to 16 bits).
// Computing the transposed products leaves each lane with 4 consecutive
// state values of one row, so the state moves with 16-byte loads and stores.
// Reference math: SRT/speculative/global16_raw256_incremental.py:50-166 and
// the kernel forms :172-238 (scores) and :258-392 (merge, including its
// M + log(exp(lse - M) + exp(d - M)) LSE update);
// SRT = vendor/sglang/python/sglang/srt.
#include "mfma_tile.h"

namespace ls {
namespace {

constexpr int kSumThreads = 256;
constexpr int kWaves = 4;
constexpr int kTileRows = 64;
constexpr int kMaxWidth = 32;

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

// Stage rows w < nrows of the keys (kept as 16-bit patterns, pitch kp) and/or
// values (widened to fp32, pitch vp) into LDS; rows nrows..wpad-1 are zero.
// koff / voff hold each row's element offset within its layer.
template <int D, typename Tag, bool kKeys, bool kValues>
__device__ __forceinline__ void stage_rows(const char* kbase, const char* vbase, const int64_t* koff,
                                           const int64_t* voff, int nrows, int wpad, uint16_t* kls, int kp,
                                           float* vls, int vp) {
  constexpr int kVecs = D / 8;
  for (int j = threadIdx.x; j < wpad * kVecs; j += kSumThreads) {
    const int w = j / kVecs, c = j - w * kVecs;
    uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
    if (kKeys) kv = load16_global(kbase + (koff[w] + c * 8) * 2);
    if (kValues) vv = load16_global(vbase + (voff[w] + c * 8) * 2);
    if (w >= nrows) {
      kv = make_uint4(0, 0, 0, 0);
      vv = make_uint4(0, 0, 0, 0);
    }
    if (kKeys) *reinterpret_cast<uint4*>(kls + w * kp + c * 8) = kv;
    if (kValues) {
      float f[8];
      unpack16<Tag>(vv, f);
      float4* dst = reinterpret_cast<float4*>(vls + w * vp + c * 8);
      dst[0] = make_float4(f[0], f[1], f[2], f[3]);
      dst[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
}

// Waves per SIMD the kernel is compiled for.  At head_dim <= 128 the
// register allocator otherwise puts the MFMA accumulators in AGPRs on top of
// ~78 VGPRs (4 waves per SIMD, 16 per CU); bounded at 6, the accumulators
// share the VGPRs (74 in all, no spills) and 24 waves per CU are resident.
#ifndef LS_SUMMARY_WAVES
#define LS_SUMMARY_WAVES 6
#endif
constexpr int summary_waves(int d) { return d <= 128 ? LS_SUMMARY_WAVES : 2; }

template <int D, int kMode, typename Tag>
__global__ __launch_bounds__(kSumThreads, summary_waves(D)) void summary_kernel(const ls_summary_args a, int tiles,
                                                                                int wpad) {
  constexpr bool kScore = kMode != LS_SUMMARY_MERGE;   // computes scores from queries and keys
  constexpr bool kMerge = kMode != LS_SUMMARY_SCORES;  // folds accepted rows into the state
  constexpr int kKB = D / 32;      // 32-deep steps of the score product
  constexpr int kDB = D / 16;      // 16-column blocks of the state
  constexpr int kKPitch = D + 16;  // 16-bit elements per LDS key row (32-byte skew: distinct banks of the 64-bank LDS)
  constexpr int kVPitch = D + 4;   // fp32 per LDS value row: rows 4 apart land 16 banks apart
  extern __shared__ __align__(16) char smem[];
  __shared__ int64_t s_koff[kMaxWidth], s_voff[kMaxWidth];
  uint16_t* kls = reinterpret_cast<uint16_t*>(smem);
  float* vls = reinterpret_cast<float*>(smem + (kScore ? wpad * kKPitch * 2 : 0));

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
  const int lane = threadIdx.x % kWave;
  const int g16 = lane >> 4, c16 = lane & 15;
  // Each lane owns one query row (c16 of its wave's 16) in every product below:
  //   S^T[w][r] = K[w] . Q[r]    lane holds w = nt*16 + 4*g16 + i,
  //   O^T[d][r] += V^T[d][w] P^T[w][r]   lane holds d = db*16 + 4*g16 + i,
  // so its state values are 4 consecutive floats of its row.
  const int r = tile * kTileRows + (threadIdx.x / kWave) * 16 + c16;
  const bool valid = r < groups * a.rows;
  const int rr = valid ? r : 0;
  const int head = kvh * groups + rr / a.rows, srow = rr % a.rows;

  int len = a.width;
  if (kMerge) {
    const int l = a.accept_lens[b];
    len = l < 0 ? 0 : (l > a.width ? a.width : l);
  }
  int64_t loc_off = 0;
  if (a.compact_locs && (kMerge || a.keys.located)) {
    for (int64_t j = lane; j < b; j += kWave) loc_off += a.accept_lens[j];
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) loc_off += __shfl_xor(loc_off, o, kWave);
    if (a.accept_offsets && threadIdx.x == 0 && layer == 0 && kvh == 0 && tile == 0)
      a.accept_offsets[b] = static_cast<int32_t>(loc_off);
  }
  if (kMerge && len <= 0) return;  // uniform over the workgroup
  const int wl = kMerge ? len : a.width;  // key/value rows that take part

  // Row offsets of the staged key/value rows (rows past wl repeat row wl-1,
  // a valid address; their data is zeroed when staged).
  if (threadIdx.x < wpad) {
    const int wr = static_cast<int>(threadIdx.x) < wl ? static_cast<int>(threadIdx.x) : wl - 1;
    const bool need_loc = (kScore && a.keys.located) || (kMerge && a.values.located);
    const int64_t loc = need_loc ? load_loc(a, b, wr, loc_off) : 0;
    if (kScore) s_koff[threadIdx.x] = row_offset(a.keys, b, wr, loc, kvh);
    if (kMerge) s_voff[threadIdx.x] = row_offset(a.values, b, wr, loc, kvh);
  }

  // State row and prior LSE (the bulk of the traffic; issued first).
  f32x4_t o[kMerge ? kDB : 1];
  float prior = 0.f;
  float* so_row = nullptr;
  float* sl_ptr = nullptr;
  if constexpr (kMerge) {
    const int64_t slot = a.state_slots ? a.state_slots[b] : b;
    so_row = a.state_output + slot * a.so_stride_c + layer * a.so_stride_l + head * a.so_stride_h +
             srow * a.so_stride_s + 4 * g16;
    sl_ptr = a.state_lse + slot * a.sl_stride_c + layer * a.sl_stride_l + head * a.sl_stride_h +
             srow * a.sl_stride_s;
    // Lanes past the last row read row 0 (a valid address) and never store.
#pragma unroll
    for (int db = 0; db < kDB; ++db) o[db] = *reinterpret_cast<const f32x4_t*>(so_row + db * 16);
    prior = *sl_ptr;
  }

  // Query row as the B operand of S^T: depth 8*g16.. of each 32-step.
  uint4 qb[kScore ? kKB : 1];
  if constexpr (kScore) {
    const char* q = static_cast<const char*>(a.query) +
                    (layer * a.q_stride_l + b * a.q_stride_b + head * a.q_stride_h + srow * a.q_stride_s) * 2;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) qb[kb] = load16(q + (kb * 32 + g16 * 8) * 2);
  }
  lds_barrier();
  stage_rows<D, Tag, kScore, kMerge>(kScore ? layer_base(a.keys, layer) : nullptr,
                                     kMerge ? layer_base(a.values, layer) : nullptr, s_koff, s_voff, wl, wpad, kls,
                                     kKPitch, vls, kVPitch);
  lds_barrier();

  // Scores of this lane's row: sc[nt][i] = S[r][nt*16 + 4*g16 + i].
  const int wtiles = wpad / 16;
  f32x4_t sc[kMaxWidth / 16];
  const float* sc_row = nullptr;
  if (kMode != LS_SUMMARY_UPDATE)
    sc_row = a.scores + layer * a.sc_stride_l + b * a.sc_stride_b + head * a.sc_stride_h + srow * a.sc_stride_s;
#pragma unroll
  for (int nt = 0; nt < kMaxWidth / 16; ++nt) {
    if (nt >= wtiles) break;
    const int w0 = nt * 16 + 4 * g16;
    if constexpr (kScore) {
      f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kls + (nt * 16 + c16) * kKPitch + kb * 32 + g16 * 8);
        t = Mma<Tag>::run(kv, qb[kb], t);
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
        sc[nt][i] = (valid && w0 + i < len) ? sc_row[(w0 + i) * a.sc_stride_w] : -__builtin_inff();
    }
    if constexpr (kMode == LS_SUMMARY_SCORES) {
      float* out = const_cast<float*>(sc_row);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (valid && w0 + i < a.width) out[(w0 + i) * a.sc_stride_w] = sc[nt][i];
    }
  }
  if constexpr (!kMerge) return;

  // Online-softmax merge of the rows w < len: each row's 16*wtiles scores sit
  // in the 4 lanes that share c16.
  float m = -__builtin_inff();
#pragma unroll
  for (int nt = 0; nt < kMaxWidth / 16; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nt < wtiles && nt * 16 + 4 * g16 + i < len) m = fmaxf(m, sc[nt][i]);
  m = col4_max(m);
  float z = 0.f;
#pragma unroll
  for (int nt = 0; nt < kMaxWidth / 16; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nt < wtiles && nt * 16 + 4 * g16 + i < len) z += expf(sc[nt][i] - m);
  z = col4_sum(z);
  const float delta = m + logf(z);
  const float big = fmaxf(prior, delta);
  const float merged = big + logf(expf(prior - big) + expf(delta - big));
  const float alpha = expf(prior - merged);
#pragma unroll
  for (int db = 0; db < kDB; ++db) o[db] *= alpha;
  // k step ks of tile nt pairs lane (g16, c16) with w = nt*16 + 4*g16 + ks on both operands.
#pragma unroll
  for (int nt = 0; nt < kMaxWidth / 16; ++nt) {
    if (nt >= wtiles || nt * 16 >= len) break;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int w = nt * 16 + 4 * g16 + ks;
      const float pb = (valid && w < len) ? expf(sc[nt][ks] - merged) : 0.f;
      const float* vrow = vls + w * kVPitch + c16;
#pragma unroll
      for (int db = 0; db < kDB; ++db) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[db * 16], pb, o[db], 0, 0, 0);
    }
  }
  if (!valid) return;
#pragma unroll
  for (int db = 0; db < kDB; ++db)
    *reinterpret_cast<f32x4_t*>(so_row + db * 16) = o[db];
  if (g16 == 0) *sl_ptr = merged;
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
    LS_CHECK(aligned16(a.state_output) && (a.so_stride_c * 4) % 16 == 0 && (a.so_stride_l * 4) % 16 == 0 &&
                 (a.so_stride_h * 4) % 16 == 0 && (a.so_stride_s * 4) % 16 == 0,
             LS_ERR_ALIGN, "%s: state rows must be 16-byte aligned", what);
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
  const size_t lds = (kScore ? static_cast<size_t>(wpad) * (d + 16) * 2 : 0) +
                     (kMerge ? static_cast<size_t>(wpad) * (d + 4) * 4 : 0);
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
