// Global16 prefill initialisation: non-causal attention of the summary query
// rows over each request's whole prefix, with the LSE, on the matrix cores.
//
// Reference: SRT/speculative/global16_raw256.py:668-784 (one FA3
// flash_attn_with_kvcache call per selected layer, causal = False, the
// request's location-table row as a page-size-1 page table), driven by
// src/longspark/engine/target.py:230-253; SRT = vendor/sglang/python/sglang/srt.
//
// Work split: one workgroup = (request, layer, KV head, row tile, prefix
// split).  A row tile is up to 128 query rows of the group that shares the
// KV head (r = g * S + s for query head kvh * G + g), one wave per 16 rows,
// so every key/value byte of the split is read from HBM once for all of them.
// The prefix split (chunk tokens) keeps the grid at a few thousand
// workgroups; split partials (unnormalised output, running maximum, sum) go
// to scratch and prefill_combine_kernel merges them.  With one split the
// main kernel finishes the rows itself.
//
// Per 32-token step (64 for head_dim 64):
//   staging  K and V rows -> LDS as they are ([token][d], 16-byte writes);
//            a lane's A operand of the P.V product (4 tokens x 2 of one d
//            column) is two transposing 8-byte reads (ds_read_b64_tr_b16).
//            The rows of the next two steps are in flight in registers while
//            a step computes.
//            The tile's query rows sit in LDS for the whole split.
//   scores   S^T[16 tok x 16 rows] = K[16 x D] . Q^T[D x 16]   (16x16x32 MFMA);
//            the lane holding row c16 gets tokens 4*g16 + i of each tile.
//   softmax  running maximum in the base-2 domain (s * log2 e), weights
//            exp2(s - m) in fp32, per-lane partial sums of the fp32 weights.
//   P.V      O^T[16 d x 16 rows] += V^T[16 x 32] . P^T[32 x 16]  (16x16x32 MFMA)
//            with P rounded to the key type (FA3 rounds P to its element
//            type before its P.V product).  The 32-deep contraction runs
//            over the lane's own tokens: k-slot 8*g16 + j <-> token
//            (2*kb + j/4)*16 + 4*g16 + j%4 on both operands.
#include "mfma_tile.h"

namespace ls {
namespace {

constexpr int kMaxRowsPerTile = 128;     // 8 waves of 16 rows
constexpr int kMinThreads = 256;         // staging loops assume at least 4 waves
constexpr int kMaxThreads = 512;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <int D>
struct PrefillShape {
  static constexpr int kBlk = D == 64 ? 64 : 32;    // prefix tokens per step
  static constexpr int kKP = D + 16;                  // 16-bit elements per LDS key / query row: a 32-byte skew per
                                                      // row keeps a 16-lane x 16-byte row read on distinct banks of
                                                      // gfx950's 64-bank LDS (D + 8 stalled 25% of LDS cycles)
  static constexpr int kVRP = D + 16;                 // 16-bit elements per LDS value row (token-major, skewed as
                                                      // the key rows, so a transposing read of 16 rows x 32
                                                      // bytes falls on each bank twice)
  static constexpr int kChunks = D / 8;               // 16-byte vectors per row
  static constexpr int kKVecs = kBlk * kChunks;       // key vectors per step
  static constexpr int kVUnits = (kBlk / 2) * kChunks;  // value units (2 tokens x 8 d) per step
  static constexpr int kKR = (kKVecs + kMinThreads - 1) / kMinThreads;   // per-thread key vectors
  static constexpr int kVR = (kVUnits + kMinThreads - 1) / kMinThreads;  // per-thread value units
  static constexpr int kNT = kBlk / 16;               // 16-token score tiles per step
  static constexpr int kKB = D / 32;                  // 32-deep steps of the score product
  static constexpr int kDB = D / 16;                  // 16-wide column blocks of the output
  static constexpr size_t kLds = static_cast<size_t>(kBlk) * kKP * 2 + static_cast<size_t>(kBlk) * kVRP * 2;
};

struct PrefillGeom {
  int chunk, nsplit, tiles, threads;
  int64_t units;
};

__device__ __forceinline__ float round_out(float x, int mode) {
  if (mode == LS_BF16) return to_f32<uint16_t>(from_f32<uint16_t>(x));
  if (mode == LS_F16) return __half2float(__float2half(x));
  return x;
}

template <typename Tag>
__device__ __forceinline__ uint32_t pack_weights(float lo, float hi);
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
// Round to nearest even (one v_cvt_pk_bf16_f32 on gfx950).
template <>
__device__ __forceinline__ uint32_t pack_weights<BF16>(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t pack_weights<F16>(float lo, float hi) {
  const __half a = __float2half(lo), b = __float2half(hi);
  return static_cast<uint32_t>(__half_as_ushort(a)) | (static_cast<uint32_t>(__half_as_ushort(b)) << 16);
}

// Location of prefix token t of request b (pool rows are below 2^31): the
// low 32-bit word of an int64 entry, read without a branch (a branch around
// a load makes the compiler wait for every load issued before it).
__device__ __forceinline__ int table_loc(const ls_prefill_args& a, int64_t b, int64_t t) {
  const int shift = a.pt_dtype == LS_I64 ? 1 : 0;
  return static_cast<const int32_t*>(a.page_table)[(b * a.pt_stride_b + t) << shift];
}

__device__ __forceinline__ int clamp_len(const ls_prefill_args& a, int64_t b) {
  const int64_t l = a.seq_lens[b];
  return static_cast<int>(l < 0 ? 0 : (l > a.max_len ? a.max_len : l));
}

template <int D, typename Tag, bool kCap>
__device__ __forceinline__ void prefill_body(const ls_prefill_args& a, const PrefillGeom& g, float* __restrict__ part_o,
                                             float* __restrict__ part_mz) {
  using Sh = PrefillShape<D>;
  constexpr int kBlk = Sh::kBlk;
  extern __shared__ __align__(16) char smem[];
  uint16_t* kls = reinterpret_cast<uint16_t*>(smem);
  uint16_t* vls = kls + kBlk * Sh::kKP;

  // XCD-aware unit: blocks go round-robin over 8 XCDs; each XCD takes a
  // contiguous range of units.  The KV head varies fastest, so the
  // workgroups that read the 256-byte head slices of the same 2 KiB token
  // rows run side by side on one XCD and move through the prefix together.
  const unsigned nb = gridDim.x, bi = blockIdx.x;
  const unsigned per = nb / 8, rem = nb % 8, xcd = bi % 8;
  int64_t u = static_cast<int64_t>(xcd) * per + min(xcd, rem) + bi / 8;
  const int kvh = static_cast<int>(u % a.kv_heads);
  u /= a.kv_heads;
  const int tile = static_cast<int>(u % g.tiles);
  u /= g.tiles;
  const int split = static_cast<int>(u % g.nsplit);
  u /= g.nsplit;
  const int layer = static_cast<int>(u % a.layers);
  const int64_t b = u / a.layers;

  const int tid = threadIdx.x, nthr = g.threads;
  const int lane = tid % kWave, wave = tid / kWave;
  const int g16 = lane >> 4, c16 = lane & 15;
  const int groups = a.q_heads / a.kv_heads;
  const int nrows = groups * a.rows;
  const int r = tile * kMaxRowsPerTile + wave * 16 + c16;
  const bool wave_rows = tile * kMaxRowsPerTile + wave * 16 < nrows;  // wave holds at least one row
  const bool valid = r < nrows;
  const int rr = valid ? r : 0;
  const int head = kvh * groups + rr / a.rows, srow = rr % a.rows;
  const bool direct = g.nsplit == 1;

  const int len = clamp_len(a, b);
  const int t0 = split * g.chunk;
  const int t_end = min(t0 + g.chunk, len);
  if (t_end <= t0) {  // uniform over the workgroup
    if (direct && valid) {  // empty prefix: zero output, LSE -inf
      float* orow = a.output + layer * a.o_stride_l + b * a.o_stride_b + head * a.o_stride_h + srow * a.o_stride_s;
#pragma unroll
      for (int db = 0; db < Sh::kDB; ++db)
        *reinterpret_cast<float4*>(orow + db * 16 + 4 * g16) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (g16 == 0)
        a.lse[layer * a.l_stride_l + b * a.l_stride_b + head * a.l_stride_h + srow * a.l_stride_s] = -__builtin_inff();
    }
    return;
  }
  const int nblk = (t_end - t0 + kBlk - 1) / kBlk;

  const char* kbase = layer_base(a.keys, layer) + kvh * a.keys.stride_h * 2;
  const char* vbase = layer_base(a.values, layer) + kvh * a.values.stride_h * 2;

  // Query rows of this tile -> LDS (pitch kKP); each wave reads its rows as
  // the B operand of S^T (depth kb*32 + 8*g16 .. +7).
  uint16_t* qls = vls + kBlk * Sh::kVRP;
  const int tile_rows = min(nrows - tile * kMaxRowsPerTile, kMaxRowsPerTile);
  for (int j = tid; j < tile_rows * Sh::kChunks; j += nthr) {
    const int rl = j / Sh::kChunks, c = j % Sh::kChunks;
    const int r2 = tile * kMaxRowsPerTile + rl;
    const int h2 = kvh * groups + r2 / a.rows, s2 = r2 % a.rows;
    const char* q = static_cast<const char*>(a.query) +
                    (layer * a.q_stride_l + b * a.q_stride_b + h2 * a.q_stride_h + s2 * a.q_stride_s) * 2;
    *reinterpret_cast<uint4*>(qls + rl * Sh::kKP + c * 8) = load16(q + c * 16);
  }
  const uint16_t* qrow = qls + min(wave * 16 + c16, tile_rows - 1) * Sh::kKP + g16 * 8;

  // Staging assignment: key vector j = i*nthr + tid (token j / kChunks,
  // chunk j % kChunks); value unit v = i*nthr + tid (tokens 2*(v / kChunks)
  // and the next, chunk v % kChunks).  Consecutive lanes take consecutive
  // chunks of a row: whole rows per 16 lanes, in the loads and in the 16-byte
  // LDS writes (which then fall on distinct banks).  Loads are issued with no branch
  // around them: indices past the step's work are clamped and tokens past
  // the prefix read the last prefix token (those rows get weight 0, so their
  // finite contents are unused).  A load behind a branch makes the compiler
  // wait for every earlier load before issuing it.
  struct Locs { int k[Sh::kKR], v[Sh::kVR][2]; };
  struct Rows { uint4 k[Sh::kKR], v[Sh::kVR][2]; };
  auto load_locs = [&](Locs& L, int tb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Sh::kKR; ++i) {
      const int j = min(i * nthr + tid, Sh::kKVecs - 1);
      L.k[i] = table_loc(a, b, min(tb + j / Sh::kChunks, t_end - 1));
    }
#pragma unroll
    for (int i = 0; i < Sh::kVR; ++i) {
      const int v = min(i * nthr + tid, Sh::kVUnits - 1);
      const int p2 = v / Sh::kChunks;
#pragma unroll
      for (int e = 0; e < 2; ++e) L.v[i][e] = table_loc(a, b, min(tb + 2 * p2 + e, t_end - 1));
    }
  };
  auto load_rows = [&](Rows& R, const Locs& L) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Sh::kKR; ++i) {
      const int j = min(i * nthr + tid, Sh::kKVecs - 1);
      R.k[i] = load16_global(kbase + (static_cast<int64_t>(L.k[i]) * a.keys.stride_loc + (j % Sh::kChunks) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < Sh::kVR; ++i) {
      const int v = min(i * nthr + tid, Sh::kVUnits - 1);
      const int c = v % Sh::kChunks;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        R.v[i][e] = load16_global(vbase + (static_cast<int64_t>(L.v[i][e]) * a.values.stride_loc + c * 8) * 2);
    }
  };
  auto store_rows = [&](const Rows& R) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Sh::kKR; ++i) {
      const int j = i * nthr + tid;
      if (j < Sh::kKVecs)
        *reinterpret_cast<uint4*>(kls + (j / Sh::kChunks) * Sh::kKP + (j % Sh::kChunks) * 8) = R.k[i];
    }
#pragma unroll
    for (int i = 0; i < Sh::kVR; ++i) {
      const int v = i * nthr + tid;
      if (v < Sh::kVUnits) {
        const int p2 = v / Sh::kChunks, c = v % Sh::kChunks;
        *reinterpret_cast<uint4*>(vls + (2 * p2) * Sh::kVRP + c * 8) = R.v[i][0];
        *reinterpret_cast<uint4*>(vls + (2 * p2 + 1) * Sh::kVRP + c * 8) = R.v[i][1];
      }
    }
  };

  const float qk_scale = kCap ? a.softmax_scale : a.softmax_scale * kLog2e;
  f32x4_t o[Sh::kDB];
#pragma unroll
  for (int db = 0; db < Sh::kDB; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), z = 0.f;

  auto compute = [&](int tb) __attribute__((always_inline)) {
    // scores of this lane's row: sc[nt][i] = s(row c16, token tb + nt*16 + 4*g16 + i), base 2
    f32x4_t sc[Sh::kNT];
#pragma unroll
    for (int nt = 0; nt < Sh::kNT; ++nt) sc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < Sh::kKB; ++kb) {
      const uint4 qv = *reinterpret_cast<const uint4*>(qrow + kb * 32);
#pragma unroll
      for (int nt = 0; nt < Sh::kNT; ++nt) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kls + (nt * 16 + c16) * Sh::kKP + kb * 32 + g16 * 8);
        sc[nt] = Mma<Tag>::run(kv, qv, sc[nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < Sh::kNT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s = sc[nt][i] * qk_scale;
        if constexpr (kCap) s = tanhf(s / a.softcap) * a.softcap * kLog2e;
        sc[nt][i] = s;
      }
    if (tb + kBlk > t_end) {  // uniform: the step runs past the prefix
#pragma unroll
      for (int nt = 0; nt < Sh::kNT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tb + nt * 16 + 4 * g16 + i >= t_end) sc[nt][i] = -__builtin_inff();
    }
    float bm = -__builtin_inff();
#pragma unroll
    for (int nt = 0; nt < Sh::kNT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) bm = fmaxf(bm, sc[nt][i]);
    bm = col4_max(bm);
    // finite after the first step (it holds at least one prefix token); a
    // padding step past the prefix leaves m unchanged and adds nothing
    const float mn = fmaxf(m, bm);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);  // exactly 1 where the maximum held
    m = mn;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // uniform: rescale only when a maximum rose
      z *= alpha;
#pragma unroll
      for (int db = 0; db < Sh::kDB; ++db) o[db] *= alpha;
    }
#pragma unroll
    for (int nt = 0; nt < Sh::kNT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pw = __builtin_amdgcn_exp2f(sc[nt][i] - mn);
        sc[nt][i] = pw;
        z += pw;
      }
#pragma unroll
    for (int kb = 0; kb < kBlk / 32; ++kb) {
      uint4 pb;
      pb.x = pack_weights<Tag>(sc[2 * kb][0], sc[2 * kb][1]);
      pb.y = pack_weights<Tag>(sc[2 * kb][2], sc[2 * kb][3]);
      pb.z = pack_weights<Tag>(sc[2 * kb + 1][0], sc[2 * kb + 1][1]);
      pb.w = pack_weights<Tag>(sc[2 * kb + 1][2], sc[2 * kb + 1][3]);
#pragma unroll
      for (int db = 0; db < Sh::kDB; ++db) {
        // tokens 32*kb + 4*g16 + 0..3 (lo) and 16 on (hi) of column db*16 + c16
        const uint16_t* piece = vls + (kb * 32 + 4 * g16 + c16 / 4) * Sh::kVRP + db * 16 + 4 * (c16 % 4);
        const uint2 lo = lds_read_col4(piece);
        const uint2 hi = lds_read_col4(piece + 16 * Sh::kVRP);
        o[db] = Mma<Tag>::run(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, o[db]);
      }
    }
  };

  // Two steps of rows in flight: at step n the rows of step n+1 are loading,
  // the rows of step n+2 are issued (into the registers step n has just
  // stored), and the locations of step n+3 are issued before them so that
  // waiting for those locations later never waits for rows still in flight.
  // The step count is padded to even (a padding step lies past the prefix:
  // every weight 0) so that the two register sets alternate without a branch.
  Locs L0, L1;
  Rows R0, R1;
  // (scheduling barriers keep the issue order of the loop body, which the
  // compiler's wait counts at the loop head assume)
  load_locs(L0, t0);
  load_locs(L1, t0 + kBlk);
  __builtin_amdgcn_sched_barrier(0);
  load_rows(R0, L0);
  __builtin_amdgcn_sched_barrier(0);
  load_locs(L0, t0 + 2 * kBlk);
  __builtin_amdgcn_sched_barrier(0);
  load_rows(R1, L1);
  __builtin_amdgcn_sched_barrier(0);
  const int nsteps = (nblk + 1) & ~1;
  for (int n = 0; n < nsteps; n += 2) {
    const int tb = t0 + n * kBlk;
    lds_barrier();  // the previous step's reads of the staged rows are done
    store_rows(R0);
    lds_barrier();
    load_locs(L1, tb + 3 * kBlk);
    __builtin_amdgcn_sched_barrier(0);
    load_rows(R0, L0);
    __builtin_amdgcn_sched_barrier(0);
    if (wave_rows) compute(tb);

    lds_barrier();
    store_rows(R1);
    lds_barrier();
    load_locs(L0, tb + 4 * kBlk);
    __builtin_amdgcn_sched_barrier(0);
    load_rows(R1, L1);
    __builtin_amdgcn_sched_barrier(0);
    if (wave_rows) compute(tb + kBlk);
  }
  if (!valid) return;
  z = col4_sum(z);

  if (direct) {
    const float inv = 1.f / z;
    float* orow = a.output + layer * a.o_stride_l + b * a.o_stride_b + head * a.o_stride_h + srow * a.o_stride_s;
#pragma unroll
    for (int db = 0; db < Sh::kDB; ++db) {
      float4 y;
      y.x = round_out(o[db][0] * inv, a.round_output);
      y.y = round_out(o[db][1] * inv, a.round_output);
      y.z = round_out(o[db][2] * inv, a.round_output);
      y.w = round_out(o[db][3] * inv, a.round_output);
      *reinterpret_cast<float4*>(orow + db * 16 + 4 * g16) = y;
    }
    if (g16 == 0)
      a.lse[layer * a.l_stride_l + b * a.l_stride_b + head * a.l_stride_h + srow * a.l_stride_s] =
          (m + log2f(z)) * kLn2;
    return;
  }
  const int64_t ub = (b * a.layers + layer) * a.kv_heads + kvh;
  const int64_t prow = (ub * g.nsplit + split) * nrows + r;
  float* po = part_o + prow * D;
#pragma unroll
  for (int db = 0; db < Sh::kDB; ++db)
    *reinterpret_cast<float4*>(po + db * 16 + 4 * g16) = make_float4(o[db][0], o[db][1], o[db][2], o[db][3]);
  if (g16 == 0) *reinterpret_cast<float2*>(part_mz + prow * 2) = make_float2(m, z);
}

// Head dims up to 128 fit four waves per SIMD; 256 keeps two.  kCap: scores
// pass through softcap * tanh(s / softcap).
template <int D, typename Tag, bool kCap>
__global__ __launch_bounds__(kMaxThreads) __attribute__((amdgpu_waves_per_eu(4))) void prefill_kernel(
    const ls_prefill_args a, const PrefillGeom g, float* __restrict__ part_o, float* __restrict__ part_mz) {
  prefill_body<D, Tag, kCap>(a, g, part_o, part_mz);
}
template <typename Tag, bool kCap>
__global__ __launch_bounds__(kMaxThreads) void prefill_kernel_d256(const ls_prefill_args a, const PrefillGeom g,
                                                                    float* __restrict__ part_o,
                                                                    float* __restrict__ part_mz) {
  prefill_body<256, Tag, kCap>(a, g, part_o, part_mz);
}

// One wave per (request, layer, query row of a KV head): merge the splits
// that cover the request's prefix, in split order.
template <int D>
__global__ __launch_bounds__(256) void prefill_combine_kernel(const ls_prefill_args a, const PrefillGeom g,
                                                              const float* __restrict__ part_o,
                                                              const float* __restrict__ part_mz) {
  const int groups = a.q_heads / a.kv_heads;
  const int nrows = groups * a.rows;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
  const int64_t total = a.batch * a.layers * a.kv_heads * static_cast<int64_t>(nrows);
  if (w >= total) return;
  const int lane = threadIdx.x % kWave;
  const int r = static_cast<int>(w % nrows);
  const int64_t ub = w / nrows;  // (b * layers + layer) * kv_heads + kvh
  const int kvh = static_cast<int>(ub % a.kv_heads);
  const int layer = static_cast<int>((ub / a.kv_heads) % a.layers);
  const int64_t b = ub / (static_cast<int64_t>(a.kv_heads) * a.layers);
  const int head = kvh * groups + r / a.rows, srow = r % a.rows;
  const int len = clamp_len(a, b);
  const int ns = (len + g.chunk - 1) / g.chunk;

  // split maxima and sums across the lanes (lane s holds split s), then the
  // output with the lanes owning 4 consecutive values of the row and four
  // splits' partial rows in flight at a time
  const float2* mz = reinterpret_cast<const float2*>(part_mz) + (ub * g.nsplit) * nrows + r;
  float mx = -__builtin_inff();
  for (int s = lane; s < ns; s += kWave) mx = fmaxf(mx, mz[static_cast<int64_t>(s) * nrows].x);
  mx = wave_max(mx);
  float zs = 0.f;
  for (int s = lane; s < ns; s += kWave) {
    const float2 v = mz[static_cast<int64_t>(s) * nrows];
    zs += v.y * __builtin_amdgcn_exp2f(v.x - mx);
  }
  zs = wave_sum(zs);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const bool mine = lane * 4 < D;
  if (mine) {
    const float* po = part_o + ((ub * g.nsplit) * nrows + r) * D + lane * 4;
    const int64_t sstride = static_cast<int64_t>(nrows) * D;
    int s = 0;
    for (; s + 4 <= ns; s += 4) {
      float4 v[4];
      float f[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = *reinterpret_cast<const float4*>(po + (s + k) * sstride);
        f[k] = __builtin_amdgcn_exp2f(mz[static_cast<int64_t>(s + k) * nrows].x - mx);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc.x += v[k].x * f[k];
        acc.y += v[k].y * f[k];
        acc.z += v[k].z * f[k];
        acc.w += v[k].w * f[k];
      }
    }
    for (; s < ns; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(po + s * sstride);
      const float f = __builtin_amdgcn_exp2f(mz[static_cast<int64_t>(s) * nrows].x - mx);
      acc.x += v.x * f;
      acc.y += v.y * f;
      acc.z += v.z * f;
      acc.w += v.w * f;
    }
  }
  float* orow = a.output + layer * a.o_stride_l + b * a.o_stride_b + head * a.o_stride_h + srow * a.o_stride_s;
  const float inv = ns > 0 ? 1.f / zs : 0.f;
  if (mine) {
    float4 y;
    y.x = round_out(acc.x * inv, a.round_output);
    y.y = round_out(acc.y * inv, a.round_output);
    y.z = round_out(acc.z * inv, a.round_output);
    y.w = round_out(acc.w * inv, a.round_output);
    *reinterpret_cast<float4*>(orow + lane * 4) = y;
  }
  if (lane == 0)
    a.lse[layer * a.l_stride_l + b * a.l_stride_b + head * a.l_stride_h + srow * a.l_stride_s] =
        ns > 0 ? (mx + log2f(zs)) * kLn2 : -__builtin_inff();
}

size_t prefill_lds(int d, int nrows) {
  const int tile_rows = nrows < kMaxRowsPerTile ? nrows : kMaxRowsPerTile;
  switch (d) {
    case 64: return PrefillShape<64>::kLds + static_cast<size_t>(tile_rows) * PrefillShape<64>::kKP * 2;
    case 128: return PrefillShape<128>::kLds + static_cast<size_t>(tile_rows) * PrefillShape<128>::kKP * 2;
    default: return PrefillShape<256>::kLds + static_cast<size_t>(tile_rows) * PrefillShape<256>::kKP * 2;
  }
}

// Workgroups resident on the device at once: CUs x per-CU limit from wave
// slots (4 waves per SIMD for head_dim <= 128, 2 for 256) and 160 KiB of LDS.
int64_t resident_slots(int d, int threads, size_t lds) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
    (void)hipGetLastError();
  }
  const int waves = threads / kWave;
  const int by_waves = (d == 256 ? 8 : 16) / waves;
  const int by_lds = static_cast<int>((160 * 1024) / lds);
  const int per_cu = by_waves < by_lds ? by_waves : by_lds;
  return static_cast<int64_t>(cus) * (per_cu > 0 ? per_cu : 1);
}

bool kv_rows_aligned(const ls_kv_rows& r) {
  return r.located && (r.stride_loc * 2) % 16 == 0 && (r.stride_h * 2) % 16 == 0 &&
         (r.layers || ((r.stride_layer * 2) % 16 == 0 && aligned16(r.base)));
}

// Validates the arguments and fixes the launch geometry.
// Pointers, strides and alignment are checked only when `launch` is set (the
// workspace query needs the sizes alone).
int prefill_geometry(const ls_prefill_args* ap, const char* what, bool launch, PrefillGeom* g, int64_t* scratch) {
  LS_CHECK(ap != nullptr, LS_ERR_VALUE, "%s: null argument block", what);
  const ls_prefill_args& a = *ap;
  LS_CHECK(a.batch >= 0 && a.layers >= 1 && a.q_heads >= 1 && a.kv_heads >= 1 && a.rows >= 1, LS_ERR_SHAPE,
           "%s: sizes must be positive", what);
  LS_CHECK(a.q_heads % a.kv_heads == 0, LS_ERR_SHAPE, "%s: query heads (%d) must be a multiple of KV heads (%d)",
           what, a.q_heads, a.kv_heads);
  LS_CHECK(a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256, LS_ERR_SHAPE,
           "%s: head_dim must be 64, 128 or 256", what);
  LS_CHECK(a.dtype == LS_BF16 || a.dtype == LS_F16, LS_ERR_DTYPE, "%s: queries/keys/values must be bf16 or fp16",
           what);
  LS_CHECK(a.round_output == LS_F32 || a.round_output == LS_BF16 || a.round_output == LS_F16, LS_ERR_VALUE,
           "%s: round_output must be LS_F32, LS_BF16 or LS_F16", what);
  LS_CHECK(a.max_len >= 0 && a.max_len < (int64_t(1) << 31), LS_ERR_SHAPE, "%s: max_len out of range", what);
  LS_CHECK(a.chunk >= 0 && a.chunk % 64 == 0, LS_ERR_VALUE, "%s: chunk must be a multiple of 64", what);
  LS_CHECK(a.softmax_scale > 0.f && a.softcap >= 0.f, LS_ERR_VALUE, "%s: softmax_scale must be > 0, softcap >= 0",
           what);
  if (launch && a.batch > 0) {
    LS_CHECK(a.query && (a.keys.base || a.keys.layers) && (a.values.base || a.values.layers) && a.seq_lens &&
                 a.output && a.lse && (a.page_table || a.max_len == 0),
             LS_ERR_VALUE, "%s: query, keys, values, page_table, seq_lens, output and lse are required", what);
    LS_CHECK(a.pt_dtype == LS_I32 || a.pt_dtype == LS_I64, LS_ERR_DTYPE, "%s: page_table must be int32/int64",
             what);
    LS_CHECK(aligned16(a.query) && (a.q_stride_l * 2) % 16 == 0 && (a.q_stride_b * 2) % 16 == 0 &&
                 (a.q_stride_h * 2) % 16 == 0 && (a.q_stride_s * 2) % 16 == 0,
             LS_ERR_ALIGN, "%s: query rows must be 16-byte aligned", what);
    LS_CHECK(kv_rows_aligned(a.keys) && kv_rows_aligned(a.values), LS_ERR_ALIGN,
             "%s: key/value rows must be located and 16-byte aligned", what);
    LS_CHECK(aligned16(a.output) && (a.o_stride_l * 4) % 16 == 0 && (a.o_stride_b * 4) % 16 == 0 &&
                 (a.o_stride_h * 4) % 16 == 0 && (a.o_stride_s * 4) % 16 == 0,
             LS_ERR_ALIGN, "%s: output rows must be 16-byte aligned", what);
  }
  const int nrows = (a.q_heads / a.kv_heads) * a.rows;
  g->tiles = (nrows + kMaxRowsPerTile - 1) / kMaxRowsPerTile;
  const int tile_rows = nrows < kMaxRowsPerTile ? nrows : kMaxRowsPerTile;
  const int waves = (tile_rows + 15) / 16;
  g->threads = (waves < kMinThreads / kWave ? kMinThreads / kWave : waves) * kWave;
  const int64_t base = a.batch * a.layers * a.kv_heads * g->tiles;
  int64_t chunk = a.chunk;
  if (chunk == 0) {
    // As many splits as fill the resident workgroup slots once (a partial
    // second round would leave most CUs idle), at least 512 prefix tokens each.
    const int64_t slots = resident_slots(a.head_dim, g->threads, prefill_lds(a.head_dim, nrows));
    const int64_t want = base > 0 && slots > base ? slots / base : 1;
    chunk = (a.max_len + want - 1) / want;
    chunk = (chunk + 63) / 64 * 64;
    if (chunk < 512) chunk = 512;
  }
  const int64_t nsplit = a.max_len > 0 ? (a.max_len + chunk - 1) / chunk : 1;
  LS_CHECK(chunk < (int64_t(1) << 30), LS_ERR_VALUE, "%s: chunk too large", what);
  g->chunk = static_cast<int>(chunk);
  g->nsplit = static_cast<int>(nsplit);
  g->units = base * nsplit;
  LS_CHECK(g->units < (int64_t(1) << 31), LS_ERR_SHAPE, "%s: grid too large", what);
  *scratch = nsplit > 1 ? a.batch * a.layers * a.kv_heads * nsplit * nrows * (a.head_dim + 2) * int64_t(4) : 0;
  return LS_OK;
}

template <int D, typename Tag>
int launch_prefill(const ls_prefill_args& a, const PrefillGeom& g, float* part_o, float* part_mz, hipStream_t st) {
  const size_t lds = prefill_lds(D, (a.q_heads / a.kv_heads) * a.rows);
  const dim3 grid(static_cast<unsigned>(g.units));
  if constexpr (D == 256) {
    if (a.softcap > 0.f)
      prefill_kernel_d256<Tag, true><<<grid, g.threads, lds, st>>>(a, g, part_o, part_mz);
    else
      prefill_kernel_d256<Tag, false><<<grid, g.threads, lds, st>>>(a, g, part_o, part_mz);
  } else {
    if (a.softcap > 0.f)
      prefill_kernel<D, Tag, true><<<grid, g.threads, lds, st>>>(a, g, part_o, part_mz);
    else
      prefill_kernel<D, Tag, false><<<grid, g.threads, lds, st>>>(a, g, part_o, part_mz);
  }
  LS_LAUNCH_CHECK();
  if (g.nsplit > 1) {
    const int64_t waves = a.batch * a.layers * a.kv_heads * static_cast<int64_t>((a.q_heads / a.kv_heads) * a.rows);
    const int64_t blocks = (waves + 3) / 4;
    LS_CHECK(blocks < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_global16_prefill: grid too large");
    prefill_combine_kernel<D><<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(a, g, part_o, part_mz);
    LS_LAUNCH_CHECK();
  }
  return LS_OK;
}

template <int D>
int launch_prefill_d(const ls_prefill_args& a, const PrefillGeom& g, float* po, float* pmz, hipStream_t st) {
  return a.dtype == LS_BF16 ? launch_prefill<D, BF16>(a, g, po, pmz, st) : launch_prefill<D, F16>(a, g, po, pmz, st);
}

}  // namespace
}  // namespace ls

extern "C" int ls_global16_prefill_workspace(const ls_prefill_args* args, int64_t* scratch_bytes) {
  using namespace ls;
  LS_CHECK(scratch_bytes != nullptr, LS_ERR_VALUE, "ls_global16_prefill_workspace: null output");
  PrefillGeom g;
  int64_t need = 0;
  const int rc = prefill_geometry(args, "ls_global16_prefill_workspace", false, &g, &need);
  if (rc != LS_OK) return rc;
  *scratch_bytes = need;
  return LS_OK;
}

extern "C" int ls_global16_prefill(const ls_prefill_args* args, void* scratch, int64_t scratch_bytes, void* stream) {
  using namespace ls;
  const char* what = "ls_global16_prefill";
  PrefillGeom g;
  int64_t need = 0;
  const int rc = prefill_geometry(args, what, true, &g, &need);
  if (rc != LS_OK) return rc;
  const ls_prefill_args& a = *args;
  if (a.batch == 0) return LS_OK;
  LS_CHECK(need == 0 || (scratch && scratch_bytes >= need && aligned16(scratch)), LS_ERR_WORKSPACE,
           "%s: scratch of %lld bytes (16-byte aligned) required", what, static_cast<long long>(need));
  const int64_t nrows = static_cast<int64_t>(a.q_heads / a.kv_heads) * a.rows;
  float* part_o = static_cast<float*>(scratch);
  float* part_mz = need ? part_o + a.batch * a.layers * a.kv_heads * int64_t(g.nsplit) * nrows * a.head_dim : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (a.head_dim) {
    case 64: return launch_prefill_d<64>(a, g, part_o, part_mz, st);
    case 128: return launch_prefill_d<128>(a, g, part_o, part_mz, st);
    default: return launch_prefill_d<256>(a, g, part_o, part_mz, st);
  }
}
