// Drafter attention over the three refreshed views in one kernel:
// Raw256 (the recent window, read through the request's page-table row),
// Global16 (the summary state) and Local7 (the in-block rows).
//
// Reference: SRT/speculative/global16_raw256_draft_all_attention.py:52-281
// (one Triton program per (request, query head)); SRT =
// vendor/sglang/python/sglang/srt.  For every query row (7 per head) the
// sources are folded in the reference's order, each as one online-softmax step
// (running maximum m, sum z, unnormalised output o):
//   raw     blocks of 64 window rows, scores = (q . k) * scale (fp32),
//           rows at or past raw_lengths[b] invisible;
//   global  16 rows per query head, scores = bf16(q . k) * scale;
//           values = the fp32 summary state rounded to bf16;
//   local   7 rows per KV head, scores = bf16(q . k) * scale, visibility
//           from the request's 7 x 7 mask.
// In every step the weights exp(s - m) enter the weighted sum of values as
// bf16 and the sum z as fp32, as the reference does; out = o / z in bf16.
//
// Here one workgroup serves (request, KV head): one wave per query head of
// the group, so each raw key/value row is read from HBM once for all of
// them (the reference reads it once per query head).  Raw rows are staged in
// LDS as they are ([row][d]; the value operand of P.V comes out of a
// transposing LDS read, ds_read_b64_tr_b16); the products run on
// v_mfma_f32_16x16x32_bf16 with the 7 query rows padded to 16:
//   S^T[16 src x 16 rows] = K[16 x 128] . Q^T,   O^T += V^T[16 x 32] . P^T[32 x 16]
// (the lane holding row c16 gets sources 4*g16 + i of each 16-source tile).
#include "mfma_tile.h"

namespace ls {
namespace {

constexpr int kD = 128;          // head_dim
constexpr int kRows = 7;         // query rows per head
constexpr int kGlobal = 16;      // summary rows per query head
constexpr int kLocal = 7;        // in-block rows per KV head
constexpr int kRaw = 256;        // window rows
constexpr int kBlk = 64;         // window rows per step (the reference's block)
constexpr int kChunks = kD / 8;  // 16-byte vectors per row
constexpr int kKP = kD + 8;      // 16-bit elements per LDS key row
constexpr int kVRP = kD + 16;    // 16-bit elements per LDS value row (token-major, skewed as the key rows)
constexpr int kMinThreads = 256;
constexpr int kKR = kBlk * kChunks / kMinThreads;         // key vectors per thread per step (4)
constexpr int kVR = (kBlk / 2) * kChunks / kMinThreads;   // value pairs per thread per step (2)
constexpr int kKB = kD / 32;
constexpr int kDB = kD / 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr size_t kLds = static_cast<size_t>(kBlk) * kKP * 2 + static_cast<size_t>(kBlk) * kVRP * 2 + kRaw * 4;

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// x rounded to bf16 (nearest even) and widened back, through the hardware
// conversion (v_cvt_pk_bf16_f32) rather than integer rounding with a NaN branch.
__device__ __forceinline__ float round_bf16(float x) { return __builtin_bit_cast(float, pack_bf16(x, 0.f) << 16); }


// Online-softmax state of the lane's query row (the 4 lanes of a row hold
// the same m; z is a per-lane partial sum).
struct RowState {
  f32x4_t o[kDB];
  float m, z;
};

// Fold one 16-or-32-source tile of base-2 scores into the row state.
// sc[t][i]: score of source t*16 + 4*g16 + i (-inf when invisible);
// vt(db, t) returns the A operand half (4 bf16 values of sources
// t*16 + 4*g16 .. +3 at column db*16 + c16) for tile t.
template <int kTiles, typename VT>
__device__ __forceinline__ void fold(RowState& st, f32x4_t (&sc)[kTiles], VT vt) {
  float bm = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) bm = fmaxf(bm, sc[t][i]);
  bm = col4_max(bm);
  const float mn = fmaxf(st.m, bm);
  // a row with nothing visible yet keeps m = -inf: subtract 0 instead
  const float base = mn == -__builtin_inff() ? 0.f : mn;
  const float alpha = __builtin_amdgcn_exp2f(st.m - base);
  st.m = mn;
  st.z *= alpha;
#pragma unroll
  for (int db = 0; db < kDB; ++db) st.o[db] *= alpha;
  float p[kTiles][4];
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[t][i] = __builtin_amdgcn_exp2f(sc[t][i] - base);
      st.z += p[t][i];
    }
#pragma unroll
  for (int kb = 0; kb < (kTiles + 1) / 2; ++kb) {
    uint4 pb;
    pb.x = pack_bf16(p[2 * kb][0], p[2 * kb][1]);
    pb.y = pack_bf16(p[2 * kb][2], p[2 * kb][3]);
    if (2 * kb + 1 < kTiles) {
      pb.z = pack_bf16(p[(2 * kb + 1) % kTiles][0], p[(2 * kb + 1) % kTiles][1]);
      pb.w = pack_bf16(p[(2 * kb + 1) % kTiles][2], p[(2 * kb + 1) % kTiles][3]);
    } else {
      pb.z = 0u;
      pb.w = 0u;
    }
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const uint2 lo = vt(db, 2 * kb);
      const uint2 hi = 2 * kb + 1 < kTiles ? vt(db, 2 * kb + 1) : make_uint2(0u, 0u);
      st.o[db] = Mma<BF16>::run(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, st.o[db]);
    }
  }
}

__global__ __launch_bounds__(1024) void draft_attention_kernel(const ls_draft_attention_args a, int threads) {
  extern __shared__ __align__(16) char smem[];
  uint16_t* kls = reinterpret_cast<uint16_t*>(smem);
  uint16_t* vls = kls + kBlk * kKP;
  int32_t* locs = reinterpret_cast<int32_t*>(vls + kBlk * kVRP);  // the request's window rows

  const int64_t b = blockIdx.x / a.kv_heads;
  const int kvh = static_cast<int>(blockIdx.x % a.kv_heads);
  const int groups = a.q_heads / a.kv_heads;
  const int tid = threadIdx.x, nthr = threads;
  const int lane = tid % kWave, wave = tid / kWave;
  const int g16 = lane >> 4, c16 = lane & 15;
  const bool head_wave = wave < groups;
  const int head = kvh * groups + (head_wave ? wave : 0);
  const bool row_ok = c16 < kRows;
  const float scale2 = a.softmax_scale * kLog2e;
  // the request's state slot (a scalar load; used after the window)
  const int64_t slot = load_uniform(a.state_slots + b);

  // Query row c16 of this wave's head as the B operand (rows 7..15 zero).
  uint4 qb[kKB];
  {
    const uint16_t* q = static_cast<const uint16_t*>(a.query) + b * a.q_stride_b + head * a.q_stride_h +
                        (row_ok ? c16 : 0) * a.q_stride_r;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      const uint4 v = load16(q + kb * 32 + g16 * 8);
      qb[kb] = row_ok ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  RowState st;
#pragma unroll
  for (int db = 0; db < kDB; ++db) st.o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -__builtin_inff();
  st.z = 0.f;

  // ---- raw window: ceil(len / 64) steps through the page-table row ----
  int raw_len = a.raw_lengths[b];
  raw_len = raw_len < 0 ? 0 : (raw_len > kRaw ? kRaw : raw_len);
  const char* kbase = static_cast<const char*>(a.key_cache) + kvh * a.kc_stride_h * 2;
  const char* vbase = static_cast<const char*>(a.value_cache) + kvh * a.vc_stride_h * 2;
  // The window's row locations, read once into LDS, so each block's loads
  // wait on no page-table round trip.
  {
    const int32_t* pt = a.page_table + b * a.pt_stride_b;
    for (int i = tid; i < raw_len; i += nthr) locs[i] = pt[i];
  }
  lds_barrier();
  for (int tb = 0; tb < raw_len; tb += kBlk) {
    // loads first (no branch around them; rows past the window read row
    // raw_len - 1 and get weight 0), then the LDS stores
    uint4 kr[kKR], vr[kVR][2];
#pragma unroll
    for (int i = 0; i < kKR; ++i) {
      const int j = min(i * nthr + tid, kBlk * kChunks - 1);
      const int64_t loc = locs[min(tb + j / kChunks, raw_len - 1)];
      kr[i] = load16_global(kbase + (loc * a.kc_stride_s + (j % kChunks) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < kVR; ++i) {
      // chunk-fastest: 16 lanes load (and below write) whole rows
      const int v = min(i * nthr + tid, (kBlk / 2) * kChunks - 1);
      const int p2 = v / kChunks, c = v % kChunks;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int64_t loc = locs[min(tb + 2 * p2 + e, raw_len - 1)];
        vr[i][e] = load16_global(vbase + (loc * a.vc_stride_s + c * 8) * 2);
      }
    }
    lds_barrier();  // previous step's reads done
#pragma unroll
    for (int i = 0; i < kKR; ++i) {
      const int j = i * nthr + tid;
      if (j < kBlk * kChunks) *reinterpret_cast<uint4*>(kls + (j / kChunks) * kKP + (j % kChunks) * 8) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < kVR; ++i) {
      const int v = i * nthr + tid;
      if (v < (kBlk / 2) * kChunks) {
        const int p2 = v / kChunks, c = v % kChunks;
        *reinterpret_cast<uint4*>(vls + (2 * p2) * kVRP + c * 8) = vr[i][0];
        *reinterpret_cast<uint4*>(vls + (2 * p2 + 1) * kVRP + c * 8) = vr[i][1];
      }
    }
    lds_barrier();
    if (!head_wave) continue;
    f32x4_t sc[kBlk / 16];
#pragma unroll
    for (int t = 0; t < kBlk / 16; ++t) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
        acc = Mma<BF16>::run(*reinterpret_cast<const uint4*>(kls + (t * 16 + c16) * kKP + kb * 32 + g16 * 8),
                             qb[kb], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[t][i] = tb + t * 16 + 4 * g16 + i < raw_len ? acc[i] * scale2 : -__builtin_inff();
    }
    // tokens t*16 + 4*g16 + 0..3 of column db*16 + c16, by a transposing read
    fold<kBlk / 16>(st, sc, [&](int db, int t) __attribute__((always_inline)) {
      return lds_read_col4(vls + (t * 16 + 4 * g16 + c16 / 4) * kVRP + db * 16 + 4 * (c16 % 4));
    });
  }
  if (!head_wave) return;

  // ---- global: 16 summary rows of this query head ----
  {
    const uint16_t* gk = static_cast<const uint16_t*>(a.global_keys) + b * a.gk_stride_b + head * a.gk_stride_h +
                         c16 * a.gk_stride_g;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) acc = Mma<BF16>::run(load16(gk + kb * 32 + g16 * 8), qb[kb], acc);
    f32x4_t sc[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[0][i] = round_bf16(acc[i]) * a.softmax_scale * kLog2e;
    const float* gv = a.global_values + slot * a.gv_stride_b + head * a.gv_stride_h;
    fold<1>(st, sc, [&](int db, int) __attribute__((always_inline)) {
      const float* col = gv + (4 * g16) * a.gv_stride_g + db * 16 + c16;
      return make_uint2(pack_bf16(col[0], col[a.gv_stride_g]), pack_bf16(col[2 * a.gv_stride_g], col[3 * a.gv_stride_g]));
    });
  }

  // ---- local: 7 in-block rows of this KV head, per-row visibility ----
  {
    const uint16_t* lk = static_cast<const uint16_t*>(a.local_keys) + b * a.lk_stride_b + kvh * a.lk_stride_h +
                         (c16 < kLocal ? c16 : 0) * a.lk_stride_l;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      const uint4 v = load16(lk + kb * 32 + g16 * 8);
      acc = Mma<BF16>::run(c16 < kLocal ? v : make_uint4(0u, 0u, 0u, 0u), qb[kb], acc);
    }
    f32x4_t sc[1];
    const uint8_t* mrow = a.local_mask + b * a.lm_stride_b + (row_ok ? c16 : 0) * a.lm_stride_r;
    // the four mask bytes read unconditionally (a clamped index): one round trip
    uint8_t mb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) mb[i] = mrow[(4 * g16 + i < kLocal ? 4 * g16 + i : 0) * a.lm_stride_l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool vis = row_ok && 4 * g16 + i < kLocal && mb[i] != 0;
      sc[0][i] = vis ? round_bf16(acc[i]) * a.softmax_scale * kLog2e : -__builtin_inff();
    }
    const uint16_t* lv = static_cast<const uint16_t*>(a.local_values) + b * a.lv_stride_b + kvh * a.lv_stride_h;
    fold<1>(st, sc, [&](int db, int) __attribute__((always_inline)) {
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int src = 4 * g16 + e;
        h[e] = src < kLocal ? lv[src * a.lv_stride_l + db * 16 + c16] : 0u;
      }
      return make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    });
  }

  float z = st.z;
  z = col4_sum(z);
  if (!row_ok) return;
  const float inv = 1.f / z;
  uint16_t* out = static_cast<uint16_t*>(a.output) + b * a.o_stride_b + head * a.o_stride_h + c16 * a.o_stride_r;
#pragma unroll
  for (int db = 0; db < kDB; ++db) {
    uint2 w;
    w.x = pack_bf16(st.o[db][0] * inv, st.o[db][1] * inv);
    w.y = pack_bf16(st.o[db][2] * inv, st.o[db][3] * inv);
    *reinterpret_cast<uint2*>(out + db * 16 + 4 * g16) = w;
  }
}

// ---------------------------------------------------------------------------
// Merge form (SRT/speculative/global16_raw256_draft_fused.py:72-312): the
// window attention arrives as (raw_output, raw_lse); the summary and local
// sources are normalised on their own and the three merged by their LSEs.
// One wave per query head; the KV head's local value rows are shared
// through LDS.

__device__ __forceinline__ float row_max4(float v) { return col4_max(v); }
__device__ __forceinline__ float row_sum4(float v) { return col4_sum(v); }

// kMaxThreads bounds the workgroup (64 x query heads per KV head); the
// smaller bounds leave the compiler registers for the loads issued up front.
// Up to 4 query heads per KV head the summary state rows (16 x 128 fp32 per
// head) go straight from memory to LDS (global_load_lds), so they hold no
// registers while the wave waits; the kernel then fits 4 waves per SIMD and
// 4,096 waves run in one residency round.
template <int kMaxThreads>
constexpr int merge_waves_per_simd() { return kMaxThreads <= 256 ? 4 : 1; }
template <int kMaxThreads>
__global__ __launch_bounds__(kMaxThreads, merge_waves_per_simd<kMaxThreads>()) void draft_merge_kernel(
    const ls_draft_attention_args a) {
  constexpr bool kStateLds = kMaxThreads <= 256;
  __shared__ float state_lds[kStateLds ? (kMaxThreads / kWave) * kGlobal * kD : 1];
  constexpr int kLVP = kD + 16;  // 16-bit elements per LDS local value row
  __shared__ __align__(16) uint16_t local_lds[16 * kLVP];
  const int64_t b = blockIdx.x / a.kv_heads;
  const int kvh = static_cast<int>(blockIdx.x % a.kv_heads);
  const int groups = a.q_heads / a.kv_heads;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g16 = lane >> 4, c16 = lane & 15;
  const int head = kvh * groups + wave;
  const bool row_ok = c16 < kRows;
  const int row = row_ok ? c16 : 0;   // lanes past the 7 query rows read row 0 and store nothing
  const float cap = a.softcap;
  auto finish = [&](float t) __attribute__((always_inline)) {
    float s = round_bf16(t) * a.softmax_scale;
    if (cap > 0.f) s = tanhf(s / cap) * cap;
    return s;
  };
  // the request's state slot: a scalar load, requested first (the state rows
  // wait for it, not for the vector loads below)
  const int64_t slot = load_uniform(a.state_slots + b);

  // Every load of the wave is issued here, before any of them is used, so
  // the wave waits for one memory round trip (plus the state slot) instead
  // of one per source.
  const int64_t tok = b * kRows + row;
  const float rlse = a.raw_lse[tok * a.rl_stride_t + head * a.rl_stride_h];
  uint2 rov[kDB];
  {
    const uint16_t* ro = static_cast<const uint16_t*>(a.raw_output) + tok * a.ro_stride_t + head * a.ro_stride_h;
#pragma unroll
    for (int db = 0; db < kDB; ++db) rov[db] = *reinterpret_cast<const uint2*>(ro + db * 16 + 4 * g16);
  }
  uint4 qb[kKB], gkb[kKB], lkb[kKB];
  {
    const uint16_t* q = static_cast<const uint16_t*>(a.query) + b * a.q_stride_b + head * a.q_stride_h +
                        row * a.q_stride_r;
    const uint16_t* gk = static_cast<const uint16_t*>(a.global_keys) + b * a.gk_stride_b + head * a.gk_stride_h +
                         c16 * a.gk_stride_g;
    const uint16_t* lk = static_cast<const uint16_t*>(a.local_keys) + b * a.lk_stride_b + kvh * a.lk_stride_h +
                         (c16 < kLocal ? c16 : 0) * a.lk_stride_l;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      qb[kb] = load16(q + kb * 32 + g16 * 8);
      gkb[kb] = load16(gk + kb * 32 + g16 * 8);
      lkb[kb] = load16(lk + kb * 32 + g16 * 8);
    }
  }
  // The 7 local value rows of the KV head are loaded once per workgroup, by
  // wave 0 (element j of a row by lane j % 64), and written to LDS before the
  // value products, which read them as the A operand with transposing reads.
  uint16_t lvh[2 * kLocal];
  if (wave == 0) {
    const uint16_t* lv = static_cast<const uint16_t*>(a.local_values) + b * a.lv_stride_b + kvh * a.lv_stride_h;
#pragma unroll
    for (int j = 0; j < 2 * kLocal; ++j) lvh[j] = lv[(j >> 1) * a.lv_stride_l + (j & 1) * kWave + lane];
  }
  // summary state rows 4*g16 .. 4*g16+3, column db*16 + c16 (fp32, rounded to bf16 as they are packed)
  float gvr[kStateLds ? 1 : kDB][4];
  float* sl = state_lds + (kStateLds ? wave * kGlobal * kD : 0);
  {
    const float* gv = a.global_values + slot * a.gv_stride_b + head * a.gv_stride_h;
    if constexpr (kStateLds) {
      // LDS word r * 128 + (col ^ 16 * (r >> 2)) holds (row r, col): the reads
      // below (rows 4*g16 + i, columns db*16 + c16) then fall on 64 distinct
      // banks.  Load j fills words j*64 .. j*64+63: row j/2, one half of it.
#pragma unroll
      for (int j = 0; j < kGlobal * kD / kWave; ++j) {
        const int r = j >> 1;
        const int col = (((j & 1) << 6) | lane) ^ (16 * (r >> 2));
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(gv + r * a.gv_stride_g + col),
                                         (__attribute__((address_space(3))) void*)(sl + j * kWave), 4, 0, 0);
      }
    } else {
      const float* g = gv + (4 * g16) * a.gv_stride_g + c16;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) gvr[db][i] = g[i * a.gv_stride_g + db * 16];
    }
  }
  // mask bytes read unconditionally (a clamped index), after the state rows
  // are requested: a wait for them then waits for no load still to be issued
  bool vis[4];
  {
    const uint8_t* mrow = a.local_mask + b * a.lm_stride_b + row * a.lm_stride_r;
    uint8_t mb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int src = 4 * g16 + i;
      mb[i] = mrow[(src < kLocal ? src : 0) * a.lm_stride_l];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) vis[i] = row_ok && 4 * g16 + i < kLocal && mb[i] != 0;
  }
  if (!row_ok) {
    // q rows past 7 take part in no product's output row, but the tile
    // products below read every lane's query operand: give them zeros
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) qb[kb] = make_uint4(0u, 0u, 0u, 0u);
  }

  // Both score tiles first, so the key and query operands are dead before
  // the value products need their registers.
  f32x4_t gacc = {0.f, 0.f, 0.f, 0.f}, lacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < kKB; ++kb) {
    gacc = Mma<BF16>::run(gkb[kb], qb[kb], gacc);
    lacc = Mma<BF16>::run(c16 < kLocal ? lkb[kb] : make_uint4(0u, 0u, 0u, 0u), qb[kb], lacc);
  }

  // ---- global: normalised over its 16 rows ----
  float gw4[4], gz, glse;
  {
    float sc[4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = finish(gacc[i]);
      mx = fmaxf(mx, sc[i]);
    }
    mx = row_max4(mx);
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gw4[i] = expf(sc[i] - mx);
      z += gw4[i];
    }
    gz = row_sum4(z);
    glse = mx + logf(gz);
  }

  // ---- local: normalised over its visible rows (none: left out) ----
  float lw4[4], lz, llse;
  bool has;
  {
    float sc[4];
    float mx = -__builtin_inff(), nvis = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = vis[i] ? finish(lacc[i]) : -__builtin_inff();
      mx = fmaxf(mx, sc[i]);
      nvis += vis[i] ? 1.f : 0.f;
    }
    mx = row_max4(mx);
    has = row_sum4(nvis) > 0.f;
    const float safe = has ? mx : 0.f;
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lw4[i] = vis[i] ? expf(sc[i] - safe) : 0.f;
      z += lw4[i];
    }
    z = row_sum4(z);
    lz = has ? z : 1.f;
    llse = has ? safe + logf(lz) : -__builtin_inff();
  }

  // ---- merge with the window attention by LSE, one 16-column block at a time ----
  const float mm = fmaxf(rlse, fmaxf(glse, llse));
  const float rw = expf(rlse - mm), gw = expf(glse - mm), lw = has ? expf(llse - mm) : 0.f;
  const float norm = rw + gw + lw;
  // weights of sources 4*g16 .. 4*g16+3 as the B operand (the second 16-source half of the 32-deep product is 0)
  const uint4 gpb = make_uint4(pack_bf16(gw4[0], gw4[1]), pack_bf16(gw4[2], gw4[3]), 0u, 0u);
  const uint4 lpb = make_uint4(pack_bf16(lw4[0], lw4[1]), pack_bf16(lw4[2], lw4[3]), 0u, 0u);
  // one reciprocal per normaliser: x * (1/z) is within one fp32 ulp of x / z, far inside the bf16 output
  const float inv_gz = 1.f / gz, inv_lz = 1.f / lz, inv_norm = 1.f / norm;
  // each source's weight in the merged row, its normaliser folded in
  const float cr = rw * inv_norm, cg = (inv_gz * gw) * inv_norm, cl = (inv_lz * lw) * inv_norm;
  uint16_t* out = static_cast<uint16_t*>(a.output) + b * a.o_stride_b + head * a.o_stride_h + row * a.o_stride_r;
  if (wave == 0) {
    // local rows 0..6 at pitch kLVP, rows 7..15 zero
#pragma unroll
    for (int j = 0; j < 2 * kLocal; ++j) local_lds[(j >> 1) * kLVP + (j & 1) * kWave + lane] = lvh[j];
#pragma unroll
    for (int r = kLocal; r < 16; ++r) reinterpret_cast<uint32_t*>(local_lds + r * kLVP)[lane] = 0u;
  }
  // the state rows' LDS writes are counted with the wave's other loads
  if constexpr (kStateLds) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int db = 0; db < kDB; ++db) {
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    float g4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      g4[i] = kStateLds ? sl[(4 * g16 + i) * kD + ((db * 16 + c16) ^ (16 * g16))] : gvr[kStateLds ? 0 : db][i];
    const f32x4_t go = Mma<BF16>::run(make_uint4(pack_bf16(g4[0], g4[1]), pack_bf16(g4[2], g4[3]), 0u, 0u), gpb, zero);
    // local rows 4*g16 + 0..3 (past 6 zero) of column db*16 + c16
    const uint2 lvr = lds_read_col4(local_lds + (4 * g16 + c16 / 4) * kLVP + db * 16 + 4 * (c16 % 4));
    const f32x4_t lo = Mma<BF16>::run(make_uint4(lvr.x, lvr.y, 0u, 0u), lpb, zero);
    const uint2 rv = rov[db];
    const float r4[4] = {bf16_lo(rv.x), bf16_hi(rv.x), bf16_lo(rv.y), bf16_hi(rv.y)};
    // the summary and local sums rounded to bf16 (two per conversion)
    const uint32_t g01 = pack_bf16(go[0], go[1]), g23 = pack_bf16(go[2], go[3]);
    const uint32_t l01 = pack_bf16(lo[0], lo[1]), l23 = pack_bf16(lo[2], lo[3]);
    const float g4r[4] = {bf16_lo(g01), bf16_hi(g01), bf16_lo(g23), bf16_hi(g23)};
    const float l4r[4] = {bf16_lo(l01), bf16_hi(l01), bf16_lo(l23), bf16_hi(l23)};
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = r4[i] * cr + g4r[i] * cg + l4r[i] * cl;
    uint2 w;
    w.x = pack_bf16(y[0], y[1]);
    w.y = pack_bf16(y[2], y[3]);
    if (row_ok) *reinterpret_cast<uint2*>(out + db * 16 + 4 * g16) = w;
  }
}

}  // namespace
}  // namespace ls

extern "C" int ls_draft_attention(const ls_draft_attention_args* args, void* stream) {
  using namespace ls;
  const char* what = "ls_draft_attention";
  LS_CHECK(args != nullptr, LS_ERR_VALUE, "%s: null argument block", what);
  const ls_draft_attention_args& a = *args;
  LS_CHECK(a.batch >= 0 && a.q_heads >= 1 && a.kv_heads >= 1 && a.q_heads % a.kv_heads == 0, LS_ERR_SHAPE,
           "%s: query heads must be a positive multiple of KV heads", what);
  LS_CHECK(a.q_heads / a.kv_heads <= 16, LS_ERR_SHAPE, "%s: at most 16 query heads per KV head", what);
  LS_CHECK(a.softmax_scale > 0.f, LS_ERR_VALUE, "%s: softmax_scale must be > 0", what);
  if (a.batch == 0) return LS_OK;
  LS_CHECK(a.query && a.global_keys && a.global_values && a.state_slots && a.local_keys && a.local_values &&
               a.local_mask && a.key_cache && a.value_cache && a.page_table && a.raw_lengths && a.output,
           LS_ERR_VALUE, "%s: every tensor is required", what);
  LS_CHECK(aligned16(a.query) && aligned16(a.global_keys) && aligned16(a.local_keys) && aligned16(a.key_cache) &&
               aligned16(a.value_cache) && aligned16(a.output) && a.q_stride_b % 8 == 0 && a.q_stride_h % 8 == 0 &&
               a.q_stride_r % 8 == 0 && a.gk_stride_b % 8 == 0 && a.gk_stride_h % 8 == 0 &&
               a.gk_stride_g % 8 == 0 && a.lk_stride_b % 8 == 0 && a.lk_stride_h % 8 == 0 &&
               a.lk_stride_l % 8 == 0 && a.kc_stride_s % 8 == 0 && a.kc_stride_h % 8 == 0 &&
               a.vc_stride_s % 8 == 0 && a.vc_stride_h % 8 == 0 && a.o_stride_b % 4 == 0 &&
               a.o_stride_h % 4 == 0 && a.o_stride_r % 4 == 0,
           LS_ERR_ALIGN, "%s: 16-bit rows must be 16-byte aligned (output rows 8-byte aligned)", what);
  const int64_t grid = a.batch * a.kv_heads;
  LS_CHECK(grid < (int64_t(1) << 31), LS_ERR_SHAPE, "%s: grid too large", what);
  const int groups = a.q_heads / a.kv_heads;
  const int threads = (groups < 4 ? 4 : groups) * kWave;
  hipStream_t st = static_cast<hipStream_t>(stream);
  draft_attention_kernel<<<dim3(static_cast<unsigned>(grid)), threads, kLds, st>>>(a, threads);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_draft_merge(const ls_draft_attention_args* args, void* stream) {
  using namespace ls;
  const char* what = "ls_draft_merge";
  LS_CHECK(args != nullptr, LS_ERR_VALUE, "%s: null argument block", what);
  const ls_draft_attention_args& a = *args;
  LS_CHECK(a.batch >= 0 && a.q_heads >= 1 && a.kv_heads >= 1 && a.q_heads % a.kv_heads == 0, LS_ERR_SHAPE,
           "%s: query heads must be a positive multiple of KV heads", what);
  LS_CHECK(a.q_heads / a.kv_heads <= 16, LS_ERR_SHAPE, "%s: at most 16 query heads per KV head", what);
  LS_CHECK(a.softmax_scale > 0.f && a.softcap >= 0.f, LS_ERR_VALUE, "%s: softmax_scale must be > 0, softcap >= 0",
           what);
  if (a.batch == 0) return LS_OK;
  LS_CHECK(a.query && a.global_keys && a.global_values && a.state_slots && a.local_keys && a.local_values &&
               a.local_mask && a.raw_output && a.raw_lse && a.output,
           LS_ERR_VALUE, "%s: every tensor is required", what);
  LS_CHECK(aligned16(a.query) && aligned16(a.global_keys) && aligned16(a.local_keys) && aligned16(a.output) &&
               (reinterpret_cast<uintptr_t>(a.raw_output) & 7u) == 0 && a.q_stride_b % 8 == 0 &&
               a.q_stride_h % 8 == 0 && a.q_stride_r % 8 == 0 && a.gk_stride_b % 8 == 0 &&
               a.gk_stride_h % 8 == 0 && a.gk_stride_g % 8 == 0 && a.lk_stride_b % 8 == 0 &&
               a.lk_stride_h % 8 == 0 && a.lk_stride_l % 8 == 0 && a.ro_stride_t % 4 == 0 &&
               a.ro_stride_h % 4 == 0 && a.o_stride_b % 4 == 0 && a.o_stride_h % 4 == 0 && a.o_stride_r % 4 == 0,
           LS_ERR_ALIGN, "%s: 16-bit rows must be 16-byte aligned (window and output rows 8-byte aligned)", what);
  const int64_t grid = a.batch * a.kv_heads;
  LS_CHECK(grid < (int64_t(1) << 31), LS_ERR_SHAPE, "%s: grid too large", what);
  const int threads = (a.q_heads / a.kv_heads) * kWave;
  const dim3 g(static_cast<unsigned>(grid));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (threads <= 256)
    draft_merge_kernel<256><<<g, threads, 0, st>>>(a);
  else if (threads <= 512)
    draft_merge_kernel<512><<<g, threads, 0, st>>>(a);
  else
    draft_merge_kernel<1024><<<g, threads, 0, st>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}
