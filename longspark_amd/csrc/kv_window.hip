// Drafter-view refresh, recent window: page tables and KV copies.
//
//   raw page table   page_table[b, i] = req_to_token[slot_b, seq_b - raw_b + i]
//                    for i < raw_b = min(seq_b, window), else 0
//                    (vendor/sglang/python/sglang/srt/speculative/
//                    global16_raw256_draft_fused.py:35-65, 372-413)
//   ring page table  pages[b, i] = slot_b * window + (len_b - raw_b + i) mod window
//                    (src/longspark/engine/draft.py:14-21)
//   window gather    out[b, l, kv, h, i, :] = pool_kv[l][loc(b, i), h, :] for the
//                    last raw_b positions, zero beyond; loc(b, i) through a paged
//                    table of any page size (src/longspark/engine/target.py:213-228
//                    export, generalised from page size 1 to paged pools)
//   ring append      ring_kv[l][slot_b * window + (prev_b + j) mod window] =
//                    src_kv[l][row] for each request's accepted rows
//                    (src/longspark/engine/draft.py:207-212, 255-259, fused with
//                    the target-side row export of target.py:213-228)
//
// All copies move 16-byte vectors; stores of the gathered view are
// non-temporal (the view is consumed by another kernel, not re-read here).
#include "common.h"

namespace ls {
namespace {

constexpr int kGT = 256;       // threads per workgroup
constexpr int kChunk = 8;      // window tokens per workgroup

template <typename T>
__device__ __forceinline__ int64_t ld_index(const void* p, int64_t i) {
  return static_cast<int64_t>(static_cast<const T*>(p)[i]);
}
__device__ __forceinline__ int64_t ld_any(const void* p, int dtype, int64_t i) {
  return dtype == LS_I64 ? ld_index<int64_t>(p, i) : ld_index<int32_t>(p, i);
}

__global__ __launch_bounds__(kGT) void raw_page_table_kernel(const int32_t* __restrict__ rtt, int64_t rtt_sb,
                                                             int64_t rtt_st, const void* slots, int slots_dtype,
                                                             const void* seq_lens, int seq_dtype, int window,
                                                             int32_t* __restrict__ table, int64_t table_sb,
                                                             int32_t* __restrict__ raw_out) {
  const int64_t b = blockIdx.x;
  const int64_t slot = ld_any(slots, slots_dtype, b);
  const int64_t seq = ld_any(seq_lens, seq_dtype, b);
  const int64_t raw = seq < window ? seq : window;
  for (int i = threadIdx.x; i < window; i += kGT) {
    int32_t v = 0;
    if (i < raw) v = rtt[slot * rtt_sb + (seq - raw + i) * rtt_st];
    table[b * table_sb + i] = v;
  }
  if (threadIdx.x == 0 && raw_out) raw_out[b] = static_cast<int32_t>(raw);
}

__global__ __launch_bounds__(kGT) void ring_page_table_kernel(const void* slots, int slots_dtype,
                                                              const void* lengths, int len_dtype, int window,
                                                              int32_t* __restrict__ pages, int64_t pages_sb,
                                                              int32_t* __restrict__ raw_out) {
  const int64_t b = blockIdx.x;
  const int64_t slot = ld_any(slots, slots_dtype, b);
  const int64_t len = ld_any(lengths, len_dtype, b);
  const int64_t raw = len < window ? len : window;
  for (int i = threadIdx.x; i < window; i += kGT) {
    int64_t pos = (len - raw + i) % window;
    if (pos < 0) pos += window;
    pages[b * pages_sb + i] = static_cast<int32_t>(slot * window + pos);
  }
  if (threadIdx.x == 0 && raw_out) raw_out[b] = static_cast<int32_t>(raw);
}

struct GatherArgs {
  const uint64_t* k_layers;  // device array of layer base addresses
  const uint64_t* v_layers;
  int n_layers;
  int esize;                 // element size in bytes
  int64_t token_stride;      // elements between consecutive token rows of a layer
  int64_t head_stride;       // elements between heads within a token row
  int heads, head_dim;
  const int32_t* table;      // page ids
  int64_t table_sb;
  const void* table_rows;    // optional request -> table row
  int table_rows_dtype;
  int page_size;
  const void* seq_lens;
  int seq_dtype;
  int window;
  char* out;
  int64_t osb, osl, oskv, osh, osw;  // output strides in elements
  int32_t* raw_out;
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte non-temporal load through a pointer read from a layer table, marked
// global so the compiler emits a global (not flat) load.
__device__ __forceinline__ uint4 load16_global_stream(const char* p) {
  const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One workgroup: kChunk window tokens of one (request, layer), keys and
// values.  The chunk's physical rows are resolved once into LDS (for both),
// then every thread copies 16-byte vectors: (K or V, head h, window token i,
// vector c) with c fastest, then i, so a wave writes contiguous runs of one
// head's output rows.  Each thread issues its kU loads, then its kU stores,
// and the workgroup ends: a second round of loads in the same thread would
// wait for the first round's stores (one counter covers both), so more,
// shorter workgroups stream faster (8 tokens x K and V: 2,048 vectors per
// workgroup, 61 registers, 8 waves per SIMD).
// kVph = 16-byte vectors per head row when it is a power of two the kernel
// was built for (index math by shifts), 0 = any (runtime division).
template <int kVph>
__global__ __launch_bounds__(kGT) void window_gather_kernel(GatherArgs a) {
  __shared__ int64_t locs[kChunk];
  const int chunks = (a.window + kChunk - 1) / kChunk;
  int64_t w = blockIdx.x;
  const int chunk = static_cast<int>(w % chunks);
  w /= chunks;
  const int layer = static_cast<int>(w % a.n_layers);
  const int64_t b = w / a.n_layers;
  const int64_t seq = ld_any(a.seq_lens, a.seq_dtype, b);
  const int64_t raw = seq < a.window ? seq : a.window;
  const int i0 = chunk * kChunk;
  if (threadIdx.x < kChunk) {
    const int i = i0 + threadIdx.x;
    int64_t loc = -1;
    if (i < raw) {
      const int64_t trow = a.table_rows ? ld_any(a.table_rows, a.table_rows_dtype, b) : b;
      const int64_t pos = seq - raw + i;
      const int64_t page = a.table[trow * a.table_sb + pos / a.page_size];
      loc = page * a.page_size + pos % a.page_size;
    }
    locs[threadIdx.x] = loc;
  }
  __syncthreads();
  const char* srck = reinterpret_cast<const char*>(a.k_layers[layer]);
  const char* srcv = reinterpret_cast<const char*>(a.v_layers[layer]);
  char* dst = a.out + (b * a.osb + layer * a.osl) * a.esize;
  const int vph = kVph ? kVph : a.head_dim * a.esize / 16;
  const int ntok = min(kChunk, a.window - i0);
  const int per_head = kChunk * vph;   // tokens past ntok are skipped
  const int per_kv = a.heads * per_head;
  const int total = 2 * per_kv;
  constexpr int kU = 8;
  for (int j0 = threadIdx.x; j0 < total; j0 += kGT * kU) {
    uint4 v[kU];
    char* dp[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = j0 + u * kGT;
      const int kv = j >= per_kv;
      const int jh = j - kv * per_kv;
      const int h = jh / per_head;
      const int r = jh - h * per_head;
      const int ti = r / vph;
      const int c = r - ti * vph;
      const bool live = j < total && ti < ntok;
      const int64_t loc = live ? locs[ti] : -1;
      dp[u] = live ? dst + (kv * a.oskv + h * a.osh + static_cast<int64_t>(i0 + ti) * a.osw) * a.esize + c * 16 : nullptr;
      // rows past raw and dead lanes read head 0 of row 0 (in bounds); rows
      // past raw store zeros, dead lanes store nothing
      v[u] = load16_global_stream((kv ? srcv : srck) + ((loc < 0 ? 0 : loc) * a.token_stride + (live ? h : 0) * a.head_stride) *
                                            a.esize + c * 16);
      if (loc < 0) v[u] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (dp[u]) store16_stream(dp[u], v[u]);
  }
  if (a.raw_out && threadIdx.x == 0 && layer == 0 && chunk == 0) a.raw_out[b] = static_cast<int32_t>(raw);
}

struct AppendArgs {
  const uint64_t* src_k;
  const uint64_t* src_v;
  const uint64_t* dst_k;
  const uint64_t* dst_v;
  int n_layers;
  int64_t row_bytes;          // bytes of one token row (multiple of 16)
  int64_t src_row_stride;     // bytes between source rows
  int64_t dst_row_stride;     // bytes between ring rows
  const void* src_locs;       // optional source row per packed row
  int src_locs_dtype;
  const int32_t* slots;
  const int32_t* prev;
  const int32_t* counts;
  int window;
};

// One workgroup per (request, layer, K or V): copy the request's rows.
__global__ __launch_bounds__(kGT) void ring_append_kernel(AppendArgs a) {
  int64_t w = blockIdx.x;
  const int kv = static_cast<int>(w % 2);
  w /= 2;
  const int layer = static_cast<int>(w % a.n_layers);
  const int64_t b = w / a.n_layers;
  int64_t off = 0;
  for (int64_t r = 0; r < b; ++r) off += a.counts[r];
  const int n = a.counts[b];
  const int64_t slot = a.slots[b];
  const int64_t prev = a.prev[b];
  const char* src = reinterpret_cast<const char*>((kv ? a.src_v : a.src_k)[layer]);
  char* dst = reinterpret_cast<char*>((kv ? a.dst_v : a.dst_k)[layer]);
  const int64_t vpr = a.row_bytes / 16;
  for (int64_t j = threadIdx.x; j < n * vpr; j += kGT) {
    const int64_t r = j / vpr, c = j % vpr;
    const int64_t srow = a.src_locs ? ld_any(a.src_locs, a.src_locs_dtype, off + r) : off + r;
    const int64_t drow = slot * a.window + (prev + r) % a.window;
    const uint4 v = load16(src + srow * a.src_row_stride + c * 16);
    *reinterpret_cast<uint4*>(dst + drow * a.dst_row_stride + c * 16) = v;
  }
}

int esize_of(int dtype) {
  switch (dtype) {
    case LS_F32: return 4;
    case LS_BF16: return 2;
    case LS_F16: return 2;
    default: return 0;
  }
}

}  // namespace
}  // namespace ls

extern "C" int ls_raw_page_table(const int32_t* req_to_token, int64_t rtt_stride_b, int64_t rtt_stride_t,
                                 const void* req_pool_indices, int32_t slots_dtype, const void* seq_lens,
                                 int32_t seq_lens_dtype, int64_t batch, int32_t window, int32_t* page_table,
                                 int64_t page_table_stride, int32_t* raw_lengths, void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && window > 0, LS_ERR_SHAPE, "ls_raw_page_table: need batch >= 0 and window > 0");
  LS_CHECK(slots_dtype == LS_I32 || slots_dtype == LS_I64, LS_ERR_DTYPE, "ls_raw_page_table: slots int32/int64");
  LS_CHECK(seq_lens_dtype == LS_I32 || seq_lens_dtype == LS_I64, LS_ERR_DTYPE, "ls_raw_page_table: seq_lens int32/int64");
  LS_CHECK(page_table_stride >= window, LS_ERR_SHAPE, "ls_raw_page_table: page table stride < window");
  if (batch == 0) return LS_OK;
  raw_page_table_kernel<<<dim3(static_cast<unsigned>(batch)), kGT, 0, static_cast<hipStream_t>(stream)>>>(
      req_to_token, rtt_stride_b, rtt_stride_t, req_pool_indices, slots_dtype, seq_lens, seq_lens_dtype, window,
      page_table, page_table_stride, raw_lengths);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_ring_page_table(const void* slots, int32_t slots_dtype, const void* lengths, int32_t lengths_dtype,
                                  int64_t batch, int32_t window, int32_t* pages, int64_t pages_stride,
                                  int32_t* raw_lengths, void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && window > 0, LS_ERR_SHAPE, "ls_ring_page_table: need batch >= 0 and window > 0");
  LS_CHECK((slots_dtype == LS_I32 || slots_dtype == LS_I64) && (lengths_dtype == LS_I32 || lengths_dtype == LS_I64),
           LS_ERR_DTYPE, "ls_ring_page_table: slots and lengths must be int32/int64");
  LS_CHECK(pages_stride >= window, LS_ERR_SHAPE, "ls_ring_page_table: pages stride < window");
  if (batch == 0) return LS_OK;
  ring_page_table_kernel<<<dim3(static_cast<unsigned>(batch)), kGT, 0, static_cast<hipStream_t>(stream)>>>(
      slots, slots_dtype, lengths, lengths_dtype, window, pages, pages_stride, raw_lengths);
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_kv_window_gather(const uint64_t* k_layers, const uint64_t* v_layers, int32_t n_layers,
                                   int32_t dtype, int64_t token_stride, int64_t head_stride, int32_t heads,
                                   int32_t head_dim, const int32_t* page_table, int64_t page_table_stride,
                                   const void* table_rows, int32_t table_rows_dtype, int32_t page_size,
                                   const void* seq_lens, int32_t seq_lens_dtype, int64_t batch, int32_t window,
                                   void* out, int64_t out_stride_b, int64_t out_stride_l, int64_t out_stride_kv,
                                   int64_t out_stride_h, int64_t out_stride_w, int32_t* raw_lengths,
                                   void* stream) {
  using namespace ls;
  const int es = esize_of(dtype);
  LS_CHECK(es > 0, LS_ERR_DTYPE, "ls_kv_window_gather: dtype must be bf16, fp16 or fp32");
  LS_CHECK(batch >= 0 && n_layers > 0 && heads > 0 && head_dim > 0 && window > 0 && page_size > 0,
           LS_ERR_SHAPE, "ls_kv_window_gather: sizes must be positive");
  LS_CHECK((head_dim * es) % 16 == 0 && (head_stride * es) % 16 == 0 && (token_stride * es) % 16 == 0 &&
               (out_stride_w * es) % 16 == 0 && (out_stride_h * es) % 16 == 0 && (out_stride_kv * es) % 16 == 0 &&
               (out_stride_l * es) % 16 == 0 && (out_stride_b * es) % 16 == 0 && aligned16(out),
           LS_ERR_ALIGN, "ls_kv_window_gather: head rows, strides and output must be 16-byte aligned");
  LS_CHECK(seq_lens_dtype == LS_I32 || seq_lens_dtype == LS_I64, LS_ERR_DTYPE, "ls_kv_window_gather: seq_lens dtype");
  LS_CHECK(!table_rows || table_rows_dtype == LS_I32 || table_rows_dtype == LS_I64, LS_ERR_DTYPE,
           "ls_kv_window_gather: table_rows dtype");
  LS_CHECK(k_layers && v_layers && page_table && seq_lens && out, LS_ERR_VALUE, "ls_kv_window_gather: null pointer");
  if (batch == 0) return LS_OK;
  GatherArgs a;
  a.k_layers = k_layers; a.v_layers = v_layers; a.n_layers = n_layers; a.esize = es;
  a.token_stride = token_stride; a.head_stride = head_stride; a.heads = heads; a.head_dim = head_dim;
  a.table = page_table; a.table_sb = page_table_stride; a.table_rows = table_rows;
  a.table_rows_dtype = table_rows_dtype; a.page_size = page_size; a.seq_lens = seq_lens;
  a.seq_dtype = seq_lens_dtype; a.window = window; a.out = static_cast<char*>(out);
  a.osb = out_stride_b; a.osl = out_stride_l; a.oskv = out_stride_kv; a.osh = out_stride_h; a.osw = out_stride_w;
  a.raw_out = raw_lengths;
  const int64_t chunks = (window + kChunk - 1) / kChunk;
  const int64_t grid = batch * n_layers * chunks;
  LS_CHECK(grid < (int64_t(1) << 31), LS_ERR_SHAPE, "ls_kv_window_gather: grid too large");
  const dim3 g(static_cast<unsigned>(grid));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (head_dim * es / 16) {
    case 8: window_gather_kernel<8><<<g, kGT, 0, st>>>(a); break;
    case 16: window_gather_kernel<16><<<g, kGT, 0, st>>>(a); break;
    case 32: window_gather_kernel<32><<<g, kGT, 0, st>>>(a); break;
    default: window_gather_kernel<0><<<g, kGT, 0, st>>>(a); break;
  }
  LS_LAUNCH_CHECK();
  return LS_OK;
}

extern "C" int ls_ring_append(const uint64_t* src_k_layers, const uint64_t* src_v_layers, const uint64_t* dst_k_layers,
                              const uint64_t* dst_v_layers, int32_t n_layers, int64_t row_bytes,
                              int64_t src_row_stride_bytes, int64_t dst_row_stride_bytes, const void* src_locs,
                              int32_t src_locs_dtype, const int32_t* slots, const int32_t* prev_lengths,
                              const int32_t* counts, int64_t batch, int32_t window, void* stream) {
  using namespace ls;
  LS_CHECK(batch >= 0 && n_layers > 0 && window > 0 && row_bytes > 0, LS_ERR_SHAPE, "ls_ring_append: bad sizes");
  LS_CHECK(row_bytes % 16 == 0 && src_row_stride_bytes % 16 == 0 && dst_row_stride_bytes % 16 == 0, LS_ERR_ALIGN,
           "ls_ring_append: rows and strides must be multiples of 16 bytes");
  LS_CHECK(!src_locs || src_locs_dtype == LS_I32 || src_locs_dtype == LS_I64, LS_ERR_DTYPE,
           "ls_ring_append: src_locs must be int32/int64");
  LS_CHECK(src_k_layers && src_v_layers && dst_k_layers && dst_v_layers && slots && prev_lengths && counts,
           LS_ERR_VALUE, "ls_ring_append: null pointer");
  if (batch == 0) return LS_OK;
  AppendArgs a;
  a.src_k = src_k_layers; a.src_v = src_v_layers; a.dst_k = dst_k_layers; a.dst_v = dst_v_layers;
  a.n_layers = n_layers; a.row_bytes = row_bytes; a.src_row_stride = src_row_stride_bytes;
  a.dst_row_stride = dst_row_stride_bytes; a.src_locs = src_locs; a.src_locs_dtype = src_locs_dtype;
  a.slots = slots; a.prev = prev_lengths; a.counts = counts; a.window = window;
  const int64_t grid = batch * n_layers * 2;
  ring_append_kernel<<<dim3(static_cast<unsigned>(grid)), kGT, 0, static_cast<hipStream_t>(stream)>>>(a);
  LS_LAUNCH_CHECK();
  return LS_OK;
}
