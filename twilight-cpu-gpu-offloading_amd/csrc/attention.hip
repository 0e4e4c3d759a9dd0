// Sparse GQA decode attention over selected rows: split-K flash-decode with a
// fused last-block combine.
//
// Reference call surface: _flash_attention_varlen_forward (mp.py:21-52) as
// used by the GQA-group decode branch (mp.py:239-279: G sequences of one
// query token x R heads against one KV head), the layer-flat branch
// (mp.py:283-321) and the per-head reference path (mp.py:424-452).  The
// semantics are softmax(q.k * scale) v over every key of the sequence (causal
// with q_len 1 sees all keys), fp32 accumulation, output in the input dtype.
//
// The kernel is written for latency: a decode layer moves tens of MB, so it
// completes in a handful of memory round trips and every round trip counts.
//   round trip 1: row count, the wavefront's row indices and masks, the
//                 group's queries -- all independent loads;
//   round trip 2: the K and V rows (16 bytes per lane, 8 rows per lane in
//                 flight), read straight from the cache by index;
//   then the block's partial (m, l, o) goes to the workspace and a second,
//   small launch merges the partials of every group that spans more than
//   one block (one round trip: all chunks' loads are issued at once).
// Every load is unconditional (clamped addresses, results masked) so the
// compiler issues them back to back instead of one branch and wait per load.
//
// Work split: block = (group g, chunk of rows); 4 wavefronts; D/8 lanes share
// a row and each lane owns 8 consecutive channels (one 16-byte load per row).
// The R query heads of the group share every K/V load.
#pragma clang fp contract(off)

#include <type_traits>

#include "tw_common.h"
#include "union_record.h"

namespace tw {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxChunks = 128;
constexpr float kLog2e = 1.4426950408889634f;

// Row loads in flight per lane: fewer when the registers go to many heads or
// to 32-bit values.
constexpr int steps_for(int elem_bytes, int rmax) { return (elem_bytes == 2 && rmax <= 4) ? 8 : 4; }

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  int G, R, D;
  const int32_t* rows;
  const uint8_t* masks;
  const int32_t* counts;
  int64_t rows_stride;
  int64_t entry_stride;
  const int32_t* cu_k;
  int Hk;
  int window_left;
  const void* cur_k;
  const void* cur_v;
  float scale_log2;
  void* out;
  // Page-plan mode: group g's rows are [0, sink_end) ++ the union pages
  // plan_pages[g][0 .. plan_counts[g]) expanded to bs rows each ++
  // [recent_start, length) ++ append_position (if >= 0).
  const int32_t* plan_pages;
  const uint8_t* plan_masks;
  const int32_t* plan_counts;
  int64_t plan_stride;
  int sink, recent, bs, length, append_position;
  // Page-plan mode with cur_k/cur_v: the decode token is attended from
  // cur_k/cur_v and also appended to the cache at append_position.
  void* k_append;
  void* v_append;
  float* part_ml;           // [G][max_chunks][R][2]  (m, l)
  float* part_o;            // [G][max_chunks][R][D]
  int32_t* union_sizes;    // [G] bitmap mode: each group's union pages, from the split-K kernel to the merge
  int max_chunks;
  int iters;                // row batches per block
  int max_rows;             // bound on every group's row count
  int phase;                // host side: 1 split-K partials, 2 merge, 3 (or 0) both
  // Page-tile kernel (16-row pages): window geometry computed on the host.
  int t_sink_tiles;         // ceil(sink_end / 16)
  int t_sink_end;
  int t_recent_start;
  int t_n_recent;           // recent rows: [recent_start, length)
  int t_has_dec;            // a decode token follows the recent rows
  int t_run;                // t_n_recent + t_has_dec
  int t_run_tiles;          // ceil(t_run / 16)
  int t_nu_cap;             // union pages the launch covers at most
  int t_per_chunk;          // tiles per chunk (waves x tiles per batch x batches)
  // Ragged page-tile launches (nullable): group g has lengths[g] tokens, its
  // window follows from it and the decode token is its row lengths[g]
  // (appended there when ragged_append is set).
  const int32_t* lengths;
  int ragged_append;
  // Resident page cache (page-tile kernel, nullable): group g keeps the K/V
  // of its union pages in HBM, res_k/res_v [G][2][res_slots][16][D] (two
  // buffers alternating with the length's parity), and res_map [G]
  // [res_map_pages] = (length << 32) | slot of the step that last stored
  // each page.  res_stats [G][2] accumulates (hit pages, union pages).
  // Over a union record (Twilight) the cache is row-granular: res_map =
  // (length << 32) | (the page's kept rows << 16) | slot, a kept row is read
  // from HBM when the previous step kept it too, and res_stats counts rows
  // (hit rows, union rows).
  void* res_k;
  void* res_v;
  int64_t* res_map;
  int res_slots;
  int res_map_pages;
  unsigned long long* res_stats;
  // Resident windows (with the resident page cache, nullable): res_win_k /
  // res_win_v [G][win_rows][D] keep group g's sink rows at [0, sink) and its
  // latest ring_rows rows (a power of two >= recent) at sink + (row &
  // (ring_rows - 1)); res_win_state [G][2] = (the history length the ring
  // serves: it holds rows [length - ring_rows + 1, length); 1 when the sink
  // rows are stored too).  A launch reads the windows from HBM only when the
  // ring serves its length (the previous launch was at length - 1 with a
  // decode row), stores the window rows it read from the slab otherwise, and
  // stores its decode row into the ring every time.  The recent window holds
  // recent - 1 history rows, so the decode row's slot is never one this
  // launch reads.
  void* res_win_k;
  void* res_win_v;
  int32_t* res_win_state;
  int win_rows, ring_rows;
  // Page metadata of the appended row (page-tile kernel, nullable): when the
  // row completes page p of its entry (row - sink + 1 a multiple of 16),
  // meta_min/meta_max [G][meta_stride] get that page's per-channel min/max
  // at p * D (p < meta_pages).
  void* meta_min;
  void* meta_max;
  int64_t meta_stride;
  int meta_pages;
  // page-tile kernel: K and V are device memory (read with the streaming hint)
  int kv_stream;
  // Rows mode with the append (16-bit, D = 128, nullable): the appended
  // row's INT4 code, scale and minimum at row (g * meta_qstride + row) of
  // meta_packed ([.][D/2] bytes) / meta_qscale / meta_qmin; the page it
  // completes as meta_min / meta_max above.
  uint8_t* meta_packed;
  void* meta_qscale;
  void* meta_qmin;
  int64_t meta_qstride;
  // Page-tile kernel, Twilight union (nullable): page_rows[g][u] (plan_stride
  // apart) has bit i set when row i of union page u is kept; every head
  // attends the kept rows, and rows not kept are neither read nor attended.
  const uint32_t* page_rows;
  // Page-tile kernel, selection bitmaps instead of a union plan (nullable):
  // bit p of sel_bits + (g*R + r) * bits_stride (32-bit words) is set when
  // head r of group g selected page p; bits_w64 64-bit words per row.  The
  // union pages are the OR of the R rows, ranked in ascending page order.
  const uint32_t* sel_bits;
  int64_t bits_stride;
  int bits_w64;
  // Page-tile kernel, Twilight union record (union_record.h) instead
  // (union_rec set): sel_bits + g * bits_stride is group g's record, its one
  // bitmap row the union pages and its row masks, from 32-bit word mask_off
  // on (mask_w4 16-byte units), the kept rows of each; every head attends
  // every kept row.
  int union_rec;
  int mask_off;
  int mask_w4;
};

// 8 consecutive channels of one row.
template <typename S>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  uint4 w;
  __device__ __forceinline__ void load(const uint16_t* p) { w = *reinterpret_cast<const uint4*>(p); }
  template <typename DT>
  __device__ __forceinline__ void to_float(float (&f)[8]) const {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = to_f32(DT{}, static_cast<uint16_t>(a[i] & 0xffffu));
      f[2 * i + 1] = to_f32(DT{}, static_cast<uint16_t>(a[i] >> 16));
    }
  }
};
template <>
struct Vec8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  template <typename DT>
  __device__ __forceinline__ void to_float(float (&f)[8]) const {
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

// DPP lane permutations (GFX9 encodings) for sums inside lane groups.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xb1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4e;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// Sum over each aligned group of N lanes (N = 1..64, power of two); every
// lane of the group receives the sum.
template <int N>
__device__ __forceinline__ float row_group_sum(float x) {
  if constexpr (N >= 2) x += dpp<kQuadXor1>(x);
  if constexpr (N >= 4) x += dpp<kQuadXor2>(x);
  if constexpr (N >= 8) x += dpp<kRowHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kRowMirror>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

// exp2(x - m), with a masked value (x = -inf) giving 0 even when m is -inf too.
__device__ __forceinline__ float exp2_rel(float x, float m) {
  return x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x - m);
}

// Row sources: an explicit row list, a varlen sequence, or a page plan.
constexpr int kModeRows = 0;
constexpr int kModeVarlen = 1;
constexpr int kModePages = 2;

// Geometry of group g's rows (identical in every block of the group).
struct GroupRows {
  int n_list;        // rows from the list / sequence / plan
  int n_rows;        // + the decode token
  int64_t base;      // element offset of the group's row 0 (position 0)
  int64_t stride;    // elements between positions
  int win_start;     // varlen: first visible position
  // page plan
  int n_pages, sink_end, page_end, recent_start, recent_end;
};

template <int MODE>
__device__ __forceinline__ GroupRows group_rows(const AttnArgs& a, int g, int D) {
  GroupRows gr;
  gr.n_pages = gr.sink_end = gr.page_end = gr.recent_start = gr.recent_end = 0;
  if (MODE == kModePages) {
    int nu = a.plan_counts[g];
    nu = nu < 0 ? 0 : (nu > a.plan_stride ? static_cast<int>(a.plan_stride) : nu);
    const int sink_end = a.sink < a.length ? a.sink : a.length;
    const int hist_recent = a.recent - 1 > 0 ? a.recent - 1 : 0;
    const int recent_start = (a.length - hist_recent) > sink_end ? (a.length - hist_recent) : sink_end;
    gr.n_pages = nu;
    gr.sink_end = sink_end;
    gr.page_end = sink_end + nu * a.bs;
    gr.recent_start = recent_start;
    gr.recent_end = gr.page_end + (a.length - recent_start);
    // the decode token comes from the cache row append_position, or from
    // cur_k/cur_v when they are given
    const int n = gr.recent_end + (a.append_position >= 0 && a.cur_k == nullptr ? 1 : 0);
    const int cap = a.max_rows - (a.cur_k != nullptr ? 1 : 0);  // max_rows counts the decode token
    gr.n_list = n > cap ? (cap > 0 ? cap : 0) : n;
    gr.base = static_cast<int64_t>(g) * a.entry_stride * D;
    gr.stride = D;
    gr.win_start = 0;
  } else if (MODE == kModeRows) {
    int n = a.counts[g];
    gr.n_list = n < 0 ? 0 : (n > a.max_rows ? a.max_rows : n);
    gr.base = static_cast<int64_t>(g) * a.entry_stride * D;
    gr.stride = D;
    gr.win_start = 0;
  } else {
    const int b = g / a.Hk;
    const int h = g - b * a.Hk;
    const int s0 = a.cu_k[b];
    int n = a.cu_k[b + 1] - s0;
    int ws = 0;
    if (a.window_left >= 0 && n > a.window_left + 1) {
      ws = n - (a.window_left + 1);
      n = a.window_left + 1;
    }
    gr.n_list = n < 0 ? 0 : (n > a.max_rows ? a.max_rows : n);
    gr.stride = static_cast<int64_t>(a.Hk) * D;
    gr.base = static_cast<int64_t>(s0) * gr.stride + static_cast<int64_t>(h) * D;
    gr.win_start = ws;
  }
  gr.n_rows = gr.n_list + (a.cur_k != nullptr ? 1 : 0);
  return gr;
}

// Page-tile mode (decode_attn_tiles): chunks count 16-row tiles.
constexpr int kModeTiles = 3;

// Host side: the metadata the rows-mode append updates (complete_row_meta).
struct RowMeta {
  int sink;
  void* page_min;
  void* page_max;
  int64_t page_stride;
  int pages;
  uint8_t* packed;
  void* qscale;
  void* qmin;
  int64_t qstride;
};

// The row the decode token of group g is appended at: append_position, or in
// rows mode with per-group lengths, lengths[g] (out of range: none).
template <int MODE>
__device__ __forceinline__ int decode_row_position(const AttnArgs& a, int g) {
  if (MODE != kModeRows || a.lengths == nullptr) return a.append_position;
  const int p = a.lengths[g];
  return (p >= 0 && p < a.entry_stride) ? p : -1;
}

// The min/max of the 16-row page the appended row `position` of group g
// completes, by wave 0 of the block: lane l owns channels 2l and 2l + 1 of
// all 16 rows (one 4-byte load per row, all in flight together), compared as
// order keys; a NaN in a channel makes that channel's min and max the
// canonical NaN -- the page rule of the metadata build, so the result equals
// a rebuild.  The appended row is read from cur_k when given.
template <typename DT>
__device__ __forceinline__ void complete_page_meta(const AttnArgs& a, int g, int position) {
  using S = typename DT::storage;
  constexpr int D = 128, BS = 16;
  if (a.meta_min == nullptr || position < a.sink || threadIdx.x >= kWave) return;
  const int j = position - a.sink;
  if ((j + 1) % BS != 0 || j / BS >= a.meta_pages) return;
  const int page = j / BS;
  const int lane = static_cast<int>(threadIdx.x);
  const S* kg = static_cast<const S*>(a.k) + static_cast<int64_t>(g) * a.entry_stride * D;
  const S* cur = a.cur_k != nullptr ? static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D : nullptr;
  uint32_t v[BS];
#pragma unroll
  for (int i = 0; i < BS; ++i) {
    const int t = a.sink + page * BS + i;
    const S* row = (t == position && cur != nullptr) ? cur : kg + static_cast<int64_t>(t) * D;
    v[i] = *reinterpret_cast<const uint32_t*>(row + 2 * lane);
  }
  uint32_t kmin[2] = {0xffffffffu, 0xffffffffu}, kmax[2] = {0u, 0u};
  bool nan[2] = {false, false};
#pragma unroll
  for (int i = 0; i < BS; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const S x = static_cast<S>(h ? (v[i] >> 16) : (v[i] & 0xffffu));
      const uint32_t k = order_key(DT{}, x);
      nan[h] |= is_nan(DT{}, x);
      kmin[h] = k < kmin[h] ? k : kmin[h];
      kmax[h] = k > kmax[h] ? k : kmax[h];
    }
  }
  const int64_t at = static_cast<int64_t>(g) * a.meta_stride + static_cast<int64_t>(page) * D + 2 * lane;
  S* mn = static_cast<S*>(a.meta_min) + at;
  S* mx = static_cast<S*>(a.meta_max) + at;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    mn[h] = nan[h] ? canonical_nan(DT{}) : from_order_key(DT{}, kmin[h]);
    mx[h] = nan[h] ? canonical_nan(DT{}) : from_order_key(DT{}, kmax[h]);
  }
}

// Rows mode: the metadata update of the appended row `position` of group g
// by wave 0 of the block (16-bit keys, D = 128, read from cur_k): its INT4
// code -- row min/max as order keys reduced over the wavefront, scale and
// codes as the metadata build computes them -- and the page it completes.
template <typename DT>
__device__ __forceinline__ void complete_row_meta(const AttnArgs& a, int g, int position) {
  if constexpr (sizeof(typename DT::storage) != 2) {
    return;
  } else {
    using S = typename DT::storage;
    if (position < 0 || threadIdx.x >= kWave || a.cur_k == nullptr) return;
    if (a.meta_packed != nullptr) {
      const int lane = static_cast<int>(threadIdx.x);
      const S* cur = static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * 128;
      const uint32_t w = *reinterpret_cast<const uint32_t*>(cur + 2 * lane);
      const S x0 = static_cast<S>(w & 0xffffu), x1 = static_cast<S>(w >> 16);
      const uint32_t k0 = order_key(DT{}, x0), k1 = order_key(DT{}, x1);
      const uint32_t kmin = wave_min_u32(k0 < k1 ? k0 : k1);
      const uint32_t kmax = wave_max_u32(k0 > k1 ? k0 : k1);
      const bool any_nan = __ballot(is_nan(DT{}, x0) || is_nan(DT{}, x1)) != 0ull;
      const S mn = any_nan ? canonical_nan(DT{}) : from_order_key(DT{}, kmin);
      const S mx = any_nan ? canonical_nan(DT{}) : from_order_key(DT{}, kmax);
      const float mnf = to_f32(DT{}, mn);
      const float mxf = to_f32(DT{}, mx);
      const S sc = from_f32(DT{}, int4_scale<DT>(mnf, mxf));
      const float sf = to_f32(DT{}, sc);
      const uint32_t lo = int4_code(to_f32(DT{}, x0), mnf, sf);
      const uint32_t hi = int4_code(to_f32(DT{}, x1), mnf, sf);
      const int64_t row = static_cast<int64_t>(g) * a.meta_qstride + position;
      a.meta_packed[row * 64 + lane] = static_cast<uint8_t>(lo | (hi << 4));
      if (lane == 0) {
        static_cast<S*>(a.meta_qscale)[row] = sc;
        static_cast<S*>(a.meta_qmin)[row] = mn;
      }
    }
    complete_page_meta<DT>(a, g, position);
  }
}
constexpr int kTileRows = 16;

// Window of group g in a page-tile launch: the host's (one length for every
// group) or, for ragged launches, derived from lengths[g] the same way.
struct TileWin {
  int sink_tiles, sink_end, recent_start, n_recent, has_dec, run, run_tiles, nu_cap;
  int append_position;  // the decode token's cache row, -1: none
  int length;           // tokens before the decode token (the resident cache's epoch)
};

__device__ __forceinline__ TileWin tile_window(const AttnArgs& a, int g) {
  TileWin w;
  if (a.lengths == nullptr) {
    w.sink_tiles = a.t_sink_tiles;
    w.sink_end = a.t_sink_end;
    w.recent_start = a.t_recent_start;
    w.n_recent = a.t_n_recent;
    w.has_dec = a.t_has_dec;
    w.run = a.t_run;
    w.run_tiles = a.t_run_tiles;
    w.nu_cap = a.t_nu_cap;
    w.append_position = a.append_position;
    w.length = a.length;
    return w;
  }
  const int lmax = static_cast<int>(a.entry_stride) - 1;  // the decode token's row stays in the entry
  int L = a.lengths[g];
  L = L < 0 ? 0 : (L > lmax ? lmax : L);
  w.sink_end = a.sink < L ? a.sink : L;
  const int hist_recent = a.recent - 1 > 0 ? a.recent - 1 : 0;
  w.recent_start = (L - hist_recent) > w.sink_end ? (L - hist_recent) : w.sink_end;
  w.n_recent = L - w.recent_start;
  w.has_dec = (a.cur_k != nullptr || a.ragged_append) ? 1 : 0;
  w.run = w.n_recent + w.has_dec;
  w.sink_tiles = (w.sink_end + kTileRows - 1) / kTileRows;
  w.run_tiles = (w.run + kTileRows - 1) / kTileRows;
  w.append_position = a.ragged_append ? L : -1;
  w.length = L;
  int cap = (a.max_rows - w.sink_end - w.run) / kTileRows;
  const int room = a.max_chunks * a.t_per_chunk - w.sink_tiles - w.run_tiles;
  cap = cap < room ? cap : room;
  cap = cap < a.plan_stride ? cap : static_cast<int>(a.plan_stride);
  w.nu_cap = cap < 0 ? 0 : cap;
  return w;
}

// Union pages of group g that a page-tile launch covers: the union plan's
// count, or with selection bitmaps the size the split-K kernel ranked
// (written by the group's chunk-0 block for the merge launch).
__device__ __forceinline__ int tile_pages(const AttnArgs& a, int g, const TileWin& w) {
  int nu = a.sel_bits != nullptr ? a.union_sizes[g] : a.plan_counts[g];
  nu = nu < 0 ? 0 : nu;
  return nu > w.nu_cap ? w.nu_cap : nu;
}

// Append the decode token of group g to its cache entry (chunk 0's block).
template <typename S>
__device__ __forceinline__ void append_decode_token(const AttnArgs& a, int g, int D, int position) {
  if (a.k_append == nullptr || position < 0) return;
  const int64_t row = (static_cast<int64_t>(g) * a.entry_stride + position) * D;
  const S* ck = static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D;
  const S* cv = static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D;
  S* dk = static_cast<S*>(a.k_append) + row;
  S* dv = static_cast<S*>(a.v_append) + row;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    dk[i] = ck[i];
    dv[i] = cv[i];
  }
}

// Split-K combine: one block per (group, head), thread t = channel t.  Runs
// as its own launch after the partial kernel, so it reads the partials with
// plain loads and issues every chunk's loads at once (one round trip); the
// chunk weights exp2(m_c - M) and 1 / sum(w_c l_c) come from a block
// reduction over the chunks' (m, l).  Groups that fit one chunk were written
// by the partial kernel itself and are skipped.
template <typename DT, int MODE, int NB>
__global__ __launch_bounds__(512) void merge_kernel(AttnArgs a, int rows_per_block) {
  using S = typename DT::storage;
  const int R = a.R;
  const int D = a.D;
  const int g = static_cast<int>(blockIdx.x) % a.G;  // group-minor, as the split-K blocks
  const int r = static_cast<int>(blockIdx.x) / a.G;
  const GroupRows gr = group_rows<MODE>(a, g, D);
  const int n_chunks = (gr.n_rows + rows_per_block - 1) / rows_per_block;
  if (n_chunks <= 1) return;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t / kWave;
  const int n_waves = (blockDim.x + kWave - 1) / kWave;
  __shared__ float s_red[8];
  __shared__ float s_w[NB];
  const int64_t base = static_cast<int64_t>(g) * a.max_chunks;
  const int ch_t = t < D ? t : D - 1;
  // every load of the merge in one batch: o of all chunks for channel t, and
  // (m, l) of chunk t
  float ov[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    const int cc = c < n_chunks ? c : n_chunks - 1;
    ov[c] = a.part_o[((base + cc) * R + r) * D + ch_t];
  }
  const int ct = t < n_chunks ? t : n_chunks - 1;
  const float2 mlv = *reinterpret_cast<const float2*>(a.part_ml + ((base + ct) * R + r) * 2);
  const float m = t < n_chunks ? mlv.x : -INFINITY;
  float mw = wave_max_f32(m);
  if (lane == 0) s_red[wave] = mw;
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < n_waves; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const float w_t = t < n_chunks ? exp2_rel(m, M) : 0.0f;
  if (t < NB) s_w[t] = w_t;
  const float lw = wave_sum_f32(w_t * (t < n_chunks ? mlv.y : 0.0f));
  if (lane == 0) s_red[wave] = lw;
  __syncthreads();
  float L = 0.0f;
  for (int w = 0; w < n_waves; ++w) L += s_red[w];
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; ++c) acc += (c < n_chunks ? s_w[c] : 0.0f) * ov[c];
  if (t < D) {
    S* out = static_cast<S*>(a.out) + (static_cast<int64_t>(g) * R + r) * D;
    out[t] = from_f32(DT{}, L > 0.0f ? acc / L : 0.0f);
  }
}

// Split-K combine for D in {64, 128, 256}: CS blocks per (group, head), each
// over D / CS channels, thread t = (chunk lane t / (D/4/CS), channel quad
// t % (D/4/CS)).  Every chunk lane loads its chunks' (m, l) and 16-byte o
// slices in one batch (at most 32 loads per thread for D <= 128 at CS = 1, 8
// at CS = 4; one memory round trip), the block finds the max m (every slice
// block of a head the same), weights its chunks by exp2(m_c - M) and the
// chunk lanes are summed in LDS.
template <typename DT, int MODE, int D, int CS = 1>
__global__ __launch_bounds__(kBlock) void merge_vec_kernel(AttnArgs a, int rows_per_block) {
  using S = typename DT::storage;
  constexpr int NQ = D / 4 / CS;                   // channel quads of the block's slice
  constexpr int NL = kBlock / NQ;                  // chunk lanes
  constexpr int MAXJ = (kMaxChunks + NL - 1) / NL; // chunks per lane
  const int R = a.R;
  // group-minor like the split-K kernels' blocks: group g on XCD g % 8
  const int g = static_cast<int>(blockIdx.x) % a.G;
  const int hs = static_cast<int>(blockIdx.x) / a.G;  // (head, slice)
  const int r = hs / CS;
  const int c0 = (hs - r * CS) * (D / CS);  // first channel of the slice
  const int t = threadIdx.x;
  const int q = t % NQ;
  const int cl = t / NQ;
  const int wave = t / kWave;
  __shared__ float s_red[kWaves];
  __shared__ float4 s_o[NL][NQ];
  __shared__ float s_l[NL];
  // The partial loads go out against the launch's chunk bound, in the same
  // round trip as the group's own chunk count; chunks past that count hold
  // stale or unwritten data and are replaced by zeros (selects, not products).
  const int64_t base = static_cast<int64_t>(g) * a.max_chunks;
  float4 ov[MAXJ];
  float2 mlv[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int c = cl + NL * j;
    const int64_t pc = base + (c < a.max_chunks ? c : a.max_chunks - 1);
    ov[j] = *reinterpret_cast<const float4*>(a.part_o + (pc * R + r) * D + c0 + 4 * q);
    mlv[j] = *reinterpret_cast<const float2*>(a.part_ml + (pc * R + r) * 2);
  }
  // rows_per_block: rows of a chunk, or tiles of a chunk in page-tile mode
  int n_chunks;
  if constexpr (MODE == kModeTiles) {
    const TileWin w = tile_window(a, g);
    const int nt = w.sink_tiles + tile_pages(a, g, w) + w.run_tiles;
    n_chunks = (nt + rows_per_block - 1) / rows_per_block;
  } else {
    const GroupRows gr = group_rows<MODE>(a, g, D);
    n_chunks = (gr.n_rows + rows_per_block - 1) / rows_per_block;
  }
  if (n_chunks <= 1) return;
  float mv[MAXJ], lv[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const bool ok = cl + NL * j < n_chunks;
    mv[j] = ok ? mlv[j].x : -INFINITY;
    lv[j] = ok ? mlv[j].y : 0.0f;
    ov[j] = ok ? ov[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) m = fmaxf(m, mv[j]);
  m = wave_max_f32(m);
  if (lane_id() == 0) s_red[wave] = m;
  __syncthreads();
  float M = s_red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_red[w]);
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float l = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const float w = exp2_rel(mv[j], M);
    o.x += w * ov[j].x;
    o.y += w * ov[j].y;
    o.z += w * ov[j].z;
    o.w += w * ov[j].w;
    l += w * lv[j];
  }
  s_o[cl][q] = o;
  if (q == 0) s_l[cl] = l;
  __syncthreads();
  if (cl == 0) {
    float4 O = s_o[0][q];
    float L = s_l[0];
#pragma unroll
    for (int k = 1; k < NL; ++k) {
      O.x += s_o[k][q].x;
      O.y += s_o[k][q].y;
      O.z += s_o[k][q].z;
      O.w += s_o[k][q].w;
      L += s_l[k];
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    S* out = static_cast<S*>(a.out) + (static_cast<int64_t>(g) * R + r) * D + c0 + 4 * q;
    out[0] = from_f32(DT{}, L > 0.0f ? O.x * inv : 0.0f);
    out[1] = from_f32(DT{}, L > 0.0f ? O.y * inv : 0.0f);
    out[2] = from_f32(DT{}, L > 0.0f ? O.z * inv : 0.0f);
    out[3] = from_f32(DT{}, L > 0.0f ? O.w * inv : 0.0f);
  }
}

// Block partial from the wavefront partials in LDS: either the final output
// (single-chunk groups) or a partial for the merge.
template <typename DT, int RMAX>
__device__ void block_partial(const AttnArgs& a, int g, int chunk, int D, bool final_out, const float* s_m,
                              const float* s_l, const float* s_o) {
  using S = typename DT::storage;
  const int R = a.R;
  for (int idx = threadIdx.x; idx < R * D; idx += kBlock) {
    const int r = idx / D;
    const int c = idx - r * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w * RMAX + r]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = exp2_rel(s_m[w * RMAX + r], M);
      L += f * s_l[w * RMAX + r];
      O += f * s_o[(w * RMAX + r) * D + c];
    }
    if (final_out) {
      S* out = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      out[idx] = from_f32(DT{}, L > 0.0f ? O / L : 0.0f);
    } else {
      const int64_t pc = static_cast<int64_t>(g) * a.max_chunks + chunk;
      a.part_o[pc * R * D + idx] = O;
      if (c == 0) *reinterpret_cast<float2*>(a.part_ml + (pc * R + r) * 2) = make_float2(M, L);
    }
  }
}

template <typename DT, int D, int RMAX, int MODE>
__global__ __launch_bounds__(kBlock, RMAX >= 8 ? 2 : 3) void decode_attn_kernel(AttnArgs a) {
  using S = typename DT::storage;
  constexpr int CPL = 8;
  constexpr int LPR = D / CPL;                       // lanes per row
  constexpr int RPI = kWave / LPR;                   // rows per load instruction
  constexpr int STEPS = steps_for(sizeof(S), RMAX);   // load instructions per batch
  constexpr int RW = STEPS * RPI;                    // rows per wavefront batch
  constexpr int RB = kWaves * RW;                    // rows per block batch
  static_assert(RW <= kWave, "one index lane per row");

  const int R = a.R;
  const int g = static_cast<int>(blockIdx.x) % a.G;  // chunk-major (group g on XCD g % 8)
  const int chunk = static_cast<int>(blockIdx.x) / a.G;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int rig = lane / LPR;
  const int c0 = (lane % LPR) * CPL;

  __shared__ float s_m[kWaves * RMAX];
  __shared__ float s_l[kWaves * RMAX];
  extern __shared__ __align__(16) float s_dyn[];   // [kWaves][RMAX][D] then merge scratch

  const GroupRows gr = group_rows<MODE>(a, g, D);
  const int rows_per_block = RB * a.iters;
  const int n_chunks = (gr.n_rows + rows_per_block - 1) / rows_per_block;
  if (gr.n_rows == 0) {
    if (chunk == 0) {
      S* o = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      for (int i = threadIdx.x; i < R * D; i += kBlock) o[i] = from_f32(DT{}, 0.0f);
    }
    return;
  }
  if (chunk >= n_chunks) return;
  if ((MODE == kModePages || MODE == kModeRows) && chunk == 0) {
    append_decode_token<S>(a, g, D, decode_row_position<MODE>(a, g));
    if (MODE == kModeRows) complete_row_meta<DT>(a, g, decode_row_position<MODE>(a, g));
  }

  const S* kbase = static_cast<const S*>(a.k);
  const S* vbase = static_cast<const S*>(a.v);
  const S* ck = a.cur_k != nullptr ? static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D : nullptr;
  const S* cv = a.cur_v != nullptr ? static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D : nullptr;

  // ---- queries (scale * log2 e folded in); rows r >= R are zero ----
  float qv[RMAX][CPL];
  {
    const S* qg = static_cast<const S*>(a.q) + static_cast<int64_t>(g) * R * D;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      Vec8<S> t;
      t.load(qg + static_cast<int64_t>(r < R ? r : R - 1) * D + c0);
      float f[CPL];
      t.template to_float<DT>(f);
#pragma unroll
      for (int i = 0; i < CPL; ++i) qv[r][i] = (r < R) ? f[i] * a.scale_log2 : 0.0f;
    }
  }

  float m_run[RMAX], l_run[RMAX], o_acc[RMAX][CPL];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) o_acc[r][i] = 0.0f;
  }

  // Row (or page) masks: when there are none, read a byte of the index list
  // instead and force every head visible (keeps the load unconditional).
  const int32_t* idx_src = MODE == kModePages ? a.plan_pages : a.rows;
  const uint8_t* mask_in = MODE == kModePages ? a.plan_masks : a.masks;
  const uint8_t* mask_src = mask_in != nullptr ? mask_in : reinterpret_cast<const uint8_t*>(idx_src);
  const uint32_t mask_force = mask_in != nullptr ? 0u : 0xffu;
  const int64_t list_base = static_cast<int64_t>(g) * (MODE == kModePages ? a.plan_stride : a.rows_stride);
  const int last_list = MODE == kModePages ? (gr.n_pages > 0 ? gr.n_pages - 1 : 0)
                                           : (gr.n_list > 0 ? gr.n_list - 1 : 0);
  const bool bs_pow2 = (a.bs & (a.bs - 1)) == 0;
  const int bs_shift = bs_pow2 && a.bs > 0 ? __ffs(a.bs) - 1 : 0;
  // Readable stand-ins for rows that are dropped or not in the list.
  const S* safe_k = gr.n_list > 0 ? kbase + gr.base : (ck != nullptr ? ck : kbase);
  const S* safe_v = gr.n_list > 0 ? vbase + gr.base : (cv != nullptr ? cv : vbase);
  const S* cur_k = ck != nullptr ? ck : safe_k;
  const S* cur_v = cv != nullptr ? cv : safe_v;

  for (int it = 0; it < a.iters; ++it) {
    const int row0 = chunk * rows_per_block + it * RB + wave * RW;
    if (row0 >= gr.n_rows) break;
    // ---- round trip 1: this lane's row indices and masks ----
    int pos[STEPS];
    uint32_t hm[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int i = row0 + s * RPI + rig;
      if (MODE == kModeRows) {
        const int64_t at = list_base + (i < last_list ? i : last_list);
        pos[s] = a.rows[at];
        hm[s] = static_cast<uint32_t>(mask_src[at]) | mask_force;
      } else if (MODE == kModePages) {
        const int j = i - gr.sink_end;
        int u = bs_pow2 ? (j >> bs_shift) : j / a.bs;
        u = u < 0 ? 0 : (u > last_list ? last_list : u);
        const int64_t at = list_base + u;
        const int page = a.plan_pages[at];
        const uint32_t pm = static_cast<uint32_t>(mask_src[at]) | mask_force;
        const bool in_pages = i >= gr.sink_end && i < gr.page_end;
        pos[s] = i < gr.sink_end ? i
                 : in_pages      ? a.sink + page * a.bs + (j - u * a.bs)
                 : i < gr.recent_end ? gr.recent_start + (i - gr.page_end)
                                     : a.append_position;
        hm[s] = in_pages ? pm : 0xffu;
      } else {
        pos[s] = gr.win_start + i;
        hm[s] = 0xffu;
      }
    }
    // ---- round trip 2: K/V rows ----
    Vec8<S> kc[STEPS], vc[STEPS];
    bool ok[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int i = row0 + s * RPI + rig;
      const bool in_list = i < gr.n_list && (MODE == kModeVarlen || (pos[s] >= 0 && pos[s] < a.entry_stride));
      const bool cur = i == gr.n_list && i < gr.n_rows;
      ok[s] = in_list || cur;
      if (cur) hm[s] = 0xffu;
      const int64_t off = gr.base + static_cast<int64_t>(in_list ? pos[s] : 0) * gr.stride;
      const S* kp = cur ? cur_k : (in_list ? kbase + off : safe_k);
      const S* vp = cur ? cur_v : (in_list ? vbase + off : safe_v);
      kc[s].load(kp + c0);
      vc[s].load(vp + c0);
    }
    // ---- scores in log2 units ----
    float sc[STEPS][RMAX];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      float kf[CPL];
      kc[s].template to_float<DT>(kf);
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc = __builtin_fmaf(qv[r][i], kf[i], acc);
        sc[s][r] = acc;
      }
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
      for (int r = 0; r < RMAX; ++r) sc[s][r] = row_group_sum<LPR>(sc[s][r]);
    }
    float mnew[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const bool vis = ok[s] && r < R && ((hm[s] >> r) & 1u);
        sc[s][r] = vis ? sc[s][r] : -INFINITY;
        mx = fmaxf(mx, sc[s][r]);
      }
#pragma unroll
      for (int o = LPR; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      mnew[r] = fmaxf(m_run[r], mx);
    }
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      const float alpha = (mnew[r] == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[r] - mnew[r]);
      m_run[r] = mnew[r];
      l_run[r] *= alpha;
#pragma unroll
      for (int i = 0; i < CPL; ++i) o_acc[r][i] *= alpha;
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      float vf[CPL];
      vc[s].template to_float<DT>(vf);
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        const float p = exp2_rel(sc[s][r], m_run[r]);
        l_run[r] += p;
#pragma unroll
        for (int i = 0; i < CPL; ++i) o_acc[r][i] = __builtin_fmaf(p, vf[i], o_acc[r][i]);
      }
    }
  }
  // ---- merge the row groups of the wavefront (same channels) ----
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1) {
      l_run[r] += __shfl_xor(l_run[r], o);
#pragma unroll
      for (int i = 0; i < CPL; ++i) o_acc[r][i] += __shfl_xor(o_acc[r][i], o);
    }
  }
  float* s_o = s_dyn;
  if (lane < LPR) {
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      if (lane == 0) {
        s_m[wave * RMAX + r] = m_run[r];
        s_l[wave * RMAX + r] = l_run[r];
      }
#pragma unroll
      for (int i = 0; i < CPL; ++i) s_o[(wave * RMAX + r) * D + c0 + i] = o_acc[r][i];
    }
  }
  __syncthreads();
  block_partial<DT, RMAX>(a, g, chunk, D, n_chunks == 1, s_m, s_l, s_o);
}

// ------------------------------------------------------------------ MFMA
// 16-bit K/V: q.k on the matrix cores, p.v with packed dot2.
//
// q.k is a [16 heads x D] x [D x 16 rows] product per tile of 16 rows: four
// (D/32) v_mfma_f32_16x16x32 steps, A = the group's queries (lane = head +
// 16 * quarter), B = K^T (lane = row + 16 * quarter), each lane loading D/2
// contiguous bytes of its row.  Quarter q, step s, element e is channel
// q*D/4 + 8s + e in both operands.  The product lands as S[4*(lane/16)+v]
// [lane%16] in register v, so lanes 0..15 hold heads 0..3 of the 16 rows
// (16..31 heads 4..7).  Heads beyond R are zero rows of A.  The R <= 8 heads
// of a GQA group pad the 16-row A operand; the padding costs matrix-core
// cycles the kernel has to spare, and it takes the dot products, conversions
// and cross-lane reductions of q.k off the vector ALU, which bounded the
// all-VALU form.
//
// p.v stays on the vector ALU: V rows are read with 8 channels per lane
// (D/8 lanes per row), p goes through LDS as the input dtype, and pairs of
// rows are combined with v_dot2_f32_{f16,bf16} (p_a v_a + p_b v_b into an
// fp32 accumulator), rounding p to the input dtype as flash-attention does.
template <int D>
struct MfmaGeom {
  static constexpr int STEPS = D / 32;   // MFMA k-steps over the head dim
  static constexpr int QC = D / 4;       // channels per quarter
  static constexpr int LPR = D / 8;      // V lanes per row
  static constexpr int RG = kWave / LPR; // V row groups
  static constexpr int VR = 16 / RG;     // V rows per lane per 16-row tile
};

constexpr int mfma_tiles(int D, int rmax) {
  return (D == 64 ? 4 : (D == 128 ? 2 : 1)) / ((rmax >= 8 && D != 256) ? 2 : 1);
}

template <typename DT>
struct Half8;
template <>
struct Half8<F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot2(uint32_t p, uint32_t v, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, p), __builtin_bit_cast(v2, v), acc, false);
  }
  static __device__ __forceinline__ void mfma(const uint4& a, const uint4& b, float (&c)[4]) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 acc = {c[0], c[1], c[2], c[3]};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), acc, 0, 0, 0);
    c[0] = acc[0]; c[1] = acc[1]; c[2] = acc[2]; c[3] = acc[3];
  }
};
template <>
struct Half8<BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot2(uint32_t p, uint32_t v, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, p), __builtin_bit_cast(v2, v), acc, false);
  }
  static __device__ __forceinline__ void mfma(const uint4& a, const uint4& b, float (&c)[4]) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 acc = {c[0], c[1], c[2], c[3]};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), acc, 0, 0, 0);
    c[0] = acc[0]; c[1] = acc[1]; c[2] = acc[2]; c[3] = acc[3];
  }
};

// Source row of list index i of a group: position, visible heads, and
// whether it is a cache row, the decode token, or neither.
struct RowRef {
  int pos;
  uint32_t hm;
  bool in_list;
  bool cur;
};

template <int MODE>
__device__ __forceinline__ RowRef row_ref(const AttnArgs& a, const GroupRows& gr, int i, int64_t list_base,
                                          int last_list, const uint8_t* mask_src, uint32_t mask_force,
                                          bool bs_pow2, int bs_shift) {
  RowRef r;
  if (MODE == kModeRows) {
    const int64_t at = list_base + (i < last_list ? i : last_list);
    r.pos = a.rows[at];
    r.hm = static_cast<uint32_t>(mask_src[at]) | mask_force;
  } else if (MODE == kModePages) {
    const int j = i - gr.sink_end;
    int u = bs_pow2 ? (j >> bs_shift) : j / a.bs;
    u = u < 0 ? 0 : (u > last_list ? last_list : u);
    const int64_t at = list_base + u;
    const int page = a.plan_pages[at];
    const uint32_t pm = static_cast<uint32_t>(mask_src[at]) | mask_force;
    const bool in_pages = i >= gr.sink_end && i < gr.page_end;
    r.pos = i < gr.sink_end ? i
            : in_pages      ? a.sink + page * a.bs + (j - u * a.bs)
            : i < gr.recent_end ? gr.recent_start + (i - gr.page_end)
                                : a.append_position;
    r.hm = in_pages ? pm : 0xffu;
  } else {
    r.pos = gr.win_start + i;
    r.hm = 0xffu;
  }
  r.in_list = i < gr.n_list && (MODE == kModeVarlen || (r.pos >= 0 && r.pos < a.entry_stride));
  r.cur = i == gr.n_list && i < gr.n_rows;
  if (r.cur) r.hm = 0xffu;
  return r;
}

template <typename DT, int D, int RMAX, int MODE>
__global__ __launch_bounds__(kBlock, 2) void decode_attn_mfma(AttnArgs a) {
  using S = typename DT::storage;
  using G = MfmaGeom<D>;
  using H = Half8<DT>;
  constexpr int TILES = mfma_tiles(D, RMAX);
  constexpr int RW = 16 * TILES;             // rows per wavefront batch
  constexpr int RB = kWaves * RW;            // rows per block batch
  constexpr int HG = (RMAX + 3) / 4;         // 16-lane head groups of the q.k product
  static_assert(RMAX <= 8, "at most 8 heads per group");

  const int R = a.R;
  const int g = static_cast<int>(blockIdx.x) % a.G;  // chunk-major (group g on XCD g % 8)
  const int chunk = static_cast<int>(blockIdx.x) / a.G;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int krow = lane & 15;                // q.k: row of the tile / head of A
  const int quarter = lane >> 4;
  const int c0v = (lane % G::LPR) * 8;       // p.v: channels
  const int rg = lane / G::LPR;              // p.v: row group

  __shared__ float s_m[kWaves * RMAX];
  __shared__ float s_l[kWaves * RMAX];
  __shared__ __align__(16) S s_p[kWaves][RMAX][RW];   // p of the batch, per head
  extern __shared__ __align__(16) float s_dyn[];

  const GroupRows gr = group_rows<MODE>(a, g, D);
  const int rows_per_block = RB * a.iters;
  const int n_chunks = (gr.n_rows + rows_per_block - 1) / rows_per_block;
  if (gr.n_rows == 0) {
    if (chunk == 0) {
      S* o = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      for (int i = threadIdx.x; i < R * D; i += kBlock) o[i] = from_f32(DT{}, 0.0f);
    }
    return;
  }
  if (chunk >= n_chunks) return;
  if ((MODE == kModePages || MODE == kModeRows) && chunk == 0) {
    append_decode_token<S>(a, g, D, decode_row_position<MODE>(a, g));
    if (MODE == kModeRows) complete_row_meta<DT>(a, g, decode_row_position<MODE>(a, g));
  }

  const S* kbase = static_cast<const S*>(a.k);
  const S* vbase = static_cast<const S*>(a.v);
  const S* ck = a.cur_k != nullptr ? static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D : nullptr;
  const S* cv = a.cur_v != nullptr ? static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D : nullptr;

  // ---- A operand: the group's queries, zero rows for heads >= R ----
  uint4 qf[G::STEPS];
  {
    const S* qh = static_cast<const S*>(a.q) + (static_cast<int64_t>(g) * R + (krow < R ? krow : 0)) * D;
#pragma unroll
    for (int s = 0; s < G::STEPS; ++s) {
      const uint4 t = *reinterpret_cast<const uint4*>(qh + quarter * G::QC + 8 * s);
      qf[s] = krow < R ? t : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  float m_run[RMAX];      // wave-uniform running max per head (log2 units)
  float l_part[4];        // this lane's partial sum of p for heads 4*quarter + v
  float o_acc[RMAX][8];   // p.v accumulators, channels c0v.., rows of group rg
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
    m_run[h] = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) o_acc[h][i] = 0.0f;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) l_part[v] = 0.0f;

  const int32_t* idx_src = MODE == kModePages ? a.plan_pages : a.rows;
  const uint8_t* mask_in = MODE == kModePages ? a.plan_masks : a.masks;
  const uint8_t* mask_src = mask_in != nullptr ? mask_in : reinterpret_cast<const uint8_t*>(idx_src);
  const uint32_t mask_force = mask_in != nullptr ? 0u : 0xffu;
  const int64_t list_base = static_cast<int64_t>(g) * (MODE == kModePages ? a.plan_stride : a.rows_stride);
  const int last_list = MODE == kModePages ? (gr.n_pages > 0 ? gr.n_pages - 1 : 0)
                                           : (gr.n_list > 0 ? gr.n_list - 1 : 0);
  const bool bs_pow2 = (a.bs & (a.bs - 1)) == 0;
  const int bs_shift = bs_pow2 && a.bs > 0 ? __ffs(a.bs) - 1 : 0;
  const S* safe_k = gr.n_list > 0 ? kbase + gr.base : (ck != nullptr ? ck : kbase);
  const S* safe_v = gr.n_list > 0 ? vbase + gr.base : (cv != nullptr ? cv : vbase);
  const S* cur_k = ck != nullptr ? ck : safe_k;
  const S* cur_v = cv != nullptr ? cv : safe_v;

  for (int it = 0; it < a.iters; ++it) {
    const int row0 = chunk * rows_per_block + it * RB + wave * RW;
    if (row0 >= gr.n_rows) break;
    // ---- round trip 1: row indices (K rows and V rows of this lane) ----
    RowRef kr[TILES], vr[TILES][G::VR];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      kr[t] = row_ref<MODE>(a, gr, row0 + 16 * t + krow, list_base, last_list, mask_src, mask_force, bs_pow2,
                            bs_shift);
#pragma unroll
      for (int j = 0; j < G::VR; ++j)
        vr[t][j] = row_ref<MODE>(a, gr, row0 + 16 * t + rg * G::VR + j, list_base, last_list, mask_src,
                                 mask_force, bs_pow2, bs_shift);
    }
    // ---- round trip 2: K fragments and V rows ----
    uint4 kf[TILES][G::STEPS];
    uint4 vf[TILES][G::VR];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const S* kp = kr[t].cur ? cur_k
                    : (kr[t].in_list ? kbase + gr.base + static_cast<int64_t>(kr[t].pos) * gr.stride : safe_k);
#pragma unroll
      for (int s = 0; s < G::STEPS; ++s)
        kf[t][s] = *reinterpret_cast<const uint4*>(kp + quarter * G::QC + 8 * s);
#pragma unroll
      for (int j = 0; j < G::VR; ++j) {
        const S* vp = vr[t][j].cur ? cur_v
                      : (vr[t][j].in_list ? vbase + gr.base + static_cast<int64_t>(vr[t][j].pos) * gr.stride
                                          : safe_v);
        vf[t][j] = *reinterpret_cast<const uint4*>(vp + c0v);
      }
    }
    // ---- q.k on the matrix cores ----
    float sc[TILES][4];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < G::STEPS; ++s) H::mfma(qf[s], kf[t][s], acc);
      const bool ok = kr[t].in_list || kr[t].cur;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int h = 4 * quarter + v;
        const bool vis = ok && h < R && ((kr[t].hm >> h) & 1u);
        sc[t][v] = vis ? acc[v] * a.scale_log2 : -INFINITY;
      }
    }
    // ---- batch max per head: over the tiles, then the 16 lanes of a row ----
    float mx[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float x = sc[0][v];
#pragma unroll
      for (int t = 1; t < TILES; ++t) x = fmaxf(x, sc[t][v]);
      x = fmaxf(x, dpp<kQuadXor1>(x));
      x = fmaxf(x, dpp<kQuadXor2>(x));
      x = fmaxf(x, dpp<kRowHalfMirror>(x));
      x = fmaxf(x, dpp<kRowMirror>(x));
      mx[v] = x;
    }
    float alpha[RMAX];
#pragma unroll
    for (int h = 0; h < RMAX; ++h) {
      const float tile_max = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx[h & 3]), 16 * (h >> 2)));
      const float mnew = fmaxf(m_run[h], tile_max);
      alpha[h] = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[h] - mnew);
      m_run[h] = mnew;
#pragma unroll
      for (int i = 0; i < 8; ++i) o_acc[h][i] *= alpha[h];
    }
    // ---- p = exp2(s - m) in the input dtype through LDS ----
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int h = 4 * quarter + v;
      // this lane's head for register v: 4*quarter + v (quarters >= HG are idle)
      const float al = HG > 1 && quarter == 1 ? alpha[(4 + v) % RMAX] : alpha[v % RMAX];
      const float m_lane = HG > 1 && quarter == 1 ? m_run[(4 + v) % RMAX] : m_run[v % RMAX];
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const float pv = exp2_rel(sc[t][v], m_lane);
        psum += pv;
        if (quarter < HG && h < RMAX) s_p[wave][h][16 * t + krow] = from_f32(DT{}, pv);
      }
      l_part[v] = l_part[v] * al + psum;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's p stores are done
    __builtin_amdgcn_wave_barrier();
    // ---- p.v: pairs of rows with v_dot2 ----
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
#pragma unroll
      for (int j = 0; j < G::VR; j += 2) {
        const uint32_t va[4] = {vf[t][j].x, vf[t][j].y, vf[t][j].z, vf[t][j].w};
        const uint32_t vb[4] = {vf[t][j + 1].x, vf[t][j + 1].y, vf[t][j + 1].z, vf[t][j + 1].w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo[i] = __builtin_amdgcn_perm(vb[i], va[i], 0x05040100u);  // (a.ch 2i, b.ch 2i)
          hi[i] = __builtin_amdgcn_perm(vb[i], va[i], 0x07060302u);  // (a.ch 2i+1, b.ch 2i+1)
        }
#pragma unroll
        for (int h = 0; h < RMAX; ++h) {
          const uint32_t pp = *reinterpret_cast<const uint32_t*>(&s_p[wave][h][16 * t + rg * G::VR + j]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            o_acc[h][2 * i] = H::dot2(pp, lo[i], o_acc[h][2 * i]);
            o_acc[h][2 * i + 1] = H::dot2(pp, hi[i], o_acc[h][2 * i + 1]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // ---- the wavefront's (m, l, o): sum o over the row groups, l over rows ----
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
#pragma unroll
    for (int o = G::LPR; o < kWave; o <<= 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i) o_acc[h][i] += __shfl_xor(o_acc[h][i], o);
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float x = l_part[v];
    x += dpp<kQuadXor1>(x);
    x += dpp<kQuadXor2>(x);
    x += dpp<kRowHalfMirror>(x);
    x += dpp<kRowMirror>(x);
    l_part[v] = x;
  }
  float* s_o = s_dyn;
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
    const float lh = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_part[h & 3]), 16 * (h >> 2)));
    if (lane == 0) {
      s_m[wave * RMAX + h] = m_run[h];
      s_l[wave * RMAX + h] = lh;
    }
    if (lane < G::LPR) {
#pragma unroll
      for (int i = 0; i < 8; ++i) s_o[(wave * RMAX + h) * D + c0v + i] = o_acc[h][i];
    }
  }
  __syncthreads();
  block_partial<DT, RMAX>(a, g, chunk, D, n_chunks == 1, s_m, s_l, s_o);
}

// ---------------------------------------------------------------------------
// Page-tile decode attention: page mode with 16-row pages, D = 128, 16-bit
// K/V, R <= 8.  The group's rows are walked as 16-row tiles -- the sink
// window in runs of 16 positions, one tile per union page (a page's rows are
// contiguous in the entry), then the recent window followed by the decode
// token.  Which source a tile has is wave-uniform, so a page id costs one
// scalar load per tile and every lane addresses its rows as the tile's base
// plus a lane offset.  The plan count and the wave's page slots are loaded in
// the same round trip (slots are read speculatively, clamped to the plan
// width), so K/V loads are the second and last dependent round trip.
//
// q.k: v_mfma_f32_16x16x32 with the heads as A rows (zero rows for heads >= R)
// and the tile's 16 rows as B columns; lane (row, quarter) holds channels
// 32 s + 8 quarter + [0, 8) of k-step s, so one K load instruction reads 64
// contiguous bytes of each of 16 rows.  The result gives lane (row, quarter)
// the scores of heads 4 quarter + [0, 4).
// p.v: lane (c8, rg) owns channels 8 c8 + [0, 8) of rows 4 rg + [0, 4) of a
// tile.  p goes through LDS as the input dtype, stored as (row 2i, row 2i+1)
// pairs per head so that one 16-byte read gives a row pair's p for four
// heads, and pairs of rows are combined with v_dot2_f32_{f16,bf16}.
// One wavefront batch is TW tiles; a wave's first batch needs no rescale.
constexpr int kTileD = 128;

// Union pages from selection bitmaps.  Each lane holds NWL consecutive
// 64-bit words of every head's row (lane l: words NWL*l ..), uw their OR,
// and incl / cnt the wavefront's inclusive prefix and own count of union
// pages.  The union page of rank u (wave-uniform, below the union size) is
// the (u - exclusive prefix)-th set bit of the first lane whose inclusive
// prefix exceeds u; every lane tests one bit position of that word, so the
// bit is found with one popcount and a ballot.  *hm gets the heads that
// selected the page.
__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, int l) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x)), l));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x >> 32)), l));
  return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}

template <int RMAX, int NWL>
__device__ __forceinline__ void bits_page(int u, int incl, int cnt, const uint64_t (&uw)[NWL],
                                          const uint64_t (&hw)[RMAX][NWL], int* page, uint32_t* hm) {
  const int lane = lane_id();
  const int L = __ffsll(static_cast<long long>(__ballot(incl > u))) - 1;
  int j = u - (__builtin_amdgcn_readlane(incl, L) - __builtin_amdgcn_readlane(cnt, L));
  int wsel = 0;
  uint64_t word = readlane_u64(uw[0], L);
  if constexpr (NWL == 2) {
    const int c0 = __popcll(word);
    wsel = j >= c0 ? 1 : 0;
    j -= wsel ? c0 : 0;
    word = wsel ? readlane_u64(uw[1], L) : word;
  }
  const bool hit = ((word >> lane) & 1ull) != 0ull && __popcll(word & lanemask_lt()) == j;
  const int b = __ffsll(static_cast<long long>(__ballot(hit))) - 1;
  *page = 64 * (NWL * L + wsel) + b;
  uint32_t m = 0u;
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
    const uint64_t x = (NWL == 2 && wsel) ? hw[h][NWL - 1] : hw[h][0];
    m |= static_cast<uint32_t>((readlane_u64(x, L) >> b) & 1ull) << h;
  }
  *hm = m;
}

struct TileSrc {
  int64_t pos0;  // position of the tile's row 0 in the entry (cache rows)
  int cnt;       // rows of the tile that exist (0..16)
  int dec;       // index of the decode token in the tile, or -1
  uint32_t hm;   // heads that see the tile's cache rows
  uint32_t rm;   // rows of the tile that are attended (bit i = row i)
  int r0;        // a row that is attended (the address of the rows that are not)
  int u;         // union-plan index of a page tile, -1 for sink / recent tiles
  int page;      // its page id
};

__device__ __forceinline__ TileSrc tile_src(const AttnArgs& a, const TileWin& w, int t, int nu, int page,
                                            uint32_t pmask, uint32_t prow, bool row_masks) {
  TileSrc s;
  s.dec = -1;
  s.hm = 0xffu;
  s.rm = 0xffffu;
  s.u = -1;
  s.page = page;
  const int ts = w.sink_tiles;
  if (t < ts) {
    s.pos0 = static_cast<int64_t>(kTileRows) * t;
    const int c = w.sink_end - kTileRows * t;
    s.cnt = c < kTileRows ? c : kTileRows;
  } else if (t < ts + nu) {
    s.pos0 = a.sink + static_cast<int64_t>(page) * kTileRows;
    s.hm = pmask;
    if (row_masks) {
      s.hm = 0xffu;  // the GQA union: every head attends every kept row
      s.rm = prow & 0xffffu;
    }
    s.cnt = (s.pos0 >= 0 && s.pos0 + kTileRows <= a.entry_stride && s.rm != 0u) ? kTileRows : 0;
    s.u = s.cnt > 0 ? t - ts : -1;
  } else {
    const int j0 = kTileRows * (t - ts - nu);
    s.pos0 = static_cast<int64_t>(w.recent_start) + j0;
    const int c = w.run - j0;
    s.cnt = c < 0 ? 0 : (c < kTileRows ? c : kTileRows);
    const int d = w.n_recent - j0;
    s.dec = (w.has_dec && d >= 0 && d < kTileRows) ? d : -1;
  }
  if (s.cnt <= 0) {
    s.cnt = 0;
    s.pos0 = 0;
  }
  s.r0 = s.rm != 0u ? __builtin_ctz(s.rm) : 0;
  return s;
}

// NT: the slab is device memory, so its K/V rows are read with the
// streaming hint (pinned host memory read over the host link keeps plain
// loads, which measured faster there).
// NWL > 0: the union comes from selection bitmaps (NWL 64-bit words per
// lane) instead of a union plan.
// MK (with NWL > 0): the union comes from a Twilight union record (one
// bitmap row, row masks staged in LDS by the block).
// Key rows are loaded like value rows (four whole 256-byte rows per load,
// 1 KB contiguous) and turned into matrix-core fragments through LDS.  Loads
// shaped as the fragments (16 rows x 64 B each) read pinned host memory at
// ~41 GB/s against ~51 GB/s for whole rows, and HBM slower too.
template <typename DT, int RMAX, int NW, int TW, bool RES, bool NT, int NWL, bool MK = false>
__global__ __launch_bounds__(NW * kWave, 2) void decode_attn_tiles(AttnArgs a) {
  using S = typename DT::storage;
  using H = Half8<DT>;
  constexpr int D = kTileD;
  constexpr int NQ = RMAX > 4 ? 2 : 1;  // quarters of the q.k result that hold heads
  constexpr int PW = RMAX / 4 > 0 ? RMAX / 4 : 1;  // 16-byte p reads per row pair
  static_assert(RMAX == 4 || RMAX == 8, "4 or 8 head slots");

  const int R = a.R;
  // chunk-major: workgroups go to the XCDs round-robin, so with G a multiple
  // of 8 every chunk of group g runs on XCD g % 8, where the group's
  // selection blocks wrote its bitmaps and its merge blocks read the partials
  // back, both through that XCD's L2
  const int g = static_cast<int>(blockIdx.x) % a.G;
  const int chunk = static_cast<int>(blockIdx.x) / a.G;
  const int wave = wave_uniform(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int krow = lane & 15;
  const int quarter = lane >> 4;
  const int c8 = (lane & 15) * 8;
  const int rg = lane >> 4;

  __shared__ float s_m[NW][RMAX];
  __shared__ float s_l[NW][RMAX];
  __shared__ __align__(16) uint32_t s_p[NW][TW][8][RMAX];
  __shared__ __align__(16) float s_o[NW][RMAX][D];
  // each wavefront's key tiles, 16-byte unit c of row r at [r][c ^ r] (whole
  // rows written and fragment columns read without bank conflicts)
  __shared__ __align__(16) uint4 s_k[NW][TW][kTileRows][D / 8];

  // ---- round trip 1: plan count, the first batch's page slots, q ----
  const int64_t plan_base = static_cast<int64_t>(g) * a.plan_stride;
  const int slot_last = static_cast<int>(a.plan_stride - 1);
  const int per_chunk = NW * TW * a.iters;
  int page[TW], page_nx[TW];
  uint32_t pmask[TW], pmask_nx[TW], prow[TW], prow_nx[TW];
  auto load_slots = [&](int t0, int (&pg)[TW], uint32_t (&pm)[TW], uint32_t (&pr)[TW]) {
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      int u = t0 + tt - a.t_sink_tiles;
      u = u < 0 ? 0 : (u > slot_last ? slot_last : u);
      pg[tt] = a.plan_pages[plan_base + u];
      pm[tt] = a.plan_masks != nullptr ? static_cast<uint32_t>(a.plan_masks[plan_base + u]) : 0xffu;
      pr[tt] = a.page_rows != nullptr ? a.page_rows[plan_base + u] : 0xffffu;
    }
  };
  // resident windows: their state rides in round trip 1 (an unconditional
  // load, from q when there are none)
  const bool win_res = RES && a.res_win_k != nullptr;
  const int2 wstate = *reinterpret_cast<const int2*>(win_res ? a.res_win_state + 2 * g : static_cast<const int32_t*>(a.q));
  uint4 qf[4];
  {
    const S* qh = static_cast<const S*>(a.q) + (static_cast<int64_t>(g) * R + (krow < R ? krow : 0)) * D + 8 * quarter;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 t = *reinterpret_cast<const uint4*>(qh + 32 * s);
      qf[s] = krow < R ? t : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  // bitmap mode: every head's words of this lane, their OR and the prefix
  // (the query loads above are already in flight)
  constexpr int kNwl = NWL > 0 ? NWL : 1;
  uint64_t hw[RMAX][kNwl], uw[kNwl];
  int b_cnt = 0, b_incl = 0;
  // union record: the group's row masks (up to 4096 NWL pages) staged in
  // LDS by the whole block, loaded in this round trip
  constexpr int kMw4 = MK ? 512 * (NWL > 0 ? NWL : 1) : 1;
  __shared__ __align__(16) uint4 s_mw[kMw4];
  if constexpr (NWL > 0) {
    const uint32_t* brow = a.sel_bits + static_cast<int64_t>(g) * (MK ? 1 : R) * a.bits_stride;
#pragma unroll
    for (int w = 0; w < NWL; ++w) {
      const int wi = NWL * lane + w;
      const int wc = wi < a.bits_w64 ? wi : a.bits_w64 - 1;
      uw[w] = 0ull;
      if constexpr (MK) {
        const uint64_t v = *reinterpret_cast<const uint64_t*>(brow + 2 * wc);
        uw[w] = wi < a.bits_w64 ? v : 0ull;
#pragma unroll
        for (int h = 0; h < RMAX; ++h) hw[h][w] = uw[w];
      } else {
        // Slots h >= R repeat row R - 1: the OR is unchanged and their mask
        // bits are never read.  No uniform condition guards a load, so the
        // compiler cannot sink them into branches that wait one by one.
#pragma unroll
        for (int h = 0; h < RMAX; ++h) {
          const int hc = h < R ? h : R - 1;
          const uint64_t v = *reinterpret_cast<const uint64_t*>(brow + hc * a.bits_stride + 2 * wc);
          hw[h][w] = wi < a.bits_w64 ? v : 0ull;
          uw[w] |= hw[h][w];
        }
      }
      b_cnt += __popcll(uw[w]);
    }
    if constexpr (MK) {
      constexpr int kPer = kMw4 / (NW * kWave);
      static_assert(kPer * NW * kWave == kMw4, "whole mask units per thread");
      const uint4* src = reinterpret_cast<const uint4*>(brow + a.mask_off);
      const int last = a.mask_w4 - 1;
      uint4 mv[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = static_cast<int>(threadIdx.x) + j * NW * kWave;
        mv[j] = src[i < last ? i : last];
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = static_cast<int>(threadIdx.x) + j * NW * kWave;
        s_mw[i] = i <= last ? mv[j] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    b_incl = wave_prefix_sum_i32(b_cnt);
  } else {
    load_slots((chunk * a.iters * NW + wave) * TW, page, pmask, prow);
  }
  const TileWin win = tile_window(a, g);
  int nu;
  if constexpr (NWL > 0) {
    nu = __builtin_amdgcn_readlane(b_incl, kWave - 1);
    nu = nu > win.nu_cap ? win.nu_cap : nu;
    if (chunk == 0 && threadIdx.x == 0) a.union_sizes[g] = nu;
  } else {
    nu = tile_pages(a, g, win);
  }
  const int n_tiles = win.sink_tiles + nu + win.run_tiles;
  const int n_chunks = (n_tiles + per_chunk - 1) / per_chunk;
  if (n_tiles == 0) {
    if (chunk == 0) {
      S* o = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      for (int i = threadIdx.x; i < R * D; i += NW * kWave) o[i] = from_f32(DT{}, 0.0f);
    }
    return;
  }
  if (chunk >= n_chunks) return;
  if constexpr (MK) __syncthreads();  // the staged row masks (every exit above is block-uniform)
  if (chunk == 0) {
    append_decode_token<S>(a, g, D, win.append_position);
    if (a.meta_packed != nullptr)
      complete_row_meta<DT>(a, g, win.append_position);  // the row's INT4 code, then its page
    else
      complete_page_meta<DT>(a, g, win.append_position);
  }

  const S* kg = static_cast<const S*>(a.k) + static_cast<int64_t>(g) * a.entry_stride * D;
  const S* vg = static_cast<const S*>(a.v) + static_cast<int64_t>(g) * a.entry_stride * D;
  const int64_t dec_off = static_cast<int64_t>(win.append_position < 0 ? 0 : win.append_position) * D;
  const S* kdec = a.cur_k != nullptr ? static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D : kg + dec_off;
  const S* vdec = a.cur_v != nullptr ? static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D : vg + dec_off;
  // resident page cache buffers of this group, in rows: previous step's and this step's
  constexpr bool res = RES;
  const int64_t res_base = static_cast<int64_t>(g) * 2 * a.res_slots;
  const int64_t res_prev = (res_base + static_cast<int64_t>((win.length - 1) & 1) * a.res_slots) * kTileRows;
  const int64_t res_cur = (res_base + static_cast<int64_t>(win.length & 1) * a.res_slots) * kTileRows;
  // the sink rows and the recent ring in HBM, when their state serves this
  // launch's length (a state written by this launch never does)
  const bool ring_ok = win_res && wstate.x == win.length;
  const bool sink_ok = ring_ok && wstate.y != 0;
  const int ring_mask = a.ring_rows - 1;
  const int64_t win_base = static_cast<int64_t>(g) * a.win_rows * D;

  float m_run[RMAX];
  float o_acc[RMAX][8];
  float l_part[4];
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
    m_run[h] = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) o_acc[h][i] = 0.0f;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) l_part[v] = 0.0f;

  for (int it = 0; it < a.iters; ++it) {
    const int t0 = ((chunk * a.iters + it) * NW + wave) * TW;
    if constexpr (NWL > 0) {
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        const int u = t0 + tt - win.sink_tiles;  // wave-uniform
        page[tt] = 0;
        pmask[tt] = 0u;
        prow[tt] = 0xffffu;
        if (u >= 0 && u < nu) {
          bits_page<RMAX, kNwl>(u, b_incl, b_cnt, uw, hw, &page[tt], &pmask[tt]);
          if constexpr (MK)
            prow[tt] = (reinterpret_cast<const uint32_t*>(s_mw)[page[tt] >> 1] >> (16 * (page[tt] & 1))) & 0xffffu;
        }
      }
    } else if (it > 0) {
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        page[tt] = page_nx[tt];
        pmask[tt] = pmask_nx[tt];
        prow[tt] = prow_nx[tt];
      }
    }
    if (t0 >= n_tiles) break;
    // ---- round trip 2: K fragments and V rows of the batch ----
    TileSrc ts[TW];
    uint4 kf[TW][4];
    uint4 vf[TW][4];
    // resident page cache: a page stored by the previous step (epoch
    // length - 1) is read from HBM instead of the slab
    int hit_slot[TW];
    uint32_t hit_rows[TW];  // rows of the tile the previous step stored (row-granular over a record)
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      ts[tt] = tile_src(a, win, t0 + tt, nu, page[tt], pmask[tt], prow[tt], MK || a.page_rows != nullptr);
      hit_slot[tt] = -1;
      hit_rows[tt] = 0u;
      if (res && ts[tt].u >= 0 && ts[tt].page >= 0 && ts[tt].page < a.res_map_pages) {
        const int64_t m = a.res_map[static_cast<int64_t>(g) * a.res_map_pages + ts[tt].page];
        const int slot = static_cast<int>(MK ? (m & 0xffffll) : (m & 0xffffffffll));
        if ((m >> 32) == static_cast<int64_t>(win.length) - 1 && slot >= 0 && slot < a.res_slots) {
          hit_slot[tt] = slot;
          hit_rows[tt] = MK ? static_cast<uint32_t>((m >> 16) & 0xffffll) : 0xffffu;
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      const bool hit = hit_slot[tt] >= 0;
      // (wave-uniform) a sink tile or a recent tile served by the HBM windows
      const bool wsink = sink_ok && t0 + tt < win.sink_tiles;
      const bool wring = ring_ok && t0 + tt >= win.sink_tiles + nu;
      const int64_t tb_res = (res_prev + static_cast<int64_t>(hit ? hit_slot[tt] : 0) * kTileRows) * D;
      const int64_t tb_src = ts[tt].pos0 * D + (wsink ? win_base : 0);
      const S* ks = wsink || wring ? static_cast<const S*>(a.res_win_k) : kg;
      const S* vs = wsink || wring ? static_cast<const S*>(a.res_win_v) : vg;
      // rows outside the tile or not kept read a kept row (the same lines,
      // no extra traffic) and are masked below
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * rg + j;
        const int vr = (r < ts[tt].cnt && ((ts[tt].rm >> r) & 1u)) ? r : ts[tt].r0;
        // a row the previous step stored comes from this step's HBM copy
        const bool rh = hit && ((hit_rows[tt] >> vr) & 1u);
        const int64_t ro =
            wring ? win_base + (a.sink + ((ts[tt].pos0 + vr) & ring_mask)) * static_cast<int64_t>(D) + c8
                  : (rh ? tb_res : tb_src) + static_cast<int64_t>(vr) * D + c8;
        const S* kt = rh ? static_cast<const S*>(a.res_k) : ks;
        const S* vt = rh ? static_cast<const S*>(a.res_v) : vs;
        const S* vp = r == ts[tt].dec ? vdec + c8 : vt + ro;
        vf[tt][j] = NT ? load_stream(vp) : *reinterpret_cast<const uint4*>(vp);
        // key row r, channels c8..c8+7, until the LDS pass below
        const S* kp = r == ts[tt].dec ? kdec + c8 : kt + ro;
        kf[tt][j] = NT ? load_stream(kp) : *reinterpret_cast<const uint4*>(kp);
      }
    }
    // the next batch's page slots ride in the same round trip
    if (NWL == 0 && it + 1 < a.iters) load_slots(t0 + NW * TW, page_nx, pmask_nx, prow_nx);
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * rg + j;
        s_k[wave][tt][r][(lane & 15) ^ r] = kf[tt][j];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's key rows are in LDS
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[tt][s] = s_k[wave][tt][krow][(4 * s + quarter) ^ krow];
    }
    // ---- q.k on the matrix cores; scores in log2 units ----
    float sc[TW][4];
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s) H::mfma(qf[s], kf[tt][s], acc);
      const bool ok = krow < ts[tt].cnt && ((ts[tt].rm >> krow) & 1u);
      const uint32_t hm = krow == ts[tt].dec ? 0xffu : ts[tt].hm;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int h = 4 * quarter + v;
        sc[tt][v] = (ok && h < R && ((hm >> h) & 1u)) ? acc[v] * a.scale_log2 : -INFINITY;
      }
    }
    // ---- batch max per head: over the tiles, then the 16 rows of a quarter ----
    float mx[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float x = sc[0][v];
#pragma unroll
      for (int tt = 1; tt < TW; ++tt) x = fmaxf(x, sc[tt][v]);
      x = fmaxf(x, dpp<kQuadXor1>(x));
      x = fmaxf(x, dpp<kQuadXor2>(x));
      x = fmaxf(x, dpp<kRowHalfMirror>(x));
      x = fmaxf(x, dpp<kRowMirror>(x));
      mx[v] = x;
    }
    float alpha[RMAX];
#pragma unroll
    for (int h = 0; h < RMAX; ++h) {
      const float bm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx[h & 3]),
                                                                           16 * (h >> 2)));
      const float mnew = fmaxf(m_run[h], bm);
      alpha[h] = (it == 0 || mnew == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[h] - mnew);
      m_run[h] = mnew;
      if (it > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o_acc[h][i] *= alpha[h];
      }
    }
    // ---- p = exp2(s - m), rounded to the input dtype, into LDS ----
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int h = 4 * quarter + v;
      const float al = NQ > 1 && quarter == 1 ? alpha[(4 + v) % RMAX] : alpha[v];
      const float ml = NQ > 1 && quarter == 1 ? m_run[(4 + v) % RMAX] : m_run[v];
      float psum = 0.0f;
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        const float pv = exp2_rel(sc[tt][v], ml);
        psum += pv;
        if (quarter < NQ) {
          S* sp = reinterpret_cast<S*>(&s_p[wave][tt][krow >> 1][h]);
          sp[krow & 1] = from_f32(DT{}, pv);
        }
      }
      l_part[v] = it == 0 ? psum : l_part[v] * al + psum;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's p stores are done
    __builtin_amdgcn_wave_barrier();
    // ---- p.v over row pairs ----
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        const uint4 va = vf[tt][2 * jp];
        const uint4 vb = vf[tt][2 * jp + 1];
        const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
        const uint32_t wb[4] = {vb.x, vb.y, vb.z, vb.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo[i] = __builtin_amdgcn_perm(wb[i], wa[i], 0x05040100u);  // (row a ch 2i, row b ch 2i)
          hi[i] = __builtin_amdgcn_perm(wb[i], wa[i], 0x07060302u);  // (row a ch 2i+1, row b ch 2i+1)
        }
        uint32_t pp[RMAX];
#pragma unroll
        for (int w = 0; w < PW; ++w) {
          const uint4 t = *reinterpret_cast<const uint4*>(&s_p[wave][tt][2 * rg + jp][4 * w]);
          pp[4 * w] = t.x;
          pp[4 * w + 1] = t.y;
          pp[4 * w + 2] = t.z;
          pp[4 * w + 3] = t.w;
        }
#pragma unroll
        for (int h = 0; h < RMAX; ++h) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            o_acc[h][2 * i] = H::dot2(pp[h], lo[i], o_acc[h][2 * i]);
            o_acc[h][2 * i + 1] = H::dot2(pp[h], hi[i], o_acc[h][2 * i + 1]);
          }
        }
      }
    }
    // ---- resident windows: the sink rows and recent rows read from the slab
    // go to HBM, and the decode row to its ring slot every launch ----
    if (win_res) {
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        const int t = t0 + tt;  // wave-uniform
        const bool sink_tile = t < win.sink_tiles;
        const bool recent_tile = t >= win.sink_tiles + nu && t < n_tiles;
        if (!(sink_tile && !sink_ok) && !recent_tile) continue;
        S* wk = static_cast<S*>(a.res_win_k) + win_base;
        S* wv = static_cast<S*>(a.res_win_v) + win_base;
        auto win_row = [&](int r) -> int64_t {   // window row of tile row r
          const int64_t pos = ts[tt].pos0 + r;
          return sink_tile ? pos : a.sink + (pos & ring_mask);
        };
        auto store_row = [&](int r) -> bool {
          return r < ts[tt].cnt && (sink_tile || !ring_ok || r == ts[tt].dec);
        };
        if (store_row(krow)) {
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4)
            *reinterpret_cast<uint4*>(wk + win_row(krow) * D + 32 * s4 + 8 * quarter) = kf[tt][s4];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * rg + j;
          if (store_row(r)) *reinterpret_cast<uint4*>(wv + win_row(r) * D + c8) = vf[tt][j];
        }
        if (t == n_tiles - 1 && lane == 0) {
          // the group's last tile: the state the next launch checks
          const int ring_len = win.length + win.has_dec;
          const int sink_stored = win.sink_end == a.sink ? 1 : 0;
          *reinterpret_cast<int2*>(a.res_win_state + 2 * g) = make_int2(ring_len, sink_stored);
        }
      }
    }
    // ---- resident page cache: every union page read goes to this step's buffer ----
    if (res) {
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) {
        if (ts[tt].u < 0 || ts[tt].u >= a.res_slots) continue;
        const int64_t db = (res_cur + static_cast<int64_t>(ts[tt].u) * kTileRows) * D;
        S* dk = static_cast<S*>(a.res_k) + db;
        S* dv = static_cast<S*>(a.res_v) + db;
#pragma unroll
        for (int s = 0; s < 4; ++s)
          *reinterpret_cast<uint4*>(dk + krow * D + 32 * s + 8 * quarter) = kf[tt][s];
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(dv + (4 * rg + j) * D + c8) = vf[tt][j];
        if (lane == 0) {
          // (over a record the rows the tile keeps are what this step stored)
          const uint32_t kept = ts[tt].rm & 0xffffu;
          if (ts[tt].page >= 0 && ts[tt].page < a.res_map_pages)
            a.res_map[static_cast<int64_t>(g) * a.res_map_pages + ts[tt].page] =
                (static_cast<int64_t>(win.length) << 32) |
                (MK ? (static_cast<int64_t>(kept) << 16) : 0ll) | static_cast<int64_t>(ts[tt].u);
          if (a.res_stats != nullptr) {
            if constexpr (MK) {
              atomicAdd(a.res_stats + 2 * g + 1, static_cast<unsigned long long>(__popc(kept)));
              if (hit_slot[tt] >= 0)
                atomicAdd(a.res_stats + 2 * g, static_cast<unsigned long long>(__popc(kept & hit_rows[tt])));
            } else {
              atomicAdd(a.res_stats + 2 * g + 1, 1ull);
              if (hit_slot[tt] >= 0) atomicAdd(a.res_stats + 2 * g, 1ull);
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // ---- the wavefront's (m, l, o): o over the 4 row groups, l over 16 rows ----
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = o_acc[h][i];
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      o_acc[h][i] = x;
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) l_part[v] = row_group_sum<16>(l_part[v]);
#pragma unroll
  for (int h = 0; h < RMAX; ++h) {
    const float lh = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_part[h & 3]), 16 * (h >> 2)));
    if (lane == 0) {
      s_m[wave][h] = m_run[h];
      s_l[wave][h] = lh;
    }
    if (lane < 16) {
      *reinterpret_cast<float4*>(&s_o[wave][h][c8]) = make_float4(o_acc[h][0], o_acc[h][1], o_acc[h][2], o_acc[h][3]);
      *reinterpret_cast<float4*>(&s_o[wave][h][c8 + 4]) =
          make_float4(o_acc[h][4], o_acc[h][5], o_acc[h][6], o_acc[h][7]);
    }
  }
  __syncthreads();
  // ---- block combine: the final output (one chunk) or a split-K partial ----
  const bool final_out = n_chunks == 1;
  for (int idx = threadIdx.x; idx < R * D; idx += NW * kWave) {
    const int r = idx / D;
    const int c = idx - r * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = exp2_rel(s_m[w][r], M);
      L += f * s_l[w][r];
      O += f * s_o[w][r][c];
    }
    if (final_out) {
      S* out = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      out[idx] = from_f32(DT{}, L > 0.0f ? O / L : 0.0f);
    } else {
      const int64_t pc = static_cast<int64_t>(g) * a.max_chunks + chunk;
      a.part_o[pc * R * D + idx] = O;
      if (c == 0) *reinterpret_cast<float2*>(a.part_ml + (pc * R + r) * 2) = make_float2(M, L);
    }
  }
}

// Generic head dimension (any even D <= 512): one row per wavefront step,
// lane owns channels lane + 64 j.  Correctness path for unusual shapes.
template <typename DT, int RMAX, int MODE>
__global__ __launch_bounds__(kBlock) void decode_attn_generic(AttnArgs a) {
  using S = typename DT::storage;
  constexpr int JMAX = 8;  // D <= 512
  const int R = a.R;
  const int D = a.D;
  const int g = static_cast<int>(blockIdx.x) % a.G;  // chunk-major (group g on XCD g % 8)
  const int chunk = static_cast<int>(blockIdx.x) / a.G;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  __shared__ float s_m[kWaves * RMAX];
  __shared__ float s_l[kWaves * RMAX];
  extern __shared__ __align__(16) float s_dyn[];

  const GroupRows gr = group_rows<MODE>(a, g, D);
  const int rows_per_block = kWaves * 16 * a.iters;
  const int n_chunks = (gr.n_rows + rows_per_block - 1) / rows_per_block;
  if (gr.n_rows == 0) {
    if (chunk == 0) {
      S* o = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      for (int i = threadIdx.x; i < R * D; i += kBlock) o[i] = from_f32(DT{}, 0.0f);
    }
    return;
  }
  if (chunk >= n_chunks) return;
  if ((MODE == kModePages || MODE == kModeRows) && chunk == 0) {
    append_decode_token<S>(a, g, D, decode_row_position<MODE>(a, g));
    if (MODE == kModeRows) complete_row_meta<DT>(a, g, decode_row_position<MODE>(a, g));
  }
  const S* kbase = static_cast<const S*>(a.k);
  const S* vbase = static_cast<const S*>(a.v);
  const S* qg = static_cast<const S*>(a.q) + static_cast<int64_t>(g) * R * D;
  float m_run[RMAX], l_run[RMAX], o_acc[RMAX][JMAX];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < JMAX; ++j) o_acc[r][j] = 0.0f;
  }
  const int first = chunk * rows_per_block;
  const int last = min(first + rows_per_block, gr.n_rows);
  for (int i = first + wave; i < last; i += kWaves) {
    const S* kp;
    const S* vp;
    uint32_t m = 0xffu;
    bool ok = true;
    if (i >= gr.n_list) {
      kp = static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D;
      vp = static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D;
    } else {
      int64_t pos;
      if (MODE == kModeRows) {
        const int64_t at = static_cast<int64_t>(g) * a.rows_stride + i;
        pos = a.rows[at];
        if (a.masks != nullptr) m = a.masks[at];
        if (pos < 0 || pos >= a.entry_stride) ok = false;
      } else if (MODE == kModePages) {
        if (i < gr.sink_end) {
          pos = i;
        } else if (i < gr.page_end) {
          const int j = i - gr.sink_end;
          const int u = j / a.bs;
          const int64_t at = static_cast<int64_t>(g) * a.plan_stride + u;
          pos = a.sink + static_cast<int64_t>(a.plan_pages[at]) * a.bs + (j - u * a.bs);
          if (a.plan_masks != nullptr) m = a.plan_masks[at];
        } else if (i < gr.recent_end) {
          pos = gr.recent_start + (i - gr.page_end);
        } else {
          pos = a.append_position;
        }
        if (pos < 0 || pos >= a.entry_stride) ok = false;
      } else {
        pos = gr.win_start + i;
      }
      if (!ok) continue;
      kp = kbase + gr.base + pos * gr.stride;
      vp = vbase + gr.base + pos * gr.stride;
    }
    float s[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      float acc = 0.0f;
      if (r < R) {
#pragma unroll
        for (int j = 0; j < JMAX; ++j) {
          const int c = lane + kWave * j;
          if (c < D) acc = __builtin_fmaf(to_f32(DT{}, qg[r * D + c]) * a.scale_log2, to_f32(DT{}, kp[c]), acc);
        }
      }
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) acc += __shfl_xor(acc, o);
      s[r] = (r < R && ((m >> r) & 1u)) ? acc : -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      const float mn = fmaxf(m_run[r], s[r]);
      const float alpha = (mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[r] - mn);
      const float p = exp2_rel(s[r], mn);
      m_run[r] = mn;
      l_run[r] = l_run[r] * alpha + p;
#pragma unroll
      for (int j = 0; j < JMAX; ++j) {
        const int c = lane + kWave * j;
        const float vf = c < D ? to_f32(DT{}, vp[c]) : 0.0f;
        o_acc[r][j] = o_acc[r][j] * alpha + p * vf;
      }
    }
  }
  float* s_o = s_dyn;
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    if (lane == 0) {
      s_m[wave * RMAX + r] = m_run[r];
      s_l[wave * RMAX + r] = l_run[r];
    }
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      const int c = lane + kWave * j;
      if (c < D) s_o[(wave * RMAX + r) * D + c] = o_acc[r][j];
    }
  }
  __syncthreads();
  block_partial<DT, RMAX>(a, g, chunk, D, n_chunks == 1, s_m, s_l, s_o);
}

bool fast_d(int D) { return D == 64 || D == 128 || D == 256; }

int rmax_for(int R) { return R <= 1 ? 1 : (R <= 2 ? 2 : (R <= 4 ? 4 : 8)); }

// Rows of one block batch.
// The matrix-core kernel serves 16-bit K/V at D in {64, 128, 256}, R <= 8.
bool use_mfma(int dtype, int D, int R) { return dtype != TW_DTYPE_F32 && fast_d(D) && R <= 8; }

int rows_per_batch(int dtype, int D, int R) {
  if (!fast_d(D)) return kWaves * 16;
  if (use_mfma(dtype, D, R)) return kWaves * 16 * mfma_tiles(D, rmax_for(R) < 4 ? 4 : rmax_for(R));
  const int lpr = D / 8;
  const int rpi = kWave / lpr;
  return kWaves * steps_for(dtype == TW_DTYPE_F32 ? 4 : 2, rmax_for(R)) * rpi;
}

// Batches per block and chunks per group for a bound on the rows.  About
// 1024 blocks fill the chip (3 resident blocks per CU); a group never has
// more than kMaxChunks chunks, so the last block merges every partial in at
// most two batched round trips.
void plan_chunks(int dtype, int G, int R, int D, int max_rows_total, int* iters, int* chunks) {
  const int rb = rows_per_batch(dtype, D, R);
  int target = 1024 / (G > 0 ? G : 1);
  target = target < 1 ? 1 : (target > kMaxChunks ? kMaxChunks : target);
  int it = (max_rows_total + rb * target - 1) / (rb * target);
  it = it < 1 ? 1 : it;
  int ch = (max_rows_total + rb * it - 1) / (rb * it);
  *iters = it;
  *chunks = ch < 1 ? 1 : ch;
}

// Page-tile kernel shape: waves per block and tiles per wavefront batch (one
// tile a wavefront: with a group's blocks on one XCD, twice the blocks of
// half the rows balance its CUs better than two tiles a wavefront)
#ifndef TW_TILE_NW
#define TW_TILE_NW 4
#endif
#ifndef TW_TILE_TW
#define TW_TILE_TW 1
#endif
// blocks per (group, head) of the split-K merge at D = 128, each over
// D / TW_MERGE_CS channels (4: the page-tile merge 4.0 -> 3.45 us at 32K, each
// thread 8 loads instead of 32)
#ifndef TW_MERGE_CS
#define TW_MERGE_CS 4
#endif
constexpr int kTileNW = TW_TILE_NW;
constexpr int kTileTW = TW_TILE_TW;

// Batches per block and chunks per group of the page-tile kernel for a bound
// on the rows (decode token included).  The tile count is bounded by
// max_rows / 16 + 3 (the sink and the recent run each round up once), and the
// plan depends on max_rows only, so the workspace query and the launch agree.
void plan_tile_chunks(int G, int max_rows_total, int* iters, int* chunks) {
  const int mt = max_rows_total / kTileRows + 3;
  const int tpb = kTileNW * kTileTW;
  int target = 1024 / (G > 0 ? G : 1);
  target = target < 1 ? 1 : (target > kMaxChunks ? kMaxChunks : target);
  int it = (mt + tpb * target - 1) / (tpb * target);
  it = it < 1 ? 1 : it;
  const int ch = (mt + tpb * it - 1) / (tpb * it);
  *iters = it;
  *chunks = ch < 1 ? 1 : ch;
}

template <typename DT, int RMAX, bool RES, bool NT>
void launch_tiles_nwl(const AttnArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  const int nwl = a.sel_bits == nullptr ? 0 : (a.bits_w64 <= kWave ? 1 : 2);
  if (a.union_rec && nwl == 1)
    hipLaunchKernelGGL((decode_attn_tiles<DT, RMAX, kTileNW, kTileTW, RES, NT, 1, true>), grid, block, 0, stream, a);
  else if (a.union_rec)
    hipLaunchKernelGGL((decode_attn_tiles<DT, RMAX, kTileNW, kTileTW, RES, NT, 2, true>), grid, block, 0, stream, a);
  else if (nwl == 0)
    hipLaunchKernelGGL((decode_attn_tiles<DT, RMAX, kTileNW, kTileTW, RES, NT, 0>), grid, block, 0, stream, a);
  else if (nwl == 1)
    hipLaunchKernelGGL((decode_attn_tiles<DT, RMAX, kTileNW, kTileTW, RES, NT, 1>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((decode_attn_tiles<DT, RMAX, kTileNW, kTileTW, RES, NT, 2>), grid, block, 0, stream, a);
}

template <typename DT>
int launch_tiles(const AttnArgs& a, hipStream_t stream) {
  const int phase = a.phase == 0 ? 3 : a.phase;
  if (phase & 1) {
    const dim3 grid(a.G * a.max_chunks);
    const dim3 block(kTileNW * kWave);
    // the resident page cache serves slabs in host memory: plain loads, over
    // a union plan (whole pages) or a union record (kept rows)
    if (a.res_map != nullptr && a.union_rec) {
      const bool one = a.bits_w64 <= kWave;
      if (a.R <= 4 && one)
        hipLaunchKernelGGL((decode_attn_tiles<DT, 4, kTileNW, kTileTW, true, false, 1, true>), grid, block, 0, stream, a);
      else if (a.R <= 4)
        hipLaunchKernelGGL((decode_attn_tiles<DT, 4, kTileNW, kTileTW, true, false, 2, true>), grid, block, 0, stream, a);
      else if (one)
        hipLaunchKernelGGL((decode_attn_tiles<DT, 8, kTileNW, kTileTW, true, false, 1, true>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((decode_attn_tiles<DT, 8, kTileNW, kTileTW, true, false, 2, true>), grid, block, 0, stream, a);
    } else if (a.res_map != nullptr) {
      if (a.R <= 4)
        hipLaunchKernelGGL((decode_attn_tiles<DT, 4, kTileNW, kTileTW, true, false, 0>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((decode_attn_tiles<DT, 8, kTileNW, kTileTW, true, false, 0>), grid, block, 0, stream, a);
    } else if (a.kv_stream) {
      if (a.R <= 4)
        launch_tiles_nwl<DT, 4, false, true>(a, grid, block, stream);
      else
        launch_tiles_nwl<DT, 8, false, true>(a, grid, block, stream);
    } else if (a.R <= 4) {
      launch_tiles_nwl<DT, 4, false, false>(a, grid, block, stream);
    } else {
      launch_tiles_nwl<DT, 8, false, false>(a, grid, block, stream);
    }
    const int rc = tw_host::check_launch();
    if (rc != TW_OK) return rc;
  }
  if (!(phase & 2) || a.max_chunks <= 1) return TW_OK;
  hipLaunchKernelGGL((merge_vec_kernel<DT, kModeTiles, kTileD, TW_MERGE_CS>), dim3(a.G * a.R * TW_MERGE_CS),
                     dim3(kBlock), 0, stream, a,
                     kTileNW * kTileTW * a.iters);
  return tw_host::check_launch();
}

size_t dyn_lds_bytes(int R, int D) { return static_cast<size_t>(kWaves) * rmax_for(R) * D * sizeof(float); }

template <typename DT, int D, int RMAX, int MODE>
int launch_one(const AttnArgs& a, hipStream_t stream) {
  const int phase = a.phase == 0 ? 3 : a.phase;
  size_t lds = dyn_lds_bytes(a.R, a.D);
  const dim3 grid(a.G * a.max_chunks);
  if (!(phase & 1)) {
    // merge only: the partials of an earlier phase-1 launch with the same arguments
  } else if constexpr (D > 0 && !std::is_same<DT, F32>::value) {
    constexpr int RM = RMAX < 4 ? 4 : RMAX;
    lds = static_cast<size_t>(kWaves) * RM * D * sizeof(float);
    auto kern = decode_attn_mfma<DT, D, RM, MODE>;
    if (lds > 64 * 1024)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds));
    hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, stream, a);
  } else if constexpr (D > 0) {
    auto kern = decode_attn_kernel<DT, D, RMAX, MODE>;
    if (lds > 64 * 1024)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds));
    hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, stream, a);
  } else {
    auto kern = decode_attn_generic<DT, RMAX, MODE>;
    if (lds > 64 * 1024)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds));
    hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, stream, a);
  }
  int rc = tw_host::check_launch();
  if (rc != TW_OK || !(phase & 2) || a.max_chunks <= 1) return rc;
  // a block must cover every chunk with one (m, l) per thread
  int threads = ((a.D + kWave - 1) / kWave) * kWave;
  threads = threads < a.max_chunks ? ((a.max_chunks + kWave - 1) / kWave) * kWave : threads;
  const int rpb = rows_per_batch(DT::code, a.D, a.R) * a.iters;
  if constexpr (D == 64 || D == 128 || D == 256) {
    constexpr int CS = D == 128 ? TW_MERGE_CS : 1;  // channel slices (a 64-lane serial sum past 4)
    hipLaunchKernelGGL((merge_vec_kernel<DT, MODE, D, CS>), dim3(a.G * a.R * CS), dim3(kBlock), 0, stream, a, rpb);
    return tw_host::check_launch();
  }
  if (a.max_chunks <= 64) {
    hipLaunchKernelGGL((merge_kernel<DT, MODE, 64>), dim3(a.G * a.R), dim3(threads), 0, stream, a, rpb);
  } else {
    hipLaunchKernelGGL((merge_kernel<DT, MODE, kMaxChunks>), dim3(a.G * a.R), dim3(threads), 0, stream, a, rpb);
  }
  return tw_host::check_launch();
}

template <typename DT, int D, int MODE>
int launch_r(const AttnArgs& a, hipStream_t stream) {
  switch (rmax_for(a.R)) {
    case 1: return launch_one<DT, D, 1, MODE>(a, stream);
    case 2: return launch_one<DT, D, 2, MODE>(a, stream);
    case 4: return launch_one<DT, D, 4, MODE>(a, stream);
    default: return launch_one<DT, D, 8, MODE>(a, stream);
  }
}

template <typename DT, int MODE>
int launch_d(const AttnArgs& a, hipStream_t stream) {
  switch (a.D) {
    case 64: return launch_r<DT, 64, MODE>(a, stream);
    case 128: return launch_r<DT, 128, MODE>(a, stream);
    case 256: return launch_r<DT, 256, MODE>(a, stream);
    default: return launch_r<DT, 0, MODE>(a, stream);
  }
}

template <typename DT>
int launch_mode(const AttnArgs& a, hipStream_t stream) {
  if (a.plan_pages != nullptr) return launch_d<DT, kModePages>(a, stream);
  return a.rows != nullptr ? launch_d<DT, kModeRows>(a, stream) : launch_d<DT, kModeVarlen>(a, stream);
}

int launch_dtype(int dtype, const AttnArgs& a, hipStream_t s) {
  switch (dtype) {
    case TW_DTYPE_F16: return launch_mode<F16>(a, s);
    case TW_DTYPE_BF16: return launch_mode<BF16>(a, s);
    default: return launch_mode<F32>(a, s);
  }
}

size_t counter_bytes(int G) { return ((static_cast<size_t>(G) * 4 + 255) / 256) * 256; }

// Workspace layout: union sizes | part_ml | part_o, sized for the largest chunk
// count any dtype can produce for max_rows (+1 decode token).
void workspace_layout(int G, int R, int D, int max_rows, size_t* ml_off, size_t* o_off, size_t* total) {
  // The chunk count is not monotonic in the row bound (more rows can mean
  // more batches per block and fewer chunks), so take the largest over both
  // bounds a launch may use, with and without the decode token.
  int chunks_max = 1;
  for (int dt : {TW_DTYPE_F16, TW_DTYPE_F32}) {
    for (int extra = 0; extra <= 1; ++extra) {
      int it, ch;
      plan_chunks(dt, G, R, D, max_rows + extra, &it, &ch);
      chunks_max = ch > chunks_max ? ch : chunks_max;
    }
  }
  {
    int it, ch;
    plan_tile_chunks(G, max_rows + 1, &it, &ch);
    chunks_max = ch > chunks_max ? ch : chunks_max;
  }
  const size_t chunks = static_cast<size_t>(chunks_max);
  const size_t ml = static_cast<size_t>(G) * chunks * R * 2 * sizeof(float);
  *ml_off = counter_bytes(G);
  *o_off = *ml_off + ((ml + 255) / 256) * 256;
  *total = *o_off + static_cast<size_t>(G) * chunks * R * D * sizeof(float);
}

}  // namespace
}  // namespace tw

extern "C" size_t tw_decode_attention_workspace_size(int G, int R, int D, int max_rows) {
  if (G <= 0 || R <= 0 || D <= 0 || max_rows < 0) return 0;
  size_t ml, o, total;
  tw::workspace_layout(G, R, D, max_rows, &ml, &o, &total);
  return total;
}

namespace {
// Rows / varlen launch shared by tw_decode_attention and
// tw_decode_attention_rows_append (append_position >= 0: chunk 0 of every
// group writes cur_k/cur_v[g] to that row of its entry).
int rows_launch(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D,
                const int32_t* rows, const uint8_t* row_masks, const int32_t* row_counts, int64_t rows_stride,
                int64_t entry_stride_rows, const int32_t* cu_seqlens_k, int Hk, int window_left, int max_rows,
                const void* cur_k, const void* cur_v, int64_t append_position, const int32_t* append_rows,
                float softmax_scale, void* out, void* workspace, size_t workspace_bytes, void* stream,
                const tw::RowMeta* meta = nullptr) {
  if (q == nullptr || out == nullptr || G <= 0 || R <= 0 || R > 8 || D <= 0 || D > 512 || (D % 2) != 0 ||
      max_rows < 0)
    return TW_EINVAL;
  if (dtype != TW_DTYPE_F16 && dtype != TW_DTYPE_BF16 && dtype != TW_DTYPE_F32) return TW_EINVAL;
  if ((cur_k == nullptr) != (cur_v == nullptr)) return TW_EINVAL;
  if (max_rows > 0 && (k_base == nullptr || v_base == nullptr)) return TW_EINVAL;
  if (rows != nullptr) {
    // rows_stride >= 1: every block may read entry 0 of its group's list.
    if (row_counts == nullptr || rows_stride < max_rows || rows_stride < 1 || entry_stride_rows <= 0)
      return TW_EINVAL;
  } else {
    if (row_masks != nullptr || cu_seqlens_k == nullptr || Hk <= 0 || (G % Hk) != 0) return TW_EINVAL;
  }
  const int es = dtype == TW_DTYPE_F32 ? 4 : 2;
  if (tw::fast_d(D)) {
    const uintptr_t align = 16;
    if ((reinterpret_cast<uintptr_t>(q) % align) || (reinterpret_cast<uintptr_t>(k_base) % align) ||
        (reinterpret_cast<uintptr_t>(v_base) % align) || (cur_k && (reinterpret_cast<uintptr_t>(cur_k) % align)) ||
        (cur_v && (reinterpret_cast<uintptr_t>(cur_v) % align)))
      return TW_EINVAL;
    if (rows == nullptr && ((static_cast<int64_t>(Hk) * D * es) % 16) != 0) return TW_EINVAL;
  }
  size_t ml_off, o_off, total;
  tw::workspace_layout(G, R, D, max_rows, &ml_off, &o_off, &total);
  if (workspace == nullptr || workspace_bytes < total) return TW_ENOMEM;
  tw::AttnArgs a{};
  a.q = q;
  a.k = k_base;
  a.v = v_base;
  a.G = G;
  a.R = R;
  a.D = D;
  a.rows = rows;
  a.masks = row_masks;
  a.counts = row_counts;
  a.rows_stride = rows_stride;
  a.entry_stride = entry_stride_rows;
  a.cu_k = cu_seqlens_k;
  a.Hk = Hk > 0 ? Hk : 1;
  a.window_left = window_left;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  a.scale_log2 = softmax_scale * tw::kLog2e;
  a.out = out;
  a.union_sizes = static_cast<int32_t*>(workspace);
  a.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ml_off);
  a.part_o = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + o_off);
  a.max_rows = max_rows;
  a.append_position = -1;
  if (append_position >= 0) {
    a.k_append = const_cast<void*>(k_base);
    a.v_append = const_cast<void*>(v_base);
    a.append_position = static_cast<int>(append_position);
    a.lengths = append_rows;  // rows mode: per-group append rows
    if (meta != nullptr) {
      a.sink = meta->sink;
      a.meta_min = meta->page_min;
      a.meta_max = meta->page_max;
      a.meta_stride = meta->page_stride;
      a.meta_pages = meta->pages;
      a.meta_packed = meta->packed;
      a.meta_qscale = meta->qscale;
      a.meta_qmin = meta->qmin;
      a.meta_qstride = meta->qstride;
    }
  }
  tw::plan_chunks(dtype, G, R, D, max_rows + (cur_k != nullptr ? 1 : 0), &a.iters, &a.max_chunks);
  return tw::launch_dtype(dtype, a, static_cast<hipStream_t>(stream));
}
}  // namespace

extern "C" int tw_decode_attention(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                   int D, const int32_t* rows, const uint8_t* row_masks, const int32_t* row_counts,
                                   int64_t rows_stride, int64_t entry_stride_rows, const int32_t* cu_seqlens_k,
                                   int Hk, int window_left, int max_rows, const void* cur_k, const void* cur_v,
                                   float softmax_scale, void* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  return rows_launch(q, k_base, v_base, dtype, G, R, D, rows, row_masks, row_counts, rows_stride, entry_stride_rows,
                     cu_seqlens_k, Hk, window_left, max_rows, cur_k, cur_v, -1, nullptr, softmax_scale, out,
                     workspace, workspace_bytes, stream);
}

extern "C" int tw_decode_attention_rows_append(
    const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D, const int32_t* rows,
    const uint8_t* row_masks, const int32_t* row_counts, int64_t rows_stride, int64_t entry_stride_rows,
    int max_rows, const void* cur_k, const void* cur_v, int64_t append_position, const int32_t* append_rows,
    float softmax_scale, int sink, void* page_min, void* page_max, int64_t page_entry_stride, int meta_pages,
    uint8_t* packed, void* quant_scale, void* quant_min, int64_t quant_entry_stride, void* out, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (rows == nullptr || cur_k == nullptr || cur_v == nullptr) return TW_EINVAL;
  if (append_rows == nullptr &&
      (append_position < 0 || append_position >= entry_stride_rows || append_position > INT32_MAX))
    return TW_EINVAL;
  const bool meta = page_min != nullptr || packed != nullptr;
  if (meta) {
    if (dtype == TW_DTYPE_F32 || D != 128 || sink < 0) return TW_EUNSUPPORTED;
    if (page_min != nullptr && (page_max == nullptr || meta_pages < 1 || page_entry_stride < 128ll * meta_pages))
      return TW_EINVAL;
    if (packed != nullptr && (quant_scale == nullptr || quant_min == nullptr || quant_entry_stride < entry_stride_rows))
      return TW_EINVAL;
    if ((reinterpret_cast<uintptr_t>(cur_k) % 4) || (reinterpret_cast<uintptr_t>(page_min) % 4) ||
        (reinterpret_cast<uintptr_t>(page_max) % 4))
      return TW_EINVAL;
  }
  tw::RowMeta m{sink, page_min, page_max, page_entry_stride, meta_pages, packed, quant_scale, quant_min,
                quant_entry_stride};
  return rows_launch(q, k_base, v_base, dtype, G, R, D, rows, row_masks, row_counts, rows_stride, entry_stride_rows,
                     nullptr, 0, -1, max_rows, cur_k, cur_v, append_rows != nullptr ? 0 : append_position,
                     append_rows, softmax_scale, out, workspace, workspace_bytes, stream, meta ? &m : nullptr);
}

extern "C" int tw_decode_attention_pages(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                         int R, int D, const int32_t* plan_pages, const uint8_t* plan_masks,
                                         const int32_t* plan_counts, int64_t plan_stride, int max_rows,
                                         int64_t entry_stride_rows, int sink, int recent, int block_size,
                                         int length, int append_position, const void* cur_k, const void* cur_v,
                                         float softmax_scale, void* out, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  return tw_decode_attention_pages_phase(q, k_base, v_base, dtype, G, R, D, plan_pages, plan_masks, plan_counts,
                                         plan_stride, max_rows, entry_stride_rows, sink, recent, block_size, length,
                                         append_position, cur_k, cur_v, softmax_scale, out, workspace,
                                         workspace_bytes, 3, stream);
}

extern "C" int tw_decode_attention_pages_phase(const void* q, const void* k_base, const void* v_base, int dtype,
                                               int G, int R, int D, const int32_t* plan_pages,
                                               const uint8_t* plan_masks, const int32_t* plan_counts,
                                               int64_t plan_stride, int max_rows, int64_t entry_stride_rows,
                                               int sink, int recent, int block_size, int length,
                                               int append_position, const void* cur_k, const void* cur_v,
                                               float softmax_scale, void* out, void* workspace,
                                               size_t workspace_bytes, int phase, void* stream) {
  if (phase < 1 || phase > 3) return TW_EINVAL;
  if (q == nullptr || out == nullptr || k_base == nullptr || v_base == nullptr || G <= 0 || R <= 0 || R > 8 ||
      D <= 0 || D > 512 || (D % 2) != 0 || max_rows < 0)
    return TW_EINVAL;
  if (dtype != TW_DTYPE_F16 && dtype != TW_DTYPE_BF16 && dtype != TW_DTYPE_F32) return TW_EINVAL;
  if (plan_pages == nullptr || plan_counts == nullptr || plan_stride < 1 || entry_stride_rows <= 0) return TW_EINVAL;
  if (sink < 0 || recent <= 0 || block_size <= 0 || length < 0 || append_position >= entry_stride_rows)
    return TW_EINVAL;
  if ((cur_k == nullptr) != (cur_v == nullptr)) return TW_EINVAL;
  if (tw::fast_d(D)) {
    const uintptr_t align = 16;
    if ((reinterpret_cast<uintptr_t>(q) % align) || (reinterpret_cast<uintptr_t>(k_base) % align) ||
        (reinterpret_cast<uintptr_t>(v_base) % align) || (reinterpret_cast<uintptr_t>(cur_k) % align) ||
        (reinterpret_cast<uintptr_t>(cur_v) % align))
      return TW_EINVAL;
  }
  size_t ml_off, o_off, total;
  tw::workspace_layout(G, R, D, max_rows, &ml_off, &o_off, &total);
  if (workspace == nullptr || workspace_bytes < total) return TW_ENOMEM;
  tw::AttnArgs a{};
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  if (cur_k != nullptr && append_position >= 0) {
    a.k_append = const_cast<void*>(k_base);
    a.v_append = const_cast<void*>(v_base);
  }
  a.q = q;
  a.k = k_base;
  a.v = v_base;
  a.G = G;
  a.R = R;
  a.D = D;
  a.entry_stride = entry_stride_rows;
  a.plan_pages = plan_pages;
  a.plan_masks = plan_masks;
  a.plan_counts = plan_counts;
  a.plan_stride = plan_stride;
  a.sink = sink;
  a.recent = recent;
  a.bs = block_size;
  a.length = length;
  a.append_position = append_position;
  a.Hk = 1;
  a.window_left = -1;
  a.scale_log2 = softmax_scale * tw::kLog2e;
  a.out = out;
  a.union_sizes = static_cast<int32_t*>(workspace);
  a.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ml_off);
  a.part_o = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + o_off);
  a.max_rows = max_rows;
  a.phase = phase;
  // 16-row pages at D = 128 in a 16-bit dtype take the page-tile kernel
  // (the sink, recent and decode rows must fit max_rows, as the plan bound
  // promises); every other shape the row kernels.
  const int sink_end = sink < length ? sink : length;
  const int hist_recent = recent - 1 > 0 ? recent - 1 : 0;
  const int recent_start = length - hist_recent > sink_end ? length - hist_recent : sink_end;
  const int has_dec = (cur_k != nullptr || append_position >= 0) ? 1 : 0;
  const int run = (length - recent_start) + has_dec;
  if (dtype != TW_DTYPE_F32 && D == tw::kTileD && block_size == tw::kTileRows && length <= entry_stride_rows &&
      max_rows >= sink_end + run) {
    tw::plan_tile_chunks(G, max_rows, &a.iters, &a.max_chunks);
    a.t_sink_tiles = (sink_end + tw::kTileRows - 1) / tw::kTileRows;
    a.t_sink_end = sink_end;
    a.t_recent_start = recent_start;
    a.t_n_recent = length - recent_start;
    a.t_has_dec = has_dec;
    a.t_run = run;
    a.t_run_tiles = (run + tw::kTileRows - 1) / tw::kTileRows;
    a.t_per_chunk = a.iters * tw::kTileNW * tw::kTileTW;
    const int64_t capacity = static_cast<int64_t>(a.max_chunks) * a.t_per_chunk;
    int64_t cap = (max_rows - sink_end - run) / tw::kTileRows;
    const int64_t room = capacity - a.t_sink_tiles - a.t_run_tiles;
    cap = cap < room ? cap : room;
    cap = cap < plan_stride ? cap : plan_stride;
    a.t_nu_cap = static_cast<int>(cap < 0 ? 0 : cap);
    a.kv_stream = tw_host::device_memory(k_base) && tw_host::device_memory(v_base);
    return dtype == TW_DTYPE_F16 ? tw::launch_tiles<tw::F16>(a, static_cast<hipStream_t>(stream))
                                 : tw::launch_tiles<tw::BF16>(a, static_cast<hipStream_t>(stream));
  }
  tw::plan_chunks(dtype, G, R, D, max_rows, &a.iters, &a.max_chunks);
  return tw::launch_dtype(dtype, a, static_cast<hipStream_t>(stream));
}

namespace tw {
namespace {

// Page-tile launch with per-group lengths from the device (lengths != NULL)
// or one host length for every group, optionally with the resident page cache.
int pages_tiles_launch(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D,
                       const int32_t* plan_pages, const uint8_t* plan_masks, const int32_t* plan_counts,
                       int64_t plan_stride, int max_rows, int64_t entry_stride_rows, int sink, int recent,
                       int block_size, const int32_t* lengths, int length, int append, const void* cur_k,
                       const void* cur_v, float softmax_scale, void* res_k, void* res_v, int64_t* res_map,
                       int res_slots, int res_map_pages, unsigned long long* res_stats, void* page_min,
                       void* page_max, int64_t page_entry_stride, int meta_pages, void* out, void* workspace,
                       size_t workspace_bytes, void* stream, const uint32_t* page_rows = nullptr,
                       uint8_t* packed = nullptr, void* qscale = nullptr, void* qmin = nullptr,
                       int64_t quant_entry_stride = 0, const uint32_t* sel_bits = nullptr, int64_t bits_stride = 0,
                       int bits_pages = 0, int phase = 3, int union_rec = 0, void* res_win_k = nullptr,
                       void* res_win_v = nullptr, int32_t* res_win_state = nullptr, int ring_rows = 0) {
  if (q == nullptr || out == nullptr || k_base == nullptr || v_base == nullptr) return TW_EINVAL;
  if (page_rows != nullptr && res_map != nullptr) return TW_EINVAL;  // the resident cache keeps whole pages
  if (packed != nullptr &&
      (qscale == nullptr || qmin == nullptr || cur_k == nullptr || append == 0 || quant_entry_stride < entry_stride_rows))
    return TW_EINVAL;
  if (page_min != nullptr &&
      (page_max == nullptr || append == 0 || meta_pages < 1 ||
       page_entry_stride < static_cast<int64_t>(meta_pages) * kTileD ||
       (reinterpret_cast<uintptr_t>(page_min) % 4) || (reinterpret_cast<uintptr_t>(page_max) % 4)))
    return TW_EINVAL;
  if (G <= 0 || R <= 0 || R > 8 || phase < 1 || phase > 3) return TW_EINVAL;
  if (sel_bits != nullptr) {
    // selection bitmaps of bits_pages pages: at most 128 64-bit words a row
    // (two per lane), 8-byte aligned rows
    // (the resident cache takes a union record, whose slots fit 16 bits)
    if (bits_pages < 1 || bits_pages > 128 * 64 || page_rows != nullptr ||
        (res_map != nullptr && (!union_rec || res_slots > 0xffff)))
      return TW_EINVAL;
    if (bits_stride < 2 * ((bits_pages + 63) / 64) || (bits_stride % 2) != 0 ||
        (reinterpret_cast<uintptr_t>(sel_bits) % 8) != 0)
      return TW_EINVAL;
    if (union_rec && (bits_stride < union_record_words(bits_pages) || (bits_stride % 4) != 0 ||
                      (reinterpret_cast<uintptr_t>(sel_bits) % 16) != 0))
      return TW_EINVAL;
    plan_stride = bits_pages;  // the union has at most this many pages
  } else if (plan_pages == nullptr || plan_counts == nullptr || plan_stride < 1) {
    return TW_EINVAL;
  }
  if (dtype != TW_DTYPE_F16 && dtype != TW_DTYPE_BF16) return TW_EUNSUPPORTED;
  if (D != kTileD || block_size != kTileRows) return TW_EUNSUPPORTED;
  if (sink < 0 || recent <= 0 || entry_stride_rows < 2 || entry_stride_rows > (1ll << 30)) return TW_EINVAL;
  if (max_rows < sink + recent) return TW_EINVAL;
  if ((cur_k == nullptr) != (cur_v == nullptr)) return TW_EINVAL;
  if (lengths == nullptr && (length < 0 || length + 1 > entry_stride_rows)) return TW_EINVAL;
  if (res_map != nullptr && (res_k == nullptr || res_v == nullptr || res_slots < 1 || res_map_pages < 1))
    return TW_EINVAL;
  // resident windows: with the page cache; a ring of a power of two rows
  // holding the recent window and the decode row
  if (res_win_k != nullptr &&
      (res_map == nullptr || res_win_v == nullptr || res_win_state == nullptr || ring_rows < recent ||
       (ring_rows & (ring_rows - 1)) != 0 || (reinterpret_cast<uintptr_t>(res_win_k) % 16) ||
       (reinterpret_cast<uintptr_t>(res_win_v) % 16) || (reinterpret_cast<uintptr_t>(res_win_state) % 8)))
    return TW_EINVAL;
  const uintptr_t align = 16;
  if ((reinterpret_cast<uintptr_t>(q) % align) || (reinterpret_cast<uintptr_t>(k_base) % align) ||
      (reinterpret_cast<uintptr_t>(v_base) % align) || (reinterpret_cast<uintptr_t>(cur_k) % align) ||
      (reinterpret_cast<uintptr_t>(cur_v) % align) || (reinterpret_cast<uintptr_t>(res_k) % align) ||
      (reinterpret_cast<uintptr_t>(res_v) % align))
    return TW_EINVAL;
  size_t ml_off, o_off, total;
  workspace_layout(G, R, D, max_rows, &ml_off, &o_off, &total);
  if (workspace == nullptr || workspace_bytes < total) return TW_ENOMEM;
  AttnArgs a{};
  a.q = q;
  a.k = k_base;
  a.v = v_base;
  a.G = G;
  a.R = R;
  a.D = D;
  a.entry_stride = entry_stride_rows;
  a.plan_pages = plan_pages;
  a.plan_masks = plan_masks;
  a.plan_counts = plan_counts;
  a.plan_stride = plan_stride;
  a.sink = sink;
  a.recent = recent;
  a.bs = block_size;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  if (cur_k != nullptr && append) {
    a.k_append = const_cast<void*>(k_base);
    a.v_append = const_cast<void*>(v_base);
  }
  a.Hk = 1;
  a.window_left = -1;
  a.scale_log2 = softmax_scale * kLog2e;
  a.out = out;
  a.union_sizes = static_cast<int32_t*>(workspace);
  a.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ml_off);
  a.part_o = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + o_off);
  a.max_rows = max_rows;
  a.res_k = res_k;
  a.res_v = res_v;
  a.res_map = res_map;
  a.res_slots = res_slots;
  a.res_map_pages = res_map_pages;
  a.res_stats = res_stats;
  a.res_win_k = res_win_k;
  a.res_win_v = res_win_v;
  a.res_win_state = res_win_state;
  a.ring_rows = ring_rows;
  a.win_rows = sink + ring_rows;
  a.meta_min = page_min;
  a.meta_max = page_max;
  a.meta_stride = page_entry_stride;
  a.meta_pages = meta_pages;
  a.page_rows = page_rows;
  a.meta_packed = packed;
  a.meta_qscale = qscale;
  a.meta_qmin = qmin;
  a.meta_qstride = quant_entry_stride;
  a.sel_bits = sel_bits;
  a.bits_stride = bits_stride;
  a.bits_w64 = (bits_pages + 63) / 64;
  a.union_rec = union_rec;
  a.mask_off = union_rec ? union_mask_offset(bits_pages) : 0;
  a.mask_w4 = union_rec ? union_mask_words(bits_pages) / 4 : 0;
  a.phase = phase;
  plan_tile_chunks(G, max_rows, &a.iters, &a.max_chunks);
  a.t_per_chunk = a.iters * kTileNW * kTileTW;
  if (lengths != nullptr) {
    a.lengths = lengths;
    a.ragged_append = append ? 1 : 0;
    a.length = 0;
    a.append_position = -1;
    // page slots are read from tile ceil(sink / 16) on (every group past its sink window)
    a.t_sink_tiles = (sink + kTileRows - 1) / kTileRows;
  } else {
    a.length = length;
    a.append_position = append ? length : -1;
    const int sink_end = sink < length ? sink : length;
    const int hist_recent = recent - 1 > 0 ? recent - 1 : 0;
    const int recent_start = length - hist_recent > sink_end ? length - hist_recent : sink_end;
    const int has_dec = (cur_k != nullptr || append) ? 1 : 0;
    const int run = (length - recent_start) + has_dec;
    a.t_sink_tiles = (sink_end + kTileRows - 1) / kTileRows;
    a.t_sink_end = sink_end;
    a.t_recent_start = recent_start;
    a.t_n_recent = length - recent_start;
    a.t_has_dec = has_dec;
    a.t_run = run;
    a.t_run_tiles = (run + kTileRows - 1) / kTileRows;
    const int64_t capacity = static_cast<int64_t>(a.max_chunks) * a.t_per_chunk;
    int64_t cap = (max_rows - sink_end - run) / kTileRows;
    const int64_t room = capacity - a.t_sink_tiles - a.t_run_tiles;
    cap = cap < room ? cap : room;
    cap = cap < plan_stride ? cap : plan_stride;
    a.t_nu_cap = static_cast<int>(cap < 0 ? 0 : cap);
  }
  a.kv_stream = tw_host::device_memory(k_base) && tw_host::device_memory(v_base);
  return dtype == TW_DTYPE_F16 ? launch_tiles<F16>(a, static_cast<hipStream_t>(stream))
                               : launch_tiles<BF16>(a, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace tw

extern "C" int tw_decode_attention_pages_resident(
    const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D, const int32_t* plan_pages,
    const uint8_t* plan_masks, const int32_t* plan_counts, int64_t plan_stride, int max_rows,
    int64_t entry_stride_rows, int sink, int recent, int block_size, const int32_t* lengths, int length, int append,
    const void* cur_k, const void* cur_v, float softmax_scale, void* res_k, void* res_v, int64_t* res_map,
    int res_slots, int res_map_pages, unsigned long long* res_stats, void* res_win_k, void* res_win_v,
    int32_t* res_win_state, int ring_rows, void* page_min, void* page_max, int64_t page_entry_stride, int meta_pages,
    void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (res_map == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, plan_pages, plan_masks, plan_counts, plan_stride,
                                max_rows, entry_stride_rows, sink, recent, block_size, lengths, length, append, cur_k,
                                cur_v, softmax_scale, res_k, res_v, res_map, res_slots, res_map_pages, res_stats,
                                page_min, page_max, page_entry_stride, meta_pages, out, workspace, workspace_bytes,
                                stream, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, 0, 3, 0, res_win_k,
                                res_win_v, res_win_state, ring_rows);
}

extern "C" int tw_decode_attention_pages_ragged(const void* q, const void* k_base, const void* v_base, int dtype,
                                                int G, int R, int D, const int32_t* plan_pages,
                                                const uint8_t* plan_masks, const int32_t* plan_counts,
                                                int64_t plan_stride, int max_rows, int64_t entry_stride_rows, int sink,
                                                int recent, int block_size, const int32_t* lengths, int append,
                                                const void* cur_k, const void* cur_v, float softmax_scale,
                                                void* page_min, void* page_max, int64_t page_entry_stride,
                                                int meta_pages, void* out, void* workspace, size_t workspace_bytes,
                                                void* stream) {
  if (lengths == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, plan_pages, plan_masks, plan_counts, plan_stride,
                                max_rows, entry_stride_rows, sink, recent, block_size, lengths, 0, append, cur_k,
                                cur_v, softmax_scale, nullptr, nullptr, nullptr, 0, 0, nullptr, page_min, page_max,
                                page_entry_stride, meta_pages, out, workspace, workspace_bytes, stream);
}

extern "C" int tw_decode_attention_page_rows(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                             int R, int D, const int32_t* plan_pages, const int32_t* plan_counts,
                                             const uint32_t* page_rows, int64_t plan_stride, int max_rows,
                                             int64_t entry_stride_rows, int sink, int recent, int block_size,
                                             const int32_t* lengths, int length, int append, const void* cur_k,
                                             const void* cur_v, float softmax_scale, void* page_min, void* page_max,
                                             int64_t page_entry_stride, int meta_pages, uint8_t* packed, void* qscale,
                                             void* qmin, int64_t quant_entry_stride, void* out, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  if (page_rows == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, plan_pages, nullptr, plan_counts, plan_stride,
                                max_rows, entry_stride_rows, sink, recent, block_size, lengths, length, append, cur_k,
                                cur_v, softmax_scale, nullptr, nullptr, nullptr, 0, 0, nullptr, page_min, page_max,
                                page_entry_stride, meta_pages, out, workspace, workspace_bytes, stream, page_rows,
                                packed, qscale, qmin, quant_entry_stride);
}

extern "C" int tw_decode_attention_pages_bits(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                              int R, int D, const uint32_t* sel_bits, int64_t bits_stride, int P,
                                              int max_rows, int64_t entry_stride_rows, int sink, int recent,
                                              int block_size, const int32_t* lengths, int length, int append,
                                              const void* cur_k, const void* cur_v, float softmax_scale,
                                              void* page_min, void* page_max, int64_t page_entry_stride,
                                              int meta_pages, void* out, void* workspace, size_t workspace_bytes,
                                              int phase, void* stream) {
  if (sel_bits == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, nullptr, nullptr, nullptr, 0, max_rows,
                                entry_stride_rows, sink, recent, block_size, lengths, length, append, cur_k, cur_v,
                                softmax_scale, nullptr, nullptr, nullptr, 0, 0, nullptr, page_min, page_max,
                                page_entry_stride, meta_pages, out, workspace, workspace_bytes, stream, nullptr,
                                nullptr, nullptr, nullptr, 0, sel_bits, bits_stride, P, phase);
}

extern "C" int tw_decode_attention_union(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                         int R, int D, const uint32_t* union_rec, int64_t rec_stride, int P,
                                         int max_rows, int64_t entry_stride_rows, int sink, int recent,
                                         int block_size, const int32_t* lengths, int length, int append,
                                         const void* cur_k, const void* cur_v, float softmax_scale, void* page_min,
                                         void* page_max, int64_t page_entry_stride, int meta_pages, uint8_t* packed,
                                         void* qscale, void* qmin, int64_t quant_entry_stride, void* out,
                                         void* workspace, size_t workspace_bytes, int phase, void* stream) {
  if (union_rec == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, nullptr, nullptr, nullptr, 0, max_rows,
                                entry_stride_rows, sink, recent, block_size, lengths, length, append, cur_k, cur_v,
                                softmax_scale, nullptr, nullptr, nullptr, 0, 0, nullptr, page_min, page_max,
                                page_entry_stride, meta_pages, out, workspace, workspace_bytes, stream, nullptr,
                                packed, qscale, qmin, quant_entry_stride, union_rec, rec_stride, P, phase, 1);
}

extern "C" int tw_decode_attention_union_resident(
    const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D, const uint32_t* union_rec,
    int64_t rec_stride, int P, int max_rows, int64_t entry_stride_rows, int sink, int recent, int block_size,
    const int32_t* lengths, int length, int append, const void* cur_k, const void* cur_v, float softmax_scale,
    void* res_k, void* res_v, int64_t* res_map, int res_slots, int res_map_pages, unsigned long long* res_stats,
    void* res_win_k, void* res_win_v, int32_t* res_win_state, int ring_rows, void* page_min, void* page_max,
    int64_t page_entry_stride, int meta_pages, uint8_t* packed, void* qscale, void* qmin,
    int64_t quant_entry_stride, void* out, void* workspace, size_t workspace_bytes, int phase, void* stream) {
  if (union_rec == nullptr || res_map == nullptr) return TW_EINVAL;
  return tw::pages_tiles_launch(q, k_base, v_base, dtype, G, R, D, nullptr, nullptr, nullptr, 0, max_rows,
                                entry_stride_rows, sink, recent, block_size, lengths, length, append, cur_k, cur_v,
                                softmax_scale, res_k, res_v, res_map, res_slots, res_map_pages, res_stats, page_min,
                                page_max, page_entry_stride, meta_pages, out, workspace, workspace_bytes, stream,
                                nullptr, packed, qscale, qmin, quant_entry_stride, union_rec, rec_stride, P, phase, 1,
                                res_win_k, res_win_v, res_win_state, ring_rows);
}
