// Quest page selection: upper-bound page score, top-k pages per query head,
// and the per-KV-group union plan consumed by the sparse decode attention.
//
// Reference: fused_quest_score / _score (twilight_fused_quest.py:12-46),
// QuestTopKOffloadedCache.prepare_layer_selection (quest_offload_cache.py:
// 299-401) and the page -> token expansion of _selected_positions (:403-511).
//
// Two kernels per layer:
//
// 1. Scores.  A block of 8 wavefronts scores a tile of 64 pages of one KV
//    group for all R query heads.  The tile is staged once in LDS with
//    16-byte loads (padded, 16-byte aligned row pitch); wavefronts w and
//    w+4 then score head w (w+4, ...) with lane = page, each summing half of
//    the 32 accumulators, so the q > 0 choice of min or max is wave-uniform.
//    Order (bit-exact with the reference for D = 128): 32 accumulators,
//    accumulator l adds the products of channels
//    l, l+32, l+64, l+96 in that order starting from +0; the 32 accumulators
//    are then summed by an adjacent-pair tree (the lane-0 result of
//    shuffle-adds at offsets 1..16).  Each product is
//    f32(q_d > 0 ? max_d : min_d) * q_d, never fused with the add.
//
// 2. Selection.  One block of 256 threads per (group, head) row finds the k
//    largest scores (order key: NaN highest, -0 == +0, ties to the lowest
//    page).  Each thread holds a contiguous run of the row's keys in
//    registers.  A pass histograms the remaining candidates into bins that
//    are monotone in the key -- 2048 bins linear in the score value over the
//    candidates' range when that range is finite, else the next 8-bit digit
//    below the candidates' common key prefix -- finds the bin holding the
//    k-th largest, takes every candidate above it and keeps the bin's keys
//    as the next candidates.  At most 256 candidates are ranked exactly by
//    (key desc, index asc); equal candidates are taken lowest index first.
//    The winners are emitted in ascending page order.  The last block of a
//    group (arrival counter, device-coherent handoff) ORs the R selections
//    into a page mask and writes the union plan: the ascending union pages
//    with the bitmask of heads that selected each, and optionally the
//    expanded row plan (sink ++ union page rows ++ recent ++ decode row).
//
// Rows longer than a block holds (P > kMaxSelPages pages, contexts past
// 131K tokens at 16-token pages) take one more launch first: a block per
// (row, segment of kMaxSelPages pages) keeps its segment's top
// min(k, segment length) pages.  The row's top k under (key desc, index
// asc) lies inside the union of its segments' top k -- a page beaten by k
// pages of its own segment is beaten by them in the whole row -- so the
// selection then runs over the compacted row (segment s's winners at
// [s*k, s*k + k_s), ascending page order within and across segments) and
// maps each compacted index back to its page.  The compaction keeps the
// index order, so ties still go to the lowest page.  The union of such rows
// goes through a page bitmap (one bit per page) instead of a byte per page.
#pragma clang fp contract(off)

#include <mutex>

#include "score_order.h"
#include "select.h"
#include "union_record.h"

namespace tw {
namespace {

using namespace sel;

constexpr int kTilePages = 64;
constexpr int kScoreBlock = 512;  // score kernel: 8 wavefronts, two per head
constexpr int kMaxD = 256;

// ------------------------------------------------------------------ scores
__device__ __forceinline__ float lds_load(const uint8_t* p, F16) {
  return to_f32(F16{}, *reinterpret_cast<const uint16_t*>(p));
}
__device__ __forceinline__ float lds_load(const uint8_t* p, BF16) {
  return to_f32(BF16{}, *reinterpret_cast<const uint16_t*>(p));
}
__device__ __forceinline__ float lds_load(const uint8_t* p, F32) { return *reinterpret_cast<const float*>(p); }

// Adjacent-pair tree over the 32 accumulators.
__device__ __forceinline__ float tree32(float (&acc)[32]) {
#pragma unroll
  for (int w = 1; w < 32; w <<= 1) {
#pragma unroll
    for (int l = 0; l < 32; l += 2 * w) acc[l] = acc[l] + acc[l + w];
  }
  return acc[0];
}

struct ScoreArgs {
  const float* q;          // [G][R][D]
  const void* pmin;        // group g page p at + g*group_stride + p*D
  const void* pmax;
  int64_t group_stride;    // elements
  int G, R, P, D;
  float* scores;           // [G][R][score_stride]
  int64_t score_stride;
  float* scores_out;       // nullable [G][R][P]
  // Ragged groups (nullable): group g scores ragged_pages(lengths[g]) <= P pages.
  const int32_t* lengths;
  int sink, recent, bs;
  // Per-tile key range (nullable): tile_mm[(g*R + r) * tiles + tile] =
  // (max, min) of score_key over the tile's scored pages, for the top-k.
  uint2* tile_mm;
  // Union records to clear (nullable): group g's at rec + g * rec_stride;
  // the block of a tile zeroes the tile's bitmap word and row-mask words.
  uint32_t* rec;
  int64_t rec_stride;
  // Arrival counters the launch after this one uses (nullable): block 0
  // zeroes n_counters of them.
  unsigned int* zero_counters;
  int n_counters;
};


// Stage a tile of pages (min then max) into LDS with a padded pitch, and the
// group's queries to q_lds.  On the vector path every global load of the
// tile is issued before the first LDS store, so a block waits for one memory
// round trip rather than one per loop trip.
template <typename DT>
__device__ __forceinline__ void stage_tile(const ScoreArgs& a, int g, int p0, int np, uint8_t* lds, int pitch,
                                           float* q_lds) {
  using S = typename DT::storage;
  const int row_bytes = a.D * static_cast<int>(sizeof(S));
  const int words = row_bytes / 4;  // D even -> row_bytes % 4 == 0
  const S* mn = static_cast<const S*>(a.pmin) + g * a.group_stride + static_cast<int64_t>(p0) * a.D;
  const S* mx = static_cast<const S*>(a.pmax) + g * a.group_stride + static_cast<int64_t>(p0) * a.D;
  const float* qg = a.q + static_cast<int64_t>(g) * a.R * a.D;
  const int nq = a.R * a.D;
  constexpr int nthreads = kScoreBlock;
  const int tid = static_cast<int>(threadIdx.x);
  const bool vec4 =
      (words % 4) == 0 && ((reinterpret_cast<uintptr_t>(mn) | reinterpret_cast<uintptr_t>(mx)) % 16) == 0;
  if (vec4) {
    constexpr int kPer = 8;  // 16-byte loads per thread: 64 pages x 2 x 256 B over 512 threads is 4
    const int quads = words / 4;
    const int total = 2 * np * quads;
    if (total <= kPer * nthreads) {
      uint4 v[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = tid + j * nthreads;
        if (i < total) {
          const int which = i / (np * quads);
          const int rem = i - which * np * quads;
          v[j] = load_stream(reinterpret_cast<const uint4*>(which ? mx : mn) + rem);
        }
      }
      for (int i = tid; i < nq; i += nthreads) q_lds[i] = qg[i];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = tid + j * nthreads;
        if (i < total) {
          const int which = i / (np * quads);
          const int rem = i - which * np * quads;
          const int page = rem / quads;
          const int qd = rem - page * quads;
          *reinterpret_cast<uint4*>(lds + (which * kTilePages + page) * pitch + qd * 16) = v[j];
        }
      }
      return;
    }
  }
  for (int i = tid; i < nq; i += nthreads) q_lds[i] = qg[i];
  if (vec4) {
    const int quads = words / 4;
    for (int i = tid; i < 2 * np * quads; i += nthreads) {
      const int which = i / (np * quads);
      const int rem = i - which * np * quads;
      const int page = rem / quads;
      const int qd = rem - page * quads;
      const uint4 v =
          load_stream(reinterpret_cast<const uint4*>(which ? mx : mn) + static_cast<int64_t>(page) * quads + qd);
      *reinterpret_cast<uint4*>(lds + (which * kTilePages + page) * pitch + qd * 16) = v;
    }
  } else {
    const int total = 2 * np * words;
    for (int i = tid; i < total; i += nthreads) {
      const int which = i / (np * words);
      const int rem = i - which * np * words;
      const int page = rem / words;
      const int w = rem - page * words;
      const uint32_t v = reinterpret_cast<const uint32_t*>(which ? mx : mn)[static_cast<int64_t>(page) * words + w];
      reinterpret_cast<uint32_t*>(lds + (which * kTilePages + page) * pitch)[w] = v;
    }
  }
}

// The (max, min) score key of one head's pages in a tile (lane = page, ok:
// the page is scored), stored for the selection's first histogram pass.
__device__ __forceinline__ void tile_key_range(const ScoreArgs& a, int64_t row, int p0, bool ok, float sc) {
  const uint32_t key = score_key(sc);
  const uint32_t kmax = wave_max_u32(ok ? key : 0u);
  const uint32_t kmin = wave_min_u32(ok ? key : 0xffffffffu);
  const int tiles = (a.P + kTilePages - 1) / kTilePages;
  if (lane_id() == 0) a.tile_mm[row * tiles + p0 / kTilePages] = make_uint2(kmax, kmin);
}

// Scores of one tile for D = DFIX and at most 4 heads, in two phases:
// channels [0, DFIX/2) of every page are stored and scored while the loads
// of channels [DFIX/2, DFIX) are still in flight.  Each accumulator takes
// its 32-channel chunks in the same order as the one-phase path (c = 0, 1
// here, then c = 2, 3), so the scores are identical.
template <typename DT, int DFIX>
__device__ void score_tile_split(const ScoreArgs& a, int g, int p0, int np_cap, int length, uint8_t* lds) {
  using S = typename DT::storage;
  constexpr int es = static_cast<int>(sizeof(S));
  constexpr int kQuads = DFIX * es / 16;  // 16-byte quads per row
  constexpr int kHq = kQuads / 2;
  constexpr int kPerHalf = (2 * kTilePages * kHq + kScoreBlock - 1) / kScoreBlock;
  constexpr int kChunks = DFIX / 32;
  constexpr int pitch = DFIX * es + 16;
  static_assert(4 * DFIX <= kScoreBlock, "one query value per thread");
  static_assert(kChunks % 2 == 0 && kHq * 16 == (DFIX / 2) * es, "channel halves are whole chunks and quads");
  const int tid = static_cast<int>(threadIdx.x);
  const S* mn = static_cast<const S*>(a.pmin) + g * a.group_stride + static_cast<int64_t>(p0) * DFIX;
  const S* mx = static_cast<const S*>(a.pmax) + g * a.group_stride + static_cast<int64_t>(p0) * DFIX;
  float* q_lds = reinterpret_cast<float*>(lds + 2 * kTilePages * pitch);
  // Loads are unconditional (indices clamped into the tile), so they issue
  // back to back and each store waits only for its own load.
  const int nq = a.R * DFIX;
  const float qv0 = a.q[static_cast<int64_t>(g) * a.R * DFIX + (tid < nq ? tid : nq - 1)];
  const int total_h = 2 * np_cap * kHq;
  uint4 va[kPerHalf], vb[kPerHalf];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int j = 0; j < kPerHalf; ++j) {
      int i = tid + j * kScoreBlock;
      i = i < total_h ? i : total_h - 1;
      const bool which = i >= np_cap * kHq;
      const int rem = i - (which ? np_cap * kHq : 0);
      const int page = rem / kHq;
      const int qd = rem % kHq + h * kHq;
      const uint4 v = load_stream(reinterpret_cast<const uint4*>(which ? mx : mn) + page * kQuads + qd);
      if (h == 0) va[j] = v; else vb[j] = v;
    }
    // the first half's loads go out first (and so arrive first)
    __builtin_amdgcn_sched_barrier(0);
  }
  auto store_half = [&](int h, const uint4 (&v)[kPerHalf]) {
#pragma unroll
    for (int j = 0; j < kPerHalf; ++j) {
      // clamped like the loads: a thread past the tile stores the last
      // quad's value to the last quad's place again
      int i = tid + j * kScoreBlock;
      i = i < total_h ? i : total_h - 1;
      const bool which = i >= np_cap * kHq;
      const int rem = i - (which ? np_cap * kHq : 0);
      const int page = rem / kHq;
      const int qd = rem % kHq + h * kHq;
      *reinterpret_cast<uint4*>(lds + ((which ? kTilePages : 0) + page) * pitch + qd * 16) = v[j];
    }
  };
  // (unconditional, so the query load is not sunk behind the tile loads;
  // threads past R*D repeat the last value)
  q_lds[tid < nq ? tid : nq - 1] = qv0;
  store_half(0, va);
  const int P = a.lengths != nullptr ? ragged_pages(length, a.sink, a.recent, a.bs, a.P) : a.P;
  if (p0 >= P) return;  // block-uniform
  const int np = (P - p0) < kTilePages ? (P - p0) : kTilePages;
  __syncthreads();
  const int wave = wave_uniform(tid / kWave);
  const int lane = lane_id();
  const int half = wave / 4;
  const int r = wave % 4;
  const bool active = r < a.R;
  const float* qh = q_lds + r * DFIX;
  const uint8_t* min_row = lds + lane * pitch;
  const uint8_t* max_row = lds + (kTilePages + lane) * pitch;
  float acc[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
  auto chunks = [&](int c_begin, int c_end) {
#pragma unroll
    for (int c = c_begin; c < c_end; ++c) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int d0 = 32 * c + 16 * half + 8 * e;
        float qv[8], x[8];
        *reinterpret_cast<float4*>(qv) = *reinterpret_cast<const float4*>(qh + d0);
        *reinterpret_cast<float4*>(qv + 4) = *reinterpret_cast<const float4*>(qh + d0 + 4);
        select8(min_row + d0 * es, max_row + d0 * es, qv, x, DT{});
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[8 * e + i] = acc[8 * e + i] + x[i] * qv[i];
      }
    }
  };
  if (active) chunks(0, kChunks / 2);
  store_half(1, vb);
  __syncthreads();
  if (active) chunks(kChunks / 2, kChunks);
#pragma unroll
  for (int w = 1; w < 16; w <<= 1) {
#pragma unroll
    for (int l = 0; l < 16; l += 2 * w) acc[l] = acc[l] + acc[l + w];
  }
  __shared__ float s_half[4][kWave];
  if (half == 1) s_half[r][lane] = acc[0];
  __syncthreads();
  if (half == 0 && active) {
    const float sc = acc[0] + s_half[r][lane];
    const int64_t row = static_cast<int64_t>(g) * a.R + r;
    if (lane < np) {
      a.scores[row * a.score_stride + p0 + lane] = sc;
      if (a.scores_out != nullptr) a.scores_out[row * a.P + p0 + lane] = sc;
    }
    if (a.tile_mm != nullptr) tile_key_range(a, row, p0, lane < np, sc);
  }
}

// Scores of one tile of kTilePages pages of group g for all R heads.
template <typename DT, int DFIX>
__device__ void score_tile(const ScoreArgs& a, int g, int tile, uint8_t* lds) {
  using S = typename DT::storage;
  const int p0 = tile * kTilePages;
  if (p0 >= a.P) return;  // block-uniform
  if (a.zero_counters != nullptr && g == 0 && tile == 0) {
    for (int i = static_cast<int>(threadIdx.x); i < a.n_counters; i += kScoreBlock) a.zero_counters[i] = 0u;
  }
  if (a.rec != nullptr) {
    // every tile of the launch (a ragged group's too): words 2 tile and
    // 2 tile + 1 of the bitmap, mask words [32 tile, 32 tile + 32)
    uint32_t* rec = a.rec + g * a.rec_stride;
    const int t = static_cast<int>(threadIdx.x);
    const int mw = (p0 >> 1) + t - 2;
    if (t < 2)
      rec[2 * tile + t] = 0u;
    else if (t < 2 + kTilePages / 2 && mw < union_mask_words(a.P))
      rec[union_mask_offset(a.P) + mw] = 0u;
  }
  // A ragged group's length is read in the same round trip as the tile: the
  // tile is staged up to the buffer's P pages (in bounds), and only the
  // scores of the group's own pages are written.
  // (an unconditional load: without lengths it reads the first query word
  // and ignores it)
  const int length = *(a.lengths != nullptr ? a.lengths + g : reinterpret_cast<const int32_t*>(a.q));
  const int np_cap = (a.P - p0) < kTilePages ? (a.P - p0) : kTilePages;
  if constexpr (DFIX > 0) {
    const uintptr_t base = reinterpret_cast<uintptr_t>(static_cast<const S*>(a.pmin) + g * a.group_stride) |
                           reinterpret_cast<uintptr_t>(static_cast<const S*>(a.pmax) + g * a.group_stride);
    if (a.R <= 4 && (base % 16) == 0) {
      score_tile_split<DT, DFIX>(a, g, p0, np_cap, length, lds);
      return;
    }
  }
  const int pitch = a.D * static_cast<int>(sizeof(S)) + 16;  // 16-byte aligned rows, padded
  float* q_lds = reinterpret_cast<float*>(lds + 2 * kTilePages * pitch);
  stage_tile<DT>(a, g, p0, np_cap, lds, pitch, q_lds);
  const int P = a.lengths != nullptr ? ragged_pages(length, a.sink, a.recent, a.bs, a.P) : a.P;
  if (p0 >= P) return;  // block-uniform
  const int np = (P - p0) < kTilePages ? (P - p0) : kTilePages;
  __syncthreads();
  const int es = static_cast<int>(sizeof(S));
  const int wave = wave_uniform(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int D = DFIX > 0 ? DFIX : a.D;
  // Two wavefronts per head: half h sums accumulators 16h .. 16h+15 (channels
  // d with d mod 32 in that range); the adjacent-pair tree over the 32
  // accumulators is the sum of the two halves' 16-accumulator trees.
  const int half = wave / 4;
  const int hw = wave % 4;
  __shared__ float s_half[4][kWave];
  for (int r0 = 0; r0 < a.R; r0 += 4) {
    const int r = r0 + hw;
    float part = 0.0f;
    if (r < a.R) {
      const float* qh = q_lds + r * D;
      float acc[16];
#pragma unroll
      for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
      const uint8_t* min_row = lds + lane * pitch;
      const uint8_t* max_row = lds + (kTilePages + lane) * pitch;
      if constexpr (DFIX > 0) {
        // 8 channels per step: 16-byte reads of both rows, then the q > 0
        // choice on the data.
#pragma unroll
        for (int c = 0; c < DFIX / 32; ++c) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int d0 = 32 * c + 16 * half + 8 * e;
            float qv[8], x[8];
            *reinterpret_cast<float4*>(qv) = *reinterpret_cast<const float4*>(qh + d0);
            *reinterpret_cast<float4*>(qv + 4) = *reinterpret_cast<const float4*>(qh + d0 + 4);
            select8(min_row + d0 * es, max_row + d0 * es, qv, x, DT{});
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[8 * e + i] = acc[8 * e + i] + x[i] * qv[i];
          }
        }
      } else {
        for (int c = 0; c * 32 < D; ++c) {
#pragma unroll
          for (int l = 0; l < 16; ++l) {
            const int d = c * 32 + 16 * half + l;
            if (d < D) {
              const float qd = qh[d];
              const uint8_t* src = (qd > 0.0f) ? max_row : min_row;
              const float x = lds_load(src + d * es, DT{});
              acc[l] = acc[l] + x * qd;
            }
          }
        }
      }
#pragma unroll
      for (int w = 1; w < 16; w <<= 1) {
#pragma unroll
        for (int l = 0; l < 16; l += 2 * w) acc[l] = acc[l] + acc[l + w];
      }
      part = acc[0];
    }
    if (half == 1) s_half[hw][lane] = part;
    __syncthreads();
    if (half == 0 && r < a.R) {
      const float sc = part + s_half[hw][lane];
      const int64_t row = static_cast<int64_t>(g) * a.R + r;
      if (lane < np) {
        a.scores[row * a.score_stride + p0 + lane] = sc;
        if (a.scores_out != nullptr) a.scores_out[row * a.P + p0 + lane] = sc;
      }
      if (a.tile_mm != nullptr) tile_key_range(a, row, p0, lane < np, sc);
    }
    __syncthreads();
  }
}

template <typename DT, int DFIX>
__global__ __launch_bounds__(kScoreBlock) void quest_score_kernel(ScoreArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  // group-minor: workgroups go to the XCDs round-robin, so with G a multiple
  // of 8 group g's blocks of every launch of the layer share XCD g % 8 (and
  // its L2)
  score_tile<DT, DFIX>(a, static_cast<int>(blockIdx.x) % a.G, static_cast<int>(blockIdx.x) / a.G, lds);
}

// --------------------------------------------------------------- selection
struct SelectArgs {
  const float* scores;     // row (g, r) at + (g*R + r)*score_stride
  int64_t score_stride;
  int vec_last4;           // vector loads: last readable float4 start of a row
  int G, R, P, k;
  int32_t* sel_ws;         // [G][R][k] (published; read by the union)
  int32_t* sel_out;        // nullable [G][R][k]
  int64_t* sel_out64;      // nullable [G][R][k]
  bool want_union;
  int32_t* plan_pages;     // nullable [G][plan_stride]
  uint8_t* plan_masks;     // nullable
  int32_t* plan_counts;    // nullable [G]
  int64_t plan_stride;
  int32_t* rows;           // nullable [G][rows_stride]
  uint8_t* row_masks;      // nullable
  int32_t* row_counts;     // nullable [G]
  int64_t rows_stride;
  int sink, recent, bs, length, append_position;
  unsigned int* counters;  // [G]
  // Ragged groups (nullable): group g selects min(k, its candidate pages)
  // among ragged_pages(lengths[g]) <= P; selection slots beyond that get -1.
  const int32_t* lengths;
  // Compacted long rows (nullable): scores holds each row's segment winners,
  // map[row * score_stride + i] the page of compacted key i and widths[row]
  // the row's key count.  keys_max bounds the keys of any row.
  const int32_t* map;
  const int32_t* widths;
  int keys_max;
  // Selection bitmaps (nullable): bit p of row (g, r) at bits + (g*R + r) *
  // bits_stride (32-bit words) is set when head r of group g selected page
  // p; bits_words words per row are written (2 * ceil(P / 64)).
  uint32_t* bits;
  int64_t bits_stride;
  int bits_words;
  // Per-tile key ranges from the score kernel (nullable; rows of
  // ceil(P / 64) tiles): the top-k takes its one-pass fast path.
  const uint2* tile_mm;
};

template <int NT, typename M>
__device__ void emit_union_plan(const SelectArgs& s, int g, int nu, const int32_t* upage, const M* umask);

// Union plan of group g: page_mask (LDS, byte per page, zero padded to a
// multiple of 8) -> ascending union pages and their head masks, then the
// optional row plan.  Thread t owns pages [8t, 8t + 8) of each 8 NT-page
// stretch.
template <int NT>
__device__ void write_union_plan(const SelectArgs& s, int g, int P, const uint8_t* page_mask, int32_t* upage,
                                 uint8_t* umask, int* scan) {
  const int tid = threadIdx.x;
  // Without a row plan (rows, row counts) the union goes straight to the
  // page plan in global memory; the row plan reads it back from LDS.
  const bool direct = s.rows == nullptr && s.row_counts == nullptr;
  int32_t* pp = s.plan_pages != nullptr ? s.plan_pages + static_cast<int64_t>(g) * s.plan_stride : nullptr;
  uint8_t* pm = s.plan_masks != nullptr ? s.plan_masks + static_cast<int64_t>(g) * s.plan_stride : nullptr;
  int nu = 0;
  for (int base = 0; base < P; base += NT * 8) {
    const int p0 = base + 8 * tid;
    uint2 w = make_uint2(0u, 0u);
    if (p0 < P) w = reinterpret_cast<const uint2*>(page_mask)[p0 >> 3];
    int cnt = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) cnt += (((w.x >> (8 * b)) & 255u) != 0u) + (((w.y >> (8 * b)) & 255u) != 0u);
    int total;
    int slot = nu + block_excl_scan<NT>(cnt, scan, &total);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t m = ((b < 4 ? w.x : w.y) >> (8 * (b & 3))) & 255u;
      if (m != 0u) {
        if (direct) {
          if (pp != nullptr) pp[slot] = p0 + b;
          if (pm != nullptr) pm[slot] = static_cast<uint8_t>(m);
        } else {
          upage[slot] = p0 + b;
          umask[slot] = static_cast<uint8_t>(m);
        }
        ++slot;
      }
    }
    nu += total;
  }
  if (direct) {
    if (tid == 0 && s.plan_counts != nullptr) s.plan_counts[g] = nu;
    return;
  }
  __syncthreads();
  emit_union_plan<NT>(s, g, nu, upage, umask);
}

// The union plan of group g from its nu union pages in LDS (ascending pages
// upage[u], head masks umask[u]): the page plan and the optional row plan.
template <int NT, typename M>
__device__ void emit_union_plan(const SelectArgs& s, int g, int nu, const int32_t* upage, const M* umask) {
  const int tid = threadIdx.x;
  const uint8_t all = static_cast<uint8_t>((1u << s.R) - 1u);
  int32_t* pp = s.plan_pages != nullptr ? s.plan_pages + static_cast<int64_t>(g) * s.plan_stride : nullptr;
  uint8_t* pm = s.plan_masks != nullptr ? s.plan_masks + static_cast<int64_t>(g) * s.plan_stride : nullptr;
  if (tid == 0 && s.plan_counts != nullptr) s.plan_counts[g] = nu;
  if (pp != nullptr) {
    for (int i = tid; i < nu; i += NT) {
      pp[i] = upage[i];
      if (pm != nullptr) pm[i] = static_cast<uint8_t>(umask[i]);
    }
  }
  const int length = s.length;
  const int bs = s.bs;
  const int sink_end = s.sink < length ? s.sink : length;
  const int hist_recent = s.recent - 1 > 0 ? s.recent - 1 : 0;
  const int recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
  const int page_end = sink_end + nu * bs;
  const int recent_end = page_end + (length - recent_start);
  const int count = recent_end + (s.append_position >= 0 ? 1 : 0);
  if (s.rows != nullptr) {
    const bool pow2 = (bs & (bs - 1)) == 0;
    const int sh = pow2 ? __ffs(bs) - 1 : 0;
    int32_t* rows = s.rows + static_cast<int64_t>(g) * s.rows_stride;
    uint8_t* masks = s.row_masks != nullptr ? s.row_masks + static_cast<int64_t>(g) * s.rows_stride : nullptr;
    for (int i = tid; i < count; i += NT) {
      int pos;
      uint8_t m = all;
      if (i < sink_end) {
        pos = i;
      } else if (i < page_end) {
        const int j = i - sink_end;
        const int u = pow2 ? (j >> sh) : j / bs;
        pos = s.sink + upage[u] * bs + (j - u * bs);
        m = static_cast<uint8_t>(umask[u]);
      } else if (i < recent_end) {
        pos = recent_start + (i - page_end);
      } else {
        pos = s.append_position;
      }
      rows[i] = pos;
      if (masks != nullptr) masks[i] = m;
    }
  }
  if (tid == 0 && s.row_counts != nullptr) s.row_counts[g] = count;
}

__device__ __forceinline__ int32_t fetch_i32(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_i32(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------- long rows
// Key count of a row of P pages after the segment pass.
__host__ __device__ __forceinline__ int long_row_width(int P, int k) {
  const int full = P / kMaxSelPages;
  const int rem = P - full * kMaxSelPages;
  return full * k + (k < rem ? k : rem);
}

struct SegArgs {
  const float* scores;     // row r at + r * score_stride
  int64_t score_stride;
  int vec_last4;           // vector loads: last readable float4 start of a row
  int P, k, nseg, R;
  float* cscore;           // [rows][kMaxSelPages] segment winners' scores
  int32_t* cidx;           // [rows][kMaxSelPages] their pages
  int32_t* cwidth;         // [rows]
  const int32_t* lengths;  // nullable: ragged groups (group = row / R)
  int sink, recent, bs;
};

// Block = (row, segment): the segment's top min(k, its pages), in ascending
// page order, at [segment * k, ...) of the compacted row.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void segment_topk_kernel(SegArgs a) {
  __shared__ __align__(16) SelShared sh;
  constexpr int KPT = kMaxSelPages / kBlock;
  const int row = blockIdx.x / a.nseg;
  const int sg = blockIdx.x - row * a.nseg;
  const int length = fetch_i32(a.lengths != nullptr ? a.lengths + row / a.R : reinterpret_cast<const int32_t*>(a.scores));
  const float* vals = a.scores + static_cast<int64_t>(row) * a.score_stride;
  const int lo = sg * kMaxSelPages;
  const int i0 = KPT * static_cast<int>(threadIdx.x);
  uint32_t key[KPT];
  if (VEC) {
#pragma unroll
    for (int q4 = 0; q4 < KPT / 4; ++q4) {
      int at = lo + i0 + 4 * q4;
      at = at < a.vec_last4 ? at : a.vec_last4;
      const float4 v = *reinterpret_cast<const float4*>(vals + at);
      key[4 * q4] = score_key(v.x);
      key[4 * q4 + 1] = score_key(v.y);
      key[4 * q4 + 2] = score_key(v.z);
      key[4 * q4 + 3] = score_key(v.w);
    }
  } else {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int i = lo + i0 + j;
      key[j] = score_key(vals[i < a.P ? i : a.P - 1]);
    }
  }
  const int P = a.lengths != nullptr ? ragged_pages(length, a.sink, a.recent, a.bs, a.P) : a.P;
  int n = P - lo;
  n = n < 0 ? 0 : (n > kMaxSelPages ? kMaxSelPages : n);
  const int ks = a.k < n ? a.k : n;
  if (sg == 0 && threadIdx.x == 0) a.cwidth[row] = long_row_width(P, a.k);
  if (ks == 0) return;  // block-uniform
  uint32_t take;
  int slot;
  block_topk<KPT>(key, n, ks, sh, &take, &slot);
  float* cs = a.cscore + static_cast<int64_t>(row) * kMaxSelPages + static_cast<int64_t>(sg) * a.k;
  int32_t* ci = a.cidx + static_cast<int64_t>(row) * kMaxSelPages + static_cast<int64_t>(sg) * a.k;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    if ((take >> j) & 1u) {
      cs[slot] = key_value(key[j]);
      ci[slot] = lo + i0 + j;
      ++slot;
    }
  }
}

// LDS of the bitmap union: page bits and word prefixes (P / 32 words each),
// then at most min(P, R * k) union pages and 32-bit head masks.
__host__ __device__ __forceinline__ size_t bitmap_union_lds_bytes(int P, int R, int k) {
  const int64_t nw = (static_cast<int64_t>(P) + 31) / 32;
  const int64_t rk = static_cast<int64_t>(R) * k;
  const int64_t u_cap = rk < P ? rk : P;
  return static_cast<size_t>(8 * nw + 8 * u_cap + 16);
}

// Union plan of group g over pages [0, P) through a page bitmap: selected
// pages set their bits, a block scan of the words' popcounts ranks the union
// pages (union page u = rank of its page), and every selection ORs its
// head's bit into the mask of its union page.  k: pages per head.
template <int NT>
__device__ void union_plan_bitmap(const SelectArgs& s, int g, int P, int k, uint8_t* dyn, int* scan) {
  const int tid = threadIdx.x;
  const int nw = (P + 31) / 32;
  const int n_sel = s.R * k;
  const int u_cap = n_sel < P ? n_sel : P;
  uint32_t* bits = reinterpret_cast<uint32_t*>(dyn);
  int* pfx = reinterpret_cast<int*>(bits + nw);
  int32_t* upage = pfx + nw;
  uint32_t* umask = reinterpret_cast<uint32_t*>(upage + u_cap);
  const int32_t* sel_g = s.sel_ws + static_cast<int64_t>(g) * s.R * s.k;
  for (int w = tid; w < nw; w += NT) bits[w] = 0u;
  for (int u = tid; u < u_cap; u += NT) umask[u] = 0u;
  __syncthreads();
  for (int i = tid; i < n_sel; i += NT) {
    const int hr = i / k;
    const int p = fetch_i32(sel_g + hr * s.k + (i - hr * k));
    atomicOr(&bits[p >> 5], 1u << (p & 31));
  }
  __syncthreads();
  constexpr int kWpt = 8;
  int U = 0;
  for (int base = 0; base < nw; base += NT * kWpt) {
    const int w0 = base + kWpt * tid;
    int c[kWpt], sum = 0;
#pragma unroll
    for (int j = 0; j < kWpt; ++j) {
      c[j] = w0 + j < nw ? __popc(bits[w0 + j]) : 0;
      sum += c[j];
    }
    int tot;
    int acc = U + block_excl_scan<NT>(sum, scan, &tot);
#pragma unroll
    for (int j = 0; j < kWpt; ++j) {
      if (w0 + j < nw) pfx[w0 + j] = acc;
      acc += c[j];
    }
    U += tot;
  }
  __syncthreads();
  for (int i = tid; i < n_sel; i += NT) {
    const int hr = i / k;
    const int p = fetch_i32(sel_g + hr * s.k + (i - hr * k));
    const int u = pfx[p >> 5] + __popc(bits[p >> 5] & ((1u << (p & 31)) - 1u));
    atomicOr(&umask[u], 1u << hr);
    upage[u] = p;
  }
  __syncthreads();
  emit_union_plan<NT>(s, g, U, upage, umask);
}

template <int KPT, bool VEC, int NT>
__global__ __launch_bounds__(NT) void quest_select_kernel(SelectArgs s) {
  __shared__ __align__(16) SelSharedT<NT> sh;
  extern __shared__ __align__(16) uint8_t dyn[];  // union scratch
  const int g = static_cast<int>(blockIdx.x) % s.G;  // group-minor (XCD g % 8)
  const int row = g * s.R + static_cast<int>(blockIdx.x) / s.G;
  // the fast top-k's histogram is cleared before the first load goes out, so
  // its barrier does not wait for the loads
  const bool fast = s.tile_mm != nullptr && s.map == nullptr;
  if (fast) {
    topk_fast_clear(sh);
    __syncthreads();
  }
  // unconditional length load (the first score word when not ragged; relaxed
  // atomic so that it is not sunk into a branch), overlapping the key loads
  const int length = fetch_i32(s.lengths != nullptr ? s.lengths + g : reinterpret_cast<const int32_t*>(s.scores));
  const float* vals = s.scores + static_cast<int64_t>(row) * s.score_stride;
  // ---- keys: one batched round trip ----
  uint32_t key[KPT];
  {
    const int i0 = KPT * static_cast<int>(threadIdx.x);
    if (VEC) {
      // Rows are 16-byte aligned and readable up to vec_last4 + 3: a float4
      // start clamped to vec_last4 (a float2 start to vec_last4 + 2, a float
      // to vec_last4 + 3) stays inside the row and below P covers the
      // thread's own keys.
      const int last4 = s.vec_last4;
      if constexpr (KPT >= 4) {
#pragma unroll
        for (int q4 = 0; q4 < KPT / 4; ++q4) {
          int at = i0 + 4 * q4;
          at = at < last4 ? at : last4;
          const float4 v = *reinterpret_cast<const float4*>(vals + at);
          key[4 * q4] = score_key(v.x);
          key[4 * q4 + 1] = score_key(v.y);
          key[4 * q4 + 2] = score_key(v.z);
          key[4 * q4 + 3] = score_key(v.w);
        }
      } else if constexpr (KPT == 2) {
        const int at = i0 < last4 + 2 ? i0 : last4 + 2;
        const float2 v = *reinterpret_cast<const float2*>(vals + at);
        key[0] = score_key(v.x);
        key[1] = score_key(v.y);
      } else {
        key[0] = score_key(vals[i0 < last4 + 3 ? i0 : last4 + 3]);
      }
    } else {
      // (clamped to the buffer's P: keys past a ragged row's end are never
      // candidates)
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int i = i0 + j;
        key[j] = score_key(vals[i < s.P ? i : s.P - 1]);
      }
    }
  }
  // the row's per-tile key ranges ride in the same round trip (two tiles a
  // lane: rows of at most 128 tiles)
  uint2 tr0 = make_uint2(0u, 0u), tr1 = make_uint2(0u, 0u);
  const int tiles = (s.P + 63) / 64;
  if (fast) {
    const uint2* tm = s.tile_mm + static_cast<int64_t>(row) * tiles;
    const int l = lane_id();
    tr0 = tm[l < tiles ? l : tiles - 1];
    tr1 = tm[l + kWave < tiles ? l + kWave : tiles - 1];
  }
  const int P = s.lengths != nullptr ? ragged_pages(length, s.sink, s.recent, s.bs, s.P) : s.P;
  const int n_keys = s.widths != nullptr ? fetch_i32(s.widths + row) : P;  // compacted long rows
  const int k = s.k < n_keys ? s.k : n_keys;
  const int32_t* map_row = s.map != nullptr ? s.map + static_cast<int64_t>(row) * s.score_stride : nullptr;
  int32_t* ws_row = s.sel_ws != nullptr ? s.sel_ws + static_cast<int64_t>(row) * s.k : nullptr;
  int32_t* out32 = s.sel_out != nullptr ? s.sel_out + static_cast<int64_t>(row) * s.k : nullptr;
  int64_t* out64 = s.sel_out64 != nullptr ? s.sel_out64 + static_cast<int64_t>(row) * s.k : nullptr;
  uint32_t take = 0u;
  const bool want_list = ws_row != nullptr || out32 != nullptr || out64 != nullptr;
  if (k > 0) {
    int slot = 0;
    bool done = false;
    if (fast) {
      // key range of the row's scored tiles
      const int tg = (n_keys + 63) / 64;
      const int l = lane_id();
      const uint32_t kmax = wave_max_u32(max(l < tg ? tr0.x : 0u, l + kWave < tg ? tr1.x : 0u));
      const uint32_t kmin = wave_min_u32(min(l < tg ? tr0.y : 0xffffffffu, l + kWave < tg ? tr1.y : 0xffffffffu));
      done = block_topk_fast<KPT>(key, n_keys, k, kmin, kmax, sh, &take);
      if (done && want_list) {
        int total;
        slot = block_excl_scan<NT>(__popc(take), sh.scan, &total);
      }
    }
    if (!done) block_topk<KPT>(key, n_keys, k, sh, &take, &slot);
    const int i0 = KPT * static_cast<int>(threadIdx.x);
    constexpr int kStage = kLinBins + 64;
    if (!want_list) {
      // bitmaps only
    } else if (k <= kStage) {
      // the selection goes through LDS (the histogram is free now) and out
      // with coalesced stores
      int32_t* st = reinterpret_cast<int32_t*>(sh.hist);
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((take >> j) & 1u) st[slot++] = i0 + j;
      }
      __syncthreads();
      for (int i = threadIdx.x; i < k; i += NT) {
        const int idx = map_row != nullptr ? map_row[st[i]] : st[i];
        if (ws_row != nullptr) publish_i32(ws_row + i, idx);
        if (out32 != nullptr) out32[i] = idx;
        if (out64 != nullptr) out64[i] = idx;
      }
    } else {
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((take >> j) & 1u) {
          const int idx = map_row != nullptr ? map_row[i0 + j] : i0 + j;
          if (ws_row != nullptr) publish_i32(ws_row + slot, idx);
          if (out32 != nullptr) out32[slot] = idx;
          if (out64 != nullptr) out64[slot] = idx;
          ++slot;
        }
      }
    }
  }
  for (int slot = k + static_cast<int>(threadIdx.x); slot < s.k; slot += NT) {
    if (out32 != nullptr) out32[slot] = -1;
    if (out64 != nullptr) out64[slot] = -1;
  }
  if (s.bits != nullptr) {
    // Thread t's KPT keys are pages KPT*t .. KPT*t + KPT - 1, so its take
    // bits are one aligned run of a 32-bit word: the 32 / KPT threads of a
    // word OR their shifted runs together and the first of them stores it.
    static_assert(KPT <= 32 && (32 % KPT) == 0, "a thread's run lies in one word");
    constexpr int kTpw = 32 / KPT;
    const int t = static_cast<int>(threadIdx.x);
    uint32_t w = take << ((KPT * t) & 31);
#pragma unroll
    for (int o = 1; o < kTpw; o <<= 1) w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), o));
    const int wi = (KPT * t) >> 5;
    if ((t % kTpw) == 0 && wi < s.bits_words) s.bits[static_cast<int64_t>(row) * s.bits_stride + wi] = w;
  }
  if (!s.want_union) return;
  if (!arrive_last(s.counters + g, static_cast<unsigned int>(s.R), &sh.flag)) return;

  // ---- last block of group g: union of the R selections ----
  if (s.map != nullptr) {
    union_plan_bitmap<NT>(s, g, P, k, dyn, sh.scan);
    return;
  }
  const int mask_bytes = ((P + 7) / 8) * 8;
  uint8_t* page_mask = dyn;
  int32_t* upage = reinterpret_cast<int32_t*>(dyn + mask_bytes);
  uint8_t* umask = reinterpret_cast<uint8_t*>(upage + P);
  const int32_t* sel_g = s.sel_ws + static_cast<int64_t>(g) * s.R * s.k;
  const int n_sel = s.R * k;
  // the first kPre selections per thread are fetched before the mask is
  // cleared (one round trip, overlapping the clear and its barrier)
  constexpr int kPre = 4;
  int pre[kPre];
  if (n_sel > 0) {
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      int i = static_cast<int>(threadIdx.x) + u * NT;
      i = i < n_sel ? i : n_sel - 1;
      const int hr = i / k;
      pre[u] = fetch_i32(sel_g + hr * s.k + (i - hr * k));
    }
  }
  for (int i = threadIdx.x; i < mask_bytes / 4; i += NT) reinterpret_cast<uint32_t*>(page_mask)[i] = 0u;
  __syncthreads();
  if (n_sel > 0) {
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int i = static_cast<int>(threadIdx.x) + u * NT;
      if (i < n_sel) {
        const int hr = i / k;
        atomicOr(reinterpret_cast<uint32_t*>(page_mask) + (pre[u] >> 2), (1u << hr) << (8 * (pre[u] & 3)));
      }
    }
  }
  for (int i = static_cast<int>(threadIdx.x) + kPre * NT; i < n_sel; i += NT) {
    const int hr = i / k;
    const int id = fetch_i32(sel_g + hr * s.k + (i - hr * k));
    atomicOr(reinterpret_cast<uint32_t*>(page_mask) + (id >> 2), (1u << hr) << (8 * (id & 3)));
  }
  __syncthreads();
  write_union_plan<NT>(s, g, P, page_mask, upage, umask, sh.scan);
}

size_t union_lds_bytes(int P) { return static_cast<size_t>((P + 7) / 8) * 8 + static_cast<size_t>(P) * 5 + 16; }

constexpr size_t kMaxLds = 160 * 1024;  // gfx950: LDS per CU

size_t select_lds_bytes(const SelectArgs& s) {
  if (!s.want_union) return 0;
  return s.map != nullptr ? bitmap_union_lds_bytes(s.P, s.R, s.k) : union_lds_bytes(s.P);
}

// Threads of a selection block (one row per block).  512 measured best at
// 2028 pages: 1024 threads paid more in 16-wave barriers than they saved.
#ifndef TW_SELECT_THREADS
#define TW_SELECT_THREADS 512
#endif
constexpr int kSelectThreads = TW_SELECT_THREADS;

template <int KPT>
int launch_select_kpt(const SelectArgs& s, int n_rows, bool vec, hipStream_t stream) {
  constexpr int NT = kSelectThreads;
  const size_t lds = select_lds_bytes(s);
  if (lds > kMaxLds) return TW_EUNSUPPORTED;
  auto kern = vec ? quest_select_kernel<KPT, true, NT> : quest_select_kernel<KPT, false, NT>;
  if (lds + sizeof(SelSharedT<NT>) > 64 * 1024)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  hipLaunchKernelGGL(kern, dim3(n_rows), dim3(NT), lds, stream, s);
  return tw_host::check_launch();
}

int launch_select(const SelectArgs& s, int n_rows, bool vec, hipStream_t stream) {
  constexpr int NT = kSelectThreads;
  const int keys = s.keys_max > 0 ? s.keys_max : s.P;
  if constexpr (NT >= 1024) {
    if (keys <= NT) return launch_select_kpt<1>(s, n_rows, vec, stream);
  }
  if constexpr (NT >= 512) {
    if (keys <= 2 * NT) return launch_select_kpt<2>(s, n_rows, vec, stream);
  }
  if (keys <= 4 * NT) return launch_select_kpt<4>(s, n_rows, vec, stream);
  if constexpr (8 * NT >= kMaxSelPages) {
    return launch_select_kpt<8>(s, n_rows, vec, stream);
  } else if constexpr (16 * NT >= kMaxSelPages) {
    if (keys <= 8 * NT) return launch_select_kpt<8>(s, n_rows, vec, stream);
    return launch_select_kpt<16>(s, n_rows, vec, stream);
  } else {
    if (keys <= 8 * NT) return launch_select_kpt<8>(s, n_rows, vec, stream);
    if (keys <= 16 * NT) return launch_select_kpt<16>(s, n_rows, vec, stream);
    return launch_select_kpt<32>(s, n_rows, vec, stream);
  }
}

// Workspace of the segment pass: compacted scores and pages per row, then
// the row widths (256-byte aligned pieces).
size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }
size_t long_row_bytes(int64_t rows, int P) {
  if (P <= kMaxSelPages) return 0;
  return 2 * align256(static_cast<size_t>(rows) * kMaxSelPages * 4) + align256(static_cast<size_t>(rows) * 4);
}

// Validity of a long-row selection: the compacted row fits a block and the
// union's bitmap fits the LDS (want_union).
int check_long_rows(int P, int R, int k, bool want_union) {
  if (P <= kMaxSelPages) return TW_OK;
  if (long_row_width(P, k) > kMaxSelPages) return TW_EUNSUPPORTED;
  if (want_union && bitmap_union_lds_bytes(P, R, k) > kMaxLds) return TW_EUNSUPPORTED;
  return TW_OK;
}

// Runs the segment pass over s's rows (scores at s.scores / s.score_stride)
// into the long-row workspace `lw`, and points s at the compacted rows.
int prepare_long_rows(SelectArgs& s, int n_rows, bool vec, uint8_t* lw, hipStream_t stream) {
  SegArgs a{};
  a.scores = s.scores;
  a.score_stride = s.score_stride;
  a.vec_last4 = s.vec_last4;
  a.P = s.P;
  a.k = s.k;
  a.nseg = (s.P + kMaxSelPages - 1) / kMaxSelPages;
  a.R = s.R;
  a.cscore = reinterpret_cast<float*>(lw);
  a.cidx = reinterpret_cast<int32_t*>(lw + align256(static_cast<size_t>(n_rows) * kMaxSelPages * 4));
  a.cwidth = reinterpret_cast<int32_t*>(lw + 2 * align256(static_cast<size_t>(n_rows) * kMaxSelPages * 4));
  a.lengths = s.lengths;
  a.sink = s.sink;
  a.recent = s.recent;
  a.bs = s.bs;
  const dim3 grid(static_cast<unsigned>(n_rows) * a.nseg);
  if (vec)
    hipLaunchKernelGGL(segment_topk_kernel<true>, grid, dim3(kBlock), 0, stream, a);
  else
    hipLaunchKernelGGL(segment_topk_kernel<false>, grid, dim3(kBlock), 0, stream, a);
  const int rc = tw_host::check_launch();
  if (rc != TW_OK) return rc;
  s.scores = a.cscore;
  s.score_stride = kMaxSelPages;
  s.vec_last4 = kMaxSelPages - 4;
  s.map = a.cidx;
  s.widths = a.cwidth;
  s.keys_max = long_row_width(s.P, s.k);
  return TW_OK;
}

template <typename DT>
int launch_score(const ScoreArgs& a, hipStream_t stream) {
  const int tiles = (a.P + kTilePages - 1) / kTilePages;
  const size_t lds = static_cast<size_t>(2 * kTilePages) *
                         (static_cast<size_t>(a.D) * sizeof(typename DT::storage) + 16) +
                     static_cast<size_t>(a.R) * a.D * sizeof(float);
  if (lds > 160 * 1024) return TW_EUNSUPPORTED;  // gfx950: 160 KB of LDS per CU
  const dim3 grid(tiles * a.G);
  auto kern = a.D == 128 ? quest_score_kernel<DT, 128> : quest_score_kernel<DT, 0>;
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  hipLaunchKernelGGL(kern, grid, dim3(kScoreBlock), lds, stream, a);
  return tw_host::check_launch();
}

int dispatch_score(int dtype, const ScoreArgs& a, hipStream_t stream) {
  switch (dtype) {
    case TW_DTYPE_F16: return launch_score<F16>(a, stream);
    case TW_DTYPE_BF16: return launch_score<BF16>(a, stream);
    case TW_DTYPE_F32: return launch_score<F32>(a, stream);
    default: return TW_EINVAL;
  }
}

bool check_score_args(const float* q, const void* pmin, const void* pmax, int G, int R, int P, int D,
                      int64_t group_stride) {
  if (q == nullptr || pmin == nullptr || pmax == nullptr) return false;
  if (G <= 0 || R <= 0 || P <= 0 || D <= 0 || D > kMaxD || (D % 2) != 0) return false;
  if (G > 1 && group_stride < static_cast<int64_t>(P) * D) return false;
  return true;
}

int64_t padded(int P) { return (static_cast<int64_t>(P) + 3) & ~static_cast<int64_t>(3); }
size_t tile_range_bytes(int G, int R, int P) {
  return align256(static_cast<size_t>(G) * R * ((P + kTilePages - 1) / kTilePages) * sizeof(uint2));
}
size_t counter_bytes(int) { return kCounterRegionBytes; }

}  // namespace
}  // namespace tw

extern "C" int tw_quest_score(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                              int R, int P, int D, int64_t page_group_stride, float* out, void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride) || out == nullptr)
    return TW_EINVAL;
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, out, P, nullptr};
  return tw::dispatch_score(dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" size_t tw_topk_sorted_workspace_size(int rows, int P) {
  if (rows <= 0 || P <= 0) return 0;
  return tw::long_row_bytes(rows, P);
}

extern "C" int tw_topk_sorted(const float* scores, int rows, int P, int64_t score_row_stride, int k,
                              int64_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (scores == nullptr || out == nullptr || rows < 0 || P <= 0 || k <= 0 || k > P) return TW_EINVAL;
  if (score_row_stride < P) return TW_EINVAL;
  {
    const int rc = tw::check_long_rows(P, 1, k, false);
    if (rc != TW_OK) return rc;
  }
  if (rows == 0) return TW_OK;
  if (P > tw::kMaxSelPages && (workspace == nullptr || workspace_bytes < tw_topk_sorted_workspace_size(rows, P)))
    return TW_ENOMEM;
  tw::SelectArgs s{};
  s.scores = scores;
  s.score_stride = score_row_stride;
  s.G = rows;
  s.R = 1;
  s.P = P;
  s.k = k;
  s.sel_out64 = out;
  s.want_union = false;
  // Vector loads only where every row is 16-byte aligned and the last float4
  // of a row ends exactly at its last score.
  const bool vec = (score_row_stride % 4) == 0 && (P % 4) == 0 && (reinterpret_cast<uintptr_t>(scores) % 16) == 0;
  s.vec_last4 = P - 4;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (P > tw::kMaxSelPages) {
    const int rc = tw::prepare_long_rows(s, rows, vec, static_cast<uint8_t*>(workspace), st);
    if (rc != TW_OK) return rc;
    return tw::launch_select(s, rows, true, st);
  }
  return tw::launch_select(s, rows, vec, st);
}

extern "C" size_t tw_quest_select_workspace_size(int G, int R, int P) {
  // arrival counters (the fixed 64 KiB region) | scores [G][R][P rounded up to 4] | selections [G][R][<= P]
  // | per-tile key ranges [G][R][ceil(P / 64)] | (P > 8192) the segment
  // pass's compacted rows
  if (G <= 0 || R <= 0 || P <= 0) return 0;
  return tw::counter_bytes(G) + tw::align256(static_cast<size_t>(G) * R * tw::padded(P) * sizeof(float)) +
         tw::align256(static_cast<size_t>(G) * R * P * sizeof(int32_t)) + tw::tile_range_bytes(G, R, P) +
         tw::long_row_bytes(static_cast<int64_t>(G) * R, P);
}

namespace tw {
namespace {
// Workspace pieces of the selection (layout of tw_quest_select_workspace_size).
struct SelectWorkspace {
  unsigned int* counters;
  float* scores;
  int32_t* sel;
  uint2* tile_mm;
  uint8_t* long_rows;
};
SelectWorkspace carve(void* workspace, int G, int R, int P) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  SelectWorkspace w{};
  w.counters = reinterpret_cast<unsigned int*>(ws);
  ws += counter_bytes(G);
  w.scores = reinterpret_cast<float*>(ws);
  ws += align256(static_cast<size_t>(G) * R * padded(P) * sizeof(float));
  w.sel = reinterpret_cast<int32_t*>(ws);
  ws += align256(static_cast<size_t>(G) * R * P * sizeof(int32_t));
  w.tile_mm = reinterpret_cast<uint2*>(ws);
  ws += tile_range_bytes(G, R, P);
  w.long_rows = ws;
  return w;
}
}  // namespace
}  // namespace tw

extern "C" int tw_quest_select(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                               int R, int P, int D, int64_t page_group_stride, int k, float* scores,
                               int32_t* sel_pages, int32_t* plan_pages, uint8_t* plan_masks, int32_t* plan_counts,
                               int64_t plan_stride, int32_t* rows, uint8_t* row_masks, int32_t* row_counts,
                               int64_t rows_stride, int sink, int recent, int block_size, int length,
                               int append_position, void* workspace, size_t workspace_bytes, void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride)) return TW_EINVAL;
  if (k <= 0 || k > P) return TW_EINVAL;
  const bool row_plan = rows != nullptr || row_counts != nullptr;
  const bool page_plan = plan_pages != nullptr || plan_counts != nullptr;
  if ((row_plan || page_plan) && R > 8) return TW_EINVAL;
  {
    const int rc = tw::check_long_rows(P, R, k, row_plan || page_plan);
    if (rc != TW_OK) return rc;
  }
  if ((plan_masks != nullptr && plan_pages == nullptr) || (row_masks != nullptr && rows == nullptr)) return TW_EINVAL;
  if (plan_pages != nullptr && plan_stride < (static_cast<int64_t>(R) * k < P ? static_cast<int64_t>(R) * k : P))
    return TW_EINVAL;
  if (row_plan) {
    if (sink < 0 || recent <= 0 || block_size <= 0 || length < 0) return TW_EINVAL;
    // Pages must lie in the eligible window (between the sink and the recent
    // window, quest_offload_cache.py:330-334) so that page rows, sink rows
    // and recent rows are disjoint.
    const int64_t sink_end = sink < length ? sink : length;
    const int64_t hist_recent = recent - 1 > 0 ? recent - 1 : 0;
    const int64_t recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
    if (static_cast<int64_t>(sink) + static_cast<int64_t>(P) * block_size > recent_start) return TW_EINVAL;
    if (rows != nullptr) {
      const int64_t union_pages = static_cast<int64_t>(R) * k < P ? static_cast<int64_t>(R) * k : P;
      const int64_t max_count = sink_end + union_pages * block_size + (length - recent_start) + 1;
      if (rows_stride < max_count) return TW_EINVAL;
    }
  }
  if (G > tw::kMaxCounterGroups) return TW_EUNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < tw_quest_select_workspace_size(G, R, P)) return TW_ENOMEM;
  const tw::SelectWorkspace w = tw::carve(workspace, G, R, P);
  unsigned int* counters = w.counters;
  float* score_ws = w.scores;
  int32_t* sel_ws = w.sel;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, score_ws, tw::padded(P), scores};
  tw::SelectArgs s{};
  s.scores = score_ws;
  s.score_stride = tw::padded(P);
  s.vec_last4 = static_cast<int>(tw::padded(P)) - 4;
  s.G = G;
  s.R = R;
  s.P = P;
  s.k = k;
  s.sel_ws = sel_ws;
  s.sel_out = sel_pages;
  s.want_union = row_plan || page_plan;
  s.plan_pages = plan_pages;
  s.plan_masks = plan_masks;
  s.plan_counts = plan_counts;
  s.plan_stride = plan_stride;
  s.rows = rows;
  s.row_masks = row_masks;
  s.row_counts = row_counts;
  s.rows_stride = rows_stride;
  s.sink = sink;
  s.recent = recent;
  s.bs = block_size;
  s.length = length;
  s.append_position = append_position;
  s.counters = counters;
  a.tile_mm = w.tile_mm;
  s.tile_mm = w.tile_mm;
  int rc = tw::dispatch_score(dtype, a, st);
  if (rc != TW_OK) return rc;
  if (P > tw::kMaxSelPages) {
    rc = tw::prepare_long_rows(s, G * R, true, w.long_rows, st);
    if (rc != TW_OK) return rc;
  }
  return tw::launch_select(s, G * R, true, st);
}

extern "C" int tw_quest_select_ragged(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                                      int R, int P_max, int D, int64_t page_group_stride, const int32_t* lengths,
                                      int k, int32_t* sel_pages, int32_t* plan_pages, uint8_t* plan_masks,
                                      int32_t* plan_counts, int64_t plan_stride, int sink, int recent,
                                      int block_size, void* workspace, size_t workspace_bytes, void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P_max, D, page_group_stride)) return TW_EINVAL;
  if (lengths == nullptr || k <= 0 || k > P_max) return TW_EINVAL;
  if (sink < 0 || recent <= 0 || block_size <= 0) return TW_EINVAL;
  const bool page_plan = plan_pages != nullptr || plan_counts != nullptr;
  if (page_plan && (R > 8 || plan_pages == nullptr || plan_counts == nullptr)) return TW_EINVAL;
  {
    const int rc = tw::check_long_rows(P_max, R, k, page_plan);
    if (rc != TW_OK) return rc;
  }
  if (plan_masks != nullptr && plan_pages == nullptr) return TW_EINVAL;
  if (plan_pages != nullptr &&
      plan_stride < (static_cast<int64_t>(R) * k < P_max ? static_cast<int64_t>(R) * k : P_max))
    return TW_EINVAL;
  if (G > tw::kMaxCounterGroups) return TW_EUNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < tw_quest_select_workspace_size(G, R, P_max)) return TW_ENOMEM;
  const tw::SelectWorkspace w = tw::carve(workspace, G, R, P_max);
  unsigned int* counters = w.counters;
  float* score_ws = w.scores;
  int32_t* sel_ws = w.sel;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P_max, D, score_ws, tw::padded(P_max), nullptr,
                  lengths, sink, recent, block_size};
  tw::SelectArgs s{};
  s.scores = score_ws;
  s.score_stride = tw::padded(P_max);
  s.vec_last4 = static_cast<int>(tw::padded(P_max)) - 4;
  s.G = G;
  s.R = R;
  s.P = P_max;
  s.k = k;
  s.sel_ws = sel_ws;
  s.sel_out = sel_pages;
  s.want_union = page_plan;
  s.plan_pages = plan_pages;
  s.plan_masks = plan_masks;
  s.plan_counts = plan_counts;
  s.plan_stride = plan_stride;
  s.sink = sink;
  s.recent = recent;
  s.bs = block_size;
  s.append_position = -1;
  s.counters = counters;
  s.lengths = lengths;
  a.tile_mm = w.tile_mm;
  s.tile_mm = w.tile_mm;
  int rc = tw::dispatch_score(dtype, a, st);
  if (rc != TW_OK) return rc;
  if (P_max > tw::kMaxSelPages) {
    rc = tw::prepare_long_rows(s, G * R, true, w.long_rows, st);
    if (rc != TW_OK) return rc;
  }
  return tw::launch_select(s, G * R, true, st);
}

extern "C" int tw_quest_select_bits(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                                    int R, int P, int D, int64_t page_group_stride, const int32_t* lengths, int k,
                                    float* scores, int32_t* sel_pages, uint32_t* sel_bits, int64_t bits_stride,
                                    int sink, int recent, int block_size, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride)) return TW_EINVAL;
  if (k <= 0 || k > P || sel_bits == nullptr) return TW_EINVAL;
  if (P > tw::kMaxSelPages) return TW_EUNSUPPORTED;  // long rows select through the segment pass and a plan
  const int words = 2 * ((P + 63) / 64);
  if (bits_stride < words || (bits_stride % 2) != 0 || (reinterpret_cast<uintptr_t>(sel_bits) % 8) != 0)
    return TW_EINVAL;
  if (lengths != nullptr && (sink < 0 || recent <= 0 || block_size <= 0)) return TW_EINVAL;
  if (workspace == nullptr || workspace_bytes < tw_quest_select_workspace_size(G, R, P)) return TW_ENOMEM;
  const tw::SelectWorkspace w = tw::carve(workspace, G, R, P);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, w.scores, tw::padded(P), scores,
                  lengths, sink, recent, block_size};
  tw::SelectArgs s{};
  s.scores = w.scores;
  s.score_stride = tw::padded(P);
  s.vec_last4 = static_cast<int>(tw::padded(P)) - 4;
  s.G = G;
  s.R = R;
  s.P = P;
  s.k = k;
  s.sel_out = sel_pages;
  s.want_union = false;
  s.sink = sink;
  s.recent = recent;
  s.bs = block_size;
  s.append_position = -1;
  s.counters = w.counters;
  s.lengths = lengths;
  s.bits = sel_bits;
  s.bits_stride = bits_stride;
  s.bits_words = words;
  a.tile_mm = w.tile_mm;
  s.tile_mm = w.tile_mm;
  const int rc = tw::dispatch_score(dtype, a, st);
  if (rc != TW_OK) return rc;
  return tw::launch_select(s, G * R, true, st);
}

namespace tw {

int fused_quest_score(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R, int P,
                      int D, int64_t page_group_stride, const int32_t* lengths, int sink, int recent, int block_size,
                      void* workspace, size_t workspace_bytes, uint32_t* rec, int64_t rec_stride,
                      unsigned int* counters, int n_counters, FusedScores* out, hipStream_t stream) {
  if (!check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride) || out == nullptr) return TW_EINVAL;
  if (P > kMaxSelPages) return TW_EUNSUPPORTED;
  if (rec != nullptr && rec_stride < union_record_words(P)) return TW_EINVAL;
  if (workspace == nullptr || workspace_bytes < tw_quest_select_workspace_size(G, R, P)) return TW_ENOMEM;
  const SelectWorkspace w = carve(workspace, G, R, P);
  ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, w.scores, padded(P), nullptr,
              lengths, sink, recent, block_size};
  a.tile_mm = w.tile_mm;
  a.rec = rec;
  a.rec_stride = rec_stride;
  a.zero_counters = counters;
  a.n_counters = counters != nullptr ? n_counters : 0;
  out->scores = w.scores;
  out->score_stride = padded(P);
  out->vec_last4 = static_cast<int>(padded(P)) - 4;
  out->tile_mm = w.tile_mm;
  return dispatch_score(dtype, a, stream);
}

}  // namespace tw

// ---------------------------------------------------------------------------
// tw_quest_select_static: tw_quest_select for callers that cannot allocate
// (code under graph capture, serving loops that forbid hipMalloc).  The
// workspace -- arrival counters, scores, selections -- lives in `scratch`, a
// file-scope device array of kStaticScratchBytes that every GPU the library
// runs on holds until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address is taken with
// hipGetSymbolAddress once per device (the first call on that device, with
// that device current) and only that address is ever passed to kernels.
// Calls on one device share the array: two calls that overlap in time on one
// GPU race.
namespace {

constexpr size_t kStaticScratchBytes = size_t{16} << 20;  // 16 MiB
constexpr int kMaxStaticDevices = 64;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxStaticDevices] = {};
size_t g_scratch_zeroed[kMaxStaticDevices] = {};  // bytes from the start known to be zero

// Zero the arrival counters at the start of the array (the only part of the
// workspace that must start at zero; the selection kernels leave them zero
// after every call).  A kernel, not a memset node, so a captured graph
// replays it correctly.
__global__ __launch_bounds__(256) void zero_scratch_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The device address of `scratch` on the current device, set up on the first
// call there, with its first `zero_bytes` (the call's arrival counters, a
// multiple of 256) known to be zero: a call that needs more of them zeroed
// than a fill outside graph capture has covered enqueues one on `stream`
// ahead of its kernels (a fill captured into a graph runs at every replay,
// so only the counters' few bytes are filled).
int static_scratch(hipStream_t stream, size_t zero_bytes, void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return tw_host::record_hip_error(err);
  if (dev < 0 || dev >= kMaxStaticDevices) return TW_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return tw_host::record_hip_error(err);
    if (p == nullptr) return TW_EHIP;
    g_scratch_ptr[dev] = p;
  }
  if (zero_bytes > g_scratch_zeroed[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &cs);
    if (err != hipSuccess) return tw_host::record_hip_error(err);
    const size_t n16 = zero_bytes / 16;
    const int blocks = static_cast<int>((n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024);
    hipLaunchKernelGGL(zero_scratch_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<uint4*>(g_scratch_ptr[dev]), n16);
    const int rc = tw_host::check_launch();
    if (rc != TW_OK) return rc;
    if (cs == hipStreamCaptureStatusNone) g_scratch_zeroed[dev] = zero_bytes;
  }
  *out = g_scratch_ptr[dev];
  return TW_OK;
}

}  // namespace

extern "C" size_t tw_quest_select_static_capacity(void) { return kStaticScratchBytes; }

extern "C" int tw_quest_select_static(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                                      int R, int P, int D, int64_t page_group_stride, int k, float* scores,
                                      int32_t* sel_pages, int32_t* plan_pages, uint8_t* plan_masks,
                                      int32_t* plan_counts, int64_t plan_stride, int32_t* rows, uint8_t* row_masks,
                                      int32_t* row_counts, int64_t rows_stride, int sink, int recent,
                                      int block_size, int length, int append_position, void* stream) {
  const size_t need = tw_quest_select_workspace_size(G, R, P);
  if (need == 0) return TW_EINVAL;
  if (need > kStaticScratchBytes) return TW_ENOMEM;  // beyond the static array: use tw_quest_select
  void* ws = nullptr;
  const int rc = static_scratch(static_cast<hipStream_t>(stream), tw::counter_bytes(G), &ws);
  if (rc != TW_OK) return rc;
  return tw_quest_select(q, page_min, page_max, dtype, G, R, P, D, page_group_stride, k, scores, sel_pages,
                         plan_pages, plan_masks, plan_counts, plan_stride, rows, row_masks, row_counts, rows_stride,
                         sink, recent, block_size, length, append_position, ws, kStaticScratchBytes, stream);
}
