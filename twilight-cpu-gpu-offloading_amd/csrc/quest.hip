// Quest page selection: upper-bound page score, top-k pages per query head,
// and the per-KV-group row plan consumed by the sparse decode attention.
//
// Reference: fused_quest_score / _score (twilight_fused_quest.py:12-46),
// QuestTopKOffloadedCache.prepare_layer_selection (quest_offload_cache.py:
// 299-401) and the page -> token expansion of _selected_positions (:403-511).
//
// Score order (bit-exact with the reference for D = 128): 32 accumulators,
// accumulator l adds the products of channels l, l+32, l+64, l+96 in that
// order starting from +0; the 32 accumulators are then summed by an
// adjacent-pair tree (the lane-0 result of shuffle-adds at offsets 1..16).
// Each product is f32(q_d > 0 ? max_d : min_d) * q_d, never fused with the add.
//
// Work split: a block of 4 wavefronts scores a tile of 64 pages of one KV
// group for all R query heads.  The tile is staged once in LDS with 16-byte
// loads (padded row pitch, conflict-free column reads); wavefront w then
// scores head w (w+4, ...) with lane = page, so the q > 0 choice of min or max
// is wave-uniform and each lane reads exactly one value per channel.
//
// Selection: the block that finishes a group last (arrival counter, no
// waiting) runs one radix select per head -- 8-bit digits, LDS histogram,
// suffix scan to find the k-th largest key -- and an ordered ballot
// compaction that emits page ids ascending with ties to the lowest index.
// It then builds the group's row plan from an LDS page-mask table.
#pragma clang fp contract(off)

#include "tw_common.h"

namespace tw {
namespace {

constexpr int kTilePages = 64;
constexpr int kBlock = 256;
constexpr int kMaxD = 256;
constexpr int kMaxPlanPages = 16384;

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
  float* scores;           // [G][R][P]
};

struct SelectArgs {
  int k;
  int32_t* sel_pages;      // nullable [G][R][k]
  int32_t* rows;           // nullable [G][rows_stride]
  uint8_t* row_masks;      // nullable
  int32_t* row_counts;     // nullable [G]
  int64_t rows_stride;
  int sink, recent, bs, length, append_position;
  unsigned int* counters;  // [G]
};

// Stage a tile of pages (min then max) into LDS with a padded pitch.
template <typename DT>
__device__ __forceinline__ void stage_tile(const ScoreArgs& a, int g, int p0, int np, uint8_t* lds, int pitch) {
  using S = typename DT::storage;
  const int row_bytes = a.D * static_cast<int>(sizeof(S));
  const int words = row_bytes / 4;  // D even -> row_bytes % 4 == 0
  const S* mn = static_cast<const S*>(a.pmin) + g * a.group_stride + static_cast<int64_t>(p0) * a.D;
  const S* mx = static_cast<const S*>(a.pmax) + g * a.group_stride + static_cast<int64_t>(p0) * a.D;
  // Source rows are contiguous; copy dword by dword (pitch is dword aligned).
  const int total = 2 * np * words;
  const bool vec4 = (words % 4) == 0 && ((reinterpret_cast<uintptr_t>(mn) | reinterpret_cast<uintptr_t>(mx)) % 16) == 0;
  if (vec4) {
    const int quads = words / 4;
    for (int i = threadIdx.x; i < 2 * np * quads; i += blockDim.x) {
      const int which = i / (np * quads);
      const int rem = i - which * np * quads;
      const int page = rem / quads;
      const int qd = rem - page * quads;
      const uint4 v = reinterpret_cast<const uint4*>(which ? mx : mn)[static_cast<int64_t>(page) * quads + qd];
      uint32_t* dst = reinterpret_cast<uint32_t*>(lds + (which * kTilePages + page) * pitch) + qd * 4;
      dst[0] = v.x;
      dst[1] = v.y;
      dst[2] = v.z;
      dst[3] = v.w;
    }
  } else {
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
      const int which = i / (np * words);
      const int rem = i - which * np * words;
      const int page = rem / words;
      const int w = rem - page * words;
      const uint32_t v = reinterpret_cast<const uint32_t*>(which ? mx : mn)[static_cast<int64_t>(page) * words + w];
      reinterpret_cast<uint32_t*>(lds + (which * kTilePages + page) * pitch)[w] = v;
    }
  }
}

template <typename DT, int DFIX>
__device__ __forceinline__ void score_tile(const ScoreArgs& a, int g, int p0, int np, const uint8_t* lds,
                                           int pitch) {
  using S = typename DT::storage;
  const int es = static_cast<int>(sizeof(S));
  const int wave = wave_uniform(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int D = DFIX > 0 ? DFIX : a.D;
  for (int r = wave; r < a.R; r += kBlock / kWave) {
    const float* qh = a.q + (static_cast<int64_t>(g) * a.R + r) * D;
    float acc[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) acc[l] = 0.0f;
    const uint8_t* min_row = lds + lane * pitch;
    const uint8_t* max_row = lds + (kTilePages + lane) * pitch;
    if (DFIX > 0) {
#pragma unroll
      for (int d = 0; d < DFIX; ++d) {
        const float qd = qh[d];
        const uint8_t* src = (qd > 0.0f) ? max_row : min_row;
        const float x = lds_load(src + d * es, DT{});
        acc[d & 31] = acc[d & 31] + x * qd;
      }
    } else {
      for (int c = 0; c * 32 < D; ++c) {
#pragma unroll
        for (int l = 0; l < 32; ++l) {
          const int d = c * 32 + l;
          if (d < D) {
            const float qd = qh[d];
            const uint8_t* src = (qd > 0.0f) ? max_row : min_row;
            const float x = lds_load(src + d * es, DT{});
            acc[l] = acc[l] + x * qd;
          }
        }
      }
    }
    const float s = tree32(acc);
    if (lane < np) a.scores[(static_cast<int64_t>(g) * a.R + r) * a.P + p0 + lane] = s;
  }
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

// Radix select of the k largest values (score_key order, ties -> lowest
// index) of vals[0..P); emit(slot, index) is called with ascending indices
// and slot = rank in ascending-index order.  hist: 256 LDS words owned by the
// calling wavefront.
template <typename Emit>
__device__ void wave_topk(const float* __restrict__ vals, int P, int k, uint32_t* hist, Emit emit) {
  const int lane = lane_id();
  uint32_t prefix = 0u, mask = 0u;
  uint32_t need = static_cast<uint32_t>(k);
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = lane; b < 256; b += kWave) hist[b] = 0u;
    wave_lds_fence();
    for (int i = lane; i < P; i += kWave) {
      const uint32_t key = score_key(vals[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    wave_lds_fence();
    const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1], c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
    const uint32_t tot = c0 + c1 + c2 + c3;
    const uint32_t incl = wave_suffix_sum_u32(tot);
    const uint32_t above = incl - tot;
    const bool has = above < need && need <= incl;
    int bin = 0;
    uint32_t new_above = above, bin_count = 0;
    if (has) {
      uint32_t acc = above;
      if (need <= acc + c3) {
        bin = 4 * lane + 3;
        bin_count = c3;
      } else if (acc += c3, need <= acc + c2) {
        bin = 4 * lane + 2;
        bin_count = c2;
      } else if (acc += c2, need <= acc + c1) {
        bin = 4 * lane + 1;
        bin_count = c1;
      } else {
        acc += c1;
        bin = 4 * lane;
        bin_count = c0;
      }
      new_above = acc;
    }
    const int src = first_lane(__ballot(has));
    bin = __shfl(bin, src);
    new_above = __shfl(new_above, src);
    bin_count = __shfl(bin_count, src);
    need -= new_above;
    prefix |= static_cast<uint32_t>(bin) << shift;
    mask |= 255u << shift;
    wave_lds_fence();
    if (bin_count == need) break;
  }
  // Ordered compaction: indices ascending; keys strictly above the prefix are
  // all taken, keys equal to it are taken lowest index first.
  uint32_t out = 0u, eq_seen = 0u;
  const uint64_t lt = lanemask_lt();
  for (int base = 0; base < P; base += kWave) {
    const int i = base + lane;
    const bool valid = i < P;
    const uint32_t mk = valid ? (score_key(vals[i]) & mask) : 0u;
    const bool gt = valid && mk > prefix;
    const bool eq = valid && mk == prefix;
    const uint64_t eqb = __ballot(eq);
    const uint32_t eq_rank = static_cast<uint32_t>(__popcll(eqb & lt));
    const bool take = gt || (eq && eq_seen + eq_rank < need);
    const uint64_t tb = __ballot(take);
    if (take) emit(static_cast<int>(out + static_cast<uint32_t>(__popcll(tb & lt))), i);
    out += static_cast<uint32_t>(__popcll(tb));
    eq_seen += static_cast<uint32_t>(__popcll(eqb));
  }
}

// Row plan of one group from the LDS page-mask table (byte per page).
__device__ void build_row_plan(const SelectArgs& s, int g, int R, int P, const uint8_t* page_mask,
                               int32_t* upage, uint8_t* umask, int* s_scan) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const uint8_t all = static_cast<uint8_t>((1u << R) - 1u);
  // Ordered compaction of the union pages.
  int total = 0;
  for (int base = 0; base < P; base += kBlock) {
    const int p = base + tid;
    const uint8_t m = p < P ? page_mask[p] : 0;
    const uint64_t b = __ballot(m != 0);
    if (lane == 0) s_scan[wave] = __popcll(b);
    __syncthreads();
    int before = total;
    for (int w = 0; w < wave; ++w) before += s_scan[w];
    int chunk_total = 0;
    for (int w = 0; w < kBlock / kWave; ++w) chunk_total += s_scan[w];
    if (m != 0) {
      const int slot = before + __popcll(b & lanemask_lt());
      upage[slot] = p;
      umask[slot] = m;
    }
    total += chunk_total;
    __syncthreads();
  }
  const int nu = total;
  const int length = s.length;
  const int sink_end = s.sink < length ? s.sink : length;
  const int hist_recent = s.recent - 1 > 0 ? s.recent - 1 : 0;
  const int recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
  const int n_page_rows = nu * s.bs;
  const int n_recent = length - recent_start;
  const int count = sink_end + n_page_rows + n_recent + (s.append_position >= 0 ? 1 : 0);
  if (s.rows != nullptr) {
    int32_t* rows = s.rows + static_cast<int64_t>(g) * s.rows_stride;
    uint8_t* masks = s.row_masks != nullptr ? s.row_masks + static_cast<int64_t>(g) * s.rows_stride : nullptr;
    for (int i = tid; i < count; i += kBlock) {
      int pos;
      uint8_t m = all;
      if (i < sink_end) {
        pos = i;
      } else if (i < sink_end + n_page_rows) {
        const int j = i - sink_end;
        const int u = j / s.bs;
        pos = s.sink + upage[u] * s.bs + (j - u * s.bs);
        m = umask[u];
      } else if (i < sink_end + n_page_rows + n_recent) {
        pos = recent_start + (i - sink_end - n_page_rows);
      } else {
        pos = s.append_position;
      }
      rows[i] = pos;
      if (masks != nullptr) masks[i] = m;
    }
  }
  if (tid == 0 && s.row_counts != nullptr) s.row_counts[g] = count;
}

template <typename DT, int DFIX, bool FUSED>
__global__ __launch_bounds__(kBlock) void quest_kernel(ScoreArgs a, SelectArgs s) {
  extern __shared__ __align__(16) uint8_t lds[];
  using S = typename DT::storage;
  const int tiles = (a.P + kTilePages - 1) / kTilePages;
  const int g = blockIdx.x / tiles;
  const int tile = blockIdx.x - g * tiles;
  const int p0 = tile * kTilePages;
  const int np = (a.P - p0) < kTilePages ? (a.P - p0) : kTilePages;
  const int pitch = a.D * static_cast<int>(sizeof(S)) + 4;
  stage_tile<DT>(a, g, p0, np, lds, pitch);
  __syncthreads();
  score_tile<DT, DFIX>(a, g, p0, np, lds, pitch);
  if (!FUSED) return;

  __shared__ int s_flag;
  if (!arrive_last(s.counters + g, static_cast<unsigned int>(tiles), &s_flag)) return;

  // ---- last block of group g: top-k per head + row plan ----
  __syncthreads();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  uint32_t* hist = reinterpret_cast<uint32_t*>(lds) + wave * 256;
  const bool plan = s.rows != nullptr || s.row_counts != nullptr;
  uint8_t* page_mask = lds + 4 * 256 * 4;  // after the 4 histograms
  const int mask_bytes = ((a.P + 3) / 4) * 4;
  if (plan) {
    for (int i = threadIdx.x; i < mask_bytes / 4; i += kBlock) reinterpret_cast<uint32_t*>(page_mask)[i] = 0u;
  }
  __syncthreads();
  for (int r = wave; r < a.R; r += kBlock / kWave) {
    const float* vals = a.scores + (static_cast<int64_t>(g) * a.R + r) * a.P;
    int32_t* out = s.sel_pages != nullptr ? s.sel_pages + (static_cast<int64_t>(g) * a.R + r) * s.k : nullptr;
    const uint32_t bit = 1u << r;
    wave_topk(vals, a.P, s.k, hist, [&](int slot, int idx) {
      if (out != nullptr) out[slot] = idx;
      if (plan) atomicOr(reinterpret_cast<uint32_t*>(page_mask) + (idx >> 2), bit << (8 * (idx & 3)));
    });
  }
  __syncthreads();
  if (!plan) return;
  __shared__ int s_scan[kBlock / kWave];
  int32_t* upage = reinterpret_cast<int32_t*>(page_mask + mask_bytes);
  uint8_t* umask = reinterpret_cast<uint8_t*>(upage + a.P);
  build_row_plan(s, g, a.R, a.P, page_mask, upage, umask, s_scan);
}

template <typename Kern>
size_t quest_lds_bytes(int P, int D, int es, bool fused) {
  (void)sizeof(Kern*);
  size_t tile = static_cast<size_t>(2 * kTilePages) * (static_cast<size_t>(D) * es + 4);
  if (!fused) return tile;
  const size_t mask_bytes = static_cast<size_t>((P + 3) / 4) * 4;
  const size_t sel = 4 * 256 * 4 + mask_bytes + static_cast<size_t>(P) * 4 + static_cast<size_t>(P);
  return tile > sel ? tile : sel;
}

template <typename DT, bool FUSED>
int launch_quest(const ScoreArgs& a, const SelectArgs& s, hipStream_t stream) {
  const int tiles = (a.P + kTilePages - 1) / kTilePages;
  const size_t lds = quest_lds_bytes<DT>(a.P, a.D, static_cast<int>(sizeof(typename DT::storage)), FUSED);
  if (lds > 160 * 1024) return TW_EUNSUPPORTED;
  dim3 grid(tiles * a.G);
  if (a.D == 128) {
    auto kern = quest_kernel<DT, 128, FUSED>;
    if (lds > 64 * 1024) (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, stream, a, s);
  } else {
    auto kern = quest_kernel<DT, 0, FUSED>;
    if (lds > 64 * 1024) (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, stream, a, s);
  }
  return tw_host::check_launch();
}

template <bool FUSED>
int dispatch_quest(int dtype, const ScoreArgs& a, const SelectArgs& s, hipStream_t stream) {
  switch (dtype) {
    case TW_DTYPE_F16: return launch_quest<F16, FUSED>(a, s, stream);
    case TW_DTYPE_BF16: return launch_quest<BF16, FUSED>(a, s, stream);
    case TW_DTYPE_F32: return launch_quest<F32, FUSED>(a, s, stream);
    default: return TW_EINVAL;
  }
}

__global__ __launch_bounds__(kBlock) void topk_rows_kernel(const float* __restrict__ scores, int rows, int P,
                                                           int64_t stride, int k, int64_t* __restrict__ out) {
  __shared__ uint32_t hist[4 * 256];
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int row = blockIdx.x * (kBlock / kWave) + wave;
  if (row >= rows) return;
  int64_t* o = out + static_cast<int64_t>(row) * k;
  wave_topk(scores + row * stride, P, k, hist + wave * 256, [&](int slot, int idx) { o[slot] = idx; });
}

bool check_score_args(const float* q, const void* pmin, const void* pmax, int G, int R, int P, int D,
                      int64_t group_stride) {
  if (q == nullptr || pmin == nullptr || pmax == nullptr) return false;
  if (G <= 0 || R <= 0 || P <= 0 || D <= 0 || D > kMaxD || (D % 2) != 0) return false;
  if (G > 1 && group_stride < static_cast<int64_t>(P) * D) return false;
  return true;
}

}  // namespace
}  // namespace tw

extern "C" int tw_quest_score(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                              int R, int P, int D, int64_t page_group_stride, float* out, void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride) || out == nullptr)
    return TW_EINVAL;
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, out};
  tw::SelectArgs s{};
  return tw::dispatch_quest<false>(dtype, a, s, static_cast<hipStream_t>(stream));
}

extern "C" int tw_topk_sorted(const float* scores, int rows, int P, int64_t score_row_stride, int k,
                              int64_t* out, void* stream) {
  if (scores == nullptr || out == nullptr || rows < 0 || P <= 0 || k <= 0 || k > P) return TW_EINVAL;
  if (score_row_stride < P) return TW_EINVAL;
  if (rows == 0) return TW_OK;
  const int blocks = (rows + 3) / 4;
  hipLaunchKernelGGL(tw::topk_rows_kernel, dim3(blocks), dim3(tw::kBlock), 0, static_cast<hipStream_t>(stream),
                     scores, rows, P, score_row_stride, k, out);
  return tw_host::check_launch();
}

extern "C" size_t tw_quest_select_workspace_size(int G, int R, int P) {
  // arrival counters (one per group, 256-byte aligned) + scores [G][R][P]
  const size_t counters = ((static_cast<size_t>(G) * 4 + 255) / 256) * 256;
  return counters + static_cast<size_t>(G) * R * P * sizeof(float);
}

extern "C" int tw_quest_select(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                               int R, int P, int D, int64_t page_group_stride, int k, float* scores,
                               int32_t* sel_pages, int32_t* rows, uint8_t* row_masks, int32_t* row_counts,
                               int64_t rows_stride, int sink, int recent, int block_size, int length,
                               int append_position, void* workspace, size_t workspace_bytes, void* stream) {
  if (!tw::check_score_args(q, page_min, page_max, G, R, P, D, page_group_stride)) return TW_EINVAL;
  if (k <= 0 || k > P) return TW_EINVAL;
  const bool plan = rows != nullptr || row_counts != nullptr;
  if (plan) {
    if (R > 8 || P > tw::kMaxPlanPages || sink < 0 || recent <= 0 || block_size <= 0 || length < 0) return TW_EINVAL;
    // Pages must lie in the eligible window (between the sink and the recent
    // window, quest_offload_cache.py:330-334) so that page rows, sink rows
    // and recent rows are disjoint.
    const int64_t sink_end = sink < length ? sink : length;
    const int64_t hist_recent = recent - 1 > 0 ? recent - 1 : 0;
    const int64_t recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
    if (static_cast<int64_t>(sink) + static_cast<int64_t>(P) * block_size > recent_start) return TW_EINVAL;
    if (row_masks != nullptr && rows == nullptr) return TW_EINVAL;
    if (rows != nullptr) {
      const int64_t union_pages = static_cast<int64_t>(R) * k < P ? static_cast<int64_t>(R) * k : P;
      const int64_t max_count = sink_end + union_pages * block_size + (length - recent_start) + 1;
      if (rows_stride < max_count) return TW_EINVAL;
    }
  }
  if (workspace == nullptr || workspace_bytes < tw_quest_select_workspace_size(G, R, P)) return TW_ENOMEM;
  const size_t counter_bytes = ((static_cast<size_t>(G) * 4 + 255) / 256) * 256;
  unsigned int* counters = static_cast<unsigned int*>(workspace);
  float* score_buf = scores != nullptr ? scores
                                       : reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + counter_bytes);
  tw::ScoreArgs a{q, page_min, page_max, page_group_stride, G, R, P, D, score_buf};
  tw::SelectArgs s{k, sel_pages, rows, row_masks, row_counts, rows_stride, sink, recent, block_size, length,
                   append_position, counters};
  return tw::dispatch_quest<true>(dtype, a, s, static_cast<hipStream_t>(stream));
}
