// Prompt metadata: per-page key min/max (Quest) fused with per-token affine
// INT4 packing (Twilight), one wavefront per page.
//
// Reference: QuestTopKOffloadedCache._build_metadata (quest_offload_cache.py:
// 276-289) and affine_int4_pack (twilight_offload_cache.py:25-37), called
// together from the Twilight override (twilight_offload_cache.py:925-936).
//
// Layout: a wavefront owns one page of bs rows (or, for rows outside complete
// pages, a chunk of 16 rows).  Lane l owns the channel pairs
// (2l + 128c, 2l + 1 + 128c), so a row of 128 16-bit keys is one coalesced
// 256-byte load and the packed INT4 row is one coalesced 64-byte store
// (lane l writes byte l, whose low nibble is channel 2l).  The row min/max
// needed by INT4 is a wave reduction; the page min/max is a per-lane running
// reduction over the page's rows, so the keys are read exactly once.
#pragma clang fp contract(off)

#include "tw_common.h"

namespace tw {
namespace {

constexpr int kMaxPairChunks = 8;  // D <= 1024

__device__ __forceinline__ void load_pair(const uint16_t* p, uint16_t& a, uint16_t& b) {
  const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
  a = static_cast<uint16_t>(w & 0xffffu);
  b = static_cast<uint16_t>(w >> 16);
}
__device__ __forceinline__ void load_pair(const float* p, float& a, float& b) {
  const float2 w = *reinterpret_cast<const float2*>(p);
  a = w.x;
  b = w.y;
}


template <typename DT>
__device__ __forceinline__ void process_row(const typename DT::storage* __restrict__ row, int D, int nchunk,
                                            int lane, bool want_pages, uint32_t (&pmin)[2 * kMaxPairChunks],
                                            uint32_t (&pmax)[2 * kMaxPairChunks], uint32_t& pnan,
                                            uint8_t* __restrict__ packed_row,
                                            typename DT::storage* __restrict__ scale_out,
                                            typename DT::storage* __restrict__ min_out) {
  using S = typename DT::storage;
  S v[2 * kMaxPairChunks];
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  bool any_nan = false;
#pragma unroll
  for (int c = 0; c < kMaxPairChunks; ++c) {
    if (c >= nchunk) break;
    const int d = 2 * lane + 128 * c;
    if (d < D) {
      load_pair(row + d, v[2 * c], v[2 * c + 1]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const S x = v[2 * c + h];
        const bool nan = is_nan(DT{}, x);
        const uint32_t k = order_key(DT{}, x);
        any_nan |= nan;
        kmin = k < kmin ? k : kmin;
        kmax = k > kmax ? k : kmax;
        if (want_pages) {
          pnan |= nan ? (1u << (2 * c + h)) : 0u;
          pmin[2 * c + h] = k < pmin[2 * c + h] ? k : pmin[2 * c + h];
          pmax[2 * c + h] = k > pmax[2 * c + h] ? k : pmax[2 * c + h];
        }
      }
    }
  }
  if (packed_row == nullptr) return;
  kmin = wave_min_u32(kmin);
  kmax = wave_max_u32(kmax);
  any_nan = __ballot(any_nan) != 0ull;
  S mn = any_nan ? canonical_nan(DT{}) : from_order_key(DT{}, kmin);
  S mx = any_nan ? canonical_nan(DT{}) : from_order_key(DT{}, kmax);
  const float mnf = to_f32(DT{}, mn);
  const float mxf = to_f32(DT{}, mx);
  const S sc = from_f32(DT{}, int4_scale<DT>(mnf, mxf));
  const float sf = to_f32(DT{}, sc);
#pragma unroll
  for (int c = 0; c < kMaxPairChunks; ++c) {
    if (c >= nchunk) break;
    const int d = 2 * lane + 128 * c;
    if (d < D) {
      const uint32_t lo = int4_code(to_f32(DT{}, v[2 * c]), mnf, sf);
      const uint32_t hi = int4_code(to_f32(DT{}, v[2 * c + 1]), mnf, sf);
      packed_row[d / 2] = static_cast<uint8_t>(lo | (hi << 4));
    }
  }
  if (lane == 0) {
    *scale_out = sc;
    *min_out = mn;
  }
}

template <typename DT>
__global__ __launch_bounds__(256) void build_metadata_kernel(
    const typename DT::storage* __restrict__ keys, int64_t key_entry_stride, int T, int D, int sink,
    int bs, int pages, int other_rows, typename DT::storage* __restrict__ page_min,
    typename DT::storage* __restrict__ page_max, int64_t page_entry_stride,
    uint8_t* __restrict__ packed, typename DT::storage* __restrict__ scale,
    typename DT::storage* __restrict__ minimum, int64_t quant_entry_stride) {
  using S = typename DT::storage;
  const int e = blockIdx.y;
  const int wave = blockIdx.x * (blockDim.x / kWave) + static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int other_chunks = (other_rows + 15) / 16;
  if (wave >= pages + other_chunks) return;
  const int nchunk = (D + 127) / 128;
  const S* kb = keys + static_cast<int64_t>(e) * key_entry_stride;
  const bool quant = packed != nullptr;

  uint32_t pmin[2 * kMaxPairChunks], pmax[2 * kMaxPairChunks], pnan = 0;
#pragma unroll
  for (int i = 0; i < 2 * kMaxPairChunks; ++i) {
    pmin[i] = 0xffffffffu;
    pmax[i] = 0u;
  }

  if (wave < pages) {
    const int t0 = sink + wave * bs;
    for (int i = 0; i < bs; ++i) {
      const int t = t0 + i;
      const int64_t qrow = static_cast<int64_t>(e) * quant_entry_stride + t;
      process_row<DT>(kb + static_cast<int64_t>(t) * D, D, nchunk, lane, page_min != nullptr, pmin, pmax,
                      pnan, quant ? packed + qrow * (D / 2) : nullptr, quant ? scale + qrow : nullptr,
                      quant ? minimum + qrow : nullptr);
    }
    if (page_min != nullptr) {
      S* mn_row = page_min + static_cast<int64_t>(e) * page_entry_stride + static_cast<int64_t>(wave) * D;
      S* mx_row = page_max + static_cast<int64_t>(e) * page_entry_stride + static_cast<int64_t>(wave) * D;
#pragma unroll
      for (int c = 0; c < kMaxPairChunks; ++c) {
        if (c >= nchunk) break;
        const int d = 2 * lane + 128 * c;
        if (d < D) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const bool nan = (pnan >> (2 * c + h)) & 1u;
            mn_row[d + h] = nan ? canonical_nan(DT{}) : from_order_key(DT{}, pmin[2 * c + h]);
            mx_row[d + h] = nan ? canonical_nan(DT{}) : from_order_key(DT{}, pmax[2 * c + h]);
          }
        }
      }
    }
    return;
  }
  // Rows outside complete pages (sink rows and the partial tail): INT4 only.
  if (!quant) return;
  const int head_rows = sink < T ? sink : T;
  const int base = (wave - pages) * 16;
  for (int i = 0; i < 16; ++i) {
    const int j = base + i;
    if (j >= other_rows) break;
    const int t = j < head_rows ? j : sink + pages * bs + (j - head_rows);
    const int64_t qrow = static_cast<int64_t>(e) * quant_entry_stride + t;
    process_row<DT>(kb + static_cast<int64_t>(t) * D, D, nchunk, lane, false, pmin, pmax, pnan,
                    packed + qrow * (D / 2), scale + qrow, minimum + qrow);
  }
}

// Decode-time update after row `position` of each entry was written: the
// row's INT4 code and, when the row completes page p = (position - sink) / bs
// (position - sink + 1 a multiple of bs), that page's min/max over its bs
// rows.  One wavefront per entry, the same row routine as the prompt build,
// so the result equals a rebuild over position + 1 rows bit for bit.
template <typename DT>
__global__ __launch_bounds__(256) void update_metadata_kernel(
    const typename DT::storage* __restrict__ keys, int64_t key_entry_stride, int n_entries, int position_all,
    const int32_t* __restrict__ positions, int max_position, int max_pages, int D,
    int sink, int bs, typename DT::storage* __restrict__ page_min, typename DT::storage* __restrict__ page_max,
    int64_t page_entry_stride, uint8_t* __restrict__ packed, typename DT::storage* __restrict__ scale,
    typename DT::storage* __restrict__ minimum, int64_t quant_entry_stride) {
  using S = typename DT::storage;
  const int e = blockIdx.x * (blockDim.x / kWave) + static_cast<int>(threadIdx.x) / kWave;
  if (e >= n_entries) return;
  // ragged entries: each its own row; rows beyond the buffers are skipped
  const int position = positions != nullptr ? positions[e] : position_all;
  if (position < 0 || position > max_position) return;
  if (page_min != nullptr && position >= sink && (position - sink + 1) % bs == 0 &&
      (position - sink) / bs >= max_pages)
    return;
  const int lane = lane_id();
  const int nchunk = (D + 127) / 128;
  const S* kb = keys + static_cast<int64_t>(e) * key_entry_stride;
  const bool quant = packed != nullptr;
  const int64_t qrow = static_cast<int64_t>(e) * quant_entry_stride + position;
  uint8_t* prow = quant ? packed + qrow * (D / 2) : nullptr;
  S* srow = quant ? scale + qrow : nullptr;
  S* mrow = quant ? minimum + qrow : nullptr;
  uint32_t pmin[2 * kMaxPairChunks], pmax[2 * kMaxPairChunks], pnan = 0;
#pragma unroll
  for (int i = 0; i < 2 * kMaxPairChunks; ++i) {
    pmin[i] = 0xffffffffu;
    pmax[i] = 0u;
  }
  const bool completes = page_min != nullptr && position >= sink && (position - sink + 1) % bs == 0;
  if (!completes) {
    if (quant)
      process_row<DT>(kb + static_cast<int64_t>(position) * D, D, nchunk, lane, false, pmin, pmax, pnan, prow,
                      srow, mrow);
    return;
  }
  const int page = (position - sink) / bs;
  const int t0 = sink + page * bs;
  for (int i = 0; i < bs; ++i) {
    const int t = t0 + i;
    const bool last = t == position;
    process_row<DT>(kb + static_cast<int64_t>(t) * D, D, nchunk, lane, true, pmin, pmax, pnan,
                    last ? prow : nullptr, last ? srow : nullptr, last ? mrow : nullptr);
  }
  S* mn_row = page_min + static_cast<int64_t>(e) * page_entry_stride + static_cast<int64_t>(page) * D;
  S* mx_row = page_max + static_cast<int64_t>(e) * page_entry_stride + static_cast<int64_t>(page) * D;
#pragma unroll
  for (int c = 0; c < kMaxPairChunks; ++c) {
    if (c >= nchunk) break;
    const int d = 2 * lane + 128 * c;
    if (d < D) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool nan = (pnan >> (2 * c + h)) & 1u;
        mn_row[d + h] = nan ? canonical_nan(DT{}) : from_order_key(DT{}, pmin[2 * c + h]);
        mx_row[d + h] = nan ? canonical_nan(DT{}) : from_order_key(DT{}, pmax[2 * c + h]);
      }
    }
  }
}

template <typename DT>
int launch_update(const void* keys, int64_t key_entry_stride, int n_entries, int position,
                  const int32_t* positions, int max_position, int max_pages, int D, int sink, int bs,
                  void* page_min, void* page_max, int64_t page_entry_stride, void* packed, void* scale,
                  void* minimum, int64_t quant_entry_stride, hipStream_t stream) {
  using S = typename DT::storage;
  hipLaunchKernelGGL(update_metadata_kernel<DT>, dim3((n_entries + 3) / 4), dim3(256), 0, stream,
                     static_cast<const S*>(keys), key_entry_stride, n_entries, position, positions, max_position,
                     max_pages, D, sink, bs,
                     static_cast<S*>(page_min), static_cast<S*>(page_max), page_entry_stride,
                     static_cast<uint8_t*>(packed), static_cast<S*>(scale), static_cast<S*>(minimum),
                     quant_entry_stride);
  return tw_host::check_launch();
}

int dispatch_update(int dtype, const void* keys, int64_t key_entry_stride, int n_entries, int position,
                    const int32_t* positions, int max_position, int max_pages, int D, int sink, int bs,
                    void* page_min, void* page_max, int64_t page_entry_stride, void* packed, void* scale,
                    void* minimum, int64_t quant_entry_stride, hipStream_t s) {
  switch (dtype) {
    case TW_DTYPE_F16:
      return launch_update<F16>(keys, key_entry_stride, n_entries, position, positions, max_position, max_pages, D,
                                sink, bs, page_min, page_max, page_entry_stride, packed, scale, minimum,
                                quant_entry_stride, s);
    case TW_DTYPE_BF16:
      return launch_update<BF16>(keys, key_entry_stride, n_entries, position, positions, max_position, max_pages, D,
                                 sink, bs, page_min, page_max, page_entry_stride, packed, scale, minimum,
                                 quant_entry_stride, s);
    case TW_DTYPE_F32:
      return launch_update<F32>(keys, key_entry_stride, n_entries, position, positions, max_position, max_pages, D,
                                sink, bs, page_min, page_max, page_entry_stride, packed, scale, minimum,
                                quant_entry_stride, s);
    default:
      return TW_EINVAL;
  }
}

template <typename DT>
__global__ __launch_bounds__(256) void int4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                           const typename DT::storage* __restrict__ scale,
                                                           const typename DT::storage* __restrict__ minimum,
                                                           int64_t N, int D, float* __restrict__ out) {
  const int64_t total = N * D;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / D;
    const int d = static_cast<int>(i - n * D);
    const uint32_t byte = packed[n * (D / 2) + d / 2];
    const uint32_t code = (d & 1) ? (byte >> 4) & 15u : byte & 15u;
    const float s = to_f32(DT{}, scale[n]);
    const float m = to_f32(DT{}, minimum[n]);
    out[i] = static_cast<float>(code) * s + m;
  }
}

template <typename DT>
int launch_build(const void* keys, int64_t key_entry_stride, int n_entries, int T, int D, int sink, int bs,
                 void* page_min, void* page_max, int64_t page_entry_stride, void* packed, void* scale,
                 void* minimum, int64_t quant_entry_stride, hipStream_t stream) {
  using S = typename DT::storage;
  const int pages = (page_min != nullptr && T > sink) ? (T - sink) / bs : 0;
  // Rows not covered by a page wave still need INT4 codes.
  int other_rows = 0;
  if (packed != nullptr) {
    const int head_rows = sink < T ? sink : T;
    const int covered = (page_min != nullptr) ? pages * bs : 0;
    other_rows = T - covered;
    (void)head_rows;
  }
  int pages_eff = pages;
  if (page_min == nullptr) pages_eff = 0;
  // Without page waves the "other" rows are simply all rows: treat sink as T
  // so the index mapping (j < head_rows -> j) covers everything.
  const int sink_eff = (page_min == nullptr) ? T : sink;
  const int waves = pages_eff + (other_rows + 15) / 16;
  if (waves == 0) return TW_OK;
  dim3 grid((waves + 3) / 4, n_entries);
  hipLaunchKernelGGL(build_metadata_kernel<DT>, grid, dim3(256), 0, stream, static_cast<const S*>(keys),
                     key_entry_stride, T, D, sink_eff, bs, pages_eff, other_rows, static_cast<S*>(page_min),
                     static_cast<S*>(page_max), page_entry_stride, static_cast<uint8_t*>(packed),
                     static_cast<S*>(scale), static_cast<S*>(minimum), quant_entry_stride);
  return tw_host::check_launch();
}

}  // namespace
}  // namespace tw

extern "C" int tw_build_page_metadata(const void* keys, int64_t key_entry_stride, int n_entries, int T,
                                      int D, int dtype, int sink, int block_size, void* page_min,
                                      void* page_max, int64_t page_entry_stride, void* packed, void* scale,
                                      void* minimum, int64_t quant_entry_stride, void* stream) {
  if (keys == nullptr || n_entries <= 0 || T < 0 || D <= 0 || (D % 2) != 0 || D > 1024) return TW_EINVAL;
  if (sink < 0 || block_size <= 0) return TW_EINVAL;
  if ((page_min == nullptr) != (page_max == nullptr)) return TW_EINVAL;
  if (!((packed == nullptr) == (scale == nullptr) && (scale == nullptr) == (minimum == nullptr)))
    return TW_EINVAL;
  if (key_entry_stride < static_cast<int64_t>(T) * D && n_entries > 1) return TW_EINVAL;
  if (packed != nullptr && n_entries > 1 && quant_entry_stride < T) return TW_EINVAL;
  if (T == 0) return TW_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TW_DTYPE_F16:
      return tw::launch_build<tw::F16>(keys, key_entry_stride, n_entries, T, D, sink, block_size, page_min,
                                       page_max, page_entry_stride, packed, scale, minimum,
                                       quant_entry_stride, s);
    case TW_DTYPE_BF16:
      return tw::launch_build<tw::BF16>(keys, key_entry_stride, n_entries, T, D, sink, block_size, page_min,
                                        page_max, page_entry_stride, packed, scale, minimum,
                                        quant_entry_stride, s);
    case TW_DTYPE_F32:
      return tw::launch_build<tw::F32>(keys, key_entry_stride, n_entries, T, D, sink, block_size, page_min,
                                       page_max, page_entry_stride, packed, scale, minimum,
                                       quant_entry_stride, s);
    default:
      return TW_EINVAL;
  }
}

extern "C" int tw_update_page_metadata(const void* keys, int64_t key_entry_stride, int n_entries, int position,
                                       int D, int dtype, int sink, int block_size, void* page_min, void* page_max,
                                       int64_t page_entry_stride, void* packed, void* scale, void* minimum,
                                       int64_t quant_entry_stride, void* stream) {
  if (keys == nullptr || n_entries <= 0 || position < 0 || D <= 0 || (D % 2) != 0 || D > 1024) return TW_EINVAL;
  if (sink < 0 || block_size <= 0) return TW_EINVAL;
  if ((page_min == nullptr) != (page_max == nullptr)) return TW_EINVAL;
  if (!((packed == nullptr) == (scale == nullptr) && (scale == nullptr) == (minimum == nullptr)))
    return TW_EINVAL;
  if (n_entries > 1 && key_entry_stride < static_cast<int64_t>(position + 1) * D) return TW_EINVAL;
  if (packed != nullptr && n_entries > 1 && quant_entry_stride <= position) return TW_EINVAL;
  if (page_min != nullptr && n_entries > 1 && position >= sink && (position - sink + 1) % block_size == 0 &&
      page_entry_stride < static_cast<int64_t>((position - sink) / block_size + 1) * D)
    return TW_EINVAL;
  if (page_min == nullptr && packed == nullptr) return TW_OK;
  const int big = 0x7fffffff;
  return tw::dispatch_update(dtype, keys, key_entry_stride, n_entries, position, nullptr, big, big, D, sink,
                             block_size, page_min, page_max, page_entry_stride, packed, scale, minimum,
                             quant_entry_stride, static_cast<hipStream_t>(stream));
}

extern "C" int tw_update_page_metadata_ragged(const void* keys, int64_t key_entry_stride, int n_entries,
                                              const int32_t* positions, int max_position, int D, int dtype, int sink,
                                              int block_size, void* page_min, void* page_max, int max_pages,
                                              int64_t page_entry_stride, void* packed, void* scale, void* minimum,
                                              int64_t quant_entry_stride, void* stream) {
  if (keys == nullptr || positions == nullptr || n_entries <= 0 || max_position < 0 || D <= 0 || (D % 2) != 0 ||
      D > 1024)
    return TW_EINVAL;
  if (sink < 0 || block_size <= 0) return TW_EINVAL;
  if ((page_min == nullptr) != (page_max == nullptr)) return TW_EINVAL;
  if (!((packed == nullptr) == (scale == nullptr) && (scale == nullptr) == (minimum == nullptr)))
    return TW_EINVAL;
  if (n_entries > 1 && key_entry_stride < static_cast<int64_t>(max_position + 1) * D) return TW_EINVAL;
  if (packed != nullptr && n_entries > 1 && quant_entry_stride <= max_position) return TW_EINVAL;
  if (page_min != nullptr && (max_pages < 0 || (n_entries > 1 && page_entry_stride < static_cast<int64_t>(max_pages) * D)))
    return TW_EINVAL;
  if (page_min == nullptr && packed == nullptr) return TW_OK;
  return tw::dispatch_update(dtype, keys, key_entry_stride, n_entries, 0, positions, max_position, max_pages, D,
                             sink, block_size, page_min, page_max, page_entry_stride, packed, scale, minimum,
                             quant_entry_stride, static_cast<hipStream_t>(stream));
}

extern "C" int tw_int4_dequantize(const void* packed, const void* scale, const void* minimum, int dtype,
                                  int64_t N, int D, float* out, void* stream) {
  if (N < 0 || D <= 0 || (D % 2) != 0) return TW_EINVAL;
  if (N == 0) return TW_OK;
  if (packed == nullptr || scale == nullptr || minimum == nullptr || out == nullptr) return TW_EINVAL;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t total = N * D;
  const int blocks = static_cast<int>((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  switch (dtype) {
    case TW_DTYPE_F16:
      hipLaunchKernelGGL(tw::int4_dequant_kernel<tw::F16>, dim3(blocks), dim3(256), 0, s,
                         static_cast<const uint8_t*>(packed), static_cast<const uint16_t*>(scale),
                         static_cast<const uint16_t*>(minimum), N, D, out);
      break;
    case TW_DTYPE_BF16:
      hipLaunchKernelGGL(tw::int4_dequant_kernel<tw::BF16>, dim3(blocks), dim3(256), 0, s,
                         static_cast<const uint8_t*>(packed), static_cast<const uint16_t*>(scale),
                         static_cast<const uint16_t*>(minimum), N, D, out);
      break;
    case TW_DTYPE_F32:
      hipLaunchKernelGGL(tw::int4_dequant_kernel<tw::F32>, dim3(blocks), dim3(256), 0, s,
                         static_cast<const uint8_t*>(packed), static_cast<const float*>(scale),
                         static_cast<const float*>(minimum), N, D, out);
      break;
    default:
      return TW_EINVAL;
  }
  return tw_host::check_launch();
}
