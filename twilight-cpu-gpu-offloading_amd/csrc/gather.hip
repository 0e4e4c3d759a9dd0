// Head-wise K/V row movement: gather by index (from HBM or zero-copy from
// mapped pinned host memory) and the per-step append of the decode token.
//
// Reference: the CPU index_select + H2D of the offload caches
// (quest_offload_cache.py:576-624, 816-936; twilight_offload_cache.py:
// 2973-3101), the mapped-host assembly kernel assemble_zero_copy
// (resident_zero_copy.cu:7-65) and the new-token D2H
// (quest_offload_cache.py:230-274; twilight_offload_cache.py:551-794).
//
// One 16-byte transfer per lane; a row of 128 16-bit values is 16 lanes, so a
// wavefront moves 4 rows per instruction and consecutive rows of a page are
// one contiguous 1 KB burst.  Over the host link the same access pattern keeps
// many 64-byte PCIe reads in flight per CU, which is what zero-copy needs.
#include "tw_common.h"

namespace tw {
namespace {

template <typename V>
__global__ __launch_bounds__(256) void gather_rows_kernel(const V* __restrict__ src_k, const V* __restrict__ src_v,
                                                          int64_t src_row_limit, const int64_t* __restrict__ src_rows,
                                                          const int64_t* __restrict__ dst_rows, int64_t n,
                                                          int64_t dst_row_limit, int vec_per_row,
                                                          V* __restrict__ dst_k, V* __restrict__ dst_v,
                                                          int32_t* error_flag) {
  const int64_t total = n * vec_per_row;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = t / vec_per_row;
    const int c = static_cast<int>(t - i * vec_per_row);
    const int64_t sr = src_rows[i];
    if (sr < 0 || sr >= src_row_limit) {
      if (c == 0 && error_flag != nullptr) *error_flag = 1;
      continue;
    }
    const int64_t dr = dst_rows != nullptr ? dst_rows[i] : i;
    if (dr < 0 || dr >= dst_row_limit) {
      if (c == 0 && error_flag != nullptr) *error_flag = 1;
      continue;
    }
    dst_k[dr * vec_per_row + c] = src_k[sr * vec_per_row + c];
    dst_v[dr * vec_per_row + c] = src_v[sr * vec_per_row + c];
  }
}

template <typename V>
__global__ void append_kv_kernel(const V* __restrict__ new_k, const V* __restrict__ new_v, int n, int vec_per_row,
                                 V* __restrict__ dst_k, V* __restrict__ dst_v, int64_t entry_stride_rows,
                                 int first_entry, int64_t position) {
  const int total = n * vec_per_row;
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    const int i = t / vec_per_row;
    const int c = t - i * vec_per_row;
    const int64_t dr = (static_cast<int64_t>(first_entry) + i) * entry_stride_rows + position;
    dst_k[dr * vec_per_row + c] = new_k[static_cast<int64_t>(i) * vec_per_row + c];
    dst_v[dr * vec_per_row + c] = new_v[static_cast<int64_t>(i) * vec_per_row + c];
  }
}

// Group-union layout (the varlen attention input of the GQA group path):
// group g's rows[g][0 .. counts[g]) then its decode token, packed back to
// back, so group g starts at off_g = sum_{h<g} (counts[h] + 1).  Block b
// covers rows [chunk*rows_per_block, ...) of group g = b / chunks; every
// block recomputes off_g from the (few) counts.  Block 0 writes cu_seqlens.
template <typename V>
__global__ __launch_bounds__(256) void gather_union_kernel(const V* __restrict__ src_k, const V* __restrict__ src_v,
                                                           int64_t src_row_limit, int64_t entry_row0,
                                                           int64_t entry_row_step, const int32_t* __restrict__ rows,
                                                           int64_t rows_stride, const int32_t* __restrict__ counts,
                                                           int G, int max_count, const V* __restrict__ cur_k,
                                                           const V* __restrict__ cur_v, int vec_per_row,
                                                           int64_t dst_capacity, V* __restrict__ dst_k,
                                                           V* __restrict__ dst_v, int32_t* cu_seqlens,
                                                           int32_t* error_flag, int chunks, int rows_per_block) {
  const int g = blockIdx.x / chunks;
  const int chunk = blockIdx.x - g * chunks;
  __shared__ int64_t s_off;
  __shared__ int s_count;
  if (threadIdx.x == 0) {
    int64_t off = 0;
    for (int h = 0; h < g; ++h) {
      int c = counts[h];
      c = c < 0 ? 0 : (c > max_count ? max_count : c);
      off += c + 1;
    }
    int c = counts[g];
    s_count = c < 0 ? 0 : (c > max_count ? max_count : c);
    s_off = off;
    if (blockIdx.x == 0) {
      int64_t run = 0;
      cu_seqlens[0] = 0;
      for (int h = 0; h < G; ++h) {
        int ch = counts[h];
        ch = ch < 0 ? 0 : (ch > max_count ? max_count : ch);
        run += ch + 1;
        cu_seqlens[h + 1] = static_cast<int32_t>(run);
      }
    }
  }
  __syncthreads();
  const int count = s_count;
  const int64_t off = s_off;
  const int first = chunk * rows_per_block;
  const int last = (first + rows_per_block) < (count + 1) ? (first + rows_per_block) : (count + 1);
  const int64_t row0 = entry_row0 + static_cast<int64_t>(g) * entry_row_step;
  for (int t = first * vec_per_row + static_cast<int>(threadIdx.x); t < last * vec_per_row; t += blockDim.x) {
    const int i = t / vec_per_row;
    const int c = t - i * vec_per_row;
    const int64_t dr = off + i;
    if (dr >= dst_capacity) {
      if (error_flag != nullptr) *error_flag = 1;
      continue;
    }
    if (i == count) {  // the decode token
      dst_k[dr * vec_per_row + c] = cur_k[static_cast<int64_t>(g) * vec_per_row + c];
      dst_v[dr * vec_per_row + c] = cur_v[static_cast<int64_t>(g) * vec_per_row + c];
      continue;
    }
    const int64_t sr = row0 + rows[static_cast<int64_t>(g) * rows_stride + i];
    if (sr < 0 || sr >= src_row_limit) {
      if (error_flag != nullptr) *error_flag = 1;
      continue;
    }
    dst_k[dr * vec_per_row + c] = src_k[sr * vec_per_row + c];
    dst_v[dr * vec_per_row + c] = src_v[sr * vec_per_row + c];
  }
}

// gather_union_kernel with the previous-token resident cache of the GQA-group
// path: res_map [G][map_stride] (int64, position-indexed, initialised to -1)
// holds (epoch << 32) | flat index of the step that last gathered each
// position, and prev_k/prev_v (with prev_cu [G + 1]) that step's flat output.
// A union row whose entry names epoch - 1 (the previous step) is copied from
// there (HBM) instead of from the slab; after the block's copies, its rows'
// entries name this step (each position is one row of one block, so no other
// block reads them in this launch).  res_stats [2] (nullable) accumulates
// (rows copied from the previous step, union rows).
template <typename V>
__global__ __launch_bounds__(256) void gather_union_resident_kernel(
    const V* __restrict__ src_k, const V* __restrict__ src_v, int64_t src_row_limit, int64_t entry_row0,
    int64_t entry_row_step, const int32_t* __restrict__ rows, int64_t rows_stride, const int32_t* __restrict__ counts,
    int G, int max_count, const V* __restrict__ cur_k, const V* __restrict__ cur_v, int vec_per_row,
    int64_t dst_capacity, V* __restrict__ dst_k, V* __restrict__ dst_v, int32_t* cu_seqlens, int32_t* error_flag,
    int chunks, int rows_per_block, int64_t* res_map, int64_t map_stride, int epoch, const V* __restrict__ prev_k,
    const V* __restrict__ prev_v, const int32_t* __restrict__ prev_cu, int64_t prev_capacity,
    unsigned long long* res_stats) {
  const int g = blockIdx.x / chunks;
  const int chunk = blockIdx.x - g * chunks;
  __shared__ int64_t s_off;
  __shared__ int s_count;
  __shared__ int64_t s_prev;
  __shared__ unsigned int s_hits, s_rows;
  if (threadIdx.x == 0) {
    int64_t off = 0;
    for (int h = 0; h < g; ++h) {
      int c = counts[h];
      c = c < 0 ? 0 : (c > max_count ? max_count : c);
      off += c + 1;
    }
    int c = counts[g];
    s_count = c < 0 ? 0 : (c > max_count ? max_count : c);
    s_off = off;
    s_prev = prev_cu[g];
    s_hits = 0u;
    s_rows = 0u;
    if (blockIdx.x == 0) {
      int64_t run = 0;
      cu_seqlens[0] = 0;
      for (int h = 0; h < G; ++h) {
        int ch = counts[h];
        ch = ch < 0 ? 0 : (ch > max_count ? max_count : ch);
        run += ch + 1;
        cu_seqlens[h + 1] = static_cast<int32_t>(run);
      }
    }
  }
  __syncthreads();
  const int count = s_count;
  const int64_t off = s_off;
  const int64_t prev0 = s_prev;
  const int first = chunk * rows_per_block;
  const int last = (first + rows_per_block) < (count + 1) ? (first + rows_per_block) : (count + 1);
  const int64_t row0 = entry_row0 + static_cast<int64_t>(g) * entry_row_step;
  int64_t* gmap = res_map + static_cast<int64_t>(g) * map_stride;
  for (int t = first * vec_per_row + static_cast<int>(threadIdx.x); t < last * vec_per_row; t += blockDim.x) {
    const int i = t / vec_per_row;
    const int c = t - i * vec_per_row;
    const int64_t dr = off + i;
    if (dr >= dst_capacity) {
      if (error_flag != nullptr) *error_flag = 1;
      continue;
    }
    if (i == count) {  // the decode token
      dst_k[dr * vec_per_row + c] = cur_k[static_cast<int64_t>(g) * vec_per_row + c];
      dst_v[dr * vec_per_row + c] = cur_v[static_cast<int64_t>(g) * vec_per_row + c];
      continue;
    }
    const int pos = rows[static_cast<int64_t>(g) * rows_stride + i];
    const int64_t sr = row0 + pos;
    if (sr < 0 || sr >= src_row_limit || pos < 0 || pos >= map_stride) {
      if (error_flag != nullptr) *error_flag = 1;
      continue;
    }
    const int64_t m = gmap[pos];
    const int64_t pr = prev0 + (m & 0xffffffffll);
    const bool hit = (m >> 32) == static_cast<int64_t>(epoch) - 1 && pr < prev_capacity;
    if (c == 0) {
      atomicAdd(&s_rows, 1u);
      if (hit) atomicAdd(&s_hits, 1u);
    }
    dst_k[dr * vec_per_row + c] = hit ? prev_k[pr * vec_per_row + c] : src_k[sr * vec_per_row + c];
    dst_v[dr * vec_per_row + c] = hit ? prev_v[pr * vec_per_row + c] : src_v[sr * vec_per_row + c];
  }
  __syncthreads();  // every map entry of the block's rows has been read
  for (int i = first + static_cast<int>(threadIdx.x); i < last && i < count; i += blockDim.x) {
    const int pos = rows[static_cast<int64_t>(g) * rows_stride + i];
    if (pos >= 0 && pos < map_stride) gmap[pos] = (static_cast<int64_t>(epoch) << 32) | static_cast<int64_t>(i);
  }
  if (threadIdx.x == 0 && res_stats != nullptr && s_rows > 0u) {
    atomicAdd(res_stats, static_cast<unsigned long long>(s_hits));
    atomicAdd(res_stats + 1, static_cast<unsigned long long>(s_rows));
  }
}

// Per-query-head layout of the Quest paths: head r of group g sees
// [0, sink_end) ++ its own pages sel[g][r][0..k) (ascending) expanded to bs
// rows ++ [recent_start, length), then the decode token; its row t goes to
// dst row g*dst_g_stride + r*dst_r_stride + t*dst_t_stride.  Every row's
// source follows from t directly, so the whole copy is one flat grid.
template <typename V>
__global__ __launch_bounds__(256) void gather_heads_kernel(
    const V* __restrict__ src_k, const V* __restrict__ src_v, int64_t src_row_limit, int64_t entry_row0,
    int64_t entry_row_step, const int32_t* __restrict__ sel, int G, int R, int k, int sink, int bs, int sink_end,
    int recent_start, int length, const V* __restrict__ cur_k, const V* __restrict__ cur_v, int vec_per_row,
    int64_t dst_g_stride, int64_t dst_r_stride, int64_t dst_t_stride, V* __restrict__ dst_k, V* __restrict__ dst_v,
    int32_t* error_flag) {
  const int per_head = sink_end + k * bs + (length - recent_start) + 1;
  const int64_t total = static_cast<int64_t>(G) * R * per_head * vec_per_row;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = t / vec_per_row;
    const int c = static_cast<int>(t - row * vec_per_row);
    const int gr = static_cast<int>(row / per_head);
    const int i = static_cast<int>(row - static_cast<int64_t>(gr) * per_head);
    const int g = gr / R;
    const int r = gr - g * R;
    const int64_t dr = g * dst_g_stride + r * dst_r_stride + i * dst_t_stride;
    if (i == per_head - 1) {
      dst_k[dr * vec_per_row + c] = cur_k[static_cast<int64_t>(g) * vec_per_row + c];
      dst_v[dr * vec_per_row + c] = cur_v[static_cast<int64_t>(g) * vec_per_row + c];
      continue;
    }
    int64_t pos;
    if (i < sink_end) {
      pos = i;
    } else if (i < sink_end + k * bs) {
      const int j = i - sink_end;
      const int u = j / bs;
      pos = sink + static_cast<int64_t>(sel[(static_cast<int64_t>(g) * R + r) * k + u]) * bs + (j - u * bs);
    } else {
      pos = recent_start + (i - sink_end - k * bs);
    }
    const int64_t sr = entry_row0 + static_cast<int64_t>(g) * entry_row_step + pos;
    if (pos < 0 || pos >= length || sr < 0 || sr >= src_row_limit) {
      if (error_flag != nullptr) *error_flag = 1;
      continue;
    }
    dst_k[dr * vec_per_row + c] = src_k[sr * vec_per_row + c];
    dst_v[dr * vec_per_row + c] = src_v[sr * vec_per_row + c];
  }
}

int vec_width(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  int w = 16;
  for (const void* p : ptrs) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    while (w > 1 && (a % w) != 0) w >>= 1;
  }
  while (w > 1 && (row_bytes % w) != 0) w >>= 1;
  return w;
}

template <typename V>
int launch_gather(const void* sk, const void* sv, int64_t limit, const int64_t* sr, const int64_t* dr, int64_t n,
                  int64_t dst_limit, int64_t row_bytes, void* dk, void* dv, int32_t* err, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  const int64_t total = n * vpr;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(gather_rows_kernel<V>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<const V*>(sk), static_cast<const V*>(sv), limit, sr, dr, n, dst_limit, vpr,
                     static_cast<V*>(dk), static_cast<V*>(dv), err);
  return tw_host::check_launch();
}

template <typename V>
int launch_append(const void* nk, const void* nv, int n, int64_t row_bytes, void* dk, void* dv, int64_t es,
                  int first, int64_t pos, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  const int total = n * vpr;
  const int blocks = (total + 255) / 256;
  hipLaunchKernelGGL(append_kv_kernel<V>, dim3(blocks), dim3(256), 0, stream, static_cast<const V*>(nk),
                     static_cast<const V*>(nv), n, vpr, static_cast<V*>(dk), static_cast<V*>(dv), es, first, pos);
  return tw_host::check_launch();
}

}  // namespace
}  // namespace tw

extern "C" int tw_gather_rows(const void* src_k, const void* src_v, int64_t src_row_limit, const int64_t* src_rows,
                              const int64_t* dst_rows, int64_t n, int64_t dst_row_limit, int D, int elem_bytes,
                              void* dst_k, void* dst_v, int32_t* error_flag, void* stream) {
  if (n < 0 || D <= 0 || dst_row_limit < 0 ||
      !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (n == 0) return TW_OK;
  // without dst_rows the destination rows are 0 .. n-1
  if (dst_rows == nullptr && n > dst_row_limit) return TW_EINVAL;
  if (src_k == nullptr || src_v == nullptr || src_rows == nullptr || dst_k == nullptr || dst_v == nullptr)
    return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (tw::vec_width(row_bytes, {src_k, src_v, dst_k, dst_v})) {
    case 16: return tw::launch_gather<uint4>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, dst_row_limit, row_bytes, dst_k, dst_v, error_flag, s);
    case 8: return tw::launch_gather<uint2>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, dst_row_limit, row_bytes, dst_k, dst_v, error_flag, s);
    case 4: return tw::launch_gather<uint32_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, dst_row_limit, row_bytes, dst_k, dst_v, error_flag, s);
    case 2: return tw::launch_gather<uint16_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, dst_row_limit, row_bytes, dst_k, dst_v, error_flag, s);
    default: return tw::launch_gather<uint8_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, dst_row_limit, row_bytes, dst_k, dst_v, error_flag, s);
  }
}

extern "C" int tw_append_kv(const void* new_k, const void* new_v, int n_entries, int D, int elem_bytes, void* dst_k,
                            void* dst_v, int64_t entry_stride_rows, int first_entry, int64_t position, void* stream) {
  if (n_entries < 0 || D <= 0 || first_entry < 0 || position < 0 || position >= entry_stride_rows ||
      !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (n_entries == 0) return TW_OK;
  if (new_k == nullptr || new_v == nullptr || dst_k == nullptr || dst_v == nullptr) return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (tw::vec_width(row_bytes, {new_k, new_v, dst_k, dst_v})) {
    case 16: return tw::launch_append<uint4>(new_k, new_v, n_entries, row_bytes, dst_k, dst_v, entry_stride_rows, first_entry, position, s);
    case 8: return tw::launch_append<uint2>(new_k, new_v, n_entries, row_bytes, dst_k, dst_v, entry_stride_rows, first_entry, position, s);
    case 4: return tw::launch_append<uint32_t>(new_k, new_v, n_entries, row_bytes, dst_k, dst_v, entry_stride_rows, first_entry, position, s);
    case 2: return tw::launch_append<uint16_t>(new_k, new_v, n_entries, row_bytes, dst_k, dst_v, entry_stride_rows, first_entry, position, s);
    default: return tw::launch_append<uint8_t>(new_k, new_v, n_entries, row_bytes, dst_k, dst_v, entry_stride_rows, first_entry, position, s);
  }
}

extern "C" int tw_host_device_pointer(void* host_ptr, void** device_ptr) {
  if (host_ptr == nullptr || device_ptr == nullptr) return TW_EINVAL;
  void* dev = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dev, host_ptr, 0);
  if (e != hipSuccess) return tw_host::record_hip_error(e);
  *device_ptr = dev;
  return TW_OK;
}

namespace tw {
namespace {

template <typename V>
int launch_union(const void* sk, const void* sv, int64_t limit, int64_t row0, int64_t step, const int32_t* rows,
                 int64_t rows_stride, const int32_t* counts, int G, int max_count, const void* ck, const void* cv,
                 int64_t row_bytes, int64_t cap, void* dk, void* dv, int32_t* cu, int32_t* err, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  // about 16 KB of row data per block
  int rpb = static_cast<int>(16384 / row_bytes);
  rpb = rpb < 1 ? 1 : rpb;
  const int chunks = (max_count + 1 + rpb - 1) / rpb;
  hipLaunchKernelGGL(gather_union_kernel<V>, dim3(G * chunks), dim3(256), 0, stream, static_cast<const V*>(sk),
                     static_cast<const V*>(sv), limit, row0, step, rows, rows_stride, counts, G, max_count,
                     static_cast<const V*>(ck), static_cast<const V*>(cv), vpr, cap, static_cast<V*>(dk),
                     static_cast<V*>(dv), cu, err, chunks, rpb);
  return tw_host::check_launch();
}

template <typename V>
int launch_union_resident(const void* sk, const void* sv, int64_t limit, int64_t row0, int64_t step,
                          const int32_t* rows, int64_t rows_stride, const int32_t* counts, int G, int max_count,
                          const void* ck, const void* cv, int64_t row_bytes, int64_t cap, void* dk, void* dv,
                          int32_t* cu, int32_t* err, int64_t* res_map, int64_t map_stride, int epoch,
                          const void* pk, const void* pv, const int32_t* prev_cu, int64_t prev_cap,
                          unsigned long long* stats, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  int rpb = static_cast<int>(16384 / row_bytes);
  rpb = rpb < 1 ? 1 : rpb;
  const int chunks = (max_count + 1 + rpb - 1) / rpb;
  hipLaunchKernelGGL(gather_union_resident_kernel<V>, dim3(G * chunks), dim3(256), 0, stream,
                     static_cast<const V*>(sk), static_cast<const V*>(sv), limit, row0, step, rows, rows_stride,
                     counts, G, max_count, static_cast<const V*>(ck), static_cast<const V*>(cv), vpr, cap,
                     static_cast<V*>(dk), static_cast<V*>(dv), cu, err, chunks, rpb, res_map, map_stride, epoch,
                     static_cast<const V*>(pk), static_cast<const V*>(pv), prev_cu, prev_cap, stats);
  return tw_host::check_launch();
}

template <typename V>
int launch_heads(const void* sk, const void* sv, int64_t limit, int64_t row0, int64_t step, const int32_t* sel, int G,
                 int R, int k, int sink, int bs, int sink_end, int recent_start, int length, const void* ck,
                 const void* cv, int64_t row_bytes, int64_t gs, int64_t rs, int64_t ts, void* dk, void* dv,
                 int32_t* err, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  const int64_t per_head = sink_end + static_cast<int64_t>(k) * bs + (length - recent_start) + 1;
  const int64_t total = static_cast<int64_t>(G) * R * per_head * vpr;
  int64_t blocks = (total + 255) / 256;
  blocks = blocks > 8192 ? 8192 : (blocks < 1 ? 1 : blocks);
  hipLaunchKernelGGL(gather_heads_kernel<V>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<const V*>(sk), static_cast<const V*>(sv), limit, row0, step, sel, G, R, k, sink, bs,
                     sink_end, recent_start, length, static_cast<const V*>(ck), static_cast<const V*>(cv), vpr, gs,
                     rs, ts, static_cast<V*>(dk), static_cast<V*>(dv), err);
  return tw_host::check_launch();
}

}  // namespace
}  // namespace tw

extern "C" int tw_gather_union(const void* src_k, const void* src_v, int64_t src_row_limit, int64_t entry_row0,
                               int64_t entry_row_step, const int32_t* rows, int64_t rows_stride,
                               const int32_t* row_counts, int G, int max_count, const void* cur_k, const void* cur_v,
                               int D, int elem_bytes, int64_t dst_capacity, void* dst_k, void* dst_v,
                               int32_t* cu_seqlens, int32_t* error_flag, void* stream) {
  if (G <= 0 || max_count < 0 || D <= 0 || rows_stride < max_count || dst_capacity <= 0 ||
      !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (src_k == nullptr || src_v == nullptr || rows == nullptr || row_counts == nullptr || cur_k == nullptr ||
      cur_v == nullptr || dst_k == nullptr || dst_v == nullptr || cu_seqlens == nullptr)
    return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
#define TW_UNION(V)                                                                                             \
  tw::launch_union<V>(src_k, src_v, src_row_limit, entry_row0, entry_row_step, rows, rows_stride, row_counts, G, \
                      max_count, cur_k, cur_v, row_bytes, dst_capacity, dst_k, dst_v, cu_seqlens, error_flag, s)
  switch (tw::vec_width(row_bytes, {src_k, src_v, dst_k, dst_v, cur_k, cur_v})) {
    case 16: return TW_UNION(uint4);
    case 8: return TW_UNION(uint2);
    case 4: return TW_UNION(uint32_t);
    case 2: return TW_UNION(uint16_t);
    default: return TW_UNION(uint8_t);
  }
#undef TW_UNION
}

extern "C" int tw_gather_union_resident(const void* src_k, const void* src_v, int64_t src_row_limit,
                                        int64_t entry_row0, int64_t entry_row_step, const int32_t* rows,
                                        int64_t rows_stride, const int32_t* row_counts, int G, int max_count,
                                        const void* cur_k, const void* cur_v, int D, int elem_bytes,
                                        int64_t dst_capacity, void* dst_k, void* dst_v, int32_t* cu_seqlens,
                                        int32_t* error_flag, int64_t* res_map, int64_t map_stride, int epoch,
                                        const void* prev_k, const void* prev_v, const int32_t* prev_cu,
                                        int64_t prev_capacity, unsigned long long* res_stats, void* stream) {
  if (G <= 0 || max_count < 0 || D <= 0 || rows_stride < max_count || dst_capacity <= 0 ||
      !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (src_k == nullptr || src_v == nullptr || rows == nullptr || row_counts == nullptr || cur_k == nullptr ||
      cur_v == nullptr || dst_k == nullptr || dst_v == nullptr || cu_seqlens == nullptr)
    return TW_EINVAL;
  if (res_map == nullptr || map_stride < 1 || epoch < 1 || prev_k == nullptr || prev_v == nullptr ||
      prev_cu == nullptr || prev_capacity < 0)
    return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
#define TW_UNION_RES(V)                                                                                           \
  tw::launch_union_resident<V>(src_k, src_v, src_row_limit, entry_row0, entry_row_step, rows, rows_stride,        \
                               row_counts, G, max_count, cur_k, cur_v, row_bytes, dst_capacity, dst_k, dst_v,      \
                               cu_seqlens, error_flag, res_map, map_stride, epoch, prev_k, prev_v, prev_cu,        \
                               prev_capacity, res_stats, s)
  switch (tw::vec_width(row_bytes, {src_k, src_v, dst_k, dst_v, cur_k, cur_v, prev_k, prev_v})) {
    case 16: return TW_UNION_RES(uint4);
    case 8: return TW_UNION_RES(uint2);
    case 4: return TW_UNION_RES(uint32_t);
    case 2: return TW_UNION_RES(uint16_t);
    default: return TW_UNION_RES(uint8_t);
  }
#undef TW_UNION_RES
}

extern "C" int tw_gather_heads(const void* src_k, const void* src_v, int64_t src_row_limit, int64_t entry_row0,
                               int64_t entry_row_step, const int32_t* sel_pages, int G, int R, int k, int sink,
                               int recent, int block_size, int length, const void* cur_k, const void* cur_v, int D,
                               int elem_bytes, int64_t dst_g_stride, int64_t dst_r_stride, int64_t dst_t_stride,
                               int64_t dst_capacity, void* dst_k, void* dst_v, int32_t* error_flag, void* stream) {
  if (G <= 0 || R <= 0 || k < 0 || sink < 0 || recent <= 0 || block_size <= 0 || length < 0 || D <= 0 ||
      dst_g_stride < 0 || dst_r_stride < 0 || dst_t_stride < 0 ||
      !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (src_k == nullptr || src_v == nullptr || (k > 0 && sel_pages == nullptr) || cur_k == nullptr ||
      cur_v == nullptr || dst_k == nullptr || dst_v == nullptr)
    return TW_EINVAL;
  const int sink_end = sink < length ? sink : length;
  const int hist_recent = recent - 1 > 0 ? recent - 1 : 0;
  const int recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
  if (k > 0 && sink + static_cast<int64_t>(k) * block_size > recent_start) return TW_EINVAL;
  const int64_t per_head = sink_end + static_cast<int64_t>(k) * block_size + (length - recent_start) + 1;
  const int64_t last_row = (G - 1) * dst_g_stride + (R - 1) * dst_r_stride + (per_head - 1) * dst_t_stride;
  if (last_row >= dst_capacity) return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
#define TW_HEADS(V)                                                                                               \
  tw::launch_heads<V>(src_k, src_v, src_row_limit, entry_row0, entry_row_step, sel_pages, G, R, k, sink,          \
                      block_size, sink_end, recent_start, length, cur_k, cur_v, row_bytes, dst_g_stride,           \
                      dst_r_stride, dst_t_stride, dst_k, dst_v, error_flag, s)
  switch (tw::vec_width(row_bytes, {src_k, src_v, dst_k, dst_v, cur_k, cur_v})) {
    case 16: return TW_HEADS(uint4);
    case 8: return TW_HEADS(uint2);
    case 4: return TW_HEADS(uint32_t);
    case 2: return TW_HEADS(uint16_t);
    default: return TW_HEADS(uint8_t);
  }
#undef TW_HEADS
}
