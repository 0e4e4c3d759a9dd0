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
                                                          int vec_per_row, V* __restrict__ dst_k,
                                                          V* __restrict__ dst_v, int32_t* error_flag) {
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
                  int64_t row_bytes, void* dk, void* dv, int32_t* err, hipStream_t stream) {
  const int vpr = static_cast<int>(row_bytes / sizeof(V));
  const int64_t total = n * vpr;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(gather_rows_kernel<V>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     static_cast<const V*>(sk), static_cast<const V*>(sv), limit, sr, dr, n, vpr, static_cast<V*>(dk),
                     static_cast<V*>(dv), err);
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
                              const int64_t* dst_rows, int64_t n, int D, int elem_bytes, void* dst_k, void* dst_v,
                              int32_t* error_flag, void* stream) {
  if (n < 0 || D <= 0 || !(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8))
    return TW_EINVAL;
  if (n == 0) return TW_OK;
  if (src_k == nullptr || src_v == nullptr || src_rows == nullptr || dst_k == nullptr || dst_v == nullptr)
    return TW_EINVAL;
  const int64_t row_bytes = static_cast<int64_t>(D) * elem_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (tw::vec_width(row_bytes, {src_k, src_v, dst_k, dst_v})) {
    case 16: return tw::launch_gather<uint4>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, row_bytes, dst_k, dst_v, error_flag, s);
    case 8: return tw::launch_gather<uint2>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, row_bytes, dst_k, dst_v, error_flag, s);
    case 4: return tw::launch_gather<uint32_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, row_bytes, dst_k, dst_v, error_flag, s);
    case 2: return tw::launch_gather<uint16_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, row_bytes, dst_k, dst_v, error_flag, s);
    default: return tw::launch_gather<uint8_t>(src_k, src_v, src_row_limit, src_rows, dst_rows, n, row_bytes, dst_k, dst_v, error_flag, s);
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
