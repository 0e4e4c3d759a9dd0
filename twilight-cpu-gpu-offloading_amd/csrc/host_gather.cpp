// Host-side K/V row gather into pinned staging (the DMA variant of the host
// path): out[i] = src[rows[i]] for the K and V planes, bit-exact, with
// contiguous source runs copied by one memcpy each.
//
// Reference natives replaced: gather_kv in cpu_kv_gather.cpp:3-16 (row memcpy,
// OpenMP static schedule, returns 1 on an out-of-range row) and gather_kv in
// cpu_kv_run_gather.cpp:4-32 (runs of consecutive rows coalesced).  Here both
// behaviours are one entry point: every worker owns a contiguous slice of the
// output, walks it once, and coalesces any run of consecutive source rows
// (there is no minimum run length, a one-row run is an ordinary row copy).
// Invalid rows are skipped and reported through the return value, matching
// the reference's "return 1" contract.
#include <omp.h>

#include <cstdint>
#include <cstring>

#include "../../include/twilight_host.h"

extern "C" int tw_host_gather_kv(const void* k, const void* v, void* out_k, void* out_v, const int64_t* rows,
                                 int64_t n, int64_t source_rows, int64_t row_bytes, int threads) {
  if (n < 0 || source_rows < 0 || row_bytes <= 0 || threads <= 0) return TW_HOST_EINVAL;
  if (n == 0) return TW_HOST_OK;
  if (k == nullptr || v == nullptr || out_k == nullptr || out_v == nullptr || rows == nullptr) return TW_HOST_EINVAL;
  const auto* ks = static_cast<const unsigned char*>(k);
  const auto* vs = static_cast<const unsigned char*>(v);
  auto* ok = static_cast<unsigned char*>(out_k);
  auto* ov = static_cast<unsigned char*>(out_v);
  int invalid = 0;
  const int workers = static_cast<int64_t>(threads) > n ? static_cast<int>(n) : threads;
#pragma omp parallel num_threads(workers) reduction(| : invalid)
  {
    const int w = omp_get_thread_num();
    const int nw = omp_get_num_threads();
    int64_t i = n * w / nw;
    const int64_t end = n * (w + 1) / nw;
    while (i < end) {
      const int64_t r = rows[i];
      if (r < 0 || r >= source_rows) {
        invalid = 1;
        ++i;
        continue;
      }
      int64_t run = 1;
      while (i + run < end && r + run < source_rows && rows[i + run] == r + run) ++run;
      std::memcpy(ok + i * row_bytes, ks + r * row_bytes, static_cast<size_t>(run * row_bytes));
      std::memcpy(ov + i * row_bytes, vs + r * row_bytes, static_cast<size_t>(run * row_bytes));
      i += run;
    }
  }
  return invalid ? TW_HOST_ERANGE : TW_HOST_OK;
}

// Sorted set union of position lists over a bounded membership array
// (replaces CpuTokenUnion, cpu_token_union.py:6-23): marks every position of
// every list, then writes the marked positions ascending.
extern "C" int64_t tw_host_token_union(const int64_t* const* lists, const int64_t* list_sizes, int n_lists,
                                       int64_t length, uint8_t* scratch, int64_t* out) {
  if (n_lists < 0 || length < 0 || (length > 0 && (scratch == nullptr || out == nullptr))) return -1;
  std::memset(scratch, 0, static_cast<size_t>(length));
  for (int l = 0; l < n_lists; ++l) {
    const int64_t* p = lists[l];
    for (int64_t j = 0; j < list_sizes[l]; ++j) {
      const int64_t x = p[j];
      if (x < 0 || x >= length) return -2;
      scratch[x] = 1;
    }
  }
  int64_t count = 0;
  for (int64_t t = 0; t < length; ++t) {
    if (scratch[t]) out[count++] = t;
  }
  return count;
}
