/*
 * twilight_host.h - C ABI of the host-side natives of the sparse-decode KV
 * path (libtwilight_host.so, built with g++ -fopenmp).  Same conventions as
 * twilight_hip.h: raw pointers, int64 sizes, int status.
 */
#ifndef TWILIGHT_HOST_H
#define TWILIGHT_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tw_host_status { TW_HOST_OK = 0, TW_HOST_ERANGE = 1, TW_HOST_EINVAL = 2 };

/* Row gather into (pinned) staging.
 * Replaces gather_kv of cpu_kv_gather.cpp:3-16 and cpu_kv_run_gather.cpp:
 * 4-32 (bound by CpuKVGather / CpuKVRunGather, cpu_kv_gather.py:9-36,
 * cpu_kv_run_gather.py:8-17).  out_k[i] = k[rows[i]], out_v[i] = v[rows[i]],
 * row_bytes each; contiguous source runs are copied as one block; rows
 * outside [0, source_rows) are skipped and the call returns TW_HOST_ERANGE
 * (the reference returns 1, mapped to ValueError).  threads: OpenMP workers. */
int tw_host_gather_kv(const void* k, const void* v, void* out_k, void* out_v, const int64_t* rows, int64_t n,
                      int64_t source_rows, int64_t row_bytes, int threads);

/* CPU token union: sorted union of n_lists int64 position lists, all in
 * [0, length).  Replaces CpuTokenUnion.__call__ (cpu_token_union.py:13-23).
 * scratch: length bytes; out: room for length positions.  Returns the union
 * size, -1 on bad arguments, -2 if a position is outside [0, length). */
int64_t tw_host_token_union(const int64_t* const* lists, const int64_t* list_sizes, int n_lists, int64_t length,
                            uint8_t* scratch, int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* TWILIGHT_HOST_H */
