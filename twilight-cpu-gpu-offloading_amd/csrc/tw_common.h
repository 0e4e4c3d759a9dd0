// Shared device helpers for the sparse-decode KV path on CDNA4 (gfx950).
//
// Every kernel in this library is written for 64-lane wavefronts.  Arithmetic
// whose rounding is part of the parity contract (page scores, INT4 scale and
// codes, QK estimates) uses the explicit IEEE intrinsics below and the whole
// library is compiled with -ffp-contract=off, so no multiply/add pair is ever
// fused behind our back.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/twilight_hip.h"

namespace tw {

constexpr int kWave = 64;

// Arrival counters (one 32-bit counter per KV group) sit in a fixed region at
// the start of every selection workspace, [0, kCounterRegionBytes); the
// workspace's data starts after it.  The kernels return every counter they
// use to zero, so with the buffer zeroed once, no later call -- whatever its
// group count or sizes -- finds data of an earlier call on its counters.
constexpr int kMaxCounterGroups = 16384;
constexpr size_t kCounterRegionBytes = static_cast<size_t>(kMaxCounterGroups) * 4;  // 64 KiB

// ---------------------------------------------------------------- dtypes
// Storage types: 16-bit formats are carried as raw uint16_t bit patterns so the
// conversions below (and therefore every rounding step) are explicit.
struct F16 {
  using storage = uint16_t;
  static constexpr int code = TW_DTYPE_F16;
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int code = TW_DTYPE_BF16;
};
struct F32 {
  using storage = float;
  static constexpr int code = TW_DTYPE_F32;
};

__device__ __forceinline__ float u32_as_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f32_as_u32(float f) { return __float_as_uint(f); }

// Exact widening conversions.
__device__ __forceinline__ float to_f32(F16, uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ float to_f32(BF16, uint16_t h) {
  return u32_as_f32(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ float to_f32(F32, float f) { return f; }

// Round-to-nearest-even narrowing conversions (NaN -> canonical quiet NaN).
__device__ __forceinline__ uint16_t from_f32(F16, float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ uint16_t from_f32(BF16, float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>(((u >> 16) & 0x8000u) | 0x7fc0u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float from_f32(F32, float f) { return f; }

// Round a float to the storage precision and back (the "compute in the key
// dtype" step of a 16-bit subtraction).
template <typename DT>
__device__ __forceinline__ float round_to(float f) {
  return to_f32(DT{}, from_f32(DT{}, f));
}

// ------------------------------------------------------- total orders
// Orderable keys: unsigned comparison of the key equals numeric comparison of
// the value, with -0 < +0.  Used for order-independent min/max reductions.
__device__ __forceinline__ uint32_t order_key16(uint16_t h) {
  return (h & 0x8000u) ? static_cast<uint32_t>(static_cast<uint16_t>(~h)) : static_cast<uint32_t>(h | 0x8000u);
}
__device__ __forceinline__ uint16_t from_order_key16(uint32_t k) {
  return (k & 0x8000u) ? static_cast<uint16_t>(k & 0x7fffu) : static_cast<uint16_t>(~k);
}
__device__ __forceinline__ uint32_t order_key32(uint32_t u) {
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t from_order_key32(uint32_t k) {
  return (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
}

__device__ __forceinline__ bool is_nan(F16, uint16_t h) { return (h & 0x7fffu) > 0x7c00u; }
__device__ __forceinline__ bool is_nan(BF16, uint16_t h) { return (h & 0x7fffu) > 0x7f80u; }
__device__ __forceinline__ bool is_nan(F32, float f) { return (f32_as_u32(f) & 0x7fffffffu) > 0x7f800000u; }

__device__ __forceinline__ uint16_t canonical_nan(F16) { return 0x7e00u; }
__device__ __forceinline__ uint16_t canonical_nan(BF16) { return 0x7fc0u; }
__device__ __forceinline__ float canonical_nan(F32) { return u32_as_f32(0x7fc00000u); }

__device__ __forceinline__ uint32_t order_key(F16, uint16_t h) { return order_key16(h); }
__device__ __forceinline__ uint32_t order_key(BF16, uint16_t h) { return order_key16(h); }
__device__ __forceinline__ uint32_t order_key(F32, float f) { return order_key32(f32_as_u32(f)); }
__device__ __forceinline__ uint16_t from_order_key(F16, uint32_t k) { return from_order_key16(k); }
__device__ __forceinline__ uint16_t from_order_key(BF16, uint32_t k) { return from_order_key16(k); }
__device__ __forceinline__ float from_order_key(F32, uint32_t k) { return u32_as_f32(from_order_key32(k)); }

// Selection key for scores: NaN ranks above everything, -0 equals +0.
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = f32_as_u32(s);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  if (u == 0x80000000u) u = 0u;
  return order_key32(u);
}

// ------------------------------------------------------- wave helpers
__device__ __forceinline__ int lane_id() {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
}
__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return (l == 0) ? 0ull : (~0ull >> (64 - l));
}
__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Wavefront reductions and scans on DPP lane permutations (a VALU operand
// modifier, no LDS round trip): a butterfly inside each 16-lane row, then the
// four row results combined through readlane.  GFX9 DPP encodings.
constexpr int kDppQuadXor1 = 0xb1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowShr1 = 0x111;       // row_shr:n = 0x110 + n

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}
// Row shift with lanes that shift in from outside the row reading 0.
template <int N>
__device__ __forceinline__ uint32_t dpp_shr_zero(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kDppRowShr1 - 1 + N, 0xf, 0xf, true));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), lane));
}

template <typename Op>
__device__ __forceinline__ uint32_t wave_allreduce_u32(uint32_t v, Op op) {
  v = op(v, dpp_u32<kDppQuadXor1>(v));
  v = op(v, dpp_u32<kDppQuadXor2>(v));
  v = op(v, dpp_u32<kDppRowHalfMirror>(v));
  v = op(v, dpp_u32<kDppRowMirror>(v));
  return op(op(readlane_u32(v, 0), readlane_u32(v, 16)), op(readlane_u32(v, 32), readlane_u32(v, 48)));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_allreduce_u32(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return wave_allreduce_u32(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ int wave_sum_i32(int v) {
  return static_cast<int>(
      wave_allreduce_u32(static_cast<uint32_t>(v), [](uint32_t a, uint32_t b) { return a + b; }));
}
__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(wave_allreduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  return __uint_as_float(wave_allreduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}

// Inclusive prefix sum over lanes (wraps modulo 2^32).
__device__ __forceinline__ uint32_t wave_prefix_sum_u32(uint32_t v) {
  v += dpp_shr_zero<1>(v);
  v += dpp_shr_zero<2>(v);
  v += dpp_shr_zero<4>(v);
  v += dpp_shr_zero<8>(v);
  const uint32_t t0 = readlane_u32(v, 15), t1 = readlane_u32(v, 31), t2 = readlane_u32(v, 47);
  const int l = lane_id();
  return v + (l >= 16 ? t0 : 0u) + (l >= 32 ? t1 : 0u) + (l >= 48 ? t2 : 0u);
}
// Inclusive prefix sum of 64-bit values over lanes: the same DPP row scan on
// the two 32-bit halves with the carry of the low half, then the row totals.
__device__ __forceinline__ uint64_t wave_prefix_sum_u64(uint64_t v) {
  uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  auto step = [&](uint32_t slo, uint32_t shi) {
    const uint32_t n = lo + slo;
    hi += shi + (n < lo ? 1u : 0u);
    lo = n;
  };
  step(dpp_shr_zero<1>(lo), dpp_shr_zero<1>(hi));
  step(dpp_shr_zero<2>(lo), dpp_shr_zero<2>(hi));
  step(dpp_shr_zero<4>(lo), dpp_shr_zero<4>(hi));
  step(dpp_shr_zero<8>(lo), dpp_shr_zero<8>(hi));
  uint64_t r = (static_cast<uint64_t>(hi) << 32) | lo;
  const uint64_t t0 = (static_cast<uint64_t>(readlane_u32(hi, 15)) << 32) | readlane_u32(lo, 15);
  const uint64_t t1 = (static_cast<uint64_t>(readlane_u32(hi, 31)) << 32) | readlane_u32(lo, 31);
  const uint64_t t2 = (static_cast<uint64_t>(readlane_u32(hi, 47)) << 32) | readlane_u32(lo, 47);
  const int l = lane_id();
  r += (l >= 16 ? t0 : 0ull) + (l >= 32 ? t1 : 0ull) + (l >= 48 ? t2 : 0ull);
  return r;
}
__device__ __forceinline__ int wave_prefix_sum_i32(int v) {
  return static_cast<int>(wave_prefix_sum_u32(static_cast<uint32_t>(v)));
}
// Inclusive suffix sum over lanes: result in lane l is sum of v over lanes >= l.
__device__ __forceinline__ uint32_t wave_suffix_sum_u32(uint32_t v) {
  const uint32_t p = wave_prefix_sum_u32(v);
  return readlane_u32(p, 63) - p + v;
}

// Index of the lowest set lane in a non-empty ballot.
__device__ __forceinline__ int first_lane(uint64_t ballot) { return __ffsll(static_cast<long long>(ballot)) - 1; }

// ------------------------------------------------ cross-block handoff
// Data handed from one block to another inside a launch goes through
// device-coherent accesses: agent-scope relaxed atomic stores and loads,
// which gfx950 issues with the device-coherence bit (write-through past the
// XCD's non-coherent L2 on store, L2 bypass on load).  The "last block"
// pattern then needs no cache maintenance: every block waits until its own
// publishing stores have completed, bumps a per-group arrival counter, and
// the block that arrives last reads every block's data.  An agent-scope
// fence would instead write back and invalidate the whole L2 of the XCD,
// which costs microseconds per block.  No block ever waits on another, so
// there is no forward-progress assumption; the last block resets the
// counter so the next launch starts from zero (no memset node, so the
// sequence is graph-capture safe).
__device__ __forceinline__ void publish_f32(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_f32x2(float* p, float a, float b) {
  const uint64_t v = static_cast<uint64_t>(__float_as_uint(a)) | (static_cast<uint64_t>(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch_f32(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ float2 fetch_f32x2(const float* p) {
  const uint64_t v =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float(static_cast<uint32_t>(v)), __uint_as_float(static_cast<uint32_t>(v >> 32)));
}

// INT4 code of one value (twilight_offload_cache.py:32-35): round half to
// even of (f32(k) - f32(min)) / f32(scale), clamped to [0, 15]; NaN -> 0.
__device__ __forceinline__ uint32_t int4_code(float k, float mn, float sf) {
  float c = rintf((k - mn) / sf);
  c = c < 0.0f ? 0.0f : c;
  c = c > 15.0f ? 15.0f : c;
  return (c == c) ? static_cast<uint32_t>(c) : 0u;
}

// Per-row scale (twilight_offload_cache.py:31): the max - min difference is
// rounded to the key dtype, clamped below at 1e-9 in fp32 (NaN stays NaN),
// divided by 15 and rounded back to the key dtype.
template <typename DT>
__device__ __forceinline__ float int4_scale(float mnf, float mxf) {
  float diff = round_to<DT>(mxf - mnf);
  if (diff < 1e-9f) diff = 1e-9f;
  return diff / 15.0f;
}

// A 16-byte load with the streaming (nontemporal) hint, for data read once
// per step (projection weights, K/V rows): it is not kept in the caches,
// which lets a stream run closer to the HBM rate.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Returns true in every thread of the block that arrives last.  All of the
// block's published data must have been written with publish_* before the
// call.
__device__ __forceinline__ bool arrive_last(unsigned int* counter, unsigned int expected, int* s_flag) {
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's publishing stores are complete
  __syncthreads();                // ... and so are every other wavefront's
  if (threadIdx.x == 0) {
    const unsigned int prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = (prev + 1u == expected);
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last ? 1 : 0;
  }
  __syncthreads();
  return *s_flag != 0;
}

}  // namespace tw

// Host-side launch bookkeeping shared by the C-ABI entry points.
namespace tw_host {
int record_hip_error(hipError_t err);
int check_launch();
// True when p is device memory (HBM); false for pinned host memory mapped
// into the device's address space, or a pointer the runtime does not know.
bool device_memory(const void* p);
}  // namespace tw_host
