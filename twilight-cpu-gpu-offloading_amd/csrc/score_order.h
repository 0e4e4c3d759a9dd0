// The Quest score's per-channel operand: for query channel value q_d the
// page's max (q_d > 0) or min, widened exactly to fp32
// (quest_offload_cache.py:371-372, twilight_fused_quest.py:17-31).  Shared by
// the score kernels of quest.hip and the fused score + INT4 QK kernel of
// twilight.hip, so both form every product from the same operands.
#pragma once

#include "tw_common.h"

namespace tw {
namespace {

// x[i] = q[i] > 0 ? max[i] : min[i] for 8 consecutive channels of one page
// (16-byte aligned LDS rows).
__device__ __forceinline__ void select8(const uint8_t* mn, const uint8_t* mx, const float (&q)[8], float (&x)[8],
                                        F16) {
  const uint4 a = *reinterpret_cast<const uint4*>(mn);
  const uint4 b = *reinterpret_cast<const uint4*>(mx);
  const uint32_t lo[4] = {a.x, a.y, a.z, a.w}, hi[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = q[i] > 0.0f ? hi[i / 2] : lo[i / 2];
    x[i] = to_f32(F16{}, static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu)));
  }
}
__device__ __forceinline__ void select8(const uint8_t* mn, const uint8_t* mx, const float (&q)[8], float (&x)[8],
                                        BF16) {
  const uint4 a = *reinterpret_cast<const uint4*>(mn);
  const uint4 b = *reinterpret_cast<const uint4*>(mx);
  const uint32_t lo[4] = {a.x, a.y, a.z, a.w}, hi[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = q[i] > 0.0f ? hi[i / 2] : lo[i / 2];
    x[i] = to_f32(BF16{}, static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu)));
  }
}
__device__ __forceinline__ void select8(const uint8_t* mn, const uint8_t* mx, const float (&q)[8], float (&x)[8],
                                        F32) {
  float lo[8], hi[8];
  *reinterpret_cast<float4*>(lo) = reinterpret_cast<const float4*>(mn)[0];
  *reinterpret_cast<float4*>(lo + 4) = reinterpret_cast<const float4*>(mn)[1];
  *reinterpret_cast<float4*>(hi) = reinterpret_cast<const float4*>(mx)[0];
  *reinterpret_cast<float4*>(hi + 4) = reinterpret_cast<const float4*>(mx)[1];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = q[i] > 0.0f ? hi[i] : lo[i];
}

}  // namespace
}  // namespace tw
