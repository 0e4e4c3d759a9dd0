// Element-wise steps of one decode token around the sparse path, fused for
// the graph-captured decode step: residual add + RMSNorm, RoPE of q and k,
// and the SiLU gate of the MLP.  Each reproduces the rounding steps of the
// HF modules it stands for on 16-bit activations (LlamaRMSNorm,
// apply_rotary_pos_emb, LlamaMLP's act_fn(gate) * up): every element-wise
// torch op on bf16/fp16 computes in fp32 and rounds its result to the input
// dtype, and so do these kernels, op by op.
#pragma clang fp contract(off)

#include "tw_common.h"

namespace tw {
namespace {

constexpr int kNormBlock = 256;

// h = bf16(h + delta) (when delta is given); out = bf16(w * bf16(h * r)),
// r = rsqrt(mean(h^2) + eps) in fp32.  One block per row; the row sum is a
// wave DPP/shuffle reduction then a sum over the block's waves.
template <typename DT>
__global__ __launch_bounds__(kNormBlock) void add_rms_norm_kernel(typename DT::storage* __restrict__ h,
                                                                  const typename DT::storage* __restrict__ delta,
                                                                  const typename DT::storage* __restrict__ w,
                                                                  float eps, typename DT::storage* __restrict__ out,
                                                                  int H) {
  using S = typename DT::storage;
  __shared__ float s_part[kNormBlock / kWave];
  const int64_t row = blockIdx.x;
  S* hr = h + row * H;
  const S* dr = delta != nullptr ? delta + row * H : nullptr;
  S* orow = out + row * H;
  float acc = 0.0f;
  for (int i = threadIdx.x; i < H; i += kNormBlock) {
    float x = to_f32(DT{}, hr[i]);
    if (dr != nullptr) {
      x = round_to<DT>(x + to_f32(DT{}, dr[i]));
      hr[i] = from_f32(DT{}, x);
    }
    acc += x * x;
  }
  acc = wave_sum_f32(acc);
  if (lane_id() == 0) s_part[threadIdx.x / kWave] = acc;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormBlock / kWave; ++i) total += s_part[i];
  const float r = 1.0f / sqrtf(total / static_cast<float>(H) + eps);
  for (int i = threadIdx.x; i < H; i += kNormBlock) {
    const float x = to_f32(DT{}, hr[i]);
    const float y = round_to<DT>(x * r);
    orow[i] = from_f32(DT{}, to_f32(DT{}, w[i]) * y);
  }
}

// In place on q [Hq][D] and k [Hk][D] at the position *pos: x' = bf16(bf16(x
// cos) + bf16(rotate_half(x) sin)), rotate_half(x)[i] = -x[i + D/2] for i <
// D/2, x[i - D/2] after; cos/sin rows of the table [positions][D].  q' also
// goes to q32 in fp32 (the Quest score's query).
template <typename DT>
__global__ __launch_bounds__(256) void rope_qk_kernel(typename DT::storage* __restrict__ q,
                                                      typename DT::storage* __restrict__ k, int Hq, int Hk, int D,
                                                      const typename DT::storage* __restrict__ cos_t,
                                                      const typename DT::storage* __restrict__ sin_t,
                                                      const int64_t* __restrict__ pos, float* __restrict__ q32) {
  using S = typename DT::storage;
  const int64_t p = *pos;
  const S* c = cos_t + p * D;
  const S* s = sin_t + p * D;
  const int half = D / 2;
  const int n = (Hq + Hk) * half;  // one thread per (head, pair i, i + D/2)
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += gridDim.x * blockDim.x) {
    const int head = t / half;
    const int i = t - head * half;
    S* x = head < Hq ? q + static_cast<int64_t>(head) * D : k + static_cast<int64_t>(head - Hq) * D;
    const float a = to_f32(DT{}, x[i]);
    const float b = to_f32(DT{}, x[i + half]);
    const float ci = to_f32(DT{}, c[i]), si = to_f32(DT{}, s[i]);
    const float cj = to_f32(DT{}, c[i + half]), sj = to_f32(DT{}, s[i + half]);
    // rotate_half: element i gets -b (after the negation, exact), element i + D/2 gets a
    const float ya = round_to<DT>(round_to<DT>(a * ci) + round_to<DT>(-b * si));
    const float yb = round_to<DT>(round_to<DT>(b * cj) + round_to<DT>(a * sj));
    x[i] = from_f32(DT{}, ya);
    x[i + half] = from_f32(DT{}, yb);
    if (head < Hq && q32 != nullptr) {
      q32[static_cast<int64_t>(head) * D + i] = ya;
      q32[static_cast<int64_t>(head) * D + i + half] = yb;
    }
  }
}

// out[i] = bf16(bf16(silu(gate[i])) * up[i]), gate = gu[0..I), up = gu[I..2I).
template <typename DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const typename DT::storage* __restrict__ gu,
                                                       typename DT::storage* __restrict__ out, int I) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < I; i += gridDim.x * blockDim.x) {
    const float g = to_f32(DT{}, gu[i]);
    const float a = round_to<DT>(g / (1.0f + expf(-g)));
    out[i] = from_f32(DT{}, a * to_f32(DT{}, gu[I + i]));
  }
}

}  // namespace
}  // namespace tw

extern "C" int tw_add_rms_norm(void* h, const void* delta, const void* weight, float eps, void* out, int rows, int H,
                               int dtype, void* stream) {
  if (h == nullptr || weight == nullptr || out == nullptr || rows <= 0 || H <= 0) return TW_EINVAL;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == TW_DTYPE_BF16) {
    hipLaunchKernelGGL(tw::add_rms_norm_kernel<tw::BF16>, dim3(rows), dim3(tw::kNormBlock), 0, st,
                       static_cast<uint16_t*>(h), static_cast<const uint16_t*>(delta),
                       static_cast<const uint16_t*>(weight), eps, static_cast<uint16_t*>(out), H);
  } else if (dtype == TW_DTYPE_F16) {
    hipLaunchKernelGGL(tw::add_rms_norm_kernel<tw::F16>, dim3(rows), dim3(tw::kNormBlock), 0, st,
                       static_cast<uint16_t*>(h), static_cast<const uint16_t*>(delta),
                       static_cast<const uint16_t*>(weight), eps, static_cast<uint16_t*>(out), H);
  } else {
    return TW_EUNSUPPORTED;
  }
  return tw_host::check_launch();
}

extern "C" int tw_rope_qk(void* q, void* k, int Hq, int Hk, int D, const void* cos_table, const void* sin_table,
                          const int64_t* position, float* q32, int dtype, void* stream) {
  if (q == nullptr || k == nullptr || cos_table == nullptr || sin_table == nullptr || position == nullptr ||
      Hq <= 0 || Hk < 0 || D <= 0 || (D % 2) != 0)
    return TW_EINVAL;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int n = (Hq + Hk) * (D / 2);
  const int blocks = (n + 255) / 256;
  if (dtype == TW_DTYPE_BF16) {
    hipLaunchKernelGGL(tw::rope_qk_kernel<tw::BF16>, dim3(blocks), dim3(256), 0, st, static_cast<uint16_t*>(q),
                       static_cast<uint16_t*>(k), Hq, Hk, D, static_cast<const uint16_t*>(cos_table),
                       static_cast<const uint16_t*>(sin_table), position, q32);
  } else if (dtype == TW_DTYPE_F16) {
    hipLaunchKernelGGL(tw::rope_qk_kernel<tw::F16>, dim3(blocks), dim3(256), 0, st, static_cast<uint16_t*>(q),
                       static_cast<uint16_t*>(k), Hq, Hk, D, static_cast<const uint16_t*>(cos_table),
                       static_cast<const uint16_t*>(sin_table), position, q32);
  } else {
    return TW_EUNSUPPORTED;
  }
  return tw_host::check_launch();
}

extern "C" int tw_silu_mul(const void* gate_up, void* out, int I, int dtype, void* stream) {
  if (gate_up == nullptr || out == nullptr || I <= 0) return TW_EINVAL;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int blocks = (I + 255) / 256;
  blocks = blocks > 1024 ? 1024 : blocks;
  if (dtype == TW_DTYPE_BF16) {
    hipLaunchKernelGGL(tw::silu_mul_kernel<tw::BF16>, dim3(blocks), dim3(256), 0, st,
                       static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), I);
  } else if (dtype == TW_DTYPE_F16) {
    hipLaunchKernelGGL(tw::silu_mul_kernel<tw::F16>, dim3(blocks), dim3(256), 0, st,
                       static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), I);
  } else {
    return TW_EUNSUPPORTED;
  }
  return tw_host::check_launch();
}
