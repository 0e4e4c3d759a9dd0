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
// r = rsqrt(mean(h^2) + eps) in fp32.  One block per row; each thread holds
// up to kNormVec 8-element chunks of the row in registers (16-byte loads, all
// issued before any store), the row sum is a wave reduction then a sum over
// the block's waves.  H % 8 == 0, H <= kNormBlock * 8 * kNormVec.
constexpr int kNormVec = 4;

template <typename DT>
__global__ __launch_bounds__(kNormBlock) void add_rms_norm_kernel(typename DT::storage* __restrict__ h,
                                                                  const typename DT::storage* __restrict__ delta,
                                                                  const typename DT::storage* __restrict__ w,
                                                                  float eps, typename DT::storage* __restrict__ out,
                                                                  int H) {
  using S = typename DT::storage;
  __shared__ float s_part[kNormBlock / kWave];
  const int64_t row = blockIdx.x;
  uint4* hr = reinterpret_cast<uint4*>(h + row * H);
  const uint4* dr = delta != nullptr ? reinterpret_cast<const uint4*>(delta + row * H) : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* orow = reinterpret_cast<uint4*>(out + row * H);
  const int nv = H / 8;
  uint4 hv[kNormVec], dv[kNormVec], wv[kNormVec];
#pragma unroll
  for (int c = 0; c < kNormVec; ++c) {
    const int i = threadIdx.x + c * kNormBlock;
    const int j = i < nv ? i : 0;
    hv[c] = hr[j];
    dv[c] = dr != nullptr ? dr[j] : make_uint4(0u, 0u, 0u, 0u);
    wv[c] = wr[j];
  }
  float x[kNormVec][8];
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < kNormVec; ++c) {
    const uint32_t hw[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
    const uint32_t dw[4] = {dv[c].x, dv[c].y, dv[c].z, dv[c].w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = to_f32(DT{}, static_cast<S>(hw[e] & 0xffffu));
      float b = to_f32(DT{}, static_cast<S>(hw[e] >> 16));
      if (dr != nullptr) {
        a = round_to<DT>(a + to_f32(DT{}, static_cast<S>(dw[e] & 0xffffu)));
        b = round_to<DT>(b + to_f32(DT{}, static_cast<S>(dw[e] >> 16)));
      }
      x[c][2 * e] = a;
      x[c][2 * e + 1] = b;
      ow[e] = static_cast<uint32_t>(from_f32(DT{}, a)) | (static_cast<uint32_t>(from_f32(DT{}, b)) << 16);
    }
    const bool in = threadIdx.x + c * kNormBlock < nv;
    if (in) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += x[c][e] * x[c][e];
      if (dr != nullptr) hr[threadIdx.x + c * kNormBlock] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
  acc = wave_sum_f32(acc);
  if (lane_id() == 0) s_part[threadIdx.x / kWave] = acc;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormBlock / kWave; ++i) total += s_part[i];
  const float r = 1.0f / sqrtf(total / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < kNormVec; ++c) {
    if (threadIdx.x + c * kNormBlock >= nv) continue;
    const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ya = round_to<DT>(x[c][2 * e] * r);
      const float yb = round_to<DT>(x[c][2 * e + 1] * r);
      const float oa = to_f32(DT{}, static_cast<S>(ww[e] & 0xffffu)) * ya;
      const float ob = to_f32(DT{}, static_cast<S>(ww[e] >> 16)) * yb;
      ow[e] = static_cast<uint32_t>(from_f32(DT{}, oa)) | (static_cast<uint32_t>(from_f32(DT{}, ob)) << 16);
    }
    orow[threadIdx.x + c * kNormBlock] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
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

// y[n] = x . W[n, :] (+ bias[n]) for one row x [K] and W [N][K] row-major
// (nn.Linear's weight), the decode token's projections.  x is staged in LDS
// once per block; wave w of a block owns rows (block * 4 + w) * RPW ..; lane
// l reads the 16-byte chunks l, l + 64, ... of each of its rows, two chunks
// of every row in flight per step, and accumulates them with
// v_dot2_f32_{bf16,f16} in fp32; a wave reduction ends each row.
constexpr int kGemvBlock = 256;

template <typename DT>
struct Dot2;
template <>
struct Dot2<BF16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), acc, false);
  }
};
template <>
struct Dot2<F16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), acc, false);
  }
};

template <typename DT>
__device__ __forceinline__ float dot8(const uint4& w, const uint4& x, float acc) {
  acc = Dot2<DT>::dot(w.x, x.x, acc);
  acc = Dot2<DT>::dot(w.y, x.y, acc);
  acc = Dot2<DT>::dot(w.z, x.z, acc);
  return Dot2<DT>::dot(w.w, x.w, acc);
}

template <typename DT, int RPW>
__global__ __launch_bounds__(kGemvBlock) void gemv_kernel(const typename DT::storage* __restrict__ W,
                                                          const typename DT::storage* __restrict__ x,
                                                          const typename DT::storage* __restrict__ bias,
                                                          typename DT::storage* __restrict__ y, int N, int K) {
  extern __shared__ __align__(16) uint4 xs[];
  const int kc = K / 8;  // 16-byte chunks per row
  const uint4* x4 = reinterpret_cast<const uint4*>(x);
  for (int i = threadIdx.x; i < kc; i += kGemvBlock) xs[i] = x4[i];
  __syncthreads();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int n0 = (blockIdx.x * (kGemvBlock / kWave) + wave) * RPW;
  if (n0 >= N) return;
  const uint4* w4 = reinterpret_cast<const uint4*>(W);
  const uint4* rowp[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) rowp[r] = w4 + static_cast<int64_t>(n0 + r < N ? n0 + r : n0) * kc;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  int c = lane;
  for (; c + kWave < kc; c += 2 * kWave) {
    uint4 wa[RPW], wb[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      wa[r] = rowp[r][c];
      wb[r] = rowp[r][c + kWave];
    }
    const uint4 xa = xs[c];
    const uint4 xb = xs[c + kWave];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = dot8<DT>(wb[r], xb, dot8<DT>(wa[r], xa, acc[r]));
  }
  if (c < kc) {
    const uint4 xa = xs[c];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = dot8<DT>(rowp[r][c], xa, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float v = wave_sum_f32(acc[r]);
    if (lane == 0 && n0 + r < N) {
      const float b = bias != nullptr ? to_f32(DT{}, bias[n0 + r]) : 0.0f;
      y[n0 + r] = from_f32(DT{}, v + b);
    }
  }
}

}  // namespace
}  // namespace tw

extern "C" int tw_gemv(const void* W, const void* x, const void* bias, void* y, int N, int K, int dtype,
                       void* stream) {
  if (W == nullptr || x == nullptr || y == nullptr || N <= 0 || K <= 0 || (K % 8) != 0 || K > 32768)
    return TW_EINVAL;
  const uintptr_t align = 16;
  if ((reinterpret_cast<uintptr_t>(W) % align) || (reinterpret_cast<uintptr_t>(x) % align)) return TW_EINVAL;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t lds = static_cast<size_t>(K) * 2;
  const int waves = tw::kGemvBlock / tw::kWave;
  const bool wide = N >= 16384;
  const int rows_per_block = waves * (wide ? 4 : 2);
  const dim3 grid((N + rows_per_block - 1) / rows_per_block);
  if (dtype == TW_DTYPE_BF16) {
    if (wide)
      hipLaunchKernelGGL((tw::gemv_kernel<tw::BF16, 4>), grid, dim3(tw::kGemvBlock), lds, st,
                         static_cast<const uint16_t*>(W), static_cast<const uint16_t*>(x),
                         static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), N, K);
    else
      hipLaunchKernelGGL((tw::gemv_kernel<tw::BF16, 2>), grid, dim3(tw::kGemvBlock), lds, st,
                         static_cast<const uint16_t*>(W), static_cast<const uint16_t*>(x),
                         static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), N, K);
  } else if (dtype == TW_DTYPE_F16) {
    if (wide)
      hipLaunchKernelGGL((tw::gemv_kernel<tw::F16, 4>), grid, dim3(tw::kGemvBlock), lds, st,
                         static_cast<const uint16_t*>(W), static_cast<const uint16_t*>(x),
                         static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), N, K);
    else
      hipLaunchKernelGGL((tw::gemv_kernel<tw::F16, 2>), grid, dim3(tw::kGemvBlock), lds, st,
                         static_cast<const uint16_t*>(W), static_cast<const uint16_t*>(x),
                         static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), N, K);
  } else {
    return TW_EUNSUPPORTED;
  }
  return tw_host::check_launch();
}

extern "C" int tw_add_rms_norm(void* h, const void* delta, const void* weight, float eps, void* out, int rows, int H,
                               int dtype, void* stream) {
  if (h == nullptr || weight == nullptr || out == nullptr || rows <= 0 || H <= 0) return TW_EINVAL;
  if ((H % 8) != 0 || H > tw::kNormBlock * 8 * tw::kNormVec) return TW_EUNSUPPORTED;
  const uintptr_t align = 16;
  if ((reinterpret_cast<uintptr_t>(h) % align) || (reinterpret_cast<uintptr_t>(delta) % align) ||
      (reinterpret_cast<uintptr_t>(weight) % align) || (reinterpret_cast<uintptr_t>(out) % align))
    return TW_EINVAL;
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
