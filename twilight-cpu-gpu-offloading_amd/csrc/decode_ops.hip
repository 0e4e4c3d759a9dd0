// Element-wise steps of one decode token around the sparse path, fused for
// the graph-captured decode step: residual add + RMSNorm, RoPE of q and k,
// and the SiLU gate of the MLP, standalone or fused into the one-token GEMV
// that consumes or produces them.  Each reproduces the rounding steps of the
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

// The residual add + RMSNorm of one row by a block of kNormBlock threads,
// in two calls so that other loads can be issued between them: load() reads
// the thread's chunks of h, delta and w; finish() stores a = bf16(h + delta)
// (a = h without delta) to h_store (nullable) and passes the 16-byte chunk i
// of bf16(w * bf16(a * r)) to put(i, chunk).  Thread t owns chunks t + c *
// kNormBlock, c < NV; the sum of squares runs over its chunks in order, then
// a wave reduction, then the waves in order, so every block computing the
// same row gets the same bits, whatever NV covers the row.  In a block of
// more than kNormBlock threads the first kNormBlock do the work and the rest
// only meet the barrier in finish().
template <typename DT, int NV>
struct NormRow {
  using S = typename DT::storage;
  uint4 hv[NV], dv[NV], wv[NV];
  bool has_delta;

  __device__ __forceinline__ void load(const S* __restrict__ h, const S* __restrict__ delta,
                                       const S* __restrict__ w, int H) {
    const uint4* hr = reinterpret_cast<const uint4*>(h);
    const uint4* dr = reinterpret_cast<const uint4*>(delta);
    const uint4* wr = reinterpret_cast<const uint4*>(w);
    const int nv = H / 8;
    has_delta = dr != nullptr;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      // (a thread past kNormBlock, in a larger block, reads chunk 0 and adds nothing)
      const int i = threadIdx.x < kNormBlock ? static_cast<int>(threadIdx.x) + c * kNormBlock : nv;
      const int j = i < nv ? i : 0;
      hv[c] = hr[j];
      dv[c] = dr != nullptr ? dr[j] : make_uint4(0u, 0u, 0u, 0u);
      wv[c] = wr[j];
    }
  }

  template <typename Put>
  __device__ __forceinline__ void finish(float eps, int H, S* h_store, float* s_part, Put put) {
    uint4* hs = reinterpret_cast<uint4*>(h_store);
    const int nv = H / 8;
    float x[NV][8];
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const uint32_t hw[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
      const uint32_t dw[4] = {dv[c].x, dv[c].y, dv[c].z, dv[c].w};
      uint32_t ow[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = to_f32(DT{}, static_cast<S>(hw[e] & 0xffffu));
        float b = to_f32(DT{}, static_cast<S>(hw[e] >> 16));
        if (has_delta) {
          a = round_to<DT>(a + to_f32(DT{}, static_cast<S>(dw[e] & 0xffffu)));
          b = round_to<DT>(b + to_f32(DT{}, static_cast<S>(dw[e] >> 16)));
        }
        x[c][2 * e] = a;
        x[c][2 * e + 1] = b;
        ow[e] = static_cast<uint32_t>(from_f32(DT{}, a)) | (static_cast<uint32_t>(from_f32(DT{}, b)) << 16);
      }
      const bool in = threadIdx.x < kNormBlock && threadIdx.x + c * kNormBlock < nv;
      if (in) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += x[c][e] * x[c][e];
        if (hs != nullptr) hs[threadIdx.x + c * kNormBlock] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
    }
    acc = wave_sum_f32(acc);
    if (lane_id() == 0 && threadIdx.x < kNormBlock) s_part[threadIdx.x / kWave] = acc;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormBlock / kWave; ++i) total += s_part[i];
    const float r = 1.0f / sqrtf(total / static_cast<float>(H) + eps);
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      if (threadIdx.x >= kNormBlock || threadIdx.x + c * kNormBlock >= nv) continue;
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
      put(threadIdx.x + c * kNormBlock, make_uint4(ow[0], ow[1], ow[2], ow[3]));
    }
  }
};

// h = bf16(h + delta) (when delta is given); out = bf16(w * bf16(h * r)),
// r = rsqrt(mean(h^2) + eps) in fp32.  One block per row; each thread holds
// up to kNormVec 8-element chunks of the row in registers (16-byte loads, all
// issued before any store).  H % 8 == 0, H <= kNormBlock * 8 * kNormVec.
template <typename DT>
__global__ __launch_bounds__(kNormBlock) void add_rms_norm_kernel(typename DT::storage* __restrict__ h,
                                                                  const typename DT::storage* __restrict__ delta,
                                                                  const typename DT::storage* __restrict__ w,
                                                                  float eps, typename DT::storage* __restrict__ out,
                                                                  int H) {
  __shared__ float s_part[kNormBlock / kWave];
  const int64_t row = blockIdx.x;
  uint4* orow = reinterpret_cast<uint4*>(out + row * H);
  NormRow<DT, kNormVec> nr;
  nr.load(h + row * H, delta != nullptr ? delta + row * H : nullptr, w, H);
  nr.finish(eps, H, delta != nullptr ? h + row * H : nullptr, s_part, [&](int i, const uint4& v) { orow[i] = v; });
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
// once per block; wave w of a block owns RPW rows; lane l reads the 16-byte
// chunks l, l + 64, ... of each of its rows, 16 / RPW chunks of every row (8
// with one row) in flight per step, and accumulates them in increasing order
// with v_dot2_f32_{bf16,f16} in fp32; a wave reduction ends each row.  The
// sums do not depend on RPW.
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

// Prologue: x given, or x = RMSNorm(h_in + delta) computed by every block
// (block 0 stores h_in + delta to h_out).  Epilogue: y[n] = bf16(x . W[n] +
// bias[n]); or RoPE pairs -- rows (head * D + i, head * D + i + D/2) of a
// concatenated q/k/v projection, rotated as tw_rope_qk for the q and k heads
// (q also to q32); or SiLU pairs -- rows (i, I + i) of a concatenated
// gate/up projection, y[i] = bf16(bf16(silu(gate)) * up).  With one row a
// wave, the two rows of a pair belong to waves 2j and 2j + 1 of a block and
// meet in LDS.
constexpr int kProX = 0, kProNorm = 1;
constexpr int kEpiPlain = 0, kEpiRope = 1, kEpiSilu = 2;

template <typename S>
struct GemvArgs {
  const S* W;
  const S* bias;
  int N, K;
  const S* x;          // kProX
  const S* h_in;       // kProNorm
  const S* delta;
  const S* norm_w;
  float eps;
  S* h_out;
  S* y;
  int Hq, Hk, D;       // kEpiRope
  const S* cos_t;
  const S* sin_t;
  const int64_t* pos;
  float* q32;
};

// NV: 16-byte chunks of x per thread held in registers while the first
// weight loads are issued (x of up to NV * 2048 elements; longer x is staged
// after them).
template <typename DT, int RPW, int PRO, int EPI, int NV, int NTB>
__global__ __launch_bounds__(NTB) void gemv_kernel(GemvArgs<typename DT::storage> a) {
  constexpr int kW = NTB / kWave;
  static_assert(NTB % kNormBlock == 0, "the norm runs in the first kNormBlock threads");
  constexpr bool kWavePairs = EPI != kEpiPlain && RPW == 1;  // a pair's rows in two waves
  static_assert(EPI == kEpiPlain || RPW % 2 == 0 || RPW == 1, "paired epilogues: rows two by two, or wave pairs");
  extern __shared__ __align__(16) uint4 xs[];
  __shared__ float s_part[kW];
  __shared__ float s_pair[kW];
  const int K = a.K;
  const int kc = K / 8;  // 16-byte chunks per row
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  // units: rows (plain) or row pairs; this wave's first unit
  const int units = EPI == kEpiPlain ? a.N : a.N / 2;
  const int unit0 = kWavePairs ? blockIdx.x * (kW / 2) + wave / 2
                               : (blockIdx.x * kW + wave) * (EPI == kEpiPlain ? RPW : RPW / 2);
  // the wave's rows
  int rows[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    if (EPI == kEpiPlain) {
      const int n = unit0 + r;
      rows[r] = n < a.N ? n : a.N - 1;
    } else {
      int p = kWavePairs ? unit0 : unit0 + r / 2;
      p = p < units ? p : units - 1;
      int na, nb;
      if (EPI == kEpiRope) {
        const int half = a.D / 2;
        const int head = p / half;
        na = head * a.D + (p - head * half);
        nb = na + half;
      } else {
        na = p;
        nb = p + units;
      }
      rows[r] = ((kWavePairs ? wave : r) & 1) ? nb : na;
    }
  }
  const uint4* w4 = reinterpret_cast<const uint4*>(a.W);
  const uint4* rowp[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) rowp[r] = w4 + static_cast<int64_t>(rows[r]) * kc;
  // A step covers chunks c + u * kWave, u < U, of every row: U * RPW
  // 16-byte loads per lane are in flight before any is used; the first
  // step's are issued right after x's (or the norm's inputs'), so x is ready
  // while they arrive.  Chunks past the row read its last chunk again (a
  // line the step already reads).
  constexpr int U = RPW == 1 ? 8 : 16 / RPW;
  int c = lane;
  uint4 wv[U][RPW];
  auto load_step = [&](int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = c0 + u * kWave;
#pragma unroll
      for (int r = 0; r < RPW; ++r) wv[u][r] = load_stream(rowp[r] + (idx < kc ? idx : kc - 1));
    }
  };
  NormRow<DT, NV> nr;
  uint4 xr[NV];
  const uint4* x4 = reinterpret_cast<const uint4*>(a.x);
  if constexpr (PRO == kProNorm) {
    nr.load(a.h_in, a.delta, a.norm_w, K);
  } else {
    // the thread's first NV chunks of x, unconditionally (clamped indices):
    // loaded under a condition the array went to scratch memory, and its
    // store there waited for the loads before the weights' were issued
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = static_cast<int>(threadIdx.x) + v * NTB;
      xr[v] = x4[i < kc ? i : 0];
    }
  }
  load_step(c);
  if (PRO == kProNorm) {
    nr.finish(a.eps, K, (blockIdx.x == 0 && a.delta != nullptr) ? a.h_out : nullptr, s_part,
              [&](int i, const uint4& v) { xs[i] = v; });
  } else {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = static_cast<int>(threadIdx.x) + v * NTB;
      if (i < kc) xs[i] = xr[v];
    }
    // x longer than NV chunks a thread: the rest after the weights' loads
    for (int i = static_cast<int>(threadIdx.x) + NV * NTB; i < kc; i += NTB) xs[i] = x4[i];
  }
  __syncthreads();
  // (wave pairs meet at a barrier below: every wave goes on)
  if (!kWavePairs && unit0 >= units) return;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  while (true) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = c + u * kWave;
      if (idx < kc) {
        const uint4 xv = xs[idx];
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = dot8<DT>(wv[u][r], xv, acc[r]);
      }
    }
    c += U * kWave;
    if (c >= kc) break;
    load_step(c);
  }
  float v[RPW > 1 ? RPW : 2];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    v[r] = wave_sum_f32(acc[r]);
    v[r] = v[r] + (a.bias != nullptr ? to_f32(DT{}, a.bias[rows[r]]) : 0.0f);
  }
  if (kWavePairs) {
    // the odd wave of a pair hands its row to the even one
    if (lane == 0) s_pair[wave] = v[0];
    __syncthreads();
    if ((wave & 1) != 0 || unit0 >= units) return;
    v[1] = s_pair[wave + 1];
  }
  if (lane != 0) return;
  if (EPI == kEpiPlain) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      if (unit0 + r < a.N) a.y[unit0 + r] = from_f32(DT{}, v[r]);
  } else {
    constexpr int kPairs = kWavePairs ? 1 : RPW / 2;
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
      const int p = unit0 + q;
      if (p >= units) continue;
      const float va = round_to<DT>(v[2 * q]);
      const float vb = round_to<DT>(v[2 * q + 1]);
      if (EPI == kEpiSilu) {
        const float g = round_to<DT>(va / (1.0f + expf(-va)));
        a.y[p] = from_f32(DT{}, g * vb);
      } else {
        const int half = a.D / 2;
        const int head = p / half;
        const int i = p - head * half;
        const int na = head * a.D + i, nb = na + half;
        float ya = va, yb = vb;
        if (head < a.Hq + a.Hk) {
          const int64_t t = *a.pos * a.D;
          const float ci = to_f32(DT{}, a.cos_t[t + i]), si = to_f32(DT{}, a.sin_t[t + i]);
          const float cj = to_f32(DT{}, a.cos_t[t + i + half]), sj = to_f32(DT{}, a.sin_t[t + i + half]);
          ya = round_to<DT>(round_to<DT>(va * ci) + round_to<DT>(-vb * si));
          yb = round_to<DT>(round_to<DT>(vb * cj) + round_to<DT>(va * sj));
          if (head < a.Hq && a.q32 != nullptr) {
            a.q32[static_cast<int64_t>(head) * a.D + i] = ya;
            a.q32[static_cast<int64_t>(head) * a.D + i + half] = yb;
          }
        }
        a.y[na] = from_f32(DT{}, ya);
        a.y[nb] = from_f32(DT{}, yb);
      }
    }
  }
}

template <typename DT, int PRO, int EPI, int NV>
void launch_gemv_nv(const GemvArgs<typename DT::storage>& a, hipStream_t st) {
  const size_t lds = static_cast<size_t>(a.K) * 2;
  const int waves = kGemvBlock / kWave;
  // a given x: one row a wave.  A norm prologue: every block normalises x
  // itself, and that work grows with the block count, so those blocks hold
  // two rows a wave (four from 16384 rows); measured on the decode shapes.
  const int rpw = PRO != kProNorm ? 1 : (a.N >= 16384 ? 4 : 2);
  const int units_per_block = EPI == kEpiPlain ? waves * rpw : (rpw == 1 ? waves / 2 : waves * rpw / 2);
  const int units = EPI == kEpiPlain ? a.N : a.N / 2;
  const dim3 grid((units + units_per_block - 1) / units_per_block);
  if constexpr (PRO != kProNorm) {
    hipLaunchKernelGGL((gemv_kernel<DT, 1, PRO, EPI, NV, kGemvBlock>), grid, dim3(kGemvBlock), lds, st, a);
  } else {
    if (rpw == 2)
      hipLaunchKernelGGL((gemv_kernel<DT, 2, PRO, EPI, NV, kGemvBlock>), grid, dim3(kGemvBlock), lds, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<DT, 4, PRO, EPI, NV, kGemvBlock>), grid, dim3(kGemvBlock), lds, st, a);
  }
}

// x of up to 4096 elements in two register chunks per thread, else four
// (the norm prologue takes K <= 8192), else for a given x eight (16384
// elements); a given x longer than that is staged past the register chunks
// after the first weight loads.
template <typename DT, int PRO, int EPI>
int launch_gemv(const GemvArgs<typename DT::storage>& a, hipStream_t st) {
  if (a.K <= 2 * 8 * kGemvBlock)
    launch_gemv_nv<DT, PRO, EPI, 2>(a, st);
  else if (PRO == kProNorm || a.K <= 4 * 8 * kGemvBlock)
    launch_gemv_nv<DT, PRO, EPI, 4>(a, st);
  else if constexpr (PRO != kProNorm)
    launch_gemv_nv<DT, PRO, EPI, 8>(a, st);
  return tw_host::check_launch();
}

template <int PRO, int EPI>
int launch_gemv_dtype(GemvArgs<uint16_t> a, int dtype, hipStream_t st) {
  if (dtype == TW_DTYPE_BF16) return launch_gemv<BF16, PRO, EPI>(a, st);
  if (dtype == TW_DTYPE_F16) return launch_gemv<F16, PRO, EPI>(a, st);
  return TW_EUNSUPPORTED;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) != 0; }

// Shared checks of the norm-prologue entry points.
int check_norm_gemv(const void* h_in, const void* delta, const void* norm_w, const void* h_out, const void* W,
                    const void* y, int N, int K) {
  if (h_in == nullptr || norm_w == nullptr || W == nullptr || y == nullptr || N <= 0 || K <= 0)
    return TW_EINVAL;
  if (delta != nullptr && (h_out == nullptr || h_out == h_in || h_out == delta)) return TW_EINVAL;
  if ((K % 8) != 0 || K > kNormBlock * 8 * kNormVec) return TW_EUNSUPPORTED;
  if (misaligned(h_in) || misaligned(delta) || misaligned(norm_w) || misaligned(h_out) || misaligned(W))
    return TW_EINVAL;
  return TW_OK;
}

}  // namespace
}  // namespace tw

extern "C" int tw_gemv(const void* W, const void* x, const void* bias, void* y, int N, int K, int dtype,
                       void* stream) {
  if (W == nullptr || x == nullptr || y == nullptr || N <= 0 || K <= 0 || (K % 8) != 0 || K > 32768)
    return TW_EINVAL;
  if (tw::misaligned(W) || tw::misaligned(x)) return TW_EINVAL;
  tw::GemvArgs<uint16_t> a{};
  a.W = static_cast<const uint16_t*>(W);
  a.bias = static_cast<const uint16_t*>(bias);
  a.N = N;
  a.K = K;
  a.x = static_cast<const uint16_t*>(x);
  a.y = static_cast<uint16_t*>(y);
  return tw::launch_gemv_dtype<tw::kProX, tw::kEpiPlain>(a, dtype, static_cast<hipStream_t>(stream));
}

namespace {
tw::GemvArgs<uint16_t> norm_gemv_args(const void* h_in, const void* delta, const void* norm_w, float eps,
                                      void* h_out, const void* W, const void* bias, void* y, int N, int K) {
  tw::GemvArgs<uint16_t> a{};
  a.W = static_cast<const uint16_t*>(W);
  a.bias = static_cast<const uint16_t*>(bias);
  a.N = N;
  a.K = K;
  a.h_in = static_cast<const uint16_t*>(h_in);
  a.delta = static_cast<const uint16_t*>(delta);
  a.norm_w = static_cast<const uint16_t*>(norm_w);
  a.eps = eps;
  a.h_out = static_cast<uint16_t*>(h_out);
  a.y = static_cast<uint16_t*>(y);
  return a;
}
}  // namespace

extern "C" int tw_rms_norm_gemv(const void* h_in, const void* delta, const void* norm_weight, float eps, void* h_out,
                                const void* W, const void* bias, void* y, int N, int K, int dtype, void* stream) {
  const int rc = tw::check_norm_gemv(h_in, delta, norm_weight, h_out, W, y, N, K);
  if (rc != TW_OK) return rc;
  return tw::launch_gemv_dtype<tw::kProNorm, tw::kEpiPlain>(
      norm_gemv_args(h_in, delta, norm_weight, eps, h_out, W, bias, y, N, K), dtype, static_cast<hipStream_t>(stream));
}

extern "C" int tw_rms_norm_gemv_rope(const void* h_in, const void* delta, const void* norm_weight, float eps,
                                     void* h_out, const void* W, const void* bias, void* y, int N, int K, int Hq,
                                     int Hk, int D, const void* cos_table, const void* sin_table,
                                     const int64_t* position, float* q32, int dtype, void* stream) {
  const int rc = tw::check_norm_gemv(h_in, delta, norm_weight, h_out, W, y, N, K);
  if (rc != TW_OK) return rc;
  if (Hq <= 0 || Hk < 0 || D <= 0 || (D % 2) != 0 || (N % D) != 0 || N / D < Hq + Hk || cos_table == nullptr ||
      sin_table == nullptr || position == nullptr)
    return TW_EINVAL;
  tw::GemvArgs<uint16_t> a = norm_gemv_args(h_in, delta, norm_weight, eps, h_out, W, bias, y, N, K);
  a.Hq = Hq;
  a.Hk = Hk;
  a.D = D;
  a.cos_t = static_cast<const uint16_t*>(cos_table);
  a.sin_t = static_cast<const uint16_t*>(sin_table);
  a.pos = position;
  a.q32 = q32;
  return tw::launch_gemv_dtype<tw::kProNorm, tw::kEpiRope>(a, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int tw_rms_norm_gemv_silu(const void* h_in, const void* delta, const void* norm_weight, float eps,
                                     void* h_out, const void* W, const void* bias, void* y, int N, int K, int dtype,
                                     void* stream) {
  const int rc = tw::check_norm_gemv(h_in, delta, norm_weight, h_out, W, y, N, K);
  if (rc != TW_OK) return rc;
  if ((N % 2) != 0) return TW_EINVAL;
  return tw::launch_gemv_dtype<tw::kProNorm, tw::kEpiSilu>(
      norm_gemv_args(h_in, delta, norm_weight, eps, h_out, W, bias, y, N, K), dtype, static_cast<hipStream_t>(stream));
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
