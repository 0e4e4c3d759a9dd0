// Sparse GQA decode attention over selected rows, split-K with a fused
// last-block combine.
//
// Reference call surface: _flash_attention_varlen_forward (mp.py:21-52) as
// used by the GQA-group decode branch (mp.py:239-279: G sequences of one
// query token x R heads against one KV head), the layer-flat branch
// (mp.py:283-321) and the per-head reference path (mp.py:424-452).  The
// reference semantics are softmax(q.k * scale) v over every key of the
// sequence (causal with q_len 1 sees all keys), fp32 accumulation, output in
// the input dtype.
//
// Work split: block = (group g, chunk of rows).  Inside a block each of the 4
// wavefronts takes 32 rows per iteration as 8 steps of 4 rows: LPR = D/8 lanes
// share a row and each lane owns 8 consecutive channels, so a K or V row is a
// 16-byte-per-lane coalesced load and the rows are read straight from the KV
// cache by index (no gathered copy).  The R query heads of the group share
// every K/V load.  Scores are reduced across the LPR lanes of a row with xor
// shuffles; each wavefront keeps an online (max, sum, acc) per head; the four
// wavefront partials are merged in LDS into one block partial; the last
// block of the group (arrival counter, no waiting) merges all block partials
// and writes the output.
#pragma clang fp contract(off)

#include "tw_common.h"

namespace tw {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  int G, R, D;
  const int32_t* rows;
  const uint8_t* masks;
  const int32_t* counts;
  int64_t rows_stride;
  int64_t entry_stride;
  const int32_t* cu_k;
  int Hk;
  int window_left;
  const void* cur_k;
  const void* cur_v;
  float scale_log2;
  void* out;
  float* partials;          // [G][max_chunks][R][2 + D]
  unsigned int* counters;   // [G]
  int max_chunks;
  int iters;                // row iterations per block
  int max_rows;             // bound on every group's row count
};

template <typename S, int CPL>
struct Chunk;
template <>
struct Chunk<uint16_t, 8> {
  uint4 w;
  __device__ __forceinline__ void load(const uint16_t* p) { w = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void zero() { w = make_uint4(0u, 0u, 0u, 0u); }
  template <typename DT>
  __device__ __forceinline__ void to_float(float (&f)[8]) const {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = to_f32(DT{}, static_cast<uint16_t>(a[i] & 0xffffu));
      f[2 * i + 1] = to_f32(DT{}, static_cast<uint16_t>(a[i] >> 16));
    }
  }
};
template <>
struct Chunk<float, 8> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void zero() {
    a = make_float4(0.f, 0.f, 0.f, 0.f);
    b = a;
  }
  template <typename DT>
  __device__ __forceinline__ void to_float(float (&f)[8]) const {
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

// Generic chunk for runtime D (one row per wavefront instruction, lane owns
// channels 8*lane .. 8*lane+7, masked against D).
template <typename S>
struct GenericChunk {
  S e[8];
  __device__ __forceinline__ void load(const S* p, int c0, int D) {
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (c0 + i < D) ? p[i] : S(0);
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = S(0);
  }
  template <typename DT>
  __device__ __forceinline__ void to_float(float (&f)[8]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = to_f32(DT{}, e[i]);
  }
};

template <typename DT, int DFIX, int RMAX, bool INDEXED>
__global__ __launch_bounds__(kBlock) void decode_attn_kernel(AttnArgs a) {
  using S = typename DT::storage;
  constexpr bool kGeneric = (DFIX == 0);
  constexpr int CPL = 8;
  constexpr int LPR = kGeneric ? 64 : DFIX / CPL;   // lanes per row
  constexpr int RPI = kWave / LPR;                   // rows per instruction
  constexpr int NSTEP = (sizeof(S) == 2) ? 8 : 4;    // instructions per iteration
  constexpr int RW = NSTEP * RPI;                    // rows per wavefront iteration
  using ChunkT = typename std::conditional<kGeneric, GenericChunk<S>, Chunk<S, CPL>>::type;

  const int D = kGeneric ? a.D : DFIX;
  const int R = a.R;
  const int g = blockIdx.x / a.max_chunks;
  const int chunk = blockIdx.x - g * a.max_chunks;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int rig = lane / LPR;            // row in instruction
  const int c0 = (lane % LPR) * CPL;     // first channel of this lane

  // ---- rows of this group ----
  int n_list;
  int64_t seg_base = 0;   // row offset of the group's first row
  int64_t row_stride = D; // elements between consecutive rows
  int64_t head_off = 0;
  int win_start = 0;
  if (INDEXED) {
    n_list = a.counts[g];
    n_list = n_list < 0 ? 0 : (n_list > a.max_rows ? a.max_rows : n_list);
    seg_base = static_cast<int64_t>(g) * a.entry_stride;
  } else {
    const int b = g / a.Hk;
    const int h = g - b * a.Hk;
    const int s0 = a.cu_k[b];
    int n = a.cu_k[b + 1] - s0;
    if (a.window_left >= 0 && n > a.window_left + 1) {
      win_start = n - (a.window_left + 1);
      n = a.window_left + 1;
    }
    n_list = n < 0 ? 0 : (n > a.max_rows ? a.max_rows : n);
    seg_base = s0;
    row_stride = static_cast<int64_t>(a.Hk) * D;
    head_off = static_cast<int64_t>(h) * D;
  }
  const bool has_cur = a.cur_k != nullptr;
  const int n_rows = n_list + (has_cur ? 1 : 0);
  const int rows_per_block = kWaves * RW * a.iters;
  const int n_chunks = (n_rows + rows_per_block - 1) / rows_per_block;

  __shared__ int s_flag;
  __shared__ float s_m[kWaves][RMAX];
  __shared__ float s_l[kWaves][RMAX];
  extern __shared__ __align__(16) float s_o[];  // [kWaves][RMAX][D]

  if (n_rows == 0) {
    // No keys at all: the output is defined as zeros (block 0 writes it).
    if (chunk == 0) {
      S* o = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
      for (int i = threadIdx.x; i < R * D; i += kBlock) o[i] = from_f32(DT{}, 0.0f);
    }
    return;
  }
  if (chunk >= n_chunks) return;

  // ---- query registers: q[r][c0 .. c0+8) * scale * log2(e) ----
  float qv[RMAX][CPL];
  {
    const S* qg = static_cast<const S*>(a.q) + static_cast<int64_t>(g) * R * D;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = c0 + i;
        qv[r][i] = (r < R && c < D) ? to_f32(DT{}, qg[static_cast<int64_t>(r) * D + c]) * a.scale_log2 : 0.0f;
      }
    }
  }

  float m_run[RMAX], l_run[RMAX], o_acc[RMAX][CPL];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) o_acc[r][i] = 0.0f;
  }

  const S* kbase = static_cast<const S*>(a.k);
  const S* vbase = static_cast<const S*>(a.v);
  const S* ck = has_cur ? static_cast<const S*>(a.cur_k) + static_cast<int64_t>(g) * D : nullptr;
  const S* cv = has_cur ? static_cast<const S*>(a.cur_v) + static_cast<int64_t>(g) * D : nullptr;

  const int block_row0 = chunk * rows_per_block;
  for (int it = 0; it < a.iters; ++it) {
    const int wave_row0 = block_row0 + (it * kWaves + wave) * RW;
    if (wave_row0 >= n_rows) break;
    ChunkT kc[NSTEP], vc[NSTEP];
    uint8_t hm[NSTEP];
    bool valid[NSTEP];
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      const int i = wave_row0 + s * RPI + rig;
      valid[s] = i < n_rows;
      hm[s] = 0xffu;
      const S* kp;
      const S* vp;
      if (!valid[s]) {
        kp = nullptr;
        vp = nullptr;
      } else if (i >= n_list) {
        kp = ck;
        vp = cv;
      } else {
        int64_t pos;
        if (INDEXED) {
          pos = a.rows[static_cast<int64_t>(g) * a.rows_stride + i];
          if (a.masks != nullptr) hm[s] = a.masks[static_cast<int64_t>(g) * a.rows_stride + i];
          // A position outside the entry is never read (row dropped).
          if (pos < 0 || pos >= a.entry_stride) {
            valid[s] = false;
            pos = 0;
          }
        } else {
          pos = win_start + i;
        }
        const int64_t off = (seg_base + pos) * row_stride + head_off;
        kp = valid[s] ? kbase + off : nullptr;
        vp = valid[s] ? vbase + off : nullptr;
      }
      if (valid[s]) {
        if constexpr (kGeneric) {
          kc[s].load(kp + c0, c0, D);
          vc[s].load(vp + c0, c0, D);
        } else {
          kc[s].load(kp + c0);
          vc[s].load(vp + c0);
        }
      } else {
        kc[s].zero();
        vc[s].zero();
      }
    }
    // scores (already in log2 units)
    float sc[NSTEP][RMAX];
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      float kf[CPL];
      kc[s].template to_float<DT>(kf);
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc = __builtin_fmaf(qv[r][i], kf[i], acc);
        sc[s][r] = acc;
      }
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) {
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) sc[s][r] += __shfl_xor(sc[s][r], o);
      }
    }
    // mask, running max
    float mnew[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
        const bool vis = valid[s] && r < R && ((hm[s] >> r) & 1u);
        sc[s][r] = vis ? sc[s][r] : -INFINITY;
        mx = fmaxf(mx, sc[s][r]);
      }
#pragma unroll
      for (int o = LPR; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      mnew[r] = fmaxf(m_run[r], mx);
    }
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      const float alpha = (mnew[r] == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[r] - mnew[r]);
      m_run[r] = mnew[r];
      l_run[r] *= alpha;
#pragma unroll
      for (int i = 0; i < CPL; ++i) o_acc[r][i] *= alpha;
    }
    float lsum[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) lsum[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      float vf[CPL];
      vc[s].template to_float<DT>(vf);
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        const float p = (sc[s][r] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[s][r] - m_run[r]);
        lsum[r] += p;
#pragma unroll
        for (int i = 0; i < CPL; ++i) o_acc[r][i] = __builtin_fmaf(p, vf[i], o_acc[r][i]);
      }
    }
#pragma unroll
    for (int r = 0; r < RMAX; ++r) l_run[r] += lsum[r];
  }
  // Merge the row groups of the wavefront (same channels, different rows).
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1) {
      l_run[r] += __shfl_xor(l_run[r], o);
#pragma unroll
      for (int i = 0; i < CPL; ++i) o_acc[r][i] += __shfl_xor(o_acc[r][i], o);
    }
  }
  if (lane < LPR) {
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      if (r < R) {
        if (lane == 0) {
          s_m[wave][r] = m_run[r];
          s_l[wave][r] = l_run[r];
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const int c = c0 + i;
          if (c < D) s_o[(wave * RMAX + r) * D + c] = o_acc[r][i];
        }
      }
    }
  }
  __syncthreads();
  // Block partial: merge the wavefront partials (waves with no rows hold
  // m = -inf, l = 0, acc = 0).
  float* part = a.partials + (static_cast<int64_t>(g) * a.max_chunks + chunk) * R * (2 + D);
  for (int idx = threadIdx.x; idx < R * D; idx += kBlock) {
    const int r = idx / D;
    const int c = idx - r * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][r]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = (s_m[w][r] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_m[w][r] - M);
      L += f * s_l[w][r];
      O += f * s_o[(w * RMAX + r) * D + c];
    }
    float* pr = part + r * (2 + D);
    if (c == 0) {
      pr[0] = M;
      pr[1] = L;
    }
    pr[2 + c] = O;
  }
  if (!arrive_last(a.counters + g, static_cast<unsigned int>(n_chunks), &s_flag)) return;

  // ---- last block of the group: merge all chunk partials ----
  const float* gp = a.partials + static_cast<int64_t>(g) * a.max_chunks * R * (2 + D);
  S* out = static_cast<S*>(a.out) + static_cast<int64_t>(g) * R * D;
  for (int idx = threadIdx.x; idx < R * D; idx += kBlock) {
    const int r = idx / D;
    const int c = idx - r * D;
    float M = -INFINITY;
    for (int ch = 0; ch < n_chunks; ++ch) M = fmaxf(M, gp[(ch * R + r) * (2 + D)]);
    float L = 0.0f, O = 0.0f;
    for (int ch = 0; ch < n_chunks; ++ch) {
      const float* pr = gp + (ch * R + r) * (2 + D);
      const float f = (pr[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(pr[0] - M);
      L += f * pr[1];
      O += f * pr[2 + c];
    }
    out[idx] = from_f32(DT{}, L > 0.0f ? O / L : 0.0f);
  }
}

int rows_per_wave_iter(int dtype, int D) {
  const bool generic = !(D == 64 || D == 128 || D == 256);
  const int lpr = generic ? 64 : D / 8;
  const int rpi = kWave / lpr;
  const int nstep = dtype == TW_DTYPE_F32 ? 4 : 8;
  return nstep * rpi;
}

constexpr int kIters = 2;

template <typename DT, int DFIX, bool INDEXED>
int launch_r(const AttnArgs& a, hipStream_t stream) {
  const size_t lds_o = static_cast<size_t>(kWaves) * 8 * a.D * sizeof(float);
  const dim3 grid(a.G * a.max_chunks);
  if (a.R <= 1) {
    hipLaunchKernelGGL((decode_attn_kernel<DT, DFIX, 1, INDEXED>), grid, dim3(kBlock), lds_o, stream, a);
  } else if (a.R <= 2) {
    hipLaunchKernelGGL((decode_attn_kernel<DT, DFIX, 2, INDEXED>), grid, dim3(kBlock), lds_o, stream, a);
  } else if (a.R <= 4) {
    hipLaunchKernelGGL((decode_attn_kernel<DT, DFIX, 4, INDEXED>), grid, dim3(kBlock), lds_o, stream, a);
  } else {
    hipLaunchKernelGGL((decode_attn_kernel<DT, DFIX, 8, INDEXED>), grid, dim3(kBlock), lds_o, stream, a);
  }
  return tw_host::check_launch();
}

template <typename DT, bool INDEXED>
int launch_d(const AttnArgs& a, hipStream_t stream) {
  switch (a.D) {
    case 64: return launch_r<DT, 64, INDEXED>(a, stream);
    case 128: return launch_r<DT, 128, INDEXED>(a, stream);
    case 256: return launch_r<DT, 256, INDEXED>(a, stream);
    default: return launch_r<DT, 0, INDEXED>(a, stream);
  }
}

template <typename DT>
int launch_mode(const AttnArgs& a, hipStream_t stream) {
  return a.rows != nullptr ? launch_d<DT, true>(a, stream) : launch_d<DT, false>(a, stream);
}

size_t counter_bytes(int G) { return ((static_cast<size_t>(G) * 4 + 255) / 256) * 256; }

int max_chunks_for(int dtype, int D, int max_rows_total) {
  const int per_block = kWaves * rows_per_wave_iter(dtype, D) * kIters;
  return (max_rows_total + per_block - 1) / per_block;
}

}  // namespace
}  // namespace tw

extern "C" size_t tw_decode_attention_workspace_size(int G, int R, int D, int max_rows) {
  if (G <= 0 || R <= 0 || D <= 0 || max_rows < 0) return 0;
  // +1 row: the decode token; sized for the largest rows-per-block layout
  // (fp32 has fewer rows per block than 16-bit types).
  const int chunks = tw::max_chunks_for(TW_DTYPE_F32, D, max_rows + 1);
  return tw::counter_bytes(G) + static_cast<size_t>(G) * (chunks > 0 ? chunks : 1) * R * (2 + D) * sizeof(float);
}

extern "C" int tw_decode_attention(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                   int D, const int32_t* rows, const uint8_t* row_masks, const int32_t* row_counts,
                                   int64_t rows_stride, int64_t entry_stride_rows, const int32_t* cu_seqlens_k,
                                   int Hk, int window_left, int max_rows, const void* cur_k, const void* cur_v,
                                   float softmax_scale, void* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (q == nullptr || out == nullptr || G <= 0 || R <= 0 || R > 8 || D <= 0 || D > 512 || max_rows < 0)
    return TW_EINVAL;
  if ((cur_k == nullptr) != (cur_v == nullptr)) return TW_EINVAL;
  if (max_rows > 0 && (k_base == nullptr || v_base == nullptr)) return TW_EINVAL;
  if (rows != nullptr) {
    if (row_counts == nullptr || rows_stride < max_rows) return TW_EINVAL;
  } else {
    if (row_masks != nullptr || cu_seqlens_k == nullptr || Hk <= 0 || (G % Hk) != 0) return TW_EINVAL;
  }
  const bool fast = (D == 64 || D == 128 || D == 256);
  const int es = dtype == TW_DTYPE_F32 ? 4 : 2;
  if (fast) {
    const uintptr_t align = 16;
    if ((reinterpret_cast<uintptr_t>(k_base) % align) || (reinterpret_cast<uintptr_t>(v_base) % align) ||
        (cur_k && (reinterpret_cast<uintptr_t>(cur_k) % align)) || (cur_v && (reinterpret_cast<uintptr_t>(cur_v) % align)))
      return TW_EINVAL;
    if (rows == nullptr && ((static_cast<int64_t>(Hk) * D * es) % 16) != 0) return TW_EINVAL;
  }
  if (workspace == nullptr || workspace_bytes < tw_decode_attention_workspace_size(G, R, D, max_rows))
    return TW_ENOMEM;
  tw::AttnArgs a{};
  a.q = q;
  a.k = k_base;
  a.v = v_base;
  a.G = G;
  a.R = R;
  a.D = D;
  a.rows = rows;
  a.masks = row_masks;
  a.counts = row_counts;
  a.rows_stride = rows_stride;
  a.entry_stride = entry_stride_rows;
  a.cu_k = cu_seqlens_k;
  a.Hk = Hk > 0 ? Hk : 1;
  a.window_left = window_left;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  a.scale_log2 = softmax_scale * tw::kLog2e;
  a.out = out;
  a.counters = static_cast<unsigned int*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + tw::counter_bytes(G));
  a.iters = tw::kIters;
  a.max_rows = max_rows;
  a.max_chunks = tw::max_chunks_for(dtype, D, max_rows + (cur_k != nullptr ? 1 : 0));
  if (a.max_chunks <= 0) a.max_chunks = 1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TW_DTYPE_F16: return tw::launch_mode<tw::F16>(a, s);
    case TW_DTYPE_BF16: return tw::launch_mode<tw::BF16>(a, s);
    case TW_DTYPE_F32: return tw::launch_mode<tw::F32>(a, s);
    default: return TW_EINVAL;
  }
}
