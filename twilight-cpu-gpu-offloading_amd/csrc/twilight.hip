// Twilight stage 2: INT4 QK estimate over the Quest B0 candidates, softmax
// top-p pruning (dynamic or matched budgets) and the per-KV-group token union.
//
// Reference: TwilightMatchedBudgetOffloadedCache.prepare_layer_selection
// (twilight_offload_cache.py:996-1843): fused_affine_int4_qk
// (twilight_fused_qk.py:12-55) and /sqrt(D) (:1197-1261), the top-p of
// ExactTopPGraph (twilight_exact_top_p_graph.py:19-32, inline :1274-1310),
// matched_budget_counts (:50-86) and the GPU GQA union (:1517-1614).
//
// Orders defined here (the reference's are unpinned: cuBLAS / tl.sum
// reductions, argsort ties, fp32 cumsum rounding):
//   * logit = qk_scale * ((scale * dot) + (min * qsum)) with dot the exact
//     integer sum of code * Q over q's fixed-point form Q (22 fraction bits
//     below max |q|), scaled back by a power of two (see the INT4 QK section);
//   * candidate order = ascending token position (B0 pages ascending);
//   * top-p: masses E_i = floor(det_exp(l_i - max l) * 2^40), exact integer
//     sums; desired = smallest c whose c largest logits (ties to the lower
//     candidate) carry >= ceil(P24 * Z / 2^24) of the total mass Z, with
//     P24 = round(top_p * 2^24).  Sums of integers do not depend on the order
//     they are taken in, so the GPU needs no sort: a mass-weighted histogram
//     selection finds the boundary, as the top-k does for counts.
#pragma clang fp contract(off)

#include <type_traits>

#include "score_order.h"
#include "select.h"
#include "union_record.h"

namespace tw {
namespace {

using namespace sel;

constexpr int kQkPagesPerBlock = 16;

// ------------------------------------------------------------ INT4 QK
// The estimate is exact integer arithmetic followed by three fp32 steps.  A
// query head is first put in fixed point: M = max_d |q_d|, E the exponent of
// M (M = f * 2^E, f in [0.5, 1)), Q_d = rint(q_d * 2^(22 - E)), so
// |Q_d| <= 2^22 (a NaN or infinite q_d makes the head's logits NaN, M = 0
// gives Q = 0).  Then for every candidate row
//   S = sum_d code_d * Q_d                                  (exact, 64-bit)
//   logit = qk_scale * ((scale * ldexp(S, E - 22)) + (min * ldexp(sum_d Q_d, E - 22)))
// Q_d is split into three byte slices, Q = h * 2^16 + m * 2^8 + l with h
// signed (|h| <= 64) and m, l unsigned, and every slice meets the codes in
// v_dot4 instructions: the codes of 8 channels are one 32-bit word whose even
// channels (w & 0x0f0f0f0f) and odd channels ((w >> 4) & 0x0f0f0f0f) are four
// bytes each, dotted with the matching bytes of a slice.  The sums are
// integers, so neither the lane layout nor the summation order changes a bit
// of the result.
struct QkArgs {
  const float* q;             // [G][R][D]
  const uint8_t* packed;      // entry g row t at + (g*qstride + t)*D/2
  const void* scale;          // [G][qstride]
  const void* minimum;
  int64_t qstride;            // entry stride in rows
  int64_t qrows;              // valid rows per entry
  int G, R, D;
  const int32_t* plan_pages;  // [G][plan_stride] union of the B0 pages, ascending
  const uint8_t* plan_masks;  // heads that chose each page
  const int32_t* plan_counts;
  int64_t plan_stride;
  int b0, sink, bs;
  float qk_scale;
  float* logits;              // [G][R][b0*bs]
  // Page-row outputs (nullable): slot_u[g][r][slot] = the union index of
  // head r's B0 slot, and page_rows[g][u] (plan_stride apart) cleared for
  // every union page, for the top-p's row bits.
  int32_t* slot_u;
  uint32_t* page_rows;
};

// Sums / maxima over aligned groups of N lanes (N = 1..16, a power of two);
// every lane of a group receives the result.
template <int N>
__device__ __forceinline__ int group_sum_i32(int x) {
  if constexpr (N >= 2) x += static_cast<int>(dpp_u32<kDppQuadXor1>(static_cast<uint32_t>(x)));
  if constexpr (N >= 4) x += static_cast<int>(dpp_u32<kDppQuadXor2>(static_cast<uint32_t>(x)));
  if constexpr (N >= 8) x += static_cast<int>(dpp_u32<kDppRowHalfMirror>(static_cast<uint32_t>(x)));
  if constexpr (N >= 16) x += static_cast<int>(dpp_u32<kDppRowMirror>(static_cast<uint32_t>(x)));
  return x;
}
template <int N>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t x) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  if constexpr (N >= 2) x = mx(x, dpp_u32<kDppQuadXor1>(x));
  if constexpr (N >= 4) x = mx(x, dpp_u32<kDppQuadXor2>(x));
  if constexpr (N >= 8) x = mx(x, dpp_u32<kDppRowHalfMirror>(x));
  if constexpr (N >= 16) x = mx(x, dpp_u32<kDppRowMirror>(x));
  if constexpr (N >= 32) x = mx(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 16)));
  if constexpr (N >= 64) x = mx(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 32)));
  return x;
}
template <int N>
__device__ __forceinline__ int group_sum_wide_i32(int x) {
  x = group_sum_i32<(N < 16 ? N : 16)>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Lane layout of one INT4 row: LPR lanes per row, each owning CPL consecutive
// channels, i.e. CPL / 2 code bytes in WPL 32-bit words (a half word when
// CPL = 4).
template <int DIM, int CPLMAX>
struct QkLane {
  static constexpr int CPL = DIM < CPLMAX ? DIM : CPLMAX;
  static constexpr int LPR = DIM / CPL;
  static constexpr int RPW = kWave / LPR;  // rows per wavefront instruction
  static constexpr int WPL = CPL >= 8 ? CPL / 8 : 1;
  static_assert(CPL >= 4 && LPR * CPL == DIM && (LPR & (LPR - 1)) == 0 && LPR <= 16, "unsupported head dim");

  __device__ static __forceinline__ void codes(const uint8_t* row, int c0, uint32_t (&w)[4]) {
    const uint8_t* p = row + c0 / 2;
    if constexpr (CPL == 32) {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (CPL == 16) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      w[0] = v.x; w[1] = v.y; w[2] = 0u; w[3] = 0u;
    } else if constexpr (CPL == 8) {
      w[0] = *reinterpret_cast<const uint32_t*>(p); w[1] = 0u; w[2] = 0u; w[3] = 0u;
    } else {
      w[0] = *reinterpret_cast<const uint16_t*>(p); w[1] = 0u; w[2] = 0u; w[3] = 0u;
    }
  }
};

// The logit of a candidate from its exact integer dot S (see above): one
// rounding of S to fp32, the power-of-two scale, then three fp32 operations.
__device__ __forceinline__ float qk_logit(int64_t S, int shift, float qsum, bool ok, float s, float m,
                                          float qk_scale) {
  if (!ok) return u32_as_f32(0x7fc00000u);
  // |S| < 2^34: exact in double, so one double -> float conversion is the
  // single round-to-nearest-even of S
  const float dotc = ldexpf(static_cast<float>(static_cast<double>(S)), shift);
  const float a = s * dotc;
  const float c = m * qsum;
  return qk_scale * (a + c);
}

// One query head in fixed point, as the byte slices of the lane's CPL
// channels laid out like its code words: [word][0] even channels, [1] odd.
template <int CPL, int LPR>
struct QFix {
  static constexpr int WPL = CPL >= 8 ? CPL / 8 : 1;
  uint32_t hs[WPL][2], ms[WPL][2], ls[WPL][2];
  int shift;
  float qsum;  // ldexp(sum_d Q_d, shift), the same in every lane
  bool ok;

  // qr: the head's D channels; c0: the lane's first channel.  Every lane of
  // a row group must call it (group reductions).
  __device__ __forceinline__ void init(const float* qr, int c0) {
    float v[CPL];
#pragma unroll
    for (int i = 0; i < CPL; i += 4) *reinterpret_cast<float4*>(v + i) = *reinterpret_cast<const float4*>(qr + c0 + i);
    uint32_t mx = 0u, bad = 0u;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t u = f32_as_u32(v[i]) & 0x7fffffffu;
      bad |= u >= 0x7f800000u ? 1u : 0u;
      mx = u > mx ? u : mx;
    }
    mx = group_max_u32<LPR>(mx);
    bad = group_max_u32<LPR>(bad);
    ok = bad == 0u;
    const float M = u32_as_f32(mx);
    int E = 22;
    if (ok && M != 0.0f) (void)frexpf(M, &E);
    shift = (ok && M != 0.0f) ? E - 22 : 0;
    int q_int[CPL];
    int part = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      q_int[i] = (ok && M != 0.0f) ? static_cast<int>(rintf(ldexpf(v[i], 22 - E))) : 0;
      part += q_int[i];
    }
    qsum = ldexpf(static_cast<float>(group_sum_i32<LPR>(part)), shift);
#pragma unroll
    for (int w = 0; w < WPL; ++w) {
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        uint32_t h = 0u, m = 0u, l = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 8 * w + 2 * j + par;
          if (i < CPL) {
            const int Q = q_int[i];
            h |= (static_cast<uint32_t>(Q >> 16) & 255u) << (8 * j);
            m |= (static_cast<uint32_t>(Q >> 8) & 255u) << (8 * j);
            l |= (static_cast<uint32_t>(Q) & 255u) << (8 * j);
          }
        }
        hs[w][par] = h;
        ms[w][par] = m;
        ls[w][par] = l;
      }
    }
  }

  // The head's slices for the lane's channels from a block's staged form
  // (stage_qfix): [head][slice][parity][DIM / 8 words].
  template <int DIM>
  __device__ __forceinline__ void load(const uint32_t* st, const int* st_shift, const float* st_qsum,
                                       const int* st_ok, int r, int c0) {
    constexpr int K = DIM >= 8 ? DIM / 8 : 1;
    const uint32_t* base = st + r * 6 * K + c0 / 8;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        hs[w][par] = base[(0 * 2 + par) * K + w];
        ms[w][par] = base[(1 * 2 + par) * K + w];
        ls[w][par] = base[(2 * 2 + par) * K + w];
      }
    }
    shift = st_shift[r];
    qsum = st_qsum[r];
    ok = st_ok[r] != 0;
  }

  // sum_d code_d * Q_d of one row (every lane of the group gets it).
  __device__ __forceinline__ int64_t dot(const uint32_t (&w)[4]) const {
    int th = 0;
    uint32_t tm = 0u, tl = 0u;
#pragma unroll
    for (int k = 0; k < WPL; ++k) {
      const uint32_t lo = w[k] & 0x0f0f0f0fu;
      const uint32_t hi = (w[k] >> 4) & 0x0f0f0f0fu;
      th = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(hs[k][0]), th, false);
      th = __builtin_amdgcn_sdot4(static_cast<int>(hi), static_cast<int>(hs[k][1]), th, false);
      tm = __builtin_amdgcn_udot4(lo, ms[k][0], tm, false);
      tm = __builtin_amdgcn_udot4(hi, ms[k][1], tm, false);
      tl = __builtin_amdgcn_udot4(lo, ls[k][0], tl, false);
      tl = __builtin_amdgcn_udot4(hi, ls[k][1], tl, false);
    }
    // per lane |th| <= 32*15*64, so th * 256 + tm stays far inside int32, and
    // so do the group sums for D <= 256
    const int t = group_sum_i32<LPR>(th * 256 + static_cast<int>(tm));
    const int l = group_sum_i32<LPR>(static_cast<int>(tl));
    return static_cast<int64_t>(t) * 256 + l;
  }

  __device__ __forceinline__ float logit(int64_t S, float s, float m, float qk_scale) const {
    return qk_logit(S, shift, qsum, ok, s, m, qk_scale);
  }
};

constexpr int kQkRows = 256;  // candidate rows per block

// Stage the fixed-point form of the group's R query heads in LDS, once per
// block: thread t converts VPT consecutive channels of head t / LH (LH =
// DIM / VPT lanes per head, an aligned group inside one wavefront, so the
// head's max |q| and sum Q are group reductions).  st: [RMAX][3][2][DIM/8]
// words (slice h, m, l; even / odd channels), byte j of word k holding
// channel 8k + 2j + parity.  The caller synchronizes before reading.
template <int DIM, int RMAX>
struct QStage {
  static constexpr int TOT = RMAX * DIM;
  static constexpr int VPT = TOT > kBlock ? TOT / kBlock : 1;  // channels per thread
  static constexpr int LH = DIM / VPT;                         // lanes per head
  static constexpr int K = DIM >= 8 ? DIM / 8 : 1;
  static_assert(LH <= kWave && (kWave % LH) == 0 && VPT <= 8 && (VPT & (VPT - 1)) == 0, "head layout");
  float v[VPT];
  // the thread's channels (issued first, so the load overlaps the block's
  // other round-trip-1 loads)
  __device__ __forceinline__ void load(const float* qg, int R) {
    const int t = static_cast<int>(threadIdx.x);
    const int r = t / LH;
    const int d0 = (t - r * LH) * VPT;
#pragma unroll
    for (int i = 0; i < VPT; ++i) v[i] = qg[static_cast<int64_t>(r < R ? r : 0) * DIM + d0 + i];
  }
};

// BALANCED: the slices are signed digits h, m, l in [-128, 127] with
// Q = h * 2^16 + m * 2^8 + l (for the matrix cores' signed int8 operands);
// otherwise h = Q >> 16 signed and m, l the unsigned bytes below it.  Both
// represent the same Q, so the integer dot is the same.
template <int DIM, int RMAX, bool BALANCED = false>
__device__ __forceinline__ void stage_qfix(const QStage<DIM, RMAX>& qv, int R, uint32_t* st, int* st_shift,
                                           float* st_qsum, int* st_ok) {
  using QS = QStage<DIM, RMAX>;
  constexpr int VPT = QS::VPT, LH = QS::LH, K = QS::K;
  const int t = static_cast<int>(threadIdx.x);
  const int r = t / LH;
  const int d0 = (t - r * LH) * VPT;
  const bool act = r < R;
  const float* v = qv.v;
  uint32_t mx = 0u, bad = 0u;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const uint32_t u = f32_as_u32(v[i]) & 0x7fffffffu;
    bad |= u >= 0x7f800000u ? 1u : 0u;
    mx = u > mx ? u : mx;
  }
  mx = group_max_u32<LH>(mx);
  bad = group_max_u32<LH>(bad);
  const bool ok = bad == 0u;
  const float M = u32_as_f32(mx);
  const bool nz = ok && M != 0.0f;
  int E = 22;
  if (nz) (void)frexpf(M, &E);
  int part = 0;
  int Q[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    Q[i] = nz ? static_cast<int>(rintf(ldexpf(v[i], 22 - E))) : 0;
    part += Q[i];
  }
  const int qs = group_sum_wide_i32<LH>(part);
  if (act) {
    uint8_t* sb = reinterpret_cast<uint8_t*>(st);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int d = d0 + i;
      const int k = d / 8, par = d & 1, j = (d % 8) / 2;
      int dig[3];
      if constexpr (BALANCED) {
        const int l = ((Q[i] + 128) & 255) - 128;
        const int q1 = (Q[i] - l) >> 8;
        const int m = ((q1 + 128) & 255) - 128;
        dig[0] = (q1 - m) >> 8;
        dig[1] = m;
        dig[2] = l;
      } else {
        dig[0] = Q[i] >> 16;
        dig[1] = Q[i] >> 8;
        dig[2] = Q[i];
      }
#pragma unroll
      for (int sl = 0; sl < 3; ++sl) sb[((r * 3 + sl) * 2 + par) * K * 4 + k * 4 + j] = static_cast<uint8_t>(dig[sl] & 255);
    }
    if (d0 == 0) {
      st_shift[r] = nz ? E - 22 : 0;
      st_qsum[r] = ldexpf(static_cast<float>(qs), nz ? E - 22 : 0);
      st_ok[r] = ok ? 1 : 0;
    }
  }
}

// Union-plan INT4 QK: block = kQkRows consecutive rows of group g's union
// pages (page u holds rows u*bs .. u*bs + bs - 1).  Round trip 1 loads the
// plan count, the block's pages and masks, the masks of every earlier union
// page (for the logit slots) and the queries; round trip 2 the rows' codes,
// scales and minima.  A head's logit slot for union page u is the number of
// earlier union pages it chose (its B0 pages are ascending).  The block's
// logits go through LDS and leave as one coalesced store per (row, head).
//
// MF (D = 128): the dots run on the matrix cores, v_mfma_i32_16x16x64_i8
// per 16 rows and 64 channels.  A row m = 4 h + t holds slice t of head h
// (balanced signed digits; row 4 h + 3 is zero) and B column n the codes of
// candidate row n, so lane group G of the product holds head G's three slice
// dots of row lane % 16 in its own registers and forms S there.  Both
// operands give a lane the same 16 channels of a 64-channel step, in the
// same byte order (even channels of a code word, then odd), so the sum over
// k pairs every q digit with its code whatever order the hardware uses
// inside a lane group.  Slices of 128 channels stay far inside int32.
template <typename DT, int DIM, int RMAX, int CPLMAX, bool MF = false>
__global__ __launch_bounds__(kBlock) void twilight_qk_kernel(QkArgs a) {
  using S = typename DT::storage;
  using L = QkLane<DIM, CPLMAX>;
  using QF = QFix<L::CPL, L::LPR>;
  static_assert(!MF || DIM == 128, "the matrix-core path takes 128 channels");
  constexpr int RPB = MF ? kWaves * 16 : kWaves * L::RPW;
  constexpr int PASSES = (kQkRows + RPB - 1) / RPB;
  constexpr int NC = RMAX / 2;  // packed head counters (two 16-bit fields each)
  constexpr int KW = DIM >= 8 ? DIM / 8 : 1;
  static_assert(RMAX == 4 || RMAX == 8, "4 or 8 head slots");
  static_assert(kQkRows == kBlock, "one block page per thread");
  const int bs = a.bs;
  const int row_blocks = static_cast<int>((a.plan_stride * bs + kQkRows - 1) / kQkRows);
  const int g = blockIdx.x / row_blocks;
  const int rb = blockIdx.x - g * row_blocks;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int R = a.R;
  const int row0 = rb * kQkRows;
  const int u_first = row0 / bs;
  const int u_cap = static_cast<int>(a.plan_stride) - 1;

  __shared__ int s_page[kQkRows];
  __shared__ int s_mask[kQkRows];
  __shared__ int s_slot[kQkRows][RMAX];
  __shared__ uint32_t s_cnt[kWaves][NC];
  __shared__ float s_log[kQkRows][RMAX];
  __shared__ __align__(16) uint32_t s_q[RMAX * 6 * KW];
  __shared__ int s_qshift[RMAX];
  __shared__ float s_qsum[RMAX];
  __shared__ int s_qok[RMAX];

  // ---- round trip 1 (all loads independent): queries, plan count, the
  // block's pages and masks, the masks of every earlier union page ----
  QStage<DIM, RMAX> qst;
  qst.load(a.q + static_cast<int64_t>(g) * R * DIM, R);
  int nu = a.plan_counts[g];
  const uint8_t* pm = a.plan_masks + static_cast<int64_t>(g) * a.plan_stride;
  uint32_t cnt[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) cnt[c] = 0u;
  for (int ub = 0; ub < u_first; ub += 4 * kBlock) {
    uint32_t m4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = ub + j * kBlock + tid;
      const uint32_t m = pm[u < u_first ? u : 0];
      m4[j] = u < u_first ? m : 0u;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int c = 0; c < NC; ++c) cnt[c] += ((m4[j] >> (2 * c)) & 1u) | (((m4[j] >> (2 * c + 1)) & 1u) << 16);
    }
  }
  int my_page, my_mask;
  {
    const int u = u_first + tid < u_cap ? u_first + tid : u_cap;
    my_page = a.plan_pages[static_cast<int64_t>(g) * a.plan_stride + u];
    my_mask = pm[u];
  }
  nu = nu < 0 ? 0 : (nu > a.plan_stride ? static_cast<int>(a.plan_stride) : nu);
  const int total_rows = nu * bs;
  if (row0 >= total_rows) return;  // block-uniform, before any barrier
  const int nrows = (total_rows - row0) < kQkRows ? (total_rows - row0) : kQkRows;
  const int npg = (row0 + nrows - 1) / bs - u_first + 1;
  s_page[tid] = my_page;
  s_mask[tid] = tid < npg ? my_mask : 0;
  if constexpr (DIM < 8) {
    // the heads stage their bytes below; the unused bytes of a D < 8 word stay zero
    for (int i = tid; i < RMAX * 6 * KW; i += kBlock) s_q[i] = 0u;
  }
  __syncthreads();
  // ---- round trip 2: the block's INT4 rows (needs only the page ids) ----
  const int c0 = (lane % L::LPR) * L::CPL;
  const int64_t N = static_cast<int64_t>(a.b0) * bs;
  const uint8_t* pk = a.packed + static_cast<int64_t>(g) * a.qstride * (DIM / 2);
  const S* sc = static_cast<const S*>(a.scale) + static_cast<int64_t>(g) * a.qstride;
  const S* mn = static_cast<const S*>(a.minimum) + static_cast<int64_t>(g) * a.qstride;
  uint32_t w[PASSES][4];
  S sv[PASSES], mv[PASSES];
#pragma unroll
  for (int i = 0; i < PASSES; ++i) {
    // row within the block: MF, tile i of the wavefront's 16-row tiles, row
    // lane % 16, lane group lane / 16 reading code bytes [16 G, 16 G + 16)
    const int lr = MF ? i * RPB + wave * 16 + (lane % 16) : i * RPB + wave * L::RPW + lane / L::LPR;
    const int row = row0 + (lr < nrows ? lr : 0);
    const int p = row / bs - u_first;
    int64_t t = static_cast<int64_t>(a.sink) + static_cast<int64_t>(s_page[p]) * bs + (row - (row / bs) * bs);
    t = (t >= 0 && t < a.qrows) ? t : 0;
    if constexpr (MF) {
      const uint4 v = *reinterpret_cast<const uint4*>(pk + t * (DIM / 2) + 16 * (lane / 16));
      w[i][0] = v.x; w[i][1] = v.y; w[i][2] = v.z; w[i][3] = v.w;
    } else {
      L::codes(pk + t * (DIM / 2), c0, w[i]);
    }
    sv[i] = sc[t];
    mv[i] = mn[t];
  }
  // ---- while they are in flight: q in fixed point, the logit slots ----
  stage_qfix<DIM, RMAX, MF>(qst, R, s_q, s_qshift, s_qsum, s_qok);
#pragma unroll
  for (int c = 0; c < NC; ++c) cnt[c] = static_cast<uint32_t>(wave_sum_i32(static_cast<int>(cnt[c])));
  if (lane == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) s_cnt[wave][c] = cnt[c];
  }
  __syncthreads();
  if (wave == 0) {
    // a head's slot for union page u = the earlier union pages it chose:
    // four block pages per lane, exclusive scan of the packed counts
    constexpr int PPL = kQkRows / kWave;
    int mk[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) mk[j] = s_mask[PPL * lane + j];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint32_t before = 0u;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) before += s_cnt[v][c];
      uint32_t e[PPL], tot = 0u;
#pragma unroll
      for (int j = 0; j < PPL; ++j) {
        e[j] = ((mk[j] >> (2 * c)) & 1) | (((mk[j] >> (2 * c + 1)) & 1) << 16);
        tot += e[j];
      }
      before += wave_prefix_sum_u32(tot) - tot;
#pragma unroll
      for (int j = 0; j < PPL; ++j) {
        s_slot[PPL * lane + j][2 * c] = static_cast<int>(before & 0xffffu);
        s_slot[PPL * lane + j][2 * c + 1] = static_cast<int>(before >> 16);
        before += e[j];
      }
    }
  }
  if constexpr (MF) {
    // ---- A operands: head tile h, step sp: lane group G holds channels
    // 32 G + 16 sp + [0, 16), i.e. code words k0 = 4 G + 2 sp and k0 + 1,
    // as [even, odd] channel bytes of each word, like B below ----
    typedef int v4i __attribute__((ext_vector_type(4)));
    constexpr int HT = RMAX / 4;
    const int G = lane / 16;
    const int mrow = lane % 16;
    v4i av[HT][2];
#pragma unroll
    for (int h = 0; h < HT; ++h) {
      const int r = 4 * h + mrow / 4;
      const int t = mrow % 4;
      const bool live = t < 3 && r < R;
      const uint32_t* st = s_q + (r < R ? r : 0) * 6 * KW + (t < 3 ? t : 0) * 2 * KW;
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        const int k0 = 4 * G + 2 * sp;
        av[h][sp][0] = live ? static_cast<int>(st[k0]) : 0;            // even channels of word k0
        av[h][sp][1] = live ? static_cast<int>(st[KW + k0]) : 0;       // odd channels of word k0
        av[h][sp][2] = live ? static_cast<int>(st[k0 + 1]) : 0;
        av[h][sp][3] = live ? static_cast<int>(st[KW + k0 + 1]) : 0;
      }
    }
    // ---- dot products: lane (G, n) of tile i gets head 4 h + G of row n ----
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int lr = i * RPB + wave * 16 + mrow;
      const float sf = to_f32(DT{}, sv[i]), mf = to_f32(DT{}, mv[i]);
      v4i b0, b1;
      b0[0] = static_cast<int>(w[i][0] & 0x0f0f0f0fu);
      b0[1] = static_cast<int>((w[i][0] >> 4) & 0x0f0f0f0fu);
      b0[2] = static_cast<int>(w[i][1] & 0x0f0f0f0fu);
      b0[3] = static_cast<int>((w[i][1] >> 4) & 0x0f0f0f0fu);
      b1[0] = static_cast<int>(w[i][2] & 0x0f0f0f0fu);
      b1[1] = static_cast<int>((w[i][2] >> 4) & 0x0f0f0f0fu);
      b1[2] = static_cast<int>(w[i][3] & 0x0f0f0f0fu);
      b1[3] = static_cast<int>((w[i][3] >> 4) & 0x0f0f0f0fu);
#pragma unroll
      for (int h = 0; h < HT; ++h) {
        v4i c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[h][0], b0, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[h][1], b1, c, 0, 0, 0);
        const int r = 4 * h + G;
        const int64_t S = (static_cast<int64_t>(c[0]) << 16) + (static_cast<int64_t>(c[1]) << 8) + c[2];
        const int rr = r < R ? r : 0;
        const float lg = qk_logit(S, s_qshift[rr], s_qsum[rr], s_qok[rr] != 0, sf, mf, a.qk_scale);
        if (r < R && lr < kQkRows) s_log[lr][r] = lg;
      }
    }
  } else {
    QF qf[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) qf[r].template load<DIM>(s_q, s_qshift, s_qsum, s_qok, r < R ? r : 0, c0);
    // ---- dot products ----
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int lr = i * RPB + wave * L::RPW + lane / L::LPR;
      const float s = to_f32(DT{}, sv[i]), m = to_f32(DT{}, mv[i]);
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        if (r >= R) break;
        const float lg = qf[r].logit(qf[r].dot(w[i]), s, m, a.qk_scale);
        if (lr < kQkRows && (lane % L::LPR) == 0) s_log[lr][r] = lg;
      }
    }
  }
  __syncthreads();
  // ---- page-row outputs: each union page's slot map and a cleared row mask ----
  if (a.slot_u != nullptr) {
    for (int idx = tid; idx < npg * R; idx += kBlock) {
      const int p = idx / R;
      const int r = idx - p * R;
      const int slot = s_slot[p][r];
      if (((s_mask[p] >> r) & 1) && slot < a.b0)
        a.slot_u[(static_cast<int64_t>(g) * R + r) * a.b0 + slot] = u_first + p;
    }
  }
  if (a.page_rows != nullptr && tid < npg) a.page_rows[static_cast<int64_t>(g) * a.plan_stride + u_first + tid] = 0u;
  // ---- out: row lr of head r to logits[g][r][slot * bs + lr's place in its
  // page]; candidates beyond the INT4 rows are skipped ----
  if (tid < nrows) {
    const int lr = tid;
    const int row = row0 + lr;
    const int p = row / bs - u_first;
    const int i = row - (row / bs) * bs;
    const int64_t t = static_cast<int64_t>(a.sink) + static_cast<int64_t>(s_page[p]) * bs + i;
    const int m = (t >= 0 && t < a.qrows) ? s_mask[p] : 0;
    for (int r = 0; r < R; ++r) {
      const int slot = s_slot[p][r];
      if (((m >> r) & 1) && slot < a.b0)
        a.logits[(static_cast<int64_t>(g) * R + r) * N + static_cast<int64_t>(slot) * bs + i] = s_log[lr][r];
    }
  }
}

// INT4 QK at explicit candidate positions, one query head per block row
// (the fused_affine_int4_qk call surface): positions[g][r][n] index entry g's
// INT4 rows.  The estimate of twilight_qk_kernel; with materialize, the
// dequantized rows k_d = f32(code_d) * f32(scale) + f32(min) instead.
template <typename DT, int DIM, int CPLMAX>
__global__ __launch_bounds__(kBlock) void int4_qk_positions_kernel(QkArgs a, const int64_t* positions, int N,
                                                                   float* out, bool materialize) {
  using S = typename DT::storage;
  using L = QkLane<DIM, CPLMAX>;
  using QF = QFix<L::CPL, L::LPR>;
  constexpr int ROWS = 64;  // candidates per block
  const int tiles = (N + ROWS - 1) / ROWS;
  const int row = blockIdx.x / tiles;  // g*R + r
  const int tile = blockIdx.x - row * tiles;
  const int g = row / a.R;
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int c0 = (lane % L::LPR) * L::CPL;
  QF qf;
  qf.init(a.q + static_cast<int64_t>(row) * DIM, c0);
  const uint8_t* pk = a.packed + static_cast<int64_t>(g) * a.qstride * (DIM / 2);
  const S* sc = static_cast<const S*>(a.scale) + static_cast<int64_t>(g) * a.qstride;
  const S* mn = static_cast<const S*>(a.minimum) + static_cast<int64_t>(g) * a.qstride;
  for (int i0 = tile * ROWS + wave * L::RPW; i0 < (tile + 1) * ROWS; i0 += kWaves * L::RPW) {
    const int n = i0 + lane / L::LPR;
    const bool ok = n < N && n < (tile + 1) * ROWS;
    int64_t t = positions[static_cast<int64_t>(row) * N + (n < N ? n : N - 1)];
    const bool in_range = t >= 0 && t < a.qrows;
    t = in_range ? t : 0;
    uint32_t w[4];
    L::codes(pk + t * (DIM / 2), c0, w);
    const float s = to_f32(DT{}, sc[t]), m = to_f32(DT{}, mn[t]);
    if (materialize) {
      if (ok) {
        float* o = out + (static_cast<int64_t>(row) * N + n) * DIM + c0;
#pragma unroll
        for (int j = 0; j < L::CPL; ++j) {
          const float k = static_cast<float>((w[j / 8] >> (4 * (j % 8))) & 15u) * s + m;
          o[j] = in_range ? k : 0.0f;
        }
      }
      continue;
    }
    const float lg = qf.logit(qf.dot(w), s, m, a.qk_scale);
    if (ok && in_range && (lane % L::LPR) == 0) out[static_cast<int64_t>(row) * N + n] = lg;
  }
}

// ---------------------------------------------------------------- top-p
// Deterministic exp of x <= 0 (the definition the CPU oracle shares):
// x < -28 -> 0; t = x*log2(e), n = rint(t), f = t - n, degree-6 Taylor
// polynomial of 2^f in Horner form, scaled by 2^n.
// Written without a branch (the argument is replaced by 0 where the result
// is 0), so that a thread's several calls interleave.
__device__ __forceinline__ float det_exp(float x) {
  const bool ok = x >= -28.0f;  // false for NaN
  const float t = (ok ? x : 0.0f) * 1.44269504088896341f;
  const float n = __builtin_rintf(t);
  const float f = t - n;
  float p = 1.54035303933816e-4f;
  p = p * f + 1.33335581464284e-3f;
  p = p * f + 9.61812910762848e-3f;
  p = p * f + 5.55041086648216e-2f;
  p = p * f + 2.40226506959101e-1f;
  p = p * f + 6.93147180559945e-1f;
  p = p * f + 1.0f;
  return ok ? __builtin_ldexpf(p, static_cast<int>(n)) : 0.0f;
}
__device__ __forceinline__ uint64_t mass_of(float logit, float lmax) {
  return static_cast<uint64_t>(det_exp(logit - lmax) * 1099511627776.0f);  // * 2^40, truncated
}

struct SelectArgs {
  const float* logits;        // [G][R][N]
  int G, R, N;
  uint32_t p24;               // round(top_p * 2^24)
  bool matched;
  bool given;                 // matched kernel only, with allocated[] as its input
  int target_total;           // matched: fixed_pages * bs * R
  const int32_t* sel_pages;   // [G][R][b0] B0 pages per head, ascending
  int b0;
  int32_t* desired;           // [G][R]
  int32_t* allocated;         // nullable [G][R]
  uint32_t* selbits;          // [G][R][words_n] published selections
  int words_n;
  int32_t* rows;              // [G][rows_stride] the GQA union, ascending
  int32_t* row_counts;        // [G]
  int64_t rows_stride;
  int sink, recent, bs, length, append_position;
  unsigned int* counters;     // [G]
  // Ragged groups (nullable, dynamic budgets): group g has lengths[g] tokens
  // (< rows_stride; `length` then bounds them all), so ragged_pages(lengths[g],
  // .., p_max) candidate pages and at most that many (<= b0) B0 pages per head.
  const int32_t* lengths;
  int p_max;
  // Page-row output (nullable, dynamic budgets): each kept candidate's row
  // bit ORed into page_rows[g][slot_u[g][r][slot]] (page_rows_stride apart),
  // instead of the published bitmaps and the group's union rows.
  const int32_t* slot_u;
  uint32_t* page_rows;
  int64_t page_rows_stride;
};

// Tokens of group g (ragged: its own length, clamped to the launch bound).
__device__ __forceinline__ int group_length(const SelectArgs& s, int g) {
  if (s.lengths == nullptr) return s.length;
  const int L = s.lengths[g];
  return L < 0 ? 0 : (L > s.length ? s.length : L);
}
// Valid candidates of group g's rows: B0 pages x bs (ragged: fewer when the
// group has fewer candidate pages).
__device__ __forceinline__ int group_candidates(const SelectArgs& s, int g) {
  if (s.lengths == nullptr) return s.N;
  const int P = ragged_pages(group_length(s, g), s.sink, s.recent, s.bs, s.p_max);
  const int k = P < s.b0 ? P : s.b0;
  return k * s.bs;
}

// Block-shared state of a top-p block of NT threads.
template <int NT>
struct TopShared {
  static constexpr int kW = NT / kWave;
  SelSharedT<NT> sel;
  __align__(16) unsigned long long bin_mass[kLinBins + 64];
  unsigned long long red64[kW];
  unsigned long long cmass[kExactMax];
  float fred[kW];
  int ires[4];
  unsigned long long lres[2];
  int fp_i[4];                 // block_top_p_fast: the first wavefront's results
  unsigned long long fp_l[2];
};

__device__ __forceinline__ uint64_t shfl_down_u64(uint64_t v, int o) {
  const uint32_t lo = static_cast<uint32_t>(__shfl_down(static_cast<int>(v & 0xffffffffu), o));
  const uint32_t hi = static_cast<uint32_t>(__shfl_down(static_cast<int>(v >> 32), o));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
// Inclusive suffix sum of 64-bit values over the lanes of a wavefront.
__device__ __forceinline__ uint64_t wave_suffix_u64(uint64_t v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint64_t w = shfl_down_u64(v, o);
    if (l + o < kWave) v += w;
  }
  return v;
}
template <int NT>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, unsigned long long* red) {
  const uint64_t s = wave_suffix_u64(v);  // lane 0 holds the wave sum
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  if (lane_id() == 0) red[wave] = s;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) t += red[w];
  __syncthreads();
  return t;
}

// ceil(p24 * z / 2^24) without 128-bit arithmetic (p24 <= 2^24, z < 2^56).
__device__ __forceinline__ uint64_t top_p_threshold(uint32_t p24, uint64_t z) {
  // p24 * z = hi * 2^32 + lo with hi < 2^56 and lo < 2^57; (hi * 2^32) is a
  // multiple of 2^24, so the ceiling only involves lo.
  const uint64_t lo = static_cast<uint64_t>(p24) * (z & 0xffffffffu);
  const uint64_t hi = static_cast<uint64_t>(p24) * (z >> 32);
  return (hi << 8) + ((lo + ((1ull << 24) - 1)) >> 24);
}

// The smallest count c of top keys (key desc, index asc) whose masses sum to
// >= need; marks them in *taken (bit j = key j of this thread).  Keys are
// KPT contiguous per thread (indices KPT*t + j).  kmin0/kmax0: the smallest
// and largest key of the row; the caller has cleared the histograms.
template <int KPT, int NT>
__device__ int block_top_mass(const uint32_t (&key)[KPT], const uint64_t (&mass)[KPT], int N, uint64_t need,
                              uint32_t kmin0, uint32_t kmax0, TopShared<NT>& sh, uint32_t* taken_out) {
  constexpr int kW = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int i0 = KPT * tid;
  uint32_t cand = 0u, taken = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) cand |= (i0 + j < N) ? (1u << j) : 0u;
  int count = 0;  // keys taken so far (block-uniform)
  int ccount = N;
  for (int level = 0;; ++level) {
    if (ccount <= kWave) {
      // exact, one wavefront: the candidates are staged in index order, lane
      // c ranks candidate c (key desc, index asc) and sums the masses ahead
      // of it with register reads; the boundary is the lane whose own mass
      // crosses need
      int total;
      const int first = block_excl_scan<NT>(__popc(cand), sh.sel.scan, &total);
      int slot = first;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((cand >> j) & 1u) {
          sh.sel.ckey[slot] = key[j];
          sh.cmass[slot] = mass[j];
          ++slot;
        }
      }
      __syncthreads();
      if (wave == 0) {
        const bool live = lane < total;
        const uint32_t mk = live ? sh.sel.ckey[lane] : 0u;
        const uint64_t mm = live ? sh.cmass[lane] : 0ull;
        const uint32_t mlo = static_cast<uint32_t>(mm), mhi = static_cast<uint32_t>(mm >> 32);
        uint64_t before = 0;
        int rank = 0;
        for (int m = 0; m < total; ++m) {
          const uint32_t km = readlane_u32(mk, m);
          const uint64_t am = (static_cast<uint64_t>(readlane_u32(mhi, m)) << 32) | readlane_u32(mlo, m);
          const bool ahead = km > mk || (km == mk && m < lane);
          before += ahead ? am : 0ull;
          rank += ahead ? 1 : 0;
        }
        const bool cross = live && before < need && need <= before + mm;
        const uint64_t cb = __ballot(cross);
        // default: every candidate (their masses fall short of need)
        const int needed = cb != 0ull ? static_cast<int>(readlane_u32(static_cast<uint32_t>(rank), first_lane(cb))) + 1
                                      : total;
        const uint64_t tm = __ballot(live && rank < needed);
        if (lane == 0) {
          sh.sel.tmask = tm;
          sh.ires[0] = needed;
        }
      }
      __syncthreads();
      const uint64_t tm = sh.sel.tmask;
      const int needed = sh.ires[0];
      int cpos = first;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const bool c = (cand >> j) & 1u;
        taken |= (c && ((tm >> cpos) & 1ull)) ? (1u << j) : 0u;
        cpos += c ? 1 : 0;
      }
      count += needed;
      break;
    }
    if (ccount <= kExactMax) {
      // exact: rank the candidates (key desc, index asc) and walk their
      // masses in rank order; slot t's rank goes to sel.selbits[t]
      int total;
      const int first = block_excl_scan<NT>(__popc(cand), sh.sel.scan, &total);
      int slot = first;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((cand >> j) & 1u) {
          sh.sel.ckey[slot] = key[j];
          sh.sel.cidx[slot] = i0 + j;
          sh.cmass[slot] = mass[j];
          ++slot;
        }
      }
      if (tid == 0) sh.ires[0] = total;  // default: every candidate
      __syncthreads();
      if (tid < total) {
        const uint32_t mk = sh.sel.ckey[tid];
        const int mi = sh.sel.cidx[tid];
        uint64_t before = 0;
        int rank = 0;
        for (int m = 0; m < total; ++m) {
          const uint32_t km = sh.sel.ckey[m];
          const int im = sh.sel.cidx[m];
          const bool ahead = km > mk || (km == mk && im < mi);
          before += ahead ? sh.cmass[m] : 0ull;
          rank += ahead ? 1 : 0;
        }
        sh.sel.selbits[tid] = static_cast<uint32_t>(rank);
        if (before < need && need <= before + sh.cmass[tid]) sh.ires[0] = rank + 1;
      }
      __syncthreads();
      const int needed = sh.ires[0];
      slot = first;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((cand >> j) & 1u) {
          taken |= static_cast<int>(sh.sel.selbits[slot]) < needed ? (1u << j) : 0u;
          ++slot;
        }
      }
      count += needed;
      break;
    }
    uint32_t cmax = kmax0, cmin = kmin0;
    if (level > 0) {
      cmax = 0u;
      cmin = 0xffffffffu;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const bool c = (cand >> j) & 1u;
        cmax = (c && key[j] > cmax) ? key[j] : cmax;
        cmin = (c && key[j] < cmin) ? key[j] : cmin;
      }
      cmax = wave_max_u32(cmax);
      cmin = wave_min_u32(cmin);
      if (lane == 0) {
        sh.sel.red_max[wave] = cmax;
        sh.sel.red_min[wave] = cmin;
      }
      __syncthreads();
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        cmax = sh.sel.red_max[w] > cmax ? sh.sel.red_max[w] : cmax;
        cmin = sh.sel.red_min[w] < cmin ? sh.sel.red_min[w] : cmin;
      }
    }
    if (cmax == cmin) {
      // equal keys carry equal masses: take ceil(need / m), lowest index first
      uint64_t m = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j) m = ((cand >> j) & 1u) ? mass[j] : m;
      if (lane == 0) sh.red64[wave] = 0;
      __syncthreads();
      if (m != 0) atomicMax(&sh.red64[wave], static_cast<unsigned long long>(m));
      __syncthreads();
      uint64_t mm = 0;
#pragma unroll
      for (int w = 0; w < kW; ++w) mm = sh.red64[w] > mm ? sh.red64[w] : mm;
      const int needed = mm == 0 ? ccount : static_cast<int>((need + mm - 1) / mm);
      int total;
      int before = block_excl_scan<NT>(__popc(cand), sh.sel.scan, &total);
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        if ((cand >> j) & 1u) {
          taken |= before < needed ? (1u << j) : 0u;
          ++before;
        }
      }
      count += needed < total ? needed : total;
      break;
    }
    BinFn fn;
    const float vmin = key_value(cmin);
    const float vmax = key_value(cmax);
    const float range = vmax - vmin;
    fn.vmin = vmin;
    fn.scale = static_cast<float>(kLinBins) / range;
    fn.linear = level < 3 && __builtin_isfinite(vmin) && __builtin_isfinite(vmax) && __builtin_isfinite(range) &&
                range > 0.0f && __builtin_isfinite(fn.scale);
    const int hi = 31 - __clz(static_cast<int>(cmax ^ cmin));
    fn.shift = hi >= 7 ? hi - 7 : 0;
    if (level > 0) {
      for (int b = tid; b < kLinBins + 64; b += NT) {
        sh.sel.hist[b] = 0u;
        sh.bin_mass[b] = 0ull;
      }
      __syncthreads();
    }
    int bin[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      bin[j] = fn(key[j]);
      if ((cand >> j) & 1u) {
        atomicAdd(&sh.sel.hist[bin[j]], 1u);
        if (mass[j] != 0) atomicAdd(&sh.bin_mass[bin[j]], static_cast<unsigned long long>(mass[j]));
      }
    }
    __syncthreads();
    // thread t owns bins kBpt t .. kBpt t + kBpt - 1 (linear) or bin t
    // (digit), read once into registers
    constexpr int kBpt = kLinBins / NT;
    static_assert(kBpt == 2 || kBpt == 4 || kBpt == 8, "whole 8-byte or 16-byte bin reads per thread");
    uint32_t hc[kBpt];
    uint64_t hm[kBpt];
    if (fn.linear) {
      if constexpr (kBpt == 2) {
        const uint2 c0 = reinterpret_cast<const uint2*>(sh.sel.hist)[tid];
        hc[0] = c0.x; hc[1] = c0.y;
      } else {
#pragma unroll
        for (int q = 0; q < kBpt / 4; ++q) {
          const uint4 c = reinterpret_cast<const uint4*>(sh.sel.hist)[kBpt / 4 * tid + q];
          hc[4 * q] = c.x; hc[4 * q + 1] = c.y; hc[4 * q + 2] = c.z; hc[4 * q + 3] = c.w;
        }
      }
#pragma unroll
      for (int q = 0; q < kBpt / 2; ++q) {
        const ulonglong2 m2 = reinterpret_cast<const ulonglong2*>(sh.bin_mass)[kBpt / 2 * tid + q];
        hm[2 * q] = m2.x;
        hm[2 * q + 1] = m2.y;
      }
    } else {
      hc[0] = sh.sel.hist[tid];
      hm[0] = sh.bin_mass[tid];
#pragma unroll
      for (int b = 1; b < kBpt; ++b) {
        hc[b] = 0u;
        hm[b] = 0ull;
      }
    }
    uint64_t tmass = 0;
    uint32_t tcnt = 0;
#pragma unroll
    for (int b = 0; b < kBpt; ++b) {
      tmass += hm[b];
      tcnt += hc[b];
    }
    // suffix sums over threads (bins descending): masses and counts
    const uint64_t wm = wave_suffix_u64(tmass);
    const uint32_t wc = wave_suffix_sum_u32(tcnt);
    if (lane == 0) {
      sh.red64[wave] = wm;
      sh.sel.scan[wave] = static_cast<int>(wc);
    }
    __syncthreads();
    uint64_t incl = wm;
    uint32_t incl_c = wc;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      incl += w > wave ? sh.red64[w] : 0ull;
      incl_c += w > wave ? static_cast<uint32_t>(sh.sel.scan[w]) : 0u;
    }
    if (incl - tmass < need && need <= incl) {
      uint64_t acc = incl - tmass;
      uint32_t acc_c = incl_c - tcnt;
      int bsel = 0;
      uint32_t cnt = 0u;
      bool found = false;
#pragma unroll
      for (int b = kBpt - 1; b >= 0; --b) {
        const bool hit = !found && need <= acc + hm[b];
        bsel = hit ? b : bsel;
        cnt = hit ? hc[b] : cnt;
        acc += (found || hit) ? 0ull : hm[b];
        acc_c += (found || hit) ? 0u : hc[b];
        found = found || hit;
      }
      sh.sel.bnd = fn.linear ? kBpt * tid + bsel : tid;
      sh.lres[0] = acc;
      sh.sel.bnd_above = acc_c;
      sh.sel.bnd_count = cnt;
    }
    __syncthreads();
    const int bnd = sh.sel.bnd;
    need -= sh.lres[0];
    count += static_cast<int>(sh.sel.bnd_above);
    ccount = static_cast<int>(sh.sel.bnd_count);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool c = (cand >> j) & 1u;
      taken |= (c && bin[j] > bnd) ? (1u << j) : 0u;
      cand &= (c && bin[j] == bnd) ? 0xffffffffu : ~(1u << j);
    }
  }
  *taken_out = taken;
  return count;
}

// Matched budgets of one group (matched_budget_counts, twilight_offload_cache
// .py:50-86): every head keeps one, the rest of target is split in proportion
// to desired in float64, floors first, then +1 by (fractional remainder desc,
// desired desc, index asc); any excess is taken from the heads with the
// smallest (desired, index).  capacity: the candidate count of every head.
// One wavefront forms it, lane i for head i of R <= 64 (every lane active,
// desired[i] >= 1 read by lane i), and every lane gets its own head's count
// (0 past R).  The serial +1 loop is taken in batches with the same outcome:
// a head with a positive remainder is picked at most once (its remainder is
// then 0), and once the best remaining key has remainder 0 every key has, so
// that head takes +1 until it reaches capacity or the target; the excess is
// taken from the same smallest head until it keeps one.  At most 3R rounds.
__device__ int wave_matched_counts(const int32_t* desired, int R, int target, int capacity) {
  const int lane = lane_id();
  const bool live = lane < R;
  const int d = live ? desired[lane] : 0;
  // the counts are integers below 2^53, so their float64 sum is exact in any order
  const double total = static_cast<double>(static_cast<int64_t>(wave_sum_i32(d)));
  const int remaining = target - R;
  double raw = live ? static_cast<double>(remaining) * static_cast<double>(d) / total : 0.0;
  int cnt = 0;
  if (live) {
    const double fl = floor(raw);
    cnt = 1 + (fl < static_cast<double>(capacity - 1) ? static_cast<int>(fl) : capacity - 1);
  }
  int sum = wave_sum_i32(cnt);
  while (sum < target) {  // wave-uniform
    const double fl = floor(raw);
    // remainders are >= +0, so their bits order them; +1 keeps a 0 remainder
    // of an eligible head above the ineligible heads' key 0
    const uint64_t key = (live && cnt < capacity) ? static_cast<uint64_t>(__double_as_longlong(raw - fl)) + 1ull : 0ull;
    const uint32_t khi = static_cast<uint32_t>(key >> 32), klo = static_cast<uint32_t>(key);
    const uint32_t mhi = wave_max_u32(khi);
    const uint32_t mlo = wave_max_u32(khi == mhi ? klo : 0u);
    if (mhi == 0u && mlo == 0u) break;  // every head at capacity
    const bool top = khi == mhi && klo == mlo;
    const uint32_t md = wave_max_u32(top ? static_cast<uint32_t>(d) : 0u);
    const int best = first_lane(__ballot(top && static_cast<uint32_t>(d) == md));
    const bool positive = mhi != 0u || mlo > 1u;  // the best remainder is above 0
    const int cb = static_cast<int>(readlane_u32(static_cast<uint32_t>(cnt), best));
    const int room = target - sum < capacity - cb ? target - sum : capacity - cb;
    const int add = positive ? 1 : room;
    if (lane == best) {
      cnt += add;
      raw = fl;
    }
    sum += add;
  }
  while (sum > target) {
    const uint32_t key = (live && cnt > 1) ? static_cast<uint32_t>(d) : 0xffffffffu;
    const uint32_t mk = wave_min_u32(key);
    if (mk == 0xffffffffu) break;  // every head keeps one
    const int worst = first_lane(__ballot(key == mk));
    const int cw = static_cast<int>(readlane_u32(static_cast<uint32_t>(cnt), worst));
    const int sub = sum - target < cw - 1 ? sum - target : cw - 1;
    if (lane == worst) cnt -= sub;
    sum -= sub;
  }
  return cnt;
}

// Bits of [a, b) within the 32-position word starting at lo.
__device__ __forceinline__ uint32_t range_bits(int lo, int a, int b) {
  const int s = a - lo < 0 ? 0 : (a - lo > 32 ? 32 : a - lo);
  const int e = b - lo < 0 ? 0 : (b - lo > 32 ? 32 : b - lo);
  const uint32_t below_e = e >= 32 ? 0xffffffffu : ((1u << e) - 1u);
  const uint32_t below_s = s >= 32 ? 0xffffffffu : ((1u << s) - 1u);
  return below_e & ~below_s;
}

// Dynamic LDS of the selection kernels: the union bitmap (one bit per
// position, padded to 16 bytes), then a staging area shared by the logits
// load (N floats) and the union compaction (2 * kBlock words = 16384
// positions of rows per window, then 64 dummy slots).  Whatever the block
// size, a window is 512 words and its first 256 threads hold two each.
constexpr int kUnionWindowWords = 512;
__host__ __device__ __forceinline__ int union_words(int length) { return (length + 31) / 32; }
__host__ __device__ __forceinline__ int stage_offset_words(int length) { return (union_words(length) + 4 + 3) & ~3; }
__host__ __device__ __forceinline__ int stage_elems(int N, int length) {
  (void)length;
  const int rows = kUnionWindowWords * 32 + kWave + 4;  // a full window, the dummy slots, an alignment shift
  const int n = (N + 3) & ~3;
  return n > rows ? n : rows;
}

// Rows of the set bits of cb (cw words) in ascending bit order, written to
// rows[total ...]; pos(c) is the token position of bit c.  Windows of
// 2 * kBlock words: thread t holds words w0 + 2t and w0 + 2t + 1 and the
// block scan gives it its first row.  Every wavefront then walks its 64
// threads: at step k all lanes take lane k's two words, lane j keeps bit j
// and, if set, puts its position in the LDS stage at lane k's first row plus
// the set bits below j (mbcnt); clear lanes write a dummy slot past the
// window, so the 64 steps have no branch.  The window's rows leave with
// full, contiguous stores.  Returns the new total.
template <int NT, typename PosFn>
__device__ int expand_bits(const uint32_t* cb, int cw, int32_t* stage, int32_t* rows, int total, int* scan,
                           PosFn pos) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const bool lo_half = lane < 32;
  const int sh = lane & 31;
  const int dummy = kUnionWindowWords * 32 + lane;
  for (int w0 = 0; w0 < cw; w0 += kUnionWindowWords) {
    const int w = w0 + 2 * tid;
    const bool holds = 2 * tid < kUnionWindowWords;
    const uint32_t v0 = holds && w < cw ? cb[w] : 0u;
    const uint32_t v1 = holds && w + 1 < cw ? cb[w + 1] : 0u;
    int n_win;
    const int first = block_excl_scan<NT>(__popc(v0) + __popc(v1), scan, &n_win);
    const int c_wave = 32 * (w0 + 2 * kWave * wave) + lane;
#pragma unroll
    for (int k = 0; k < kWave; ++k) {
      const uint32_t a = readlane_u32(v0, k);
      const uint32_t b = readlane_u32(v1, k);
      const int base = static_cast<int>(readlane_u32(static_cast<uint32_t>(first), k));
      const uint32_t rank = __builtin_amdgcn_mbcnt_hi(b, __builtin_amdgcn_mbcnt_lo(a, 0u));
      const uint32_t mine = ((lo_half ? a : b) >> sh) & 1u;
      stage[mine ? base + static_cast<int>(rank) : dummy] = pos(c_wave + 64 * k);
    }
    __syncthreads();
    for (int i = tid; i < n_win; i += 4 * NT) {
      int32_t r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = i + u * NT < n_win ? stage[i + u * NT] : 0;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i + u * NT < n_win) rows[total + i + u * NT] = r[u];
    }
    total += n_win;
    __syncthreads();  // the next window reuses the stage
  }
  return total;
}

// The last block of group g: token union of the R selections plus the sink
// and recent windows, compacted ascending into the group's row list.
// scratch_a (kLinBins + 64 words) and scratch_b (2 * (kLinBins + 64) words)
// are free block-shared memory.
template <int NT>
__device__ void build_token_union(const SelectArgs& s, int g, uint32_t* bits, int32_t* stage, int* scan,
                                  uint32_t* scratch_a, int32_t* scratch_b) {
  const int tid = threadIdx.x;
  const int length = group_length(s, g);
  const int sink_end = s.sink < length ? s.sink : length;
  const int hist_recent = s.recent - 1 > 0 ? s.recent - 1 : 0;
  const int recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
  const int words = (length + 31) / 32;
  int32_t* rows = s.rows + static_cast<int64_t>(g) * s.rows_stride;
  // Page by page: the bs candidates of head r's page pi are bits
  // [pi*bs, pi*bs + bs) of its selection and positions sink + page*bs + [0, bs)
  // of the union, so one page moves as one shifted bit field.  Four pages per
  // thread are fetched before any is used (one round trip per 1024 pages);
  // the first batch is in flight while the path is chosen.
  const int n_words = s.words_n;
  const int bs = s.bs;
  const int total_pages = s.R * s.b0;
  int page[4], n0[4];
  uint32_t lo[4], hi[4];
  bool act[4];
  auto fetch = [&](int base) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = base + j * NT + tid;
      act[j] = idx < total_pages;
      const int ii = act[j] ? idx : 0;
      const int r = ii / s.b0;
      const int pi = ii - r * s.b0;
      page[j] = __hip_atomic_load(s.sel_pages + (static_cast<int64_t>(g) * s.R + r) * s.b0 + pi, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      n0[j] = pi * bs;
      const uint32_t* sb = s.selbits + (static_cast<int64_t>(g) * s.R + r) * n_words;
      const int w0 = n0[j] >> 5;
      const int w1 = (n0[j] + (bs < 32 ? bs : 32) - 1) >> 5;
      lo[j] = __hip_atomic_load(sb + w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      hi[j] = __hip_atomic_load(sb + (w1 < n_words ? w1 : w0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  auto page_mask = [&](int j) -> uint32_t {
    const uint64_t both = (static_cast<uint64_t>(hi[j]) << 32) | lo[j];
    return static_cast<uint32_t>(both >> (n0[j] & 31)) & (bs == 32 ? 0xffffffffu : ((1u << bs) - 1u));
  };
  if (total_pages > 0) fetch(0);

  // ---- page path: pages of a power-of-two size <= 32, one fetch batch, every
  // selected page between the sink and the recent window.  The union pages
  // are ranked through a page bitmap (union page u = rank of its page id) and
  // their head masks ORed into umask[u]; a scan over the union pages gives
  // each page its first row, and one thread per union page writes its set
  // offsets (through the LDS stage: at most one window of rows).
  const int n_pages = recent_start > s.sink ? (recent_start - s.sink) / bs : 0;  // pages below the recent window
  const int pbw = (n_pages + 31) / 32;
  const bool pow2 = bs > 0 && (bs & (bs - 1)) == 0 && bs <= 32;
  constexpr int kScratchB = 2 * (kLinBins + 64);
  if (pow2 && total_pages <= 4 * NT && 2 * pbw <= kLinBins + 64 && 3 * total_pages <= kScratchB &&
      total_pages * bs <= kUnionWindowWords * 32) {
    uint32_t m[4];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m[j] = act[j] ? page_mask(j) : 0u;
      // a selected page outside [sink, recent_start) would overlap a window
      bad = bad || (m[j] != 0u && (page[j] < 0 || page[j] >= n_pages));
    }
    uint32_t* pb = scratch_a;
    int* pfx = reinterpret_cast<int*>(scratch_a + pbw);
    const int u_cap = total_pages < n_pages ? total_pages : n_pages;
    int32_t* upage = scratch_b;
    uint32_t* umask = reinterpret_cast<uint32_t*>(scratch_b + u_cap);
    int32_t* ubase = scratch_b + 2 * u_cap;
    for (int w = tid; w < pbw; w += NT) pb[w] = 0u;
    for (int u = tid; u < u_cap; u += NT) umask[u] = 0u;
    if (__syncthreads_or(bad ? 1 : 0) == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (m[j] != 0u) atomicOr(&pb[page[j] >> 5], 1u << (page[j] & 31));
      __syncthreads();
      int U = 0;
      for (int w0 = 0; w0 < pbw; w0 += NT) {
        const int w = w0 + tid;
        int tot;
        const int ex = block_excl_scan<NT>(w < pbw ? __popc(pb[w]) : 0, scan, &tot);
        if (w < pbw) pfx[w] = U + ex;
        U += tot;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (m[j] != 0u) {
          const int p = page[j];
          const int u = pfx[p >> 5] + __popc(pb[p >> 5] & ((1u << (p & 31)) - 1u));
          atomicOr(&umask[u], m[j]);
          upage[u] = p;
        }
      }
      // sink rows meanwhile
      for (int i = tid; i < sink_end; i += NT) rows[i] = i;
      __syncthreads();
      // first row of every union page: thread t sums union pages 4t .. 4t + 3
      int union_rows;
      {
        int c[4], sum = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int u = 4 * tid + q;
          c[q] = u < U ? __popc(umask[u]) : 0;
          sum += c[q];
        }
        int acc = block_excl_scan<NT>(sum, scan, &union_rows);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int u = 4 * tid + q;
          if (u < U) ubase[u] = acc;
          acc += c[q];
        }
      }
      __syncthreads();
      // one thread per union page puts its set offsets, ascending, into the
      // LDS stage (scattered LDS stores are cheap; scattered global stores
      // are not), then the rows leave with full, contiguous stores
      const int lbs = __ffs(bs) - 1;
      const int sink = s.sink;
      // Branch-free: offsets are written in ascending order at the running
      // count k, so an unset offset's value is overwritten by the next set
      // one; offsets past the page's highest set bit go to a dummy slot.
      int32_t* urows = rows + sink_end;
      // the stage is shifted so that stage row i and urows[i] agree modulo
      // 16 bytes (vector copies below); the dummy slots follow the window
      const int lead = static_cast<int>((4u - ((reinterpret_cast<uintptr_t>(urows) >> 2) & 3u)) & 3u);
      int32_t* st = stage + ((4 - lead) & 3);
      const int dummy = kUnionWindowWords * 32 + lane_id();
      auto put_pages = [&](auto bs_c) {
        constexpr int kBs = decltype(bs_c)::value;
        for (int u = tid; u < U; u += NT) {
          const uint32_t mu = umask[u];  // non-zero: u is a union page
          const int hb = 31 - __clz(static_cast<int>(mu));
          const int b0 = ubase[u];
          const int v0 = sink + (upage[u] << lbs);
          int k = b0;
#pragma unroll
          for (int o = 0; o < (kBs > 0 ? kBs : 32); ++o) {
            if (kBs > 0 || o < bs) st[o <= hb ? k : dummy] = v0 + o;
            k += static_cast<int>((mu >> o) & 1u);
          }
        }
      };
      if (bs == 16)
        put_pages(std::integral_constant<int, 16>{});
      else
        put_pages(std::integral_constant<int, 0>{});
      __syncthreads();
      // rows [0, lead) and the tail one by one, the rest as 16-byte copies,
      // four per thread in flight
      const int n4 = union_rows > lead ? (union_rows - lead) >> 2 : 0;
      const int4* src4 = reinterpret_cast<const int4*>(st + lead);
      int4* dst4 = reinterpret_cast<int4*>(urows + lead);
      for (int i = tid; i < n4; i += 4 * NT) {
        int4 r[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = src4[i + q * NT < n4 ? i + q * NT : i];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (i + q * NT < n4) dst4[i + q * NT] = r[q];
      }
      if (tid < lead && tid < union_rows) urows[tid] = st[tid];
      {
        const int i = lead + 4 * n4 + tid;
        if (tid < 4 && i < union_rows) urows[i] = st[i];
      }
      int total = sink_end + union_rows;
      const int n_recent = length - recent_start;
      for (int i = tid; i < n_recent; i += NT) rows[total + i] = recent_start + i;
      total += n_recent;
      const int count = total + (s.append_position >= 0 ? 1 : 0);
      if (tid == 0) {
        if (s.append_position >= 0) rows[total] = s.append_position;
        s.row_counts[g] = count;
      }
      return;
    }
  }

  // ---- bitmap path: one bit per position of [0, length)
  for (int w = tid; w < words; w += NT) {
    const int lo_pos = 32 * w;
    bits[w] = range_bits(lo_pos, 0, sink_end) | range_bits(lo_pos, recent_start, length);
  }
  __syncthreads();
  for (int base = 0; base < total_pages; base += 4 * NT) {
    if (base > 0) fetch(base);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!act[j]) continue;
      const int64_t pos0 = static_cast<int64_t>(s.sink) + static_cast<int64_t>(page[j]) * bs;
      if (bs <= 32) {
        const uint32_t m = page_mask(j);
        if (m == 0u || pos0 < 0 || pos0 + bs > length) continue;
        const uint64_t field = static_cast<uint64_t>(m) << (pos0 & 31);
        atomicOr(&bits[pos0 >> 5], static_cast<uint32_t>(field));
        if (static_cast<uint32_t>(field >> 32) != 0u) atomicOr(&bits[(pos0 >> 5) + 1], static_cast<uint32_t>(field >> 32));
      } else {
        // pages wider than a word: bit by bit
        const int r = (base + j * NT + tid) / s.b0;
        const uint32_t* sb = s.selbits + (static_cast<int64_t>(g) * s.R + r) * n_words;
        for (int i = 0; i < bs; ++i) {
          const int n = n0[j] + i;
          const uint32_t v = __hip_atomic_load(sb + (n >> 5), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const int64_t pos = pos0 + i;
          if (((v >> (n & 31)) & 1u) && pos >= 0 && pos < length) atomicOr(&bits[pos >> 5], 1u << (pos & 31));
        }
      }
    }
  }
  __syncthreads();
  const int total = expand_bits<NT>(bits, words, stage, rows, 0, scan, [](int c) { return c; });
  const int count = total + (s.append_position >= 0 ? 1 : 0);
  if (tid == 0) {
    if (s.append_position >= 0) rows[total] = s.append_position;
    s.row_counts[g] = count;
  }
}

// Fast path of block_top_mass for a row whose key range [kmin, kmax] is
// known, with the top-p threshold found on the way: one pass of kFastBins
// bins linear in the value over that range accumulates each bin's count and
// integer mass (the caller has cleared both and the staging counter); the
// first wavefront then reads all bins (8 per lane), takes the total mass Z
// and the threshold need = ceil(p24 * Z / 2^24) from them, and finds the bin
// where the mass of the bins above it falls short of need and with it
// reaches it.  At most 64 keys of that bin are staged, and the first
// wavefront ranks them by (key desc, index asc), summing the masses ranked
// ahead of each: the key whose own mass crosses the rest of need ends the
// selection.  Work that is the same for the whole row runs in one wavefront
// (the others wait at the barrier that hands its result over), since the
// block's wavefronts would otherwise issue it twice on each SIMD.  Four
// barriers.  Returns false -- block-uniformly, with the bins dirty -- when the
// range is not finite and positive, need is 0 (no mass or p24 = 0) or the
// boundary bin holds more than 64 keys; on true, *taken and *count are what
// block_top_mass gives for that need.
template <int KPT, int NT>
__device__ bool block_top_p_fast(const uint32_t (&key)[KPT], const uint64_t (&mass)[KPT], int N, uint32_t p24,
                                 uint32_t kmin, uint32_t kmax, TopShared<NT>& sh, uint32_t* taken_out,
                                 int* count_out) {
  constexpr int kBins = kFastBins;
  constexpr int kBpl = kBins / kWave;  // bins per lane
  static_assert(kBpl % 8 == 0, "whole 16-byte count and mass reads per lane");
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const bool first_wave = tid < kWave;
  const int i0 = KPT * tid;
  const float vmin = key_value(kmin);
  const float vmax = key_value(kmax);
  const float range = vmax - vmin;
  const float scale = static_cast<float>(kBins) / range;
  if (!(__builtin_isfinite(vmin) && __builtin_isfinite(vmax) && __builtin_isfinite(range) && range > 0.0f &&
        __builtin_isfinite(scale)))
    return false;
  int bin[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int b = static_cast<int>((key_value(key[j]) - vmin) * scale);
    bin[j] = (i0 + j < N) ? (b < kBins - 1 ? b : kBins - 1) : -1;
  }
  // no branch: keys past the row count into bin kBins, which nothing reads
  // (the bins hold kLinBins + 64 > kBins entries)
  static_assert(kBins < kLinBins + 64, "a spare bin");
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int b = bin[j] >= 0 ? bin[j] : kBins;
    atomicAdd(&sh.sel.hist[b], 1u);
    atomicAdd(&sh.bin_mass[b], static_cast<unsigned long long>(mass[j]));
  }
  __syncthreads();
  if (first_wave) {
    uint32_t hc[kBpl];
    uint64_t hm[kBpl];
    {
      const uint4* c4 = reinterpret_cast<const uint4*>(sh.sel.hist) + (kBpl / 4) * lane;
#pragma unroll
      for (int q = 0; q < kBpl / 4; ++q) {
        const uint4 v = c4[q];
        hc[4 * q] = v.x;
        hc[4 * q + 1] = v.y;
        hc[4 * q + 2] = v.z;
        hc[4 * q + 3] = v.w;
      }
      const ulonglong2* m2 = reinterpret_cast<const ulonglong2*>(sh.bin_mass) + (kBpl / 2) * lane;
#pragma unroll
      for (int q = 0; q < kBpl / 2; ++q) {
        const ulonglong2 v = m2[q];
        hm[2 * q] = v.x;
        hm[2 * q + 1] = v.y;
      }
    }
    uint64_t tm = 0;
    uint32_t tc = 0u;
#pragma unroll
    for (int b = 0; b < kBpl; ++b) {
      tm += hm[b];
      tc += hc[b];
    }
    const uint64_t pm = wave_prefix_sum_u64(tm);
    const uint64_t z = (static_cast<uint64_t>(readlane_u32(static_cast<uint32_t>(pm >> 32), kWave - 1)) << 32) |
                       readlane_u32(static_cast<uint32_t>(pm), kWave - 1);
    const uint64_t sm = z - pm + tm;  // mass of the bins of lanes >= this one
    const uint32_t sc = wave_suffix_sum_u32(tc);
    const uint64_t need = top_p_threshold(p24, z);
    // lanes 0 .. L have a suffix mass >= need (need == 0: any lane; unused)
    const uint64_t bl = __ballot(sm >= need);
    const int L = 63 - __clzll(static_cast<long long>(bl));
    uint64_t acc = sm - tm;     // mass of the bins above this lane's
    uint32_t cacc = sc - tc;    // and their keys
    int bsel = 0;
    uint32_t cnt = 0u;
    bool found = false;
#pragma unroll
    for (int b = kBpl - 1; b >= 0; --b) {
      const bool hit = !found && need <= acc + hm[b];
      bsel = hit ? b : bsel;
      cnt = hit ? hc[b] : cnt;
      acc += (found || hit) ? 0ull : hm[b];
      cacc += (found || hit) ? 0u : hc[b];
      found = found || hit;
    }
    const int bnd = kBpl * L + static_cast<int>(readlane_u32(static_cast<uint32_t>(bsel), L));
    const uint64_t above = (static_cast<uint64_t>(readlane_u32(static_cast<uint32_t>(acc >> 32), L)) << 32) |
                           readlane_u32(static_cast<uint32_t>(acc), L);
    // (lane reads ahead of the lane-0 branch: inside it, the compiler could
    // compute the per-lane values for lane 0 alone)
    const uint32_t c_above = readlane_u32(cacc, L);
    const uint32_t ccount = readlane_u32(cnt, L);
    if (lane == 0) {
      sh.fp_l[0] = need;
      sh.fp_l[1] = above;
      sh.fp_i[0] = bnd;
      sh.fp_i[1] = static_cast<int>(c_above);
      sh.fp_i[2] = static_cast<int>(ccount);
    }
  }
  __syncthreads();  // (the first wavefront is also done with the bins)
  const uint64_t need = sh.fp_l[0];
  const uint64_t above = sh.fp_l[1];
  const int bnd = sh.fp_i[0];
  const uint32_t c_above = static_cast<uint32_t>(sh.fp_i[1]);
  const uint32_t ccount = static_cast<uint32_t>(sh.fp_i[2]);
  if (need == 0 || ccount > static_cast<uint32_t>(kWave)) return false;
  const uint64_t need2 = need - above;  // 1 .. the bin's mass
  uint32_t t = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) t |= (bin[j] > bnd) ? (1u << j) : 0u;
  uint32_t inbin = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) inbin |= (bin[j] == bnd) ? (1u << j) : 0u;
  uint32_t cslot[KPT];
  {
    uint32_t slot = stage_slots(inbin, &sh.sel.ncand);
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      cslot[j] = slot;
      if ((inbin >> j) & 1u) {
        sh.sel.cpair[slot] = rank_key(key[j], i0 + j);
        sh.cmass[slot] = mass[j];
      }
      slot += (inbin >> j) & 1u;
    }
  }
  __syncthreads();
  if (first_wave) {
    // lane m ranks staged key m against all of them, read from LDS by every
    // lane at once (broadcast reads, four in flight): one 64-bit compare
    // each, no branch (slots past ccount hold key 0, which never outranks a
    // key, so their stale masses never count)
    const bool live = static_cast<uint32_t>(lane) < ccount;
    const unsigned long long c = sh.sel.cpair[lane];
    const uint64_t cm = live ? static_cast<uint64_t>(sh.cmass[lane]) : 0ull;
    uint64_t before = 0;
    uint32_t rank = 0u;
    for (int m = 0; m < static_cast<int>(ccount); m += 4) {
      unsigned long long o[4];
      uint64_t om[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        o[u] = sh.sel.cpair[m + u];
        om[u] = sh.cmass[m + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool ahead = o[u] > c;
        before += ahead ? om[u] : 0ull;
        rank += ahead ? 1u : 0u;
      }
    }
    const bool cross = live && before < need2 && need2 <= before + cm;
    const uint64_t cb = __ballot(cross);
    // (need2 <= the bin's mass, so some key crosses; all of them otherwise)
    const uint32_t needed = cb != 0ull ? readlane_u32(rank, first_lane(cb)) + 1u : ccount;
    const uint64_t tmk = __ballot(live && rank < needed);
    if (lane == 0) {
      sh.fp_l[0] = tmk;
      sh.fp_i[3] = static_cast<int>(needed);
    }
  }
  __syncthreads();
  const uint64_t tmk = sh.fp_l[0];
  const uint32_t needed = static_cast<uint32_t>(sh.fp_i[3]);
#pragma unroll
  for (int j = 0; j < KPT; ++j) t |= (((inbin >> j) & 1u) && ((tmk >> cslot[j]) & 1ull)) ? (1u << j) : 0u;
  *taken_out = t;
  *count_out = static_cast<int>(c_above + needed);
  return true;
}

// The row's logits as KPT contiguous keys per thread (16-byte loads of the
// thread's own logits; rows that are not 16-byte aligned go through the LDS
// stage); the largest logit and the smallest and largest key of the row in
// one block reduction.
template <int KPT, int NT>
__device__ __forceinline__ void load_logits(const float* row, int N, float* stage, uint32_t (&key)[KPT],
                                            float& lmax, uint32_t& kmin, uint32_t& kmax, TopShared<NT>& sh) {
  const int tid = static_cast<int>(threadIdx.x);
  const int i0 = KPT * tid;
  float mx = -INFINITY;
  uint32_t kmx = 0u, kmn = 0xffffffffu;
  if (N > 0 && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
    // the thread's KPT contiguous logits straight from memory, 16 bytes a load
    // (indices past the row read its last float4 and are masked below)
    float v[KPT];
    if constexpr (KPT >= 4) {
      const float4* r4 = reinterpret_cast<const float4*>(row);
      const int last4 = (N >> 2) - 1;
#pragma unroll
      for (int j = 0; j < KPT / 4; ++j) {
        const int i4 = (i0 >> 2) + j;
        const float4 t = r4[i4 < last4 ? i4 : last4];
        v[4 * j] = t.x;
        v[4 * j + 1] = t.y;
        v[4 * j + 2] = t.z;
        v[4 * j + 3] = t.w;
      }
    } else if constexpr (KPT == 2) {
      const float2* r2 = reinterpret_cast<const float2*>(row);
      const int last2 = (N >> 1) - 1;
      const int i2 = i0 >> 1;
      const float2 t = r2[i2 < last2 ? i2 : last2];
      v[0] = t.x;
      v[1] = t.y;
    } else {
      v[0] = row[i0 < N - 1 ? i0 : N - 1];
    }
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int i = i0 + j;
      key[j] = score_key(v[j]);
      mx = (i < N && v[j] > mx) ? v[j] : mx;
      kmx = (i < N && key[j] > kmx) ? key[j] : kmx;
      kmn = (i < N && key[j] < kmn) ? key[j] : kmn;
    }
  } else {
    for (int i = tid; i < N; i += NT) stage[i] = row[i];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int i = i0 + j;
      const float v = stage[i < N ? i : N - 1];
      key[j] = score_key(v);
      mx = (i < N && v > mx) ? v : mx;
      kmx = (i < N && key[j] > kmx) ? key[j] : kmx;
      kmn = (i < N && key[j] < kmn) ? key[j] : kmn;
    }
  }
  mx = wave_max_f32(mx);
  kmx = wave_max_u32(kmx);
  kmn = wave_min_u32(kmn);
  const int wave = tid / kWave;
  if (lane_id() == 0) {
    sh.fred[wave] = mx;
    sh.sel.red_max[wave] = kmx;
    sh.sel.red_min[wave] = kmn;
  }
  __syncthreads();
  lmax = sh.fred[0];
  kmax = sh.sel.red_max[0];
  kmin = sh.sel.red_min[0];
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) {
    lmax = fmaxf(lmax, sh.fred[w]);
    kmax = sh.sel.red_max[w] > kmax ? sh.sel.red_max[w] : kmax;
    kmin = sh.sel.red_min[w] < kmin ? sh.sel.red_min[w] : kmin;
  }
  __syncthreads();
}

// Publish this row's selection bits (bit n = candidate n selected): the
// 32 / KPT consecutive threads of a word OR their shifted bits together
// (lane shuffles within the wavefront) and the first of them stores the
// word; words past the block's keys are zero.
template <int KPT, int NT>
__device__ __forceinline__ void publish_selection(uint32_t* row_bits, int words, uint32_t taken, TopShared<NT>& sh) {
  (void)sh;
  const int tid = static_cast<int>(threadIdx.x);
  static_assert(KPT <= 32 && (32 % KPT) == 0, "whole threads per word");
  constexpr int kLpw = 32 / KPT;  // threads per word
  uint32_t w = KPT == 32 ? taken : (taken << ((tid % kLpw) * KPT));
#pragma unroll
  for (int o = 1; o < kLpw; o <<= 1) w |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(w), o));
  if (tid % kLpw == 0 && tid / kLpw < words)
    __hip_atomic_store(row_bits + tid / kLpw, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int i = NT / kLpw + tid; i < words; i += NT)
    __hip_atomic_store(row_bits + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage A: the top-p count of every (group, head) row; in dynamic mode also
// the selection and the group's token union.
template <int KPT, int NT>
__global__ __launch_bounds__(NT) void twilight_topp_kernel(SelectArgs s) {
  __shared__ __align__(16) TopShared<NT> sh;
  extern __shared__ __align__(16) uint32_t union_bits[];
  float* stage = reinterpret_cast<float*>(union_bits + stage_offset_words(s.length));
  const int row = blockIdx.x;
  const int g = row / s.R;
  const int N = group_candidates(s, g);  // valid candidates; logits rows are s.N apart
  // the first pass's histograms, cleared before load_logits' barrier
  for (int b = threadIdx.x; b < kLinBins + 64; b += NT) {
    sh.sel.hist[b] = 0u;
    sh.bin_mass[b] = 0ull;
  }
  if (N == 0) {
    // a ragged group with no candidate page: sink and recent windows only
    if (threadIdx.x == 0) {
      s.desired[row] = 0;
      if (s.allocated != nullptr) s.allocated[row] = 0;
    }
    if (s.page_rows != nullptr) return;  // no row of this head is kept
    publish_selection<KPT>(s.selbits + static_cast<int64_t>(row) * s.words_n, s.words_n, 0u, sh);
    if (!arrive_last(s.counters + g, static_cast<unsigned int>(s.R), &sh.sel.flag)) return;
    build_token_union<NT>(s, g, union_bits, reinterpret_cast<int32_t*>(stage), sh.sel.scan, sh.sel.hist,
                      reinterpret_cast<int32_t*>(sh.bin_mass));
    return;
  }
  uint32_t key[KPT];
  float lmax;
  uint32_t kmin, kmax;
  load_logits<KPT>(s.logits + static_cast<int64_t>(row) * s.N, N, stage, key, lmax, kmin, kmax, sh);
  uint64_t mass[KPT];
  uint64_t local = 0;
  const int i0 = KPT * static_cast<int>(threadIdx.x);
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    mass[j] = mass_of((i0 + j < N) ? key_value(key[j]) : -INFINITY, lmax);  // 0 past the row
    local += mass[j];
  }
  const uint64_t z = block_sum_u64<NT>(local, sh.red64);
  uint64_t need = top_p_threshold(s.p24, z);
  if (need == 0) {
    // no mass at all (non-finite logits): one key, the largest, as on the CPU
#pragma unroll
    for (int j = 0; j < KPT; ++j) mass[j] = (i0 + j < N) ? 1ull : 0ull;
    need = 1;
  }
  uint32_t taken;
  int desired = block_top_mass<KPT>(key, mass, N, need, kmin, kmax, sh, &taken);
  desired = desired < 1 ? 1 : (desired > N ? N : desired);
  if (threadIdx.x == 0) s.desired[row] = desired;
  if (s.matched) return;
  if (threadIdx.x == 0 && s.allocated != nullptr) s.allocated[row] = desired;
  if (s.page_rows != nullptr) {
    // the thread's KPT candidates lie in one B0 slot (bs % KPT == 0) or
    // cover KPT / bs whole slots (KPT % bs == 0), as the host checks: one OR
    // of their row bits into each such union page's mask
    const int c0 = KPT * static_cast<int>(threadIdx.x);
    const int span = KPT < s.bs ? KPT : s.bs;
    const uint32_t low = span >= 32 ? 0xffffffffu : ((1u << span) - 1u);
    for (int j = 0; j < KPT; j += span) {
      const uint32_t m = (taken >> j) & low;
      if (m != 0u) {  // set bits are candidates < N, so the slot is < b0
        const int slot = (c0 + j) / s.bs;
        const int u = s.slot_u[static_cast<int64_t>(row) * s.b0 + slot];
        atomicOr(s.page_rows + static_cast<int64_t>(g) * s.page_rows_stride + u, m << (c0 + j - slot * s.bs));
      }
    }
    return;
  }
  publish_selection<KPT>(s.selbits + static_cast<int64_t>(row) * s.words_n, s.words_n, taken, sh);
  if (!arrive_last(s.counters + g, static_cast<unsigned int>(s.R), &sh.sel.flag)) return;
  build_token_union<NT>(s, g, union_bits, reinterpret_cast<int32_t*>(stage), sh.sel.scan, sh.sel.hist,
                      reinterpret_cast<int32_t*>(sh.bin_mass));
}

// Stage B (matched budgets): allocation from the group's desired counts, the
// top-allocated selection of each head and the group's token union.
template <int KPT, int NT>
__global__ __launch_bounds__(NT) void twilight_matched_kernel(SelectArgs s) {
  __shared__ __align__(16) TopShared<NT> sh;
  extern __shared__ __align__(16) uint32_t union_bits[];
  const int row = blockIdx.x;
  const int g = row / s.R;
  const int r = row - g * s.R;
  const int N = s.N;
  if (s.given) {
    if (threadIdx.x == 0) sh.ires[1] = s.allocated[row];
  } else if (threadIdx.x < kWave) {  // the first wavefront, whole
    const int c = wave_matched_counts(s.desired + static_cast<int64_t>(g) * s.R, s.R, s.target_total, N);
    const int cr = static_cast<int>(readlane_u32(static_cast<uint32_t>(c), r));
    if (threadIdx.x == 0) sh.ires[1] = cr;
  }
  float* stage = reinterpret_cast<float*>(union_bits + stage_offset_words(s.length));
  uint32_t key[KPT];
  float lmax;
  uint32_t kmin, kmax;
  load_logits<KPT>(s.logits + static_cast<int64_t>(row) * N, N, stage, key, lmax, kmin, kmax, sh);  // (barriers)
  int k = sh.ires[1];
  k = k < 1 ? 1 : (k > N ? N : k);
  if (threadIdx.x == 0 && s.allocated != nullptr && !s.given) s.allocated[row] = k;
  uint32_t taken = 0u;
  int first_slot;  // (the selection is published as a bitmap)
  block_topk<KPT>(key, N, k, sh.sel, &taken, &first_slot);
  publish_selection<KPT>(s.selbits + static_cast<int64_t>(row) * s.words_n, s.words_n, taken, sh);
  if (!arrive_last(s.counters + g, static_cast<unsigned int>(s.R), &sh.sel.flag)) return;
  build_token_union<NT>(s, g, union_bits, reinterpret_cast<int32_t*>(stage), sh.sel.scan, sh.sel.hist,
                      reinterpret_cast<int32_t*>(sh.bin_mass));
}

// ------------------------------------------------ fused Twilight selection
// Two launches (three with matched budgets) select a whole layer.
//
// twilight_score_qk_kernel: block = (group g, tile of kSqTile pages), 512
// threads, over every page the launch scores.  It
//   1. scores the tile's pages for the group's R heads in the Quest order of
//      quest_score_kernel (32 accumulators over channels d mod 32, chunk by
//      chunk, then the adjacent-pair tree; every product an unfused fp32
//      multiply of the page's max or min by q_d), so the scores are the same
//      bits, and stores each head's per-tile key range for the top-k;
//   2. estimates the INT4 QK of every row of those pages for all R heads on
//      the matrix cores: v_mfma_i32_16x16x64_i8 with A row 4 h + t holding
//      slice t of head h's balanced fixed-point digits (rows 4 h + 3 zero; two
//      A tiles for R > 4) and B column n the codes of row n of one 16-row
//      page, so lane group h of the product holds head h's three slice dots
//      of row lane % 16 and forms the exact integer S in-lane (the integers
//      twilight_qk_kernel forms, hence the same logits); the logits go to a
//      per-head array indexed by row within the scored span.
// The INT4 rows are read once for all R heads, from every CU at once, while
// the B0 pages are still unknown: the scored span's rows rather than only
// the union of the heads' B0 candidates, so that no launch waits on a top-k
// before it reads them.  It also clears the group's union record.
//
// twilight_topp_head_kernel: block = one (group, head) row, 512 threads.  It
//   1. picks the head's B0 pages (the top b0 page scores: block top-k with the
//      one-pass fast path over the tile key ranges, the digit search when the
//      fast path gives up), ascending;
//   2. gathers the logits of those pages' rows (candidate n = row n % 16 of
//      the (n / 16)-th B0 page) and their max and key range (one block
//      reduction);
//   3. runs the top-p with dynamic budgets (the exact integer-mass rule of
//      twilight_topp_kernel);
//   4. ORs each page's kept rows into its 16-bit mask and the page's bit into
//      the group's page bitmap (global atomics into the cleared record; a
//      page whose rows no head keeps is not in the union).
// With matched budgets it stops after the top-p count and leaves the
// candidates' logits and key ranges for twilight_matched_rec_kernel.
// D = 128, 16-row pages, 16-bit keys.
constexpr int kHeadThreads = 512;
constexpr int kSqTile = 64;       // pages per block of the score + QK launch
constexpr int kSqThreads = 512;   // 8 wavefronts: two per head for the score, 8 pages each for the QK

struct ScoreQkArgs {
  const float* q;          // [G][R][128]
  const void* pmin;        // group g page p at + g * group_stride + p * 128
  const void* pmax;
  int64_t group_stride;
  int G, R, P;             // P: pages the launch scores (every group's P_g <= P)
  const int32_t* lengths;  // nullable: group g has lengths[g] tokens (its P_g from the windows)
  int sink, recent;
  const uint8_t* packed;   // entry g row t at + (g * qstride + t) * 64
  const void* scale;
  const void* minimum;
  int64_t qstride, qrows;
  float qk_scale;
  float* scores;           // [G * R][score_stride]
  int64_t score_stride;
  uint2* tile_mm;          // [G * R][tiles] (max, min) score key of a tile's pages
  float* logits;           // [G * R][logit_stride]: row sink + 16 p + i at 16 p + i
  int64_t logit_stride;
  uint32_t* rec;           // union records to clear, rec_stride words apart
  int64_t rec_stride;
  unsigned int* zero_counters;  // nullable: block 0 zeroes n_counters of them
  int n_counters;
};

template <typename DT, int RMAX>
__global__ __launch_bounds__(kSqThreads) void twilight_score_qk_kernel(ScoreQkArgs a) {
  using S = typename DT::storage;
  constexpr int D = 128;
  constexpr int BS = 16;
  constexpr int KW = D / 8;                      // code words of a row
  constexpr int kWv = kSqThreads / kWave;        // wavefronts
  constexpr int kPitch = D * 2 + 16;             // padded LDS row of page extrema (bytes)
  constexpr int kQuads = D * 2 / 16;             // 16-byte quads of a row of extrema
  constexpr int kMetaPer = 2 * kSqTile * kQuads / kSqThreads;
  constexpr int kPg = kSqTile / kWv;             // 16-row pages a wavefront estimates
  constexpr int HT = RMAX / 4;                   // A tiles of four heads
  typedef int v4i __attribute__((ext_vector_type(4)));
  static_assert(RMAX == 4 || RMAX == 8, "4 or 8 head slots");
  static_assert(kMetaPer * kSqThreads == 2 * kSqTile * kQuads && kPg * kWv == kSqTile, "tile shape");
  __shared__ __align__(16) uint8_t s_meta[2 * kSqTile * kPitch];
  __shared__ __align__(16) float s_qv[RMAX * D];
  __shared__ float s_half[RMAX][kWave];
  __shared__ __align__(16) uint32_t s_q[RMAX * 6 * KW];
  __shared__ int s_qshift[RMAX];
  __shared__ float s_qsum[RMAX];
  __shared__ int s_qok[RMAX];
  // group-minor: group g's blocks of every launch of the layer on XCD g % 8
  const int tiles = (a.P + kSqTile - 1) / kSqTile;
  const int g = static_cast<int>(blockIdx.x) % a.G;
  const int tile = static_cast<int>(blockIdx.x) / a.G;
  const int p0 = tile * kSqTile;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = wave_uniform(tid / kWave);
  const int R = a.R;
  const int np_cap = (a.P - p0) < kSqTile ? (a.P - p0) : kSqTile;

  // ---- round trip 1: the length, q, the tile's extrema and INT4 rows ----
  // (every load unconditional, indices clamped, so they issue back to back)
  const int length = *(a.lengths != nullptr ? a.lengths + g : reinterpret_cast<const int32_t*>(a.q));
  const int nq = R * D;
  const float* qg = a.q + static_cast<int64_t>(g) * nq;
  const float qv0 = qg[tid < nq ? tid : nq - 1];
  const float qv1 = qg[tid + kSqThreads < nq ? tid + kSqThreads : nq - 1];
  QStage<D, RMAX> qst;
  qst.load(qg, R);
  const S* mn = static_cast<const S*>(a.pmin) + g * a.group_stride + static_cast<int64_t>(p0) * D;
  const S* mx = static_cast<const S*>(a.pmax) + g * a.group_stride + static_cast<int64_t>(p0) * D;
  const int meta_last = 2 * np_cap * kQuads - 1;
  uint4 mv[kMetaPer];
#pragma unroll
  for (int j = 0; j < kMetaPer; ++j) {
    int i = tid + j * kSqThreads;
    i = i < meta_last ? i : meta_last;
    const bool hi = i >= np_cap * kQuads;
    const int rem = i - (hi ? np_cap * kQuads : 0);
    mv[j] = load_stream(reinterpret_cast<const uint4*>(hi ? mx : mn) + rem);
  }
  const int G4 = lane / 16;
  const int n = lane % 16;
  const uint8_t* pk = a.packed + static_cast<int64_t>(g) * a.qstride * (D / 2);
  const S* scl = static_cast<const S*>(a.scale) + static_cast<int64_t>(g) * a.qstride;
  const S* mnq = static_cast<const S*>(a.minimum) + static_cast<int64_t>(g) * a.qstride;
  uint4 cw[kPg];
  S sv[kPg], mq[kPg];
#pragma unroll
  for (int i = 0; i < kPg; ++i) {
    const int pl = wave + kWv * i;
    int64_t t = static_cast<int64_t>(a.sink) + static_cast<int64_t>(p0 + (pl < np_cap ? pl : np_cap - 1)) * BS + n;
    t = (t >= 0 && t < a.qrows) ? t : 0;
    cw[i] = load_stream(pk + t * (D / 2) + 16 * G4);
    sv[i] = scl[t];
    mq[i] = mnq[t];
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- the launch's bookkeeping: the group's union record, the counters ----
  if (a.zero_counters != nullptr && g == 0 && tile == 0) {
    for (int i = tid; i < a.n_counters; i += kSqThreads) a.zero_counters[i] = 0u;
  }
  if (a.rec != nullptr) {
    // bitmap words 2 tile and 2 tile + 1, mask words [32 tile, 32 tile + 32)
    uint32_t* rec = a.rec + g * a.rec_stride;
    const int mw = (p0 >> 1) + tid - 2;
    if (tid < 2)
      rec[2 * tile + tid] = 0u;
    else if (tid < 2 + kSqTile / 2 && mw < union_mask_words(a.P))
      rec[union_mask_offset(a.P) + mw] = 0u;
  }
  // ---- extrema and q to LDS, q in fixed point ----
#pragma unroll
  for (int j = 0; j < kMetaPer; ++j) {
    int i = tid + j * kSqThreads;
    i = i < meta_last ? i : meta_last;
    const bool hi = i >= np_cap * kQuads;
    const int rem = i - (hi ? np_cap * kQuads : 0);
    const int page = rem / kQuads;
    const int qd = rem - page * kQuads;
    *reinterpret_cast<uint4*>(s_meta + ((hi ? kSqTile : 0) + page) * kPitch + qd * 16) = mv[j];
  }
  s_qv[tid < nq ? tid : nq - 1] = qv0;
  if (RMAX > 4) s_qv[tid + kSqThreads < nq ? tid + kSqThreads : nq - 1] = qv1;
  stage_qfix<D, RMAX, true>(qst, R, s_q, s_qshift, s_qsum, s_qok);
  const int P = a.lengths != nullptr ? ragged_pages(length, a.sink, a.recent, BS, a.P) : a.P;
  const int np = (P - p0) < kSqTile ? (P - p0) : kSqTile;  // <= 0: a ragged group's tile past its pages
  __syncthreads();

  // ---- 1. scores: wavefronts w and w + 4 sum halves of head w (+4), lane = page ----
  const int half = wave / 4;
  const int hw = wave % 4;
  {
    const uint8_t* min_row = s_meta + lane * kPitch;
    const uint8_t* max_row = s_meta + (kSqTile + lane) * kPitch;
    float part[HT];
#pragma unroll
    for (int h = 0; h < HT; ++h) {
      const int r = 4 * h + hw;
      part[h] = 0.0f;
      if (r < R) {
        const float* qh = s_qv + r * D;
        float acc[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int d0 = 32 * c + 16 * half + 8 * e;
            float qv[8], x[8];
            *reinterpret_cast<float4*>(qv) = *reinterpret_cast<const float4*>(qh + d0);
            *reinterpret_cast<float4*>(qv + 4) = *reinterpret_cast<const float4*>(qh + d0 + 4);
            select8(min_row + d0 * 2, max_row + d0 * 2, qv, x, DT{});
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[8 * e + i] = acc[8 * e + i] + x[i] * qv[i];
          }
        }
#pragma unroll
        for (int w = 1; w < 16; w <<= 1) {
#pragma unroll
          for (int l = 0; l < 16; l += 2 * w) acc[l] = acc[l] + acc[l + w];
        }
        part[h] = acc[0];
      }
      if (half == 1) s_half[r < RMAX ? r : RMAX - 1][lane] = part[h];
    }
    __syncthreads();
    if (half == 0 && np > 0) {
#pragma unroll
      for (int h = 0; h < HT; ++h) {
        const int r = 4 * h + hw;
        if (r >= R) continue;
        const float sc = part[h] + s_half[r][lane];
        const int64_t row = static_cast<int64_t>(g) * R + r;
        if (lane < np) a.scores[row * a.score_stride + p0 + lane] = sc;
        const uint32_t key = score_key(sc);
        const uint32_t kmax = wave_max_u32(lane < np ? key : 0u);
        const uint32_t kmin = wave_min_u32(lane < np ? key : 0xffffffffu);
        if (lane == 0) a.tile_mm[row * tiles + tile] = make_uint2(kmax, kmin);
      }
    }
  }

  // ---- 2. INT4 QK of the tile's rows for every head ----
  v4i av[HT][2];
  {
    const int mrow = lane % 16;
#pragma unroll
    for (int h = 0; h < HT; ++h) {
      const int r = 4 * h + mrow / 4;
      const int t = mrow % 4;
      const bool live = t < 3 && r < R;
      const uint32_t* st = s_q + (r < R ? r : 0) * 6 * KW + (t < 3 ? t : 0) * 2 * KW;
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        const int k0 = 4 * G4 + 2 * sp;
        av[h][sp][0] = live ? static_cast<int>(st[k0]) : 0;
        av[h][sp][1] = live ? static_cast<int>(st[KW + k0]) : 0;
        av[h][sp][2] = live ? static_cast<int>(st[k0 + 1]) : 0;
        av[h][sp][3] = live ? static_cast<int>(st[KW + k0 + 1]) : 0;
      }
    }
  }
  float* lbase[HT];
  int qshift[HT];
  float qsum[HT];
  bool qok[HT];
#pragma unroll
  for (int h = 0; h < HT; ++h) {
    const int r = 4 * h + G4 < R ? 4 * h + G4 : R - 1;
    lbase[h] = a.logits + (static_cast<int64_t>(g) * R + r) * a.logit_stride + static_cast<int64_t>(p0) * BS + n;
    qshift[h] = s_qshift[r];
    qsum[h] = s_qsum[r];
    qok[h] = s_qok[r] != 0;
  }
#pragma unroll
  for (int i = 0; i < kPg; ++i) {
    const int pl = wave + kWv * i;
    v4i b0v, b1v;
    b0v[0] = static_cast<int>(cw[i].x & 0x0f0f0f0fu);
    b0v[1] = static_cast<int>((cw[i].x >> 4) & 0x0f0f0f0fu);
    b0v[2] = static_cast<int>(cw[i].y & 0x0f0f0f0fu);
    b0v[3] = static_cast<int>((cw[i].y >> 4) & 0x0f0f0f0fu);
    b1v[0] = static_cast<int>(cw[i].z & 0x0f0f0f0fu);
    b1v[1] = static_cast<int>((cw[i].z >> 4) & 0x0f0f0f0fu);
    b1v[2] = static_cast<int>(cw[i].w & 0x0f0f0f0fu);
    b1v[3] = static_cast<int>((cw[i].w >> 4) & 0x0f0f0f0fu);
    const float sf = to_f32(DT{}, sv[i]), mf = to_f32(DT{}, mq[i]);
#pragma unroll
    for (int h = 0; h < HT; ++h) {
      v4i c = {0, 0, 0, 0};
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[h][0], b0v, c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[h][1], b1v, c, 0, 0, 0);
      const int64_t Sd = (static_cast<int64_t>(c[0]) << 16) + (static_cast<int64_t>(c[1]) << 8) + c[2];
      const float lg = qk_logit(Sd, qshift[h], qsum[h], qok[h], sf, mf, a.qk_scale);
      if (4 * h + G4 < R && pl < np) lbase[h][pl * BS] = lg;
    }
  }
}

struct HeadArgs {
  const float* scores;   // score_qk's page scores
  int64_t score_stride;
  int vec_last4;
  const uint2* tile_mm;
  int G, R, P, b0;       // P: scored pages of the launch; b0: B0 pages per head
  int parts;             // range entries per row over kWave (1: one per wavefront)
  const int32_t* lengths;  // nullable: group g has min(lengths[g], length) tokens
  int length;
  int sink, recent;
  const float* qk_logits;  // score_qk's logits, [G * R][logit_stride]
  int64_t logit_stride;
  uint32_t p24;
  float* ws_logits;        // matched: [G * R][b0 * 16] the candidates' logits
  uint32_t* ws_range;      // matched: [G * R][8][4] each wavefront's (max logit, max key, min key, 0)
  int32_t* sel_pages;    // nullable [G][R][b0]: B0 pages ascending, -1 past a ragged group's
  float* logits;         // nullable [G][R][b0 * 16]
  int32_t* desired;      // [G][R]
  uint32_t* rec;         // union records, rec_stride words apart
  int64_t rec_stride;
  int matched;           // matched budgets: stop after the top-p count (the record is
                         // written by twilight_matched_rec_kernel)
};

// ORs the kept candidates of a row (bit j of taken: candidate KPB t + j, row
// n % 16 of B0 page s_page[n / 16]) into its group's union record: the
// page's 16-bit row mask and its bit in the page bitmap.
template <int KPB>
__device__ __forceinline__ void or_into_record(uint32_t taken, const int* s_page, uint32_t* rec, int P) {
  const int tid = static_cast<int>(threadIdx.x);
  uint32_t* masks = rec + union_mask_offset(P);
  if constexpr (KPB == 8) {
    // two threads per page: the even one ORs both halves
    uint32_t m = (taken & 0xffu) << (8 * (tid & 1));
    m |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 1));
    if ((tid & 1) == 0 && m != 0u) {
      const int p = s_page[tid >> 1];
      atomicOr(masks + (p >> 1), m << (16 * (p & 1)));
      atomicOr(rec + (p >> 5), 1u << (p & 31));
    }
  } else {
    const uint32_t m = taken & 0xffffu;
    if (m != 0u) {
      const int p = s_page[tid];
      atomicOr(masks + (p >> 1), m << (16 * (p & 1)));
      atomicOr(rec + (p >> 5), 1u << (p & 31));
    }
  }
}

template <int KPA, int KPB>
__global__ __launch_bounds__(kHeadThreads) void twilight_topp_head_kernel(HeadArgs a) {
  constexpr int NT = kHeadThreads;
  constexpr int BS = 16;
  constexpr int kSlots = KPB * NT / BS;  // B0 pages a row holds
  constexpr int kWv = NT / kWave;        // wavefronts
  static_assert(KPA % 4 == 0 && (KPB == 8 || KPB == 16), "block shape");
  __shared__ __align__(16) TopShared<NT> sh;
  __shared__ int s_page[kSlots];
  __shared__ float s_rmax[kWv];
  __shared__ uint32_t s_rkx[kWv], s_rkn[kWv];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int g = static_cast<int>(blockIdx.x) % a.G;  // group-minor (XCD g % 8)
  const int row = g * a.R + static_cast<int>(blockIdx.x) / a.G;
  topk_fast_clear(sh.sel);
  __syncthreads();
  // ---- round trip 1: length, the row's keys and tile ranges ----
  int length = __hip_atomic_load(a.lengths != nullptr ? a.lengths + g : reinterpret_cast<const int32_t*>(a.scores),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t key[KPA];
  {
    const float* vals = a.scores + static_cast<int64_t>(row) * a.score_stride;
    const int i0 = KPA * tid;
#pragma unroll
    for (int q4 = 0; q4 < KPA / 4; ++q4) {
      int at = i0 + 4 * q4;
      at = at < a.vec_last4 ? at : a.vec_last4;
      const float4 v = *reinterpret_cast<const float4*>(vals + at);
      key[4 * q4] = score_key(v.x);
      key[4 * q4 + 1] = score_key(v.y);
      key[4 * q4 + 2] = score_key(v.z);
      key[4 * q4 + 3] = score_key(v.w);
    }
  }
  const int tiles = (a.P + kSqTile - 1) / kSqTile;
  uint2 tr0, tr1;
  {
    const uint2* tm = a.tile_mm + static_cast<int64_t>(row) * tiles;
    tr0 = tm[lane < tiles ? lane : tiles - 1];
    tr1 = tm[lane + kWave < tiles ? lane + kWave : tiles - 1];
  }

  length = a.lengths != nullptr ? (length < 0 ? 0 : (length > a.length ? a.length : length)) : a.length;
  const int P = a.lengths != nullptr ? ragged_pages(length, a.sink, a.recent, BS, a.P) : a.P;
  const int b0 = a.b0 < P ? a.b0 : P;  // block-uniform
  const int N = b0 * BS;

  // ---- 1. the B0 pages ----
  uint32_t take = 0u;
  if (b0 > 0) {
    const int tg = (P + kSqTile - 1) / kSqTile;
    const uint32_t kmax = wave_max_u32(max(lane < tg ? tr0.x : 0u, lane + kWave < tg ? tr1.x : 0u));
    const uint32_t kmin =
        wave_min_u32(min(lane < tg ? tr0.y : 0xffffffffu, lane + kWave < tg ? tr1.y : 0xffffffffu));
    if (!block_topk_fast<KPA>(key, P, b0, kmin, kmax, sh.sel, &take)) {
      int first;
      block_topk<KPA>(key, P, b0, sh.sel, &take, &first);
    }
  }
  {
    int total;
    int slot = block_excl_scan<NT>(__popc(take), sh.sel.scan, &total);
#pragma unroll
    for (int j = 0; j < KPA; ++j) {
      if ((take >> j) & 1u) s_page[slot++] = KPA * tid + j;
    }
  }
  // the top-p's histograms and staging counter start at zero (the top-k is
  // done with them)
  for (int b = tid; b < kLinBins + 64; b += NT) {
    sh.sel.hist[b] = 0u;
    sh.bin_mass[b] = 0ull;
  }
  if (tid == 0) sh.sel.ncand = 0u;
  if (tid < kWave) sh.sel.cpair[tid] = 0ull;
  __syncthreads();
  if (a.sel_pages != nullptr) {
    for (int i = tid; i < a.b0; i += NT) a.sel_pages[static_cast<int64_t>(row) * a.b0 + i] = i < b0 ? s_page[i] : -1;
  }
  if (N == 0) {
    if (tid == 0) a.desired[row] = 0;
    return;  // block-uniform: no candidate
  }

  // ---- 2. round trip 2: the candidates' logits (KPB consecutive rows of one
  // B0 page a thread), their max and key range ----
  const int c0 = KPB * tid;
  float v[KPB];
  {
    const int slot = c0 < N ? c0 / BS : 0;
    const float* src = a.qk_logits + static_cast<int64_t>(row) * a.logit_stride +
                       static_cast<int64_t>(s_page[slot]) * BS + (c0 % BS);
#pragma unroll
    for (int j = 0; j < KPB; j += 4) {
      const float4 t = *reinterpret_cast<const float4*>(src + j);
      v[j] = t.x;
      v[j + 1] = t.y;
      v[j + 2] = t.z;
      v[j + 3] = t.w;
    }
  }
  uint32_t lkey[KPB];
  float wmx = -INFINITY;
  uint32_t wkx = 0u, wkn = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < KPB; ++j) {
    lkey[j] = score_key(v[j]);
    const bool ok = c0 + j < N;
    wmx = (ok && v[j] > wmx) ? v[j] : wmx;
    wkx = (ok && lkey[j] > wkx) ? lkey[j] : wkx;
    wkn = (ok && lkey[j] < wkn) ? lkey[j] : wkn;
  }
  if (a.logits != nullptr) {
    float* lo = a.logits + static_cast<int64_t>(row) * a.b0 * BS;
#pragma unroll
    for (int j = 0; j < KPB; ++j)
      if (c0 + j < N) lo[c0 + j] = v[j];
  }
  wmx = wave_max_f32(wmx);
  wkx = wave_max_u32(wkx);
  wkn = wave_min_u32(wkn);
  if (lane == 0) {
    s_rmax[wave] = wmx;
    s_rkx[wave] = wkx;
    s_rkn[wave] = wkn;
  }
  if (a.matched) {
    // the allocation launch reads the candidates' logits and the wavefronts' ranges back
    float* wl = a.ws_logits + static_cast<int64_t>(row) * a.b0 * BS;
#pragma unroll
    for (int j = 0; j < KPB; j += 4) {
      if (c0 + j < N) *reinterpret_cast<float4*>(wl + c0 + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
    }
    if (lane == 0)
      *reinterpret_cast<uint4*>(a.ws_range + (static_cast<int64_t>(row) * kWv + wave) * 4) =
          make_uint4(__float_as_uint(wmx), wkx, wkn, 0u);
  }
  __syncthreads();
  float lmax = s_rmax[0];
  uint32_t kmax = s_rkx[0], kmin = s_rkn[0];
#pragma unroll
  for (int w = 1; w < kWv; ++w) {
    lmax = s_rmax[w] > lmax ? s_rmax[w] : lmax;
    kmax = s_rkx[w] > kmax ? s_rkx[w] : kmax;
    kmin = s_rkn[w] < kmin ? s_rkn[w] : kmin;
  }

  // ---- 3. top-p over the row's logits ----
  uint64_t mass[KPB];
  uint64_t local = 0;
#pragma unroll
  for (int j = 0; j < KPB; ++j) {
    mass[j] = mass_of((c0 + j < N) ? key_value(lkey[j]) : -INFINITY, lmax);  // 0 past the row
    local += mass[j];
  }
  uint32_t taken;
  int desired;
  if (!block_top_p_fast<KPB>(lkey, mass, N, a.p24, kmin, kmax, sh, &taken, &desired)) {
    // the general search, on cleared bins
    for (int b = tid; b < kLinBins + 64; b += NT) {
      sh.sel.hist[b] = 0u;
      sh.bin_mass[b] = 0ull;
    }
    const uint64_t z = block_sum_u64<NT>(local, sh.red64);  // (its barriers order the clear)
    uint64_t need = top_p_threshold(a.p24, z);
    if (need == 0) {
      // no mass at all (non-finite logits): one key, the largest
#pragma unroll
      for (int j = 0; j < KPB; ++j) mass[j] = (c0 + j < N) ? 1ull : 0ull;
      need = 1;
    }
    desired = block_top_mass<KPB>(lkey, mass, N, need, kmin, kmax, sh, &taken);
  }
  desired = desired < 1 ? 1 : (desired > N ? N : desired);
  if (tid == 0) a.desired[row] = desired;
  if (a.matched) return;

  // ---- 4. publish: row masks and the page bitmap of the union record ----
  or_into_record<KPB>(taken, s_page, a.rec + static_cast<int64_t>(g) * a.rec_stride, a.P);
}

// Matched budgets over the fused selection: one block per (group, head)
// after twilight_topp_head_kernel (matched) has written every head's top-p
// count and left its candidates' logits, B0 pages and wavefront key ranges in
// the workspace.
// Every block of a group forms the same allocation (wave_matched_counts), takes
// its head's top-allocated logits (key desc, candidate index asc: the
// selection twilight_matched_kernel makes) and ORs their rows into the
// union record the score kernel cleared.  With lengths (device), group g's
// candidate pages, B0 pages and target come from its own length, as the
// cache forms them on the host: fixed = min(candidates, max(1, ceil(frac *
// eligible / 16))) pages, target = fixed * 16 * R (at most every candidate).
struct MatchedRecArgs {
  const float* ws_logits;     // [G * R][b0 * 16]
  const uint32_t* ws_range;   // [G * R][parts * 8][4] (max logit, max key, min key, 0)
  const int32_t* sel_pages;   // [G][R][b0] ascending
  const int32_t* desired;     // [G][desired_stride]: the top-p counts of every head of the group
  int64_t desired_stride;
  int32_t* allocated;         // nullable [G][R]
  int G, R, P, b0, parts, target_total;
  int heads_all, head0;       // the group's heads (<= 64); this launch's are head0 .. head0 + R - 1
  const int32_t* lengths;     // nullable [G]: group g has min(lengths[g], length) tokens
  int length, sink, recent;
  double frac;                // matched_budget_fraction (with lengths)
  uint32_t* rec;
  int64_t rec_stride;
};

template <int KPB>
__global__ __launch_bounds__(kHeadThreads) void twilight_matched_rec_kernel(MatchedRecArgs a) {
  constexpr int NT = kHeadThreads;
  constexpr int BS = 16;
  constexpr int kSlots = KPB * NT / BS;
  constexpr int kWv = NT / kWave;
  __shared__ __align__(16) TopShared<NT> sh;
  __shared__ int s_page[kSlots];
  __shared__ int s_k;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int g = static_cast<int>(blockIdx.x) % a.G;  // group-minor (XCD g % 8)
  const int r = static_cast<int>(blockIdx.x) / a.G;
  const int row = g * a.R + r;
  int N = a.b0 * BS;
  int target = a.target_total;
  if (a.lengths != nullptr) {
    int L = a.lengths[g];
    L = L < 0 ? 0 : (L > a.length ? a.length : L);
    const int Pg = ragged_pages(L, a.sink, a.recent, BS, a.P);
    N = (a.b0 < Pg ? a.b0 : Pg) * BS;
    const int sink_end = a.sink < L ? a.sink : L;
    const int hist_recent = a.recent - 1 > 0 ? a.recent - 1 : 0;
    const int recent_start = L - hist_recent > sink_end ? L - hist_recent : sink_end;
    const double f = ceil(a.frac * static_cast<double>(recent_start - sink_end) / static_cast<double>(BS));
    int fixed = f < 1.0 ? 1 : (f > static_cast<double>(Pg) ? Pg : static_cast<int>(f));
    fixed = fixed < Pg ? fixed : Pg;
    target = fixed * BS * a.heads_all;
    target = target < a.heads_all * N ? target : a.heads_all * N;
  }
  if (N == 0) {  // block-uniform: no candidate, nothing kept, nothing allocated
    if (tid == 0 && a.allocated != nullptr) a.allocated[row] = 0;
    return;
  }
  topk_fast_clear(sh.sel);
  // ---- one round trip: the group's counts, the row's pages, logits and ranges ----
  for (int i = tid; i < a.b0; i += NT) s_page[i] = a.sel_pages[static_cast<int64_t>(row) * a.b0 + i];
  uint32_t lkey[KPB];
  uint32_t kmin, kmax;
  {
    const float* wl = a.ws_logits + static_cast<int64_t>(row) * a.b0 * BS;
    const int i0 = KPB * tid;
#pragma unroll
    for (int j = 0; j < KPB; j += 4) {
      const int i = i0 + j < N ? i0 + j : 0;
      const float4 t = *reinterpret_cast<const float4*>(wl + i);
      lkey[j] = score_key(t.x);
      lkey[j + 1] = score_key(t.y);
      lkey[j + 2] = score_key(t.z);
      lkey[j + 3] = score_key(t.w);
    }
    const int n_rng = a.parts * kWv;  // <= 128
    const uint32_t* rr = a.ws_range + static_cast<int64_t>(row) * n_rng * 4;
    uint32_t kmx = 0u, kmn = 0xffffffffu;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = lane + kWave * h < n_rng ? lane + kWave * h : n_rng - 1;
      const uint4 t = *reinterpret_cast<const uint4*>(rr + 4 * e);
      kmx = t.y > kmx ? t.y : kmx;
      kmn = t.z < kmn ? t.z : kmn;
    }
    kmax = wave_max_u32(kmx);
    kmin = wave_min_u32(kmn);
  }
  // the allocation, by the first wavefront (whole) while the others' loads land
  if (tid < kWave) {
    const int c = wave_matched_counts(a.desired + static_cast<int64_t>(g) * a.desired_stride, a.heads_all, target,
                                      N);
    const int cr = static_cast<int>(readlane_u32(static_cast<uint32_t>(c), a.head0 + r));
    const int k = cr < 1 ? 1 : (cr > N ? N : cr);
    if (tid == 0) {
      s_k = k;
      if (a.allocated != nullptr) a.allocated[row] = k;
    }
  }
  __syncthreads();  // s_k, s_page and the cleared histogram
  const int k = s_k;
  uint32_t taken = 0u;
  if (!block_topk_fast<KPB>(lkey, N, k, kmin, kmax, sh.sel, &taken)) {
    int first;
    block_topk<KPB>(lkey, N, k, sh.sel, &taken, &first);
  }
  or_into_record<KPB>(taken, s_page, a.rec + static_cast<int64_t>(g) * a.rec_stride, a.P);
}

// --------------------------------------------------------------- launch
template <typename DT, int DIM>
int launch_qk_r(const QkArgs& a, hipStream_t stream) {
  const int row_blocks = static_cast<int>((a.plan_stride * a.bs + kQkRows - 1) / kQkRows);
  const dim3 grid(a.G * row_blocks);
  constexpr bool kMf = DIM == 128;  // matrix cores at 128 channels
  if (a.R <= 4) {
    hipLaunchKernelGGL((twilight_qk_kernel<DT, DIM, 4, 32, kMf>), grid, dim3(kBlock), 0, stream, a);
  } else {
    hipLaunchKernelGGL((twilight_qk_kernel<DT, DIM, 8, 16, kMf>), grid, dim3(kBlock), 0, stream, a);
  }
  return tw_host::check_launch();
}

template <typename DT>
int launch_qk(const QkArgs& a, hipStream_t stream) {
  switch (a.D) {
    case 4: return launch_qk_r<DT, 4>(a, stream);
    case 8: return launch_qk_r<DT, 8>(a, stream);
    case 16: return launch_qk_r<DT, 16>(a, stream);
    case 32: return launch_qk_r<DT, 32>(a, stream);
    case 64: return launch_qk_r<DT, 64>(a, stream);
    case 128: return launch_qk_r<DT, 128>(a, stream);
    case 256: return launch_qk_r<DT, 256>(a, stream);
    default: return TW_EUNSUPPORTED;
  }
}

template <typename DT, int DIM>
void launch_qk_positions_d(const QkArgs& a, const int64_t* positions, int N, float* out, bool materialize,
                           hipStream_t stream) {
  const dim3 grid(a.G * a.R * ((N + 63) / 64));
  hipLaunchKernelGGL((int4_qk_positions_kernel<DT, DIM, 32>), grid, dim3(kBlock), 0, stream, a, positions, N, out,
                     materialize);
}

template <typename DT>
int launch_qk_positions(const QkArgs& a, const int64_t* positions, int N, float* out, bool materialize,
                        hipStream_t stream) {
  switch (a.D) {
    case 4: launch_qk_positions_d<DT, 4>(a, positions, N, out, materialize, stream); break;
    case 8: launch_qk_positions_d<DT, 8>(a, positions, N, out, materialize, stream); break;
    case 16: launch_qk_positions_d<DT, 16>(a, positions, N, out, materialize, stream); break;
    case 32: launch_qk_positions_d<DT, 32>(a, positions, N, out, materialize, stream); break;
    case 64: launch_qk_positions_d<DT, 64>(a, positions, N, out, materialize, stream); break;
    case 128: launch_qk_positions_d<DT, 128>(a, positions, N, out, materialize, stream); break;
    case 256: launch_qk_positions_d<DT, 256>(a, positions, N, out, materialize, stream); break;
    default: return TW_EUNSUPPORTED;
  }
  return tw_host::check_launch();
}

// Threads of a top-p block (one (group, head) row per block).  512 measured
// best at 4096 candidates: two wavefronts per SIMD hide part of each other's
// instruction latency, while 1024 threads paid more in 16-wave barriers.
#ifndef TW_TOPP_THREADS
#define TW_TOPP_THREADS 512
#endif
constexpr int kToppThreads = TW_TOPP_THREADS;
// Candidates per head a top-p block holds: 32 per thread (one 32-bit
// selection mask each).
constexpr int kMaxCandidates = 32 * kToppThreads;

template <int KPT>
int launch_select_kpt(const SelectArgs& s, hipStream_t stream) {
  constexpr int NT = kToppThreads;
  const size_t lds = (static_cast<size_t>(stage_offset_words(s.length)) + stage_elems(s.N, s.length)) * 4;
  if (lds + sizeof(TopShared<NT>) > 160 * 1024) return TW_EUNSUPPORTED;
  if (lds + sizeof(TopShared<NT>) > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(twilight_topp_kernel<KPT, NT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void*>(twilight_matched_kernel<KPT, NT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
      return tw_host::check_launch();
  }
  const dim3 grid(s.G * s.R);
  if (!s.given) {
    hipLaunchKernelGGL((twilight_topp_kernel<KPT, NT>), grid, dim3(NT), lds, stream, s);
    const int rc = tw_host::check_launch();
    if (rc != TW_OK || !s.matched) return rc;
  }
  hipLaunchKernelGGL((twilight_matched_kernel<KPT, NT>), grid, dim3(NT), lds, stream, s);
  return tw_host::check_launch();
}

// Candidates per thread of the top-p launch for N candidates per head (the
// KPT launch_select picks).
int candidates_per_thread(int N) {
  constexpr int NT = kToppThreads;
  int kpt = 1;
  while (kpt * NT < N && kpt < 32) kpt *= 2;
  if (NT < 1024 && kpt < 2) kpt = 2;
  if (NT < 512 && kpt < 4) kpt = 4;
  return kpt;
}

int launch_select(const SelectArgs& s, hipStream_t stream) {
  constexpr int NT = kToppThreads;
  if constexpr (NT >= 1024) {
    if (s.N <= NT) return launch_select_kpt<1>(s, stream);
  }
  if constexpr (NT >= 512) {
    if (s.N <= 2 * NT) return launch_select_kpt<2>(s, stream);
  }
  if (s.N <= 4 * NT) return launch_select_kpt<4>(s, stream);
  if (s.N <= 8 * NT) return launch_select_kpt<8>(s, stream);
  if (s.N <= 16 * NT) return launch_select_kpt<16>(s, stream);
  return launch_select_kpt<32>(s, stream);  // N <= kMaxCandidates, checked by the caller
}

size_t counter_bytes(int) { return kCounterRegionBytes; }

}  // namespace
}  // namespace tw

extern "C" int tw_twilight_qk(const float* q, int G, int R, int D, const uint8_t* packed, const void* scale,
                              const void* minimum, int dtype, int64_t quant_entry_stride, int64_t quant_rows,
                              const int32_t* plan_pages,
                              const uint8_t* plan_masks, const int32_t* plan_counts, int64_t plan_stride,
                              int b0_pages, int sink, int block_size, float qk_scale, float* logits,
                              int32_t* slot_u, uint32_t* page_rows, void* stream) {
  if (q == nullptr || packed == nullptr || scale == nullptr || minimum == nullptr || plan_pages == nullptr ||
      plan_masks == nullptr || plan_counts == nullptr || logits == nullptr)
    return TW_EINVAL;
  if ((slot_u == nullptr) != (page_rows == nullptr)) return TW_EINVAL;
  if (G <= 0 || R <= 0 || R > 8 || b0_pages <= 0 || sink < 0 || block_size <= 0 || plan_stride < 1 ||
      quant_entry_stride <= 0 || quant_rows <= 0 || quant_rows > quant_entry_stride)
    return TW_EINVAL;
  if (D < 4 || D > 256 || (D & (D - 1)) != 0) return TW_EUNSUPPORTED;
  // each lane reads min(D, 32) / 2 code bytes of a row with one load
  const uintptr_t pk_align = D >= 32 ? 16 : static_cast<uintptr_t>(D / 2);
  if ((reinterpret_cast<uintptr_t>(q) % 16) || (reinterpret_cast<uintptr_t>(packed) % pk_align)) return TW_EINVAL;
  tw::QkArgs a{q, packed, scale, minimum, quant_entry_stride, quant_rows, G, R, D, plan_pages, plan_masks, plan_counts,
               plan_stride, b0_pages, sink, block_size, qk_scale, logits, slot_u, page_rows};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TW_DTYPE_F16: return tw::launch_qk<tw::F16>(a, s);
    case TW_DTYPE_BF16: return tw::launch_qk<tw::BF16>(a, s);
    case TW_DTYPE_F32: return tw::launch_qk<tw::F32>(a, s);
    default: return TW_EINVAL;
  }
}

extern "C" int tw_int4_qk_positions(const float* q, int G, int R, int D, const uint8_t* packed, const void* scale,
                                    const void* minimum, int dtype, int64_t quant_entry_stride, int64_t quant_rows,
                                    const int64_t* positions, int N, float qk_scale, int materialize, float* out,
                                    void* stream) {
  if (q == nullptr || packed == nullptr || scale == nullptr || minimum == nullptr || out == nullptr) return TW_EINVAL;
  if (G <= 0 || R <= 0 || N < 0 || quant_entry_stride <= 0 || quant_rows <= 0 || quant_rows > quant_entry_stride)
    return TW_EINVAL;
  if (N == 0) return TW_OK;
  if (positions == nullptr) return TW_EINVAL;
  if (D < 4 || D > 256 || (D & (D - 1)) != 0) return TW_EUNSUPPORTED;
  const uintptr_t pk_align = D >= 32 ? 16 : static_cast<uintptr_t>(D / 2);
  if ((reinterpret_cast<uintptr_t>(q) % 16) || (reinterpret_cast<uintptr_t>(packed) % pk_align)) return TW_EINVAL;
  tw::QkArgs a{q, packed, scale, minimum, quant_entry_stride, quant_rows, G, R, D, nullptr, nullptr, nullptr, 0,
               0, 0, 1, qk_scale, nullptr, nullptr, nullptr};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TW_DTYPE_F16: return tw::launch_qk_positions<tw::F16>(a, positions, N, out, materialize != 0, s);
    case TW_DTYPE_BF16: return tw::launch_qk_positions<tw::BF16>(a, positions, N, out, materialize != 0, s);
    case TW_DTYPE_F32: return tw::launch_qk_positions<tw::F32>(a, positions, N, out, materialize != 0, s);
    default: return TW_EINVAL;
  }
}

extern "C" int tw_twilight_max_candidates(void) { return tw::kMaxCandidates; }

extern "C" size_t tw_twilight_select_workspace_size(int G, int R, int N) {
  if (G <= 0 || R <= 0 || N <= 0) return 0;
  const size_t words = static_cast<size_t>((N + 31) / 32);
  return tw::counter_bytes(G) + static_cast<size_t>(G) * R * words * 4 + static_cast<size_t>(G) * R * 4;
}

namespace {
int select_launch(const float* logits, int G, int R, int N, const int32_t* sel_pages, int b0_pages, float top_p,
                  int budget_mode, int target_total, int32_t* desired, int32_t* allocated, uint32_t* head_bits,
                  int32_t* rows, int32_t* row_counts, int64_t rows_stride, int sink, int recent, int block_size,
                  int length, const int32_t* lengths, int p_max, int append_position, void* workspace,
                  size_t workspace_bytes, void* stream, const int32_t* slot_u = nullptr,
                  uint32_t* page_rows = nullptr, int64_t page_rows_stride = 0) {
  const bool pr = page_rows != nullptr;
  if (logits == nullptr || sel_pages == nullptr || (!pr && (rows == nullptr || row_counts == nullptr)))
    return TW_EINVAL;
  if (G <= 0 || R <= 0 || R > 8 || N <= 0 || b0_pages <= 0 || N != b0_pages * block_size) return TW_EINVAL;
  if (N > tw::kMaxCandidates) return TW_EUNSUPPORTED;
  if (!(top_p > 0.0f) || !(top_p <= 1.0f) || budget_mode < 0 || budget_mode > 2) return TW_EINVAL;
  if (budget_mode == 2 && allocated == nullptr) return TW_EINVAL;
  if (sink < 0 || recent <= 0 || block_size <= 0 || length < 0) return TW_EINVAL;
  if (budget_mode == 1 && (target_total < R || target_total > static_cast<int64_t>(R) * N)) return TW_EINVAL;
  // every union row fits: sink + recent + R*N selected + the decode row
  if (!pr && rows_stride < static_cast<int64_t>(length) + 1) return TW_EINVAL;
  if (pr) {
    // dynamic budgets only; a thread's candidates in one page's row mask
    const int kpt = tw::candidates_per_thread(N);
    if (slot_u == nullptr || budget_mode != 0 || block_size > 32 || (block_size % kpt != 0 && kpt % block_size != 0) ||
        page_rows_stride < 1)
      return TW_EINVAL;
  }
  if (G > tw::kMaxCounterGroups) return TW_EUNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < tw_twilight_select_workspace_size(G, R, N)) return TW_ENOMEM;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int words = (N + 31) / 32;
  tw::SelectArgs s{};
  s.logits = logits;
  s.G = G;
  s.R = R;
  s.N = N;
  s.p24 = static_cast<uint32_t>(__builtin_rintf(top_p * 16777216.0f));
  s.matched = budget_mode >= 1;
  s.given = budget_mode == 2;
  s.target_total = target_total;
  s.sel_pages = sel_pages;
  s.b0 = b0_pages;
  s.counters = reinterpret_cast<unsigned int*>(ws);
  s.selbits = head_bits != nullptr ? head_bits : reinterpret_cast<uint32_t*>(ws + tw::counter_bytes(G));
  s.words_n = words;
  s.desired = desired != nullptr ? desired
                                 : reinterpret_cast<int32_t*>(ws + tw::counter_bytes(G) +
                                                              static_cast<size_t>(G) * R * words * 4);
  s.allocated = allocated;
  s.rows = rows;
  s.row_counts = row_counts;
  s.rows_stride = rows_stride;
  s.sink = sink;
  s.recent = recent;
  s.bs = block_size;
  s.length = length;
  s.append_position = append_position;
  s.lengths = lengths;
  s.p_max = p_max;
  s.slot_u = slot_u;
  s.page_rows = page_rows;
  s.page_rows_stride = page_rows_stride;
  return tw::launch_select(s, static_cast<hipStream_t>(stream));
}
}  // namespace

extern "C" int tw_twilight_select(const float* logits, int G, int R, int N, const int32_t* sel_pages, int b0_pages,
                                  float top_p, int budget_mode, int target_total, int32_t* desired,
                                  int32_t* allocated, uint32_t* head_bits, int32_t* rows, int32_t* row_counts,
                                  int64_t rows_stride, int sink, int recent, int block_size, int length,
                                  int append_position, void* workspace, size_t workspace_bytes, void* stream) {
  return select_launch(logits, G, R, N, sel_pages, b0_pages, top_p, budget_mode, target_total, desired, allocated,
                       head_bits, rows, row_counts, rows_stride, sink, recent, block_size, length, nullptr, 0,
                       append_position, workspace, workspace_bytes, stream);
}

extern "C" int tw_twilight_select_ragged(const float* logits, int G, int R, int N, const int32_t* sel_pages,
                                         int b0_pages, float top_p, int32_t* desired, int32_t* allocated,
                                         uint32_t* head_bits, int32_t* rows, int32_t* row_counts,
                                         int64_t rows_stride, int sink, int recent, int block_size,
                                         const int32_t* lengths, int max_length, int page_capacity,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (lengths == nullptr || max_length < 0 || page_capacity < 0) return TW_EINVAL;
  return select_launch(logits, G, R, N, sel_pages, b0_pages, top_p, 0, 0, desired, allocated, head_bits, rows,
                       row_counts, rows_stride, sink, recent, block_size, max_length, lengths, page_capacity, -1,
                       workspace, workspace_bytes, stream);
}

extern "C" int tw_twilight_select_pages(const float* logits, int G, int R, int N, const int32_t* sel_pages,
                                        int b0_pages, float top_p, const int32_t* slot_u, uint32_t* page_rows,
                                        int64_t page_rows_stride, int32_t* desired, int sink, int recent,
                                        int block_size, int length, const int32_t* lengths, int page_capacity,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  if (page_rows == nullptr || length < 0 || page_capacity < 0) return TW_EINVAL;
  return select_launch(logits, G, R, N, sel_pages, b0_pages, top_p, 0, 0, desired, nullptr, nullptr, nullptr,
                       nullptr, 0, sink, recent, block_size, length, lengths, lengths != nullptr ? page_capacity : 0,
                       -1, workspace, workspace_bytes, stream, slot_u, page_rows, page_rows_stride);
}

namespace tw {
namespace {

template <int KPA, int KPB>
int launch_head_kpb(const HeadArgs& h, hipStream_t stream) {
  hipLaunchKernelGGL((twilight_topp_head_kernel<KPA, KPB>), dim3(h.G * h.R), dim3(kHeadThreads), 0, stream, h);
  return tw_host::check_launch();
}

int launch_head(const HeadArgs& h, hipStream_t stream) {
  const bool wide = h.b0 * 16 > 8 * kHeadThreads;
  if (h.P <= 4 * kHeadThreads) return wide ? launch_head_kpb<4, 16>(h, stream) : launch_head_kpb<4, 8>(h, stream);
  if (h.P <= 8 * kHeadThreads) return wide ? launch_head_kpb<8, 16>(h, stream) : launch_head_kpb<8, 8>(h, stream);
  return wide ? launch_head_kpb<16, 16>(h, stream) : launch_head_kpb<16, 8>(h, stream);
}

template <typename DT>
int launch_score_qk(const ScoreQkArgs& s, hipStream_t stream) {
  const dim3 grid(s.G * ((s.P + kSqTile - 1) / kSqTile));
  if (s.R <= 4)
    hipLaunchKernelGGL((twilight_score_qk_kernel<DT, 4>), grid, dim3(kSqThreads), 0, stream, s);
  else
    hipLaunchKernelGGL((twilight_score_qk_kernel<DT, 8>), grid, dim3(kSqThreads), 0, stream, s);
  return tw_host::check_launch();
}

// Workspace of the fused selection, 256-byte aligned pieces: page scores
// [G * R][P rounded up to 4] | tile key ranges [G * R][ceil(P / 64)] | row
// logits [G * R][16 P] | (matched) the candidates' logits [G * R][16 b0] and
// the head launch's wavefront ranges [G * R][8][4].
struct FusedWorkspace {
  float* scores;
  int64_t score_stride;
  uint2* tile_mm;
  float* qk_logits;
  int64_t logit_stride;
  float* cand_logits;
  uint32_t* ranges;
  size_t bytes;
};

FusedWorkspace fused_layout(void* base, int G, int R, int P, int b0_pages) {
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t rows = static_cast<size_t>(G) * R;
  FusedWorkspace w{};
  w.score_stride = (static_cast<int64_t>(P) + 3) & ~static_cast<int64_t>(3);
  w.logit_stride = static_cast<int64_t>(P) * 16;
  uint8_t* p = static_cast<uint8_t*>(base);
  size_t off = 0;
  w.scores = reinterpret_cast<float*>(p + off);
  off += al(rows * w.score_stride * sizeof(float));
  w.tile_mm = reinterpret_cast<uint2*>(p + off);
  off += al(rows * ((P + kSqTile - 1) / kSqTile) * sizeof(uint2));
  w.qk_logits = reinterpret_cast<float*>(p + off);
  off += al(rows * w.logit_stride * sizeof(float));
  w.cand_logits = reinterpret_cast<float*>(p + off);
  off += al(rows * static_cast<size_t>(b0_pages) * 16 * sizeof(float));
  w.ranges = reinterpret_cast<uint32_t*>(p + off);
  off += al(rows * (kHeadThreads / kWave) * 4 * sizeof(uint32_t));
  w.bytes = off;
  return w;
}

}  // namespace
}  // namespace tw

extern "C" int tw_twilight_union_record_words(int P) {
  return P > 0 ? static_cast<int>(tw::union_record_words(P)) : 0;
}

extern "C" size_t tw_twilight_select_fused_workspace_size(int G, int R, int P, int b0_pages) {
  if (G <= 0 || R <= 0 || P <= 0 || b0_pages <= 0) return 0;
  return tw::fused_layout(nullptr, G, R, P, b0_pages).bytes;
}

namespace tw {
namespace {

// tw_twilight_select_fused (matched false) and tw_twilight_select_fused_matched.
// phase 1: the score + INT4 QK launch; 2: it and the head launch; 3: the whole
// selection; 4 (matched): the allocation + top-allocated launch alone, after
// a phase-2 call with the same workspace.  desired_all (nullable, matched):
// the top-p counts of all heads_all heads of each group ([G][heads_all]), of
// which this call's R heads are head0 .. head0 + R - 1; null means this call's
// own R counts.
int select_fused(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R, int P, int D,
                 int64_t page_group_stride, const uint8_t* packed, const void* qscale, const void* qmin,
                 int64_t quant_entry_stride, int64_t quant_rows, int b0_pages, float top_p, float qk_scale, int sink,
                 int recent, int block_size, const int32_t* lengths, int length, int32_t* sel_pages, float* logits,
                 int32_t* desired, uint32_t* union_rec, int64_t rec_stride, void* workspace, size_t workspace_bytes,
                 bool matched, int target_total, double matched_fraction, int32_t* allocated, void* stream,
                 int phase = 3, const int32_t* desired_all = nullptr, int heads_all = 0, int head0 = 0) {
  if (phase < 1 || phase > 4 || (phase == 4 && !matched)) return TW_EINVAL;
  if (q == nullptr || page_min == nullptr || page_max == nullptr || packed == nullptr || qscale == nullptr ||
      qmin == nullptr || desired == nullptr || union_rec == nullptr)
    return TW_EINVAL;
  const int32_t* dall = desired_all != nullptr ? desired_all : desired;
  const int hall = desired_all != nullptr ? heads_all : R;
  const int h0 = desired_all != nullptr ? head0 : 0;
  // matched: the B0 pages as an output the last launch reads; a target for
  // one length (over all hall heads), or the matched fraction for device
  // lengths; one wavefront allocates, a lane a head
  if (matched && (sel_pages == nullptr || hall < R || hall > kWave || h0 < 0 || h0 + R > hall ||
                  (lengths == nullptr && (target_total < hall || static_cast<int64_t>(target_total) >
                                                                     static_cast<int64_t>(hall) * b0_pages * 16)) ||
                  (lengths != nullptr && !(matched_fraction > 0.0 && matched_fraction <= 1.0))))
    return TW_EINVAL;
  if (dtype != TW_DTYPE_F16 && dtype != TW_DTYPE_BF16) return TW_EUNSUPPORTED;
  if (D != 128 || block_size != 16) return TW_EUNSUPPORTED;
  if (G <= 0 || R <= 0 || R > 8 || P <= 0 || b0_pages <= 0 || b0_pages > P) return TW_EINVAL;
  if (P > 16 * tw::kHeadThreads || b0_pages * 16 > 16 * tw::kHeadThreads) return TW_EUNSUPPORTED;
  if (!(top_p > 0.0f) || !(top_p <= 1.0f) || sink < 0 || recent <= 0 || length < 0) return TW_EINVAL;
  // every candidate row (a page below P, so a row below sink + 16 P) has its INT4 code
  if (quant_entry_stride < quant_rows || quant_rows < static_cast<int64_t>(sink) + 16ll * P ||
      (G > 1 && quant_entry_stride <= 0))
    return TW_EINVAL;
  if (rec_stride < tw::union_record_words(P) || (rec_stride % 4) != 0 ||
      (reinterpret_cast<uintptr_t>(union_rec) % 16) != 0)
    return TW_EINVAL;
  if ((reinterpret_cast<uintptr_t>(packed) % 16) != 0) return TW_EINVAL;
  if (workspace == nullptr || workspace_bytes < tw_twilight_select_fused_workspace_size(G, R, P, b0_pages))
    return TW_ENOMEM;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const FusedWorkspace w = fused_layout(workspace, G, R, P, b0_pages);
  int rc = TW_OK;
  if (phase != 4) {
    ScoreQkArgs sq{};
    sq.q = q;
    sq.pmin = page_min;
    sq.pmax = page_max;
    sq.group_stride = page_group_stride;
    sq.G = G;
    sq.R = R;
    sq.P = P;
    sq.lengths = lengths;
    sq.sink = sink;
    sq.recent = recent;
    sq.packed = packed;
    sq.scale = qscale;
    sq.minimum = qmin;
    sq.qstride = quant_entry_stride;
    sq.qrows = quant_rows;
    sq.qk_scale = qk_scale;
    sq.scores = w.scores;
    sq.score_stride = w.score_stride;
    sq.tile_mm = w.tile_mm;
    sq.logits = w.qk_logits;
    sq.logit_stride = w.logit_stride;
    sq.rec = union_rec;
    sq.rec_stride = rec_stride;
    rc = dtype == TW_DTYPE_F16 ? launch_score_qk<F16>(sq, st) : launch_score_qk<BF16>(sq, st);
    if (rc != TW_OK || phase == 1) return rc;
    HeadArgs h{};
    h.scores = w.scores;
    h.score_stride = w.score_stride;
    h.vec_last4 = static_cast<int>(w.score_stride) - 4;
    h.tile_mm = w.tile_mm;
    h.G = G;
    h.R = R;
    h.P = P;
    h.b0 = b0_pages;
    h.parts = 1;
    h.qk_logits = w.qk_logits;
    h.logit_stride = w.logit_stride;
    h.ws_logits = w.cand_logits;
    h.ws_range = w.ranges;
    h.lengths = lengths;
    h.length = length;
    h.sink = sink;
    h.recent = recent;
    h.p24 = static_cast<uint32_t>(__builtin_rintf(top_p * 16777216.0f));
    h.sel_pages = sel_pages;
    h.logits = logits;
    h.desired = desired;
    h.rec = union_rec;
    h.rec_stride = rec_stride;
    h.matched = matched ? 1 : 0;
    rc = launch_head(h, st);
    if (rc != TW_OK || !matched || phase == 2) return rc;
  }
  tw::MatchedRecArgs m{};
  m.ws_logits = w.cand_logits;
  m.ws_range = w.ranges;
  m.sel_pages = sel_pages;
  m.desired = dall;
  m.desired_stride = hall;
  m.heads_all = hall;
  m.head0 = h0;
  m.allocated = allocated;
  m.G = G;
  m.R = R;
  m.P = P;
  m.b0 = b0_pages;
  m.parts = 1;
  m.target_total = target_total;
  m.lengths = lengths;
  m.length = length;
  m.sink = sink;
  m.recent = recent;
  m.frac = matched_fraction;
  m.rec = union_rec;
  m.rec_stride = rec_stride;
  if (b0_pages * 16 > 8 * tw::kHeadThreads)
    hipLaunchKernelGGL((tw::twilight_matched_rec_kernel<16>), dim3(G * R), dim3(tw::kHeadThreads), 0, st, m);
  else
    hipLaunchKernelGGL((tw::twilight_matched_rec_kernel<8>), dim3(G * R), dim3(tw::kHeadThreads), 0, st, m);
  return tw_host::check_launch();
}

}  // namespace
}  // namespace tw

extern "C" int tw_twilight_select_fused(const float* q, const void* page_min, const void* page_max, int dtype,
                                        int G, int R, int P, int D, int64_t page_group_stride, const uint8_t* packed,
                                        const void* qscale, const void* qmin, int64_t quant_entry_stride,
                                        int64_t quant_rows, int b0_pages, float top_p, float qk_scale, int sink,
                                        int recent, int block_size, const int32_t* lengths, int length,
                                        int32_t* sel_pages, float* logits, int32_t* desired, uint32_t* union_rec,
                                        int64_t rec_stride, void* workspace, size_t workspace_bytes, void* stream) {
  return tw::select_fused(q, page_min, page_max, dtype, G, R, P, D, page_group_stride, packed, qscale, qmin,
                          quant_entry_stride, quant_rows, b0_pages, top_p, qk_scale, sink, recent, block_size,
                          lengths, length, sel_pages, logits, desired, union_rec, rec_stride, workspace,
                          workspace_bytes, false, 0, 0.0, nullptr, stream);
}

extern "C" int tw_twilight_select_fused_phase(const float* q, const void* page_min, const void* page_max, int dtype,
                                              int G, int R, int P, int D, int64_t page_group_stride,
                                              const uint8_t* packed, const void* qscale, const void* qmin,
                                              int64_t quant_entry_stride, int64_t quant_rows, int b0_pages,
                                              float top_p, float qk_scale, int sink, int recent, int block_size,
                                              const int32_t* lengths, int length, int32_t* sel_pages, float* logits,
                                              int32_t* desired, uint32_t* union_rec, int64_t rec_stride,
                                              void* workspace, size_t workspace_bytes, int phase, void* stream) {
  if (phase != 1 && phase != 3) return TW_EINVAL;
  return tw::select_fused(q, page_min, page_max, dtype, G, R, P, D, page_group_stride, packed, qscale, qmin,
                          quant_entry_stride, quant_rows, b0_pages, top_p, qk_scale, sink, recent, block_size,
                          lengths, length, sel_pages, logits, desired, union_rec, rec_stride, workspace,
                          workspace_bytes, false, 0, 0.0, nullptr, stream, phase);
}

extern "C" int tw_twilight_select_fused_matched(const float* q, const void* page_min, const void* page_max,
                                                int dtype, int G, int R, int P, int D, int64_t page_group_stride,
                                                const uint8_t* packed, const void* qscale, const void* qmin,
                                                int64_t quant_entry_stride, int64_t quant_rows, int b0_pages,
                                                float top_p, float qk_scale, int sink, int recent, int block_size,
                                                const int32_t* lengths, int length, int target_total,
                                                double matched_fraction, int32_t* sel_pages, float* logits,
                                                int32_t* desired, int32_t* allocated, uint32_t* union_rec,
                                                int64_t rec_stride, void* workspace, size_t workspace_bytes,
                                                void* stream) {
  return tw::select_fused(q, page_min, page_max, dtype, G, R, P, D, page_group_stride, packed, qscale, qmin,
                          quant_entry_stride, quant_rows, b0_pages, top_p, qk_scale, sink, recent, block_size,
                          lengths, length, sel_pages, logits, desired, union_rec, rec_stride, workspace,
                          workspace_bytes, true, target_total, matched_fraction, allocated, stream);
}

extern "C" int tw_twilight_select_fused_matched_part(
    const float* q, const void* page_min, const void* page_max, int dtype, int G, int R, int P, int D,
    int64_t page_group_stride, const uint8_t* packed, const void* qscale, const void* qmin,
    int64_t quant_entry_stride, int64_t quant_rows, int b0_pages, float top_p, float qk_scale, int sink, int recent,
    int block_size, const int32_t* lengths, int length, int target_total, double matched_fraction,
    int32_t* sel_pages, float* logits, int32_t* desired, int32_t* allocated, uint32_t* union_rec, int64_t rec_stride,
    int part, const int32_t* desired_all, int heads_all, int head0, void* workspace, size_t workspace_bytes,
    void* stream) {
  if ((part != 1 && part != 2) || desired_all == nullptr) return TW_EINVAL;
  return tw::select_fused(q, page_min, page_max, dtype, G, R, P, D, page_group_stride, packed, qscale, qmin,
                          quant_entry_stride, quant_rows, b0_pages, top_p, qk_scale, sink, recent, block_size,
                          lengths, length, sel_pages, logits, desired, union_rec, rec_stride, workspace,
                          workspace_bytes, true, target_total, matched_fraction, allocated, stream,
                          part == 1 ? 2 : 4, desired_all, heads_all, head0);
}
