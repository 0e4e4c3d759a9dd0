// Block-wide exact top-k over register-resident keys, shared by the Quest
// page selection and the Twilight token selection.
//
// A block of NT threads (256 or more) holds one row of scores as KPT
// contiguous order keys per thread (score_key: NaN highest, -0 == +0).  A
// pass histograms the remaining candidates into bins that are monotone in
// the key -- 2048 bins linear in the score value over the candidates' range
// when that range is finite, else the next 8-bit digit below the candidates'
// common key prefix -- finds the bin holding the k-th largest, takes every
// candidate above it and keeps the bin's keys as the next candidates.  At
// most 256 candidates (kExactMax, whatever NT) are ranked exactly by (key
// desc, index asc); equal candidates are taken lowest index first.  The
// winners are reported in ascending index order.
#pragma once

#include "tw_common.h"

namespace tw {
namespace sel {

constexpr int kBlock = 256;  // threads of a selection block unless a kernel says otherwise
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxSelPages = 8192;  // longest row
constexpr int kLinBins = 2048;
constexpr int kExactMax = 256;      // at most this many candidates are ranked pairwise
// Bins of the fast path's single pass: 8 per lane keep each wavefront's
// in-lane boundary search short; the boundary bin then holds a few keys.
constexpr int kFastBins = 512;

// Block-shared state of a selection block of NT threads (NT a multiple of
// 256: the linear bins split evenly over the threads).
template <int NT>
struct SelSharedT {
  static constexpr int kW = NT / kWave;
  static_assert(NT % 256 == 0 && NT <= kLinBins, "whole bins per thread");
  uint32_t hist[kLinBins + 64];
  uint32_t ckey[kExactMax];
  int32_t cidx[kExactMax];
  uint32_t selbits[kMaxSelPages / 32];
  uint32_t red_max[kW];
  uint32_t red_min[kW];
  int scan[kW];
  unsigned long long tmask;
  int bnd;
  uint32_t bnd_above;
  uint32_t bnd_count;
  int flag;
  // fast path: boundary candidates as (key << 32) | ~index, so that one
  // unsigned compare orders them by (key desc, index asc); unused slots are
  // 0, which never outranks a candidate
  unsigned long long cpair[kWave];
  uint32_t ncand;      // fast path: staging slots handed out
};
using SelShared = SelSharedT<kBlock>;

__device__ __forceinline__ float key_value(uint32_t key) { return __uint_as_float(from_order_key32(key)); }

// Exclusive prefix of v over the block's NT threads (thread order); *total
// gets the block sum.  scan: NT / 64 ints.  Two barriers, so consecutive
// calls never race on scan[].
template <int NT>
__device__ __forceinline__ int block_excl_scan(int v, int* scan, int* total) {
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int incl = wave_prefix_sum_i32(v);
  if (lane == kWave - 1) scan[wave] = incl;
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) {
    const int t = scan[w];
    before += w < wave ? t : 0;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return before + incl - v;
}

// Bin of a key in the current pass: linear in the value (2048 bins) or an
// 8-bit digit of the key.  Both are monotone over the candidates.
struct BinFn {
  bool linear;
  float vmin, scale;
  int shift;
  __device__ __forceinline__ int operator()(uint32_t key) const {
    if (linear) {
      const int b = static_cast<int>((key_value(key) - vmin) * scale);
      return b < kLinBins - 1 ? b : kLinBins - 1;
    }
    return static_cast<int>((key >> shift) & 255u);
  }
};

// Top-k of one row held as KPT contiguous keys per thread (indices
// KPT*t .. KPT*t + KPT - 1).  On return, bit j of *take marks index
// KPT*t + j as selected, and *first is the rank (in ascending index order)
// of this thread's first selected index among all selected ones.
template <int KPT, int NT>
__device__ void block_topk(const uint32_t (&key)[KPT], int P, int k, SelSharedT<NT>& sh, uint32_t* take,
                           int* first) {
  constexpr int kW = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int i0 = KPT * tid;
  uint32_t cand = 0u, taken = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) cand |= (i0 + j < P) ? (1u << j) : 0u;
  uint32_t need = static_cast<uint32_t>(k);
  uint32_t ccount = static_cast<uint32_t>(P);
  // 0: take every candidate, 1: exact rank, 2: equal keys, lowest indices
  int mode = 0;
  uint4* hist4 = reinterpret_cast<uint4*>(sh.hist);
  for (int level = 0;; ++level) {
    if (ccount == need) break;
    // after a pass, few candidates go straight to the exact rank (it orders
    // equal keys by index too), with no bounds reduction
    if (level > 0 && ccount <= static_cast<uint32_t>(kExactMax)) {
      mode = 1;
      break;
    }
    uint32_t cmax = 0u, cmin = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool c = (cand >> j) & 1u;
      cmax = (c && key[j] > cmax) ? key[j] : cmax;
      cmin = (c && key[j] < cmin) ? key[j] : cmin;
    }
    cmax = wave_max_u32(cmax);
    cmin = wave_min_u32(cmin);
    if (lane == 0) {
      sh.red_max[wave] = cmax;
      sh.red_min[wave] = cmin;
    }
    // the histogram is cleared in the same barrier interval: the previous
    // pass's reads of it ended at its last barrier
    for (int b = tid; b < (kLinBins + 64) / 4; b += NT) hist4[b] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      cmax = sh.red_max[w] > cmax ? sh.red_max[w] : cmax;
      cmin = sh.red_min[w] < cmin ? sh.red_min[w] : cmin;
    }
    if (cmax == cmin) {
      mode = 2;
      break;
    }
    if (ccount <= static_cast<uint32_t>(kExactMax)) {
      mode = 1;
      break;
    }
    BinFn fn;
    const float vmin = key_value(cmin);
    const float vmax = key_value(cmax);
    const float range = vmax - vmin;
    fn.vmin = vmin;
    fn.scale = static_cast<float>(kLinBins) / range;
    // A few linear passes resolve real score distributions; after that (or
    // for non-finite ranges) the digit passes bound the work at 4 more.
    fn.linear = level < 3 && __builtin_isfinite(vmin) && __builtin_isfinite(vmax) && __builtin_isfinite(range) &&
                range > 0.0f && __builtin_isfinite(fn.scale);
    const int hi = 31 - __clz(static_cast<int>(cmax ^ cmin));
    fn.shift = hi >= 7 ? hi - 7 : 0;
    int bin[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      bin[j] = fn(key[j]);
      if ((cand >> j) & 1u) atomicAdd(&sh.hist[bin[j]], 1u);
    }
    __syncthreads();
    // thread t owns bins kBpt t .. kBpt t + kBpt - 1 (linear) or bin t (digit)
    constexpr int kBpt = kLinBins / NT;
    static_assert(kBpt == 2 || kBpt == 4 || kBpt == 8, "16-byte or 8-byte histogram reads");
    uint32_t hv[kBpt];
    if (fn.linear) {
      if constexpr (kBpt == 2) {
        const uint2 h0 = reinterpret_cast<const uint2*>(sh.hist)[tid];
        hv[0] = h0.x; hv[1] = h0.y;
      } else {
#pragma unroll
        for (int q = 0; q < kBpt / 4; ++q) {
          const uint4 h = hist4[kBpt / 4 * tid + q];
          hv[4 * q] = h.x; hv[4 * q + 1] = h.y; hv[4 * q + 2] = h.z; hv[4 * q + 3] = h.w;
        }
      }
    } else {
      hv[0] = sh.hist[tid];
#pragma unroll
      for (int b = 1; b < kBpt; ++b) hv[b] = 0u;
    }
    uint32_t tot = 0u;
#pragma unroll
    for (int b = 0; b < kBpt; ++b) tot += hv[b];
    // suffix sums over threads (bins descending)
    const uint32_t wincl = wave_suffix_sum_u32(tot);
    if (lane == 0) sh.scan[wave] = static_cast<int>(wincl);
    __syncthreads();
    uint32_t incl = wincl;
#pragma unroll
    for (int w = 0; w < kW; ++w) incl += w > wave ? static_cast<uint32_t>(sh.scan[w]) : 0u;
    if (incl - tot < need && need <= incl) {
      uint32_t acc = incl - tot;
      int bsel = 0;
      uint32_t cnt = 0u;
      bool found = false;
#pragma unroll
      for (int b = kBpt - 1; b >= 0; --b) {
        const bool hit = !found && need <= acc + hv[b];
        bsel = hit ? b : bsel;
        cnt = hit ? hv[b] : cnt;
        acc += (found || hit) ? 0u : hv[b];
        found = found || hit;
      }
      sh.bnd = fn.linear ? kBpt * tid + bsel : tid;
      sh.bnd_above = acc;
      sh.bnd_count = cnt;
    }
    __syncthreads();
    const int bnd = sh.bnd;
    need -= sh.bnd_above;
    ccount = sh.bnd_count;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool c = (cand >> j) & 1u;
      taken |= (c && bin[j] > bnd) ? (1u << j) : 0u;
      cand &= (c && bin[j] == bnd) ? 0xffffffffu : ~(1u << j);
    }
  }
  int total;
  if (mode == 1 && ccount > static_cast<uint32_t>(kWave)) {
    // exact rank of at most kExactMax candidates; slot t's rank goes to
    // selbits[t] and back to the thread that owns slot t
    static_assert(kMaxSelPages / 32 >= kExactMax, "one rank per candidate slot");
    const int first = block_excl_scan<NT>(__popc(cand), sh.scan, &total);
    int slot = first;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if ((cand >> j) & 1u) {
        sh.ckey[slot] = key[j];
        sh.cidx[slot] = i0 + j;
        ++slot;
      }
    }
    __syncthreads();
    if (tid < static_cast<int>(ccount)) {
      const uint32_t mk = sh.ckey[tid];
      const int mi = sh.cidx[tid];
      uint32_t rank = 0u;
      for (int m = 0; m < static_cast<int>(ccount); ++m) {
        const uint32_t km = sh.ckey[m];
        const int im = sh.cidx[m];
        rank += (km > mk || (km == mk && im < mi)) ? 1u : 0u;
      }
      sh.selbits[tid] = rank;
    }
    __syncthreads();
    slot = first;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if ((cand >> j) & 1u) {
        taken |= sh.selbits[slot] < need ? (1u << j) : 0u;
        ++slot;
      }
    }
    cand = 0u;
    mode = 0;
  }
  if (mode == 0) {
    taken |= cand;
    cand = 0u;
  }
  // One scan gives both the taken keys (low half) and the candidates (high
  // half) in earlier threads; candidate c (in index order) is taken when
  // its rank is below need (mode 1: tmask bit c) or c < need (mode 2).
  const int pre = block_excl_scan<NT>(__popc(taken) | (__popc(cand) << 16), sh.scan, &total);
  const int a_before = pre & 0xffff;
  const int c_before = pre >> 16;
  uint64_t tmask = 0ull;
  if (mode == 1) {
    // at most one wavefront of candidates: staged in index order, ranked by
    // (key desc, index asc) in wavefront 0
    int slot = c_before;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if ((cand >> j) & 1u) sh.ckey[slot++] = key[j];
    }
    __syncthreads();
    if (wave == 0) {
      const int n = static_cast<int>(ccount);
      const uint32_t mk = lane < n ? sh.ckey[lane] : 0u;
      uint32_t rank = 0u;
      for (int m = 0; m < n; ++m) {
        const uint32_t km = readlane_u32(mk, m);
        rank += (km > mk || (km == mk && m < lane)) ? 1u : 0u;
      }
      const uint64_t t = __ballot(lane < n && rank < need);
      if (lane == 0) sh.tmask = t;
    }
    __syncthreads();
    tmask = sh.tmask;
  }
  int out = a_before;
  if (mode == 1) {
    out += c_before > 0 ? __popcll(tmask & (~0ull >> (64 - c_before))) : 0;
  } else {
    out += c_before < static_cast<int>(need) ? c_before : static_cast<int>(need);
  }
  int cpos = c_before;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const bool c = (cand >> j) & 1u;
    const bool t = mode == 1 ? ((tmask >> cpos) & 1ull) != 0ull : cpos < static_cast<int>(need);
    taken |= (c && t) ? (1u << j) : 0u;
    cpos += c ? 1 : 0;
  }
  *take = taken;
  *first = out;
}

// Clears the fast path's histogram and staging counter.  The caller puts a
// barrier between this and block_topk_fast (at kernel entry, ahead of the
// key loads, so the barrier does not wait for them).
template <int NT>
__device__ __forceinline__ void topk_fast_clear(SelSharedT<NT>& sh) {
  uint4* hist4 = reinterpret_cast<uint4*>(sh.hist);
  for (int b = threadIdx.x; b < kFastBins / 4; b += NT) hist4[b] = make_uint4(0u, 0u, 0u, 0u);
  if (threadIdx.x < kWave) sh.cpair[threadIdx.x] = 0ull;
  if (threadIdx.x == 0) sh.ncand = 0u;
}

// Packed rank key of a candidate (see cpair).
__device__ __forceinline__ unsigned long long rank_key(uint32_t key, int index) {
  return (static_cast<unsigned long long>(key) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(index));
}

// Staging slots for the candidates of a thread whose bits are set in sel
// (bit j = its j-th key): one LDS atomic per wavefront hands out a run of
// slots (the wavefront's total) and each thread takes its part of the run
// in lane order.  Returns the thread's first slot.
__device__ __forceinline__ uint32_t stage_slots(uint32_t sel, uint32_t* counter) {
  const uint32_t n = static_cast<uint32_t>(__popc(sel));
  const uint32_t incl = static_cast<uint32_t>(wave_prefix_sum_i32(static_cast<int>(n)));
  const uint32_t total = readlane_u32(incl, kWave - 1);
  uint32_t base = 0u;
  if (lane_id() == kWave - 1 && total != 0u) base = atomicAdd(counter, total);
  base = readlane_u32(base, kWave - 1);
  return base + incl - n;
}

// Fast path of block_topk for a row whose key range [kmin, kmax] is known
// before the keys are looked at (the score kernel reduces it per tile).  One
// pass of kFastBins bins linear in the value over that range (histogram cleared
// by topk_fast_clear), every wavefront then scans the bins itself (8 per
// lane, a wavefront suffix sum, no barrier) and finds the bin holding the
// k-th largest; at most 64 keys of that bin are staged through an LDS slot
// counter and every wavefront ranks them by (key desc, index asc) with
// readlane, four at a time.  Two barriers after the clear.  Returns false --
// block-uniformly, the caller then runs block_topk -- when the range is not
// finite and positive or the boundary bin holds more than 64 keys.  On true,
// bit j of *take marks index KPT*t + j as selected: the same set block_topk
// selects.
template <int KPT, int NT>
__device__ bool block_topk_fast(const uint32_t (&key)[KPT], int P, int k, uint32_t kmin, uint32_t kmax,
                                SelSharedT<NT>& sh, uint32_t* take) {
  constexpr int kBins = kFastBins;
  constexpr int kBpl = kBins / kWave;  // bins per lane
  static_assert(kBpl % 4 == 0, "16-byte bin reads");
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int i0 = KPT * tid;
  if (k >= P) {
    uint32_t t = 0u;
#pragma unroll
    for (int j = 0; j < KPT; ++j) t |= (i0 + j < P) ? (1u << j) : 0u;
    *take = t;
    return true;
  }
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
    bin[j] = (i0 + j < P) ? (b < kBins - 1 ? b : kBins - 1) : -1;
    if (bin[j] >= 0) atomicAdd(&sh.hist[bin[j]], 1u);
  }
  __syncthreads();
  // lane l: bins kBpl*l ..; the suffix over lanes counts the bins above
  const uint4* hist4 = reinterpret_cast<const uint4*>(sh.hist);
  uint32_t hv[kBpl];
#pragma unroll
  for (int q = 0; q < kBpl / 4; ++q) {
    const uint4 h = hist4[kBpl / 4 * lane + q];
    hv[4 * q] = h.x;
    hv[4 * q + 1] = h.y;
    hv[4 * q + 2] = h.z;
    hv[4 * q + 3] = h.w;
  }
  uint32_t tot = 0u;
#pragma unroll
  for (int b = 0; b < kBpl; ++b) tot += hv[b];
  const uint32_t incl = wave_suffix_sum_u32(tot);
  const uint32_t need = static_cast<uint32_t>(k);
  // lanes 0 .. L have incl >= need (incl does not grow with the lane)
  const uint64_t bl = __ballot(incl >= need);
  const int L = 63 - __clzll(static_cast<long long>(bl));
  uint32_t acc = incl - tot;
  int bsel = 0;
  uint32_t cnt = 0u;
  bool found = false;
#pragma unroll
  for (int b = kBpl - 1; b >= 0; --b) {
    const bool hit = !found && need <= acc + hv[b];
    bsel = hit ? b : bsel;
    cnt = hit ? hv[b] : cnt;
    acc += (found || hit) ? 0u : hv[b];
    found = found || hit;
  }
  const int bnd = kBpl * L + static_cast<int>(readlane_u32(static_cast<uint32_t>(bsel), L));
  const uint32_t above = readlane_u32(acc, L);
  const uint32_t ccount = readlane_u32(cnt, L);
  if (ccount > static_cast<uint32_t>(kWave)) {
    __syncthreads();  // every wavefront is done with the bins before block_topk reuses them
    return false;
  }
  const uint32_t need2 = need - above;  // 1 .. ccount
  uint32_t t = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) t |= (bin[j] > bnd) ? (1u << j) : 0u;
  if (need2 == ccount) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) t |= (bin[j] == bnd) ? (1u << j) : 0u;
    *take = t;
    return true;
  }
  uint32_t inbin = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) inbin |= (bin[j] == bnd) ? (1u << j) : 0u;
  uint32_t cslot[KPT];
  {
    uint32_t slot = stage_slots(inbin, &sh.ncand);
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      cslot[j] = slot;
      if ((inbin >> j) & 1u) sh.cpair[slot] = rank_key(key[j], i0 + j);
      slot += (inbin >> j) & 1u;
    }
  }
  __syncthreads();
  // every wavefront ranks the staged candidates (lane m holds candidate m)
  // against all of them, read from LDS by every lane at once (broadcast
  // reads, four in flight): one 64-bit compare each, no branch (the slots
  // past ccount are 0 and never count), and no barrier hands the ranks back
  const unsigned long long c = sh.cpair[lane];
  uint32_t rank = 0u;
  for (int m = 0; m < static_cast<int>(ccount); m += 4) {
    unsigned long long o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = sh.cpair[m + u];
#pragma unroll
    for (int u = 0; u < 4; ++u) rank += o[u] > c ? 1u : 0u;
  }
  const uint64_t tm = __ballot(static_cast<uint32_t>(lane) < ccount && rank < need2);
#pragma unroll
  for (int j = 0; j < KPT; ++j) t |= (((inbin >> j) & 1u) && ((tm >> cslot[j]) & 1ull)) ? (1u << j) : 0u;
  *take = t;
  return true;
}

// Candidate pages of a group with `length` tokens: the whole pages between
// the sink and the recent window (quest_offload_cache.py:326-346), at most
// P_max.
__device__ __forceinline__ int ragged_pages(int length, int sink, int recent, int bs, int P_max) {
  length = length < 0 ? 0 : length;
  const int sink_end = sink < length ? sink : length;
  const int hist_recent = recent - 1 > 0 ? recent - 1 : 0;
  const int recent_start = (length - hist_recent) > sink_end ? (length - hist_recent) : sink_end;
  const int cand = (recent_start - sink_end) / bs;
  return cand < P_max ? cand : P_max;
}

}  // namespace sel
}  // namespace tw
