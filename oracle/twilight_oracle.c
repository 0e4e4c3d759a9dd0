/*
 * twilight_oracle.c -- CPU restatement of the reference's sparse-decode KV
 * arithmetic.  TEST INFRASTRUCTURE ONLY: used by tests/, by smoke() and by
 * bench.py's cpu_baseline leg, to verify results and as the CPU baseline.  Nothing in the
 * product links or calls it.
 *
 * Scalar, single-threaded, IEEE single precision (x86-64 SSE, built with
 * -ffp-contract=off), every rounding step written out.  Each function cites
 * the reference file:line it restates (paths relative to
 * source/headinfer/headinfer/).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F16 = 0, OR_BF16 = 1, OR_F32 = 2 };

/* ------------------------------------------------------------ dtypes */
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else {
      int shift = 0;
      while (!(m & 0x400u)) { m <<= 1; ++shift; }
      m &= 0x3ffu;
      x = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  return u2f(x);
}

/* IEEE round-to-nearest-even, NaN -> 0x7e00 (sign kept). */
uint16_t or_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;
  if (ax >= 0x477ff000u) return sign | 0x7c00u;   /* >= 65520 rounds to inf */
  if (ax <= 0x33000000u) return sign;              /* <= 2^-25 rounds to 0 */
  int e = (int)(ax >> 23);
  uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  if (e < 113) {                                   /* half subnormal */
    int shift = 126 - e;
    uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return sign | (uint16_t)q;
  }
  uint32_t q = ((uint32_t)(e - 112) << 10) | ((m >> 13) & 0x3ffu);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  return sign | (uint16_t)q;
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int esize(int dt) { return dt == OR_F32 ? 4 : 2; }

static float load_f(const void* base, int64_t i, int dt) {
  if (dt == OR_F32) return ((const float*)base)[i];
  uint16_t h = ((const uint16_t*)base)[i];
  return dt == OR_F16 ? or_f16_to_f32(h) : or_bf16_to_f32(h);
}
static uint32_t load_bits(const void* base, int64_t i, int dt) {
  return dt == OR_F32 ? ((const uint32_t*)base)[i] : ((const uint16_t*)base)[i];
}
static void store_bits(void* base, int64_t i, int dt, uint32_t bits) {
  if (dt == OR_F32) ((uint32_t*)base)[i] = bits;
  else ((uint16_t*)base)[i] = (uint16_t)bits;
}
static uint32_t round_bits(float f, int dt) {
  if (dt == OR_F32) return f2u(f);
  return dt == OR_F16 ? or_f32_to_f16(f) : or_f32_to_bf16(f);
}
static float bits_f(uint32_t bits, int dt) {
  if (dt == OR_F32) return u2f(bits);
  return dt == OR_F16 ? or_f16_to_f32((uint16_t)bits) : or_bf16_to_f32((uint16_t)bits);
}
static int bits_nan(uint32_t b, int dt) {
  if (dt == OR_F32) return (b & 0x7fffffffu) > 0x7f800000u;
  if (dt == OR_F16) return (b & 0x7fffu) > 0x7c00u;
  return (b & 0x7fffu) > 0x7f80u;
}
static uint32_t canon_nan(int dt) { return dt == OR_F32 ? 0x7fc00000u : (dt == OR_F16 ? 0x7e00u : 0x7fc0u); }
/* IEEE total order on non-NaN values: -0 < +0. */
static uint32_t okey(uint32_t b, int dt) {
  if (dt == OR_F32) return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (b & 0x8000u) ? (uint32_t)(uint16_t)~b : (b | 0x8000u);
}

/* Min and max of n values (stride `stride`) in the total order; any NaN gives
 * the canonical NaN.  amin/amax of quest_offload_cache.py:288-289 and
 * twilight_offload_cache.py:29-30. */
static void minmax_bits(const void* base, int64_t start, int64_t stride, int64_t n, int dt, uint32_t* mn,
                        uint32_t* mx) {
  uint32_t bmn = 0, bmx = 0, kmn = 0xffffffffu, kmx = 0;
  int nan = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t b = load_bits(base, start + i * stride, dt);
    if (bits_nan(b, dt)) { nan = 1; continue; }
    uint32_t k = okey(b, dt);
    if (k < kmn) { kmn = k; bmn = b; }
    if (k >= kmx) { kmx = k; bmx = b; }
  }
  if (nan) { bmn = bmx = canon_nan(dt); }
  *mn = bmn;
  *mx = bmx;
}

/* ------------------------------------------------------------ metadata */
/* Page min/max (quest_offload_cache.py:276-289): pages = (T - sink) // bs
 * complete pages of rows [sink + p*bs, sink + (p+1)*bs).  INT4
 * (twilight_offload_cache.py:25-37) for every row.  Either output group may
 * be NULL. */
int or_build_page_metadata(const void* keys, int T, int D, int dt, int sink, int bs, void* page_min,
                           void* page_max, uint8_t* packed, void* scale, void* minimum) {
  if (T < 0 || D <= 0 || (D & 1) || bs <= 0 || sink < 0) return 1;
  if (page_min) {
    int pages = T > sink ? (T - sink) / bs : 0;
    for (int p = 0; p < pages; ++p) {
      for (int d = 0; d < D; ++d) {
        uint32_t mn, mx;
        minmax_bits(keys, (int64_t)(sink + p * bs) * D + d, D, bs, dt, &mn, &mx);
        store_bits(page_min, (int64_t)p * D + d, dt, mn);
        store_bits(page_max, (int64_t)p * D + d, dt, mx);
      }
    }
  }
  if (packed) {
    for (int t = 0; t < T; ++t) {
      uint32_t bmn, bmx;
      minmax_bits(keys, (int64_t)t * D, 1, D, dt, &bmn, &bmx);
      float mnf = bits_f(bmn, dt), mxf = bits_f(bmx, dt);
      /* (maximum - minimum) is computed in the key dtype */
      float diff = bits_f(round_bits(mxf - mnf, dt), dt);
      /* .float().clamp_min(1e-9): NaN propagates */
      if (diff < 1e-9f) diff = 1e-9f;
      float s = diff / 15.0f;
      uint32_t sbits = round_bits(s, dt);
      float sf = bits_f(sbits, dt);
      for (int j = 0; j < D / 2; ++j) {
        uint32_t code[2];
        for (int h = 0; h < 2; ++h) {
          float k = load_f(keys, (int64_t)t * D + 2 * j + h, dt);
          float c = rintf((k - mnf) / sf); /* torch.round: half to even */
          if (c < 0.0f) c = 0.0f;          /* clamp_(0, 15); NaN stays NaN */
          if (c > 15.0f) c = 15.0f;
          code[h] = (c == c) ? (uint32_t)c : 0u; /* NaN code stored as 0 */
        }
        packed[(int64_t)t * (D / 2) + j] = (uint8_t)(code[0] | (code[1] << 4));
      }
      store_bits(scale, t, dt, sbits);
      store_bits(minimum, t, dt, bmn);
    }
  }
  return 0;
}

/* affine_int4_dequantize (twilight_offload_cache.py:40-47). */
void or_int4_dequantize(const uint8_t* packed, const void* scale, const void* minimum, int dt, int64_t N, int D,
                        float* out) {
  for (int64_t n = 0; n < N; ++n) {
    float s = load_f(scale, n, dt), m = load_f(minimum, n, dt);
    for (int d = 0; d < D; ++d) {
      uint32_t b = packed[n * (D / 2) + d / 2];
      uint32_t code = (d & 1) ? (b >> 4) & 15u : b & 15u;
      float prod = (float)code * s;
      out[n * D + d] = prod + m;
    }
  }
}

/* ------------------------------------------------ Quest page score */
/* twilight_fused_quest.py:12-32: 32 lanes, lane l accumulates channels
 * l, l+32, l+64, l+96 (chunk order) starting from 0; then shuffle-adds at
 * offsets 1, 2, 4, 8, 16 and lane 0's value is the score.  Lane 0's value
 * after those shuffle-adds is the adjacent-pair tree over the 32 lanes. */
float or_quest_score_one(const float* q, const void* lo, const void* hi, int64_t off, int D, int dt) {
  float acc[32];
  for (int l = 0; l < 32; ++l) acc[l] = 0.0f;
  for (int c = 0; c * 32 < D; ++c) {
    for (int l = 0; l < 32; ++l) {
      int d = c * 32 + l;
      if (d >= D) continue;
      float ext = q[d] > 0.0f ? load_f(hi, off + d, dt) : load_f(lo, off + d, dt);
      float prod = ext * q[d];
      acc[l] = acc[l] + prod;
    }
  }
  for (int shift = 1; shift < 32; shift <<= 1) {
    float nxt[32];
    for (int l = 0; l < 32; ++l) nxt[l] = acc[l] + acc[(l + shift) % 32];
    memcpy(acc, nxt, sizeof(acc));
  }
  return acc[0];
}

void or_quest_score(const float* q, const void* page_min, const void* page_max, int dt, int G, int R, int P, int D,
                    int64_t group_stride, float* out) {
  for (int g = 0; g < G; ++g)
    for (int r = 0; r < R; ++r)
      for (int p = 0; p < P; ++p)
        out[((int64_t)g * R + r) * P + p] =
            or_quest_score_one(q + ((int64_t)g * R + r) * D, page_min, page_max, g * group_stride + (int64_t)p * D,
                               D, dt);
}

/* ------------------------------------------------ top-k, sorted */
/* torch.topk(sorted=False).indices.sort() (quest_offload_cache.py:373-374)
 * with ties to the lowest index, NaN ranked highest and -0 == +0. */
static uint32_t score_key(float s) {
  uint32_t u = f2u(s);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
typedef struct { uint32_t key; int32_t idx; } kv_t;
static int cmp_desc(const void* a, const void* b) {
  const kv_t* x = (const kv_t*)a;
  const kv_t* y = (const kv_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}
static int cmp_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return x < y ? -1 : (x > y);
}
void or_topk_sorted(const float* scores, int rows, int P, int64_t stride, int k, int64_t* out) {
  kv_t* tmp = (kv_t*)malloc(sizeof(kv_t) * (size_t)P);
  for (int r = 0; r < rows; ++r) {
    for (int p = 0; p < P; ++p) { tmp[p].key = score_key(scores[r * stride + p]); tmp[p].idx = p; }
    qsort(tmp, (size_t)P, sizeof(kv_t), cmp_desc);
    for (int i = 0; i < k; ++i) out[(int64_t)r * k + i] = tmp[i].idx;
    qsort(out + (int64_t)r * k, (size_t)k, sizeof(int64_t), cmp_i64);
  }
  free(tmp);
}

/* --------------------------------------------------- GQA row plan */
/* Per group: [0, sink_end) ++ every page selected by any of the R heads
 * (ascending, each expanded to sink + p*bs + [0, bs), quest_offload_cache.py:
 * 484-490) ++ [recent_start, length) ++ append_position (if >= 0).  Window
 * per quest_offload_cache.py:330-332.  masks: heads that see each row.
 * Returns the row count. */
int or_quest_row_plan(const int64_t* sel, int R, int k, int P, int sink, int recent, int bs, int length,
                      int append_position, int32_t* rows, uint8_t* masks) {
  uint8_t* pm = (uint8_t*)calloc((size_t)(P > 0 ? P : 1), 1);
  for (int r = 0; r < R; ++r)
    for (int i = 0; i < k; ++i) pm[sel[(int64_t)r * k + i]] |= (uint8_t)(1u << r);
  int sink_end = sink < length ? sink : length;
  int hist_recent = recent - 1 > 0 ? recent - 1 : 0;
  int recent_start = length - hist_recent > sink_end ? length - hist_recent : sink_end;
  uint8_t all = (uint8_t)((1u << R) - 1u);
  int n = 0;
  for (int t = 0; t < sink_end; ++t) { rows[n] = t; masks[n++] = all; }
  for (int p = 0; p < P; ++p) {
    if (!pm[p]) continue;
    for (int i = 0; i < bs; ++i) { rows[n] = sink + p * bs + i; masks[n++] = pm[p]; }
  }
  for (int t = recent_start; t < length; ++t) { rows[n] = t; masks[n++] = all; }
  if (append_position >= 0) { rows[n] = append_position; masks[n++] = all; }
  free(pm);
  return n;
}

/* ================================================================ Twilight */
/* Deterministic exp of x <= 0, the one definition the GPU kernels share:
 *   x < -28 -> 0 (e^-28 < 2^-40, below the top-p mass resolution);
 *   t = x * log2(e) (fp32), n = round-half-even(t), f = t - n (exact),
 *   2^f by its Taylor polynomial sum_k (ln 2)^k f^k / k! to degree 6 in
 *   Horner form (separate multiply and add), scaled by 2^n exactly.
 * Every step is one IEEE fp32 operation, so CPU and GPU agree bit for bit. */
float or_det_exp(float x) {
  if (!(x >= -28.0f)) return 0.0f;
  const float t = x * 1.44269504088896341f;
  const float n = rintf(t);
  const float f = t - n;
  float p = 1.54035303933816e-4f;
  p = p * f + 1.33335581464284e-3f;
  p = p * f + 9.61812910762848e-3f;
  p = p * f + 5.55041086648216e-2f;
  p = p * f + 2.40226506959101e-1f;
  p = p * f + 6.93147180559945e-1f;
  p = p * f + 1.0f;
  return ldexpf(p, (int)n);
}

/* Fixed-point form of one query head for the INT4 QK estimate:
 * M = max_d |q_d|, E the exponent of M (M = f * 2^E, f in [0.5, 1)), and
 * Q_d = round_half_even(q_d * 2^(22 - E)), so |Q_d| <= 2^22.  Returns the
 * shift E - 22 that scales an integer dot product back, with *qs = sum_d Q_d;
 * *ok = 0 when a q_d is not finite (the estimate is then NaN); M = 0 gives
 * Q = 0 and shift 0. */
int or_qfix(const float* q, int D, int32_t* Q, int32_t* qs, int* ok) {
  float M = 0.0f;
  *ok = 1;
  for (int d = 0; d < D; ++d) {
    if (!isfinite(q[d])) *ok = 0;
    const float a = fabsf(q[d]);
    M = a > M ? a : M;
  }
  int32_t sum = 0;
  if (!*ok || M == 0.0f) {
    for (int d = 0; d < D; ++d) Q[d] = 0;
    *qs = 0;
    return 0;
  }
  int E = 0;
  (void)frexpf(M, &E);
  for (int d = 0; d < D; ++d) {
    Q[d] = (int32_t)rintf(ldexpf(q[d], 22 - E));
    sum += Q[d];
  }
  *qs = sum;
  return E - 22;
}

/* INT4 QK estimate of one query head (twilight_fused_qk.py:12-55,
 * twilight_offload_cache.py:1197-1261) in the arithmetic defined here.
 * The reference dequantizes k_d = f32(code_d) * f32(scale) + f32(min)
 * (:40-47) and reduces k . q in an unpinned fp32 order (cuBLAS / tl.sum).
 * Here the dot product is exact: with q in the fixed-point form of or_qfix,
 *   S = sum_d code_d * Q_d                      (exact integer, int64)
 *   dotc = ldexp(f32(S), shift), qsum = ldexp(f32(sum_d Q_d), shift)
 *   logit = qk_scale * ((scale * dotc) + (min * qsum))   (each op rounded)
 * which is sum_d (code_d * scale + min) * q~_d for q~ = Q * 2^shift, with
 * one rounding per fp32 operation.  rows[n] selects the packed row of
 * candidate n (low nibble = even channel).  D = 4 .. 256, a power of two. */
void or_int4_qk(const float* q, int D, const uint8_t* packed, const void* scale, const void* minimum, int dt,
                const int64_t* rows, int N, float qk_scale, float* out) {
  int32_t Q[256];
  int32_t qs = 0;
  int ok = 1;
  const int shift = or_qfix(q, D, Q, &qs, &ok);
  const float qsum = ldexpf((float)qs, shift);
  for (int n = 0; n < N; ++n) {
    const int64_t t = rows[n];
    if (!ok) {
      out[n] = u2f(0x7fc00000u);
      continue;
    }
    const float s = load_f(scale, t, dt), m = load_f(minimum, t, dt);
    int64_t S = 0;
    for (int d = 0; d < D; ++d) {
      const uint32_t b = packed[t * (D / 2) + d / 2];
      const uint32_t code = (d & 1) ? (b >> 4) & 15u : b & 15u;
      S += (int64_t)code * Q[d];
    }
    const float dotc = ldexpf((float)S, shift);
    const float a = s * dotc;
    const float c = m * qsum;
    out[n] = qk_scale * (a + c);
  }
}

/* Top-p count (twilight_exact_top_p_graph.py:19-32; inline
 * twilight_offload_cache.py:1274-1310) in the exact definition used here:
 *   e_i = det_exp(l_i - max l), mass E_i = floor(e_i * 2^40) (int64),
 *   Z = sum E_i, T = ceil(P24 * Z / 2^24) with P24 = round(top_p * 2^24),
 *   desired = the smallest c >= 1 such that the c largest logits (ties to the
 *   lowest index) carry mass >= T; at most N.
 * All sums are exact integers, so the count does not depend on a summation
 * order (the reference's fp32 argsort/softmax/cumsum order is unpinned).
 * Returns desired; *z_out (nullable) gets Z. */
typedef struct { uint32_t key; int32_t idx; } lk_t;
static int cmp_lk(const void* a, const void* b) {
  const lk_t* x = (const lk_t*)a;
  const lk_t* y = (const lk_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}
uint64_t or_top_p_threshold(uint64_t z, float top_p) {
  const uint64_t p24 = (uint64_t)rintf(top_p * 16777216.0f);
  const unsigned __int128 prod = (unsigned __int128)p24 * z;
  return (uint64_t)((prod + ((1u << 24) - 1u)) >> 24);
}
uint64_t or_mass(float logit, float lmax) {
  const float e = or_det_exp(logit - lmax);
  return (uint64_t)(e * 1099511627776.0f); /* 2^40, exact scaling; truncation */
}
int or_top_p_count(const float* logits, int N, float top_p, uint64_t* z_out) {
  if (N <= 0) return 0;
  float lmax = logits[0];
  for (int i = 1; i < N; ++i) lmax = logits[i] > lmax ? logits[i] : lmax;
  lk_t* v = (lk_t*)malloc(sizeof(lk_t) * (size_t)N);
  uint64_t z = 0;
  for (int i = 0; i < N; ++i) {
    v[i].key = score_key(logits[i]);
    v[i].idx = i;
    z += or_mass(logits[i], lmax);
  }
  const uint64_t T = or_top_p_threshold(z, top_p);
  qsort(v, (size_t)N, sizeof(lk_t), cmp_lk);
  int desired = N;
  uint64_t cum = 0;
  for (int c = 0; c < N; ++c) {
    cum += or_mass(logits[v[c].idx], lmax);
    if (cum >= T) { desired = c + 1; break; }
  }
  free(v);
  if (z_out) *z_out = z;
  return desired;
}
