/*
 * vkv_oracle.c -- CPU restatement of the reference's KV-cache arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see vkv_oracle.h).  Built with
 * -ffp-contract=off so every float expression rounds exactly as written:
 * the quantizer below must reproduce the reference's fp32 arithmetic bit for
 * bit, and a fused multiply-add would change its rounding.
 *
 * Parity pins for this file (tests/test_oracle_golden.py):
 *   vkvo_quantize   -- IntegrationTests.swift:3890-3923 aggregates on the
 *                      reproduced MLX stream (seed 869), plus closed-form
 *                      invariants and a brute-force tiny-alphabet sweep.
 *   vkvo_dequantize -- both rules against independent library arithmetic
 *                      (numpy fp64 + torch casts), |w - deq| <= |scale|/2
 *                      away from the clamp, exact edge reconstruction; which
 *                      rule the reference uses is unpinned (counted).
 *   vkvo_sdpa       -- MLXFastKernelTests.swift:101-111 known answer (seed 0),
 *                      single-key / uniform-score / fully-masked special cases.
 *   vkvo_quantized_sdpa -- exact mode equals vkvo_sdpa on the dequantized
 *                      cache with the input-dtype query scaling; rounding
 *                      modes pinned by closed-form cases (scores closer than
 *                      half a T ulp weigh the same; three equal scores give
 *                      weights T(1/3)); fully masked row = mean(V).
 *   vkvo_mla_decode -- equals vkvo_sdpa with Hkv = 1 on dequantized entries.
 *   conversions     -- exhaustive bf16/f16 round trips and numpy's f16 cast.
 */
#include "vkv_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t vkvo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float vkvo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t vkvo_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: inf */
  if (a >= 0x38800000u) {                                  /* normal f16 */
    uint32_t r = a + 0x0fffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
  }
  if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to zero */
  /* subnormal f16: value = m * 2^-24 with m = round(a_value * 2^24) */
  {
    uint32_t e = a >> 23;                 /* 102..112 */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;            /* 14..24: m >> shift = integer part */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
}

float vkvo_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t m = (uint32_t)h & 0x3ffu;
  if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float load_val(const void *p, int dtype, int64_t i) {
  switch (dtype) {
    case 1: return vkvo_f16_to_f32(((const uint16_t *)p)[i]);
    case 2: return vkvo_bf16_to_f32(((const uint16_t *)p)[i]);
    default: return ((const float *)p)[i];
  }
}

static inline void store_val(void *p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case 1: ((uint16_t *)p)[i] = vkvo_f32_to_f16(v); break;
    case 2: ((uint16_t *)p)[i] = vkvo_f32_to_bf16(v); break;
    default: ((float *)p)[i] = v; break;
  }
}

static inline float round_to(float v, int dtype) {
  switch (dtype) {
    case 1: return vkvo_f16_to_f32(vkvo_f32_to_f16(v));
    case 2: return vkvo_bf16_to_f32(vkvo_f32_to_bf16(v));
    default: return v;
  }
}

void vkvo_to_f32(const void *src, int dtype, int64_t n, float *dst) {
  for (int64_t i = 0; i < n; i++) dst[i] = load_val(src, dtype, i);
}

void vkvo_from_f32(const float *src, int64_t n, int dtype, void *dst) {
  for (int64_t i = 0; i < n; i++) store_val(dst, dtype, i, src[i]);
}

/* Largest finite value of the element type: the Metal kernel starts its
 * running minimum there (quantized.h:2422, Limits<T>::max). */
static float type_max(int dtype) {
  switch (dtype) {
    case 1: return 65504.0f;
    case 2: return u2f(0x7f7f0000u);
    default: return FLT_MAX;
  }
}

/* Lowest finite value: the fill of masked scores (KVCache.swift:1950-1975). */
static double type_lowest(int dtype) {
  switch (dtype) {
    case 1: return -65504.0;
    case 2: return -(double)u2f(0x7f7f0000u);
    default: return -(double)FLT_MAX;
  }
}

static inline int is_tie(float x) { return fabsf(x - truncf(x)) == 0.5f; }

/* quantized.h:2393-2497 (affine_quantize).  Group statistics in fp32 with
 * the running max starting at 0 and the running min at Limits<T>::max
 * (:2422-2431); scale = max((max - min) / n_bins, 1e-7) (:2436); the edge
 * with the larger magnitude is represented exactly: scale is negated when
 * the max is the edge (:2437-2438), q0 = round(edge / scale), and unless q0
 * is zero the scale is re-derived as edge / q0 with bias = edge (:2439-2443).
 * Codes use the unrounded fp32 scale/bias: min(round((w - bias) / scale),
 * n_bins) (:2458); scale/bias are then stored cast to T (:2447-2450).  Metal
 * round() is half away from zero, the same as C roundf. */
int64_t vkvo_quantize(const void *w, int dtype, int64_t rows, int D, int group,
                      int bits, uint32_t *wq, void *scales, void *biases) {
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int per_word = 32 / bits;
  const int words_per_row = D / per_word;
  const int groups = D / group;
  int64_t ties = 0;
  float *vals = (float *)malloc(sizeof(float) * (size_t)group);
  for (int64_t r = 0; r < rows; r++) {
    uint32_t *orow = wq + r * words_per_row;
    memset(orow, 0, sizeof(uint32_t) * (size_t)words_per_row);
    for (int g = 0; g < groups; g++) {
      float w_min = type_max(dtype);
      float w_max = 0.0f;
      for (int i = 0; i < group; i++) {
        float v = load_val(w, dtype, r * D + (int64_t)g * group + i);
        vals[i] = v;
        w_min = fminf(w_min, v);
        w_max = fmaxf(w_max, v);
      }
      float scale = fmaxf((w_max - w_min) / n_bins, eps);
      int side = fabsf(w_min) > fabsf(w_max);
      scale = side ? scale : -scale;
      float edge = side ? w_min : w_max;
      float e_over_s = edge / scale;
      ties += is_tie(e_over_s);
      float q0 = roundf(e_over_s);
      int at_zero = q0 == 0.0f;
      scale = at_zero ? scale : edge / q0;
      float bias = at_zero ? 0.0f : edge;
      store_val(scales, dtype, r * groups + g, scale);
      store_val(biases, dtype, r * groups + g, bias);
      for (int i = 0; i < group; i++) {
        float x = (vals[i] - bias) / scale;
        ties += is_tie(x);
        float qv = fminf(roundf(x), n_bins);
        uint32_t code = qv > 0.0f ? (uint32_t)qv : 0u;
        int e = g * group + i;
        orow[e / per_word] |= code << (bits * (e % per_word));
      }
    }
  }
  free(vals);
  return ties;
}

static inline uint32_t code_at(const uint32_t *row, int e, int bits) {
  const int per_word = 32 / bits;
  return (row[e / per_word] >> (bits * (e % per_word))) & ((1u << bits) - 1u);
}

/* quantized.h:2498-2560 (affine_dequantize): out[i] = scale * d + bias with
 * `T scale`, `T bias` (:2538-2539) and the code d an integer (:2548-2559).
 * Evaluated in T, that expression rounds twice (the product to T, then the
 * sum) unless the compiler contracts it into one fused multiply-add, which
 * rounds once.  Which of the two the reference's build does is not fixed by
 * any file in the reference tree (it depends on the Metal compiler's
 * contraction setting), so both are restated: rule 0 = one rounding of the
 * exact s*q + b (the fused form; this build's kernels), rule 1 = T(T(s*q) + b).
 * vkvo_dequantize_rule_split counts the elements where they differ. */
static inline float deq_rule(float s, float q, float b, int dtype, int rule) {
  if (rule == 0 || dtype == 0) return round_to(fmaf(s, q, b), dtype);
  return round_to(round_to(s * q, dtype) + b, dtype);
}

void vkvo_dequantize(const uint32_t *wq, const void *scales, const void *biases,
                     int dtype, int64_t rows, int D, int group, int bits, int rule,
                     void *out) {
  const int words_per_row = D * bits / 32;
  const int groups = D / group;
  for (int64_t r = 0; r < rows; r++) {
    for (int e = 0; e < D; e++) {
      float s = load_val(scales, dtype, r * groups + e / group);
      float b = load_val(biases, dtype, r * groups + e / group);
      float q = (float)code_at(wq + r * words_per_row, e, bits);
      store_val(out, dtype, r * D + e, deq_rule(s, q, b, dtype, rule));
    }
  }
}

int64_t vkvo_dequantize_rule_split(const uint32_t *wq, const void *scales,
                                   const void *biases, int dtype, int64_t rows, int D,
                                   int group, int bits) {
  const int words_per_row = D * bits / 32;
  const int groups = D / group;
  int64_t n = 0;
  for (int64_t r = 0; r < rows; r++)
    for (int e = 0; e < D; e++) {
      float s = load_val(scales, dtype, r * groups + e / group);
      float b = load_val(biases, dtype, r * groups + e / group);
      float q = (float)code_at(wq + r * words_per_row, e, bits);
      n += deq_rule(s, q, b, dtype, 0) != deq_rule(s, q, b, dtype, 1);
    }
  return n;
}

static inline int mask_visible(int mask_mode, const uint8_t *bmask, const float *fmask,
                               int64_t mo, int l, int L, int t, int T, double *add) {
  *add = 0.0;
  if (mask_mode == 1) return t <= T - L + l;
  if (mask_mode == 2) return bmask[mo] != 0;
  if (mask_mode == 3) {
    *add = fmask[mo];
    return fmask[mo] >= -FLT_MAX;
  }
  return 1;
}

/* MLXFast.swift:173-218 semantics as computed by sdpa_vector.h:15-177:
 * q scaled in fp32, softmax over visible keys, zero output for an empty row.
 * An additive mask is read in the query dtype q_dtype (the kernel's `const
 * device T* fmask`, :15-38): each value is rounded to it, and a key whose
 * rounded mask is below the dtype's lowest finite value is skipped
 * (:105-121).  sinks (NULL = none): per query head logit [Hq] that starts
 * the running max with sum 1 (:93-96), i.e. one more softmax term whose
 * value row is zero. */
void vkvo_sdpa(const float *q, const float *k, const float *v, int B, int Hq,
               int Hkv, int L, int T, int D, int Dv, float scale, int mask_mode,
               const uint8_t *bmask, const float *fmask, int64_t msb, int64_t msh,
               int64_t msl, int64_t mst, int q_dtype, const float *sinks, double *out) {
  const int rep = Hq / Hkv;
  double *sc = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
  unsigned char *vis = (unsigned char *)malloc((size_t)(T > 0 ? T : 1));
  for (int b = 0; b < B; b++)
    for (int h = 0; h < Hq; h++)
      for (int l = 0; l < L; l++) {
        const float *qr = q + (((int64_t)b * Hq + h) * L + l) * D;
        const int hk = h / rep;
        double mx = sinks ? (double)sinks[h] : -INFINITY;
        for (int t = 0; t < T; t++) {
          double add;
          int64_t mo = b * msb + h * msh + l * msl + t * mst;
          vis[t] = (unsigned char)mask_visible(mask_mode, bmask, fmask, mo, l, L, t, T, &add);
          if (mask_mode == 3) {
            add = (double)round_to((float)add, q_dtype);
            vis[t] = add >= -(double)type_max(q_dtype);
          }
          if (!vis[t]) continue;
          const float *kr = k + (((int64_t)b * Hkv + hk) * T + t) * D;
          double s = 0.0;
          for (int d = 0; d < D; d++) s += (double)(scale * qr[d]) * (double)kr[d];
          /* the kernel adds the mask to its fp32 score (U = float) */
          sc[t] = mask_mode == 3 ? (double)((float)s + (float)add) : s;
          if (sc[t] > mx) mx = sc[t];
        }
        double den = sinks ? exp((double)sinks[h] - mx) : 0.0;
        double *o = out + (((int64_t)b * Hq + h) * L + l) * Dv;
        for (int d = 0; d < Dv; d++) o[d] = 0.0;
        for (int t = 0; t < T; t++) {
          if (!vis[t]) continue;
          double p = exp(sc[t] - mx);
          den += p;
          const float *vr = v + (((int64_t)b * Hkv + hk) * T + t) * Dv;
          for (int d = 0; d < Dv; d++) o[d] += p * (double)vr[d];
        }
        if (den > 0.0)
          for (int d = 0; d < Dv; d++) o[d] /= den;
      }
  free(sc);
  free(vis);
}

/* Dequantized element of a reference-layout row: the exact value
 * scale * q + bias (fp64, as qmv's fp32 `scale * sum(x q) + bias * sum(x)`
 * forms it, quantized.h:1493-1648), or that value rounded once to the
 * storage dtype when the multi-row qmm path first dequantizes its tiles into
 * threadgroup memory of type T (quantized.h:568-576, :686-713). */
static inline double deq_at(const uint32_t *row, const float *s, const float *b, int d,
                            int group, int bits, int round_dt) {
  const double x = (double)s[d / group] * (double)code_at(row, d, bits) + (double)b[d / group];
  return round_dt >= 0 ? (double)round_to((float)x, round_dt) : x;
}

/* K or V element (t, d) of one (batch row, kv head): from the
 * pre-dequantized [T][D] values when given, else dequantized in place. */
static inline double kv_val(const double *pre, const uint32_t *codes, const float *s,
                            const float *b, int64_t t, int d, int D, int group, int bits,
                            int deq_dt) {
  if (pre) return pre[t * D + d];
  const int wpr = D * bits / 32, G = D / group;
  return deq_at(codes + t * wpr, s + t * G, b + t * G, d, group, bits, deq_dt);
}

static inline double round_d(double x, int dtype) {
  return (double)round_to((float)x, dtype);
}

/* Softmax weights of one row of scores (KVCache.swift:1982: softmax over the
 * last axis with precise: false, Source/MLX/Ops.swift:2702-2710).
 * rnd == 0: exact fp64.  Otherwise the scores sc[] already carry the
 * reference's rounding and:
 *   acc_t < 0 : internal arithmetic in fp32, weights
 *               T(exp(s - max) * (1 / sum)) rounded to wdt;
 *   acc_t >= 0: internal arithmetic in AccT = T, the kernels' default
 *               template argument (softmax.h:10, :100), which the
 *               non-precise softmax uses for T = f16/bf16; T's simd_sum and
 *               simd_max reduce in fp32 and round once (bf16_math.h:328-378).
 *               Rows of up to 4096 keys follow softmax_single_row
 *               (softmax.h:10-98): 4 consecutive keys per thread summed in
 *               T, 32-thread sums, then the sum of those; longer rows follow
 *               softmax_looped (softmax.h:100-200) with 1024 threads, each
 *               keeping a running (max, sum) over keys lid*4 + 4096 r + i,
 *               rescaled by exp(old max - new max) at every level.  The
 *               order of the fp32 additions inside one simd_sum is the
 *               hardware's and is not in the tree (fp64 here).
 * pe[] receives the exact fp64 softmax of the same scores (the unrounded
 * weights a kernel that does not round them would use). */
#define SOFTMAX_N_READS 4
#define SOFTMAX_LOOPED_LIMIT 4096
#define SOFTMAX_LOOPED_THREADS 1024

static double t_exp(double x, int dt) { return round_d(exp(x), dt); }

static void softmax_row(const double *sc, int T, int rnd, int acc_t, int wdt, double *p,
                        double *pe) {
  double mx = -INFINITY;
  for (int t = 0; t < T; t++) mx = sc[t] > mx ? sc[t] : mx;
  double den = 0.0;
  for (int t = 0; t < T; t++) {
    pe[t] = exp(sc[t] - mx);
    den += pe[t];
  }
  for (int t = 0; t < T; t++) pe[t] /= den;
  if (!rnd) {
    for (int t = 0; t < T; t++) p[t] = pe[t];
    return;
  }
  if (acc_t < 0) {
    double sum = 0.0;
    for (int t = 0; t < T; t++) {
      p[t] = (double)(float)exp((double)(float)(sc[t] - mx));
      sum += p[t];
    }
    const float r = (float)(1.0 / (double)(float)sum);
    for (int t = 0; t < T; t++) p[t] = round_d((double)((float)p[t] * r), wdt);
    return;
  }
  const int dt = acc_t;
  if (T <= SOFTMAX_LOOPED_LIMIT) {
    /* softmax_single_row */
    double total = 0.0, simd = 0.0, thr = 0.0;
    for (int t = 0; t < T; t++) {
      p[t] = t_exp(round_d(sc[t] - mx, dt), dt);
      thr = round_d(thr + p[t], dt);
      if ((t & 3) == 3 || t == T - 1) {
        simd += thr;
        thr = 0.0;
      }
      if ((t & 127) == 127 || t == T - 1) {
        total += round_d(simd, dt);
        simd = 0.0;
      }
    }
    const double r = round_d(1.0 / round_d(total, dt), dt);
    for (int t = 0; t < T; t++) p[t] = round_d(p[t] * r, dt);
    return;
  }
  /* softmax_looped: per-thread running max and sum */
  const double fmin = -type_max(dt);
  const int NT = SOFTMAX_LOOPED_THREADS, stride = SOFTMAX_N_READS * NT;
  const int rounds = (T + stride - 1) / stride;
  double lmax[SOFTMAX_LOOPED_THREADS], lsum[SOFTMAX_LOOPED_THREADS];
  for (int lid = 0; lid < NT; lid++) {
    double m = fmin, n = 0.0;
    for (int r = 0; r < rounds; r++) {
      double v[SOFTMAX_N_READS];
      const int off = r * stride + lid * SOFTMAX_N_READS;
      const double prev = m;
      for (int i = 0; i < SOFTMAX_N_READS; i++) {
        v[i] = off + i < T ? sc[off + i] : -INFINITY;
        m = v[i] > m ? v[i] : m;
      }
      n = round_d(n * t_exp(round_d(prev - m, dt), dt), dt);
      for (int i = 0; i < SOFTMAX_N_READS; i++)
        n = round_d(n + t_exp(round_d(v[i] - m, dt), dt), dt);
    }
    lmax[lid] = m;
    lsum[lid] = n;
  }
  double gmax = fmin, smax[SOFTMAX_LOOPED_THREADS / 32], ssum[SOFTMAX_LOOPED_THREADS / 32];
  for (int g = 0; g < NT / 32; g++) {
    double m = fmin, acc = 0.0;
    for (int l = 0; l < 32; l++) m = lmax[g * 32 + l] > m ? lmax[g * 32 + l] : m;
    for (int l = 0; l < 32; l++)
      acc += round_d(lsum[g * 32 + l] * t_exp(round_d(lmax[g * 32 + l] - m, dt), dt), dt);
    smax[g] = m;
    ssum[g] = round_d(acc, dt);
    gmax = m > gmax ? m : gmax;
  }
  double total = 0.0;
  for (int g = 0; g < NT / 32; g++)
    total += round_d(ssum[g] * t_exp(round_d(smax[g] - gmax, dt), dt), dt);
  const double r = round_d(1.0 / round_d(total, dt), dt);
  for (int t = 0; t < T; t++) p[t] = round_d(t_exp(round_d(sc[t] - gmax, dt), dt) * r, dt);
}

/* Neighbours of the T value r (T = f16 or bf16): the adjacent representable
 * values below and above. */
static void t_neighbours(double r, int dtype, double *below, double *above) {
  const float rf = (float)r;
  if (dtype == 2) {
    uint16_t h = vkvo_f32_to_bf16(rf);
    const int neg = (h & 0x8000u) != 0;
    uint16_t up = (uint16_t)(neg ? h - 1 : h + 1), dn = (uint16_t)(neg ? h + 1 : h - 1);
    if ((h & 0x7fffu) == 0) { up = 0x0001u; dn = 0x8001u; }
    *above = vkvo_bf16_to_f32(up);
    *below = vkvo_bf16_to_f32(dn);
  } else {
    uint16_t h = vkvo_f32_to_f16(rf);
    const int neg = (h & 0x8000u) != 0;
    uint16_t up = (uint16_t)(neg ? h - 1 : h + 1), dn = (uint16_t)(neg ? h + 1 : h - 1);
    if ((h & 0x7fffu) == 0) { up = 0x0001u; dn = 0x8001u; }
    *above = vkvo_f16_to_f32(up);
    *below = vkvo_f16_to_f32(dn);
  }
}

/* One query row against one KV head of a quantized cache (reference layout
 * rows of length D).  Shared by the batch and the CPU-baseline entry.
 * rnd: 0 exact, 1 qmv rounding, 2 qmm rounding, 3 qmv rounding with an
 * AccT = T softmax (see vkvo_quantized_sdpa).  sdt: dtype the scores are
 * rounded to (the query dtype); fmask_f32: an f32 additive mask was added
 * (MLX promotes T + f32 to f32, so the scores and weights stay f32).
 * wb (optional), per output dim: the most the reference's two roundings can
 * move the output against the exact softmax of the rounded scores:
 *   sum_t |w_t - pe_t| |v_t|  (the weights stored in T), plus
 *   for every score within eps_t = 2^-17 sum_d |q_d k_td| of a T rounding
 *   boundary, the exact change of the output if that score rounded to the
 *   other side: an fp32 accumulation (the reference's qmv, or any kernel)
 *   lands on either side of such a boundary depending on its order of
 *   summation.  2^-17 is twice the largest relative score error measured
 *   for this build's decode kernel on x20-outlier data. */
static void qsdpa_row(const float *qs, const uint32_t *kq, const float *ks,
                      const float *kb, const uint32_t *vq, const float *vs,
                      const float *vb, int T, int D, int group, int bits,
                      const double *add, const unsigned char *vis, double fill,
                      int rnd, int sdt, double *sc, double *pw, double *pe, double *o,
                      double *wb, double *fb, const double *kd, const double *vd) {
    const int deq_dt = (rnd == 2 || rnd == 4) ? sdt : -1;
  const int wdt = add ? 0 : sdt;
  /* flip factors exp(n_t - r_t) for scores near a rounding boundary (0: none),
   * and the flipped score itself (the other neighbour, mask added) */
  double *flip = ((wb || fb) && rnd) ? (double *)calloc((size_t)(T > 0 ? T : 1), sizeof(double)) : NULL;
  double *alt = (fb && rnd) ? (double *)calloc((size_t)(T > 0 ? T : 1), sizeof(double)) : NULL;
  const int acc_t = ((rnd == 3 || rnd == 4) && !add) ? sdt : -1;
  for (int t = 0; t < T; t++) {
    double s = fill;
    if (!vis || vis[t]) {
      s = 0.0;
      double mag = 0.0;
      for (int d = 0; d < D; d++) {
        const double kv = kv_val(kd, kq, ks, kb, t, d, D, group, bits, deq_dt);
        s += (double)qs[d] * kv;
        mag += fabs((double)qs[d] * kv);
      }
      if (rnd) {
        const double r = round_d(s, sdt);
        if (flip) {
          double below, above;
          t_neighbours(r, sdt, &below, &above);
          const double eps = ldexp(mag, -17);
          if (fabs(s - 0.5 * (r + above)) < eps) {
            flip[t] = exp(above - r);
            if (alt) alt[t] = add ? (double)(float)(above + add[t]) : above;
          }
          if (fabs(s - 0.5 * (r + below)) < eps) {
            flip[t] = exp(below - r);
            if (alt) alt[t] = add ? (double)(float)(below + add[t]) : below;
          }
        }
        s = r;
      }
      if (add) s = rnd ? (double)(float)(s + add[t]) : s + add[t];
    }
    sc[t] = s;
  }
  softmax_row(sc, T, rnd, acc_t, wdt, pw, pe);
  double *o1 = (wb || fb) ? (double *)calloc((size_t)D, sizeof(double)) : NULL;
  for (int d = 0; d < D; d++) o[d] = 0.0;
  if (wb)
    for (int d = 0; d < D; d++) wb[d] = 0.0;
  if (fb)
    for (int d = 0; d < D; d++) fb[d] = 0.0;
  for (int t = 0; t < T; t++) {
    for (int d = 0; d < D; d++) {
      const double vv = kv_val(vd, vq, vs, vb, t, d, D, group, bits, deq_dt);
      o[d] += pw[t] * vv;
      if (wb) wb[d] += fabs(pw[t] - pe[t]) * fabs(vv);
      if (o1) o1[d] += pe[t] * vv;
    }
  }
  if (flip && wb) {
    /* a flipped score t scales its exponential by f: the output becomes
     * (o1 + (f - 1) pe_t v_t) / (1 + (f - 1) pe_t) */
    for (int t = 0; t < T; t++) {
      if (flip[t] == 0.0) continue;
      const double a = (flip[t] - 1.0) * pe[t];
      for (int d = 0; d < D; d++) {
        const double vv = kv_val(vd, vq, vs, vb, t, d, D, group, bits, deq_dt);
        wb[d] += fabs((o1[d] + a * vv) / (1.0 + a) - o1[d]);
      }
    }
  }
  if (flip && fb) {
    /* fb: the move of the output, in this mode's own arithmetic (the same
     * rounded softmax, weights and P.V), when one flipped score t is
     * stored the other way: a flip can move the rounded normaliser and so
     * every weight, which the exact-softmax formula above does not see.
     * Flips of one row are added. */
    double *sc2 = (double *)malloc(sizeof(double) * (size_t)T);
    double *pw2 = (double *)malloc(sizeof(double) * (size_t)T);
    double *pe2 = (double *)malloc(sizeof(double) * (size_t)T);
    double *o2 = (double *)malloc(sizeof(double) * (size_t)D);
    for (int t = 0; t < T; t++) {
      if (flip[t] == 0.0) continue;
      memcpy(sc2, sc, sizeof(double) * (size_t)T);
      sc2[t] = alt[t];
      softmax_row(sc2, T, rnd, acc_t, wdt, pw2, pe2);
      for (int d = 0; d < D; d++) o2[d] = 0.0;
      for (int u = 0; u < T; u++) {
        if (pw2[u] == pw[u]) continue;
        for (int d = 0; d < D; d++)
          o2[d] += (pw2[u] - pw[u]) * kv_val(vd, vq, vs, vb, u, d, D, group, bits, deq_dt);
      }
      for (int d = 0; d < D; d++) fb[d] += fabs(o2[d]);
    }
    free(sc2);
    free(pw2);
    free(pe2);
    free(o2);
  }
  free(flip);
  free(alt);
  free(o1);
}

/* KVCache.swift:1909-1997 (quantizedScaledDotProductAttention).  Each
 * (batch row, kv head)'s K and V are dequantized once (as the rounding mode
 * rounds them); its query rows run in parallel (OpenMP), each on its own
 * scratch, so the result does not depend on the thread count. */
void vkvo_quantized_sdpa(const float *q, int q_dtype, const uint32_t *kq,
                         const float *ks, const float *kb, const uint32_t *vq,
                         const float *vs, const float *vb, int B, int Hq, int Hkv,
                         int L, int T, int D, int group, int bits, float scale,
                         int mask_mode, const uint8_t *bmask, const float *fmask,
                         int64_t msb, int64_t msh, int64_t msl, int64_t mst,
                         int rounding, double *out, double *wbound, double *fbound) {
  const int rep = Hq / Hkv;
  const int wpr = D * bits / 32;
  const int G = D / group;
  const float scale_t = round_to(scale, q_dtype);
  const double fill = type_lowest(q_dtype);
  const size_t nT = (size_t)(T > 0 ? T : 1);
  const int deq_dt = (rounding == 2 || rounding == 4) ? q_dtype : -1;
  double *kd = (double *)malloc(sizeof(double) * nT * (size_t)D);
  double *vd = (double *)malloc(sizeof(double) * nT * (size_t)D);
  for (int b = 0; b < B; b++)
    for (int hk = 0; hk < Hkv; hk++) {
      const int64_t kv_row0 = ((int64_t)b * Hkv + hk) * T;
      for (int t = 0; t < T; t++)
        for (int d = 0; d < D; d++) {
          const int64_t r = kv_row0 + t;
          kd[(int64_t)t * D + d] = deq_at(kq + r * wpr, ks + r * G, kb + r * G, d, group, bits, deq_dt);
          vd[(int64_t)t * D + d] = deq_at(vq + r * wpr, vs + r * G, vb + r * G, d, group, bits, deq_dt);
        }
#ifdef _OPENMP
#pragma omp parallel
#endif
      {
        float *qs = (float *)malloc(sizeof(float) * (size_t)D);
        double *sc = (double *)malloc(sizeof(double) * nT);
        double *pw = (double *)malloc(sizeof(double) * nT);
        double *pe = (double *)malloc(sizeof(double) * nT);
        double *add = (double *)malloc(sizeof(double) * nT);
        unsigned char *vis = (unsigned char *)malloc(nT);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int rl = 0; rl < rep * L; rl++) {
          const int h = hk * rep + rl / L, l = rl % L;
          const float *qr = q + (((int64_t)b * Hq + h) * L + l) * D;
          for (int d = 0; d < D; d++) qs[d] = round_to(qr[d] * scale_t, q_dtype);
          const int64_t orow = (((int64_t)b * Hq + h) * L + l) * D;
          for (int t = 0; t < T; t++) {
            double a;
            int64_t mo = b * msb + h * msh + l * msl + t * mst;
            if (mask_mode == 1) {
              /* causal: query row l sits at key position l + (T - L) */
              vis[t] = (unsigned char)(l + (T - L) >= t);
              add[t] = 0.0;
            } else {
              vis[t] = (unsigned char)mask_visible(mask_mode == 3 ? 0 : mask_mode, bmask, fmask,
                                                   mo, l, L, t, T, &a);
              add[t] = mask_mode == 3 ? (double)fmask[mo] : 0.0;
            }
          }
          if (T == 0) {
            for (int d = 0; d < D; d++) out[orow + d] = 0.0;
            if (wbound)
              for (int d = 0; d < D; d++) wbound[orow + d] = 0.0;
            if (fbound)
              for (int d = 0; d < D; d++) fbound[orow + d] = 0.0;
            continue;
          }
          qsdpa_row(qs, kq + kv_row0 * wpr, ks + kv_row0 * G, kb + kv_row0 * G,
                    vq + kv_row0 * wpr, vs + kv_row0 * G, vb + kv_row0 * G, T, D, group,
                    bits, mask_mode == 3 ? add : NULL, vis, fill, rounding, q_dtype, sc, pw, pe,
                    out + orow, wbound ? wbound + orow : NULL, fbound ? fbound + orow : NULL, kd,
                    vd);
        }
        free(qs);
        free(sc);
        free(pw);
        free(pe);
        free(add);
        free(vis);
      }
    }
  free(kd);
  free(vd);
}

void vkvo_quantized_decode_batch(const float *q, int q_dtype, const uint32_t *kq,
                                 const float *ks, const float *kb, const uint32_t *vq,
                                 const float *vs, const float *vb, int nseq,
                                 const int32_t *lens, const int64_t *tok_off, int Hq,
                                 int Hkv, int D, int group, int bits, float scale,
                                 int rounding, int threads, double *out) {
  const int rep = Hq / Hkv;
  const int wpr = D * bits / 32;
  const int G = D / group;
  const float scale_t = round_to(scale, q_dtype);
  int maxT = 1;
  for (int s = 0; s < nseq; s++) maxT = lens[s] > maxT ? lens[s] : maxT;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
  {
    float *qs = (float *)malloc(sizeof(float) * (size_t)D);
    double *sc = (double *)malloc(sizeof(double) * (size_t)maxT);
    double *pw = (double *)malloc(sizeof(double) * (size_t)maxT);
    double *pe = (double *)malloc(sizeof(double) * (size_t)maxT);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1) collapse(2)
#endif
    for (int s = 0; s < nseq; s++)
      for (int h = 0; h < Hq; h++) {
        const float *qr = q + ((int64_t)s * Hq + h) * D;
        for (int d = 0; d < D; d++) qs[d] = round_to(qr[d] * scale_t, q_dtype);
        const int64_t T = lens[s];
        /* sequence s is stored [Hkv, T, ...] starting at token row tok_off[s] */
        const int64_t row0 = tok_off[s] + (int64_t)(h / rep) * T;
        qsdpa_row(qs, kq + row0 * wpr, ks + row0 * G, kb + row0 * G, vq + row0 * wpr,
                  vs + row0 * G, vb + row0 * G, (int)T, D, group, bits, NULL, NULL, 0.0,
                  rounding, q_dtype, sc, pw, pe, out + ((int64_t)s * Hq + h) * D, NULL, NULL, NULL,
                  NULL);
      }
    free(qs);
    free(sc);
    free(pw);
    free(pe);
  }
}

/* GLM4MOELite.swift:233-290 absorbed MLA decode through
 * AttentionUtils.swift:43-75 (L == 1 promoted to fp32 SDPA with one KV head):
 * keys are the cache entries (dequantized to the storage dtype, here given as
 * f32 values), values are their first Dv dims. */
void vkvo_mla_decode(const float *q, const uint32_t *cq, const float *cs,
                     const float *cb, int B, int H, int T, const int32_t *lens,
                     int Dk, int Dv, int group, int bits, float scale, double *out) {
  const int wpr = Dk * bits / 32;
  const int G = Dk / group;
  double *kv = (double *)malloc(sizeof(double) * (size_t)Dk * (size_t)(T > 0 ? T : 1));
  double *sc = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
  for (int b = 0; b < B; b++) {
    const int n = lens[b];
    for (int t = 0; t < n; t++) {
      const int64_t row = (int64_t)b * T + t;
      for (int d = 0; d < Dk; d++) {
        /* dequantize to the storage dtype (bf16 for this cache) */
        float s = cs[row * G + d / group], bb = cb[row * G + d / group];
        float deq = fmaf(s, (float)code_at(cq + row * wpr, d, bits), bb);
        kv[(int64_t)t * Dk + d] = (double)vkvo_bf16_to_f32(vkvo_f32_to_bf16(deq));
      }
    }
    for (int h = 0; h < H; h++) {
      const float *qr = q + ((int64_t)b * H + h) * Dk;
      double mx = -INFINITY;
      for (int t = 0; t < n; t++) {
        double s = 0.0;
        for (int d = 0; d < Dk; d++) s += (double)(scale * qr[d]) * kv[(int64_t)t * Dk + d];
        sc[t] = s;
        if (s > mx) mx = s;
      }
      double *o = out + ((int64_t)b * H + h) * Dv;
      for (int d = 0; d < Dv; d++) o[d] = 0.0;
      double den = 0.0;
      for (int t = 0; t < n; t++) {
        double p = exp(sc[t] - mx);
        den += p;
        for (int d = 0; d < Dv; d++) o[d] += p * kv[(int64_t)t * Dk + d];
      }
      if (den > 0.0)
        for (int d = 0; d < Dv; d++) o[d] /= den;
    }
  }
  free(kv);
  free(sc);
}
