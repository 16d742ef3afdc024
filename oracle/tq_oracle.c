/*
 * tq_oracle.c -- CPU restatement of the reference's TurboQuant KV codec
 * (Libraries/MLXLMCommon/TurboQuant/, arXiv:2504.19874).
 *
 * TEST INFRASTRUCTURE ONLY (see vkv_oracle.h): tests/, the smoke check and
 * the CPU-baseline leg of bench.py load it as the checker; the product never
 * links it.  Built with -ffp-contract=off, so every float expression below
 * rounds exactly as written; the fused multiply-adds are explicit fmaf calls.
 *
 * Where the reference leaves an order of operations to MLX (the two f32
 * matrix products and the three row sums), this file fixes one and says
 * which: sums of squares are accumulated in double in index order and
 * rounded once; matrix products are f32 fused multiply-add chains in index
 * order starting from zero.  MLX's own orders are unpinned (no MLX build
 * exists here); the checks in tests/test_oracle_turboquant.py bound how far
 * any f32 order can move each result.
 *
 * Parity pins (tests/test_oracle_turboquant.py):
 *   tqo_codebook     -- Lloyd-Max conditions re-derived with scipy
 *                       quadrature on the same Beta density; the Gaussian
 *                       Lloyd-Max levels (Max 1960) in the large-dim limit;
 *                       symmetry and sortedness.
 *   tqo_random_signs -- glibc's srand48/drand48 against the POSIX LCG
 *                       written out in Python.
 *   tqo_erfinv       -- scipy.special.erfinv within 3 f32 ulps, and the
 *                       reference's seeded normal known answers.
 *   tqo_hadamard     -- scipy.linalg.hadamard / sqrt(n) on power-of-two
 *                       blocks; H H = I; the block split of non-powers.
 *   tqo_encode/decode -- reconstruction error of the Lloyd-Max quantizer
 *                       against its expected distortion, the unbiasedness of
 *                       the QJL inner-product estimate, exact round trips of
 *                       codebook points, and sink / tail / promotion rules.
 */
#define _DEFAULT_SOURCE /* M_PI, srand48 / drand48 under -std=c11 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vkv_oracle.h"

static inline float rnd(float v, int dtype) {
  switch (dtype) {
    case 1: return vkvo_f16_to_f32(vkvo_f32_to_f16(v));
    case 2: return vkvo_bf16_to_f32(vkvo_f32_to_bf16(v));
    default: return v;
  }
}

/* TQCodebook.betaPDF (TQCodebook.swift:71-78): the density of one
 * coordinate of a uniform point on the unit sphere in R^d, in double,
 * returned as float. */
static float beta_pdf(float x, int d) {
  const double df = (double)d;
  const double log_const = lgamma(df / 2.0) - 0.5 * log(M_PI) - lgamma((df - 1.0) / 2.0);
  const double xd = (double)x;
  double safe = 1.0 - xd * xd;
  if (safe < 1e-30) safe = 1e-30;
  return (float)exp(log_const + (df - 3.0) / 2.0 * log(safe));
}

/* TQCodebook.trapezoid (TQCodebook.swift:83-90), float accumulation. */
static float trapezoid(const float *y, const float *x, int n) {
  if (n < 2) return 0.0f;
  float r = 0.0f;
  for (int i = 0; i < n - 1; i++) r += (x[i + 1] - x[i]) * (y[i] + y[i + 1]) / 2.0f;
  return r;
}

static int cmp_float(const void *a, const void *b) {
  const float x = *(const float *)a, y = *(const float *)b;
  return (x > y) - (x < y);
}

/* TQCodebook.computeCodebook (TQCodebook.swift:103-160): Lloyd-Max on a
 * 10000-point grid of [-1, 1] under beta_pdf, centroids started evenly on
 * [-3/sqrt(d), 3/sqrt(d)], `iterations` rounds of (midpoint boundaries,
 * conditional means by the trapezoid rule over grid points in [lo, hi)),
 * then sorted.  out has 2^bits entries. */
void tqo_codebook(int dim, int bits, int iterations, float *out) {
  enum { NG = 10000 };
  const int nc = 1 << bits;
  float *grid = malloc(sizeof(float) * NG), *pdf = malloc(sizeof(float) * NG);
  float *mx = malloc(sizeof(float) * NG), *mp = malloc(sizeof(float) * NG);
  float *xm = malloc(sizeof(float) * NG);
  float *bnd = malloc(sizeof(float) * (nc + 1));
  for (int i = 0; i < NG; i++) grid[i] = -1.0f + 2.0f * (float)i / (float)(NG - 1);
  for (int i = 0; i < NG; i++) pdf[i] = beta_pdf(grid[i], dim);
  const float mass0 = trapezoid(pdf, grid, NG);
  if (mass0 > 0)
    for (int i = 0; i < NG; i++) pdf[i] /= mass0;
  const float support = 3.0f / sqrtf(fmaxf((float)dim, 1.0f));
  for (int i = 0; i < nc; i++)
    out[i] = -support + 2.0f * support * (float)i / (float)(nc - 1 > 1 ? nc - 1 : 1);
  for (int it = 0; it < iterations; it++) {
    bnd[0] = -1.0f;
    bnd[nc] = 1.0f;
    for (int i = 0; i < nc - 1; i++) bnd[i + 1] = (out[i] + out[i + 1]) / 2.0f;
    for (int i = 0; i < nc; i++) {
      const float lo = bnd[i], hi = bnd[i + 1];
      int m = 0;
      for (int j = 0; j < NG; j++)
        if (grid[j] >= lo && grid[j] < hi) {
          mx[m] = grid[j];
          mp[m] = pdf[j];
          m++;
        }
      if (m < 2) continue;
      const float mass = trapezoid(mp, mx, m);
      for (int j = 0; j < m; j++) xm[j] = mx[j] * mp[j];
      const float moment = trapezoid(xm, mx, m);
      out[i] = moment / fmaxf(mass, 1e-10f);
    }
  }
  qsort(out, nc, sizeof(float), cmp_float);
  free(grid);
  free(pdf);
  free(mx);
  free(mp);
  free(xm);
  free(bnd);
}

/* TQHadamard.generateRandomSigns (TQHadamard.swift:52-62): srand48(seed),
 * then drand48() < 0.5 -> -1, else +1, for each dimension in order. */
void tqo_random_signs(int dim, long seed, float *out) {
  srand48(seed);
  for (int i = 0; i < dim; i++) out[i] = drand48() < 0.5 ? -1.0f : 1.0f;
}

/* MLX's erfinv (mlx-generated/metal/erf.h:43-76): a single-precision
 * approximation on t = log(1 - a^2), two polynomial branches evaluated with
 * fused multiply-adds, result a * p. */
float tqo_erfinv(float a) {
  static const float hi[9] = {3.03697567e-10f, 2.93243101e-8f, 1.22150334e-6f,
                              2.84108955e-5f,  3.93552968e-4f, 3.02698812e-3f,
                              4.83185798e-3f,  -2.64646143e-1f, 8.40016484e-1f};
  static const float lo[10] = {5.43877832e-9f,  1.43285448e-7f,  1.22774793e-6f,
                               1.12963626e-7f,  -5.61530760e-5f, -1.47697632e-4f,
                               2.31468678e-3f,  1.15392581e-2f,  -2.32015476e-1f,
                               8.86226892e-1f};
  const float t = logf(fmaf(a, 0.0f - a, 1.0f));
  float p;
  if (fabsf(t) > 6.125f) {
    p = hi[0];
    for (int i = 1; i < 9; i++) p = fmaf(p, t, hi[i]);
  } else {
    p = lo[0];
    for (int i = 1; i < 10; i++) p = fmaf(p, t, lo[i]);
  }
  return a * p;
}

/* MLXRandom.normal's map of its uniform draws (random.cpp normal:
 * sqrt(2) * erfinv(u), the constant held as an f32 array). */
void tqo_normal_from_uniform(const float *u, int64_t n, float *out) {
  const float s2 = (float)sqrt(2.0);
  for (int64_t i = 0; i < n; i++) out[i] = s2 * tqo_erfinv(u[i]);
}

/* TQHadamard.hadamardTransform (TQHadamard.swift:85-107) on one block of
 * n = 2^k floats: butterflies (a + b, a - b) for h = 1, 2, 4, ... over
 * pairs (g 2h + j, g 2h + h + j), then each element times the f32
 * 1 / sqrt(n). */
static void hadamard_block(float *x, int n) {
  for (int h = 1; h < n; h *= 2)
    for (int g = 0; g < n; g += 2 * h)
      for (int j = 0; j < h; j++) {
        const float a = x[g + j], b = x[g + h + j];
        x[g + j] = a + b;
        x[g + h + j] = a - b;
      }
  const float scale = 1.0f / sqrtf((float)n);
  for (int i = 0; i < n; i++) x[i] = x[i] * scale;
}

/* TQHadamard.decomposePow2Blocks (TQHadamard.swift:23-33): the largest
 * power of two first, then the rest.  Returns the number of blocks. */
int tqo_pow2_blocks(int dim, int *blocks) {
  int n = 0;
  while (dim > 0) {
    int p = 1;
    while (p * 2 <= dim) p *= 2;
    blocks[n++] = p;
    dim -= p;
  }
  return n;
}

/* hadamardRotate (:117-133) with inverse = 0: blockwise transform of
 * x * signs; hadamardInverse (:136-153) with inverse = 1: blockwise
 * transform, then times signs.  Rows of length dim, in place. */
void tqo_hadamard(float *x, int64_t rows, int dim, const float *signs, int inverse) {
  int blocks[32];
  const int nb = tqo_pow2_blocks(dim, blocks);
  for (int64_t r = 0; r < rows; r++) {
    float *v = x + r * dim;
    if (!inverse)
      for (int i = 0; i < dim; i++) v[i] = v[i] * signs[i];
    int off = 0;
    for (int b = 0; b < nb; b++) {
      hadamard_block(v + off, blocks[b]);
      off += blocks[b];
    }
    if (inverse)
      for (int i = 0; i < dim; i++) v[i] = v[i] * signs[i];
  }
}

/* TQCodebook.quantizeScalar (TQCodebook.swift:172-182): the number of
 * boundaries (midpoints of neighbouring levels, f32) the value exceeds. */
static inline int quantize_scalar(float y, const float *cb, int nc) {
  int idx = 0;
  for (int i = 0; i < nc - 1; i++) idx += y > (cb[i] + cb[i + 1]) / 2.0f;
  return idx;
}

/* TQEncoder.encodeKeys / encodeValues (TQEncoder.swift:135-206, :262-312)
 * for `rows` vectors of `dim` values of dtype `dtype` (given as f32 values):
 *   norm  = T(sqrt(T(sum T(x_i^2)))), unit_i = T(x_i / T(norm + T(1e-8)))
 *           (the scalar takes the array's dtype before the add)
 *   y     = hadamardRotate(unit, signs)            (f32)
 *   idx_i = quantizeScalar(y_i, codebook)
 * keys (S != NULL) also:
 *   r_i = y_i - cb[idx_i]; p_j = sum_i r_i S[j][i]; sign_j = p_j >= 0
 *   rnorm = sqrt(f32(sum f32(r_i^2)))
 * Outputs: idx (u8, rows x dim), sgn (u8 0/1, rows x dim, keys only),
 * vnorm (the T-typed norm as f32), rnorm (f32, keys only), proj (p, keys
 * only, may be NULL), rot (y, may be NULL). */
void tqo_encode(const float *x, int dtype, int64_t rows, int dim, const float *signs,
                const float *cb, int bits, const float *S, uint8_t *idx, uint8_t *sgn,
                float *vnorm, float *rnorm, float *proj, float *rot) {
  const int nc = 1 << bits;
  float *y = malloc(sizeof(float) * dim), *r = malloc(sizeof(float) * dim);
  for (int64_t n = 0; n < rows; n++) {
    const float *v = x + n * dim;
    double s2 = 0.0;
    for (int i = 0; i < dim; i++) s2 += (double)rnd(v[i] * v[i], dtype);
    const float nrm = rnd(sqrtf(rnd((float)s2, dtype)), dtype);
    const float den = rnd(nrm + rnd(1e-8f, dtype), dtype);
    vnorm[n] = nrm;
    for (int i = 0; i < dim; i++) y[i] = rnd(v[i] / den, dtype);
    tqo_hadamard(y, 1, dim, signs, 0);
    if (rot) memcpy(rot + n * dim, y, sizeof(float) * dim);
    for (int i = 0; i < dim; i++) idx[n * dim + i] = (uint8_t)quantize_scalar(y[i], cb, nc);
    if (!S) continue;
    double rs = 0.0;
    for (int i = 0; i < dim; i++) {
      r[i] = y[i] - cb[idx[n * dim + i]];
      rs += (double)(r[i] * r[i]);
    }
    rnorm[n] = sqrtf((float)rs);
    for (int j = 0; j < dim; j++) {
      float p = 0.0f;
      for (int i = 0; i < dim; i++) p = fmaf(r[i], S[(int64_t)j * dim + i], p);
      sgn[n * dim + j] = p >= 0.0f;
      if (proj) proj[n * dim + j] = p;
    }
  }
  free(y);
  free(r);
}

/* TQEncoder.decodeKeys / decodeValues (TQEncoder.swift:214-255, :315-345):
 *   z_j = cb[idx_j] (+ (f32(sqrt(pi/2)) / dim * rnorm) * sum_i s_i S[i][j]
 *         for keys, s_i = +-1)
 *   w   = hadamardInverse(z, signs) * vnorm;  out = f16(w)
 * vnorm / rnorm are the stored f16 norms as f32.  out holds f16 values as
 * f32. */
void tqo_decode(const uint8_t *idx, const uint8_t *sgn, const float *vnorm, const float *rnorm,
                int64_t rows, int dim, const float *signs, const float *cb, const float *S,
                float *out) {
  const float qs = (float)sqrt(M_PI / 2.0) / (float)dim;
  float *z = malloc(sizeof(float) * dim);
  for (int64_t n = 0; n < rows; n++) {
    for (int j = 0; j < dim; j++) z[j] = cb[idx[n * dim + j]];
    if (S) {
      const float a = qs * rnorm[n];
      for (int j = 0; j < dim; j++) {
        float q = 0.0f;
        for (int i = 0; i < dim; i++)
          q = fmaf(sgn[n * dim + i] ? 1.0f : -1.0f, S[(int64_t)i * dim + j], q);
        z[j] = z[j] + a * q;
      }
    }
    tqo_hadamard(z, 1, dim, signs, 1);
    for (int j = 0; j < dim; j++) out[n * dim + j] = rnd(z[j] * vnorm[n], 1);
  }
  free(z);
}
