/*
 * CPU oracle for the Familywise (FW) loss -- TEST INFRASTRUCTURE ONLY (see fwl_oracle.h).
 *
 * Pinned by tests/test_oracle_*.py against: exact rational brute force over all subsets and the
 * root of sum_j max(z_j - t, 0) = 1 (small rows), closed forms (C = 1, constant rows, a top gap
 * >= 1, two-level rows), invariants (shift equivariance, permutation invariance, grad rows summing
 * to 0), the golden vectors in tests/golden/ written by the compiled reference CPU path, and that
 * compiled reference itself when oracle/_ref is built.
 */
#include "fwl_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

float fwo_round_down(double t) {
  /* fw_cpu.cpp:96-101: x > t  <=>  x > round_down(t) for every float x */
  float r = (float)t;
  if ((double)r > t) r = nextafterf(r, -INFINITY);
  return r;
}

static int cmp_desc(const void* a, const void* b) {
  const double x = *(const double*)a, w = *(const double*)b;
  return (x < w) - (x > w);
}

/* ------------------------------------------------------------------ definition (reference_impl.py:11-35) */
static void def_row(const float* z, int64_t C, int64_t yr, double scale, double* v, float* Hout,
                    double* tau_out, double* loss64_out, float* loss_out, int32_t* kappa_out,
                    float* g, int32_t* flag_out) {
  for (int64_t j = 0; j < C; ++j) v[j] = (double)z[j];
  qsort(v, (size_t)C, sizeof(double), cmp_desc);       /* torch.sort(descending)  :17 */
  double S = 0.0, best = -INFINITY;
  int64_t kbest = 0, kcond = 0;
  for (int64_t k = 1; k <= C; ++k) {
    S += v[k - 1];                                     /* cumsum                   :18 */
    const double f = (S - 1.0) / (double)k;            /* (S_k - 1)/k              :19 */
    if (f > best || k == 1) { best = f; kbest = k; }   /* max, first argmax        :21-24 */
    if (v[k - 1] > f) kcond = k;                       /* z_(k) > f(k): k in the support */
  }
  /* tau < max(z) always; fp64 can only break this when the 1 of S - 1 is lost (|z| >= 2^53) */
  const double tau = (best >= v[0] && isfinite(v[0])) ? nextafter(v[0], -INFINITY) : best;
  int64_t kap = 0;
  for (int64_t j = 0; j < C; ++j) kap += (double)z[j] > tau;
  int32_t flag = 0;
  if (kap != kbest) flag |= 1;
  if (kap != kcond) flag |= 2;
  const double zy = (double)z[yr];
  const double l64 = (1.0 - zy) + tau;                 /* losses = 1 - z_at_y + H  :26 */
  *Hout = fwo_round_down(tau);
  if (tau_out) *tau_out = tau;
  if (loss64_out) *loss64_out = l64;
  if (loss_out) *loss_out = (float)l64;
  *kappa_out = (int32_t)kap;
  if (flag_out) *flag_out = flag;
  if (g) {
    const float inv = (float)(scale / (double)kap);    /* fw_cpu.cpp:602 */
    for (int64_t j = 0; j < C; ++j) g[j] = (double)z[j] > tau ? inv : 0.0f;
    g[yr] -= (float)scale;                             /* fw_cpu.cpp:613 */
  }
}

int fwo_definition(const float* z, const int64_t* y, int64_t N, int64_t C, double scale,
                   float* H, double* tau64, double* loss64, float* loss, int32_t* kappa,
                   float* grad, int32_t* flags, int nthreads) {
  if (N < 0 || C < 1) return -1;
  int bad = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) reduction(| : bad)
  {
    double* v = (double*)malloc((size_t)C * sizeof(double));
    if (!v) bad = 1;
#pragma omp for schedule(static)
    for (int64_t r = 0; r < N; ++r) {
      if (!v) continue;
      const int64_t yr = y[r];
      if (yr < 0 || yr >= C) { bad = 1; continue; }
      def_row(z + r * C, C, yr, scale, v, H + r, tau64 ? tau64 + r : NULL, loss64 ? loss64 + r : NULL,
              loss ? loss + r : NULL, kappa + r, grad ? grad + r * C : NULL, flags ? flags + r : NULL);
    }
    free(v);
  }
  return bad ? -2 : 0;
}

/* ------------------------------------------------------------------ streaming path (fw_cpu.cpp:340-390) */
/* keep the buffer entries > t, s = sum over them of (x - t) in fp64 (fw_cpu.cpp:331-335) */
static int64_t filter_sum(float* bv, int32_t* bi, int64_t n, double t, double* s) {
  const float r = fwo_round_down(t);
  double acc = 0.0;
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float x = bv[i];
    if (x > r) { acc += (double)x - t; bv[m] = x; bi[m] = bi[i]; ++m; }
  }
  *s = acc;
  return m;
}

/* status 0: support = bi[0:c), tau/thr set.  status 2: breakdown or work cap reached. */
static int chunked_row(const float* z, int64_t K, float* bv, int32_t* bi, int64_t chunk, int64_t cap,
                       double* tau, double* thr, int64_t* c) {
  int64_t n = 0, next = 256;
  double t = -INFINITY, s = 0.0;
  int fresh = 0;
  for (int64_t off = 0; off < K; off += chunk) {
    const int64_t len = K - off < chunk ? K - off : chunk;
    float cm = z[off];
    for (int64_t i = 1; i < len; ++i) if (z[off + i] > cm) cm = z[off + i];
    const double tm = (double)cm - 1.0;                /* chunk max - 1 is a lower bound     :347-348 */
    if (tm > t) { t = tm; fresh = 0; }
    const float r = fwo_round_down(t);
    const int64_t n0 = n;
    for (int64_t i = 0; i < len; ++i)                  /* compress z > t into the buffer     :350 */
      if (z[off + i] > r) { bv[n] = z[off + i]; bi[n] = (int32_t)(off + i); ++n; }
    if (n != n0) fresh = 0;
    if (n >= next) {                                   /* tighten: up to 4 Newton steps      :352-366 */
      n = filter_sum(bv, bi, n, t, &s);
      if (n == 0) return 2;
      for (int it = 0; it < 4; ++it) {
        const double tn = t + (s - 1.0) / (double)n;
        if (!(tn > t)) break;
        double s2;
        const int64_t n2 = filter_sum(bv, bi, n, tn, &s2);
        if (n2 == 0) return 2;
        const int same = n2 == n;
        t = tn; n = n2; s = s2;
        if (same) break;
      }
      next = 4 * n + 256;
      fresh = 1;
    }
  }
  if (!fresh) n = filter_sum(bv, bi, n, t, &s);
  if (n == 0) return 2;
  int64_t work = 0;
  for (;;) {                                           /* final Newton to the fixed point    :371-380 */
    const double tn = t + (s - 1.0) / (double)n;
    if (!(tn > t)) { *thr = t; *tau = tn; *c = n; return isfinite(tn) ? 0 : 2; }
    double s2;
    const int64_t n2 = filter_sum(bv, bi, n, tn, &s2);
    if (n2 == 0) return 2;
    if (n2 == n) { *thr = tn; *tau = tn + (s2 - 1.0) / (double)n2; *c = n; return 0; }
    t = tn; n = n2; s = s2;
    work += n;
    if (work > cap * K) return 2;
  }
}

int64_t fwo_single_pass(const float* z, const int64_t* y, int64_t N, int64_t C, double scale,
                        double* loss64, int64_t* kappa, float* grad, int nthreads,
                        int64_t chunk, int64_t cap_factor) {
  if (N < 0 || C < 1) return -1;
  if (chunk <= 0) chunk = 2048;
  if (cap_factor < 0) cap_factor = 4;
  int64_t fallbacks = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) reduction(+ : fallbacks)
  {
    float* bv = (float*)malloc((size_t)(C + 64) * sizeof(float));
    int32_t* bi = (int32_t*)malloc((size_t)(C + 64) * sizeof(int32_t));
    double* v = (double*)malloc((size_t)C * sizeof(double));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < N; ++r) {
      const float* zr = z + r * C;
      float* g = grad ? grad + r * C : NULL;
      const int64_t yr = y[r];
      double tau, thr;
      int64_t c;
      const int st = chunked_row(zr, C, bv, bi, chunk, cap_factor, &tau, &thr, &c);
      if (st == 0) {
        /* fw_cpu.cpp:601-614: scatter scale/c at the support, subtract scale at y */
        if (g) {
          memset(g, 0, (size_t)C * sizeof(float));
          const float inv = (float)(scale / (double)c);
          for (int64_t q = 0; q < c; ++q) g[bi[q]] = inv;
          g[yr] -= (float)scale;
        }
        loss64[r] = 1.0 + (thr - (double)zr[yr]) + (tau - thr);
        kappa[r] = c;
      } else {
        /* the reference falls back to Condat / median-of-medians (fw_cpu.cpp:417-479); any exact
           solver gives the same support, so the definition is used here */
        float H;
        int32_t k32;
        double t64, l64;
        def_row(zr, C, yr, scale, v, &H, &t64, &l64, NULL, &k32, g, NULL);
        loss64[r] = l64;
        kappa[r] = k32;
        fallbacks += 1;
      }
    }
    free(bv);
    free(bi);
    free(v);
  }
  return fallbacks;
}
