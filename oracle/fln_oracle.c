/*
 * fln_oracle.c -- plain-C restatement of the fused normalization path (TEST INFRASTRUCTURE ONLY:
 * used by tests/ as a checker at the full benchmark sizes and by bench.py's cpu_baseline leg as the
 * CPU port that is timed; never linked into the product library).
 *
 * Scalar, single-threaded, float64 accumulation.  Inputs are float32 arrays (bf16/f16 values
 * widen to float32 exactly).  Row-major [rows, cols]; statistics recomputed here in float64.
 *
 * LayerNorm forward follows `layernorm_kernel` (reference csrc/layernorm_cuda_kernel.cu:39-92):
 * mean = sum/N (:57-66), two-pass biased variance (:69-80), rstd = 1/sqrt(var + eps) (:79),
 * y = (x - mean) * rstd * gamma + beta (:84-91).  The backward closed forms restate the
 * contract the reference declares but never defines (csrc/layernorm.h:24-32).  RMSNorm and the
 * fp8 output are new on this path (no reference code); see oracle/norms.py for the same
 * formulas in numpy.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static void row_stats_ln(const float* x, int64_t n, double eps, double* mean, double* rstd) {
  double s = 0.0;
  for (int64_t j = 0; j < n; ++j) s += x[j];
  const double mu = s / (double)n;
  double q = 0.0;
  for (int64_t j = 0; j < n; ++j) {
    const double d = x[j] - mu;
    q += d * d;
  }
  *mean = mu;
  *rstd = 1.0 / sqrt(q / (double)n + eps);
}

static double row_rstd_rms(const float* x, int64_t n, double eps) {
  double q = 0.0;
  for (int64_t j = 0; j < n; ++j) q += (double)x[j] * (double)x[j];
  return 1.0 / sqrt(q / (double)n + eps);
}

/* y (float32, rounded once from float64), mean/rstd (float64, may be NULL). */
void orc_layernorm_fwd(const float* x, const float* gamma, const float* beta, int64_t rows,
                       int64_t cols, double eps, float* y, double* mean, double* rstd) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double mu, rs;
    row_stats_ln(xr, cols, eps, &mu, &rs);
    if (mean) mean[r] = mu;
    if (rstd) rstd[r] = rs;
    float* yr = y + r * cols;
    for (int64_t j = 0; j < cols; ++j) {
      double v = (xr[j] - mu) * rs;
      if (gamma) v *= gamma[j];
      if (beta) v += beta[j];
      yr[j] = (float)v;
    }
  }
}

void orc_rmsnorm_fwd(const float* x, const float* weight, int64_t rows, int64_t cols, double eps,
                     float* y, double* rstd) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    const double rs = row_rstd_rms(xr, cols, eps);
    if (rstd) rstd[r] = rs;
    float* yr = y + r * cols;
    for (int64_t j = 0; j < cols; ++j) {
      double v = xr[j] * rs;
      if (weight) v *= weight[j];
      yr[j] = (float)v;
    }
  }
}

/* dx (float32, may be NULL); dgamma/dbeta (float64 [cols], may be NULL; overwritten). */
void orc_layernorm_bwd(const float* dy, const float* x, const float* gamma, int64_t rows,
                       int64_t cols, double eps, float* dx, double* dgamma, double* dbeta) {
  if (dgamma) memset(dgamma, 0, sizeof(double) * (size_t)cols);
  if (dbeta) memset(dbeta, 0, sizeof(double) * (size_t)cols);
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    const float* dr = dy + r * cols;
    double mu, rs;
    row_stats_ln(xr, cols, eps, &mu, &rs);
    double s1 = 0.0, s2 = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const double xh = (xr[j] - mu) * rs;
      const double g = (double)dr[j] * (gamma ? gamma[j] : 1.0);
      s1 += g;
      s2 += g * xh;
    }
    const double c1 = s1 / (double)cols, c2 = s2 / (double)cols;
    for (int64_t j = 0; j < cols; ++j) {
      const double xh = (xr[j] - mu) * rs;
      const double g = (double)dr[j] * (gamma ? gamma[j] : 1.0);
      if (dx) dx[r * cols + j] = (float)(rs * (g - c1 - xh * c2));
      if (dgamma) dgamma[j] += dr[j] * xh;
      if (dbeta) dbeta[j] += dr[j];
    }
  }
}

void orc_rmsnorm_bwd(const float* dy, const float* x, const float* weight, int64_t rows,
                     int64_t cols, double eps, float* dx, double* dweight) {
  if (dweight) memset(dweight, 0, sizeof(double) * (size_t)cols);
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    const float* dr = dy + r * cols;
    const double rs = row_rstd_rms(xr, cols, eps);
    double s2 = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const double xh = xr[j] * rs;
      s2 += (double)dr[j] * (weight ? weight[j] : 1.0) * xh;
    }
    const double c2 = s2 / (double)cols;
    for (int64_t j = 0; j < cols; ++j) {
      const double xh = xr[j] * rs;
      const double g = (double)dr[j] * (weight ? weight[j] : 1.0);
      if (dx) dx[r * cols + j] = (float)(rs * (g - xh * c2));
      if (dweight) dweight[j] += dr[j] * xh;
    }
  }
}

/* OCP e4m3fn, saturating, round-to-nearest-even (same definition as norms.fp8_e4m3fn_encode). */
uint8_t orc_fp8_e4m3fn(double v) {
  if (isnan(v)) return 0x7F;
  const uint8_t sign = signbit(v) ? 0x80 : 0x00;
  double a = fabs(v);
  if (a > 448.0) a = 448.0;
  int code;
  if (a < 0.015625) { /* 2^-6: subnormal range, step 2^-9 */
    code = (int)nearbyint(a * 512.0);
  } else {
    int k;
    const double f = frexp(a, &k); /* a = f 2^k, f in [0.5, 1) */
    int e = k - 1;
    int m = (int)nearbyint(16.0 * f - 8.0);
    if (m == 8) {
      m = 0;
      e += 1;
    }
    code = ((e + 7) << 3) | m;
  }
  if (code > 0x7E) code = 0x7E;
  return (uint8_t)(code | sign);
}

void orc_layernorm_fp8(const float* x, const float* gamma, const float* beta, int64_t rows,
                       int64_t cols, double eps, uint8_t* q, float* scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double mu, rs;
    row_stats_ln(xr, cols, eps, &mu, &rs);
    double amax = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      double v = (xr[j] - mu) * rs;
      if (gamma) v *= gamma[j];
      if (beta) v += beta[j];
      if (fabs(v) > amax || v != v) amax = fabs(v); /* a NaN propagates, as in amax */
    }
    const double sc = amax / 448.0;
    scale[r] = (float)sc;
    for (int64_t j = 0; j < cols; ++j) {
      double v = (xr[j] - mu) * rs;
      if (gamma) v *= gamma[j];
      if (beta) v += beta[j];
      q[r * cols + j] = amax > 0.0 ? orc_fp8_e4m3fn(v / sc) : 0;
    }
  }
}

/* RMSNorm -> fp8: the same row rule on rms-normalized values (weight may be NULL). */
void orc_rmsnorm_fp8(const float* x, const float* weight, int64_t rows, int64_t cols, double eps,
                     uint8_t* q, float* scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    const double rs = row_rstd_rms(xr, cols, eps);
    double amax = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      double v = xr[j] * rs;
      if (weight) v *= weight[j];
      if (fabs(v) > amax || v != v) amax = fabs(v); /* a NaN propagates, as in amax */
    }
    const double sc = amax / 448.0;
    scale[r] = (float)sc;
    for (int64_t j = 0; j < cols; ++j) {
      double v = xr[j] * rs;
      if (weight) v *= weight[j];
      q[r * cols + j] = amax > 0.0 ? orc_fp8_e4m3fn(v / sc) : 0;
    }
  }
}
