/* One row of the C1 program for oracle/c/baseline.c: the sum over the row of
 * tanh(x*y + 0.5)*x - max(y, 0), in double from the f32 inputs (the numpy
 * oracle's c1_rowsum, oracle/ops.py). tanh is written out so the loop
 * vectorizes: tanh(t) = sign(t) (1 - e) / (1 + e), e = exp(-2|t|), with exp by
 * the textbook reduction -2|t| = k ln2 + r (k rounded by the 1.5 * 2^52 shift) (|r| <= ln2 / 2, ln2 split in a
 * high part with trailing zero bits and a low part, Cody & Waite) and the
 * Taylor series of exp(r) to r^13 / 13! (truncation below 2^-60), scaled by
 * 2^k through the exponent bits. |t| is clamped to 40, where tanh is 1 in
 * double. Absolute error of tanh below 1e-15 (tests/test_oracle_c.py pins
 * it against numpy). Test infrastructure, like the rest of oracle/. */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline double exp_neg(double x) { /* x in [-80, 0] */
  const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
  /* k = round(x / ln2): adding 1.5 * 2^52 leaves k in the low bits */
  const double kd = x * 1.44269504088896338700e+00 + 6755399441055744.0;
  const double k = kd - 6755399441055744.0;
  const double r = (x - k * ln2_hi) - k * ln2_lo;
  double p = 1.0 / 6227020800.0; /* 1/13! */
  p = p * r + 1.0 / 479001600.0;
  p = p * r + 1.0 / 39916800.0;
  p = p * r + 1.0 / 3628800.0;
  p = p * r + 1.0 / 362880.0;
  p = p * r + 1.0 / 40320.0;
  p = p * r + 1.0 / 5040.0;
  p = p * r + 1.0 / 720.0;
  p = p * r + 1.0 / 120.0;
  p = p * r + 1.0 / 24.0;
  p = p * r + 1.0 / 6.0;
  p = p * r + 0.5;
  p = p * r + 1.0;
  p = p * r + 1.0;
  uint64_t kb;
  memcpy(&kb, &kd, 8);
  const uint64_t bits = (kb + 1023u) << 52; /* 2^k (k >= -116: normal): kd's high bits shift out */
  double s;
  memcpy(&s, &bits, 8);
  return p * s;
}

double pjrtx_oracle_tanh(double t) {
  const double a = fmin(fabs(t), 40.0);
  const double e = exp_neg(-2.0 * a);
  const double v = (1.0 - e) / (1.0 + e);
  return t < 0 ? -v : v;
}

double pjrtx_oracle_c1_row(const float* xr, const float* yr, int64_t cols) {
  double s = 0.0;
#pragma omp simd reduction(+ : s)
  for (int64_t i = 0; i < cols; ++i) {
    const double a = xr[i], b = yr[i];
    s += pjrtx_oracle_tanh(a * b + 0.5) * a - (b > 0.0 ? b : 0.0);
  }
  return s;
}
