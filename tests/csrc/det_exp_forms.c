/*
 * Bit-equality check of the window-score kernels' exp forms against the
 * oracle's exp_det (test infrastructure; built and run by
 * tests/test_det_exp_forms.py on the CPU).
 *
 * The kernels (DetExp in hotcold-kv-cache_amd/csrc/hc_common.h) evaluate the
 * contract's exp with the same IEEE operations rearranged:
 *   - rint(x / ln2) as (t + 1.5*2^52 + bias) - (1.5*2^52 + bias), t = x * (1/ln2)
 *     rounded first (bias 0, or 44 for the fixed-point path: even biases keep
 *     round-to-nearest-even), k + bias from the low mantissa bits;
 *   - 2^k scaling by ldexp;
 *   - the clamp max(x, -708) with the result zeroed below -708 (exp form), or,
 *     for the fixed-point sums, exp(-708) kept (rint(e * 2^44) is 0 either way);
 *   - rint(e * 2^44) as ldexp(p, k + 44) + 2^52 minus the bias pattern.
 * Each form is restated here in plain C and compared bit for bit with the
 * oracle's exp_det / rint(exp_det * 2^44) on edge arguments (every k boundary
 * and rounding tie of x / ln2, -708, 0, -0, -inf, NaN, tiny) and N random ones.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/hc_oracle.c"

static double kernel_exp(double x) {
  const int ok = x >= -708.0;
  const double xc = fmax(x, -708.0);
  volatile double t = xc * INV_LN2;
  volatile double sh = t + 6755399441055744.0;
  const double kf = sh - 6755399441055744.0;
  uint64_t b;
  memcpy(&b, (const void*)&sh, 8);
  const int k = (int)(uint32_t)b;
  double r = fma(-kf, LN2_HI, xc);
  r = fma(-kf, LN2_LO, r);
  static const double c[13] = {
      2.08767569878680989792e-09, 2.50521083854417187751e-08, 2.75573192239858906526e-07,
      2.75573192239858906526e-06, 2.48015873015873015873e-05, 1.98412698412698412698e-04,
      1.38888888888888888889e-03, 8.33333333333333333333e-03, 4.16666666666666666667e-02,
      1.66666666666666666667e-01, 5.00000000000000000000e-01, 1.0, 1.0};
  double p = c[0];
  for (int i = 1; i < 13; ++i) p = fma(p, r, c[i]);
  return ok ? ldexp(p, k) : 0.0;
}

static uint64_t kernel_fixed(double x) {
  const double xc = fmax(x, -708.0);
  volatile double t = xc * INV_LN2;
  volatile double sh = t + (6755399441055744.0 + 44.0);
  const double kf = sh - (6755399441055744.0 + 44.0);
  uint64_t b;
  memcpy(&b, (const void*)&sh, 8);
  const int k44 = (int)(uint32_t)b;
  double r = fma(-kf, LN2_HI, xc);
  r = fma(-kf, LN2_LO, r);
  static const double c[13] = {
      2.08767569878680989792e-09, 2.50521083854417187751e-08, 2.75573192239858906526e-07,
      2.75573192239858906526e-06, 2.48015873015873015873e-05, 1.98412698412698412698e-04,
      1.38888888888888888889e-03, 8.33333333333333333333e-03, 4.16666666666666666667e-02,
      1.66666666666666666667e-01, 5.00000000000000000000e-01, 1.0, 1.0};
  double p = c[0];
  for (int i = 1; i < 13; ++i) p = fma(p, r, c[i]);
  volatile double u = ldexp(p, k44);
  volatile double v = u + 4503599627370496.0;
  uint64_t bv;
  memcpy(&bv, (const void*)&v, 8);
  return bv - 0x4330000000000000ull;
}

static long n_checked = 0, n_bad = 0;
static void check(double x) {
  const double a = hco_exp_det(x), b = kernel_exp(x);
  ++n_checked;
  if (memcmp(&a, &b, 8) != 0) {
    if (n_bad < 5) printf("exp mismatch at x=%.17g: oracle %.17g kernel %.17g\n", x, a, b);
    ++n_bad;
  }
  const uint64_t fa = fix44(hco_exp_det(x)), fb = kernel_fixed(x);
  if (fa != fb) {
    if (n_bad < 5) printf("fixed mismatch at x=%.17g: oracle %llu kernel %llu\n", x, (unsigned long long)fa,
                          (unsigned long long)fb);
    ++n_bad;
  }
}

int main(int argc, char** argv) {
  const long n = argc > 1 ? atol(argv[1]) : 1000000;
  check(0.0);
  check(-0.0);
  check(-708.0);
  check(nextafter(-708.0, 0.0));
  check(nextafter(-708.0, -1e9));
  check(-INFINITY);
  check(NAN);
  check(-5e-324);
  check(-1e-300);
  for (int k = -1022; k <= 1; ++k) {
    const double xs[2] = {(k + 0.5) * 0.6931471805599453, k * 0.6931471805599453};
    for (int j = 0; j < 2; ++j) {
      double y = xs[j];
      for (int d = 0; d < 24; ++d) y = nextafter(y, -2000.0);
      for (int d = 0; d < 48; ++d) {
        if (y <= 0.0) check(y);
        y = nextafter(y, 2000.0);
      }
    }
  }
  uint64_t s = 0x9E3779B97F4A7C15ull;
  for (long i = 0; i < n; ++i) {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    double x;
    switch (i & 3) {
      case 0: x = -708.0 * ((s >> 11) * 0x1p-53); break;  /* uniform [-708, 0] */
      case 1: x = -30.0 * ((s >> 11) * 0x1p-53); break;   /* the softmax bulk */
      case 2: x = -ldexp((double)((s >> 11) | 1), -53 - (int)(s & 63)); break;  /* tiny */
      default: {  /* random bit patterns, negative, exponents around 1 */
        const uint64_t b = (s & 0x000FFFFFFFFFFFFFull) | ((uint64_t)(0x3F0 + (s >> 60)) << 52) | 0x8000000000000000ull;
        memcpy(&x, &b, 8);
      }
    }
    check(x);
  }
  printf("checked %ld arguments, %ld mismatches\n", n_checked, n_bad);
  return n_bad != 0;
}
