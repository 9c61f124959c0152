// hp_exp.h -- double-precision exp by fdlibm's algorithm (e_exp.c, Sun
// Microsystems 1993, freely redistributable; the form in FreeBSD's msun),
// which V8 ships as ieee754::exp for Math.exp.  The reference's sampling
// softmax (packages/engine/src/generation.ts:157-165) calls Math.exp; with
// the same published algorithm, IEEE double operations and no contraction
// the results agree bit for bit (pinned against Math.exp outputs of the JS
// engine in tests/golden/v8_exp.json).
#pragma once

#include "hp_tanh.h"

namespace hp {

// exp(x): x = k*ln2 + r with |r| <= 0.5*ln2, exp(r) from a degree-5
// minimax polynomial in r*r (the Remez form R(r^2) with exp(r) = 1 + 2r /
// (R - r)), then scaled by 2^k.
__host__ __device__ inline double hp_exp(double x) {
  const double o_threshold = 7.09782712893383973096e+02;
  const double u_threshold = -7.45133219101941108420e+02;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  const double invln2 = 1.44269504088896338700e+00;
  const double P1 = 1.66666666666666019037e-01;
  const double P2 = -2.77777777770155933842e-03;
  const double P3 = 6.61375632143793436117e-05;
  const double P4 = -1.65339022054652515390e-06;
  const double P5 = 4.13813679705723846039e-08;
  const double E = 2.718281828459045;
  const double huge = 1.0e+300;
  const double twom1000 = 9.33263618503218878990e-302;  // 2^-1000
  const double two1023 = 8.988465674311579539e307;      // 2^1023
  double hi = 0.0, lo = 0.0, c, t, y;
  int32_t k = 0;
  uint32_t hx = hi_word(x);
  const int xsb = (int)(hx >> 31);
  hx &= 0x7fffffffu;
  if (hx >= 0x40862E42u) {  // |x| >= 709.78...
    if (hx >= 0x7ff00000u) {
      if (((hx & 0xfffffu) | lo_word(x)) != 0) return x + x;  // NaN
      return xsb == 0 ? x : 0.0;                              // exp(+-inf) = inf, 0
    }
    if (x > o_threshold) return huge * huge;          // overflow
    if (x < u_threshold) return twom1000 * twom1000;  // underflow
  }
  if (hx > 0x3FD62E42u) {    // |x| > 0.5 ln2
    if (hx < 0x3FF0A2B2u) {  // and |x| < 1.5 ln2
      if (x == 1.0) return E;  // the JS engine returns the correctly rounded e here
      hi = xsb == 0 ? x - ln2_hi : x + ln2_hi;
      lo = xsb == 0 ? ln2_lo : -ln2_lo;
      k = 1 - xsb - xsb;
    } else {
      k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5 : -0.5));
      t = (double)k;
      hi = x - t * ln2_hi;  // exact: t*ln2_hi has 32 significant bits at most
      lo = t * ln2_lo;
    }
    x = hi - lo;
  } else if (hx < 0x3E300000u) {  // |x| < 2^-28
    if (huge + x > 1.0) return 1.0 + x;
  } else {
    k = 0;
  }
  t = x * x;
  const double twopk = k >= -1021 ? from_words(0x3FF00000u + ((uint32_t)k << 20), 0)
                                  : from_words(0x3FF00000u + ((uint32_t)(k + 1000) << 20), 0);
  c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) {
    if (k == 1024) return y * 2.0 * two1023;
    return y * twopk;
  }
  return y * twopk * twom1000;
}

}  // namespace hp
