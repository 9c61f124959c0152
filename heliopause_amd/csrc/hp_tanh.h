// hp_tanh.h -- double-precision tanh by fdlibm's algorithm (s_tanh.c over
// s_expm1.c, Sun Microsystems 1993, freely redistributable), the algorithm
// V8 ships for Math.tanh.  The reference evaluates Math.tanh in gelu
// (packages/engine/src/runner/wasm/layers.ts:1062-1076) and in the logit
// softcap (layers.ts:407-412); using the same published algorithm with IEEE
// double operations and no contraction reproduces its results bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hp {

__host__ __device__ __forceinline__ uint32_t hi_word(double x) {
  return (uint32_t)(__builtin_bit_cast(uint64_t, x) >> 32);
}
__host__ __device__ __forceinline__ uint32_t lo_word(double x) {
  return (uint32_t)__builtin_bit_cast(uint64_t, x);
}
__host__ __device__ __forceinline__ double from_words(uint32_t hi, uint32_t lo) {
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// exp(x) - 1 (fdlibm s_expm1.c): reduction x = k*ln2 + r, |r| <= 0.5*ln2,
// then a rational approximation of r with a correction term.
__host__ __device__ inline double hp_expm1(double x) {
  const double o_threshold = 7.09782712893383973096e+02;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  const double invln2 = 1.44269504088896338700e+00;
  const double Q1 = -3.33333333333331316428e-02;
  const double Q2 = 1.58730158725481460165e-03;
  const double Q3 = -7.93650757867487942473e-05;
  const double Q4 = 4.00821782732936239552e-06;
  const double Q5 = -2.01099218183624371326e-07;
  const double huge = 1.0e+300, tiny = 1.0e-300;
  double y, hi, lo, c = 0.0, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = hi_word(x);
  const uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4043687Au) {  // |x| >= 56*ln2
    if (hx >= 0x40862E42u) {  // |x| >= 709.78...
      if (hx >= 0x7ff00000u) {
        if (((hx & 0xfffffu) | lo_word(x)) != 0) return x + x;  // NaN
        return xsb == 0 ? x : -1.0;                             // exp(+-inf) - 1
      }
      if (x > o_threshold) return huge * huge;  // overflow
    }
    if (xsb != 0) {  // x < -56*ln2: -1 with inexact
      if (x + tiny < 0.0) return tiny - 1.0;
    }
  }
  if (hx > 0x3fd62e42u) {    // |x| > 0.5 ln2
    if (hx < 0x3FF0A2B2u) {  // and |x| < 1.5 ln2
      if (xsb == 0) {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      } else {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      }
    } else {
      k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5 : -0.5));
      t = k;
      hi = x - t * ln2_hi;  // exact
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x3c900000u) {  // |x| < 2^-54
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5 * x;
  hxs = x * hfx;
  r1 = 1.0 + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0 - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0 - x * t));
  if (k == 0) return x - (x * e - hxs);
  const double twopk = from_words(0x3ff00000u + ((uint32_t)k << 20), 0);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5 * (x - e) - 0.5;
  if (k == 1) {
    if (x < -0.25) return -2.0 * (e - (x + 0.5));
    return 1.0 + 2.0 * (x - e);
  }
  if (k <= -2 || k > 56) {
    y = 1.0 - (e - x);
    if (k == 1024)
      y = y * 2.0 * 8.98846567431158e+307;  // 2^1023
    else
      y = y * twopk;
    return y - 1.0;
  }
  if (k < 20) {
    t = from_words(0x3ff00000u - (0x200000u >> k), 0);  // 1 - 2^-k
    y = t - (e - x);
    y = y * twopk;
  } else {
    t = from_words((uint32_t)(0x3ff - k) << 20, 0);  // 2^-k
    y = x - (e + t);
    y += 1.0;
    y = y * twopk;
  }
  return y;
}

// tanh(x) (fdlibm s_tanh.c).
__host__ __device__ inline double hp_tanh(double x) {
  const double tiny = 1.0e-300, huge = 1.0e300;
  double t, z;
  const uint32_t jx = hi_word(x);
  const uint32_t ix = jx & 0x7fffffffu;
  const bool neg = (jx & 0x80000000u) != 0;
  if (ix >= 0x7ff00000u) {  // inf or NaN
    if (!neg) return 1.0 / x + 1.0;
    return 1.0 / x - 1.0;
  }
  if (ix < 0x40360000u) {    // |x| < 22
    if (ix < 0x3e300000u) {  // |x| < 2^-28
      if (huge + x > 1.0) return x;
    }
    if (ix >= 0x3ff00000u) {  // |x| >= 1
      t = hp_expm1(2.0 * fabs(x));
      z = 1.0 - 2.0 / (t + 2.0);
    } else {
      t = hp_expm1(-2.0 * fabs(x));
      z = -t / (t + 2.0);
    }
  } else {
    z = 1.0 - tiny;  // |x| >= 22: +-1
  }
  return neg ? -z : z;
}

}  // namespace hp
