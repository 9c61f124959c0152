// hp_gelu.h -- the reference's gelu, as the JS engine evaluates it.
//
// packages/engine/src/runner/wasm/layers.ts:1062-1076: every Math.fround is an
// f64 -> f32 rounding, every other step an IEEE f64 operation, Math.tanh is
// fdlibm's tanh (hp_tanh.h) and the f16 round trips use quant.ts:632-669
// (round to nearest even, |v| < 2^-24 -> signed zero, |v| >= 65504 -> 65504).
// The constant c = sqrt(2/pi) comes from the host (Math.sqrt(2 / Math.PI)).
#pragma once

#include <hip/hip_runtime.h>

#include "hp_tanh.h"

namespace hp {

// float32ToFloat16 then float16ToFloat32 (quant.ts:618-669) of an f32 value.
__device__ __forceinline__ float ts_f16_round(float v) {
  if (v != v) return __builtin_bit_cast(float, 0x7fc00000u);  // 0x7e00 -> NaN
  const float a = fabsf(v);
  if (a == __builtin_inff()) return v;
  if (a >= 65504.0f) return copysignf(65504.0f, v);
  if (a < 5.9604644775390625e-08f) return copysignf(0.0f, v);  // 2^-24
  return (float)(_Float16)v;  // round to nearest even
}

// gelu past its range checks, as a function of x = the f16 round trip of its
// input.
__device__ __forceinline__ float gelu_of_x(double x, double c) {
  const double t1 = (float)(c * x);
  const double x2 = (float)(x * x);
  const double t2 = (float)(0.044715 * x2);
  const double t3 = (float)(1.0 + t2);
  const double inner = (float)(t1 * t3);
  const double half = (float)(0.5 * x);
  const double t4 = (float)(1.0 + hp_tanh(inner));
  const double act = (float)(half * t4);
  return ts_f16_round((float)act);
}

__device__ __forceinline__ float gelu_ts(float vf, double c) {
  const double value = vf;
  if (value <= -10.0) return 0.0f;
  if (value >= 10.0) return vf;
  return gelu_of_x(ts_f16_round(vf), c);
}

// The same gelu from a table: inside (-10, 10) the result depends only on the
// 16 bits of x = ts_f16_round(vf), so lut[bits] = gelu_of_x(x, c) for every
// f16 pattern (built by launch_gelu_lut; each entry is an f16 value, NaN as
// 0x7e00) gives gelu_ts exactly, in one gather instead of f64 tanh.
__device__ __forceinline__ float gelu_lut(float vf, const uint16_t *__restrict__ lut) {
  const double value = vf;
  if (value <= -10.0) return 0.0f;
  if (value >= 10.0) return vf;
  const uint16_t x = __builtin_bit_cast(uint16_t, (_Float16)ts_f16_round(vf));
  return (float)__builtin_bit_cast(_Float16, lut[x]);
}

// GeGLU of one element (layers.ts:450-456): fround(gelu(gate) * up).
__device__ __forceinline__ float geglu_ts(float gate, float up, double c) {
  return (float)((double)gelu_ts(gate, c) * (double)up);
}

__device__ __forceinline__ float geglu_lut(float gate, float up, const uint16_t *__restrict__ lut) {
  return (float)((double)gelu_lut(gate, lut) * (double)up);
}

}  // namespace hp
