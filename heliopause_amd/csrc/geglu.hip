// geglu.hip -- the reference's GeGLU epilogue on gfx950.
//
// packages/engine/src/runner/wasm/layers.ts:450-456:
//   out[i] = fround(gelu(gate[i]) * up[i])
// with gelu (layers.ts:1062-1076) evaluated as the JS engine does: every
// Math.fround is an f64 -> f32 rounding, every other step an IEEE f64
// operation, Math.tanh is fdlibm's tanh (hp_tanh.h) and the f16 round trips
// use quant.ts:632-669 (round to nearest even, |v| < 2^-24 -> signed zero,
// |v| >= 65504 -> 65504).  The constant sqrt(2/pi) is computed on the host
// as Math.sqrt(2 / Math.PI) is (correctly rounded f64).
#include "hp_common.h"
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

__device__ __forceinline__ float gelu_ts(float vf, double c) {
  const double value = vf;
  if (value <= -10.0) return 0.0f;
  if (value >= 10.0) return vf;
  const double x = ts_f16_round(vf);
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

__global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                    size_t n, double c, float *__restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = (float)((double)gelu_ts(gate[i], c) * (double)up[i]);
}

hipError_t launch_geglu(const float *gate, const float *up, size_t n, double c, float *out, int num_cus,
                        hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  const size_t cap = (size_t)num_cus * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(geglu_kernel, dim3((unsigned)blocks), dim3(256), 0, s, gate, up, n, c, out);
  return hipGetLastError();
}

}  // namespace hp
