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
#include "hp_gelu.h"

namespace hp {

__global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                    size_t n, double c, float *__restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = geglu_ts(gate[i], up[i], c);
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
