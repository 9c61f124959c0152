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
#include "hp_q8k16.h"

namespace hp {

// lut[bits] = gelu of the f16 value with those bits (hp_gelu.h gelu_lut).
__global__ __launch_bounds__(256) void gelu_lut_kernel(double c, uint16_t *__restrict__ lut) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 65536) return;
  const double x = (float)__builtin_bit_cast(_Float16, (uint16_t)i);
  lut[i] = __builtin_bit_cast(uint16_t, (_Float16)gelu_of_x(x, c));
}

hipError_t launch_gelu_lut(double c, uint16_t *lut, hipStream_t s) {
  hipLaunchKernelGGL(gelu_lut_kernel, dim3(256), dim3(256), 0, s, c, lut);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                    size_t n, const uint16_t *__restrict__ lut,
                                                    float *__restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = geglu_lut(gate[i], up[i], lut);
}

// One workgroup per 256-element block of one column: each thread takes one
// element's GeGLU (stored to out and to LDS), then one 16-lane group
// quantises the block from LDS into the image.
__global__ __launch_bounds__(256) void geglu_q8k_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                        int rows, int blocks, const uint16_t *__restrict__ lut,
                                                        float *__restrict__ out, uint8_t *__restrict__ img) {
  __shared__ float hs[kQK];
  const int q = blockIdx.x, t = threadIdx.x;
  const int nb = rows / kQK, m = q / nb, b = q - m * nb;
  const size_t off = (size_t)m * rows + (size_t)b * kQK;
  const float h = geglu_lut(gate[off + t], up[off + t], lut);
  out[off + t] = h;
  hs[t] = h;
  __syncthreads();
  if (t < 16) {
    float v[16];
    const int j = t >> 1, u = t & 1;
#pragma unroll
    for (int cc = 0; cc < 4; cc++)
#pragma unroll
      for (int i = 0; i < 4; i++) v[4 * cc + i] = hs[32 * j + 8 * cc + 4 * u + i];
    q8k_block16(v, t, img + (size_t)q * kQ8BlockBytes,
                reinterpret_cast<float *>(img + (size_t)blocks * kQ8BlockBytes) + q);
  }
}

hipError_t launch_geglu_q8k(const float *gate, const float *up, int rows, int cols, const uint16_t *lut, float *out,
                            uint8_t *q8img, hipStream_t s) {
  if (rows <= 0 || rows % kQK != 0 || cols < 1) return hipErrorInvalidValue;
  const int blocks = cols * (rows / kQK);
  hipLaunchKernelGGL(geglu_q8k_kernel, dim3((unsigned)blocks), dim3(256), 0, s, gate, up, rows, blocks, lut, out,
                     q8img);
  return hipGetLastError();
}

hipError_t launch_geglu(const float *gate, const float *up, size_t n, const uint16_t *lut, float *out, int num_cus,
                        hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  const size_t cap = (size_t)num_cus * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(geglu_kernel, dim3((unsigned)blocks), dim3(256), 0, s, gate, up, n, lut, out);
  return hipGetLastError();
}

}  // namespace hp
