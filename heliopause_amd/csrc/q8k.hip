// q8k.hip -- Q8_K activation quantisation on gfx950.
//
// Semantics: packages/engine/wasm-kernels/src/lib.rs:1774-1811
// (quantize_q8_k).  Per 256-element block: `max` is the first element with
// the largest |x| (strictly-greater scan); amax == 0 gives d = 0 and zero
// quants; otherwise is = -127/max (correctly rounded f32 divide),
// q = (i8) min(127, roundf(is * x)) with ties away from zero and Rust's
// saturating cast, d = 1/is, bsums32 = sums of 32 consecutive quants.
//
// One wave per (block, column); lane L owns elements 4L..4L+3.  Output goes
// to the transposed layout described in hp_common.h.
#include "hp_common.h"

namespace hp {

__device__ __forceinline__ int8_t sat_i8(float r) {
  if (r != r) return 0;
  if (r >= 127.0f) return 127;
  if (r <= -128.0f) return -128;
  return (int8_t)(int)r;
}

__global__ __launch_bounds__(64) void q8k_quantize_kernel(const float *__restrict__ x, int k, int nb,
                                                          uint8_t *__restrict__ q8, float *__restrict__ q8d) {
  const int b = blockIdx.x;
  const int m = blockIdx.y;
  const int lane = threadIdx.x;
  const float4 v4 = reinterpret_cast<const float4 *>(x + (size_t)m * k + (size_t)b * kQK)[lane];
  const float v[4] = {v4.x, v4.y, v4.z, v4.w};

  // first index of the largest |x| within the lane, then across the wave
  float amax = 0.0f, vmax = 0.0f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float a = fabsf(v[i]);
    if (a > amax) {
      amax = a;
      vmax = v[i];
      idx = 4 * lane + i;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float oa = __shfl_xor(amax, off);
    float ov = __shfl_xor(vmax, off);
    int oi = __shfl_xor(idx, off);
    if (oa > amax || (oa == amax && oi < idx)) {
      amax = oa;
      vmax = ov;
      idx = oi;
    }
  }

  int8_t q[4] = {0, 0, 0, 0};
  float inv = 0.0f;
  const bool zero = !(amax != 0.0f);
  if (!zero) {
    inv = __fdiv_rn(-127.0f, vmax);
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = sat_i8(fminf(roundf(__fmul_rn(inv, v[i])), 127.0f));
  }

  // sums of 32 = 8 lanes
  int s = (int)q[0] + (int)q[1] + (int)q[2] + (int)q[3];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);

  uint8_t *blk = q8 + ((size_t)m * nb + b) * kQ8BlockBytes;
  // element e = 4*lane + i -> sub-block j = lane/8, c = (lane%8)/2, l = 4*(lane%2)+i
  const int j = lane >> 3;
  const int c = (lane & 7) >> 1;
  const int lbase = 4 * (lane & 1);
#pragma unroll
  for (int i = 0; i < 4; i++) blk[32 * j + 4 * (lbase + i) + c] = (uint8_t)q[i];
  if ((lane & 7) == 0) reinterpret_cast<int16_t *>(blk + 256)[j] = (int16_t)s;
  if (lane == 0) q8d[(size_t)m * nb + b] = zero ? 0.0f : __fdiv_rn(1.0f, inv);
}

hipError_t launch_q8k_quantize(const float *x, int k, int cols, uint8_t *q8, float *q8d, hipStream_t s) {
  const int nb = k / kQK;
  hipLaunchKernelGGL(q8k_quantize_kernel, dim3(nb, cols), dim3(64), 0, s, x, k, nb, q8, q8d);
  return hipGetLastError();
}

}  // namespace hp
