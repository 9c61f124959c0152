// q8k.hip -- standalone Q8_K quantisation (test hook).
//
// Writes the reference's own layout (lib.rs:1540-1544 QuantizedQ8K): qs
// [cols][K] int8 in element order, d [cols][K/256] f32, bsums32 [cols][K/32]
// int16, so the activation quantisation the matvec prologue performs can be
// compared bit-for-bit with the oracle.  The matvec kernels run the same
// device function (hp_q8k.h) into LDS.
#include "hp_common.h"
#include "hp_q8k.h"

namespace hp {

__global__ __launch_bounds__(64) void q8k_natural_kernel(const float *__restrict__ x, int k, int nb,
                                                         int8_t *__restrict__ qs, float *__restrict__ d,
                                                         int16_t *__restrict__ bsums) {
  const int b = blockIdx.x;
  const int m = blockIdx.y;
  const int lane = threadIdx.x;
  const Q8KLane r = q8k_block(x + (size_t)m * k + (size_t)b * kQK, lane);
  int8_t *qb = qs + (size_t)m * k + (size_t)b * kQK + 4 * lane;
#pragma unroll
  for (int i = 0; i < 4; i++) qb[i] = r.q[i];
  if ((lane & 7) == 0) bsums[(size_t)m * (k / 32) + (size_t)b * 8 + (lane >> 3)] = (int16_t)r.bsum;
  if (lane == 0) d[(size_t)m * nb + b] = r.d;
}

hipError_t launch_q8k_natural(const float *x, int k, int cols, int8_t *qs, float *d, int16_t *bsums,
                              hipStream_t s) {
  const int nb = k / kQK;
  hipLaunchKernelGGL(q8k_natural_kernel, dim3(nb, cols), dim3(64), 0, s, x, k, nb, qs, d, bsums);
  return hipGetLastError();
}

}  // namespace hp
