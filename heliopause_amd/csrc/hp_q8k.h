// hp_q8k.h -- wave-level Q8_K quantisation of one 256-element block.
//
// Semantics: packages/engine/wasm-kernels/src/lib.rs:1774-1811 (quantize_q8_k).
// `max` is the first element with the largest |x| (strictly-greater scan);
// amax == 0 gives d = 0 and zero quants; otherwise is = -127/max (correctly
// rounded f32 divide), q = (i8) min(127, roundf(is * x)) with ties away from
// zero and Rust's saturating cast (NaN -> 0), d = 1/is, and the block sums
// are sums of 32 consecutive quants.
//
// One wave handles a block; lane L owns elements 4L..4L+3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hp {

__device__ __forceinline__ int8_t q8k_sat_i8(float r) {
  if (r != r) return 0;
  if (r >= 127.0f) return 127;
  if (r <= -128.0f) return -128;
  return (int8_t)(int)r;
}

struct Q8KLane {
  int8_t q[4];  // quants of elements 4L..4L+3
  int bsum;     // sum of the 32 quants of this lane's sub-block (all 8 lanes agree)
  float d;      // block scale (all lanes agree)
};

__device__ __forceinline__ Q8KLane q8k_block(const float *__restrict__ xb, int lane) {
  const float4 v4 = reinterpret_cast<const float4 *>(xb)[lane];
  const float v[4] = {v4.x, v4.y, v4.z, v4.w};
  float amax = 0.0f, vmax = 0.0f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float a = fabsf(v[i]);
    if (a > amax) {
      amax = a;
      vmax = v[i];
      idx = 4 * lane + i;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float oa = __shfl_xor(amax, off);
    const float ov = __shfl_xor(vmax, off);
    const int oi = __shfl_xor(idx, off);
    if (oa > amax || (oa == amax && oi < idx)) {
      amax = oa;
      vmax = ov;
      idx = oi;
    }
  }
  Q8KLane r;
  r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
  r.d = 0.0f;
  if (amax != 0.0f) {
    const float inv = __fdiv_rn(-127.0f, vmax);
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = q8k_sat_i8(fminf(roundf(__fmul_rn(inv, v[i])), 127.0f));
    r.d = __fdiv_rn(1.0f, inv);
  }
  int s = (int)r.q[0] + (int)r.q[1] + (int)r.q[2] + (int)r.q[3];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  r.bsum = s;
  return r;
}

// Stores one block in the transposed 272-byte layout (hp_common.h):
// element e = 4L+i -> byte 32j + 4l + c with j = L/8, c = (L%8)/2, l = 4(L%2)+i;
// the 8 int16 sums at byte 256.
__device__ __forceinline__ void q8k_store_transposed(uint8_t *blk, const Q8KLane &r, int lane) {
  const int j = lane >> 3;
  const int c = (lane & 7) >> 1;
  const int lbase = 4 * (lane & 1);
#pragma unroll
  for (int i = 0; i < 4; i++) blk[32 * j + 4 * (lbase + i) + c] = (uint8_t)r.q[i];
  if ((lane & 7) == 0) reinterpret_cast<int16_t *>(blk + 256)[j] = (int16_t)r.bsum;
}

}  // namespace hp
