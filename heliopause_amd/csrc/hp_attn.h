// hp_attn.h -- numerics shared by the attention kernels (decode_layer.hip
// for decode and drafts, attn_prefill.hip for prefill chunks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hp {

// float32_to_float16 of lib.rs:2534-2569 as selects instead of branches
// (divergent branches cost every lane all of them): round half up on the 13
// dropped mantissa bits, a finite overflow saturates to 0x7bff, below 2^-14
// the hidden bit joins the mantissa and rounds half up at shift 14 - he,
// below 2^-25 the result is a signed zero, NaN becomes 0x7e00.  Adding 0x1000
// to exponent and mantissa together carries a mantissa overflow into the
// exponent as the reference's separate case does.
__host__ __device__ inline uint32_t rs_f16_bits(uint32_t bits) {
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t a = bits & 0x7fffffffu;
  const int e = (int)(a >> 23);
  uint32_t n = (a - (112u << 23) + 0x1000u) >> 13;  // he >= 1
  n = n < 0x7bffu ? n : 0x7bffu;
  const int sh = e < 102 ? 24 : 126 - e;  // 14 - he, 14..24 where it is used
  const uint32_t mh = (a & 0x7fffffu) | 0x800000u;
  uint32_t s = (mh + (1u << ((sh - 1) & 31))) >> (sh & 31);
  s = e >= 102 ? s : 0u;
  const uint32_t h = sign | (e >= 113 ? n : s);
  // inf keeps its sign as 0x7c00, NaN becomes 0x7e00 (masks, not a branch)
  const uint32_t special = (a & 0x7fffffu) == 0 ? (sign | 0x7c00u) : 0x7e00u;
  const uint32_t m255 = 0u - (uint32_t)(e == 255);
  return (h & ~m255) | (special & m255);
}

// float32_to_float16 then float16_to_float32 of lib.rs:2507-2568.
__device__ __forceinline__ float rs_f16_round(float v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)rs_f16_bits(__builtin_bit_cast(uint32_t, v)));
}

// Two f32 values as packed f16 (round to nearest even).
__device__ __forceinline__ uint32_t pack2_f16(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// Attention window of the token at `pos`: [start, start + count).
__device__ __forceinline__ void window_of(int pos, int capacity, int window, int *start, int *count) {
  int c = pos + 1;
  if (c > capacity) c = capacity;
  if (window > 0 && c > window) c = window;
  *count = c;
  *start = pos + 1 - c;
}

}  // namespace hp
