// hp_attn.h -- numerics shared by the attention kernels (decode_layer.hip
// for decode and drafts, attn_prefill.hip for prefill chunks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hp {

// float32_to_float16 then float16_to_float32 of lib.rs:2507-2568.
__device__ __forceinline__ float rs_f16_round(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int e = (int)((bits >> 23) & 0xffu);
  const uint32_t man = bits & 0x7fffffu;
  uint32_t h;
  if (e == 0xff) {
    h = man == 0 ? (sign | 0x7c00u) : 0x7e00u;
  } else {
    const int he = e - 112;
    if (he >= 31) {
      h = sign | 0x7bffu;
    } else if (he <= 0) {
      if (he < -10) {
        h = sign;
      } else {
        const uint32_t mh = man | 0x800000u;
        const int sh = 14 - he;
        h = sign | ((mh + (1u << (sh - 1))) >> sh);
      }
    } else {
      const uint32_t rm = man + 0x1000u;
      if (rm & 0x800000u)
        h = he + 1 >= 31 ? (sign | 0x7bffu) : (sign | ((uint32_t)(he + 1) << 10));
      else
        h = sign | ((uint32_t)he << 10) | (rm >> 13);
    }
  }
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
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
