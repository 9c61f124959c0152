// hp_mfma.h -- f16 operand helpers shared by the matrix-core kernels
// (kquant_mfma.hip for decode columns, kquant_prefill.hip for prefill).
//
// Weights enter v_mfma_f32_16x16x32_f16 as sc * q, exact in f16: a 4- or
// 6-bit quant q (as the byte of a dword) is turned into the f16 1024 + q by a
// byte permute under the exponent byte 0x64, and one packed f16 FMA with the
// scale gives s * (q + 1024 - off) = s * q' exactly (all values < 2^11 in
// magnitude and integer).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hp {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f_bits(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint32_t u4at(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }
__device__ __forceinline__ uint32_t as_u32(half2v v) { return __builtin_bit_cast(uint32_t, v); }

// Halves (1024 + byte a, 1024 + byte b) of dword v: the f16 with exponent
// bits 0x64 and mantissa = the byte is exactly 1024 + byte (byte < 1024).
template <uint32_t SEL>
__device__ __forceinline__ half2v magic_pair(uint32_t v) {
  return as_h2(__builtin_amdgcn_perm(0x64646464u, v, SEL));
}
constexpr uint32_t kSel01 = 0x04010400u;  // bytes 0, 1
constexpr uint32_t kSel23 = 0x04030402u;  // bytes 2, 3
constexpr uint32_t kSel02 = 0x04020400u;  // bytes 0, 2
constexpr uint32_t kSel13 = 0x04030401u;  // bytes 1, 3

// Halves of dword v under the exponent bits 0x64, with no byte permute:
// MASK 0x000F000F gives (1024 + v[3:0], 1024 + v[19:16]), MASK 0x00F000F0
// gives (1024 + 16 v[7:4], 1024 + 16 v[23:20]) (mantissas below 1024, exact).
// `exp` is 0x64006400 in a vector register (magic_nib_exp), so the mask can
// be the one scalar operand of a single v_and_or_b32.
template <uint32_t MASK>
__device__ __forceinline__ half2v magic_nib(uint32_t v, uint32_t exp) {
  return as_h2((v & MASK) | exp);
}
__device__ __forceinline__ uint32_t magic_nib_exp() {
  uint32_t e;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(e));  // opaque: not folded back into a literal
  return e;
}
constexpr uint32_t kNibLo = 0x000F000Fu;
constexpr uint32_t kNibHi = 0x00F000F0u;

// (s, s) for scale byte `idx` of dword v (unsigned bytes) and the matching
// addend -off * s, both exact in f16: fma((1024 + q), s, -off * s) = s * (q + 1024 - off).
__device__ __forceinline__ half2v dup_byte(uint32_t v, int idx, float bias) {
  const uint32_t sel = (uint32_t)idx | 0x04000400u | ((uint32_t)idx << 16);
  const half2v h = as_h2(__builtin_amdgcn_perm(0x64646464u, v, sel));
  return h - (half2v){(_Float16)bias, (_Float16)bias};
}

// (s / 16, s / 16) for scale byte `idx` of dword v and, with it, a scale for
// magic_nib<kNibHi>'s halves: the f16 with exponent bits 0x54 and mantissa =
// the byte is 64 + byte / 16 exactly.
__device__ __forceinline__ half2v dup_byte_16th(uint32_t v, int idx) {
  const uint32_t sel = (uint32_t)idx | 0x04000400u | ((uint32_t)idx << 16);
  const half2v h = as_h2(__builtin_amdgcn_perm(0x54545454u, v, sel));
  return h - (half2v){(_Float16)64.0f, (_Float16)64.0f};
}

__device__ __forceinline__ half2v fma2(half2v a, half2v b, half2v c) { return __builtin_elementwise_fma(a, b, c); }

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8 cat(half2v a, half2v b, half2v c, half2v d) {
  return (half8){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

}  // namespace hp
