// hp_q8k16.h -- Q8_K of one 256-element block by one 16-lane DPP row, in
// the transposed 272-byte layout the vector-ALU matvec kernels read from LDS
// (hp_common.h: kQ8BlockBytes), and the element order its lanes load in.
// Shared by the matvec prologues and by the kernels that hand a matvec its
// input already quantised.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hp_common.h"
#include "hp_wave.h"

namespace hp {

// Q8_K of block (m, b) by one 16-lane DPP row (lib.rs:1774-1811).  Lane
// i16 = 2j + u owns the 16 elements 32j + 8c + 4u + i (c, i = 0..3), i.e.
// bytes 32j + 16u .. +15 of the transposed layout, so its quants are one
// 16-byte LDS store; its elements are scanned in increasing index order.
__device__ __forceinline__ void load_x16(float (&v)[16], const float *__restrict__ xb, int i16) {
  const int j = i16 >> 1, u = i16 & 1;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const float4 f = *reinterpret_cast<const float4 *>(xb + 32 * j + 8 * c + 4 * u);
    v[4 * c] = f.x;
    v[4 * c + 1] = f.y;
    v[4 * c + 2] = f.z;
    v[4 * c + 3] = f.w;
  }
}

__device__ __forceinline__ void store_x16(float *__restrict__ xb, const float (&v)[16], int i16) {
  const int j = i16 >> 1, u = i16 & 1;
#pragma unroll
  for (int c = 0; c < 4; c++)
    *reinterpret_cast<float4 *>(xb + 32 * j + 8 * c + 4 * u) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2],
                                                                           v[4 * c + 3]);
}

// One butterfly step of the (|x| desc, index asc) maximum with the partner
// lane selected by the DPP control.
template <int CTRL>
__device__ __forceinline__ void lexmax_step(float &amax, float &vmax, int &idx) {
  const float oa = dpp_f32<CTRL>(amax);
  const float ov = dpp_f32<CTRL>(vmax);
  const int oi = (int)dpp_u32<CTRL>((uint32_t)idx);
  const bool take = oa > amax || (oa == amax && oi < idx);
  amax = take ? oa : amax;
  vmax = take ? ov : vmax;
  idx = take ? oi : idx;
}

// -127 / (the block's first element of largest |x|), the same in all 16
// lanes of the row; nz: some element is not zero.
__device__ __forceinline__ float q8k_inv16(const float (&v)[16], int i16, bool &nz) {
  const int j = i16 >> 1, u = i16 & 1;
  float amax = 0.0f, vmax = 0.0f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float x = v[4 * c + i];
      const float av = fabsf(x);
      const bool gt = av > amax;  // strictly greater: the first maximum wins
      amax = gt ? av : amax;
      vmax = gt ? x : vmax;
      idx = gt ? 32 * j + 8 * c + 4 * u + i : idx;
    }
  // (amax desc, idx asc) across the 16 lanes of the row
  lexmax_step<kDppXor1>(amax, vmax, idx);
  lexmax_step<kDppXor2>(amax, vmax, idx);
  lexmax_step<kDppRowHalfMirror>(amax, vmax, idx);
  lexmax_step<kDppRowMirror>(amax, vmax, idx);
  nz = amax != 0.0f;
  return __fdiv_rn(-127.0f, vmax);
}

// Rust: (is * x).round().min(127.0) as i8.  For a finite is, |is * x| <= 127
// (1 + 2^-23); when the block's maximum is below ~3.7e-37 in magnitude, is
// overflows to -inf or +inf and the saturating cast gives -128 for products
// of -inf (the max(., -128) here); NaN (0 * inf) -> min() -> 127.  round()
// (half away from zero) as trunc(p + copysign(0.5 - 2^-25, p)): equal for
// every f32 |p| < 128 (checked exhaustively); the int conversion truncates,
// and truncation commutes with the clamp to [-128, 127].
__device__ __forceinline__ int q8k_round(float inv, float x) {
  const float p = __fmul_rn(inv, x);
  return (int)fmaxf(fminf(__fadd_rn(p, copysignf(0.49999997f, p)), 127.0f), -128.0f);
}

// The quantised block as one 16-lane row holds it: lane i16 = 2j + u owns
// dwords 8j + 4u .. 8j + 4u + 3 of the transposed layout (word[l4]: element
// 32j + 8c + 4u + l4 in byte c), sum: the sum of sub-block j's 32 quants
// (the image's bsums), in both lanes of the pair; inv: -127 / (the block's first
// element of largest |x|); nz: some element is not zero (else every quant
// is 0).
struct Q8Words {
  uint32_t word[4];
  int sum;
  float inv;
  bool nz;
};

__device__ __forceinline__ Q8Words q8k_words16(const float (&v)[16], int i16) {
  Q8Words r;
  r.inv = q8k_inv16(v, i16, r.nz);
  int sum = 0;
#pragma unroll
  for (int l4 = 0; l4 < 4; l4++) {
    int q[4];
#pragma unroll
    for (int c = 0; c < 4; c++) q[c] = q8k_round(r.inv, v[4 * c + l4]);
    // bytes q0..q3 (low to high): the low bytes of two packed int16 pairs
    const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(q[0], q[1]));
    const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(q[2], q[3]));
    const uint32_t wv = __builtin_amdgcn_perm(hi, lo, 0x06040200u);
    r.word[l4] = r.nz ? wv : 0u;  // dword l = 4u + l4 of sub-block j
    sum = __builtin_amdgcn_sdot4((int)r.word[l4], 0x01010101, sum, false);
  }
  r.sum = sum + (int)dpp_u32<kDppXor1>((uint32_t)sum);
  return r;
}

// The 272-byte block (256 quants, 8 sub-block sums) and its f32 scale.
__device__ __forceinline__ void q8k_store16(const Q8Words &q, int i16, uint8_t *blk, float *dptr) {
  const int j = i16 >> 1, u = i16 & 1;
  *reinterpret_cast<uint4 *>(blk + 32 * j + 16 * u) = make_uint4(q.word[0], q.word[1], q.word[2], q.word[3]);
  if (u == 0) reinterpret_cast<int16_t *>(blk + 256)[j] = (int16_t)q.sum;
  if (i16 == 0) *dptr = q.nz ? __fdiv_rn(1.0f, q.inv) : 0.0f;
}

__device__ __forceinline__ void q8k_block16(const float (&v)[16], int i16, uint8_t *blk, float *dptr) {
  q8k_store16(q8k_words16(v, i16), i16, blk, dptr);
}

// The block's quants as two masked 256-byte copies in the same order: lo
// keeps bytes 0, 1 of every dword (c = 0, 1: the first 16-element group of
// the dword's 32), hi bytes 2, 3 (the second group); and its f32 scale.  The
// Q6_K kernels' input (q6k_ints_split).
__device__ __forceinline__ void q8k_store16_split(const Q8Words &q, int i16, uint8_t *lo, uint8_t *hi,
                                                  float *dptr) {
  const int j = i16 >> 1, u = i16 & 1;
  *reinterpret_cast<uint4 *>(lo + 32 * j + 16 * u) =
      make_uint4(q.word[0] & 0xFFFFu, q.word[1] & 0xFFFFu, q.word[2] & 0xFFFFu, q.word[3] & 0xFFFFu);
  *reinterpret_cast<uint4 *>(hi + 32 * j + 16 * u) = make_uint4(
      q.word[0] & 0xFFFF0000u, q.word[1] & 0xFFFF0000u, q.word[2] & 0xFFFF0000u, q.word[3] & 0xFFFF0000u);
  if (i16 == 0) *dptr = q.nz ? __fdiv_rn(1.0f, q.inv) : 0.0f;
}

}  // namespace hp
