// hp_f2tile.h -- the fast prefill kernel's activation tiles: Q8_K of the
// input (quantize_q8_k, packages/engine/wasm-kernels/src/lib.rs:1774-1811)
// stored as f16 in the order its B fragments are read.  Written by the
// prefill pre-pass (kquant_prefill.hip) and, for a launch whose input is a
// norm's output, by the norm kernel (decode_layer.hip).
//
// Tile (column tile ct, block b) at xt + (ct * nb + b) * kF2XTile, 64 columns:
//   f16 quants [class l][quarter][column][8]        32768 bytes
//     (the 8: the quarter's two 4-element runs r = 0, 1, each stored as
//     elements 0, 2, 1, 3 -- the order in which the kernel's Q4_K weight
//     fragments come out of a quant dword without a byte permute)
//   f16 16-element sums [group / 8][column][8]       2048 bytes
//   f32 d per column                                   256 bytes
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hp_mfma.h"
#include "hp_q8k16.h"
#include "hp_wave.h"

namespace hp {

constexpr int kF2Cols = 64;
constexpr int kF2XTile = 32768 + 2048 + 256;  // 35,072 bytes per (column tile, block)

// One 16-lane row's block (load_x16 order; zeros for a padding column) into
// column n of its tile.
__device__ __forceinline__ void f2_tile_store16(const float (&v)[16], int i16, uint8_t *tile, int n) {
  _Float16 *xh = reinterpret_cast<_Float16 *>(tile);
  _Float16 *xb = reinterpret_cast<_Float16 *>(tile + 32768);
  float *xd = reinterpret_cast<float *>(tile + 32768 + 2048);
  bool nz;
  const float inv = q8k_inv16(v, i16, nz);
  int q[16];
#pragma unroll
  for (int e = 0; e < 16; e++) q[e] = nz ? q8k_round(inv, v[e]) : 0;
  const int j = i16 >> 1, u = i16 & 1, qq = j >> 1;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int l = 4 * u + i;
    const half2v lo = (half2v){(_Float16)q[i], (_Float16)q[8 + i]};
    const half2v hi = (half2v){(_Float16)q[4 + i], (_Float16)q[12 + i]};
    *reinterpret_cast<uint2 *>(xh + ((l * 4 + qq) * kF2Cols + n) * 8 + 4 * (j & 1)) =
        make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
  }
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s0 += q[i];
    s1 += q[8 + i];
  }
  s0 += (int)dpp_u32<kDppXor1>((uint32_t)s0);
  s1 += (int)dpp_u32<kDppXor1>((uint32_t)s1);
  const int h = 2 * j + u;  // lane u writes group 2j + u
  xb[((h >> 3) * kF2Cols + n) * 8 + (h & 7)] = (_Float16)(u ? s1 : s0);
  if (i16 == 0) xd[n] = nz ? __fdiv_rn(1.0f, inv) : 0.0f;
}

}  // namespace hp
