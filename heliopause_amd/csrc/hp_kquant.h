// hp_kquant.h -- the integer core of the vector-ALU Q4_K / Q6_K matvec
// kernels (one lane per row-block, all eight accumulator lanes of the
// reference's SIMD dot product) and their residual-norm prologue, shared by
// kquant_matvec.hip and kquant_wide.hip.
//
// Numerics follow packages/engine/wasm-kernels/src/lib.rs:2116-2172 (Q4_K)
// and 1923-1968 (Q6_K): per row-block and accumulator lane l the exact i32
// aux32[l] (and the Q4_K min sum sumi), formed with v_dot4_i32_i8 and the
// Abel summation described in kquant_matvec.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hp_common.h"
#include "hp_q8k16.h"
#include "hp_wave.h"

namespace hp {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// a * b + c with 24-bit multiplicands; here |T| < 2^23 and |sc_j - sc_j+1|
// < 2^8, so the product is exact.  Left to the compiler (no inline asm): its
// hazard recognizer must see the v_dot4c result being read.
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ uint32_t u4get(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Raw 16-byte chunks of one (row, block) lane: Q4_K uses c[0..8], Q6_K
// c[0..12] plus its f16 d from the side plane.
struct Regs {
  uint4 c[13];
  uint32_t d6;
};


// Integer part of one Q4_K row-block for M columns (exact aux32, sumi).
template <int M>
__device__ __forceinline__ void q4k_ints(const Regs &rg, const uint8_t *xq, int nb, int b, int (&aux)[M][8],
                                         int (&sumi)[M]) {
  const uint4 c0 = rg.c[0];
  const uint32_t s0 = c0.y, s1 = c0.z, s2 = c0.w;
  int sc[8], mn[8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    sc[j] = (s0 >> (8 * j)) & 63;
    mn[j] = (s1 >> (8 * j)) & 63;
    sc[j + 4] = ((s2 >> (8 * j)) & 15) | (((s0 >> (8 * j + 6)) & 3) << 4);
    mn[j + 4] = ((s2 >> (8 * j + 4)) & 15) | (((s1 >> (8 * j + 6)) & 3) << 4);
  }
  int dsc[8];  // Abel weights: sum_j sc_j d_j = sum_j T_j (sc_j - sc_{j+1})
#pragma unroll
  for (int j = 0; j < 8; j++) dsc[j] = j < 7 ? sc[j] - sc[j + 1] : sc[7];
  int T[M][8];
#pragma unroll
  for (int m = 0; m < M; m++) {
#pragma unroll
    for (int l = 0; l < 8; l++) {
      aux[m][l] = 0;
      T[m][l] = 0;
    }
    const uint4 bs = *reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes + 256);
    int si = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int v = (int)(int16_t)(u4get(bs, j >> 1) >> (16 * (j & 1)));
      si += __mul24(v, mn[j]);
    }
    sumi[m] = si;
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int p = j >> 1;
#pragma unroll
    for (int lq = 0; lq < 2; lq++) {
      const uint4 D = rg.c[1 + 2 * p + lq];
      uint32_t w[4];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        const uint32_t d = u4get(D, li);
        w[li] = (j & 1) ? ((d >> 4) & 0x0F0F0F0Fu) : (d & 0x0F0F0F0Fu);
      }
#pragma unroll
      for (int m = 0; m < M; m++) {
        const uint4 xv = reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes)[2 * j + lq];
#pragma unroll
        for (int li = 0; li < 4; li++) {
          const int l = 4 * lq + li;
          T[m][l] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xv, li), T[m][l], false);
          aux[m][l] = mad24(T[m][l], dsc[j], aux[m][l]);
        }
      }
    }
  }
}

// Integer part of one Q6_K row-block for M columns (exact aux32).  Bytes of
// the unpacked weight carry 4 * (q6 - 32); each dword covers groups 2j (c =
// 0,1) and 2j+1 (c = 2,3), split by masking.
template <int M>
__device__ __forceinline__ void q6k_ints(const Regs &rg, const uint8_t *xq, int nb, int b, int (&aux)[M][8]) {
  const uint4 csc = rg.c[12];
  int sc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) sc[g] = (int)(int8_t)(u4get(csc, g >> 2) >> (8 * (g & 3)));
  int dsc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) dsc[g] = g < 15 ? sc[g] - sc[g + 1] : sc[15];
  int T[M][8];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) {
      aux[m][l] = 0;
      T[m][l] = 0;
    }
#pragma unroll
  for (int j = 0; j < 8; j++) {
#pragma unroll
    for (int lq = 0; lq < 2; lq++) {
      const uint4 Dl = rg.c[2 * (j >> 1) + lq];
      const uint4 Dh = rg.c[8 + 2 * (j >> 2) + lq];
      uint32_t wlo[4], whi[4];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        const uint32_t ql = u4get(Dl, li), qh = u4get(Dh, li);
        const uint32_t nib = (j & 1) ? ((ql >> 2) & 0x3C3C3C3Cu) : ((ql << 2) & 0x3C3C3C3Cu);
        const int u = j & 3;
        const uint32_t w = nib | ((qh << (6 - 2 * u)) & 0xC0C0C0C0u);  // bytes = 4 * (q6 - 32)
        wlo[li] = w & 0x0000FFFFu;
        whi[li] = w & 0xFFFF0000u;
      }
#pragma unroll
      for (int m = 0; m < M; m++) {
        const uint4 xv = reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes)[2 * j + lq];
#pragma unroll
        for (int li = 0; li < 4; li++) {
          const int l = 4 * lq + li;
          T[m][l] = __builtin_amdgcn_sdot4((int)wlo[li], (int)u4get(xv, li), T[m][l], false);
          aux[m][l] = mad24(T[m][l], dsc[2 * j], aux[m][l]);
          T[m][l] = __builtin_amdgcn_sdot4((int)whi[li], (int)u4get(xv, li), T[m][l], false);
          aux[m][l] = mad24(T[m][l], dsc[2 * j + 1], aux[m][l]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) aux[m][l] >>= 2;  // weights carried 4 * (q6 - 32)
}

// q6k_ints with the input as two masked copies (q8k_store16_split): xlo
// keeps bytes 0, 1 of every dword of the Q8_K quants, xhi bytes 2, 3, 256
// bytes per block each at a stride of STRIDE bytes.  A dword of the unpacked weight covers group 2j
// (bytes 0, 1) and group 2j+1 (bytes 2, 3), so the Abel running dot steps
// T_2j = T_2j-1 + dot(w, xlo), T_2j+1 = T_2j + dot(w, xhi) in place: the same
// integers as q6k_ints with neither the weight masked nor T copied.
template <int M, int STRIDE>
__device__ __forceinline__ void q6k_ints_split(const Regs &rg, const uint8_t *xlo, const uint8_t *xhi, int nb, int b,
                                               int (&aux)[M][8]) {
  const uint4 csc = rg.c[12];
  int sc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) sc[g] = (int)(int8_t)(u4get(csc, g >> 2) >> (8 * (g & 3)));
  int dsc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) dsc[g] = g < 15 ? sc[g] - sc[g + 1] : sc[15];
  int T[M][8];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) {
      aux[m][l] = 0;
      T[m][l] = 0;
    }
#pragma unroll
  for (int j = 0; j < 8; j++) {
#pragma unroll
    for (int lq = 0; lq < 2; lq++) {
      const uint4 Dl = rg.c[2 * (j >> 1) + lq];
      const uint4 Dh = rg.c[8 + 2 * (j >> 2) + lq];
      uint32_t w[4];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        const uint32_t ql = u4get(Dl, li), qh = u4get(Dh, li);
        const uint32_t nib = (j & 1) ? ((ql >> 2) & 0x3C3C3C3Cu) : ((ql << 2) & 0x3C3C3C3Cu);
        const int u = j & 3;
        w[li] = nib | ((qh << (6 - 2 * u)) & 0xC0C0C0C0u);  // bytes = 4 * (q6 - 32)
      }
#pragma unroll
      for (int m = 0; m < M; m++) {
        const size_t off = ((size_t)m * nb + b) * STRIDE;
        const uint4 xl = reinterpret_cast<const uint4 *>(xlo + off)[2 * j + lq];
        const uint4 xh = reinterpret_cast<const uint4 *>(xhi + off)[2 * j + lq];
#pragma unroll
        for (int li = 0; li < 4; li++) {
          const int l = 4 * lq + li;
          T[m][l] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xl, li), T[m][l], false);
          aux[m][l] = mad24(T[m][l], dsc[2 * j], aux[m][l]);
          T[m][l] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xh, li), T[m][l], false);
          aux[m][l] = mad24(T[m][l], dsc[2 * j + 1], aux[m][l]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) aux[m][l] >>= 2;  // weights carried 4 * (q6 - 32)
}

// Half row-blocks: lane classes l = 4h .. 4h+3 of one (row, block) only
// (the half-split and wide kernels).  A half loads chunk 0 (Q4_K) or the
// scales (Q6_K) and the nibble (and high-bit) chunks of its classes.
struct HalfRegs {
  uint4 c0;    // bytes 0..15 of the block (Q4_K) / the 16 scales (Q6_K)
  uint4 d[4];  // Q4_K nibble chunks 1 + 2p + h; Q6_K low-nibble chunks 2p + h
  uint4 e[2];  // Q6_K high-bit chunks 8 + 2p + h
  uint32_t d6;
};

template <int M>
__device__ __forceinline__ void q4k_ints_half(const HalfRegs &rg, const uint8_t *xq, int nb, int b, int h,
                                              int (&aux)[M][4], int (&sumi)[M]) {
  const uint32_t s0 = rg.c0.y, s1 = rg.c0.z, s2 = rg.c0.w;
  int sc[8], mn[8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    sc[j] = (s0 >> (8 * j)) & 63;
    mn[j] = (s1 >> (8 * j)) & 63;
    sc[j + 4] = ((s2 >> (8 * j)) & 15) | (((s0 >> (8 * j + 6)) & 3) << 4);
    mn[j + 4] = ((s2 >> (8 * j + 4)) & 15) | (((s1 >> (8 * j + 6)) & 3) << 4);
  }
  int dsc[8];  // Abel weights: sum_j sc_j d_j = sum_j T_j (sc_j - sc_{j+1})
#pragma unroll
  for (int j = 0; j < 8; j++) dsc[j] = j < 7 ? sc[j] - sc[j + 1] : sc[7];
  int T[M][4];
#pragma unroll
  for (int m = 0; m < M; m++) {
#pragma unroll
    for (int l = 0; l < 4; l++) aux[m][l] = T[m][l] = 0;
    const uint4 bs = *reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes + 256);
    int si = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int v = (int)(int16_t)(u4get(bs, j >> 1) >> (16 * (j & 1)));
      si += __mul24(v, mn[j]);
    }
    sumi[m] = si;
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint4 D = rg.d[j >> 1];
    uint32_t w[4];
#pragma unroll
    for (int li = 0; li < 4; li++) {
      const uint32_t d = u4get(D, li);
      w[li] = (j & 1) ? ((d >> 4) & 0x0F0F0F0Fu) : (d & 0x0F0F0F0Fu);
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint4 xv = reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes)[2 * j + h];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        T[m][li] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xv, li), T[m][li], false);
        aux[m][li] = mad24(T[m][li], dsc[j], aux[m][li]);
      }
    }
  }
}

template <int M>
__device__ __forceinline__ void q6k_ints_half(const HalfRegs &rg, const uint8_t *xq, int nb, int b, int h,
                                              int (&aux)[M][4]) {
  int sc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) sc[g] = (int)(int8_t)(u4get(rg.c0, g >> 2) >> (8 * (g & 3)));
  int dsc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) dsc[g] = g < 15 ? sc[g] - sc[g + 1] : sc[15];
  int T[M][4];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 4; l++) aux[m][l] = T[m][l] = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint4 Dl = rg.d[j >> 1];
    const uint4 Dh = rg.e[j >> 2];
    uint32_t wlo[4], whi[4];
#pragma unroll
    for (int li = 0; li < 4; li++) {
      const uint32_t ql = u4get(Dl, li), qh = u4get(Dh, li);
      const uint32_t nib = (j & 1) ? ((ql >> 2) & 0x3C3C3C3Cu) : ((ql << 2) & 0x3C3C3C3Cu);
      const int u = j & 3;
      const uint32_t w = nib | ((qh << (6 - 2 * u)) & 0xC0C0C0C0u);  // bytes = 4 * (q6 - 32)
      wlo[li] = w & 0x0000FFFFu;
      whi[li] = w & 0xFFFF0000u;
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint4 xv = reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes)[2 * j + h];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        T[m][li] = __builtin_amdgcn_sdot4((int)wlo[li], (int)u4get(xv, li), T[m][li], false);
        aux[m][li] = mad24(T[m][li], dsc[2 * j], aux[m][li]);
        T[m][li] = __builtin_amdgcn_sdot4((int)whi[li], (int)u4get(xv, li), T[m][li], false);
        aux[m][li] = mad24(T[m][li], dsc[2 * j + 1], aux[m][li]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 4; l++) aux[m][l] >>= 2;  // weights carried 4 * (q6 - 32)
}

// q6k_ints_half with the input as the two masked copies of q6k_ints_split:
// the same integers for lane classes 4h .. 4h+3.
template <int M, int STRIDE>
__device__ __forceinline__ void q6k_ints_half_split(const HalfRegs &rg, const uint8_t *xlo, const uint8_t *xhi, int nb,
                                                    int b, int h, int (&aux)[M][4]) {
  int sc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) sc[g] = (int)(int8_t)(u4get(rg.c0, g >> 2) >> (8 * (g & 3)));
  int dsc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) dsc[g] = g < 15 ? sc[g] - sc[g + 1] : sc[15];
  int T[M][4];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 4; l++) aux[m][l] = T[m][l] = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint4 Dl = rg.d[j >> 1];
    const uint4 Dh = rg.e[j >> 2];
    uint32_t w[4];
#pragma unroll
    for (int li = 0; li < 4; li++) {
      const uint32_t ql = u4get(Dl, li), qh = u4get(Dh, li);
      const uint32_t nib = (j & 1) ? ((ql >> 2) & 0x3C3C3C3Cu) : ((ql << 2) & 0x3C3C3C3Cu);
      const int u = j & 3;
      w[li] = nib | ((qh << (6 - 2 * u)) & 0xC0C0C0C0u);  // bytes = 4 * (q6 - 32)
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const size_t off = ((size_t)m * nb + b) * STRIDE;
      const uint4 xl = reinterpret_cast<const uint4 *>(xlo + off)[2 * j + h];
      const uint4 xh = reinterpret_cast<const uint4 *>(xhi + off)[2 * j + h];
#pragma unroll
      for (int li = 0; li < 4; li++) {
        T[m][li] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xl, li), T[m][li], false);
        aux[m][li] = mad24(T[m][li], dsc[2 * j], aux[m][li]);
        T[m][li] = __builtin_amdgcn_sdot4((int)w[li], (int)u4get(xh, li), T[m][li], false);
        aux[m][li] = mad24(T[m][li], dsc[2 * j + 1], aux[m][li]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 4; l++) aux[m][l] >>= 2;  // weights carried 4 * (q6 - 32)
}

// Norm prologue of a one-column launch (NormIn, hp_common.h): group grp < nb
// of 16 lanes holds block grp in load_x16's element order; the sums of
// squares are f64 sums over the workgroup (256 threads).
struct NormRegs {
  float y[16], r[16], wp[16], wn[16];
};

// Every group loads (groups grp >= nb re-read block nb - 1; norm_finish
// zeroes them): no branch around the loads, so nothing that consumes them can
// be placed ahead of the weight loads issued next.
template <int MODE>
__device__ __forceinline__ void norm_load(const NormIn &n, NormRegs &nr, int grp, int nb, int i16) {
  const size_t off = (size_t)min(grp, nb - 1) * kQK;
  load_x16(nr.y, n.y + off, i16);
  if (MODE == 2) {
    load_x16(nr.r, n.x_res + off, i16);
    load_x16(nr.wp, n.w_post + off, i16);
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) nr.r[i] = nr.wp[i] = 0.0f;
  }
  load_x16(nr.wn, n.w_next + off, i16);
}

// Sum over the workgroup's first four waves (the 16 groups a norm prologue
// uses; waves past them, in workgroups of more than four, hold none), the
// same order at any workgroup size; sh (4 doubles) must not have been used by
// an earlier call in the kernel (no barrier guards its reuse).  Every thread
// of the workgroup must call it.
__device__ __forceinline__ double wg_sum_f64(double v, double *sh) {
  v = wave_sum_f64(v);
  if ((threadIdx.x & 63) == 0 && threadIdx.x < 256) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

template <int MODE>
__device__ __forceinline__ void norm_finish(const NormIn &n, NormRegs &nr, float (&xv)[16], int grp, int nb,
                                            int i16, int k, double *sh) {
  if (grp >= nb) {
#pragma unroll
    for (int i = 0; i < 16; i++) nr.y[i] = nr.r[i] = 0.0f;
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 16; i++) ss += (double)nr.y[i] * (double)nr.y[i];
  double sc = 1.0 / sqrt(wg_sum_f64(ss, sh) / (double)k + n.eps);
  if (MODE == 2) {
    ss = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float t = (float)(((double)nr.y[i] * sc) * (double)nr.wp[i]);
      const float x1 = (nr.r[i] + t) * n.scale;
      nr.y[i] = x1;
      ss += (double)x1 * (double)x1;
    }
    if (blockIdx.x == 0 && grp < nb) store_x16(n.x_out + (size_t)grp * kQK, nr.y, i16);
    sc = 1.0 / sqrt(wg_sum_f64(ss, sh + 4) / (double)k + n.eps);
  }
#pragma unroll
  for (int i = 0; i < 16; i++) xv[i] = (float)(((double)nr.y[i] * sc) * (double)nr.wn[i]);
}

}  // namespace hp
