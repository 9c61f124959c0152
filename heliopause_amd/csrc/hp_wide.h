// hp_wide.h -- LDS layout and norm prologue of the row-block ("wide")
// matvec, shared by kquant_wide.hip and the persistent decode step
// (decode_fused.hip), whose projection stages run the same three phases
// (products in LDS, block-order chains, tails).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "hp_common.h"
#include "hp_kquant.h"
#include "hp_q8k16.h"
#include "hp_wave.h"

namespace hp {

// LDS carve-up of one workgroup (byte offsets).  The input: Q4_K reads the
// Q8_K image (cols * nb blocks of kQ8BlockBytes), Q6_K two masked copies of
// its quants (q8k_store16_split, 256 bytes per block each, at a stride of
// kSplitStride bytes).  Lanes of a wave read the same 16 bytes of
// consecutive blocks; a stride of 68 dwords (4 mod 32 banks) spreads eight
// such lanes over all banks, where 256 bytes would put them in one.
constexpr int kSplitStride = kQ8BlockBytes;

struct WideLayout {
  int nbp;        // products per (row, col, class) row: nb rounded up to 4, == 4 (mod 8)
  size_t xhi;     // Q6_K: [cols][nb] upper-half copies (the lower ones at 0)
  size_t xd;      // [cols * nb] f32 Q8_K scales (padded to 4 entries)
  size_t prod;    // [rows][cols][NC][nbp] f32 products
  size_t fin;     // [rows][cols][NC] f32 chain results
  size_t total;
};

__host__ __device__ inline WideLayout wide_layout(int cols, int nb, int type, int rows) {
  WideLayout L;
  const int nc = type == kTypeQ4K ? 9 : 8;
  const size_t nq = (size_t)cols * nb;
  L.nbp = ((nb + 3) & ~3) | 4;
  L.xhi = type == kTypeQ6K ? nq * kSplitStride : 0;
  L.xd = type == kTypeQ6K ? 2 * nq * kSplitStride : nq * kQ8BlockBytes;
  L.prod = L.xd + (size_t)((nq + 3) & ~3) * 4;
  L.fin = L.prod + (size_t)rows * cols * nc * L.nbp * 4;
  L.total = L.fin + (size_t)rows * cols * nc * 4;
  return L;
}

// The norm prologue's finish (hp_kquant.h norm_finish: the same arithmetic
// in the same order, so the same bits) where only the waves that hold one of
// the input's blocks do the math: with eight waves and a 10-block input,
// five would otherwise repeat it on zeros.  `active`: this wave holds a
// group below nb (wave-uniform).  Of the first four waves an inactive one
// contributes +0.0 to the two sums, as its zeroed lanes would.  Every thread
// of the workgroup calls it (two barriers).  `store_x`: this workgroup
// writes x1 (mode 2) through `put_x(grp, values)`.  y, r, wp, wn: the
// prologue's inputs (hp_kquant.h NormRegs), as separate arrays.
template <int MODE, class PutX>
__device__ __forceinline__ void wide_norm_finish_with(const NormIn &n, float (&y)[16], float (&r)[16],
                                                      const float (&wp)[16], const float (&wn)[16], float (&xv)[16],
                                                      int grp, int nb, int k, double *sh, bool active, bool store_x,
                                                      PutX put_x) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double part = 0.0;
  if (active) {
    if (grp >= nb) {
#pragma unroll
      for (int i = 0; i < 16; i++) y[i] = r[i] = 0.0f;
    }
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) ss += (double)y[i] * (double)y[i];
    part = wave_sum_f64(ss);
  }
  if (lane == 0 && wave < 4) sh[wave] = part;
  __syncthreads();
  double sc = 1.0 / sqrt(((sh[0] + sh[1]) + (sh[2] + sh[3])) / (double)k + n.eps);
  if (MODE == 2) {
    part = 0.0;
    if (active) {
      double ss = 0.0;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float t = (float)(((double)y[i] * sc) * (double)wp[i]);
        const float x1 = (r[i] + t) * n.scale;
        y[i] = x1;
        ss += (double)x1 * (double)x1;
      }
      if (store_x && grp < nb) put_x(grp, y);
      part = wave_sum_f64(ss);
    }
    if (lane == 0 && wave < 4) sh[4 + wave] = part;
    __syncthreads();
    sc = 1.0 / sqrt(((sh[4] + sh[5]) + (sh[6] + sh[7])) / (double)k + n.eps);
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = (float)(((double)y[i] * sc) * (double)wn[i]);
  }
}

// The wide kernel's form: workgroup 0 stores x1 to n.x_out.
template <int MODE>
__device__ __forceinline__ void wide_norm_finish(const NormIn &n, NormRegs &nr, float (&xv)[16], int grp, int nb,
                                                 int i16, int k, double *sh, bool active) {
  wide_norm_finish_with<MODE>(n, nr.y, nr.r, nr.wp, nr.wn, xv, grp, nb, k, sh, active, blockIdx.x == 0,
                              [&](int g, const float (&v)[16]) { store_x16(n.x_out + (size_t)g * kQK, v, i16); });
}

}  // namespace hp
