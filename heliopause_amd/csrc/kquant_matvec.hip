// kquant_matvec.hip -- Q4_K / Q6_K x Q8_K matvec for M = 1..8 columns (gfx950).
//
// Numerics (bit-exact with the reference's WASM path):
//   packages/engine/wasm-kernels/src/lib.rs:2116-2172 (Q4_K), 1923-1968 (Q6_K),
//   multi-weight launch with one shared Q8_K: lib.rs:300-426.
// Per row r, block b and accumulator lane l:
//   Q4_K aux32[l] = sum_j sc_j * sum_{c<4} q4(32j+8c+l) * q8(32j+8c+l)   (exact i32)
//        sumi     = sum_j bsums32_j * min_j
//   Q6_K aux32[l] = sum_g sc_g * sum_{c<2} (q6(16g+8c+l) - 32) * q8(16g+8c+l)
//   float tail, in block order, no FMA:
//        d = dW_b * dX_b; sums[l] += d * f32(aux32[l]);
//        Q4_K: sumf -= (dminW_b * dX_b) * f32(sumi)
//   result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
//
// Work split: a wave owns one tile (R rows x S block slots per iteration,
// layout in hp_common.h).  Every lane computes the exact integers of one
// (row, block) with v_dot4_i32_i8 on four elements that share lane l, then
// forms the f32 products d*f32(aux32[l]).  The order-dependent additions
// run in LDS: lane (row, chain) adds the S products of its chain in block
// order.  The activation (Q8_K) is staged once per workgroup in LDS.
#include "hp_common.h"

namespace hp {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, 0, false);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t u4get(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Integer part of one Q4_K row-block for M columns.
template <int M>
__device__ __forceinline__ void q4k_ints(const uint4 *__restrict__ ch, int stride, const uint8_t *xq,
                                         int nb, int b, int (&aux)[M][8], int (&sumi)[M], uint32_t &dbits) {
  const uint4 c0 = ch[0];
  uint4 cw[8];
#pragma unroll
  for (int c = 0; c < 8; c++) cw[c] = ch[(1 + c) * stride];
  dbits = c0.x;
  const uint32_t s0 = c0.y, s1 = c0.z, s2 = c0.w;
  int sc[8], mn[8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    sc[j] = (s0 >> (8 * j)) & 63;
    mn[j] = (s1 >> (8 * j)) & 63;
    sc[j + 4] = ((s2 >> (8 * j)) & 15) | (((s0 >> (8 * j + 6)) & 3) << 4);
    mn[j + 4] = ((s2 >> (8 * j + 4)) & 15) | (((s1 >> (8 * j + 6)) & 3) << 4);
  }
#pragma unroll
  for (int m = 0; m < M; m++) {
#pragma unroll
    for (int l = 0; l < 8; l++) aux[m][l] = 0;
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
  for (int p = 0; p < 4; p++) {
#pragma unroll
    for (int lq = 0; lq < 2; lq++) {
      const uint4 D = cw[2 * p + lq];
#pragma unroll
      for (int m = 0; m < M; m++) {
        const uint4 *xb = reinterpret_cast<const uint4 *>(xq + ((size_t)m * nb + b) * kQ8BlockBytes);
        const uint4 xlo = xb[4 * p + lq];      // X[2p][4lq..4lq+3]
        const uint4 xhi = xb[4 * p + 2 + lq];  // X[2p+1][4lq..4lq+3]
#pragma unroll
        for (int li = 0; li < 4; li++) {
          const uint32_t d = u4get(D, li);
          const uint32_t lo = d & 0x0F0F0F0Fu;
          const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;
          int a = aux[m][4 * lq + li];
          a += __mul24(sc[2 * p], dot4(lo, u4get(xlo, li)));
          a += __mul24(sc[2 * p + 1], dot4(hi, u4get(xhi, li)));
          aux[m][4 * lq + li] = a;
        }
      }
    }
  }
}

// Integer part of one Q6_K row-block for M columns (aux32 exact).
template <int M>
__device__ __forceinline__ void q6k_ints(const uint4 *__restrict__ ch, int stride, const uint8_t *xq, int nb,
                                         int b, int (&aux)[M][8]) {
  uint4 cq[8], ch4[4];
#pragma unroll
  for (int c = 0; c < 8; c++) cq[c] = ch[c * stride];
#pragma unroll
  for (int c = 0; c < 4; c++) ch4[c] = ch[(8 + c) * stride];
  const uint4 csc = ch[12 * stride];
  int sc[16];
#pragma unroll
  for (int g = 0; g < 16; g++) sc[g] = (int)(int8_t)(u4get(csc, g >> 2) >> (8 * (g & 3)));
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) aux[m][l] = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
#pragma unroll
    for (int lq = 0; lq < 2; lq++) {
      const uint4 Dl = cq[2 * (j >> 1) + lq];
      const uint4 Dh = ch4[2 * (j >> 2) + lq];
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
          int a = aux[m][4 * lq + li];
          a += __mul24(sc[2 * j], dot4(wlo[li], u4get(xv, li)));
          a += __mul24(sc[2 * j + 1], dot4(whi[li], u4get(xv, li)));
          aux[m][4 * lq + li] = a;
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int l = 0; l < 8; l++) aux[m][l] >>= 2;  // weights carried 4 * (q6 - 32)
}

template <int M>
__global__ __launch_bounds__(256) void kquant_matvec_kernel(const MatvecArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const TileGeom g = a.g;
  const int nb = g.nb, S = g.S, R = g.R;
  uint8_t *xq = smem;
  float *xd = reinterpret_cast<float *>(smem + (size_t)M * nb * kQ8BlockBytes);
  const int xd_floats = (M * nb + 3) & ~3;
  const int per_wave = R * 9 * S + M * R * 9;

  // stage the Q8_K activations of this launch's columns
  {
    const int n16 = M * nb * kQ8BlockBytes / 16;
    const uint4 *src = reinterpret_cast<const uint4 *>(a.q8);
    uint4 *dst = reinterpret_cast<uint4 *>(xq);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
    for (int i = threadIdx.x; i < M * nb; i += blockDim.x) xd[i] = a.q8d[i];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpg = blockDim.x >> 6;
  float *prod = xd + xd_floats + wave * per_wave;  // [R][9][S]
  float *acc = prod + R * 9 * S;                    // [M][R][9]

  for (int t = blockIdx.x * wpg + wave; t < a.total_tiles; t += gridDim.x * wpg) {
    WeightDesc W = a.w[0];
    if (a.count > 1 && t >= a.w[1].tile_begin) W = a.w[1];
    if (a.count > 2 && t >= a.w[2].tile_begin) W = a.w[2];
    if (a.count > 3 && t >= a.w[3].tile_begin) W = a.w[3];
    const int row0 = (t - W.tile_begin) * R;
    const int Rt = min(R, W.rows - row0);
    const int lanes = Rt * S;
    const bool q4 = W.type == kTypeQ4K;
    const int CH = q4 ? 9 : 13;
    const int NCH = q4 ? 9 : 8;
    const uint8_t *tile = W.data + (size_t)row0 * nb * CH * 16;
    const int r = lane / S;
    const int s = lane - r * S;

    for (int it = 0; it < g.iters; it++) {
      const int b = it * S + s;
      int aux[M][8];
      int sumi[M];
      float dw = 0.0f, dminw = 0.0f;
      if (lane < lanes) {
        const uint4 *ch = reinterpret_cast<const uint4 *>(tile + ((size_t)it * CH * lanes + lane) * 16);
        if (q4) {
          uint32_t dbits;
          q4k_ints<M>(ch, lanes, xq, nb, b, aux, sumi, dbits);
          dw = h2f(dbits & 0xFFFFu);
          dminw = h2f(dbits >> 16);
        } else {
          q6k_ints<M>(ch, lanes, xq, nb, b, aux);
          dw = h2f(W.dplane[(size_t)row0 * nb + (size_t)it * lanes + lane]);
#pragma unroll
          for (int m = 0; m < M; m++) sumi[m] = 0;
        }
      }
#pragma unroll
      for (int m = 0; m < M; m++) {
        if (lane < lanes) {
          const float dx = xd[m * nb + b];
          const float dd = __fmul_rn(dw, dx);
          float *pr = prod + (r * 9) * S + s;
#pragma unroll
          for (int l = 0; l < 8; l++) pr[l * S] = __fmul_rn(dd, (float)aux[m][l]);
          if (q4) pr[8 * S] = __fmul_rn(__fmul_rn(dminw, dx), (float)sumi[m]);
        }
        wave_lds_sync();
        for (int cid = lane; cid < Rt * NCH; cid += 64) {
          const int rr = cid / NCH;
          const int chn = cid - rr * NCH;
          const float *pp = prod + (rr * 9 + chn) * S;
          float *ap = acc + (m * R + rr) * 9 + chn;
          float v = it == 0 ? 0.0f : *ap;
          if (chn == 8) {
            for (int q = 0; q < S; q++) v = __fsub_rn(v, pp[q]);
          } else {
            for (int q = 0; q < S; q++) v = __fadd_rn(v, pp[q]);
          }
          *ap = v;
        }
        wave_lds_sync();
      }
    }

    // final combine: [sumf +] ((((-0 + s0) + s1) + ...) + s7)
    for (int cid = lane; cid < M * Rt; cid += 64) {
      const int m = cid / Rt;
      const int rr = cid - m * Rt;
      const float *ap = acc + (m * R + rr) * 9;
      float tsum = -0.0f;
#pragma unroll
      for (int l = 0; l < 8; l++) tsum = __fadd_rn(tsum, ap[l]);
      const float res = q4 ? __fadd_rn(ap[8], tsum) : tsum;
      W.out[(size_t)(a.out_col0 + m) * W.rows + row0 + rr] = res;
    }
    wave_lds_sync();
  }
}

static size_t matvec_lds_bytes(int cols, const TileGeom &g, int wpg) {
  size_t x = (size_t)cols * g.nb * kQ8BlockBytes + (size_t)((cols * g.nb + 3) & ~3) * 4;
  size_t per_wave = (size_t)(g.R * 9 * g.S + cols * g.R * 9) * 4;
  return x + per_wave * wpg;
}

template <int M>
static hipError_t launch_m(const MatvecArgs &a, int num_cus, hipStream_t s) {
  int wpg = a.total_tiles / (2 * num_cus);
  wpg = wpg < 1 ? 1 : wpg > 4 ? 4 : wpg;
  int grid = (a.total_tiles + wpg - 1) / wpg;
  const int cap = num_cus * 8;
  if (grid > cap) grid = cap;
  size_t lds = matvec_lds_bytes(M, a.g, wpg);
  hipLaunchKernelGGL(kquant_matvec_kernel<M>, dim3(grid), dim3(64 * wpg), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_matvec(const MatvecArgs &a, int num_cus, hipStream_t s) {
  switch (a.cols) {
    case 1: return launch_m<1>(a, num_cus, s);
    case 2: return launch_m<2>(a, num_cus, s);
    case 3: return launch_m<3>(a, num_cus, s);
    case 4: return launch_m<4>(a, num_cus, s);
    case 5: return launch_m<5>(a, num_cus, s);
    case 6: return launch_m<6>(a, num_cus, s);
    case 7: return launch_m<7>(a, num_cus, s);
    case 8: return launch_m<8>(a, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

TileGeom choose_geometry(int nb) {
  // Largest divisor S of nb (S <= 64) whose tile keeps >= 48 of 64 lanes busy.
  TileGeom g{nb, 1, 64, nb};
  for (int s = nb < 64 ? nb : 64; s >= 1; s--) {
    if (nb % s) continue;
    int r = 64 / s;
    if (r * s >= 48 || s == 1) {
      g.S = s;
      g.R = r;
      g.iters = nb / s;
      break;
    }
  }
  return g;
}

}  // namespace hp
