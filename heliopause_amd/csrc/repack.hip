// repack.hip -- one-time upload repack of GGUF super-blocks into the wave
// tile layout (hp_common.h), and the dequantisation test hook.
//
// The repack is a byte permutation of each block (plus Q6_K's d moved to a
// side plane and its high-bit fields stored as hi ^ 2); the byte count is
// unchanged.  Dequantisation follows packages/engine/wasm-kernels/src/lib.rs
// 1630-1664 (Q4_K: (d*sc)*q - (dmin*m)) and 1709-1744 (Q6_K: (d*sc)*(q-32)),
// f32 with no FMA, so it is bit-exact with the reference.
#include "hp_common.h"

namespace hp {

// Position of tile-order row-block `gidx` (0 .. rows*nb-1).
struct TilePos {
  int row, block, lane, lanes;
  size_t iter_base;  // byte offset of (tile, iteration) chunk 0, lane 0
};

__device__ __forceinline__ TilePos tile_pos(size_t gidx, int rows, const TileGeom g, int CH) {
  const size_t per_tile = (size_t)g.R * g.nb;
  const int t = (int)(gidx / per_tile);
  const int row0 = t * g.R;
  const int Rt = min(g.R, rows - row0);
  const size_t q = gidx - (size_t)t * per_tile;
  const int lanes = Rt * g.S;
  const int it = (int)(q / lanes);
  const int k = (int)(q - (size_t)it * lanes);
  TilePos p;
  p.row = row0 + k / g.S;
  p.block = it * g.S + k % g.S;
  p.lane = k;
  p.lanes = lanes;
  p.iter_base = ((size_t)row0 * g.nb * CH + (size_t)it * CH * lanes) * 16;
  return p;
}

__global__ void repack_q4k_kernel(const uint8_t *__restrict__ raw, int rows, TileGeom g, uint8_t *__restrict__ out) {
  const size_t gidx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gidx >= (size_t)rows * g.nb) return;
  const TilePos p = tile_pos(gidx, rows, g, 9);
  const uint8_t *src = raw + ((size_t)p.row * g.nb + p.block) * 144;  // 16-byte aligned
  const uint4 *s16 = reinterpret_cast<const uint4 *>(src);
  uint4 *dst = reinterpret_cast<uint4 *>(out + p.iter_base) + p.lane;
  dst[0] = s16[0];
  uint8_t qs[128];
#pragma unroll
  for (int i = 0; i < 8; i++) *reinterpret_cast<uint4 *>(qs + 16 * i) = s16[1 + i];
#pragma unroll
  for (int ck = 0; ck < 8; ck++) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int dw = 4 * ck + e, pp = dw >> 3, l = dw & 7;
      w[e] = (uint32_t)qs[32 * pp + l] | ((uint32_t)qs[32 * pp + 8 + l] << 8) |
             ((uint32_t)qs[32 * pp + 16 + l] << 16) | ((uint32_t)qs[32 * pp + 24 + l] << 24);
    }
    dst[(size_t)(1 + ck) * p.lanes] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// f16_flag: set to 1 when some sub-block scale s is odd with |s| >= 67.  The
// matrix-core kernels take sc * (q - 32) as an f16 operand; with |q - 32| <=
// 32 that product is odd and above 2048 in magnitude (so not exact in f16)
// only for such scales (67 * 31 = 2077; 65 * 31 = 2015; even scales give even
// products of at most 4096).
__global__ void repack_q6k_kernel(const uint8_t *__restrict__ raw, int rows, TileGeom g, uint8_t *__restrict__ out,
                                  uint16_t *__restrict__ dplane, uint32_t *__restrict__ f16_flag) {
  const size_t gidx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gidx >= (size_t)rows * g.nb) return;
  const TilePos p = tile_pos(gidx, rows, g, 13);
  const uint8_t *src = raw + ((size_t)p.row * g.nb + p.block) * 210;  // 2-byte aligned
  uint8_t b[210];
  const uint16_t *s2 = reinterpret_cast<const uint16_t *>(src);
#pragma unroll
  for (int i = 0; i < 105; i++) {
    const uint16_t v = s2[i];
    b[2 * i] = (uint8_t)v;
    b[2 * i + 1] = (uint8_t)(v >> 8);
  }
  const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
  uint4 *dst = reinterpret_cast<uint4 *>(out + p.iter_base) + p.lane;
  // chunks 0..7: Dql[pp][l], byte c = nib(2pp, c, l) | nib(2pp+1, c, l) << 4
  // element (j, c, l): h = j/4, t = j%4, ql byte = 64h + 8c + l + 32(t&1), nibble t>>1
#pragma unroll
  for (int ck = 0; ck < 8; ck++) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int dw = 4 * ck + e, pp = dw >> 3, l = dw & 7;
      const int h = pp >> 1, sh = 4 * (pp & 1);
      uint32_t v = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const uint32_t lo = (ql[64 * h + 8 * c + l] >> sh) & 15;       // j = 2pp   (t even)
        const uint32_t hi = (ql[64 * h + 32 + 8 * c + l] >> sh) & 15;  // j = 2pp+1 (t odd)
        v |= (lo | (hi << 4)) << (8 * c);
      }
      w[e] = v;
    }
    dst[(size_t)ck * p.lanes] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  // chunks 8..11: Dqh[q][l], byte c = qh[32q + 8c + l] ^ 0xAA
#pragma unroll
  for (int ck = 0; ck < 4; ck++) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int dw = 4 * ck + e, q = dw >> 3, l = dw & 7;
      uint32_t v = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) v |= (uint32_t)(qh[32 * q + 8 * c + l] ^ 0xAA) << (8 * c);
      w[e] = v;
    }
    dst[(size_t)(8 + ck) * p.lanes] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  uint32_t s[4];
#pragma unroll
  for (int e = 0; e < 4; e++)
    s[e] = (uint32_t)sc[4 * e] | ((uint32_t)sc[4 * e + 1] << 8) | ((uint32_t)sc[4 * e + 2] << 16) |
           ((uint32_t)sc[4 * e + 3] << 24);
  dst[(size_t)12 * p.lanes] = make_uint4(s[0], s[1], s[2], s[3]);
  dplane[gidx] = (uint16_t)(b[208] | (b[209] << 8));
  bool wide_product = false;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int v = (int)(int8_t)sc[i];
    wide_product |= (v & 1) && (v >= 67 || v <= -67);
  }
  if (wide_product) *f16_flag = 1u;
}

__device__ __forceinline__ float h2f_r(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// One thread per (row, block) of [row_start, row_start+row_count).
__global__ void dequant_kernel(int type, const uint8_t *__restrict__ tiles, const uint16_t *__restrict__ dplane,
                               int rows, TileGeom g, int row_start, int row_count, float *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)row_count * g.nb) return;
  const int row = row_start + (int)(i / g.nb);
  const int block = (int)(i % g.nb);
  const int t = row / g.R;
  const int row0 = t * g.R;
  const int Rt = min(g.R, rows - row0);
  const int lanes = Rt * g.S;
  const int it = block / g.S;
  const int k = (row - row0) * g.S + block % g.S;
  const int CH = type == kTypeQ4K ? 9 : 13;
  const uint4 *ch = reinterpret_cast<const uint4 *>(tiles + ((size_t)row0 * g.nb * CH + (size_t)it * CH * lanes) * 16) + k;
  float *o = out + (size_t)(row - row_start) * g.nb * kQK + (size_t)block * kQK;
  if (type == kTypeQ4K) {
    const uint4 c0 = ch[0];
    const float d = h2f_r(c0.x & 0xFFFFu), dmin = h2f_r(c0.x >> 16);
    const uint32_t s0 = c0.y, s1 = c0.z, s2 = c0.w;
    for (int j = 0; j < 8; j++) {
      int sc, mn;
      if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        mn = (s1 >> (8 * j)) & 63;
      } else {
        sc = ((s2 >> (8 * (j - 4))) & 15) | (((s0 >> (8 * (j - 4) + 6)) & 3) << 4);
        mn = ((s2 >> (8 * (j - 4) + 4)) & 15) | (((s1 >> (8 * (j - 4) + 6)) & 3) << 4);
      }
      const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
      const int pp = j >> 1, sh = 4 * (j & 1);
      for (int c = 0; c < 4; c++)
        for (int l = 0; l < 8; l++) {
          const int dw = 8 * pp + l;
          const uint4 v = ch[(size_t)(1 + (dw >> 2)) * lanes];
          const uint32_t word = (dw & 3) == 0 ? v.x : (dw & 3) == 1 ? v.y : (dw & 3) == 2 ? v.z : v.w;
          const int q = (word >> (8 * c + sh)) & 15;
          o[32 * j + 8 * c + l] = __fsub_rn(__fmul_rn(d1, (float)q), m1);
        }
    }
  } else {
    const float d = h2f_r(dplane[(size_t)row0 * g.nb + (size_t)it * lanes + k]);
    const uint4 csc = ch[(size_t)12 * lanes];
    for (int j = 0; j < 8; j++) {
      for (int l = 0; l < 8; l++) {
        const int dq = 8 * (j >> 1) + l, dh = 8 * (j >> 2) + l;
        const uint4 vq = ch[(size_t)(dq >> 2) * lanes];
        const uint4 vh = ch[(size_t)(8 + (dh >> 2)) * lanes];
        const uint32_t ql = (dq & 3) == 0 ? vq.x : (dq & 3) == 1 ? vq.y : (dq & 3) == 2 ? vq.z : vq.w;
        const uint32_t qh = (dh & 3) == 0 ? vh.x : (dh & 3) == 1 ? vh.y : (dh & 3) == 2 ? vh.z : vh.w;
        for (int c = 0; c < 4; c++) {
          const int nib = (ql >> (8 * c + 4 * (j & 1))) & 15;
          const int fld = (qh >> (8 * c + 2 * (j & 3))) & 3;  // stored as hi ^ 2
          const int q = (int)(int8_t)(uint8_t)((nib | (fld << 4)) << 2) >> 2;  // q6 - 32
          const int gidx = 2 * j + (c >> 1);
          const uint32_t sw = gidx < 4 ? csc.x : gidx < 8 ? csc.y : gidx < 12 ? csc.z : csc.w;
          const int sc = (int)(int8_t)(sw >> (8 * (gidx & 3)));
          o[32 * j + 8 * c + l] = __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
        }
      }
    }
  }
}

hipError_t launch_repack(int type, const uint8_t *raw, int rows, const TileGeom &g, uint8_t *tiles, uint16_t *dplane,
                         uint32_t *f16_flag, hipStream_t s) {
  const size_t n = (size_t)rows * g.nb;
  const int tpb = 128;
  const int blocks = (int)((n + tpb - 1) / tpb);
  if (type == kTypeQ4K)
    hipLaunchKernelGGL(repack_q4k_kernel, dim3(blocks), dim3(tpb), 0, s, raw, rows, g, tiles);
  else
    hipLaunchKernelGGL(repack_q6k_kernel, dim3(blocks), dim3(tpb), 0, s, raw, rows, g, tiles, dplane, f16_flag);
  return hipGetLastError();
}

hipError_t launch_dequantize(int type, const uint8_t *tiles, const uint16_t *dplane, int rows, const TileGeom &g,
                             int row_start, int row_count, float *out, hipStream_t s) {
  const size_t n = (size_t)row_count * g.nb;
  const int tpb = 128;
  const int blocks = (int)((n + tpb - 1) / tpb);
  hipLaunchKernelGGL(dequant_kernel, dim3(blocks), dim3(tpb), 0, s, type, tiles, dplane, rows, g, row_start,
                     row_count, out);
  return hipGetLastError();
}

}  // namespace hp
