// kquant_mfma.hip -- Q4_K / Q6_K x Q8_K matvec on the gfx950 matrix cores,
// bit-exact with the reference's WASM path (the numerics are those of
// kquant_matvec.hip: packages/engine/wasm-kernels/src/lib.rs:2116-2172,
// 1923-1968, 300-426).
//
// Why matrix cores for a bandwidth-bound matvec: exact parity needs, per
// (row, block, column), the eight integers aux32[l] = sum_g sc_g *
// sum_{e in g, e = l mod 8} q_e * q8_e.  On the vector ALU that is a dot4 and
// a multiply-add per four weights per column, so columns multiply the ALU
// work.  Here the scales are folded into the weights: A = sc_g * q_e (Q4_K
// <= 945, Q6_K |.| <= 1024) and B = q8 (|.| <= 128) are exact in f16, every
// product and partial sum is an integer below 2^24 (|aux32| <= 4,194,304),
// so v_mfma_f32_16x16x32_f16 accumulates them exactly in f32 and f32(aux32)
// is the reference's value.  The vector ALU only unpacks the weights, once
// for all columns.
//
// Lanes (v_mfma_f32_16x16x32_f16): A lane i = (row i%16, quarter q = i/16)
// holds k = 8q..8q+7; B lane i = (column n = i%16, quarter q) the same k;
// D lane i holds rows 4(i/16)+j (j = 0..3) of column n.
// Columns n = m + 4s: m = input column of the set (4 per set), s = class
// slot.  MFMA (g, u), g in {0,1}, u in {0..3}: quarter q carries lane class
// l = 2q + g, elements (j = 2u, c = 0..3) then (j = 2u+1, c = 0..3) with
// e = 32j + 8c + l; B is x_m of the same elements when q == s, else zero.
// So D(g) of lane (rows, n) accumulates aux32 of class 2s + g: every
// (row, column, class) chain lives in one lane, and the f32 tail runs in
// registers in block order:
//   d = dW_b * dX_b; sums[l] += d * f32(aux32[l]);
//   Q4_K: sumf -= (dminW_b * dX_b) * f32(sumi)   (sumi by one more MFMA:
//         mins x half-block sums of q8)
//   result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
//
// Weights come from one of two places per weight.  The matrix-core segments
// (a second copy, repacked at upload, same byte count per 16-row tile; rows
// past the weight in the last tile are zero): segment (tile T, block b) at
// (b * tiles + T) * SEG, block-major, so the waves that stream block b of
// neighbouring tiles at the same time read one contiguous range.
//   Q4_K, SEG = 2304: [0,256) the 16 rows' first 16 GGUF bytes (d, dmin,
//     packed scales/mins); [256,2304) chunk c in {0,1} x lane i: dword u of
//     class 2q + c holds in byte cc: q(2u, cc) | q(2u+1, cc) << 4.
//   Q6_K, SEG = 3360: [0,256) 16 rows x 16 int8 scales; [256,288) 16 f16 d;
//     [288,3360) chunks 0,1 as Q4_K with the low 4 bits of q6; chunk 2
//     dword 2*cls + h holds in byte cc the high 2 bits of q6 at
//     (j = 4h + jj, cc, class 2q + cls) in bits 2jj.
// Or, for a weight uploaded with one layout only (hp_hip_set_weight_layouts),
// the vector-ALU tile layout (hp_common.h), read a row at a time (tile_row).
// Lane i = (row rho = i%16 of the 16-row segment, quarter q) needs the
// dwords D[u][l] (u = 0..3) of classes l = 2q and 2q + 1: they are the
// 8-byte pair at byte 8(q%2) of quant chunk 2u + q/2 of its row-block, four
// 8-byte loads.  Q4_K: chunk 0 (header), quant chunks 1..8.  Q6_K: low-bit
// chunks 0..7 the same way; high-bit dwords Dqh[h][l] (h = 0, 1) the pair at
// byte 8(q%2) of chunk 8 + 2h + q/2, stored ^ 0xAA per byte; the 16 scales
// are chunk 12; d from the d plane.  Rows past the weight in the last
// segment re-read its last row (their sums are never stored).  These loads
// touch a cache line per lane (a row's blocks are interleaved in the tile
// layout), against one line per 8 lanes in the segments.
#include "hp_common.h"
#include "hp_mfma.h"

namespace hp {

namespace {

struct MfmaWeight {
  const uint8_t *seg;       // segments of this weight (null: kept in one layout)
  const uint8_t *wt;        // tiles of this weight
  const uint16_t *dplane;   // Q6_K d plane
  float *out;
  int type, rows, tiles, tile_begin;  // tiles: 16-row segments
};

struct MfmaArgs {
  MfmaWeight w[kMaxWeights];
  int count;
  int total_tiles;
  int nb, S, R;     // tile geometry of the launch's weights
  const float *x;  // f32 input of the launch's first column, [cols][k]
  int k;
  int cols;        // columns of this launch (<= 8)
  int out_col0;
};

// LDS layout: xh [nb][M4] regions of kXRegion bytes, each 8 classes of
// kXClass bytes (32 f16 + 16 bytes of padding); bs16 [nb][M4][16] f16;
// dx [nb][M4] f32; 16 zero bytes; per wave fin [16 rows][16 n][2] f32 and
// finf [16 rows][4] f32.  The padding makes the 16 B-operand reads of one
// MFMA (4 columns x 4 class slots, 16 bytes each) use every 16-byte bank
// slot exactly twice: slot = (2s + g) * 5 + m (mod 8).
struct Lds {
  _Float16 *xh, *bs;
  float *dx;
  uint8_t *zero;
  float *fin, *finf;
};

constexpr int kFinFloats = 16 * 16 * 2 + 16 * 4;
constexpr int kXClass = 80;              // bytes per class: 64 + 16 padding
constexpr int kXRegion = 8 * kXClass + 16;  // bytes per (block, column): 656 = 16 mod 128

__device__ __forceinline__ Lds lds_layout(uint8_t *smem, int m4, int nb, int wave) {
  Lds L;
  L.xh = reinterpret_cast<_Float16 *>(smem);
  L.bs = reinterpret_cast<_Float16 *>(smem + (size_t)m4 * nb * kXRegion);
  L.dx = reinterpret_cast<float *>(L.bs + (size_t)m4 * nb * 16);  // bs16: 32 bytes per (b, m)
  L.zero = reinterpret_cast<uint8_t *>(L.dx + (size_t)m4 * nb);
  L.fin = reinterpret_cast<float *>(L.zero + 16) + (size_t)wave * kFinFloats;
  L.finf = L.fin + 16 * 16 * 2;
  return L;
}

// Q8_K of block (m, b) by one 16-lane DPP row (lib.rs:1774-1811), written as
// f16 for the B operand.  Lane i16 = 2j + u owns elements 32j + 8c + 4u + i
// (c, i = 0..3): class l = 4u + i, t = 4j + c, stored at xh[m][b][l][t].
template <int CTRL>
__device__ __forceinline__ float dppf_(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi_(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ void lexmax_(float &amax, float &vmax, int &idx) {
  const float oa = dppf_<CTRL>(amax);
  const float ov = dppf_<CTRL>(vmax);
  const int oi = dppi_<CTRL>(idx);
  const bool take = oa > amax || (oa == amax && oi < idx);
  amax = take ? oa : amax;
  vmax = take ? ov : vmax;
  idx = take ? oi : idx;
}

// f16 x of class l of (block b, column m); element t at +t.
__device__ __forceinline__ _Float16 *x_class(const Lds &L, int m4, int b, int m, int l) {
  return reinterpret_cast<_Float16 *>(reinterpret_cast<uint8_t *>(L.xh) + ((size_t)b * m4 + m) * kXRegion +
                                      l * kXClass);
}

__device__ __forceinline__ void load_x16_(float (&v)[16], const float *__restrict__ xb, int i16) {
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

__device__ __forceinline__ void q8k_block16_f16(const float (&v)[16], int i16, const Lds &L, int m4, int m, int b) {
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
  lexmax_<0xB1>(amax, vmax, idx);   // quad_perm [1,0,3,2]
  lexmax_<0x4E>(amax, vmax, idx);   // quad_perm [2,3,0,1]
  lexmax_<0x141>(amax, vmax, idx);  // row_half_mirror
  lexmax_<0x140>(amax, vmax, idx);  // row_mirror
  const bool nz = amax != 0.0f;
  const float inv = __fdiv_rn(-127.0f, vmax);
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    half2v p0, p1;
    int qv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      // Rust: (is * x).round().min(127.0) as i8 (saturating)
      const float r = fmaxf(fminf(roundf(__fmul_rn(inv, v[4 * c + i])), 127.0f), -128.0f);
      qv[c] = nz ? (int)r : 0;
      sum += qv[c];
    }
    p0 = (half2v){(_Float16)qv[0], (_Float16)qv[1]};
    p1 = (half2v){(_Float16)qv[2], (_Float16)qv[3]};
    const int l = 4 * u + i;
    *reinterpret_cast<uint2 *>(x_class(L, m4, b, m, l) + 4 * j) = make_uint2(as_u32(p0), as_u32(p1));
  }
  L.bs[((size_t)b * m4 + m) * 16 + i16] = (_Float16)sum;  // |sum| <= 2048: exact
  if (i16 == 0) L.dx[(size_t)b * m4 + m] = nz ? __fdiv_rn(1.0f, inv) : 0.0f;
}

__device__ __forceinline__ half8 lds_h8(const void *p) {
  return __builtin_bit_cast(half8, *reinterpret_cast<const uint4 *>(p));
}

// Raw loads of one (segment, block) for lane i (per weight type, so a Q4_K
// segment carries only its 12 registers).  c0 / c1: dwords D[u][2q] /
// D[u][2q + 1], u = 0..3.
template <bool Q4>
struct Seg;
template <>
struct Seg<true> {
  uint4 hdr;  // row header: d | dmin, 12 packed scale/min bytes
  uint4 c0, c1;
};
template <>
struct Seg<false> {
  uint4 hdr;  // 16 int8 scales of row i%16
  uint4 c0, c1, c2;  // c2: high-bit dwords Dqh[h][2q + cls] at 2h + cls (tiles: ^ 0xAA per byte)
  uint32_t d;  // f16 d of row i%16
};

// Lane offsets of one row for load_tiles: the row's place, and the byte of its
// first 8-byte quant pair within a row-block.
struct RowLoads {
  TileRow tr;
  uint32_t oq;  // Q4_K: chunk 1 + q/2, Q6_K: chunk q/2; + 8 (q%2)
};

__device__ __forceinline__ RowLoads row_loads(int row, int rows, int nb, int S, int R, bool q4, int q) {
  RowLoads r;
  r.tr = tile_row(row, rows, nb, S, R, q4 ? 9 : 13);
  r.oq = (uint32_t)((q4 ? 1 : 0) + (q >> 1)) * r.tr.chunk + 8u * (uint32_t)(q & 1);
  return r;
}

// One (tile, block) segment for lane i.
template <bool Q4>
__device__ __forceinline__ Seg<Q4> load_seg(const uint8_t *seg, int lane) {
  const int rho = lane & 15;
  Seg<Q4> r;
  r.hdr = *reinterpret_cast<const uint4 *>(seg + 16 * rho);
  if constexpr (Q4) {
    r.c0 = *reinterpret_cast<const uint4 *>(seg + 256 + 16 * lane);
    r.c1 = *reinterpret_cast<const uint4 *>(seg + 256 + 1024 + 16 * lane);
  } else {
    r.d = *reinterpret_cast<const uint16_t *>(seg + 256 + 2 * rho);
    r.c0 = *reinterpret_cast<const uint4 *>(seg + 288 + 16 * lane);
    r.c1 = *reinterpret_cast<const uint4 *>(seg + 288 + 1024 + 16 * lane);
    r.c2 = *reinterpret_cast<const uint4 *>(seg + 288 + 2048 + 16 * lane);
  }
  return r;
}

// The same registers from the weight's tiles (c2 as the tiles store it).
template <bool Q4>
__device__ __forceinline__ Seg<Q4> load_tiles(const uint8_t *wt, const uint16_t *dplane, const RowLoads &rl, int b,
                                              int S) {
  int i, s;
  block_split(b, S, i, s);
  const uint32_t off = rl.tr.base + (uint32_t)i * rl.tr.iter + 16u * (uint32_t)s;
  const uint32_t ch = rl.tr.chunk;
  auto ld8 = [&](uint32_t o) { return *reinterpret_cast<const uint2 *>(wt + o); };
  Seg<Q4> r;
  uint2 p[4];
#pragma unroll
  for (int u = 0; u < 4; u++) p[u] = ld8(off + rl.oq + 2u * (uint32_t)u * ch);
  r.c0 = make_uint4(p[0].x, p[1].x, p[2].x, p[3].x);
  r.c1 = make_uint4(p[0].y, p[1].y, p[2].y, p[3].y);
  if constexpr (Q4) {
    r.hdr = *reinterpret_cast<const uint4 *>(wt + off);
  } else {
    r.hdr = *reinterpret_cast<const uint4 *>(wt + off + 12u * ch);
    r.d = dplane[rl.tr.dbase + (uint32_t)i * rl.tr.diter + (uint32_t)s];
    const uint2 h0 = ld8(off + rl.oq + 8u * ch), h1 = ld8(off + rl.oq + 10u * ch);
    r.c2 = make_uint4(h0.x, h0.y, h1.x, h1.y);
  }
  return r;
}

struct Chains {
  float s[2][4];  // class 2s+g chains of rows 4(i/16)+j
  float f[4];     // Q4_K sumf of rows 4(i/16)+j (valid in lanes n < 4)
};

// A operand of MFMA (g, u): quarter q's class 2q + g, elements (j = 2u,
// c = 0..3) then (j = 2u+1, c = 0..3), each sc_j * q as exact f16.
__device__ __forceinline__ half8 a_q4k(const Seg<true> &r, int g, int u, const half2v (&S)[8],
                                       const half2v (&N)[8]) {
  const uint32_t dw = u4at(g ? r.c1 : r.c0, u);
  const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
  return cat(fma2(magic_pair<kSel01>(lo), S[2 * u], N[2 * u]), fma2(magic_pair<kSel23>(lo), S[2 * u], N[2 * u]),
             fma2(magic_pair<kSel01>(hi), S[2 * u + 1], N[2 * u + 1]),
             fma2(magic_pair<kSel23>(hi), S[2 * u + 1], N[2 * u + 1]));
}

// Q6_K: groups 4u, 4u+1 (j = 2u; c = 0,1 | c = 2,3) and 4u+2, 4u+3 (j = 2u+1);
// the weights are sc_g * (q6 - 32).
template <bool TILE>
__device__ __forceinline__ half8 a_q6k(const Seg<false> &r, int g, int u, const half2v (&S)[4],
                                       const half2v (&N)[4]) {
  const int jj = 2 * (u & 1);
  const uint32_t ql = u4at(g ? r.c1 : r.c0, u);
  // the tiles store the fields as hi ^ 2
  const uint32_t qh = u4at(r.c2, 2 * (u >> 1) + g) ^ (TILE ? 0xAAAAAAAAu : 0u);
  const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * jj)) & 0x03030303u) << 4);
  const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * jj + 2)) & 0x03030303u) << 4);
  return cat(fma2(magic_pair<kSel01>(lo), S[0], N[0]), fma2(magic_pair<kSel23>(lo), S[1], N[1]),
             fma2(magic_pair<kSel01>(hi), S[2], N[2]), fma2(magic_pair<kSel23>(hi), S[3], N[3]));
}

// One block of a tile for every column set: A operands are built one at a
// time right before their MFMAs; then the f32 tail in block order.
template <int NSET, bool Q4, bool TILE>
__device__ __forceinline__ void process_block(Chains (&ch)[NSET], const Seg<Q4> &r, const Lds &L, int b, int nb,
                                              int lane) {
  const int n = lane & 15, q = lane >> 4;
  const int s = n >> 2;
  // B operand addresses (x of class 2q + g when q == s, else the zero bytes)
  const _Float16 *xq[NSET];  // class 2q of (b, column 4st + n%4); class 2q+1 is kXClass further
#pragma unroll
  for (int st = 0; st < NSET; st++) xq[st] = x_class(L, 4 * NSET, b, 4 * st + (n & 3), 2 * q);
  f32x4 acc[NSET][2];
#pragma unroll
  for (int st = 0; st < NSET; st++) acc[st][0] = acc[st][1] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  float dw[4], dmw[4];
  const int src = ((lane >> 4) * 4) << 2;  // lane index = row of the D layout's row 4(i/16)
  if constexpr (Q4) {
    const uint32_t s0 = r.hdr.y, s2 = r.hdr.w;
    // scale bytes sc0..3 | sc4..7 (6-bit, one per byte)
    const uint32_t sclo = s0 & 0x3F3F3F3Fu;
    const uint32_t schi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    half2v S[8], N[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      S[j] = dup_byte(j < 4 ? sclo : schi, j & 3, 1024.0f);  // (sc_j, sc_j)
      N[j] = S[j] * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
    }
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const half8 a = a_q4k(r, g, u, S, N);
#pragma unroll
        for (int st = 0; st < NSET; st++) {
          const half8 bf = lds_h8(q == s ? (const void *)(xq[st] + g * (kXClass / 2) + 8 * u) : (const void *)L.zero);
          acc[st][g] = mfma(a, bf, acc[st][g]);
        }
      }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t v = (uint32_t)__builtin_amdgcn_ds_bpermute(src + 4 * j, (int)r.hdr.x);
      dw[j] = h2f_bits(v & 0xFFFFu);
      dmw[j] = h2f_bits(v >> 16);
    }
  } else {
    // signed scales: bytes ^ 0x80 are s + 128; (1024 + 128 + s) - 1152 = s
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t gs = u4at(r.hdr, u) ^ 0x80808080u;
      half2v S[4], N[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        S[e] = dup_byte(gs, e, 1152.0f);
        N[e] = S[e] * (half2v){(_Float16)-1056.0f, (_Float16)-1056.0f};  // -(1024 + 32) * sc
      }
#pragma unroll
      for (int g = 0; g < 2; g++) {
        const half8 a = a_q6k<TILE>(r, g, u, S, N);
#pragma unroll
        for (int st = 0; st < NSET; st++) {
          const half8 bf = lds_h8(q == s ? (const void *)(xq[st] + g * (kXClass / 2) + 8 * u) : (const void *)L.zero);
          acc[st][g] = mfma(a, bf, acc[st][g]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t v = (uint32_t)__builtin_amdgcn_ds_bpermute(src + 4 * j, (int)r.d);
      dw[j] = h2f_bits(v & 0xFFFFu);
      dmw[j] = 0.0f;
    }
  }
#pragma unroll
  for (int st = 0; st < NSET; st++) {
    const int m = 4 * st + (n & 3);
    const float dx = L.dx[(size_t)b * 4 * NSET + m];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float dd = __fmul_rn(dw[j], dx);
#pragma unroll
      for (int g = 0; g < 2; g++) ch[st].s[g][j] = __fadd_rn(ch[st].s[g][j], __fmul_rn(dd, acc[st][g][j]));
    }
  }
  if constexpr (Q4) {
    // mins: quarter q < 2 carries k = 8q + e -> (j = 4q + e/2, half e%2)
    const uint32_t s1 = r.hdr.z, s2 = r.hdr.w;
    const uint32_t mn = q == 0 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
    const half8 am = q < 2 ? cat(dup_byte(mn, 0, 1024.0f), dup_byte(mn, 1, 1024.0f), dup_byte(mn, 2, 1024.0f),
                                 dup_byte(mn, 3, 1024.0f))
                           : (half8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < NSET; st++) {
      const int m = 4 * st + (n & 3);
      const half8 bm = lds_h8(q < 2 && s == 0 ? (const void *)(L.bs + ((size_t)b * 4 * NSET + m) * 16 + 8 * q)
                                              : (const void *)L.zero);
      const f32x4 sm = mfma(am, bm, (f32x4){0.0f, 0.0f, 0.0f, 0.0f});
      const float dx = L.dx[(size_t)b * 4 * NSET + m];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float dm = __fmul_rn(dmw[j], dx);
        ch[st].f[j] = __fsub_rn(ch[st].f[j], __fmul_rn(dm, sm[j]));
      }
    }
  }
}

// All blocks of one tile, in order; three register buffers keep the loads of
// the next two blocks in flight while a block computes.
template <int NSET, bool Q4, bool TILE>
__device__ __forceinline__ void run_tile(Chains (&ch)[NSET], const MfmaWeight &W, int tt, const RowLoads &rl, int S,
                                         const Lds &L, int nb, int lane) {
  // every load unconditional (a block index past the last re-reads it): a
  // path that skipped a load would turn the wait for one block into a wait
  // for the blocks loaded after it
  const int segb = Q4 ? 2304 : 3360;
  auto ld = [&](int b) {
    if constexpr (TILE)
      return load_tiles<Q4>(W.wt, W.dplane, rl, min(b, nb - 1), S);
    else
      return load_seg<Q4>(W.seg + ((size_t)min(b, nb - 1) * W.tiles + tt) * segb, lane);
  };
  Seg<Q4> r0 = ld(0), r1 = ld(1), r2;
  for (int b = 0; b < nb; b += 3) {
    r2 = ld(b + 2);
    process_block<NSET, Q4, TILE>(ch, r0, L, b, nb, lane);
    r0 = ld(b + 3);
    if (b + 1 < nb) process_block<NSET, Q4, TILE>(ch, r1, L, b + 1, nb, lane);
    r1 = ld(b + 4);
    if (b + 2 < nb) process_block<NSET, Q4, TILE>(ch, r2, L, b + 2, nb, lane);
  }
}

// result(row, m) = [sumf +] ((((-0 + s0) + s1) + ...) + s7); chains of class
// l = 2s + g of (row 4G + j, m) sit in lane 16G + m + 4s, group g, register j.
template <int NSET>
__device__ __forceinline__ void finish_tile(const Chains (&ch)[NSET], const Lds &L, int lane, bool q4,
                                            float *out, int rows, int row0, int out_col0, int cols) {
  const int n = lane & 15, G = lane >> 4;
#pragma unroll
  for (int st = 0; st < NSET; st++) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      L.fin[((4 * G + j) * 16 + n) * 2 + 0] = ch[st].s[0][j];
      L.fin[((4 * G + j) * 16 + n) * 2 + 1] = ch[st].s[1][j];
      if (n < 4) L.finf[(4 * G + j) * 4 + n] = ch[st].f[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int rho = lane >> 2, m4 = lane & 3;
    float tot = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) tot = __fadd_rn(tot, L.fin[(rho * 16 + m4 + 4 * (l >> 1)) * 2 + (l & 1)]);
    if (q4) tot = __fadd_rn(L.finf[rho * 4 + m4], tot);
    const int m = 4 * st + m4;
    if (row0 + rho < rows && m < cols) out[(size_t)(out_col0 + m) * rows + row0 + rho] = tot;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// TILE: every weight is read from its tiles (a launch with a weight kept in
// one layout); else from its segments.
template <int NSET, bool TILE>
__global__ __launch_bounds__(256) void kquant_mfma_kernel(const MfmaArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int nb = a.nb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const Lds L = lds_layout(smem, 4 * NSET, nb, wave);

  // prologue: Q8_K of the launch's columns (f16 B layout), 16 lanes per
  // block; columns past `cols` are zero
  const int grp = wave * 4 + (lane >> 4), i16 = lane & 15;
  const int nq = 4 * NSET * nb;
  if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(L.zero)[threadIdx.x] = 0;
  // the inputs of the first three passes load together, before any pass
  // (a block past the last, or of a column past `cols`, re-reads a valid one
  // and is not used)
  auto x_of = [&](int qb) {
    const int qc = min(qb, nq - 1), m = qc / nb, b = qc - m * nb;
    return a.x + (size_t)min(m, a.cols - 1) * a.k + (size_t)b * kQK;
  };
  float xp[3][16];
#pragma unroll
  for (int p = 0; p < 3; p++) load_x16_(xp[p], x_of(grp + 16 * p), i16);
  __builtin_amdgcn_sched_barrier(0);
  for (int qb = grp, p = 0; qb < nq; qb += 16, p++) {
    const int m = qb / nb, b = qb - m * nb;
    if (m < a.cols) {
      float xv[16];
      if (p < 3) {
#pragma unroll
        for (int i = 0; i < 16; i++) xv[i] = p == 0 ? xp[0][i] : p == 1 ? xp[1][i] : xp[2][i];
      } else {
        load_x16_(xv, a.x + (size_t)m * a.k + (size_t)b * kQK, i16);
      }
      q8k_block16_f16(xv, i16, L, 4 * NSET, m, b);
    } else {
      // 16 lanes clear the region's 8 classes of 64 data bytes
      _Float16 *xc = x_class(L, 4 * NSET, b, m, i16 >> 1) + 16 * (i16 & 1);
      *reinterpret_cast<uint4 *>(xc) = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4 *>(xc + 8) = make_uint4(0, 0, 0, 0);
      L.bs[((size_t)b * 4 * NSET + m) * 16 + i16] = (_Float16)0.0f;
      if (i16 == 0) L.dx[(size_t)b * 4 * NSET + m] = 0.0f;
    }
  }
  __syncthreads();

  const int stride = gridDim.x * 4;
  for (int t = blockIdx.x * 4 + wave; t < a.total_tiles; t += stride) {
    MfmaWeight W = a.w[0];
    if (a.count > 1 && t >= a.w[1].tile_begin) W = a.w[1];
    if (a.count > 2 && t >= a.w[2].tile_begin) W = a.w[2];
    if (a.count > 3 && t >= a.w[3].tile_begin) W = a.w[3];
    const bool q4 = W.type == kTypeQ4K;
    const int tt = t - W.tile_begin;
    const RowLoads rl =
        TILE ? row_loads(min(16 * tt + (lane & 15), W.rows - 1), W.rows, nb, a.S, a.R, q4, lane >> 4) : RowLoads{};
    Chains ch[NSET];
#pragma unroll
    for (int st = 0; st < NSET; st++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        ch[st].s[0][j] = 0.0f;
        ch[st].s[1][j] = 0.0f;
        ch[st].f[j] = 0.0f;
      }
    if (q4)
      run_tile<NSET, true, TILE>(ch, W, tt, rl, a.S, L, nb, lane);
    else
      run_tile<NSET, false, TILE>(ch, W, tt, rl, a.S, L, nb, lane);
    finish_tile<NSET>(ch, L, lane, q4, W.out, W.rows, 16 * tt, a.out_col0, a.cols);
  }
}

// One thread per (tile, block, row-in-tile), the row fastest: the 16 lanes of
// one (tile, block) write whole 256-byte runs of its segment.  Each thread
// loads its GGUF block once with vector loads, then builds every output word
// from registers (zeros for rows past the weight).
__global__ void repack_mfma_kernel(const uint8_t *__restrict__ raw, int type, int rows, int nb,
                                   uint8_t *__restrict__ segs) {
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int tiles = (rows + 15) / 16;
  if (tid >= (long long)tiles * 16 * nb) return;
  const int rho = (int)(tid & 15);
  const int b = (int)((tid >> 4) % nb);
  const int T = (int)((tid >> 4) / nb);
  const int r = T * 16 + rho;
  const bool live = r < rows;
  if (type == kTypeQ4K) {
    uint8_t *seg = segs + ((size_t)b * tiles + T) * 2304;
    uint32_t w[36];  // the 144-byte block as 36 little-endian words
    const uint4 *src = reinterpret_cast<const uint4 *>(raw + ((size_t)(live ? r : 0) * nb + b) * 144);
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const uint4 v = live ? src[i] : make_uint4(0, 0, 0, 0);
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
    auto byte = [&](int o) -> uint32_t { return (w[o >> 2] >> (8 * (o & 3))) & 0xFFu; };
    reinterpret_cast<uint4 *>(seg)[rho] = make_uint4(w[0], w[1], w[2], w[3]);
    // lane (c, i = 16qq + rho), element class l = 2qq + c: byte 4u + cc =
    // block byte 16 + 32u + 8cc + l (nibbles of j = 2u, 2u + 1)
#pragma unroll
    for (int qq = 0; qq < 4; qq++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int l = 2 * qq + c;
        uint32_t o[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
          o[u] = byte(16 + 32 * u + l) | (byte(16 + 32 * u + 8 + l) << 8) | (byte(16 + 32 * u + 16 + l) << 16) |
                 (byte(16 + 32 * u + 24 + l) << 24);
        reinterpret_cast<uint4 *>(seg + 256)[c * 64 + qq * 16 + rho] = make_uint4(o[0], o[1], o[2], o[3]);
      }
  } else {
    uint8_t *seg = segs + ((size_t)b * tiles + T) * 3360;
    uint32_t h[105];  // the 210-byte block as 105 little-endian half-words (2-byte aligned)
    const uint16_t *src = reinterpret_cast<const uint16_t *>(raw + ((size_t)(live ? r : 0) * nb + b) * 210);
#pragma unroll
    for (int i = 0; i < 105; i++) h[i] = live ? src[i] : 0u;
    auto byte = [&](int o) -> uint32_t { return (h[o >> 1] >> (8 * (o & 1))) & 0xFFu; };
    auto word = [&](int o) -> uint32_t { return h[o >> 1] | (h[(o >> 1) + 1] << 16); };  // o even
    reinterpret_cast<uint4 *>(seg)[rho] = make_uint4(word(192), word(196), word(200), word(204));
    reinterpret_cast<uint16_t *>(seg + 256)[rho] = (uint16_t)h[104];
    // q6 of element e = 128h + 32t + l5: low nibble of ql[64h + l5 + 32(t&1)]
    // (shifted by 4(t>>1)), high 2 bits qh[32h + l5] >> 2t.  For lane class
    // l: nibble byte 4u + cc pairs j = 2u (low) and 2u + 1 (high nibble); the
    // high-bit byte 4(2hh + cls) + cc is qh[32hh + 8cc + l] as stored (hh
    // major, so a quarter's two classes are one aligned 8-byte pair).
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int l = 2 * qq + c;
        uint32_t o[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int hh = u >> 1, sh = 4 * (u & 1);
          uint32_t v = 0;
#pragma unroll
          for (int cc = 0; cc < 4; cc++) {
            const uint32_t lo = (byte(64 * hh + 8 * cc + l) >> sh) & 15u;
            const uint32_t hi = (byte(64 * hh + 32 + 8 * cc + l) >> sh) & 15u;
            v |= (lo | (hi << 4)) << (8 * cc);
          }
          o[u] = v;
        }
        reinterpret_cast<uint4 *>(seg + 288)[c * 64 + qq * 16 + rho] = make_uint4(o[0], o[1], o[2], o[3]);
      }
      uint32_t q[4];
#pragma unroll
      for (int cls = 0; cls < 2; cls++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          const int l = 2 * qq + cls;
          q[2 * hh + cls] = byte(128 + 32 * hh + l) | (byte(128 + 32 * hh + 8 + l) << 8) |
                            (byte(128 + 32 * hh + 16 + l) << 16) | (byte(128 + 32 * hh + 24 + l) << 24);
        }
      reinterpret_cast<uint4 *>(seg + 288)[128 + qq * 16 + rho] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
}

}  // namespace

size_t mfma_segment_bytes(int type, int rows, int nb) {
  return (size_t)((rows + 15) / 16) * nb * (type == kTypeQ4K ? 2304 : 3360);
}

size_t mfma_lds_bytes(int cols, int nb) {
  const int m4 = cols <= 4 ? 4 : 8;
  return (size_t)m4 * nb * (kXRegion + 32 + 4) + 16 + 4 * kFinFloats * 4;
}

hipError_t launch_repack_mfma(int type, const uint8_t *raw, int rows, int nb, uint8_t *segs, hipStream_t s) {
  const long long n = (long long)((rows + 15) / 16) * 16 * nb;
  const int threads = 256;
  hipLaunchKernelGGL(repack_mfma_kernel, dim3((unsigned)((n + threads - 1) / threads)), dim3(threads), 0, s, raw,
                     type, rows, nb, segs);
  return hipGetLastError();
}

hipError_t launch_matvec_mfma(const MfmaLaunch &l, int num_cus, hipStream_t s) {
  if (l.cols < 1 || l.cols > 8 || l.count < 1 || l.count > kMaxWeights || !mfma_geometry_ok(l))
    return hipErrorInvalidValue;
  MfmaArgs a{};
  a.count = l.count;
  int tiles = 0;
  for (int i = 0; i < l.count; i++) {
    a.w[i].seg = l.seg[i];
    a.w[i].wt = l.wt[i];
    a.w[i].dplane = l.dplane[i];
    a.w[i].out = l.out[i];
    a.w[i].type = l.type[i];
    a.w[i].rows = l.rows[i];
    a.w[i].tiles = (l.rows[i] + 15) / 16;
    a.w[i].tile_begin = tiles;
    tiles += a.w[i].tiles;
  }
  a.total_tiles = tiles;
  a.nb = l.k / kQK;
  a.S = l.S;
  a.R = l.R;
  a.x = l.x;
  a.k = l.k;
  a.cols = l.cols;
  a.out_col0 = l.out_col0;
  int grid = (tiles + 3) / 4;
  if (grid > num_cus * 8) grid = num_cus * 8;
  const size_t lds = mfma_lds_bytes(l.cols, a.nb);
  if (launch_reads_tiles(l)) {
    if (l.cols <= 4)
      hipLaunchKernelGGL((kquant_mfma_kernel<1, true>), dim3(grid), dim3(256), lds, s, a);
    else
      hipLaunchKernelGGL((kquant_mfma_kernel<2, true>), dim3(grid), dim3(256), lds, s, a);
  } else if (l.cols <= 4) {
    hipLaunchKernelGGL((kquant_mfma_kernel<1, false>), dim3(grid), dim3(256), lds, s, a);
  } else {
    hipLaunchKernelGGL((kquant_mfma_kernel<2, false>), dim3(grid), dim3(256), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace hp
