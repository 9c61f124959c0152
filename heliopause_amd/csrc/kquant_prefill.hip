// kquant_prefill.hip -- Q4_K / Q6_K x Q8_K projections of many columns
// (prefill chunks, M >= 32) on the gfx950 matrix cores, bit-exact with the
// reference's WASM path (packages/engine/wasm-kernels/src/lib.rs:224-426 with
// the vec-dots 2116-2172 and 1923-1968).
//
// Numerics are those of kquant_mfma.hip: per (row, column, block) the eight
// integers aux32[l] (l = element index mod 8) come out of one
// v_mfma_f32_16x16x32_f16 each, exactly, with A = sc * q (f16) and B = q8
// (f16); the f32 tail then runs in block order per class:
//   sums[l] += (dW_b * dX_b) * f32(aux32[l]);  Q4_K: sumf -= (dminW_b * dX_b) * f32(sumi)
//   result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
// Here the 16 MFMA columns are 16 input columns and the K = 32 dimension is
// the 32 elements of one class (quarter q of the A/B lanes carries elements
// j = 2q, 2q + 1, c = 0..3 of e = 32j + 8c + l), so every MFMA does useful
// work.  Exactness forces nine f32 chains per output, so the 8 classes are
// split over the 4 waves of a workgroup: wave w keeps classes 2w, 2w+1 of a
// 32-row x 64-column tile (64 chains per lane) and the Q4_K min chain of
// column slice w; the chains are added in class order through LDS at the end
// of the tile.
//
// Data flow per block: the tile's two 16-row weight segments (the
// matrix-core layout of kquant_mfma.hip, or, for a weight kept in one
// layout, gathered from its tiles into the same LDS image: see stage_store;
// each byte read once per column tile) and the 64 columns' Q8_K quants
// (int8, class-major, written by the pre-pass below) are staged in LDS,
// double-buffered through registers; A fragments (one dword per lane and
// class) and B fragments (8 bytes per lane) are built from LDS.
#include "hp_common.h"
#include "hp_f2tile.h"
#include "hp_gelu.h"
#include "hp_mfma.h"
#include "hp_q8k.h"
#include "hp_q8k16.h"

namespace hp {

namespace {

constexpr int kPfRows = 32;                        // rows per workgroup tile (2 segments)
constexpr int kPfCols = 64;                        // columns per workgroup tile
constexpr int kPfXStride = 272;                    // LDS bytes per column of one block's quants (256 + 16)
constexpr int kPfWBytes = 2 * 3360;                // two segments (Q6_K size)
constexpr int kPfXQ = kPfWBytes;                   // offsets within one stage buffer
constexpr int kPfXB = kPfXQ + kPfCols * kPfXStride;
constexpr int kPfXD = kPfXB + kPfCols * 32;
constexpr int kPfStage = kPfXD + kPfCols * 4;      // 26,432 bytes
constexpr int kPfFinStride = 68;                   // floats per row of the combine buffer
constexpr int kPfLds = 2 * kPfStage + kPfRows * kPfFinStride * 4;

// Q8_K pre-pass: one wave per (column, block) (hp_q8k.h, lib.rs:1774-1811).
// xq[(m * nb + b) * 256 + 32 l + 4 j + c] = q8 of element 32 j + 8 c + l;
// xb[(m * nb + b) * 16 + h] = f16 sum of the 16 quants 16 h .. 16 h + 15;
// xd[m * nb + b] = d.
__global__ __launch_bounds__(64) void q8k_prefill_kernel(const float *__restrict__ x, int k, int nb,
                                                         int8_t *__restrict__ xq, _Float16 *__restrict__ xb,
                                                         float *__restrict__ xd) {
  const int b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const Q8KLane r = q8k_block(x + (size_t)m * k + (size_t)b * kQK, lane);
  int8_t *dst = xq + ((size_t)m * nb + b) * kQK;
  // lane owns elements e = 4 lane + i: j = lane / 8, c = (lane / 2) % 4, l = 4 (lane % 2) + i
  const int base = 4 * (lane >> 3) + ((lane >> 1) & 3);
#pragma unroll
  for (int i = 0; i < 4; i++) dst[(4 * (lane & 1) + i) * 32 + base] = r.q[i];
  int s = (int)r.q[0] + (int)r.q[1] + (int)r.q[2] + (int)r.q[3];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  if ((lane & 3) == 0) xb[((size_t)m * nb + b) * 16 + (lane >> 2)] = (_Float16)s;  // |s| <= 2048: exact
  if (lane == 0) xd[(size_t)m * nb + b] = r.d;
}

struct PfWeight {
  const uint8_t *seg;      // segments of this weight (null: kept in one layout)
  const uint8_t *wt;       // tiles of this weight
  const uint16_t *dplane;  // Q6_K d plane
  float *out;
  int type, rows, tiles, rt_begin;  // tiles: 16-row segments; rt: 32-row workgroup tiles
};

struct PfArgs {
  PfWeight w[kMaxWeights];
  int count, total_rt, col_tiles, nb, cols;
  int S, R;  // tile geometry of the weights
  const int8_t *xq;
  const _Float16 *xb;
  const float *xd;
};

// Registers holding one block's staging loads of this thread: 16-byte weight
// units u = tid + 256 r of the two segments (TILE: tile-layout chunk c = u /
// 32 of tile row u % 32, and the Q6_K d of tile row tid < 32), the columns'
// quants and sums.
struct Stage {
  uint4 w[2], x[4], e;
  uint32_t d;
};

// Tile-layout place of this thread's weight row, tile row tid % 32 (both its
// chunks and its d; a row past the weight re-reads the weight's last row,
// whose sums are never stored).
__device__ __forceinline__ TileRow stage_row(const PfWeight &W, int T0, const PfArgs &a, int tid, int CH) {
  return tile_row(min(16 * T0 + (tid & 31), W.rows - 1), W.rows, a.nb, a.S, a.R, CH);
}

template <bool Q4, bool TILE>
__device__ __forceinline__ void stage_load(Stage &st, const PfWeight &W, int T0, const TileRow &tr, int b,
                                           const PfArgs &a, int col0, int tid) {
  st.d = 0;
  if constexpr (TILE) {
    constexpr int CH = Q4 ? 9 : 13;
    int bi, bs;
    block_split(b, a.S, bi, bs);
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int u = tid + 256 * r;
      st.w[r] = u < 32 * CH ? *reinterpret_cast<const uint4 *>(W.wt + tr.base + (uint32_t)bi * tr.iter +
                                                               (uint32_t)(u >> 5) * tr.chunk + 16u * (uint32_t)bs)
                            : make_uint4(0, 0, 0, 0);
    }
    if (!Q4 && tid < 32) st.d = W.dplane[tr.dbase + (uint32_t)bi * tr.diter + (uint32_t)bs];
  } else {
    constexpr int segb = Q4 ? 2304 : 3360;
    const int nseg = T0 + 1 < W.tiles ? 2 : 1;
    const uint8_t *src = W.seg + ((size_t)b * W.tiles + T0) * segb;  // segments T0, T0 + 1 are adjacent
    const int n16 = nseg * segb / 16;
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int i = tid + 256 * r;
      st.w[r] = i < n16 ? reinterpret_cast<const uint4 *>(src)[i] : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int i = tid + 256 * r, col = i >> 4, part = i & 15;
    const int m = col0 + col;
    st.x[r] = m < a.cols ? reinterpret_cast<const uint4 *>(a.xq + ((size_t)m * a.nb + b) * kQK)[part]
                         : make_uint4(0, 0, 0, 0);
  }
  st.e = make_uint4(0, 0, 0, 0);
  if (tid < 128) {  // bs16: 64 columns x 32 bytes
    const int col = tid >> 1, m = col0 + col;
    st.e = m < a.cols ? reinterpret_cast<const uint4 *>(a.xb + ((size_t)m * a.nb + b) * 16)[tid & 1]
                      : make_uint4(0, 0, 0, 0);
  } else if (tid < 144) {  // d: 64 columns x 4 bytes
    const int c4 = tid - 128;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = col0 + 4 * c4 + i;
      v[i] = m < a.cols ? a.xd[(size_t)m * a.nb + b] : 0.0f;
    }
    st.e = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
  }
}

// The weights go to LDS as two 16-row segments, in the order the A
// fragments read them.  Segment units are copied as they are; tile chunks
// are scattered (dword D[p][l] of row rho -> unit (class l, row rho) of the
// segment, dword p):
//   Q4_K, 2304 bytes: [0,256) the 16 row headers; [256,2304) unit (l, rho)
//     at 256 + 1024 (l % 2) + 16 (16 (l / 2) + rho), dword p = D[p][l].
//   Q6_K, 3360 bytes: [0,256) the 16 rows' scales; [256,288) their f16 d;
//     [288,2336) low-bit units as Q4_K's; [2336,3360) high-bit unit (l / 2,
//     rho) dword 2h + l % 2 = Dqh[h][l] ^ 0xAA.. (the fields as GGUF stores them).
template <bool Q4, bool TILE>
__device__ __forceinline__ void stage_store(const Stage &st, uint8_t *buf, int tid) {
  constexpr int CH = Q4 ? 9 : 13, segb = Q4 ? 2304 : 3360;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int u = tid + 256 * r;
    if (!TILE) {
      if (u < kPfWBytes / 16) reinterpret_cast<uint4 *>(buf)[u] = st.w[r];
      continue;
    }
    if (u >= 32 * CH) continue;
    const int c = u >> 5, rl = u & 31, rho = rl & 15;
    uint8_t *seg = buf + (rl >> 4) * segb;
    const uint32_t wv[4] = {st.w[r].x, st.w[r].y, st.w[r].z, st.w[r].w};
    if (c == (Q4 ? 0 : 12)) {
      *reinterpret_cast<uint4 *>(seg + 16 * rho) = st.w[r];
    } else if (Q4 || c < 8) {
      const int ck = Q4 ? c - 1 : c;  // dwords 4 ck + e = D[ck / 2][4 (ck % 2) + e]
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int l = 4 * (ck & 1) + e;
        *reinterpret_cast<uint32_t *>(seg + (Q4 ? 256 : 288) + 1024 * (l & 1) + 16 * (16 * (l >> 1) + rho) +
                                      4 * (ck >> 1)) = wv[e];
      }
    } else {
      const int ck = c - 8;  // dwords 4 ck + e = Dqh[ck / 2][4 (ck % 2) + e]
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int l = 4 * (ck & 1) + e;
        *reinterpret_cast<uint32_t *>(seg + 2336 + 16 * (16 * (l >> 1) + rho) + 4 * (2 * (ck >> 1) + (l & 1))) =
            wv[e] ^ 0xAAAAAAAAu;
      }
    }
  }
  if (TILE && !Q4 && tid < 32)
    *reinterpret_cast<uint16_t *>(buf + (tid >> 4) * segb + 256 + 2 * (tid & 15)) = (uint16_t)st.d;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int i = tid + 256 * r, col = i >> 4, part = i & 15;
    *reinterpret_cast<uint4 *>(buf + kPfXQ + col * kPfXStride + 16 * part) = st.x[r];
  }
  if (tid < 128)
    reinterpret_cast<uint4 *>(buf + kPfXB)[tid] = st.e;
  else if (tid < 144)
    reinterpret_cast<uint4 *>(buf + kPfXD)[tid - 128] = st.e;
}

// B fragment: 8 int8 quants of (column n, class l, quarter q) as f16.
__device__ __forceinline__ half8 b_frag(const uint8_t *xq_col, int l, int q) {
  const uint2 v = *reinterpret_cast<const uint2 *>(xq_col + 32 * l + 8 * q);
  // (byte ^ 0x80) is q8 + 128 < 256: 1024 + that as f16, minus 1152, is q8 exactly
  const uint32_t lo = v.x ^ 0x80808080u, hi = v.y ^ 0x80808080u;
  const half2v off = (half2v){(_Float16)1152.0f, (_Float16)1152.0f};
  return cat(magic_pair<kSel01>(lo) - off, magic_pair<kSel23>(lo) - off, magic_pair<kSel01>(hi) - off,
             magic_pair<kSel23>(hi) - off);
}

// A fragment of class l for the 16 rows of one segment: lane (row n,
// quarter q) takes the dword of (chunk l % 2, u = q) that segment lane
// (n, l / 2) holds, i.e. elements j = 2q, 2q + 1, c = 0..3 of class l.
template <bool Q4>
__device__ __forceinline__ half8 a_frag(const uint8_t *seg, int l, int n, int q) {
  const int g = l & 1, src = n + 16 * (l >> 1);
  if constexpr (Q4) {
    const uint4 hdr = *reinterpret_cast<const uint4 *>(seg + 16 * n);
    const uint32_t sclo = hdr.y & 0x3F3F3F3Fu;
    const uint32_t schi = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    const uint32_t sc = q < 2 ? sclo : schi;  // scales of j = 2q, 2q + 1 are bytes 2(q%2), 2(q%2)+1
    const half2v S0 = dup_byte(sc, 2 * (q & 1), 1024.0f), S1 = dup_byte(sc, 2 * (q & 1) + 1, 1024.0f);
    const half2v m1024 = (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v N0 = S0 * m1024, N1 = S1 * m1024;
    const uint32_t dw = *reinterpret_cast<const uint32_t *>(seg + 256 + 1024 * g + 16 * src + 4 * q);
    const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
    return cat(fma2(magic_pair<kSel01>(lo), S0, N0), fma2(magic_pair<kSel23>(lo), S0, N0),
               fma2(magic_pair<kSel01>(hi), S1, N1), fma2(magic_pair<kSel23>(hi), S1, N1));
  } else {
    // groups 16-element: g(j, c) = 2j + c/2; for u = q: 4q, 4q+1 (j = 2q) and 4q+2, 4q+3 (j = 2q+1)
    const uint32_t gs = *reinterpret_cast<const uint32_t *>(seg + 16 * n + 4 * q) ^ 0x80808080u;
    half2v S[4], N[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      S[e] = dup_byte(gs, e, 1152.0f);
      N[e] = S[e] * (half2v){(_Float16)-1056.0f, (_Float16)-1056.0f};
    }
    const int jj = 2 * (q & 1);
    const uint32_t ql = *reinterpret_cast<const uint32_t *>(seg + 288 + 1024 * g + 16 * src + 4 * q);
    const uint32_t qh = *reinterpret_cast<const uint32_t *>(seg + 288 + 2048 + 16 * src + 4 * (2 * (q >> 1) + g));
    const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * jj)) & 0x03030303u) << 4);
    const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * jj + 2)) & 0x03030303u) << 4);
    return cat(fma2(magic_pair<kSel01>(lo), S[0], N[0]), fma2(magic_pair<kSel23>(lo), S[1], N[1]),
               fma2(magic_pair<kSel01>(hi), S[2], N[2]), fma2(magic_pair<kSel23>(hi), S[3], N[3]));
  }
}

struct PfChains {
  float s[2][2][4][4];  // [class of the wave][row segment][column slice][row j of the D layout]
  float f[2][4];        // Q4_K min chain of the wave's column slice: [row segment][j]
};

// One block of the tile from stage buffer `buf`.
template <bool Q4>
__device__ __forceinline__ void pf_block(PfChains &ch, const uint8_t *buf, int wave, int lane) {
  const int n = lane & 15, q = lane >> 4;
  const int segb = Q4 ? 2304 : 3360;
  // dW of rows 16 rs + 4q + j, dX of columns 16 cs + n
  float dw[2][4], dmw[2][4], dx[4];
#pragma unroll
  for (int rs = 0; rs < 2; rs++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int row = 4 * q + j;
      if constexpr (Q4) {
        const uint32_t v = *reinterpret_cast<const uint32_t *>(buf + rs * segb + 16 * row);
        dw[rs][j] = h2f_bits(v & 0xFFFFu);
        dmw[rs][j] = h2f_bits(v >> 16);
      } else {
        dw[rs][j] = h2f_bits(*reinterpret_cast<const uint16_t *>(buf + rs * segb + 256 + 2 * row));
        dmw[rs][j] = 0.0f;
      }
    }
#pragma unroll
  for (int cs = 0; cs < 4; cs++) dx[cs] = reinterpret_cast<const float *>(buf + kPfXD)[16 * cs + n];
  float dd[2][4][4];
#pragma unroll
  for (int rs = 0; rs < 2; rs++)
#pragma unroll
    for (int cs = 0; cs < 4; cs++)
#pragma unroll
      for (int j = 0; j < 4; j++) dd[rs][cs][j] = __fmul_rn(dw[rs][j], dx[cs]);
#pragma unroll
  for (int li = 0; li < 2; li++) {
    const int l = 2 * wave + li;
    const half8 a0 = a_frag<Q4>(buf, l, n, q);
    const half8 a1 = a_frag<Q4>(buf + segb, l, n, q);
#pragma unroll
    for (int cs = 0; cs < 4; cs++) {
      const half8 bf = b_frag(buf + kPfXQ + (16 * cs + n) * kPfXStride, l, q);
      const f32x4 z = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
      const f32x4 d0 = mfma(a0, bf, z);
      const f32x4 d1 = mfma(a1, bf, z);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        ch.s[li][0][cs][j] = __fadd_rn(ch.s[li][0][cs][j], __fmul_rn(dd[0][cs][j], d0[j]));
        ch.s[li][1][cs][j] = __fadd_rn(ch.s[li][1][cs][j], __fmul_rn(dd[1][cs][j], d1[j]));
      }
    }
  }
  if constexpr (Q4) {
    // sumi = sum_j mn_j * bsums32_j by one MFMA per segment: quarter q < 2
    // carries k = 8q + e -> (j = 4q + e/2, half e%2); B = the 16 half sums
    const int cs = wave;
    const uint8_t *xcol = buf + kPfXB + (16 * cs + n) * 32;
    const half8 bm = q < 2 ? __builtin_bit_cast(half8, *reinterpret_cast<const uint4 *>(xcol + 16 * q))
                           : (half8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int rs = 0; rs < 2; rs++) {
      const uint4 hdr = *reinterpret_cast<const uint4 *>(buf + rs * segb + 16 * n);
      const uint32_t mn = q == 0 ? (hdr.z & 0x3F3F3F3Fu) : (((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u));
      const half8 am = q < 2 ? cat(dup_byte(mn, 0, 1024.0f), dup_byte(mn, 1, 1024.0f), dup_byte(mn, 2, 1024.0f),
                                   dup_byte(mn, 3, 1024.0f))
                             : (half8){0, 0, 0, 0, 0, 0, 0, 0};
      const f32x4 sm = mfma(am, bm, (f32x4){0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
      for (int j = 0; j < 4; j++) ch.f[rs][j] = __fsub_rn(ch.f[rs][j], __fmul_rn(__fmul_rn(dmw[rs][j], dx[cs]), sm[j]));
    }
  }
}

template <bool Q4, bool TILE>
__device__ void pf_tile(const PfArgs &a, const PfWeight &W, int T0, int col0, uint8_t *smem, int wave, int lane,
                        int tid) {
  PfChains ch;
#pragma unroll
  for (int li = 0; li < 2; li++)
#pragma unroll
    for (int rs = 0; rs < 2; rs++)
#pragma unroll
      for (int cs = 0; cs < 4; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) ch.s[li][rs][cs][j] = 0.0f;
#pragma unroll
  for (int rs = 0; rs < 2; rs++)
#pragma unroll
    for (int j = 0; j < 4; j++) ch.f[rs][j] = 0.0f;

  Stage st;
  const TileRow tr = TILE ? stage_row(W, T0, a, tid, Q4 ? 9 : 13) : TileRow{};
  stage_load<Q4, TILE>(st, W, T0, tr, 0, a, col0, tid);
  stage_store<Q4, TILE>(st, smem, tid);
  __syncthreads();
  for (int b = 0; b < a.nb; b++) {
    if (b + 1 < a.nb) stage_load<Q4, TILE>(st, W, T0, tr, b + 1, a, col0, tid);
    pf_block<Q4>(ch, smem + (b & 1) * kPfStage, wave, lane);
    if (b + 1 < a.nb) stage_store<Q4, TILE>(st, smem + ((b + 1) & 1) * kPfStage, tid);
    __syncthreads();
  }

  // class chains in order l = 0..7 through LDS, then [sumf +] and the store
  float *fin = reinterpret_cast<float *>(smem + 2 * kPfStage);
  const int n = lane & 15, q = lane >> 4;
  for (int p = 0; p < 4; p++) {
    if (wave == p) {
#pragma unroll
      for (int rs = 0; rs < 2; rs++)
#pragma unroll
        for (int cs = 0; cs < 4; cs++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            float *slot = fin + (16 * rs + 4 * q + j) * kPfFinStride + 16 * cs + n;
            const float t = __fadd_rn(p == 0 ? -0.0f : *slot, ch.s[0][rs][cs][j]);
            *slot = __fadd_rn(t, ch.s[1][rs][cs][j]);
          }
    }
    __syncthreads();
  }
  const int cs = wave;
  const int m = col0 + 16 * cs + n;
#pragma unroll
  for (int rs = 0; rs < 2; rs++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int row = 16 * (T0 + rs) + 4 * q + j;
      float v = fin[(16 * rs + 4 * q + j) * kPfFinStride + 16 * cs + n];
      if (Q4) v = __fadd_rn(ch.f[rs][j], v);
      if (row < W.rows && m < a.cols) W.out[(size_t)m * W.rows + row] = v;
    }
  __syncthreads();  // fin and the stage buffers are reused by the next tile
}

// TILE: every weight is read from its tiles (a launch with a weight kept in
// one layout); else from its segments.
template <bool TILE>
__global__ __launch_bounds__(256) void kquant_prefill_kernel(const PfArgs a) {
  kernarg_warm<PfArgs>();
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int items = a.total_rt * a.col_tiles;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    // column tiles innermost: neighbouring workgroups share a weight tile
    const int rt = it / a.col_tiles, ct = it - rt * a.col_tiles;
    PfWeight W = a.w[0];
    if (a.count > 1 && rt >= a.w[1].rt_begin) W = a.w[1];
    if (a.count > 2 && rt >= a.w[2].rt_begin) W = a.w[2];
    if (a.count > 3 && rt >= a.w[3].rt_begin) W = a.w[3];
    const int T0 = 2 * (rt - W.rt_begin);
    if (W.type == kTypeQ4K)
      pf_tile<true, TILE>(a, W, T0, ct * kPfCols, smem, wave, lane, tid);
    else
      pf_tile<false, TILE>(a, W, T0, ct * kPfCols, smem, wave, lane, tid);
  }
}

// ---- fast prefill (within the stated tolerance, not bit-exact) -------------
//
// Per (row, column, block) the eight class MFMAs accumulate into one f32
// D = sum_l aux32[l] (exact integer products; partial sums may round above
// 2^24), then out += (dW_b * dX_b) * D and, for Q4_K, out -= (dminW_b * dX_b) *
// sumi, with fused multiply-adds.  That reorders the reference's f32 tail, so
// outputs agree to within a relative 1e-4 (the stated tolerance for
// projections), and cuts the vector-ALU tail from 18 to at most 4 operations
// per output and block.
//
// Workgroup tile: 8 waves; a wave owns 32 rows (two 16-row segments) x 64
// columns.  256 rows x 64 columns (PAIR: 128 rows of gate, waves 0-3, and
// the same 128 rows of up, waves 4-7).
//
// Weights go straight from global memory to registers: each wave's rows are
// its own, so staging them in LDS would buy no reuse.  The 64 columns'
// activation tile (written by the pre-pass in the order the fragments are
// read) is shared by the 8 waves through two LDS stages:
//   XH f16 [class l][quarter q][column n (64)][8]   32768 bytes
//   XB f16 [q < 2][n][8]  (half-block sums 16h..16h+15, h = 8q + e)  2048
//   XD f32 [n]                                                         256
// Per block b the loads of block b + 1 (its weights into the other register
// set, its activation tile into staging registers) are issued first and land
// while block b computes; the staged tile is then written to the other LDS
// stage, and one barrier per block separates the stages' readers and writers.
//
// Operand order: the activation tile is the MFMA's first operand and the
// weights the second, so lane (n, q)'s accumulator holds weight row n of the
// segment and columns 4q .. 4q + 3 of the column set: the row's d and dmin
// come with the lane's own header load.
// Two waves per SIMD: measured against one wave per SIMD with 128-column
// tiles (kF3Waves 4, kF3CS 8: 4.3 instead of 6.5 vector-ALU instructions per
// MFMA, 374 registers), which took gate/up from 79 to 98 us on the 512-column
// chunk: a lone wave per SIMD stalls on each block's loads and barrier.
constexpr int kF3Waves = 8;                                          // per workgroup
constexpr int kF3PerSIMD = kF3Waves / 4;                             // waves per SIMD (one workgroup per CU)
constexpr int kF3PerCU = 1;                                          // workgroups per CU
constexpr int kF3RS = 2;                                             // 16-row segments per wave
constexpr int kF3CS = 4;                                             // 16-column sets per wave
constexpr int kF3Tiles = kF3CS / 4;                                  // 64-column activation tiles per work tile
constexpr int kF3Cols = 16 * kF3CS;                                  // columns per work tile
constexpr int kF3Threads = 64 * kF3Waves;
constexpr int kF3Segs = kF3RS * kF3Waves;                            // segments per workgroup tile
constexpr int kF3Full = kF2XTile / 1024;                             // whole 1 KB chunks per activation tile
constexpr int kF3Part = kF2XTile % 1024;                             // bytes of the last, partial chunk

// The fast kernel's activation tiles (f16 quants [class][quarter][column][8],
// f16 16-element sums, f32 d per column) from Q8_K of x, one 16-lane row per
// (block, column): 16 columns per workgroup, vector loads of the column and 8-byte stores of four quants of
// one class.  Lane i16 = 2j + u holds elements 32j + 8c + 4u + i (c, i < 4):
// class l = 4u + i, quarter j / 2, position 4 (j & 1) + c of the quarter's
// eight; its 16-element sums are halves of groups 2j (c < 2) and 2j + 1.
__global__ __launch_bounds__(256) void q8k_prefill_tiles16_kernel(const float *__restrict__ x, int k, int nb,
                                                                  int cols, uint8_t *__restrict__ xt) {
  const int b = blockIdx.x, i16 = threadIdx.x & 15;
  const int m = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int ct = m / kF2Cols, n = m % kF2Cols;
  uint8_t *tile = xt + ((size_t)ct * nb + b) * kF2XTile;
  float v[16];
  load_x16(v, x + (size_t)min(m, cols - 1) * k + (size_t)b * kQK, i16);
  if (m >= cols) {
#pragma unroll
    for (int e = 0; e < 16; e++) v[e] = 0.0f;
  }
  f2_tile_store16(v, i16, tile, n);
}

struct F2Args {
  PfWeight w[kMaxWeights];  // rt_begin counts 256-row workgroup tiles here
  int count, total_rt, col_tiles, nb, cols;
  int S, R;  // tile geometry of the weights
  const uint8_t *xt;
  // ksplit > 1: block range r of a tile writes its sums to part + r * part_stride
  // + part_off[weight] + m * rows + row instead of the output
  int ksplit;
  float *part;
  size_t part_stride;
  size_t part_off[kMaxWeights];
  // gate/up + GeGLU tiles (w[0] gate, w[1] up): pair_out[m][row]
  float *pair_out;
  const uint16_t *gelu_lut;
  // tail_full > 0 (gate/up): the items from tail_full on, fewer than half a
  // round, run as two block ranges each; the ranges write their sums to
  // tail_part (f2_geglu_tail_kernel adds them and applies the GeGLU)
  int tail_full;
  float *tail_part;
};

// One segment's weights in a lane's registers, loaded with 16- and 8-byte
// loads (few memory instructions), from one of two places:
//   segments (matrix-core layout): lane (n, r) holds unit n + 16r of chunk g,
//     dwords u = 0..3, and f3_transpose turns them into what the A fragments
//     take: lane (n, q) holds dword q of units n + 16t, t = 0..3 (class
//     l = 2t + g);
//   tiles (a weight kept in one layout, hp_common.h): lane (row n, quarter
//     q) takes the two quant chunks holding dwords D[q][l], l = 0..3 and
//     4..7, which are what its A fragments need (class l = 2t + g: dword
//     l % 4 of chunk l / 4), no transpose.
// Q4_K: row n's header (d | dmin, then the 12 bytes of 6-bit scales and
// mins) and the quants (qa[g] / qa[l / 4]).
struct W4 {
  uint4 hdr;
  uint4 qa[2];
};
// Q6_K: low-bit units or chunks as Q4_K's; high bits: for class l = 2t + g
// dword 2 (t % 2) + g of qh[t / 2] (segments: the two dwords of unit n + 16t
// for quarter pair q / 2; tiles: chunks 8 + 2h, 9 + 2h, h = q / 2, fields
// stored ^ 2); row n's scales 4q .. 4q + 3 and its d (f16 bits).
struct W6 {
  uint4 qa[2];
  uint4 qh[2];
  uint32_t gs, d16;
};
template <bool Q4>
struct WSel {
  using T = W6;
};
template <>
struct WSel<true> {
  using T = W4;
};

// A lane's offsets into one of its rows' row-blocks (tile_row) and the
// chunks it loads: oq = its first quant chunk, oh = its first high-bit chunk.
struct F3Row {
  TileRow tr;
  uint32_t oq, oh;
};

template <bool Q4>
__device__ __forceinline__ F3Row f3_row(int row, int rows, int nb, int S, int R, int q) {
  F3Row f;
  f.tr = tile_row(row, rows, nb, S, R, Q4 ? 9 : 13);
  f.oq = (uint32_t)(Q4 ? 1 + 2 * q : 2 * q) * f.tr.chunk;
  f.oh = (uint32_t)(8 + 2 * (q >> 1)) * f.tr.chunk;
  return f;
}

// Segment layouts of the matrix-core repack (kquant_mfma.hip): Q4_K [16 rows
// x 16-byte header][2 chunks x 64 units x 16 bytes of quants]; Q6_K [16 rows x
// 16 scales][16 x f16 d][2 chunks x 1024 low bits][1024 high bits].
template <bool Q4>
__device__ __forceinline__ void f3_wload_seg(typename WSel<Q4>::T &w, const uint8_t *seg, int lane) {
  const int n = lane & 15, q = lane >> 4;
  if constexpr (Q4) {
    w.hdr = *reinterpret_cast<const uint4 *>(seg + 16 * n);
#pragma unroll
    for (int g = 0; g < 2; g++) w.qa[g] = *reinterpret_cast<const uint4 *>(seg + 256 + 1024 * g + 16 * lane);
  } else {
    w.gs = *reinterpret_cast<const uint32_t *>(seg + 16 * n + 4 * q);
    w.d16 = *reinterpret_cast<const uint16_t *>(seg + 256 + 2 * n);
#pragma unroll
    for (int g = 0; g < 2; g++) w.qa[g] = *reinterpret_cast<const uint4 *>(seg + 288 + 1024 * g + 16 * lane);
    uint2 h[4];
#pragma unroll
    for (int t = 0; t < 4; t++) h[t] = *reinterpret_cast<const uint2 *>(seg + 2336 + 256 * t + 16 * n + 8 * (q >> 1));
    w.qh[0] = make_uint4(h[0].x, h[0].y, h[1].x, h[1].y);
    w.qh[1] = make_uint4(h[2].x, h[2].y, h[3].x, h[3].y);
  }
}

// 4 x 4 transpose across the wave's four 16-lane rows: in, lane (n, r) holds
// v[u] = element (r, u); out, lane (n, q) holds v[t] = element (t, q).
__device__ __forceinline__ void f3_transpose(uint32_t (&v)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  v[0] = c[0];
  v[1] = c[1];
  v[2] = d[0];
  v[3] = d[1];
}

// Block (bi, bs) = bi * S + bs of row f into w, from the tiles.
template <bool Q4>
__device__ __forceinline__ void f3_wload_tile(typename WSel<Q4>::T &w, const uint8_t *wt, const uint16_t *dplane,
                                              const F3Row &f, int bi, int bs, int q) {
  const uint32_t off = f.tr.base + (uint32_t)bi * f.tr.iter + 16u * (uint32_t)bs;
  auto ld16 = [&](uint32_t o) { return *reinterpret_cast<const uint4 *>(wt + o); };
  w.qa[0] = ld16(off + f.oq);
  w.qa[1] = ld16(off + f.oq + f.tr.chunk);
  if constexpr (Q4) {
    w.hdr = ld16(off);
  } else {
    w.qh[0] = ld16(off + f.oh);
    w.qh[1] = ld16(off + f.oh + f.tr.chunk);
    w.gs = *reinterpret_cast<const uint32_t *>(wt + off + 12u * f.tr.chunk + 4u * (uint32_t)q);
    w.d16 = dplane[f.tr.dbase + (uint32_t)bi * f.tr.diter + (uint32_t)bs];
  }
}

// Weight fragment of class l = 2t + g (sc * q as exact f16); qd[g][t] are the
// quant dwords D[q][l].  Element order: bytes 0, 2, 1, 3 of the dword's
// low nibbles (or low 6-bit values), then the same of its high ones -- the
// activation tiles store their runs the same way.  Q4_K: (S[0], N[0]) scale
// the low nibbles, (S[1], N[1]) the high ones as 16 q (their scale / 16).
// Q6_K: S[0] = (s0, s1) for the low values, S[1] = (s2, s3) for the high.
template <bool Q4, bool TILE>
__device__ __forceinline__ half8 f3_a(const typename WSel<Q4>::T &w, const uint32_t (&qd)[2][4], int l, int q,
                                      const half2v (&S)[2], const half2v (&N)[2], uint32_t exp) {
  const int g = l & 1, t = l >> 1;
  if constexpr (Q4) {
    const uint32_t dw = qd[g][t], d8 = dw >> 8;
    return cat(fma2(magic_nib<kNibLo>(dw, exp), S[0], N[0]), fma2(magic_nib<kNibLo>(d8, exp), S[0], N[0]),
               fma2(magic_nib<kNibHi>(dw, exp), S[1], N[1]), fma2(magic_nib<kNibHi>(d8, exp), S[1], N[1]));
  } else {
    const int jj = 2 * (q & 1);
    // the tiles store the fields as hi ^ 2
    const uint32_t ql = qd[g][t], qh = u4at(w.qh[t >> 1], 2 * (t & 1) + g) ^ (TILE ? 0xAAAAAAAAu : 0u);
    const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * jj)) & 0x03030303u) << 4);
    const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * jj + 2)) & 0x03030303u) << 4);
    return cat(fma2(magic_pair<kSel02>(lo), S[0], N[0]), fma2(magic_pair<kSel13>(lo), S[0], N[0]),
               fma2(magic_pair<kSel02>(hi), S[1], N[1]), fma2(magic_pair<kSel13>(hi), S[1], N[1]));
  }
}

// One block of the wave's tile (kF3RS segments x 64 columns): weights w
// against the activation tile at xl.  Segments past the weight's end repeat
// the last one and are never stored.
template <bool Q4, bool TILE>
__device__ __forceinline__ void f3_block(float (&out)[kF3RS][kF3CS][4], const typename WSel<Q4>::T (&w)[kF3RS],
                                         const uint8_t *xl, int lane, uint32_t exp) {
  // Wave priority: the block's set-up and class loop (the matrix cores'
  // work) issue ahead of the other wave of the SIMD while that one runs its
  // f32 tail, which lowers it again below: the MFMA pipe stays fed through
  // the other wave's tail (the 512-token prefill chunk about 2 % faster
  // than at one priority throughout).
  __builtin_amdgcn_s_setprio(1);
  const int n = lane & 15, q = lane >> 4;
  // column set cs: 16-column slice cs % 4 of activation tile cs / 4
  auto xh = [&](int cs) { return reinterpret_cast<const _Float16 *>(xl + (cs >> 2) * kF2XTile); };
  half2v S[kF3RS][2], N[kF3RS][2];
#pragma unroll
  for (int rs = 0; rs < kF3RS; rs++) {
    if constexpr (Q4) {
      const uint4 hdr = w[rs].hdr;
      const uint32_t sclo = hdr.y & 0x3F3F3F3Fu;
      const uint32_t schi = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
      const uint32_t sc = q < 2 ? sclo : schi;
      S[rs][0] = dup_byte(sc, 2 * (q & 1), 1024.0f);
      S[rs][1] = dup_byte_16th(sc, 2 * (q & 1) + 1);
      const half2v m1024 = (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
#pragma unroll
      for (int e = 0; e < 2; e++) N[rs][e] = S[rs][e] * m1024;
    } else {
      // signed scales: bytes ^ 0x80 are s + 128; (1024 + 128 + s) - 1152 = s
      const uint32_t gs = w[rs].gs ^ 0x80808080u;
      const half2v b1152 = (half2v){(_Float16)1152.0f, (_Float16)1152.0f};
      S[rs][0] = magic_pair<kSel01>(gs) - b1152;  // (s0, s1)
      S[rs][1] = magic_pair<kSel23>(gs) - b1152;  // (s2, s3)
#pragma unroll
      for (int e = 0; e < 2; e++)
        N[rs][e] = S[rs][e] * (half2v){(_Float16)-1056.0f, (_Float16)-1056.0f};  // -(1024 + 32) * sc
    }
  }
  uint32_t qd[kF3RS][2][4];  // [rs][g][t]: dword D[q][2t + g]
#pragma unroll
  for (int rs = 0; rs < kF3RS; rs++)
#pragma unroll
    for (int g = 0; g < 2; g++) {
      if constexpr (TILE) {
#pragma unroll
        for (int t = 0; t < 4; t++) qd[rs][g][t] = u4at(w[rs].qa[t >> 1], 2 * (t & 1) + g);
      } else {
        const uint4 v = w[rs].qa[g];
        qd[rs][g][0] = v.x;
        qd[rs][g][1] = v.y;
        qd[rs][g][2] = v.z;
        qd[rs][g][3] = v.w;
        f3_transpose(qd[rs][g]);
      }
    }
  f32x4 D[kF3RS][kF3CS];
  // Software pipeline over the classes: while class l's MFMAs run, class
  // l + 1's B fragments are read from LDS and its weight fragments unpacked
  // (interleaved: one MFMA, then a few vector-ALU instructions).
  half8 B[2][kF3CS];
#pragma unroll
  for (int cs = 0; cs < kF3CS; cs++)
    B[0][cs] = __builtin_bit_cast(half8,
                                  *reinterpret_cast<const uint4 *>(xh(cs) + (q * kF2Cols + 16 * (cs & 3) + n) * 8));
  half8 An[kF3RS];
#pragma unroll
  for (int rs = 0; rs < kF3RS; rs++) An[rs] = f3_a<Q4, TILE>(w[rs], qd[rs], 0, q, S[rs], N[rs], exp);
#pragma unroll
  for (int l = 0; l < 8; l++) {
    half8 A[kF3RS];
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++) A[rs] = An[rs];
    if (l < 7) {
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
        B[(l + 1) & 1][cs] = __builtin_bit_cast(
            half8, *reinterpret_cast<const uint4 *>(xh(cs) + (((l + 1) * 4 + q) * kF2Cols + 16 * (cs & 3) + n) * 8));
#pragma unroll
      for (int rs = 0; rs < kF3RS; rs++) An[rs] = f3_a<Q4, TILE>(w[rs], qd[rs], l + 1, q, S[rs], N[rs], exp);
    }
#pragma unroll
    for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
      for (int rs = 0; rs < kF3RS; rs++)
        D[rs][cs] = mfma(B[l & 1][cs], A[rs], l == 0 ? (f32x4){0.0f, 0.0f, 0.0f, 0.0f} : D[rs][cs]);
    if (l < 7) {
      __builtin_amdgcn_sched_group_barrier(0x100, kF3CS, 0);  // the B reads first
#pragma unroll
      for (int k = 0; k < kF3CS * kF3RS; k++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to 3 vector-ALU
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);  // the tail below the other wave's class loop
  f32x4 dx[kF3CS];
#pragma unroll
  for (int cs = 0; cs < kF3CS; cs++)
    dx[cs] = *reinterpret_cast<const f32x4 *>(xl + (cs >> 2) * kF2XTile + 32768 + 2048 + 4 * (16 * (cs & 3) + 4 * q));
  if constexpr (Q4) {
    // sumi = sum_j mn_j * bsums32_j: quarter q < 2 carries k = 8q + e ->
    // (j = 4q + e/2, half e%2) against the 16 half-block sums (quarters 2, 3
    // read the same sums against zero mins); out += dx * (dw * D - dmin * sumi)
    half8 bm[kF3CS];
#pragma unroll
    for (int cs = 0; cs < kF3CS; cs++) {
      const _Float16 *xb = reinterpret_cast<const _Float16 *>(xl + (cs >> 2) * kF2XTile + 32768);
      bm[cs] = __builtin_bit_cast(
          half8, *reinterpret_cast<const uint4 *>(xb + (((q & 1) * kF2Cols) + 16 * (cs & 3) + n) * 8));
    }
    // each stage over all 16 sums of a segment before the next, so the
    // sums' independent chains interleave instead of waiting on each other
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++) {
      const uint4 hdr = w[rs].hdr;
      const float dw = h2f_bits(hdr.x & 0xFFFFu), dmw = h2f_bits(hdr.x >> 16);
      const uint32_t mn0 = hdr.z & 0x3F3F3F3Fu, mn1 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
      const uint32_t mn = q == 0 ? mn0 : q == 1 ? mn1 : 0u;
      half8 am = cat(dup_byte(mn, 0, 1024.0f), dup_byte(mn, 1, 1024.0f), dup_byte(mn, 2, 1024.0f),
                     dup_byte(mn, 3, 1024.0f));
      f32x4 sm[kF3CS];
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++) sm[cs] = mfma(bm[cs], am, (f32x4){0.0f, 0.0f, 0.0f, 0.0f});
      float t[kF3CS][4];
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) t[cs][j] = dw * D[rs][cs][j];
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) t[cs][j] = __builtin_fmaf(-dmw, sm[cs][j], t[cs][j]);
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) out[rs][cs][j] = __builtin_fmaf(dx[cs][j], t[cs][j], out[rs][cs][j]);
    }
  } else {
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++) {
      const float dw = h2f_bits(w[rs].d16);
      float t[kF3CS][4];
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) t[cs][j] = dw * D[rs][cs][j];
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) out[rs][cs][j] = __builtin_fmaf(dx[cs][j], t[cs][j], out[rs][cs][j]);
    }
  }
}

// Block b of the wave's segments s0 .. s0 + kF3RS - 1 (each clamped to the
// weight's last), from its segments or (TILE) its tiles at rows f[rs].
template <bool Q4, bool TILE>
__device__ __forceinline__ void f3_wloads(typename WSel<Q4>::T (&w)[kF3RS], const PfWeight &W, const F3Row (&f)[kF3RS],
                                          int s0, int b, int S, int lane) {
  if constexpr (TILE) {
    int bi, bs;
    block_split(b, S, bi, bs);
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++) f3_wload_tile<Q4>(w[rs], W.wt, W.dplane, f[rs], bi, bs, lane >> 4);
  } else {
    constexpr int segb = Q4 ? 2304 : 3360;
    const uint8_t *base = W.seg + (size_t)b * W.tiles * segb;
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++) f3_wload_seg<Q4>(w[rs], base + (size_t)min(s0 + rs, W.tiles - 1) * segb, lane);
  }
}

// The two activation-tile stages.  Two distinct arrays, so the compiler sees
// that a direct global->LDS copy into one does not touch reads of the other
// and issues no wait for it.
__shared__ __align__(16) uint8_t f3_st0[kF3Tiles * kF2XTile];
__shared__ __align__(16) uint8_t f3_st1[kF3Tiles * kF2XTile];

// Copies block b of the work tile's activation tiles (xt[i], i < kF3Tiles)
// into a stage with direct global->LDS loads (1 KB per wave and load;
// chunk c of a tile by wave c % kF3Waves).  Branch-free: chunk indices past
// the end repeat the last whole chunk (the same bytes to the same place).
__device__ __forceinline__ void f3_xcopy(const uint8_t *const (&xt)[kF3Tiles], int b, uint8_t *stage, int wave,
                                         int lane) {
#pragma unroll
  for (int t = 0; t < kF3Tiles; t++) {
    const uint8_t *src = xt[t] + (size_t)b * kF2XTile;
    uint8_t *dst = stage + t * kF2XTile;
#pragma unroll
    for (int i = 0; i < (kF3Full + kF3Waves - 1) / kF3Waves; i++) {
      const int c = min(wave + i * kF3Waves, kF3Full - 1);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src + c * 1024 + 16 * lane),
                                       (__attribute__((address_space(3))) void *)(dst + c * 1024), 16, 0, 0);
    }
    if (wave == kF3Full % kF3Waves && 16 * lane < kF3Part)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src + kF3Full * 1024 + 16 * lane),
                                       (__attribute__((address_space(3))) void *)(dst + kF3Full * 1024), 16, 0, 0);
  }
}

// Blocks [b0, b1) of one tile for this wave's segments s0 .. s0 + kF3RS - 1
// of weight W (each clamped to the weight's last segment, and rows to its
// last row; their sums are never stored); xt is the column tile's activation
// tiles.  Loads are unconditional (the block index is clamped), so they never
// sit behind a branch; every copy has landed (vmcnt(0)) before the barrier
// that ends its block.
template <bool Q4, bool TILE>
__device__ __forceinline__ void f3_tile(float (&out)[kF3RS][kF3CS][4], const PfWeight &W, int nb, int S, int R,
                                        int s0, const uint8_t *const (&xt)[kF3Tiles], int b0, int b1) {
  if (b1 <= b0) return;  // (block ranges hold at least two blocks)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4;
  F3Row f[kF3RS] = {};
  if constexpr (TILE) {
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++)
      f[rs] = f3_row<Q4>(min(16 * min(s0 + rs, W.tiles - 1) + (lane & 15), W.rows - 1), W.rows, nb, S, R, q);
  }
  typename WSel<Q4>::T wa[kF3RS], wb[kF3RS];
  const uint32_t exp = magic_nib_exp();
  f3_xcopy(xt, b0, f3_st0, wave, lane);
  f3_wloads<Q4, TILE>(wa, W, f, s0, b0, S, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int b = b0;; b += 2) {
    const int bn = min(b + 1, b1 - 1);
    f3_xcopy(xt, bn, f3_st1, wave, lane);
    f3_wloads<Q4, TILE>(wb, W, f, s0, bn, S, lane);
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the block's compute
    f3_block<Q4, TILE>(out, wa, f3_st0, lane, exp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (b + 1 >= b1) break;
    const int bn2 = min(b + 2, b1 - 1);
    f3_xcopy(xt, bn2, f3_st0, wave, lane);
    f3_wloads<Q4, TILE>(wa, W, f, s0, bn2, S, lane);
    __builtin_amdgcn_sched_barrier(0);
    f3_block<Q4, TILE>(out, wb, f3_st1, lane, exp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (b + 2 >= b1) break;
  }
}

// Work index `it` of `total` -> its place in the (block range, row tile,
// column tile) order.  Workgroup i runs on XCD i % 8 and index it on
// workgroup it % gridDim.x, so within each round of gridDim.x indices every
// XCD takes a contiguous share of the order: the column tiles of one row tile
// share its weights in that XCD's L2.
__device__ __forceinline__ int f3_order(int it, int total) {
  const int G = gridDim.x, base = it - it % G, size = min(G, total - base), p = it - base;
  const int per = size / 8, rem = size % 8, x = p & 7, j = p >> 3;
  return base + (x < rem ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j);
}

constexpr int kF3WaveFloats = kF3RS * kF3CS * 4 * 64;  // a wave's sums (out) of one tile

// kF3PerCU workgroups per CU, kF3PerSIMD waves per SIMD in all.  PAIR: a tile is kF3Segs / 2 segments of gate (the first
// half of the waves) and the same rows of up (the second half); up's sums go
// through LDS to the gate wave of the same rows, which stores
// fround(gelu(gate) * up).  total_rt then counts those tiles, ksplit is 1.
// TILE: every weight is read from its tiles (a launch with a weight kept in
// one layout); else from its segments.
template <bool PAIR, bool TILE>
__global__ __launch_bounds__(kF3Threads) __attribute__((amdgpu_waves_per_eu(kF3PerSIMD, kF3PerSIMD))) void
kquant_prefill_fast_kernel(
    const F2Args a) {
  kernarg_warm<F2Args>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles = a.total_rt * a.col_tiles;
  const int items = tiles * a.ksplit;
  const int full = PAIR && a.tail_full > 0 ? a.tail_full : items;
  const int work = full + 2 * (items - full);  // trailing items as two block ranges each
  constexpr int kHalf = kF3Waves / 2;
  for (int it = blockIdx.x; it < work; it += gridDim.x) {
    const int nat0 = f3_order(it, work);
    const bool split = PAIR && nat0 >= full;
    const int hidx = nat0 - full;  // split: range hidx & 1 of item full + hidx / 2
    const int nat = split ? full + (hidx >> 1) : nat0;
    const int kr = nat / tiles, t2 = nat - kr * tiles;
    const int rt = t2 / a.col_tiles, ct = t2 - rt * a.col_tiles;
    int b_begin = (int)((long long)kr * a.nb / a.ksplit), b_end = (int)((long long)(kr + 1) * a.nb / a.ksplit);
    if (split) {
      b_begin = (hidx & 1) ? a.nb / 2 : 0;
      b_end = (hidx & 1) ? a.nb : a.nb / 2;
    }
    PfWeight W = a.w[0];
    size_t poff = a.part_off[0];
    if (!PAIR) {
      if (a.count > 1 && rt >= a.w[1].rt_begin) W = a.w[1], poff = a.part_off[1];
      if (a.count > 2 && rt >= a.w[2].rt_begin) W = a.w[2], poff = a.part_off[2];
      if (a.count > 3 && rt >= a.w[3].rt_begin) W = a.w[3], poff = a.part_off[3];
    }
    float *dst = a.ksplit > 1 ? a.part + kr * a.part_stride + poff : W.out;
    constexpr int kTileSegs = PAIR ? kF3Segs / 2 : kF3Segs;  // 16-row segments per weight and tile
    const int T0 = kTileSegs * (rt - W.rt_begin);
    const int nseg_tile = W.tiles - T0 < kTileSegs ? W.tiles - T0 : kTileSegs;
    const int my_seg = kF3RS * (PAIR ? wave % kHalf : wave);  // within this wave's weight
    const int nseg = nseg_tile - my_seg;                       // this wave's live segments (<= 0: none)
    const PfWeight &WW = PAIR && wave >= kHalf ? a.w[1] : W;  // the weight of this wave's rows
    float out[kF3RS][kF3CS][4];
#pragma unroll
    for (int rs = 0; rs < kF3RS; rs++)
#pragma unroll
      for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
        for (int j = 0; j < 4; j++) out[rs][cs][j] = 0.0f;
    // the work tile's 64-column activation tiles; one past the input's last
    // re-reads the last (its columns are never stored)
    const int xtiles = (a.cols + kF2Cols - 1) / kF2Cols;
    const uint8_t *xt[kF3Tiles];
#pragma unroll
    for (int t = 0; t < kF3Tiles; t++) xt[t] = a.xt + (size_t)min(ct * kF3Tiles + t, xtiles - 1) * a.nb * kF2XTile;
    if (W.type == kTypeQ4K)
      f3_tile<true, TILE>(out, WW, a.nb, a.S, a.R, T0 + my_seg, xt, b_begin, b_end);
    else
      f3_tile<false, TILE>(out, WW, a.nb, a.S, a.R, T0 + my_seg, xt, b_begin, b_end);
    const int n = lane & 15, q = lane >> 4;
    if (PAIR && split) {
      float *part = a.tail_part + ((size_t)hidx * kF3Waves + wave) * kF3WaveFloats + lane;
#pragma unroll
      for (int rs = 0; rs < kF3RS; rs++)
#pragma unroll
        for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
          for (int j = 0; j < 4; j++) part[((rs * kF3CS + cs) * 4 + j) * 64] = out[rs][cs][j];
    } else if (PAIR) {
      // up waves hand their sums to the gate wave of the same rows (the
      // stages are free: the tile's last barrier has passed)
      float *xch = reinterpret_cast<float *>(f3_st0) + (wave % kHalf) * kF3WaveFloats + lane;
      if (wave >= kHalf) {
#pragma unroll
        for (int rs = 0; rs < kF3RS; rs++)
#pragma unroll
          for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
            for (int j = 0; j < 4; j++) xch[((rs * kF3CS + cs) * 4 + j) * 64] = out[rs][cs][j];
      }
      __syncthreads();
      if (wave < kHalf && nseg > 0) {
#pragma unroll
        for (int rs = 0; rs < kF3RS; rs++) {
          const int row = 16 * (T0 + my_seg + rs) + n;
#pragma unroll
          for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const int m = ct * kF3Cols + 16 * cs + 4 * q + j;
              const float up = xch[((rs * kF3CS + cs) * 4 + j) * 64];
              if (rs < nseg && row < W.rows && m < a.cols)
                a.pair_out[(size_t)m * W.rows + row] = geglu_lut(out[rs][cs][j], up, a.gelu_lut);
            }
        }
      }
      __syncthreads();  // the next tile's first stage overwrites the exchange
    } else if (nseg > 0) {
#pragma unroll
      for (int rs = 0; rs < kF3RS; rs++) {
        const int row = 16 * (T0 + my_seg + rs) + n;
#pragma unroll
        for (int cs = 0; cs < kF3CS; cs++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int m = ct * kF3Cols + 16 * cs + 4 * q + j;
            if (rs < nseg && row < W.rows && m < a.cols) dst[(size_t)m * W.rows + row] = out[rs][cs][j];
          }
      }
    }
  }
}

// The gate/up items run as two block ranges (a.tail_full on): gate = range 0
// + range 1, up likewise, then fround(gelu(gate) * up).  One thread per
// output: (item, gate wave, sum index, lane), lane fastest.
__global__ __launch_bounds__(256) void f2_geglu_tail_kernel(const F2Args a, int rem) {
  kernarg_warm<F2Args>();
  constexpr int kHalf = kF3Waves / 2;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  constexpr int kSums = kF3RS * kF3CS * 4;  // a lane's sums
  const int lane = t & 63, k = (t >> 6) % kSums, w = (t >> 6) / kSums % kHalf;
  const int i = (t >> 6) / kSums / kHalf;
  if (i >= rem) return;
  const int rs = k / (kF3CS * 4), cs = (k >> 2) % kF3CS, j = k & 3;  // k = (rs * kF3CS + cs) * 4 + j
  const int nat = a.tail_full + i, rt = nat / a.col_tiles, ct = nat - rt * a.col_tiles;
  const PfWeight &W = a.w[0];
  constexpr int kTileSegs = kF3Segs / 2;
  const int T0 = kTileSegs * rt, my_seg = kF3RS * w;
  const int nseg = (W.tiles - T0 < kTileSegs ? W.tiles - T0 : kTileSegs) - my_seg;
  const int n = lane & 15, q = lane >> 4;
  const int row = 16 * (T0 + my_seg + rs) + n, m = ct * kF3Cols + 16 * cs + 4 * q + j;
  if (rs >= nseg || row >= W.rows || m >= a.cols) return;
  const float *p0 = a.tail_part + (size_t)(2 * i) * kF3Waves * kF3WaveFloats + k * 64 + lane;
  const float *p1 = p0 + (size_t)kF3Waves * kF3WaveFloats;
  const size_t gi = (size_t)w * kF3WaveFloats, ui = gi + (size_t)kHalf * kF3WaveFloats;
  a.pair_out[(size_t)m * W.rows + row] = geglu_lut(p0[gi] + p1[gi], p0[ui] + p1[ui], a.gelu_lut);
}

// The pre-pass (q8k_prefill_tiles16_kernel) of a launch whose input x is a
// gate/up + GeGLU output with its trailing tiles left as two block ranges'
// sums (GegluTail): lane i16 = 2j + u of a (block b, column m) row holds
// rows 256 b + 32 j + 8 c + 4 u + i (c, i < 4), all in gate/up row tile
// 2 b + j / 4; where that tile and column's item is a trailing one, the
// lane forms its 16 inputs as f2_geglu_tail_kernel does -- fround(gelu(g0 +
// g1) * (u0 + u1)) from the two ranges' gate and up sums -- else it loads
// them from x.  Same bits as the tail kernel followed by the plain pre-pass.
__global__ __launch_bounds__(256) void q8k_prefill_tiles16_tail_kernel(const float *__restrict__ x, int k, int nb,
                                                                       int cols, uint8_t *__restrict__ xt,
                                                                       const GegluTail t) {
  const int b = blockIdx.x, i16 = threadIdx.x & 15;
  const int m = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int ct = m / kF2Cols, n = m % kF2Cols;
  uint8_t *tile = xt + ((size_t)ct * nb + b) * kF2XTile;
  const int j = i16 >> 1, u = i16 & 1;
  const int nat = (2 * b + (j >> 2)) * t.col_tiles + m / kF3Cols;  // the gate/up item of these rows
  float v[16];
  if (m < cols && nat >= t.tail_full) {
    constexpr int kHalf = kF3Waves / 2;
    const int w = j & 3;  // gate wave of the rows; their segment rs = c / 2, row n = 8 (c % 2) + 4 u + i
    const int mm = m % kF3Cols, cs = mm >> 4, q = (mm & 15) >> 2, jj = mm & 3;
    const float *p0 = t.part + (size_t)(2 * (nat - t.tail_full)) * kF3Waves * kF3WaveFloats;
    const float *p1 = p0 + (size_t)kF3Waves * kF3WaveFloats;
    const size_t gi = (size_t)w * kF3WaveFloats, ui = gi + (size_t)kHalf * kF3WaveFloats;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int kk = ((c >> 1) * kF3CS + cs) * 4 + jj;          // the sum's index in its lane
      const size_t o = (size_t)kk * 64 + 8 * (c & 1) + 4 * u + 16 * q;  // lane n + 16 q, n = 8 (c % 2) + 4 u
      const float4 g0 = *reinterpret_cast<const float4 *>(p0 + gi + o);
      const float4 g1 = *reinterpret_cast<const float4 *>(p1 + gi + o);
      const float4 u0 = *reinterpret_cast<const float4 *>(p0 + ui + o);
      const float4 u1 = *reinterpret_cast<const float4 *>(p1 + ui + o);
      v[4 * c] = geglu_lut(g0.x + g1.x, u0.x + u1.x, t.gelu_lut);
      v[4 * c + 1] = geglu_lut(g0.y + g1.y, u0.y + u1.y, t.gelu_lut);
      v[4 * c + 2] = geglu_lut(g0.z + g1.z, u0.z + u1.z, t.gelu_lut);
      v[4 * c + 3] = geglu_lut(g0.w + g1.w, u0.w + u1.w, t.gelu_lut);
    }
  } else {
    load_x16(v, x + (size_t)min(m, cols - 1) * k + (size_t)b * kQK, i16);
    if (m >= cols) {
#pragma unroll
      for (int e = 0; e < 16; e++) v[e] = 0.0f;
    }
  }
  f2_tile_store16(v, i16, tile, n);
}

// out = ((part_0 + part_1) + ...) + part_{ks-1} over the launch's outputs
// (the weights' [cols][rows] outputs end to end), four floats per thread.
__global__ __launch_bounds__(256) void f2_reduce_kernel(const F2Args a, size_t total) {
  kernarg_warm<F2Args>();
  const size_t i = 4 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= total) return;
  int w = 0;
  if (a.count > 1 && i >= a.part_off[1]) w = 1;
  if (a.count > 2 && i >= a.part_off[2]) w = 2;
  if (a.count > 3 && i >= a.part_off[3]) w = 3;
  const size_t end = w + 1 < a.count ? a.part_off[w + 1] : total;
  float *out = a.w[w].out + (i - a.part_off[w]);
  if (i + 4 <= end && (((uintptr_t)out) & 15) == 0) {
    float4 acc = *reinterpret_cast<const float4 *>(a.part + i);
    for (int r = 1; r < a.ksplit; r++) {
      const float4 p = *reinterpret_cast<const float4 *>(a.part + r * a.part_stride + i);
      acc.x += p.x;
      acc.y += p.y;
      acc.z += p.z;
      acc.w += p.w;
    }
    *reinterpret_cast<float4 *>(out) = acc;
  } else {
    for (size_t e = i; e < i + 4 && e < total; e++) {
      int we = 0;
      if (a.count > 1 && e >= a.part_off[1]) we = 1;
      if (a.count > 2 && e >= a.part_off[2]) we = 2;
      if (a.count > 3 && e >= a.part_off[3]) we = 3;
      float acc = a.part[e];
      for (int r = 1; r < a.ksplit; r++) acc += a.part[r * a.part_stride + e];
      a.w[we].out[e - a.part_off[we]] = acc;
    }
  }
}

// Block ranges per tile: enough to give every workgroup slot a tile's worth
// of work when the launch has fewer tiles, at least two blocks a range.  One
// round rather than two: each range's partial sums cost a write and a read in
// the reduction (measured on the 42-layer chunk: O 20.8 -> 16.7 us, down
// 54.3 -> 50.8 us, against two rounds' worth).
int f2_ksplit(int tiles, int nb, int slots) {
  if (tiles <= 0 || tiles >= slots) return 1;
  int ks = slots / tiles;
  if (ks > nb / 2) ks = nb / 2;
  if (ks > 8) ks = 8;
  return ks < 1 ? 1 : ks;
}

struct F2Shape {
  int nb, col_tiles, xtiles, total_rt, ks;  // col_tiles of kF3Cols, xtiles of kF2Cols
  size_t outs;    // floats of all outputs
  size_t stride;  // floats between block ranges' partial sums (16-byte multiple)
};

F2Shape f2_shape(const MfmaLaunch &l, int num_cus) {
  F2Shape sh{};
  sh.nb = l.k / kQK;
  sh.col_tiles = (l.cols + kF3Cols - 1) / kF3Cols;
  sh.xtiles = (l.cols + kF2Cols - 1) / kF2Cols;
  for (int i = 0; i < l.count; i++) {
    sh.total_rt += ((l.rows[i] + 15) / 16 + kF3Segs - 1) / kF3Segs;
    sh.outs += (size_t)l.cols * l.rows[i];
  }
  sh.ks = f2_ksplit(sh.total_rt * sh.col_tiles, sh.nb, kF3PerCU * num_cus);
  sh.stride = (sh.outs + 3) & ~(size_t)3;
  return sh;
}

}  // namespace

size_t prefill_q8k_bytes(int k, int cols) {
  const size_t nb = (size_t)(k / kQK);
  return (size_t)cols * nb * (kQK + 32 + 4);
}

hipError_t launch_q8k_prefill(const float *x, int k, int cols, uint8_t *scratch, hipStream_t s) {
  const int nb = k / kQK;
  int8_t *xq = reinterpret_cast<int8_t *>(scratch);
  _Float16 *xb = reinterpret_cast<_Float16 *>(scratch + (size_t)cols * nb * kQK);
  float *xd = reinterpret_cast<float *>(scratch + (size_t)cols * nb * (kQK + 32));
  hipLaunchKernelGGL(q8k_prefill_kernel, dim3(nb, cols), dim3(64), 0, s, x, k, nb, xq, xb, xd);
  return hipGetLastError();
}

size_t prefill_lds_bytes() { return kPfLds; }

// gate/up launch shape: the workgroup tiles (128 rows of each weight x 64
// columns), the grid, and where the trailing items start when fewer than
// half a round of them remain (0: none split).
struct F2Pair {
  int nb, col_tiles, xtiles, total_rt, items, grid, tail_full;  // col_tiles of kF3Cols, xtiles of kF2Cols
};

F2Pair f2_pair(const MfmaLaunch &l, int num_cus) {
  F2Pair p{};
  p.nb = l.k / kQK;
  p.col_tiles = (l.cols + kF3Cols - 1) / kF3Cols;
  p.xtiles = (l.cols + kF2Cols - 1) / kF2Cols;
  p.total_rt = ((l.rows[0] + 15) / 16 + kF3Segs / 2 - 1) / (kF3Segs / 2);
  p.items = p.total_rt * p.col_tiles;
  p.grid = p.items < kF3PerCU * num_cus ? p.items : kF3PerCU * num_cus;
  const int full = p.items / p.grid * p.grid, rem = p.items - full;
  p.tail_full = rem > 0 && 2 * rem <= p.grid && p.nb >= 2 ? full : 0;
  return p;
}

int prefill_fast_geglu_launches(const MfmaLaunch &l, int num_cus) { return f2_pair(l, num_cus).tail_full ? 3 : 2; }

size_t prefill_fast_geglu_tail_bytes(const MfmaLaunch &l, int num_cus) {
  const F2Pair p = f2_pair(l, num_cus);
  return p.tail_full ? (size_t)2 * (p.items - p.tail_full) * kF3Waves * kF3WaveFloats * sizeof(float) : 0;
}

size_t prefill_fast_geglu_bytes(const MfmaLaunch &l, int num_cus) {
  const F2Pair p = f2_pair(l, num_cus);
  const size_t xt = (size_t)p.xtiles * p.nb * kF2XTile;
  const size_t tail = p.tail_full ? (size_t)2 * (p.items - p.tail_full) * kF3Waves * kF3WaveFloats * sizeof(float) : 0;
  return xt + tail;
}

hipError_t launch_prefill_fast_geglu(const MfmaLaunch &l, const float *x, uint8_t *scratch, const uint16_t *gelu_lut,
                                     float *out, int num_cus, hipStream_t s, bool tiles_ready, GegluTail *defer,
                                     float *tail_part) {
  if (l.count != 2 || l.cols < 1 || l.k % kQK != 0 || l.type[0] != l.type[1] || l.rows[0] != l.rows[1] ||
      !mfma_geometry_ok(l))
    return hipErrorInvalidValue;
  const F2Pair p = f2_pair(l, num_cus);
  const int nb = p.nb, col_tiles = p.col_tiles;
  hipError_t e;
  if (!tiles_ready) {
    hipLaunchKernelGGL(q8k_prefill_tiles16_kernel, dim3(nb, p.xtiles * kF2Cols / 16), dim3(256), 0, s, x, l.k, nb,
                       l.cols, scratch);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  F2Args a{};
  a.count = 2;
  for (int i = 0; i < 2; i++) {
    a.w[i].seg = l.seg[i];
    a.w[i].wt = l.wt[i];
    a.w[i].dplane = l.dplane[i];
    a.w[i].out = nullptr;
    a.w[i].type = l.type[i];
    a.w[i].rows = l.rows[i];
    a.w[i].tiles = (l.rows[i] + 15) / 16;
    a.w[i].rt_begin = 0;
  }
  a.total_rt = p.total_rt;
  a.col_tiles = col_tiles;
  a.nb = nb;
  a.S = l.S;
  a.R = l.R;
  a.cols = l.cols;
  a.xt = scratch;
  a.ksplit = 1;
  a.pair_out = out;
  a.gelu_lut = gelu_lut;
  a.tail_full = p.tail_full;
  a.tail_part = defer && tail_part ? tail_part : reinterpret_cast<float *>(scratch + (size_t)p.xtiles * nb * kF2XTile);
  if (defer) *defer = GegluTail{};
  if (launch_reads_tiles(l))
    hipLaunchKernelGGL((kquant_prefill_fast_kernel<true, true>), dim3(p.grid), dim3(kF3Threads), 0, s, a);
  else
    hipLaunchKernelGGL((kquant_prefill_fast_kernel<true, false>), dim3(p.grid), dim3(kF3Threads), 0, s, a);
  if (!p.tail_full) return hipGetLastError();
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (defer && tail_part) {
    // the next launch's pre-pass adds the trailing tiles' ranges
    *defer = GegluTail{tail_part, gelu_lut, p.tail_full, col_tiles};
    return hipSuccess;
  }
  const int rem = p.items - p.tail_full, threads = rem * (kF3Waves / 2) * kF3WaveFloats;
  hipLaunchKernelGGL(f2_geglu_tail_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, a, rem);
  return hipGetLastError();
}

int prefill_fast_launches(const MfmaLaunch &l, int num_cus) { return f2_shape(l, num_cus).ks > 1 ? 3 : 2; }

size_t prefill_fast_bytes(const MfmaLaunch &l, int num_cus) {
  const F2Shape sh = f2_shape(l, num_cus);
  const size_t xt = (size_t)sh.xtiles * sh.nb * kF2XTile;
  return xt + (sh.ks > 1 ? (size_t)sh.ks * sh.stride * sizeof(float) : 0);
}

size_t prefill_fast_lds_bytes() { return 2 * (size_t)kF3Tiles * kF2XTile; }  // the two static stages

size_t prefill_fast_part_bytes(const MfmaLaunch &l, int num_cus) {
  const F2Shape sh = f2_shape(l, num_cus);
  return sh.ks > 1 && sh.ks <= kNormParts ? (size_t)sh.ks * sh.stride * sizeof(float) : 0;
}

hipError_t launch_prefill_fast(const MfmaLaunch &l, const float *x, uint8_t *scratch, int num_cus, hipStream_t s,
                               bool tiles_ready, PrefillParts *defer, const GegluTail *tail) {
  if (l.count < 1 || l.count > kMaxWeights || l.cols < 1 || l.k % kQK != 0 || !mfma_geometry_ok(l))
    return hipErrorInvalidValue;
  const bool tail_in = tail && tail->part;
  if (tail_in && (tiles_ready || tail->col_tiles != (l.cols + kF3Cols - 1) / kF3Cols || !tail->gelu_lut))
    return hipErrorInvalidValue;
  const F2Shape sh = f2_shape(l, num_cus);
  const int nb = sh.nb, col_tiles = sh.col_tiles;
  hipError_t e;
  if (tail_in) {
    hipLaunchKernelGGL(q8k_prefill_tiles16_tail_kernel, dim3(nb, sh.xtiles * kF2Cols / 16), dim3(256), 0, s, x, l.k,
                       nb, l.cols, scratch, *tail);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  } else if (!tiles_ready) {
    hipLaunchKernelGGL(q8k_prefill_tiles16_kernel, dim3(nb, sh.xtiles * kF2Cols / 16), dim3(256), 0, s, x, l.k, nb,
                       l.cols, scratch);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  F2Args a{};
  a.count = l.count;
  int rt = 0;
  size_t off = 0;
  for (int i = 0; i < l.count; i++) {
    a.w[i].seg = l.seg[i];
    a.w[i].wt = l.wt[i];
    a.w[i].dplane = l.dplane[i];
    a.w[i].out = l.out[i];
    a.w[i].type = l.type[i];
    a.w[i].rows = l.rows[i];
    a.w[i].tiles = (l.rows[i] + 15) / 16;
    a.w[i].rt_begin = rt;
    rt += (a.w[i].tiles + kF3Segs - 1) / kF3Segs;
    a.part_off[i] = off;
    off += (size_t)l.cols * l.rows[i];
  }
  a.total_rt = rt;
  a.col_tiles = col_tiles;
  a.nb = nb;
  a.S = l.S;
  a.R = l.R;
  a.cols = l.cols;
  a.xt = scratch;
  a.ksplit = sh.ks;
  a.part = reinterpret_cast<float *>(scratch + (size_t)sh.xtiles * nb * kF2XTile);
  a.part_stride = sh.stride;
  const bool deferred = defer && prefill_fast_part_bytes(l, num_cus) > 0;
  if (defer) {
    defer->ks = deferred ? sh.ks : 1;
    defer->stride = sh.stride;
    for (int i = 0; i < l.count; i++) defer->off[i] = a.part_off[i];
    if (deferred) a.part = defer->part;
  }
  const long long items = (long long)a.total_rt * a.col_tiles * a.ksplit;
  const int grid = (int)(items < kF3PerCU * num_cus ? items : kF3PerCU * num_cus);
  if (launch_reads_tiles(l))
    hipLaunchKernelGGL((kquant_prefill_fast_kernel<false, true>), dim3(grid), dim3(kF3Threads), 0, s, a);
  else
    hipLaunchKernelGGL((kquant_prefill_fast_kernel<false, false>), dim3(grid), dim3(kF3Threads), 0, s, a);
  if (a.ksplit == 1 || deferred) return hipGetLastError();
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t threads = (sh.outs + 3) / 4;
  hipLaunchKernelGGL(f2_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a, sh.outs);
  return hipGetLastError();
}

hipError_t launch_prefill(const MfmaLaunch &l, const uint8_t *scratch, int num_cus, hipStream_t s) {
  if (l.count < 1 || l.count > kMaxWeights || l.cols < 1 || l.k % kQK != 0 || !mfma_geometry_ok(l))
    return hipErrorInvalidValue;
  PfArgs a{};
  a.count = l.count;
  int rt = 0;
  for (int i = 0; i < l.count; i++) {
    a.w[i].seg = l.seg[i];
    a.w[i].wt = l.wt[i];
    a.w[i].dplane = l.dplane[i];
    a.w[i].out = l.out[i];
    a.w[i].type = l.type[i];
    a.w[i].rows = l.rows[i];
    a.w[i].tiles = (l.rows[i] + 15) / 16;
    a.w[i].rt_begin = rt;
    rt += (a.w[i].tiles + 1) / 2;
  }
  a.total_rt = rt;
  a.nb = l.k / kQK;
  a.S = l.S;
  a.R = l.R;
  a.cols = l.cols;
  a.col_tiles = (l.cols + kPfCols - 1) / kPfCols;
  a.xq = reinterpret_cast<const int8_t *>(scratch);
  a.xb = reinterpret_cast<const _Float16 *>(scratch + (size_t)l.cols * a.nb * kQK);
  a.xd = reinterpret_cast<const float *>(scratch + (size_t)l.cols * a.nb * (kQK + 32));
  const long long items = (long long)a.total_rt * a.col_tiles;
  const int grid = (int)(items < (long long)num_cus * 2 ? items : (long long)num_cus * 2);
  if (launch_reads_tiles(l))
    hipLaunchKernelGGL(kquant_prefill_kernel<true>, dim3(grid), dim3(256), kPfLds, s, a);
  else
    hipLaunchKernelGGL(kquant_prefill_kernel<false>, dim3(grid), dim3(256), kPfLds, s, a);
  return hipGetLastError();
}

}  // namespace hp
