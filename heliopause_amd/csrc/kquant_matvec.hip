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
// (row, block) with v_dot4_i32_i8 on four elements that share lane l.  The
// scale sum sum_j sc_j * dot_j is formed by Abel summation: one running
// dot T_j = dot_0 + .. + dot_j per lane l and aux += T_j * (sc_j - sc_{j+1}),
// so each (j, l) costs one dot4 and one 24-bit multiply-add.  The lane then
// forms the f32 products d*f32(aux32[l]); the order-dependent additions run
// across the S lanes of a row with DPP wave_shr:1: at step k lane k adds its
// product to lane k-1's running value, which is the reference's sequential
// block order.  Each workgroup first quantises the f32 input to Q8_K into
// LDS (16 lanes per 256-element block), so a projection is one launch.
#include "hp_common.h"
#include "hp_gelu.h"
#include "hp_q8k.h"
#include "hp_wave.h"
#include "hp_q8k16.h"
#include "hp_kquant.h"

namespace hp {


template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

constexpr int kDppWaveShr1 = 0x138;    // wave_shr:1


// Wave-uniform context of one tile.
struct TileCtx {
  const uint8_t *tile;
  const uint16_t *dpl;
  float *out;
  int rows, row0, Rt, lanes, CH;
  bool q4;
};

// TYPE: kTypeQ4K or kTypeQ6K when every weight of the launch has that type
// (then the type tests fold away), 0 for a mixed launch.
template <int TYPE>
__device__ __forceinline__ TileCtx make_ctx(const MatvecArgs &a, int t, int nb, int R, int S) {
  WeightDesc W = a.w[0];
  if (a.count > 1 && t >= a.w[1].tile_begin) W = a.w[1];
  if (a.count > 2 && t >= a.w[2].tile_begin) W = a.w[2];
  if (a.count > 3 && t >= a.w[3].tile_begin) W = a.w[3];
  TileCtx cx;
  cx.q4 = TYPE == kTypeQ4K ? true : TYPE == kTypeQ6K ? false : W.type == kTypeQ4K;
  cx.CH = cx.q4 ? 9 : 13;
  cx.rows = W.rows;
  cx.row0 = (t - W.tile_begin) * R;
  cx.Rt = min(R, W.rows - cx.row0);
  cx.lanes = cx.Rt * S;
  cx.tile = W.data + (size_t)cx.row0 * nb * cx.CH * 16;
  cx.dpl = W.dplane;
  cx.out = W.out;
  return cx;
}

// lane < cx.lanes: no bounds check.  In a mixed launch (TYPE 0) a Q4_K
// block issues 9 loads and a Q6_K block 14, so a wait for loads issued
// before these also waits for the first 5 of a Q6_K block's: the price of
// mixing types in one launch.
template <int TYPE>
__device__ __forceinline__ void load_regs_from(Regs &rg, const TileCtx &cx, int it, int lane, int nb) {
  const uint4 *ch = reinterpret_cast<const uint4 *>(cx.tile + ((size_t)it * cx.CH * cx.lanes + lane) * 16);
#pragma unroll
  for (int c = 0; c < 9; c++) rg.c[c] = ch[(size_t)c * cx.lanes];
  if (!cx.q4) {
#pragma unroll
    for (int c = 9; c < 13; c++) rg.c[c] = ch[(size_t)c * cx.lanes];
    rg.d6 = cx.dpl[(size_t)cx.row0 * nb + (size_t)it * cx.lanes + lane];
  }
}

template <int TYPE>
__device__ __forceinline__ void load_regs(Regs &rg, const TileCtx &cx, int it, int lane, int nb) {
  if (lane < cx.lanes) load_regs_from<TYPE>(rg, cx, it, lane, nb);
}

// lane L receives lane L-1's value (DPP wave_shr:1).
__device__ __forceinline__ float shr1(float v) {
  return dppf<kDppWaveShr1>(v);
}

// PAIR: gate/up + GeGLU (layers.ts:435-456).  Weight 0 is gate, weight 1 up,
// with equal row counts; a wave takes gate tile p and then up tile p, which
// cover the same rows, so the lane that finishes row r's gate sum keeps it
// and, after the up pass, writes fround(gelu(gate) * up) to a.pair_out.
template <int M, bool PREFETCH, bool PAIR, int NORM, int TYPE>
__global__ __launch_bounds__(256) void kquant_matvec_kernel(const MatvecArgs a) {
  // the argument lines in one round trip (measured: two Q4_K 10240 x 2560
  // in one launch 11.1 -> 10.8 us; the head unchanged)
  kernarg_warm<MatvecArgs>();
  extern __shared__ __align__(16) uint8_t smem[];
  const TileGeom g = a.g;
  const int nb = g.nb, S = g.S, R = g.R;
  uint8_t *xq = smem;
  float *xd = reinterpret_cast<float *>(smem + (size_t)M * nb * kQ8BlockBytes);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wpg = blockDim.x >> 6;
  const int stride = gridDim.x * wpg;
  const int r = lane / S;
  const int s = lane - r * S;

  // prologue inputs first (vector loads return in order), then the first
  // weight unit, so the weights stream in while the prologue computes
  const int grp = wave * 4 + (lane >> 4);
  const int i16 = lane & 15;
  const int nq = M * nb;
  float xv[16], xv2[16], xv3[16];  // the blocks of this group's first three passes
  __shared__ double norm_sh[8];  // two workgroup sums
  NormRegs nr;
  auto x_block = [&](int q) { return a.x + (size_t)(q / nb) * a.k + (size_t)(q % nb) * kQK; };
  // two or more columns may come already quantised (a.q8img): the image
  // is copied in place of the Q8_K passes
  const bool pre = M >= 2 && a.q8img != nullptr;
  if (NORM) {
    norm_load<NORM>(a.norm, nr, grp, nb, i16);
  } else if (!pre) {
    // every pass's input before the weights: vector loads return in order,
    // so a pass loaded after them would wait for the weights
    if (grp < nq) load_x16(xv, x_block(grp), i16);
    if (grp + wpg * 4 < nq) load_x16(xv2, x_block(grp + wpg * 4), i16);
    if (grp + wpg * 8 < nq) load_x16(xv3, x_block(grp + wpg * 8), i16);
  }

  // the i-th tile of this wave (-1: none); with PAIR, gate then up tile
  const int t0 = blockIdx.x * wpg + wave;
  auto tile_of = [&](int i) -> int {
    if (!PAIR) {
      const int tt = t0 + i * stride;
      return tt < a.total_tiles ? tt : -1;
    }
    const int p = t0 + (i >> 1) * stride;
    return p < a.w[0].tiles ? p + (i & 1) * a.w[0].tiles : -1;
  };
  int ti = 0;
  int t = tile_of(0);
  // unconditional first loads (an idle wave reads the last tile, an idle lane
  // its tile's last lane): a path that skipped them would make the
  // prologue's first wait on its input a wait on every load
  TileCtx cx = make_ctx<TYPE>(a, t >= 0 ? t : PAIR ? 2 * a.w[0].tiles - 1 : a.total_tiles - 1, nb, R, S);
  Regs cur;
  load_regs_from<TYPE>(cur, cx, 0, min(lane, cx.lanes - 1), nb);
  __builtin_amdgcn_sched_barrier(0);  // keep the prologue's work after the weight loads
  if (NORM) norm_finish<NORM>(a.norm, nr, xv, grp, nb, i16, a.k, norm_sh);

  if (pre) {
    const int n16 = (int)(q8_image_bytes(M, nb) / 16);
    const uint4 *src = reinterpret_cast<const uint4 *>(a.q8img);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) reinterpret_cast<uint4 *>(smem)[i] = src[i];
  } else {
    int q = grp;
    if (q < nq) q8k_block16(xv, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    q += wpg * 4;
    if (q < nq) q8k_block16(xv2, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    q += wpg * 4;
    if (q < nq) q8k_block16(xv3, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    for (q += wpg * 4; q < nq; q += wpg * 4) {  // more than three passes (several columns)
      load_x16(xv, x_block(q), i16);
      q8k_block16(xv, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    }
  }
  __syncthreads();

  float carry[M][9];
  float gkeep[M];  // PAIR: this lane's gate results
  while (t >= 0) {
    for (int it = 0; it < g.iters; it++) {
      Regs nxt;
      if (PREFETCH) {
        int nt = t, nit = it + 1;
        TileCtx ncx = cx;
        if (nit == g.iters) {
          nt = tile_of(ti + 1);
          nit = 0;
          if (nt >= 0) ncx = make_ctx<TYPE>(a, nt, nb, R, S);
        }
        // every iteration loads (the wave's last block re-reads itself): an
        // iteration without these loads would make the wait below for the
        // current block a wait for the next one too
        if (nt < 0) nit = it;
        load_regs_from<TYPE>(nxt, ncx, nit, min(lane, ncx.lanes - 1), nb);
        __builtin_amdgcn_sched_barrier(0);  // the current block's work after the next block's loads
      }
      const int b = it * S + s;
      const bool active = lane < cx.lanes;
      int aux[M][8];
      int sumi[M];
      float dw = 0.0f, dminw = 0.0f;
      if (active) {
        if (cx.q4) {
          q4k_ints<M>(cur, xq, nb, b, aux, sumi);
          dw = h2f(cur.c[0].x & 0xFFFFu);
          dminw = h2f(cur.c[0].x >> 16);
        } else {
          q6k_ints<M>(cur, xq, nb, b, aux);
          dw = h2f(cur.d6);
#pragma unroll
          for (int m = 0; m < M; m++) sumi[m] = 0;
        }
      } else {
#pragma unroll
        for (int m = 0; m < M; m++) {
          sumi[m] = 0;
#pragma unroll
          for (int l = 0; l < 8; l++) aux[m][l] = 0;
        }
      }
      const bool last = it + 1 == g.iters;
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float dx = xd[m * nb + (b < nb ? b : 0)];
        const float dd = __fmul_rn(dw, dx);
        float p[9];
#pragma unroll
        for (int l = 0; l < 8; l++) p[l] = __fmul_rn(dd, (float)aux[m][l]);
        p[8] = __fmul_rn(__fmul_rn(dminw, dx), (float)sumi[m]);
        // step 0 (slot 0): chain start = previous iteration's value, or 0
        float v[9];
#pragma unroll
        for (int c = 0; c < 8; c++) v[c] = __fadd_rn(it == 0 ? 0.0f : carry[m][c], p[c]);
        v[8] = __fsub_rn(it == 0 ? 0.0f : carry[m][8], p[8]);
        // steps 1..S-1: lane k adds its product to lane k-1's value
        for (int k = 1; k < S; k++) {
#pragma unroll
          for (int c = 0; c < 8; c++) v[c] = __fadd_rn(shr1(v[c]), p[c]);
          v[8] = __fsub_rn(shr1(v[8]), p[8]);
        }
        if (!last) {
          // lane (r, 0) continues from lane (r, S-1)
          const int src = (r * S + S - 1) << 2;
#pragma unroll
          for (int c = 0; c < 9; c++)
            carry[m][c] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v[c])));
        } else if (active && s == S - 1) {
          // result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
          float tsum = -0.0f;
#pragma unroll
          for (int l = 0; l < 8; l++) tsum = __fadd_rn(tsum, v[l]);
          const float res = cx.q4 ? __fadd_rn(v[8], tsum) : tsum;
          if (!PAIR)
            cx.out[(size_t)(a.out_col0 + m) * cx.rows + cx.row0 + r] = res;
          else if ((ti & 1) == 0)
            gkeep[m] = res;
          else
            a.pair_out[(size_t)(a.out_col0 + m) * cx.rows + cx.row0 + r] = geglu_lut(gkeep[m], res, a.gelu_lut);
        }
      }
      if (PREFETCH) {
        cur = nxt;
      } else if (!last) {
        load_regs<TYPE>(cur, cx, it + 1, lane, nb);
      }
    }
    t = tile_of(++ti);
    if (t >= 0) {
      cx = make_ctx<TYPE>(a, t, nb, R, S);
      if (!PREFETCH) load_regs<TYPE>(cur, cx, 0, lane, nb);
    }
  }
}

// ---------------------------------------------------------------------------
// Half-split variant: two lanes per (row, block).  Lane (rr, h, s) =
// lane (2 rr + h) * S + s handles lane classes l = 4h .. 4h+3 of row
// row0 + rr, block it * S + s: it loads chunk 0 and the nibble (Q4_K) or
// nibble / high-bit (Q6_K) chunks of its classes only, forms aux32 of its four
// classes, and chains four sums (h = 0 also sumf) across the S block lanes
// in block order.  The h = 0 lane then takes its partner's four sums
// (ds_bpermute) and finishes ((((-0 + s0) + ...) + s7), the reference's
// order.  Each row-block costs each lane half the integer work and the chain
// carries 5 values instead of 9; units of Rh = 32 / S rows make twice as
// many waves as the full kernel, which fills the CUs on small projections.
// Lanes address the tile layout (hp_common.h) from their own row, so a unit
// may span two tiles.

template <int M, int NORM, int TYPE>
__global__ __launch_bounds__(256) void kquant_matvec_half_kernel(const MatvecArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  // the argument lines in one round trip (measured: Q/K/V 5.89 -> 5.37 us)
  kernarg_warm<MatvecArgs>();
  const TileGeom g = a.g;
  const int nb = g.nb, S = g.S, R = g.R, Rh = a.Rh;
  uint8_t *xq = smem;
  float *xd = reinterpret_cast<float *>(smem + (size_t)M * nb * kQ8BlockBytes);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpg = blockDim.x >> 6;
  const int stride = gridDim.x * wpg;
  const int grp2 = mdiv(lane, a.mg_S);  // 2 rr + h (lane / S)
  const int rr = grp2 >> 1, h = grp2 & 1;
  const int s = lane - grp2 * S;

  // unit u: rows u * Rh .. u * Rh + Rh - 1 of the launch (the weights' rows
  // end to end, so a unit may span two weights and the units fill the grid
  // without a partial unit per weight); this lane's weight, row, tile and
  // chunk index
  struct Unit {
    WeightDesc W;
    bool q4, active;
    int CH, row, t, Rt, k;
    const uint8_t *tile;
  };
  // An idle lane addresses a launch row that exists (the unit's last, or the
  // launch's last for u >= total_units), so its loads need no branch
  auto unit_of = [&](int u) {
    Unit n;
    const int grow = u * Rh + rr;
    n.active = u < a.total_units && rr < Rh && grow < a.total_rows;
    const int arow = n.active ? grow : min(min(u, a.total_units - 1) * Rh + min(rr, Rh - 1), a.total_rows - 1);
    n.W = a.w[0];
    if (a.count > 1 && arow >= a.w[1].row_begin) n.W = a.w[1];
    if (a.count > 2 && arow >= a.w[2].row_begin) n.W = a.w[2];
    if (a.count > 3 && arow >= a.w[3].row_begin) n.W = a.w[3];
    n.q4 = TYPE == kTypeQ4K ? true : TYPE == kTypeQ6K ? false : n.W.type == kTypeQ4K;
    n.CH = n.q4 ? 9 : 13;
    n.row = arow - n.W.row_begin;
    n.t = mdiv(n.row, a.mg_R);  // n.row / R
    n.Rt = min(R, n.W.rows - n.t * R);
    n.k = (n.row - n.t * R) * S + s;
    n.tile = n.W.data + (size_t)n.t * R * nb * n.CH * 16;
    return n;
  };
  // No branch on the type: a Q4_K unit issues 5 loads, a Q6_K unit 8; in a
  // mixed launch (TYPE 0) a Q4_K unit also issues the 3 Q6_K-only loads at
  // its chunk 0, so both paths leave the same count in flight and a wait for
  // an earlier load never waits for these.
  auto load_unit = [&](HalfRegs &rg, const Unit &n, int it) {
    const uint4 *ch = reinterpret_cast<const uint4 *>(n.tile + ((size_t)it * n.CH * n.Rt * S + n.k) * 16);
    const size_t cs = (size_t)n.Rt * S;  // uint4 stride between chunks
    rg.c0 = ch[(n.q4 ? 0 : 12) * cs];
#pragma unroll
    for (int p = 0; p < 4; p++) rg.d[p] = ch[(n.q4 ? 1 + 2 * p + h : 2 * p + h) * cs];
    if (TYPE == kTypeQ4K) return;
#pragma unroll
    for (int p = 0; p < 2; p++) rg.e[p] = ch[(n.q4 ? 0 : 8 + 2 * p + h) * cs];
    const uint16_t *dp = n.q4 ? reinterpret_cast<const uint16_t *>(ch)
                              : n.W.dplane + (size_t)n.t * R * nb + (size_t)it * n.Rt * S + n.k;
    rg.d6 = *dp;
  };

  // prologue inputs of up to three passes first, then the first unit's first
  // block (vector loads return in order), so the weights stream in while the
  // prologue computes
  const int grp = wave * 4 + (lane >> 4);
  const int i16 = lane & 15;
  const int nq = M * nb;
  float xv[16], xv2[16], xv3[16];
  __shared__ double norm_sh[8];  // two workgroup sums
  NormRegs nr;
  // block q of the columns' input (one column: block q itself)
  auto x_block = [&](int q) {
    if (M == 1) return a.x + (size_t)q * kQK;
    const int col = mdiv(q, a.mg_nb);
    return a.x + (size_t)col * a.k + (size_t)(q - col * nb) * kQK;
  };
  // two or more columns may come already quantised (a.q8img): the image
  // is copied in place of the Q8_K passes
  const bool pre = M >= 2 && a.q8img != nullptr;
  if (NORM) {
    norm_load<NORM>(a.norm, nr, grp, nb, i16);
  } else if (!pre) {
    if (grp < nq) load_x16(xv, x_block(grp), i16);
    if (grp + wpg * 4 < nq) load_x16(xv2, x_block(grp + wpg * 4), i16);
    if (grp + wpg * 8 < nq) load_x16(xv3, x_block(grp + wpg * 8), i16);
  }
  // unconditional loads: a path that skipped them would make the prologue's
  // first wait on its input a wait on every load
  const int u0 = blockIdx.x * wpg + wave;
  HalfRegs first;
  const Unit un0 = unit_of(u0);
  load_unit(first, un0, 0);
  __builtin_amdgcn_sched_barrier(0);  // keep the prologue's work after the weight loads
  if (NORM) norm_finish<NORM>(a.norm, nr, xv, grp, nb, i16, a.k, norm_sh);
  if (pre) {
    const int n16 = (int)(q8_image_bytes(M, nb) / 16);
    const uint4 *src = reinterpret_cast<const uint4 *>(a.q8img);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) reinterpret_cast<uint4 *>(smem)[i] = src[i];
  } else {
    int q = grp;
    if (q < nq) q8k_block16(xv, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    q += wpg * 4;
    if (q < nq) q8k_block16(xv2, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    q += wpg * 4;
    if (q < nq) q8k_block16(xv3, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    for (q += wpg * 4; q < nq; q += wpg * 4) {  // more than three passes (several columns)
      load_x16(xv, x_block(q), i16);
      q8k_block16(xv, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    }
  }
  __syncthreads();

  float carry[M][5];
  for (int u = u0; u < a.total_units; u += stride) {
    const Unit un = u == u0 ? un0 : unit_of(u);
    const WeightDesc &W = un.W;
    const bool q4 = un.q4, active = un.active;
    const int row = un.row;
    for (int it = 0; it < g.iters; it++) {
      HalfRegs rg;
      if (u == u0 && it == 0)
        rg = first;
      else if (active)
        load_unit(rg, un, it);
      const int b = it * S + s;
      int aux[M][4];
      int sumi[M];
      float dw = 0.0f, dminw = 0.0f;
      if (active) {
        if (q4) {
          q4k_ints_half<M>(rg, xq, nb, b, h, aux, sumi);
          dw = h2f(rg.c0.x & 0xFFFFu);
          dminw = h2f(rg.c0.x >> 16);
        } else {
          q6k_ints_half<M>(rg, xq, nb, b, h, aux);
          dw = h2f(rg.d6);
#pragma unroll
          for (int m = 0; m < M; m++) sumi[m] = 0;
        }
      } else {
#pragma unroll
        for (int m = 0; m < M; m++) {
          sumi[m] = 0;
#pragma unroll
          for (int l = 0; l < 4; l++) aux[m][l] = 0;
        }
      }
      const bool last = it + 1 == g.iters;
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float dx = xd[m * nb + (b < nb ? b : 0)];
        const float dd = __fmul_rn(dw, dx);
        float p[5];
#pragma unroll
        for (int l = 0; l < 4; l++) p[l] = __fmul_rn(dd, (float)aux[m][l]);
        p[4] = __fmul_rn(__fmul_rn(dminw, dx), (float)sumi[m]);
        float v[5];
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = __fadd_rn(it == 0 ? 0.0f : carry[m][c], p[c]);
        v[4] = __fsub_rn(it == 0 ? 0.0f : carry[m][4], p[4]);
        for (int kk = 1; kk < S; kk++) {
#pragma unroll
          for (int c = 0; c < 4; c++) v[c] = __fadd_rn(shr1(v[c]), p[c]);
          v[4] = __fsub_rn(shr1(v[4]), p[4]);
        }
        if (!last) {
          // lane (rr, h, 0) continues from lane (rr, h, S-1)
          const int src = (grp2 * S + S - 1) << 2;
#pragma unroll
          for (int c = 0; c < 5; c++)
            carry[m][c] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v[c])));
        } else {
          // lane (rr, 0, S-1) takes classes 4..7 from lane (rr, 1, S-1)
          const int partner = (lane + S < 64 ? lane + S : lane) << 2;
          float o[4];
#pragma unroll
          for (int c = 0; c < 4; c++)
            o[c] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(partner, __builtin_bit_cast(int, v[c])));
          if (active && h == 0 && s == S - 1) {
            // result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
            float tsum = -0.0f;
#pragma unroll
            for (int l = 0; l < 4; l++) tsum = __fadd_rn(tsum, v[l]);
#pragma unroll
            for (int l = 0; l < 4; l++) tsum = __fadd_rn(tsum, o[l]);
            const float res = q4 ? __fadd_rn(v[4], tsum) : tsum;
            W.out[(size_t)(a.out_col0 + m) * W.rows + row] = res;
          }
        }
      }
    }
  }
}

// The weight type shared by every weight of the launch, or 0.
static int uniform_type(const MatvecArgs &a) {
  for (int i = 1; i < a.count; i++)
    if (a.w[i].type != a.w[0].type) return 0;
  return a.w[0].type == kTypeQ4K || a.w[0].type == kTypeQ6K ? a.w[0].type : 0;
}

template <int M, int NORM>
static void launch_half_typed(const MatvecArgs &a, dim3 grid, size_t lds, hipStream_t s) {
  const int t = uniform_type(a);
  if (t == kTypeQ4K)
    hipLaunchKernelGGL((kquant_matvec_half_kernel<M, NORM, kTypeQ4K>), grid, dim3(256), lds, s, a);
  else if (t == kTypeQ6K)
    hipLaunchKernelGGL((kquant_matvec_half_kernel<M, NORM, kTypeQ6K>), grid, dim3(256), lds, s, a);
  else
    hipLaunchKernelGGL((kquant_matvec_half_kernel<M, NORM, 0>), grid, dim3(256), lds, s, a);
}

static size_t matvec_lds_bytes(int cols, const TileGeom &g, int wpg) {
  (void)wpg;
  return (size_t)cols * g.nb * kQ8BlockBytes + (size_t)((cols * g.nb + 3) & ~3) * 4;
}


template <int M, bool PAIR, int NORM>
static void launch_typed(const MatvecArgs &a, dim3 grid, size_t lds, hipStream_t s) {
  constexpr bool PF = M <= 3;
  const int t = PF ? uniform_type(a) : 0;
  if (t == kTypeQ4K)
    hipLaunchKernelGGL((kquant_matvec_kernel<M, PF, PAIR, NORM, (PF ? kTypeQ4K : 0)>), grid, dim3(256), lds, s, a);
  else if (t == kTypeQ6K)
    hipLaunchKernelGGL((kquant_matvec_kernel<M, PF, PAIR, NORM, (PF ? kTypeQ6K : 0)>), grid, dim3(256), lds, s, a);
  else
    hipLaunchKernelGGL((kquant_matvec_kernel<M, PF, PAIR, NORM, 0>), grid, dim3(256), lds, s, a);
}

template <int M, bool PAIR>
static void launch_full(const MatvecArgs &a, dim3 grid, size_t lds, hipStream_t s) {
  if (M == 1 && a.norm.mode == 1)
    launch_typed<1, PAIR, 1>(a, grid, lds, s);
  else if (M == 1 && a.norm.mode == 2)
    launch_typed<1, PAIR, 2>(a, grid, lds, s);
  else
    launch_typed<M, PAIR, 0>(a, grid, lds, s);
}

template <int M>
static hipError_t launch_m(const MatvecArgs &a, int num_cus, hipStream_t s) {
  const int wpg = 4;
  int grid = (a.total_tiles + wpg - 1) / wpg;
  const int cap = num_cus * 8;
  if (grid > cap) grid = cap;
  launch_full<M, false>(a, dim3(grid), matvec_lds_bytes(M, a.g, wpg), s);
  return hipGetLastError();
}

template <int M>
static hipError_t launch_half_m(const MatvecArgs &a, int num_cus, hipStream_t s) {
  const int wpg = 4;
  int grid = (a.total_units + wpg - 1) / wpg;
  const int cap = num_cus * 8;
  if (grid > cap) grid = cap;
  const size_t lds = matvec_lds_bytes(M, a.g, wpg);
  if (M == 1 && a.norm.mode == 1)
    launch_half_typed<1, 1>(a, dim3(grid), lds, s);
  else if (M == 1 && a.norm.mode == 2)
    launch_half_typed<1, 2>(a, dim3(grid), lds, s);
  else
    launch_half_typed<M, 0>(a, dim3(grid), lds, s);
  return hipGetLastError();
}

hipError_t launch_matvec_half(const MatvecArgs &args, int num_cus, hipStream_t s) {
  if (args.q8img && (args.cols < 2 || args.norm.mode != 0)) return hipErrorInvalidValue;
  if (args.norm.mode < 0 || args.norm.mode > 2 || (args.norm.mode != 0 && (args.cols != 1 || args.g.nb > 16)))
    return hipErrorInvalidValue;
  if (args.g.S > 32 || args.Rh < 1 || 2 * args.Rh * args.g.S > 64) return hipErrorInvalidValue;
  // divisions by S, R and nb as high multiplies (mdiv: dividends below 2^20)
  if (args.total_rows >= (1 << 20) || args.cols * args.g.nb >= (1 << 20) || args.g.nb > 256)
    return hipErrorInvalidValue;
  MatvecArgs a = args;
  a.mg_nb = div_magic(a.g.nb);
  a.mg_S = div_magic(a.g.S);
  a.mg_R = div_magic(a.g.R);
  switch (a.cols) {
    case 1: return launch_half_m<1>(a, num_cus, s);
    case 2: return launch_half_m<2>(a, num_cus, s);
    case 3: return launch_half_m<3>(a, num_cus, s);
    case 4: return launch_half_m<4>(a, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

template <int M>
static hipError_t launch_pair_m(const MatvecArgs &a, int num_cus, hipStream_t s) {
  const int wpg = 4;
  int grid = (a.w[0].tiles + wpg - 1) / wpg;
  const int cap = num_cus * 8;
  if (grid > cap) grid = cap;
  launch_full<M, true>(a, dim3(grid), matvec_lds_bytes(M, a.g, wpg), s);
  return hipGetLastError();
}

hipError_t launch_matvec_pair(const MatvecArgs &a, int num_cus, hipStream_t s) {
  if (a.q8img) return hipErrorInvalidValue;
  if (a.norm.mode < 0 || a.norm.mode > 2 || (a.norm.mode != 0 && (a.cols != 1 || a.g.nb > 16)))
    return hipErrorInvalidValue;
  if (a.count != 2 || a.w[0].rows != a.w[1].rows || a.w[0].tiles != a.w[1].tiles || !a.pair_out)
    return hipErrorInvalidValue;
  switch (a.cols) {
    case 1: return launch_pair_m<1>(a, num_cus, s);
    case 2: return launch_pair_m<2>(a, num_cus, s);
    case 3: return launch_pair_m<3>(a, num_cus, s);
    case 4: return launch_pair_m<4>(a, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_matvec(const MatvecArgs &a, int num_cus, hipStream_t s) {
  if (a.q8img && (a.cols < 2 || a.norm.mode != 0)) return hipErrorInvalidValue;
  if (a.norm.mode < 0 || a.norm.mode > 2 || (a.norm.mode != 0 && (a.cols != 1 || a.g.nb > 16)))
    return hipErrorInvalidValue;
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
