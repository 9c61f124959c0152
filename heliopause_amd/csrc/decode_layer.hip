// decode_layer.hip -- the non-projection steps of one decoder layer for one
// decode token (forwardAttentionLayer, packages/engine/src/runner/wasm/
// layers.ts:161-379, and forwardFfn, 418-473): RMSNorms fused with the
// residual adds and the layer output scale, the per-head q/k/v norms with
// RoPE and the KV-cache append, and GQA decode attention over an f16 KV ring.
// The projections between them are the runner's matvec launches.
//
// The decode position is read from device memory (one int32), so a captured
// graph of a step can be replayed for every position.
//
// Reference steps and how they are evaluated here:
//   rmsNormVector (layers.ts:871-885): sum of squares in f64, scale =
//     1 / sqrt(sum / n + eps), out = f32((x * scale) * w) with the products
//     in f64; rmsNormRowsNoWeight (834-849): out = f32(x * scale);
//   residualAdd (851-860): f32(a + b); layer output scale (364-369):
//     f32(x * scale);
//   ropeNeox (990-1033): theta_0 = position, theta_{i+1} = f32(theta_i *
//     base^(-2/nDims)), angle theta_i / freq_factor_i, cos and sin in f64,
//     out = f32(f32(x0 * cos) - f32(x1 * sin)) and f32(f32(x0 * sin) +
//     f32(x1 * cos)) for the pair (i, i + nDims/2);
//   hp_gqa_attention_f32 (packages/engine/wasm-kernels/src/lib.rs:538-654):
//     query rounded to f16 with float32_to_float16 (lib.rs:2534-2568: round
//     half up in magnitude, saturating at 65504), scores q.k (scale 1, no
//     mask within the window), p = f32(exp(f64(score - max))), out =
//     sum(p / sum(p) * v); castF16Rows of the output (layers.ts:982-988,
//     round to nearest even).
// The sums (f64 sum of squares, f32 dot products, softmax sums) are tree or
// chunked sums here where the reference sums in index order, so results
// agree within a tolerance rather than bit for bit.
//
// KV cache: f16 keys and values, [kv head][slot][head_dim], slot = position
// % capacity, entries rounded to nearest even.  The attention window is the
// last count = min(capacity, window, position + 1) positions
// (attentionRange, layers.ts:972-980).
#include "hp_common.h"
#include "hp_gelu.h"
#include "hp_wave.h"
#include "hp_q8k16.h"
#include "hp_attn.h"
#include "hp_f2tile.h"

namespace hp {

namespace {

constexpr int kNormPer = 16;  // elements per thread of the 256-thread norm: n <= 4096

// Sum over the 256 threads of the workgroup (every thread gets the total).
// Sum over the workgroup's four waves; sh (4 doubles) must not have been
// used by an earlier call in the kernel (no barrier guards its reuse).
__device__ __forceinline__ double block_sum_f64(double v, double *sh) {
  v = wave_sum_f64(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

template <int NPER>
__device__ __forceinline__ double rms_scale(const float (&v)[NPER], int n, double eps, double *sh) {
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < NPER; j++) s += (double)v[j] * (double)v[j];  // exact squares; padding is 0
  const double total = block_sum_f64(s, sh);
  return 1.0 / sqrt(total / (double)n + eps);
}

// 256 threads per row (element i of thread t: i = t + 256 j, j < NPER; the
// launch takes the smallest instance with 256 NPER >= n, which keeps the
// clamped re-reads of the row's last element few; a larger NPER only adds
// zeros at the end of each thread's sum and gives the same bits).
//   x_res == null:  next_out = rmsnorm(y) * w_next
//   otherwise:      x1 = f32(f32(x_res + rmsnorm(y) * w_post) * scale) -> x_out
//                   and, if next_out, next_out = rmsnorm(x1) * w_next.
// Workgroup r handles row r of [rows][n].  w_post / w_next null: the norm
// has no weight (rmsNormRowsNoWeight).
template <int NPER>
__global__ __launch_bounds__(256) void norm_residual_kernel(const NormArgs a) {
  __shared__ double sh[8];  // two workgroup sums
  const int tid = threadIdx.x;
  if (a.xt && (int)blockIdx.x >= a.rows) {
    // a padding column of the last activation tile: zero blocks, as the
    // prefill pre-pass writes them
    const int g = tid >> 4, i16 = tid & 15, nb = a.n / kQK;
    float z[16];
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    for (int b = g; b < nb; b += 16)
      f2_tile_store16(z, i16, a.xt + ((size_t)(blockIdx.x / kF2Cols) * nb + b) * kF2XTile, blockIdx.x % kF2Cols);
    return;
  }
  const size_t row = (size_t)blockIdx.x * a.n;
  // every input first, one memory round trip: the loads take no branch
  // (indexes past n re-read element n - 1, absent operands re-read y), so
  // none of them waits for another
  float v[NPER], r[NPER], wp[NPER], wn[NPER];
  const float *py = a.y + row;
  const float *pr = a.x_res ? a.x_res + row : py;
  const float *pwp = a.w_post ? a.w_post : py;
  const float *pwn = a.w_next ? a.w_next : py;
#pragma unroll
  for (int j = 0; j < NPER; j++) {
    const int ic = min(tid + 256 * j, a.n - 1);
    v[j] = py[ic];
    r[j] = pr[ic];
    wp[j] = pwp[ic];
    wn[j] = pwn[ic];
  }
  if (a.y_ks > 1) {
    // y as block-range partial sums: every range's loads first, then the
    // sums in range order
    float pv[kNormParts - 1][NPER];
#pragma unroll
    for (int r = 1; r < kNormParts; r++)
#pragma unroll
      for (int j = 0; j < NPER; j++) {
        const int ic = min(tid + 256 * j, a.n - 1);
        pv[r - 1][j] = r < a.y_ks ? py[r * a.y_stride + ic] : 0.0f;
      }
#pragma unroll
    for (int r = 1; r < kNormParts; r++)
#pragma unroll
      for (int j = 0; j < NPER; j++)
        if (r < a.y_ks) v[j] += pv[r - 1][j];
  }
#pragma unroll
  for (int j = 0; j < NPER; j++) {
    const bool in = tid + 256 * j < a.n;
    v[j] = in ? v[j] : 0.0f;
    r[j] = in && a.x_res ? r[j] : 0.0f;
    wp[j] = in && a.w_post ? wp[j] : 1.0f;
    wn[j] = in && a.w_next ? wn[j] : 1.0f;
  }
  if (a.x_res) {
    const double sc = rms_scale(v, a.n, a.eps, sh);
#pragma unroll
    for (int j = 0; j < NPER; j++) {
      const int i = tid + 256 * j;
      const float t = a.w_post ? (float)(((double)v[j] * sc) * (double)wp[j]) : (float)((double)v[j] * sc);
      v[j] = i < a.n ? (r[j] + t) * a.scale : 0.0f;
      if (i < a.n) a.x_out[row + i] = v[j];
    }
  }
  if (a.next_out) {
    const double sc = rms_scale(v, a.n, a.eps, sh + 4);
    __shared__ float xs[256 * NPER];  // the row, for the image below
#pragma unroll
    for (int j = 0; j < NPER; j++) {
      const int i = tid + 256 * j;
      const float o = a.w_next ? (float)(((double)v[j] * sc) * (double)wn[j]) : (float)((double)v[j] * sc);
      if (i < a.n && !a.next_image_only) a.next_out[row + i] = o;
      if (a.q8img || a.xt) xs[i] = o;
    }
    if (a.q8img || a.xt) {
      // the row as Q8_K blocks (n a multiple of 256) of a matvec input
      // image, or of the fast prefill's activation tiles (column blockIdx.x):
      // 16-lane group g quantises blocks g, g + 16, ...
      __syncthreads();
      const int g = tid >> 4, i16 = tid & 15, nb = a.n / kQK;
      for (int b = g; b < nb; b += 16) {
        float xv[16];
        const int jj = i16 >> 1, u = i16 & 1;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
          for (int i = 0; i < 4; i++) xv[4 * c + i] = xs[b * kQK + 32 * jj + 8 * c + 4 * u + i];
        if (a.q8img) {
          const size_t q = (size_t)blockIdx.x * nb + b;
          q8k_block16(xv, i16, a.q8img + q * kQ8BlockBytes,
                      reinterpret_cast<float *>(a.q8img + (size_t)a.rows * nb * kQ8BlockBytes) + q);
        }
        if (a.xt)
          f2_tile_store16(xv, i16, a.xt + ((size_t)(blockIdx.x / kF2Cols) * nb + b) * kF2XTile,
                          blockIdx.x % kF2Cols);
      }
    }
  }
}

// The same norm for the rows that feed a projection (NormArgs::x16; n a
// multiple of 256, at most 16 blocks), which may leave as Q8_K blocks (a
// matvec input image or the fast prefill's activation tiles): 16-lane group
// g holds block g in load_x16's element order from the loads on, so each
// block is quantised from registers (no pass through LDS) and every operand
// moves in 16-byte loads and stores.  Per element the arithmetic is
// norm_residual_kernel's; the f64 sums of squares add in this layout's
// order (a lane's 16, then the wave's DPP tree, then the four waves), the
// same with or without the image or tiles.
__global__ __launch_bounds__(256) void norm_residual_x16_kernel(const NormArgs a) {
  __shared__ double sh[8];  // two workgroup sums
  const int tid = threadIdx.x, g = tid >> 4, i16 = tid & 15, nb = a.n / kQK;
  if (a.xt && (int)blockIdx.x >= a.rows) {
    // a padding column of the last activation tile: zero blocks, as the
    // prefill pre-pass writes them
    float z[16];
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    if (g < nb)
      f2_tile_store16(z, i16, a.xt + ((size_t)(blockIdx.x / kF2Cols) * nb + g) * kF2XTile, blockIdx.x % kF2Cols);
    return;
  }
  const bool live = g < nb;
  // every input first, one memory round trip; groups past the row's blocks
  // re-read its last block (zeroed below), absent operands re-read y
  const size_t row = (size_t)blockIdx.x * a.n, boff = (size_t)min(g, nb - 1) * kQK;
  const float *py = a.y + row + boff;
  float v[16], r[16], wp[16], wn[16];
  load_x16(v, py, i16);
  load_x16(r, a.x_res ? a.x_res + row + boff : py, i16);
  load_x16(wp, a.w_post ? a.w_post + boff : py, i16);
  load_x16(wn, a.w_next ? a.w_next + boff : py, i16);
  if (a.y_ks > 1) {
    float pv[kNormParts - 1][16];
#pragma unroll
    for (int k = 1; k < kNormParts; k++) load_x16(pv[k - 1], k < a.y_ks ? py + k * a.y_stride : py, i16);
#pragma unroll
    for (int k = 1; k < kNormParts; k++)
#pragma unroll
      for (int e = 0; e < 16; e++)
        if (k < a.y_ks) v[e] += pv[k - 1][e];
  }
#pragma unroll
  for (int e = 0; e < 16; e++) {
    v[e] = live ? v[e] : 0.0f;
    r[e] = live && a.x_res ? r[e] : 0.0f;
    wp[e] = a.w_post ? wp[e] : 1.0f;
    wn[e] = a.w_next ? wn[e] : 1.0f;
  }
  if (a.x_res) {
    const double sc = rms_scale<16>(v, a.n, a.eps, sh);
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float t = a.w_post ? (float)(((double)v[e] * sc) * (double)wp[e]) : (float)((double)v[e] * sc);
      v[e] = live ? (r[e] + t) * a.scale : 0.0f;
    }
    if (live) store_x16(a.x_out + row + (size_t)g * kQK, v, i16);
  }
  const double sc = rms_scale<16>(v, a.n, a.eps, sh + 4);
  float o[16];
#pragma unroll
  for (int e = 0; e < 16; e++)
    o[e] = a.w_next ? (float)(((double)v[e] * sc) * (double)wn[e]) : (float)((double)v[e] * sc);
  if (!live) return;
  if (!a.next_image_only) store_x16(a.next_out + row + (size_t)g * kQK, o, i16);
  if (a.q8img) {
    const size_t q = (size_t)blockIdx.x * nb + g;
    q8k_block16(o, i16, a.q8img + q * kQ8BlockBytes,
                reinterpret_cast<float *>(a.q8img + (size_t)a.rows * nb * kQ8BlockBytes) + q);
  }
  if (a.xt)
    f2_tile_store16(o, i16, a.xt + ((size_t)(blockIdx.x / kF2Cols) * nb + g) * kF2XTile, blockIdx.x % kF2Cols);
}

// One wave per head: query heads (norm with wq, RoPE, f32 out or its f16
// rounding for the prefill attention), key heads
// (norm with wk, RoPE, f16 into the key cache) and value heads (norm without
// weight, f16 into the value cache).
__global__ __launch_bounds__(64) void qkv_post_kernel(const QkvPostArgs a) {
  __shared__ float xs[kHeadDim];
  const int h = blockIdx.x, lane = threadIdx.x;
  int kind, head;  // kind 0 query, 1 key, 2 value
  if (h < a.nq) {
    kind = 0;
    head = h;
  } else if (h < a.nq + a.nkv) {
    kind = 1;
    head = h - a.nq;
  } else {
    kind = 2;
    head = h - a.nq - a.nkv;
  }
  const int t = blockIdx.y;  // token: position *a.position + a.pos_offset + t
  const size_t qrow = (size_t)t * a.nq, kvrow = (size_t)t * a.nkv;
  const float *src = kind == 0 ? a.q + (qrow + head) * kHeadDim
                               : (kind == 1 ? a.k : a.v) + (kvrow + head) * kHeadDim;
  const float *w = kind == 0 ? a.wq : kind == 1 ? a.wk : nullptr;
  const int half = a.rope_dims >> 1;
  // every load first, none in a branch (an absent weight re-reads the row)
  float x[4], wv[4];
  const float *pw = w ? w : src;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    x[j] = src[lane + 64 * j];
    wv[j] = pw[lane + 64 * j];
  }
  if (a.src_ks > 1) {
    // the projection as block-range partial sums: every range's loads, then
    // the sums in range order
    float pv[kNormParts - 1][4];
#pragma unroll
    for (int r = 1; r < kNormParts; r++)
#pragma unroll
      for (int j = 0; j < 4; j++) pv[r - 1][j] = r < a.src_ks ? src[r * a.src_stride + lane + 64 * j] : 0.0f;
#pragma unroll
    for (int r = 1; r < kNormParts; r++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (r < a.src_ks) x[j] += pv[r - 1][j];
  }
  double2 tab[2] = {make_double2(1.0, 0.0), make_double2(1.0, 0.0)};
  if (a.rope_table_mode == 2 && kind != 2 && half > 0) {
#pragma unroll
    for (int p = 0; p < 2; p++) tab[p] = a.rope_table[t * (kHeadDim / 2) + min(lane + 64 * p, half - 1)];
  }
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < 4; j++) s += (double)x[j] * (double)x[j];
  const double sc = 1.0 / sqrt(wave_sum_f64(s) / (double)kHeadDim + a.eps);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int i = lane + 64 * j;
    xs[i] = w ? (float)(((double)x[j] * sc) * (double)wv[j]) : (float)((double)x[j] * sc);
  }
  __syncthreads();
  const int pos = *a.position + a.pos_offset + t;
  if (kind != 2) {
    float r0[2], r1[2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int i = lane + 64 * p;
      r0[p] = r1[p] = 0.0f;
      if (i < half) {
        double c, sn;
        if (a.rope_table_mode == 2) {
          c = tab[p].x;
          sn = tab[p].y;
        } else {
          double theta = (double)pos;
          for (int it = 0; it < i; it++) theta = (double)(float)(theta * a.theta_scale);
          const double ang = a.freq_factors ? theta / (double)a.freq_factors[i] : theta;
          sincos(ang, &sn, &c);
          if (a.rope_table_mode == 1 && h == 0) a.rope_table[t * (kHeadDim / 2) + i] = make_double2(c, sn);
        }
        const double x0 = xs[i], x1 = xs[i + half];
        r0[p] = (float)(x0 * c) - (float)(x1 * sn);
        r1[p] = (float)(x0 * sn) + (float)(x1 * c);
      }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int i = lane + 64 * p;
      if (i < half) {
        xs[i] = r0[p];
        xs[i + half] = r1[p];
      }
    }
    __syncthreads();
  }
  if (kind == 0) {
    if (a.q_half) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        a.q_half[(qrow + head) * kHeadDim + lane + 64 * j] =
            (uint16_t)rs_f16_bits(__builtin_bit_cast(uint32_t, xs[lane + 64 * j]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) a.q_out[(qrow + head) * kHeadDim + lane + 64 * j] = xs[lane + 64 * j];
    }
  } else if (pos >= 0) {  // a negative position (invalid) writes no cache entry
    const int slot = pos % a.capacity;
    _Float16 *dst = (kind == 1 ? a.k_cache : a.v_cache) + ((size_t)head * a.capacity + slot) * kHeadDim;
#pragma unroll
    for (int j = 0; j < 4; j++) dst[lane + 64 * j] = (_Float16)xs[lane + 64 * j];
  }
}

// Attention partials: workgroup (chunk c, kv head g, part hs) takes the cache
// slots [32 c, 32 c + 32) -- those inside the token's window -- for G of the
// group's query heads, G (nq / nkv) / a.qsplit of them from head hs G on (the
// parts of one chunk share its keys through the L2 and each keeps a shorter
// chain; every head's arithmetic is the same either way).  Softmax and the
// weighted sum do not depend on the order of the keys, so the chunks follow
// slots and the loads need no position.
// With a.prep it first computes, from the projections, the group's queries
// (norm, RoPE) and the token's own key (norm, RoPE) and value (norm); the
// workgroup whose slots hold position % capacity appends them to the caches,
// and uses them in place of the rows it read.  Then the chunk's scores, their
// maximum m and sum l of exp(score - m) (m = -inf, l = 0 for a chunk with no
// slot in the window), and the exp-weighted value sums.
//   loads, in this order (vector loads return in order): the projection rows
//   and norm weights, the RoPE table, then K (thread t: slot t / 8, dims
//   8 (8 i + t % 8) .. + 7 for i < 4; a wave reads 128 contiguous bytes of 8
//   rows per load) and V (wave w: slots 8 w .. 8 w + 7, lane l dims 4 l ..
//   4 l + 3; one 512-byte row per load).
//   prep: each wave normalises and rotates its own rows; lane l holds
//   elements l + 64 j, so for rope_dims 128 or 256 the RoPE pairs (i,
//   i + rope_dims / 2) sit in one lane and need no exchange.
// RoPE angles: a.rope_table_mode 0 computes them, 1 also stores them to
// a.rope_table (workgroup (0, 0)), 2 reads them from there (a later layer
// with the same RoPE parameters at the same position).
template <int G>
__global__ __launch_bounds__(256) void attn_partial_kernel(const AttnArgs a) {
  __shared__ float xs[G + 2][kHeadDim];       // queries, then the new key and value
  __shared__ float sc[G][kAttnChunk];         // scores, then exp(score - m)
  __shared__ float4 red[4][G][kHeadDim / 4];  // per-wave value sums
  const int c = blockIdx.x, g = blockIdx.y / a.qsplit, hs = blockIdx.y - g * a.qsplit, tid = threadIdx.x;
  const int qh0 = (g * a.qsplit + hs) * G;  // the first query head of this workgroup
  const int wave = tid >> 6, lane = tid & 63;
  const int cap = a.capacity;
  const size_t head_base = (size_t)g * cap * kHeadDim;
  const int half = a.rope_dims >> 1;
  const bool lane_pairs = (half & 63) == 0;  // half in {0, 64, 128}

  constexpr int kRows = (G + 2 + 3) / 4;  // rows per wave: queries, key, value
  float px[kRows][4], pw[kRows][4];
  double2 tab[2] = {make_double2(1.0, 0.0), make_double2(1.0, 0.0)};
  // Loads take no branch on a lane or wave (rows past the last re-read it,
  // absent weights re-read the row, slots past the capacity re-read the last
  // slot; what they bring is masked later): a path that skipped loads would
  // make the compiler's first wait on an early load a wait on every load.
  if (a.prep) {
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++) {
      const int r = min(wave + 4 * k3, G + 1);
      const float *src = r < G ? a.q + (size_t)(qh0 + r) * kHeadDim : (r == G ? a.k : a.v) + (size_t)g * kHeadDim;
      const float *w = r < G ? a.wq : (r == G ? a.wk : nullptr);
      const float *pwr = w ? w : src;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        px[k3][j] = src[lane + 64 * j];
        pw[k3][j] = pwr[lane + 64 * j];
      }
    }
    if (a.rope_table_mode == 2 && lane_pairs && half > 0) {
#pragma unroll
      for (int p = 0; p < 2; p++) tab[p] = a.rope_table[min(lane + 64 * p, half - 1)];
    }
  }
  const int kj = tid >> 3, kp = tid & 7;
  const int kslot = c * kAttnChunk + kj;
  uint4 kraw[4];
  {
    const _Float16 *kr = a.k_cache + head_base + (size_t)min(kslot, cap - 1) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 4; i++) kraw[i] = *reinterpret_cast<const uint4 *>(kr + 8 * (8 * i + kp));
  }
  const int vslot0 = c * kAttnChunk + 8 * wave;
  uint2 vraw[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
    vraw[j] = *reinterpret_cast<const uint2 *>(a.v_cache + head_base + (size_t)min(vslot0 + j, cap - 1) * kHeadDim +
                                               4 * lane);
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the prologue's first use of one

  // tokens at *a.position .. + a.tokens - 1 share the window of the last
  // (attentionRange of the largest position); token blockIdx.z sees the keys
  // up to its own position (causalMask).  Read after the cache loads are
  // issued (they take slots, not positions): a scalar read of device memory
  // placed before them made them wait for its round trip.
  const int tok = blockIdx.z;
  const int pos = *a.position + a.pos_offset + (a.tokens - 1);
  const int pos_t = pos - (a.tokens - 1) + tok;

  int start, count;
  window_of(pos, cap, a.window, &start, &count);
  const int s0 = pos < 0 ? 0 : start % cap;
  const int last_w = pos_t - start;  // window index of the token's own position
  auto in_window = [&](int slot) {
    int w = slot - s0;  // window index of the slot (both in [0, cap))
    w += w < 0 ? cap : 0;
    return pos >= 0 && slot < cap && w < count && w <= last_w;
  };
  const int new_slot = pos < 0 ? -1 : pos % cap;

  if (a.prep) {
    if (!lane_pairs || a.rope_table_mode != 2) {
      // angles of pairs lane and lane + 64: theta_0 = pos, theta_{i+1} = f32(theta_i * scale)
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const int i = lane + 64 * p;
        if (lane_pairs && i < half) {
          double theta = (double)pos;
          for (int it = 0; it < i; it++) theta = (double)(float)(theta * a.theta_scale);
          const double ang = a.freq_factors ? theta / (double)a.freq_factors[i] : theta;
          double sn, cn;
          sincos(ang, &sn, &cn);
          tab[p] = make_double2(cn, sn);
          if (a.rope_table_mode == 1 && c == 0 && blockIdx.y == 0 && wave == 0) a.rope_table[i] = tab[p];
        }
      }
    }
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++) {
      const int r = wave + 4 * k3;
      if (r < G + 2) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 4; j++) ss += (double)px[k3][j] * (double)px[k3][j];
        const double scl = 1.0 / sqrt(wave_sum_f64(ss) / (double)kHeadDim + a.eps);
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
          x[j] = r <= G && (r < G ? a.wq : a.wk) ? (float)(((double)px[k3][j] * scl) * (double)pw[k3][j])
                                                   : (float)((double)px[k3][j] * scl);
        if (r <= G && lane_pairs) {
          const int hj = half >> 6;  // pair (j, j + hj) for j < hj
#pragma unroll
          for (int j = 0; j < 2; j++) {
            if (j < hj) {
              const double x0 = x[j], x1 = x[j + hj];
              const double cc = tab[j].x, sn = tab[j].y;
              x[j] = (float)(x0 * cc) - (float)(x1 * sn);
              x[j + hj] = (float)(x0 * sn) + (float)(x1 * cc);
            }
          }
        }
        // queries as the scorer rounds them; the new key and value as the
        // cache stores them (other RoPE widths: after the pass over LDS)
#pragma unroll
        for (int j = 0; j < 4; j++)
          xs[r][lane + 64 * j] = !lane_pairs ? x[j] : r < G ? rs_f16_round(x[j]) : (float)(_Float16)x[j];
      }
    }
    __syncthreads();
    if (!lane_pairs) {
      // RoPE over LDS for other widths: thread per (row, pair)
      for (int idx = tid; idx < (G + 1) * half; idx += 256) {
        const int r = idx / half, i = idx - r * half;
        double theta = (double)pos;
        for (int it = 0; it < i; it++) theta = (double)(float)(theta * a.theta_scale);
        const double ang = a.freq_factors ? theta / (double)a.freq_factors[i] : theta;
        double sn, cn;
        sincos(ang, &sn, &cn);
        const double x0 = xs[r][i], x1 = xs[r][i + half];
        xs[r][i] = (float)(x0 * cn) - (float)(x1 * sn);
        xs[r][i + half] = (float)(x0 * sn) + (float)(x1 * cn);
      }
      __syncthreads();
      for (int idx = tid; idx < (G + 2) * kHeadDim; idx += 256) {
        const int r = idx >> 8, i = idx & 255;
        const float v = xs[r][i];
        xs[r][i] = r < G ? rs_f16_round(v) : (float)(_Float16)v;
      }
      __syncthreads();
    }
    if (new_slot >= 0 && new_slot / kAttnChunk == c && hs == 0) {
      const size_t o = head_base + (size_t)new_slot * kHeadDim + tid;
      a.k_cache[o] = (_Float16)xs[G][tid];
      a.v_cache[o] = (_Float16)xs[G + 1][tid];
    }
  } else {
    for (int idx = tid; idx < G * kHeadDim; idx += 256)
      xs[idx >> 8][idx & 255] = rs_f16_round(a.q[((size_t)tok * a.nq + qh0) * kHeadDim + idx]);
    __syncthreads();
  }

  // scores (the token's own key from LDS)
  const bool kvalid = in_window(kslot);
  if (a.prep && kslot == new_slot) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 lo = *reinterpret_cast<const float4 *>(&xs[G][8 * (8 * i + kp)]);
      const float4 hi = *reinterpret_cast<const float4 *>(&xs[G][8 * (8 * i + kp) + 4]);
      kraw[i] = make_uint4(pack2_f16(lo.x, lo.y), pack2_f16(lo.z, lo.w), pack2_f16(hi.x, hi.y),
                           pack2_f16(hi.z, hi.w));
    }
  }
  float dot[G];
#pragma unroll
  for (int h = 0; h < G; h++) dot[h] = 0.0f;
  if (kvalid) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int d0 = 8 * (8 * i + kp);
      const _Float16 *k8 = reinterpret_cast<const _Float16 *>(&kraw[i]);
      float kf[8];
#pragma unroll
      for (int e = 0; e < 8; e++) kf[e] = (float)k8[e];
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float4 qa = *reinterpret_cast<const float4 *>(&xs[h][d0]);
        const float4 qb = *reinterpret_cast<const float4 *>(&xs[h][d0 + 4]);
        float t = dot[h];
        t = __builtin_fmaf(qa.x, kf[0], t);
        t = __builtin_fmaf(qa.y, kf[1], t);
        t = __builtin_fmaf(qa.z, kf[2], t);
        t = __builtin_fmaf(qa.w, kf[3], t);
        t = __builtin_fmaf(qb.x, kf[4], t);
        t = __builtin_fmaf(qb.y, kf[5], t);
        t = __builtin_fmaf(qb.z, kf[6], t);
        t = __builtin_fmaf(qb.w, kf[7], t);
        dot[h] = t;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float t = oct_sum_f32(dot[h]);
    if (kp == 0) sc[h][kj] = kvalid ? t : -__builtin_inff();
  }
  __syncthreads();
  // softmax within the chunk: half-wave hw = tid / 32 takes query head hw
  {
    const int h = tid >> 5, j = tid & 31;
    if (h < G) {
      const float sv = sc[h][j];
      float m = fmaxf(sv, dpp_f32<kDppXor1>(sv));
      m = fmaxf(m, dpp_f32<kDppXor2>(m));
      m = fmaxf(m, dpp_f32<kDppRowHalfMirror>(m));
      m = fmaxf(m, dpp_f32<kDppRowMirror>(m));
      m = fmaxf(m, __shfl_xor(m, 16));
      const float p = sv == -__builtin_inff() ? 0.0f : (float)exp((double)(sv - m));
      float l = p + dpp_f32<kDppXor1>(p);
      l += dpp_f32<kDppXor2>(l);
      l += dpp_f32<kDppRowHalfMirror>(l);
      l += dpp_f32<kDppRowMirror>(l);
      l += __shfl_xor(l, 16);
      sc[h][j] = p;
      if (j == 0) {
        const size_t base = (((size_t)tok * a.nkv + g) * a.chunks + c) * kAttnMaxGroup + hs * G + h;
        a.part_m[base] = m;
        a.part_l[base] = l;
      }
    }
  }
  __syncthreads();
  // exp-weighted values (the token's own value from LDS)
  if (a.prep && new_slot >= vslot0 && new_slot < vslot0 + 8) {
    const float4 nvv = *reinterpret_cast<const float4 *>(&xs[G + 1][4 * lane]);
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (vslot0 + j == new_slot) vraw[j] = make_uint2(pack2_f16(nvv.x, nvv.y), pack2_f16(nvv.z, nvv.w));
  }
  float4 acc[G];
#pragma unroll
  for (int h = 0; h < G; h++) acc[h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    if (in_window(vslot0 + j)) {
      const _Float16 *v4 = reinterpret_cast<const _Float16 *>(&vraw[j]);
      const float f0 = (float)v4[0], f1 = (float)v4[1], f2 = (float)v4[2], f3 = (float)v4[3];
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float p = sc[h][8 * wave + j];
        acc[h].x = __builtin_fmaf(p, f0, acc[h].x);
        acc[h].y = __builtin_fmaf(p, f1, acc[h].y);
        acc[h].z = __builtin_fmaf(p, f2, acc[h].z);
        acc[h].w = __builtin_fmaf(p, f3, acc[h].w);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) red[wave][h][lane] = acc[h];
  __syncthreads();
  for (int idx = tid; idx < G * (kHeadDim / 4); idx += 256) {
    const int h = idx >> 6, d4 = idx & 63;
    const float4 r0 = red[0][h][d4], r1 = red[1][h][d4], r2 = red[2][h][d4], r3 = red[3][h][d4];
    *reinterpret_cast<float4 *>(
        &a.part_o[((((size_t)tok * a.nkv + g) * a.chunks + c) * kAttnMaxGroup + hs * G + h) * kHeadDim + 4 * d4]) =
        make_float4((r0.x + r1.x) + (r2.x + r3.x), (r0.y + r1.y) + (r2.y + r3.y), (r0.z + r1.z) + (r2.z + r3.z),
                    (r0.w + r1.w) + (r2.w + r3.w));
  }
}

__device__ __forceinline__ float block_max_f32(float v, float *sh) {
  v = wave_max_f32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}

__device__ __forceinline__ float block_sum_f32(float v, float *sh) {
  v = wave_sum_f32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// Merge of the chunks of query head blockIdx.x for dims 64 blockIdx.y ..
// + 63: thread t sums chunks t / 64, t / 64 + 4, ... of dim t % 64, scaled by
// exp(m_c - m); then castF16Rows of o / l.  The chunk outputs are loaded
// together with the chunk maxima (one memory round trip per 128 chunks).
constexpr int kMergeTile = 128;  // chunks per round trip: 32 per thread
__global__ __launch_bounds__(256) void attn_reduce_kernel(const AttnArgs a) {
  __shared__ float fs[kMergeTile];
  __shared__ float sh[4];
  __shared__ float red[4][64];
  const int qh = blockIdx.x, tid = threadIdx.x;
  const int group = a.nq / a.nkv, g = qh / group, h = qh % group;
  const int chunks = a.chunks;
  const int tok = blockIdx.z;
  const size_t row0 = ((size_t)tok * a.nkv + g) * a.chunks * kAttnMaxGroup + h;  // chunk c at row0 + c * kAttnMaxGroup
  const int d = blockIdx.y * 64 + (tid & 63), cg = tid >> 6;
  if (chunks <= kMergeTile) {
    // One tile: every wave forms m, the factors exp(m_c - m) and l itself
    // (lane L takes chunks L and L + 64), so the only barrier is the final
    // sum over the four chunk groups.  Loads take no branch (chunks past the
    // last re-read it and are masked).
    __shared__ float fw[4][kMergeTile];
    const int lane = tid & 63;
    const int n = chunks;
    float po[kMergeTile / 4];
#pragma unroll
    for (int i = 0; i < kMergeTile / 4; i++)
      po[i] = a.part_o[(row0 + (size_t)min(cg + 4 * i, n - 1) * kAttnMaxGroup) * kHeadDim + d];
    float mc[2], lc[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const size_t base = row0 + (size_t)min(lane + 64 * k, n - 1) * kAttnMaxGroup;
      mc[k] = a.part_m[base];
      lc[k] = a.part_l[base];
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
      mc[k] = lane + 64 * k < n ? mc[k] : -__builtin_inff();
      lc[k] = lane + 64 * k < n ? lc[k] : 0.0f;
    }
    const float m = wave_max_f32(fmaxf(mc[0], mc[1]));
    float lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      // a chunk with no slot in the window (m_c = -inf) adds nothing
      const float f = mc[k] == -__builtin_inff() ? 0.0f : (float)exp((double)(mc[k] - m));
      fw[cg][lane + 64 * k] = f;
      lsum = __builtin_fmaf(f, lc[k], lsum);
    }
    const float l = wave_sum_f32(lsum);
    float o = 0.0f;  // this wave's own LDS row: no barrier between the writes above and these reads
#pragma unroll
    for (int i = 0; i < kMergeTile / 4; i++) o = __builtin_fmaf(fw[cg][cg + 4 * i], cg + 4 * i < n ? po[i] : 0.0f, o);
    red[cg][lane] = o;
    __syncthreads();
    if (tid < 64) {
      const float oo = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
      a.out[((size_t)tok * a.nq + qh) * kHeadDim + d] = l > 0.0f ? ts_f16_round(oo / l) : 0.0f;  // l == 0: no key
    }
    return;
  }
  // several tiles: the maximum over all chunks first
  float m = -__builtin_inff();
  for (int c = tid; c < chunks; c += 256) m = fmaxf(m, a.part_m[row0 + (size_t)c * kAttnMaxGroup]);
  float l = 0.0f, o = 0.0f;
  for (int c0 = 0; c0 < chunks; c0 += kMergeTile) {
    const int n = chunks - c0 < kMergeTile ? chunks - c0 : kMergeTile;
    // the tile's loads take no branch (chunks past n re-read chunk n - 1 and
    // are masked), so none waits for another
    float po[kMergeTile / 4];
#pragma unroll
    for (int i = 0; i < kMergeTile / 4; i++)
      po[i] = a.part_o[(row0 + (size_t)(c0 + min(cg + 4 * i, n - 1)) * kAttnMaxGroup) * kHeadDim + d];
    const size_t base = row0 + (size_t)(c0 + min(tid, n - 1)) * kAttnMaxGroup;
    float mc = a.part_m[base], lc = a.part_l[base];
#pragma unroll
    for (int i = 0; i < kMergeTile / 4; i++) po[i] = cg + 4 * i < n ? po[i] : 0.0f;
    mc = tid < n ? mc : -__builtin_inff();
    lc = tid < n ? lc : 0.0f;
    if (c0 == 0) m = block_max_f32(fmaxf(m, mc), sh);
    // a chunk with no slot in the window (m_c = -inf) adds nothing
    const float f = mc == -__builtin_inff() ? 0.0f : (float)exp((double)(mc - m));
    l = __builtin_fmaf(f, lc, l);
    __syncthreads();
    if (tid < kMergeTile) fs[tid] = f;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMergeTile / 4; i++) o = __builtin_fmaf(fs[cg + 4 * i], po[i], o);
  }
  l = block_sum_f32(l, sh);
  red[cg][tid & 63] = o;
  __syncthreads();
  if (tid < 64) {
    const float oo = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    a.out[((size_t)tok * a.nq + qh) * kHeadDim + d] = l > 0.0f ? ts_f16_round(oo / l) : 0.0f;  // l == 0: no key
  }
}

}  // namespace

hipError_t launch_norm_residual(const NormArgs &a, hipStream_t s) {
  if (a.n < 1 || a.n > 256 * kNormPer || a.rows < 1) return hipErrorInvalidValue;
  if ((a.q8img || a.xt) && (a.n % kQK != 0 || !a.next_out)) return hipErrorInvalidValue;
  if (a.next_image_only && !a.q8img && !a.xt) return hipErrorInvalidValue;
  if (a.y_ks > kNormParts || (a.y_ks > 1 && a.y_stride < (size_t)a.rows * a.n)) return hipErrorInvalidValue;
  const int grid = a.xt ? (a.rows + kF2Cols - 1) / kF2Cols * kF2Cols : a.rows;
  if (a.x16 && a.next_out && a.n % kQK == 0 && a.n <= 16 * kQK) {
    // rows that feed a projection: the block-per-group form
    hipLaunchKernelGGL(norm_residual_x16_kernel, dim3(grid), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  const int per = (a.n + 255) / 256;
  if (per <= 4)
    hipLaunchKernelGGL(norm_residual_kernel<4>, dim3(grid), dim3(256), 0, s, a);
  else if (per <= 8)
    hipLaunchKernelGGL(norm_residual_kernel<8>, dim3(grid), dim3(256), 0, s, a);
  else if (per <= 10)
    hipLaunchKernelGGL(norm_residual_kernel<10>, dim3(grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(norm_residual_kernel<kNormPer>, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_qkv_post(const QkvPostArgs &a, hipStream_t s) {
  if (a.nq < 1 || a.nkv < 1 || a.capacity < 1 || a.rope_dims < 0 || a.rope_dims > kHeadDim || (a.rope_dims & 1))
    return hipErrorInvalidValue;
  if (a.tokens < 1 || a.tokens > kMaxChunkTokens || a.src_ks > kNormParts || (!a.q_out && !a.q_half))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(qkv_post_kernel, dim3(a.nq + 2 * a.nkv, a.tokens), dim3(64), 0, s, a);
  return hipGetLastError();
}

int attn_max_chunks(int capacity) { return (capacity + kAttnChunk - 1) / kAttnChunk; }

size_t attn_partial_floats(int nkv, int capacity, int tokens) {
  return (size_t)tokens * nkv * attn_max_chunks(capacity) * kAttnMaxGroup * (kHeadDim + 2);
}

hipError_t launch_attention(AttnArgs a, float *partials, hipStream_t s) {
  if (a.nkv < 1 || a.nq % a.nkv != 0 || a.nq / a.nkv > kAttnMaxGroup || a.capacity < 1 || a.window < 0 ||
      a.rope_dims < 0 || a.rope_dims > kHeadDim || (a.rope_dims & 1) || a.tokens < 1 || a.tokens > kMaxTokens ||
      (a.prep && a.tokens != 1))
    return hipErrorInvalidValue;
  a.chunks = attn_max_chunks(a.capacity);
  const size_t slots = (size_t)a.tokens * a.nkv * a.chunks * kAttnMaxGroup;
  a.part_m = partials;
  a.part_l = partials + slots;
  a.part_o = partials + 2 * slots;
  // one or two tokens: two workgroups per (chunk, kv head) when the group
  // splits evenly (a 42-layer decode step 2.00 -> 1.97 ms, a 2-token draft
  // 2.82 -> 2.81 ms); longer drafts keep one, their grid already fills the
  // CUs (4 tokens: 3.73 ms against 3.80 split)
  const int group = a.nq / a.nkv;
  a.qsplit = a.tokens <= 2 && group % 2 == 0 ? 2 : 1;
  const dim3 grid(a.chunks, a.nkv * a.qsplit, a.tokens);
  switch (group / a.qsplit) {
    case 1: hipLaunchKernelGGL(attn_partial_kernel<1>, grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(attn_partial_kernel<2>, grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL(attn_partial_kernel<3>, grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(attn_partial_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 5: hipLaunchKernelGGL(attn_partial_kernel<5>, grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL(attn_partial_kernel<6>, grid, dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL(attn_partial_kernel<7>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(attn_partial_kernel<8>, grid, dim3(256), 0, s, a); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_merge(a, s);
}

hipError_t launch_attention_merge(const AttnArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(attn_reduce_kernel, dim3(a.nq, kHeadDim / 64, a.tokens), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace hp
