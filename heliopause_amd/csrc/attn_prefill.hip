// attn_prefill.hip -- causal GQA attention of a prefill chunk (many tokens)
// over the f16 KV ring, on the matrix cores.
//
// forwardAttentionLayer (packages/engine/src/runner/wasm/layers.ts:270-335)
// attends every token of a chunk over one window (attentionRange of the
// largest position, 972-980) with a causal mask (913-925), through
// hp_gqa_attention_f32 (packages/engine/wasm-kernels/src/lib.rs:538-654):
// query rounded to f16 (float32_to_float16), scores q . k (scale 1),
// p = f32(exp(f64(score - max))), out = sum(p / sum(p) * v), then
// castF16Rows.  The caches already hold the chunk's keys and values.
//
// Here a workgroup takes 64 query rows -- Tq = 64 / G tokens x the G query
// heads of one KV head -- and one of `ranges` slices of the window, and
// walks its keys 32 at a time:
//   scores  S^T = K Q^T on v_mfma_f32_16x16x32_f16 (keys as the A rows, the
//           wave's 16 query rows as the B columns): the f16 query and the
//           f16 keys multiply exactly, so only the order of the f32 sums
//           differs from the reference.  Lane (q, c) of the wave then holds
//           query row c's scores for keys 4q..4q+3 and 16+4q..16+4q+3;
//   softmax online: a running maximum m and sum l per query row, p =
//           exp(s - m) in f32 (hardware exp2); m moves, and the earlier
//           sums are rescaled by exp(m_old - m), only when a tile's maximum
//           passes it by more than e^8, so p stays below e^8 and most tiles
//           skip the rescale.  The tile maximum is the lane's 8 scores and
//           the three other lanes of its column (permlane swaps); l is kept
//           as per-lane partial sums until the end;
//   values  O^T += V^T P^T on the matrix cores with p split into two f16
//           parts (hi + lo carries 22 bits of p), so p * v is formed from
//           exact products.  The MFMA's k index runs over the lane's own 8
//           keys: V^T's key columns are stored in that order (key 4b + i at
//           column 8 (b % 4) + 4 (b / 4) + i), so P^T never leaves the
//           registers and each lane rescales its output by its own row's
//           factor.
// Each (row, slice) leaves (m, l, unnormalised o) in the partial layout of
// attn_reduce_kernel, which merges the slices, divides by l and applies
// castF16Rows.  Results agree with the reference within a tolerance (the
// sums run in another order), like the decode attention's.
//
// LDS: two buffers of one tile each -- the 32 keys as rows (K) and the 32
// values transposed (V^T, dim rows of 32 keys) -- so the next tile is
// stored while this one is read and one barrier per tile suffices.  Row
// strides are padded so the 16 lanes of an MFMA operand read hit distinct
// 16-byte slots, and the staging stores are laid out to do the same.
//
// Every token block of one (KV head, slice) reads the same keys and values.
// Workgroup i runs on XCD i % 8, so the work items are dealt out such that
// the blocks of one (KV head, slice) share an XCD and its L2: the keys and
// values then cross from HBM once per slice instead of once per block.
#include "hp_attn.h"
#include "hp_common.h"
#include "hp_f2tile.h"
#include "hp_gelu.h"
#include "hp_mfma.h"
#include "hp_wave.h"

namespace hp {

namespace {

constexpr int kPfRows = 64;               // query rows per workgroup, 16 per wave
constexpr int kPfKeys = 32;               // keys per step
constexpr int kKStride = kHeadDim + 8;    // halfs per key row (528 bytes)
constexpr int kVStride = kPfKeys + 8;     // halfs per transposed value row (80 bytes)
constexpr float kLazyRescale = 8.0f;      // largest score excess over the running maximum

struct PfTile {
  _Float16 k[kPfKeys][kKStride];
  _Float16 vt[kHeadDim][kVStride];
};

// Dim c (0..3) of the two keys held in uint2 a (dims 0..3 of one key) and b
// (the next key) as one dword: byte select 0x05040100 takes the low halves
// of (b, a), 0x07060302 the high halves.
__device__ __forceinline__ uint32_t pair_dim(uint2 a, uint2 b, int c) {
  const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
  return __builtin_amdgcn_perm((c >> 1) ? b.y : b.x, (c >> 1) ? a.y : a.x, sel);
}

// e^x as 2^(x log2 e) on the hardware exp2 (about 1 ulp, plus the rounding
// of the product: a relative error near 1e-6 at x = -20).
__device__ __forceinline__ float exp_of(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// max / sum over the four lanes c, c + 16, c + 32, c + 48.  A permlane swap
// of a value with itself leaves each lane its own value in one result and
// its partner's (lane ^ 32, then lane ^ 16) in the other, in an order that a
// symmetric operation does not see.  The results are taken out of the
// returned vector as integers before any bit cast: a bit cast of a vector
// element reads element 0.
__device__ __forceinline__ void swap_pair(float v, bool across32, float *x, float *y) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  uint32_t r0, r1;
  if (across32) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    r0 = r[0];
    r1 = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    r0 = r[0];
    r1 = r[1];
  }
  *x = __builtin_bit_cast(float, r0);
  *y = __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float col4_max(float v) {
  float x, y;
  swap_pair(v, true, &x, &y);
  swap_pair(fmaxf(x, y), false, &x, &y);
  return fmaxf(x, y);
}

__device__ __forceinline__ float col4_sum(float v) {
  float x, y;
  swap_pair(v, true, &x, &y);
  swap_pair(x + y, false, &x, &y);
  return x + y;
}

constexpr int kXcds = 8;

// Two workgroups per CU (the register budget then holds each wave to 256,
// and two double-buffered tiles of 37 KB each fit the 160 KB of LDS): a
// step waits on its next K/V tile's loads, and the other workgroup's waves
// compute meanwhile.
__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(const AttnArgs a, int blocks, int items) {
  __shared__ __align__(16) PfTile sh[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, c16 = lane & 15;
  const int G = a.nq / a.nkv, Tq = kPfRows / G;
  // work item (slice-major: item = (g * ranges + range) * blocks + block):
  // XCD x takes the contiguous items [x * per_xcd, (x + 1) * per_xcd)
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int item = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
  if (item >= items) return;
  const int pair = item / blocks;
  const int t0 = (item - pair * blocks) * Tq, g = pair / a.chunks, range = pair - g * a.chunks;
  const int M = a.tokens, cap = a.capacity;
  const size_t head_base = (size_t)g * cap * kHeadDim;

  // the window of the chunk's last position, this slice of it, and how far
  // this block's last token may look
  const int pos_base = *a.position + a.pos_offset;
  const int pos_last = pos_base + M - 1;
  int start = 0, count = 0;
  if (pos_last >= 0) window_of(pos_last, cap, a.window, &start, &count);
  const int s0 = start % cap;
  const int per = ((count + a.chunks - 1) / a.chunks + kPfKeys - 1) / kPfKeys * kPfKeys;
  const int w_begin = range * per;
  const int t_last = min(t0 + Tq, M) - 1;
  const int w_stop = min(min(w_begin + per, count), pos_base + t_last - start + 1);

  // this lane's query row (wave * 16 + c16): its token and head, and the
  // last window index it may see (-1 for a row past the chunk)
  const int row = wave * 16 + c16;
  const int qt = t0 + row / G, qh = row - (row / G) * G;
  const bool qvalid = row < Tq * G && qt < M;
  const int limit = qvalid ? min(w_stop - 1, pos_base + qt - start) : -1;
  // tiles that end at or below every row's limit skip the mask
  int lim_all = limit;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) lim_all = min(lim_all, __shfl_xor(lim_all, o));
  lim_all = __builtin_amdgcn_readfirstlane(lim_all);

  // the query fragments, rounded to f16 as the reference rounds the query
  // (already rounded when a.q_half is given); a row past the chunk
  // multiplies as zeros
  half8 qf[8];
  {
    const size_t qoff = ((size_t)min(qt, M - 1) * a.nq + g * G + (qvalid ? qh : 0)) * kHeadDim;
    const uint32_t qmask = qvalid ? 0xffffffffu : 0u;
    if (a.q_half) {
      const uint4 *qrow = reinterpret_cast<const uint4 *>(a.q_half + qoff);
      uint4 w[8];
#pragma unroll
      for (int s = 0; s < 8; s++) w[s] = qrow[4 * s + q4];
#pragma unroll
      for (int s = 0; s < 8; s++)
        qf[s] = __builtin_bit_cast(half8, make_uint4(w[s].x & qmask, w[s].y & qmask, w[s].z & qmask, w[s].w & qmask));
    } else {
      const float *qrow = a.q + qoff;
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const float4 lo = *reinterpret_cast<const float4 *>(qrow + 32 * s + 8 * q4);
        const float4 hi = *reinterpret_cast<const float4 *>(qrow + 32 * s + 8 * q4 + 4);
        const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int e = 0; e < 8; e++)
          qf[s][e] = __builtin_bit_cast(_Float16, (uint16_t)rs_f16_bits(__builtin_bit_cast(uint32_t, f[e]) & qmask));
      }
    }
  }

  f32x4 acc[16];
#pragma unroll
  for (int d = 0; d < 16; d++) acc[d] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -__builtin_inff(), l_part = 0.0f;

  // staging, the same for every thread (no branch, so no load waits on
  // another path's).  Values: 8 bytes (dims 4 v_dg .. + 3) of each of the
  // keys at V^T columns 8 v_q .. + 7 -- keys 4 v_q + i and 16 + 4 v_q + i --
  // stored as four 16-byte column runs.  Keys: a quarter row of key k_j,
  // 16-byte chunks k_e + 8 i, turned by 7 chunks on odd rows.  With the
  // padded strides each store's 8 (and 16) consecutive lanes then fill
  // distinct 16-byte slots of 128 (and 256) bytes.
  const int v_q = tid & 3, v_dg = tid >> 2;   // columns 8 v_q.., dims 4 v_dg..
  const int k_j = tid >> 3, k_e = tid & 7;    // key k_j, chunks (k_e + 8 i + 7 (k_j & 1)) % 32
  const int k_rot = k_e + 7 * (k_j & 1);
  uint2 vk[8];
  uint4 k0, k1, k2, k3;
  auto slot_of = [&](int w) {  // s0 < cap and w < count <= cap
    const int slot = s0 + min(w, w_stop - 1);
    return slot >= cap ? slot - cap : slot;
  };
  auto vrow = [&](int w) {
    return reinterpret_cast<const uint2 *>(a.v_cache + head_base + (size_t)slot_of(w) * kHeadDim + 4 * v_dg);
  };
  auto krow = [&](int w) {
    return reinterpret_cast<const uint4 *>(a.k_cache + head_base + (size_t)slot_of(w) * kHeadDim);
  };
#define HP_PF_LOAD(w0)                                                                      \
  do {                                                                                      \
    _Pragma("unroll") for (int i = 0; i < 8; i++)                                           \
        vk[i] = *vrow((w0) + 4 * v_q + (i & 3) + 16 * (i >> 2));                            \
    const uint4 *kr = krow((w0) + k_j);                                                     \
    k0 = kr[k_rot & 31];                                                                    \
    k1 = kr[(k_rot + 8) & 31];                                                              \
    k2 = kr[(k_rot + 16) & 31];                                                             \
    k3 = kr[(k_rot + 24) & 31];                                                             \
  } while (0)
#define HP_PF_STORE(t)                                                                      \
  do {                                                                                      \
    _Pragma("unroll") for (int c = 0; c < 4; c++)                                           \
        *reinterpret_cast<uint4 *>(&(t).vt[4 * v_dg + c][8 * v_q]) =                        \
            make_uint4(pair_dim(vk[0], vk[1], c), pair_dim(vk[2], vk[3], c),                 \
                       pair_dim(vk[4], vk[5], c), pair_dim(vk[6], vk[7], c));                \
    uint4 *kd = reinterpret_cast<uint4 *>(&(t).k[k_j][0]);                                  \
    kd[k_rot & 31] = k0;                                                                    \
    kd[(k_rot + 8) & 31] = k1;                                                              \
    kd[(k_rot + 16) & 31] = k2;                                                             \
    kd[(k_rot + 24) & 31] = k3;                                                             \
  } while (0)

  if (w_begin < w_stop) {
    HP_PF_LOAD(w_begin);
    HP_PF_STORE(sh[0]);
  }
  __syncthreads();
  int cur = 0;
  for (int w0 = w_begin; w0 < w_stop; w0 += kPfKeys, cur ^= 1) {
    const bool more = w0 + kPfKeys < w_stop;
    if (more) HP_PF_LOAD(w0 + kPfKeys);  // the next tile streams in while this one computes
    const PfTile &t = sh[cur];

    // S^T of the 32 keys (two 16-key halves) x the wave's 16 query rows.
    // All 16 key fragments are read before the first product, and the 16
    // value fragments before the softmax, so LDS latency overlaps work
    // instead of stalling each MFMA.
    half8 kb[2][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++) kb[hf][ks] = *reinterpret_cast<const half8 *>(&t.k[hf * 16 + c16][32 * ks + 8 * q4]);
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the products
    f32x4 s[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++) s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[hf][ks], qf[ks], s[hf], 0, 0, 0);
    half8 va[16];
#pragma unroll
    for (int d = 0; d < 16; d++) va[d] = *reinterpret_cast<const half8 *>(&t.vt[16 * d + c16][8 * q4]);
    // causal mask and window (only where a row's limit falls in this tile):
    // lane (q4, c16) holds row c16's keys w0 + 16 hf + 4 q4 + j
    if (w0 + kPfKeys - 1 > lim_all) {
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (w0 + 16 * hf + 4 * q4 + j > limit) s[hf][j] = -__builtin_inff();
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = col4_max(mx);
    // the running maximum moves only when the tile's exceeds it by more than
    // kLazyRescale (or it was -inf): p = exp(s - m) <= e^kLazyRescale, and
    // the rescale of l and the 64 sums runs on few tiles.  m, l and o stay
    // consistent, so o / l is unchanged.
    const bool bump = mx > m_run + kLazyRescale;
    if (__any(bump)) {
      const float alpha = bump ? exp_of(m_run - mx) : 1.0f;  // exp(-inf) = 0
      m_run = bump ? mx : m_run;
      l_part *= alpha;
#pragma unroll
      for (int d = 0; d < 16; d++) acc[d] *= alpha;
    }
    // a row with no key so far keeps m = -inf; exp(-inf - 0) = 0 then
    const float m_use = m_run == -__builtin_inff() ? 0.0f : m_run;
    half8 ph, pl;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float p = exp_of(s[i >> 2][i & 3] - m_use);
      psum += p;
      ph[i] = (_Float16)p;
      pl[i] = (_Float16)__builtin_fmaf((float)ph[i], -1.0f, p);  // p - hi, exact
    }
    l_part += psum;
    // O^T += V^T P^T; lane (q4, c16) holds dims 16 d + 4 q4 .. + 3 of row c16
#pragma unroll
    for (int d = 0; d < 16; d++) {
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[d], ph, acc[d], 0, 0, 0);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[d], pl, acc[d], 0, 0, 0);
    }
    if (more) HP_PF_STORE(sh[cur ^ 1]);  // its last readers finished before the previous barrier
    __syncthreads();
  }

#undef HP_PF_LOAD
#undef HP_PF_STORE
// partials in attn_reduce_kernel's layout: chunk = this slice
  auto part_row = [&](int t, int h) {
    return (((size_t)t * a.nkv + g) * a.chunks + range) * kAttnMaxGroup + h;
  };
  const float l_run = col4_sum(l_part);
  if (qvalid) {
    if (q4 == 0) {
      a.part_m[part_row(qt, qh)] = m_run;
      a.part_l[part_row(qt, qh)] = l_run;
    }
    float *orow = a.part_o + part_row(qt, qh) * kHeadDim;
#pragma unroll
    for (int d = 0; d < 16; d++)
      *reinterpret_cast<float4 *>(orow + 16 * d + 4 * q4) = make_float4(acc[d][0], acc[d][1], acc[d][2], acc[d][3]);
  }
}

// The slices of one (token, query head) per wave, four heads of a token per
// workgroup: lane i merges dims 4 i .. 4 i + 3,
// o = sum_c exp(m_c - m) o_c / sum_c exp(m_c - m) l_c with m the largest m_c,
// then castF16Rows (a row with no key in its window is 0).  Every slice's
// loads are issued before the first sum (one memory round trip per row).
// With a.o_tiles the four rows also leave as Q8_K activation tiles of the
// next projection: wave 0's 16-lane row r quantises head 4 blockIdx.x + r
// as q8k_prefill_tiles16_kernel would from the stored rows (the same f32
// values, the same element order), and workgroups past the last token
// write the padding columns as zeros.
__global__ __launch_bounds__(256) void attn_merge_slices_kernel(const AttnArgs a) {
  __shared__ float4 rows[4][kHeadDim / 4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qh = 4 * blockIdx.x + wave, tok = blockIdx.y;
  float4 res = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (qh < a.nq && tok < a.tokens) {
    const int G = a.nq / a.nkv, g = qh / G, h = qh - g * G;
    const size_t row0 = ((size_t)tok * a.nkv + g) * a.chunks * kAttnMaxGroup + h;  // slice c at row0 + c * 8
    float mc[kAttnPrefillMaxRanges], lc[kAttnPrefillMaxRanges];
    float4 oc[kAttnPrefillMaxRanges];
#pragma unroll
    for (int c = 0; c < kAttnPrefillMaxRanges; c++) {
      if (c < a.chunks) {
        const size_t r = row0 + (size_t)c * kAttnMaxGroup;
        mc[c] = a.part_m[r];
        lc[c] = a.part_l[r];
        oc[c] = *reinterpret_cast<const float4 *>(a.part_o + r * kHeadDim + 4 * lane);
      }
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < kAttnPrefillMaxRanges; c++)
      if (c < a.chunks) m = fmaxf(m, mc[c]);
    float l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kAttnPrefillMaxRanges; c++) {
      if (c < a.chunks) {
        const float f = mc[c] == -__builtin_inff() ? 0.0f : expf(mc[c] - m);
        l = __builtin_fmaf(f, lc[c], l);
        o[0] = __builtin_fmaf(f, oc[c].x, o[0]);
        o[1] = __builtin_fmaf(f, oc[c].y, o[1]);
        o[2] = __builtin_fmaf(f, oc[c].z, o[2]);
        o[3] = __builtin_fmaf(f, oc[c].w, o[3]);
      }
    }
    res.x = l > 0.0f ? ts_f16_round(o[0] / l) : 0.0f;
    res.y = l > 0.0f ? ts_f16_round(o[1] / l) : 0.0f;
    res.z = l > 0.0f ? ts_f16_round(o[2] / l) : 0.0f;
    res.w = l > 0.0f ? ts_f16_round(o[3] / l) : 0.0f;
    *reinterpret_cast<float4 *>(a.out + ((size_t)tok * a.nq + qh) * kHeadDim + 4 * lane) = res;
  }
  if (!a.o_tiles) return;  // the same for the whole workgroup
  rows[wave][lane] = res;
  __syncthreads();
  if (wave == 0) {
    // row r, lane i16 = 2j + u: elements 32 j + 8 c + 4 u .. + 3 (load_x16's order)
    const int r = lane >> 4, i16 = lane & 15, j = i16 >> 1, u = i16 & 1, hb = 4 * blockIdx.x + r;
    if (hb < a.nq) {
      float v[16];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float4 f = rows[r][8 * j + 2 * c + u];
        v[4 * c] = f.x;
        v[4 * c + 1] = f.y;
        v[4 * c + 2] = f.z;
        v[4 * c + 3] = f.w;
      }
      f2_tile_store16(v, i16, a.o_tiles + ((size_t)(tok / kF2Cols) * a.nq + hb) * kF2XTile, tok % kF2Cols);
    }
  }
}

}  // namespace

int attn_prefill_ranges(int tokens, int nq, int nkv, int capacity, int num_cus) {
  const int G = nq / nkv, Tq = kPfRows / G;
  const int blocks = (tokens + Tq - 1) / Tq * nkv;
  int r = (2 * num_cus + blocks - 1) / blocks;
  const int max_r = (capacity + 4 * kPfKeys - 1) / (4 * kPfKeys);  // at least four key steps per slice
  if (r > max_r) r = max_r;
  if (r > kAttnPrefillMaxRanges) r = kAttnPrefillMaxRanges;
  return r < 1 ? 1 : r;
}

size_t attn_prefill_partial_floats(int nkv, int tokens, int ranges) {
  return (size_t)tokens * nkv * ranges * kAttnMaxGroup * (kHeadDim + 2);
}

hipError_t launch_attention_prefill(AttnArgs a, float *partials, int ranges, hipStream_t s) {
  if (a.nkv < 1 || a.nq % a.nkv != 0 || a.nq / a.nkv > kAttnMaxGroup || a.capacity < 1 || a.window < 0 ||
      a.tokens < 1 || a.tokens > kMaxChunkTokens || a.tokens > a.capacity || a.prep || ranges < 1 ||
      ranges > kAttnPrefillMaxRanges || (!a.q && !a.q_half))
    return hipErrorInvalidValue;
  a.chunks = ranges;
  const size_t slots = (size_t)a.tokens * a.nkv * ranges * kAttnMaxGroup;
  a.part_m = partials;
  a.part_l = partials + slots;
  a.part_o = partials + 2 * slots;
  const int Tq = kPfRows / (a.nq / a.nkv);
  const int blocks = (a.tokens + Tq - 1) / Tq;
  const int items = blocks * a.nkv * ranges;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(per_xcd * kXcds), dim3(256), 0, s, a, blocks, items);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int merge_cols = a.o_tiles ? (a.tokens + kF2Cols - 1) / kF2Cols * kF2Cols : a.tokens;
  hipLaunchKernelGGL(attn_merge_slices_kernel, dim3((a.nq + 3) / 4, merge_cols), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace hp
