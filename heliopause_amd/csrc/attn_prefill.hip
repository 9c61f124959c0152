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
//   scores  S = Q K^T on v_mfma_f32_16x16x32_f16: the f16 query and the f16
//           keys multiply exactly, so only the order of the f32 sums differs
//           from the reference;
//   softmax online: a running maximum m and sum l per row, p = exp(s - m)
//           in f32, earlier sums rescaled by exp(m_old - m);
//   values  O^T += V^T P^T on the matrix cores with p split into two f16
//           parts (hi + lo carries 22 bits of p), so p * v is formed from
//           exact products.
// Each (row, slice) leaves (m, l, unnormalised o) in the partial layout of
// attn_reduce_kernel, which merges the slices, divides by l and applies
// castF16Rows.  Results agree with the reference within a tolerance (the
// sums run in another order), like the decode attention's.
//
// LDS per tile: the 32 keys as rows (K), the 32 values transposed (V^T, dim
// rows of 32 keys), and per wave its P tile.  Row strides are padded so the
// 16 lanes of an MFMA operand read hit distinct 16-byte slots.
#include "hp_attn.h"
#include "hp_common.h"
#include "hp_mfma.h"
#include "hp_wave.h"

namespace hp {

namespace {

constexpr int kPfRows = 64;               // query rows per workgroup, 16 per wave
constexpr int kPfKeys = 32;               // keys per step
constexpr int kKStride = kHeadDim + 8;    // halfs per key row (528 bytes)
constexpr int kVStride = kPfKeys + 8;     // halfs per transposed value row (80 bytes)
constexpr int kPStride = kPfKeys + 8;     // halfs per P row (80 bytes)

struct PfShared {
  _Float16 k[kPfKeys][kKStride];
  _Float16 vt[kHeadDim][kVStride];
  _Float16 p_hi[4][16][kPStride];
  _Float16 p_lo[4][16][kPStride];
  float alpha[4][16];
};

// Halves c of the eight dwords d[r] (r = 0..7) as four dwords (rows 0..7 of
// column c): byte select 0x05040100 takes the low halves of (y, x), 0x07060302
// the high halves.
__device__ __forceinline__ uint4 column8(const uint4 (&v)[8], int c) {
  const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
  uint32_t w[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t lo = u4at(v[2 * r], c >> 1), hi = u4at(v[2 * r + 1], c >> 1);
    w[r] = __builtin_amdgcn_perm(hi, lo, sel);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
  return fmaxf(v, dpp_f32<kDppRowMirror>(v));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);
  return v + dpp_f32<kDppRowMirror>(v);
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(const AttnArgs a) {
  __shared__ __align__(16) PfShared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, c16 = lane & 15;
  const int G = a.nq / a.nkv, Tq = kPfRows / G;
  const int t0 = blockIdx.x * Tq, g = blockIdx.y, range = blockIdx.z;
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

  // rows of this lane: as the MFMA A/B operand row (c16) and as score rows (4 q4 + j)
  auto row_token = [&](int r, int *t, int *h) {
    *t = t0 + r / G;
    *h = r - (r / G) * G;
    return r < Tq * G && *t < M;
  };
  int qt, qh;
  const bool qvalid = row_token(wave * 16 + c16, &qt, &qh);
  int last_w[4];
  bool svalid[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    int t, h;
    svalid[j] = row_token(wave * 16 + 4 * q4 + j, &t, &h);
    last_w[j] = pos_base + t - start;
  }

  // the query fragments, rounded to f16 as the reference rounds the query
  half8 qf[8];
  {
    const float *qrow = a.q + ((size_t)min(qt, M - 1) * a.nq + g * G + (qvalid ? qh : 0)) * kHeadDim;
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const float4 lo = *reinterpret_cast<const float4 *>(qrow + 32 * s + 8 * q4);
      const float4 hi = *reinterpret_cast<const float4 *>(qrow + 32 * s + 8 * q4 + 4);
      const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int e = 0; e < 8; e++) qf[s][e] = qvalid ? (_Float16)rs_f16_round(f[e]) : (_Float16)0.0f;
    }
  }

  f32x4 acc[16];
#pragma unroll
  for (int d = 0; d < 16; d++) acc[d] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[4], l_run[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    m_run[j] = -__builtin_inff();
    l_run[j] = 0.0f;
  }

  // staging: threads 0..127 load an 8-key x 8-dim block of values and
  // transpose it; threads 128..255 load one key's 64 dims
  const bool vstage = tid < 128;
  const int b = tid & 127;
  const int v_ko = b & 3, v_do = b >> 2;   // keys 8 v_ko.., dims 8 v_do..
  const int k_j = b >> 2, k_u = b & 3;     // key k_j, dims 64 k_u..
  uint4 stg[8];
  auto slot_of = [&](int w) { return (s0 + min(w, w_stop - 1)) % cap; };
  auto load_tile = [&](int w0) {
    if (vstage) {
#pragma unroll
      for (int r = 0; r < 8; r++)
        stg[r] = *reinterpret_cast<const uint4 *>(a.v_cache + head_base + (size_t)slot_of(w0 + 8 * v_ko + r) * kHeadDim +
                                                  8 * v_do);
    } else {
      const _Float16 *krow = a.k_cache + head_base + (size_t)slot_of(w0 + k_j) * kHeadDim + 64 * k_u;
#pragma unroll
      for (int r = 0; r < 8; r++) stg[r] = *reinterpret_cast<const uint4 *>(krow + 8 * r);
    }
  };
  auto store_tile = [&]() {
    if (vstage) {
#pragma unroll
      for (int c = 0; c < 8; c++) *reinterpret_cast<uint4 *>(&sh.vt[8 * v_do + c][8 * v_ko]) = column8(stg, c);
    } else {
#pragma unroll
      for (int r = 0; r < 8; r++) *reinterpret_cast<uint4 *>(&sh.k[k_j][64 * k_u + 8 * r]) = stg[r];
    }
  };

  if (w_begin < w_stop) {
    load_tile(w_begin);
    store_tile();
  }
  __syncthreads();
  for (int w0 = w_begin; w0 < w_stop; w0 += kPfKeys) {
    const bool more = w0 + kPfKeys < w_stop;
    if (more) load_tile(w0 + kPfKeys);  // the next tile streams in while this one computes

    // scores of the wave's 16 rows x 32 keys (two 16-key halves)
    f32x4 s[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      s[hf] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 8; ks++) {
        const half8 kb = *reinterpret_cast<const half8 *>(&sh.k[hf * 16 + c16][32 * ks + 8 * q4]);
        s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qf[ks], kb, s[hf], 0, 0, 0);
      }
    }
    // causal mask and window, online softmax per row 4 q4 + j
    float p[2][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float v[2];
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int w = w0 + hf * 16 + c16;
        v[hf] = svalid[j] && w < w_stop && w <= last_w[j] ? s[hf][j] : -__builtin_inff();
      }
      const float m_new = fmaxf(m_run[j], row16_max(fmaxf(v[0], v[1])));
      const float alpha = m_new == -__builtin_inff() ? 1.0f : expf(m_run[j] - m_new);
      float psum = 0.0f;
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        p[hf][j] = v[hf] == -__builtin_inff() ? 0.0f : expf(v[hf] - m_new);
        psum += p[hf][j];
      }
      l_run[j] = l_run[j] * alpha + row16_sum(psum);
      m_run[j] = m_new;
      if (c16 == 0) sh.alpha[wave][4 * q4 + j] = alpha;
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const _Float16 hi = (_Float16)p[hf][j];
        sh.p_hi[wave][4 * q4 + j][hf * 16 + c16] = hi;
        sh.p_lo[wave][4 * q4 + j][hf * 16 + c16] = (_Float16)(p[hf][j] - (float)hi);
      }
    }
    __syncthreads();
    // rescale the running sums of row c16, then O^T += V^T P^T
    const float al = sh.alpha[wave][c16];
    const half8 ph = *reinterpret_cast<const half8 *>(&sh.p_hi[wave][c16][8 * q4]);
    const half8 pl = *reinterpret_cast<const half8 *>(&sh.p_lo[wave][c16][8 * q4]);
#pragma unroll
    for (int d = 0; d < 16; d++) {
      acc[d] *= al;
      const half8 va = *reinterpret_cast<const half8 *>(&sh.vt[16 * d + c16][8 * q4]);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, acc[d], 0, 0, 0);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, acc[d], 0, 0, 0);
    }
    __syncthreads();
    if (more) store_tile();
    __syncthreads();
  }

  // partials in attn_reduce_kernel's layout: chunk = this slice
  auto part_row = [&](int t, int h) {
    return (((size_t)t * a.nkv + g) * a.chunks + range) * kAttnMaxGroup + h;
  };
  if (c16 == 0) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int t, h;
      if (row_token(wave * 16 + 4 * q4 + j, &t, &h)) {
        a.part_m[part_row(t, h)] = m_run[j];
        a.part_l[part_row(t, h)] = l_run[j];
      }
    }
  }
  if (qvalid) {
    float *orow = a.part_o + part_row(qt, qh) * kHeadDim;
#pragma unroll
    for (int d = 0; d < 16; d++)
      *reinterpret_cast<float4 *>(orow + 16 * d + 4 * q4) = make_float4(acc[d][0], acc[d][1], acc[d][2], acc[d][3]);
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
      ranges > kAttnPrefillMaxRanges)
    return hipErrorInvalidValue;
  a.chunks = ranges;
  const size_t slots = (size_t)a.tokens * a.nkv * ranges * kAttnMaxGroup;
  a.part_m = partials;
  a.part_l = partials + slots;
  a.part_o = partials + 2 * slots;
  const int Tq = kPfRows / (a.nq / a.nkv);
  const dim3 grid((a.tokens + Tq - 1) / Tq, a.nkv, ranges);
  hipLaunchKernelGGL(attn_prefill_kernel, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_merge(a, s);
}

}  // namespace hp
