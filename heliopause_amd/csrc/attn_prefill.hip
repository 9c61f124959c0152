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
//           in f32 (hardware exp2), earlier sums rescaled by exp(m_old - m);
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
//
// Every token block of one (KV head, slice) reads the same keys and values.
// Workgroup i runs on XCD i % 8, so the work items are dealt out such that
// the blocks of one (KV head, slice) share an XCD and its L2: the keys and
// values then cross from HBM once per slice instead of once per block.
#include "hp_attn.h"
#include "hp_common.h"
#include "hp_gelu.h"
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

// Halves c of the four dwords v[r].c/2 (keys r = 0..3 of dim c) as two
// dwords: byte select 0x05040100 takes the low halves of (y, x), 0x07060302
// the high halves.
__device__ __forceinline__ uint2 column4(const uint4 (&v)[4], int c) {
  const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
  const uint32_t w0 = __builtin_amdgcn_perm(u4at(v[1], c >> 1), u4at(v[0], c >> 1), sel);
  const uint32_t w1 = __builtin_amdgcn_perm(u4at(v[3], c >> 1), u4at(v[2], c >> 1), sel);
  return make_uint2(w0, w1);
}

// e^x for x <= 0 as 2^(x log2 e) on the hardware exp2 (about 1 ulp, plus the
// rounding of the product: a relative error near 1e-6 at x = -20).
__device__ __forceinline__ float exp_of(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

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

constexpr int kXcds = 8;

// Two workgroups per CU (the register budget then holds each wave to 256):
// a step waits on its next K/V tile's loads, and the other workgroup's
// waves compute meanwhile.  512-token chunk of the 42-layer model: 5.7 ->
// 3.9 ms of attention (one workgroup per CU, 272 registers, before); three
// per CU spilled and took 6.8 ms.
__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(const AttnArgs a, int blocks, int items) {
  __shared__ __align__(16) PfShared sh;
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

  // staging, the same for every thread (no branch, so no load waits on
  // another path's): 32 bytes of values -- keys 4 v_kq .. + 3 at dims
  // 8 v_dq .. + 7, stored transposed -- and a quarter row of one key
  const int v_kq = tid & 7, v_dq = tid >> 3;  // keys 4 v_kq.., dims 8 v_dq..
  const int k_j = tid >> 3, k_e = tid & 7;    // key k_j, dims 32 k_e..
  uint4 v0, v1, v2, v3, k0, k1, k2, k3;
  auto slot_of = [&](int w) {  // s0 < cap and w < count <= cap
    const int slot = s0 + min(w, w_stop - 1);
    return slot >= cap ? slot - cap : slot;
  };
  auto vrow = [&](int w) {
    return reinterpret_cast<const uint4 *>(a.v_cache + head_base + (size_t)slot_of(w) * kHeadDim + 8 * v_dq);
  };
  auto krow = [&](int w) {
    return reinterpret_cast<const uint4 *>(a.k_cache + head_base + (size_t)slot_of(w) * kHeadDim + 32 * k_e);
  };
#define HP_PF_LOAD(w0)                                                                      \
  do {                                                                                      \
    v0 = *vrow((w0) + 4 * v_kq);                                                            \
    v1 = *vrow((w0) + 4 * v_kq + 1);                                                        \
    v2 = *vrow((w0) + 4 * v_kq + 2);                                                        \
    v3 = *vrow((w0) + 4 * v_kq + 3);                                                        \
    const uint4 *kr = krow((w0) + k_j);                                                     \
    k0 = kr[0];                                                                             \
    k1 = kr[1];                                                                             \
    k2 = kr[2];                                                                             \
    k3 = kr[3];                                                                             \
  } while (0)
#define HP_PF_STORE()                                                                       \
  do {                                                                                      \
    const uint4 vv[4] = {v0, v1, v2, v3};                                                   \
    _Pragma("unroll") for (int c = 0; c < 8; c++)                                           \
        *reinterpret_cast<uint2 *>(&sh.vt[8 * v_dq + c][4 * v_kq]) = column4(vv, c);        \
    uint4 *kd = reinterpret_cast<uint4 *>(&sh.k[k_j][32 * k_e]);                            \
    kd[0] = k0;                                                                             \
    kd[1] = k1;                                                                             \
    kd[2] = k2;                                                                             \
    kd[3] = k3;                                                                             \
  } while (0)

  if (w_begin < w_stop) {
    HP_PF_LOAD(w_begin);
    HP_PF_STORE();
  }
  __syncthreads();
  for (int w0 = w_begin; w0 < w_stop; w0 += kPfKeys) {
    const bool more = w0 + kPfKeys < w_stop;
    if (more) HP_PF_LOAD(w0 + kPfKeys);  // the next tile streams in while this one computes

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
      const float alpha = m_new == -__builtin_inff() ? 1.0f : exp_of(m_run[j] - m_new);
      float psum = 0.0f;
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        p[hf][j] = v[hf] == -__builtin_inff() ? 0.0f : exp_of(v[hf] - m_new);
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
    if (more) HP_PF_STORE();
    __syncthreads();
  }

#undef HP_PF_LOAD
#undef HP_PF_STORE
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

// The slices of one (token, query head): thread d merges dim d,
// o = sum_c exp(m_c - m) o_c / sum_c exp(m_c - m) l_c with m the largest m_c,
// then castF16Rows (a row with no key in its window is 0).
__global__ __launch_bounds__(kHeadDim) void attn_merge_slices_kernel(const AttnArgs a) {
  const int qh = blockIdx.x, tok = blockIdx.y, d = threadIdx.x;
  const int G = a.nq / a.nkv, g = qh / G, h = qh - g * G;
  const size_t row0 = ((size_t)tok * a.nkv + g) * a.chunks * kAttnMaxGroup + h;  // slice c at row0 + c * 8
  float m = -__builtin_inff();
  for (int c = 0; c < a.chunks; c++) m = fmaxf(m, a.part_m[row0 + (size_t)c * kAttnMaxGroup]);
  float l = 0.0f, o = 0.0f;
  for (int c = 0; c < a.chunks; c++) {
    const size_t r = row0 + (size_t)c * kAttnMaxGroup;
    const float mc = a.part_m[r];
    const float f = mc == -__builtin_inff() ? 0.0f : expf(mc - m);
    l = __builtin_fmaf(f, a.part_l[r], l);
    o = __builtin_fmaf(f, a.part_o[r * kHeadDim + d], o);
  }
  a.out[((size_t)tok * a.nq + qh) * kHeadDim + d] = l > 0.0f ? ts_f16_round(o / l) : 0.0f;
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
  const int blocks = (a.tokens + Tq - 1) / Tq;
  const int items = blocks * a.nkv * ranges;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(per_xcd * kXcds), dim3(256), 0, s, a, blocks, items);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_merge_slices_kernel, dim3(a.nq, a.tokens), dim3(kHeadDim), 0, s, a);
  return hipGetLastError();
}

}  // namespace hp
