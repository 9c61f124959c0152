// kquant_wide.hip -- Q4_K / Q6_K x Q8_K matvec with one workgroup per block of
// rows (gfx950), for one-column launches whose waves would otherwise each walk
// long rows alone.
//
// Numerics: the same integers and f32 tail as kquant_matvec.hip
// (packages/engine/wasm-kernels/src/lib.rs:2116-2172 Q4_K, 1923-1968 Q6_K):
//   d = dW_b * dX_b; sums[l] += d * f32(aux32[l])  (blocks in order, no FMA)
//   Q4_K: sumf -= (dminW_b * dX_b) * f32(sumi)
//   result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
//
// Work split.  Workgroup w owns launch rows w*R .. w*R+R-1 (the weights'
// rows end to end) and every block of them, so no row is split across
// workgroups.  Three phases, separated by workgroup barriers:
//   1. every thread owns one (row, block) task at a time: it loads the
//      block's raw chunks from the tile layout (hp_common.h) before the
//      prologue, forms the exact aux32[l] (and sumi) for each column and
//      leaves the f32 products d * f32(aux32[l]) in LDS, [row][col][l][b];
//   2. one thread per (row, column, lane class l) adds its row's products in
//      block order -- the reference's sequential chain, so the split across
//      threads changes no bit;
//   3. one thread per (row, column) forms the tail and stores the result.
// Rows never wait on each other and every task's loads are in flight from
// the first instruction, so a launch of 2560 rows x 40 blocks runs as 256
// workgroups of ten waves (one per CU) instead of 854 waves that each walk
// 120 blocks in sequence.
//
// Prologue: the f32 input is quantised to Q8_K in LDS (16 lanes per
// 256-element block); Q6_K launches keep it as two masked copies
// (q8k_store16_split, q6k_ints_split), which saves masking the weights.  From
// two columns the input may come already quantised (a.q8img).
#include "hp_common.h"
#include "hp_gelu.h"
#include "hp_kquant.h"
#include "hp_q8k16.h"
#include "hp_wave.h"
#include "hp_wide.h"

#include <type_traits>

namespace hp {

namespace {

// Threads per workgroup at most: eight waves (two per SIMD leave each wave
// 256 registers, room for a task's raw chunks twice: the next task's loads
// are issued before the current one's work).
constexpr int kWideMaxThreads = 512;
// With half tasks (HALF: a thread forms lane classes 4h .. 4h+3 of a
// row-block, half the integer work and half the chunks) up to sixteen waves:
// four per SIMD hide the latency of the products' LDS reads and dot chains
// that two leave exposed, and a Q8_K prologue of up to 64 blocks runs as one
// pass.  128 registers per wave.
constexpr int kWideHalfThreads = 1024;

// 16-byte pieces of an input image each thread loads ahead of the weights:
// four columns of 40 blocks over 512 threads need six (three over 1024).
template <bool HALF>
constexpr int kImgRegs = HALF ? 3 : 6;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));


// One (row, block) task's addresses in the tile layout.
struct WideTask {
  const uint4 *ch;     // chunk 0 of this row-block
  size_t cs;           // uint4 stride between chunks (the tile's lanes)
  const uint16_t *d6;  // Q6_K: f16 d of this row-block
};

// Launch row lrow of the launch's weights end to end, or with PAIR virtual
// row vr of the workgroup (gate rows, then the same rows of up).
__device__ __forceinline__ WeightDesc weight_of(const MatvecArgs &a, int lrow) {
  WeightDesc W = a.w[0];
  if (a.count > 1) {  // wave-uniform: single-weight launches skip the selects
    if (lrow >= a.w[1].row_begin) W = a.w[1];
    if (a.count > 2 && lrow >= a.w[2].row_begin) W = a.w[2];
    if (a.count > 3 && lrow >= a.w[3].row_begin) W = a.w[3];
  }
  return W;
}

template <int TYPE>
__device__ __forceinline__ WideTask wide_task(const MatvecArgs &a, const WeightDesc &W, int row, int b) {
  constexpr int CH = TYPE == kTypeQ4K ? 9 : 13;
  const int nb = a.g.nb, S = a.g.S, RG = a.g.R;
  const int tile = mdiv(row, a.mg_R);
  const int r = row - tile * RG;
  const int Rt = min(RG, W.rows - tile * RG);
  const int it = mdiv(b, a.mg_S);
  const int s = b - it * S;
  const int lanes = Rt * S;
  const int k = r * S + s;
  WideTask t;
  t.ch = reinterpret_cast<const uint4 *>(W.data + (size_t)tile * RG * nb * CH * 16) + (size_t)it * CH * lanes + k;
  t.cs = (size_t)lanes;
  t.d6 = W.dplane + (size_t)tile * RG * nb + (size_t)it * lanes + k;
  return t;
}

// Task (vr, b) of the workgroup whose first row is row0 (VRh: its rows of
// each weight with PAIR).
template <int TYPE, bool PAIR>
__device__ __forceinline__ WideTask task_at(const MatvecArgs &a, int row0, int VRh, int vr, int b) {
  if (PAIR) {
    const bool up = vr >= VRh;
    return wide_task<TYPE>(a, up ? a.w[1] : a.w[0], row0 + vr - (up ? VRh : 0), b);
  }
  const WeightDesc W = weight_of(a, row0 + vr);
  return wide_task<TYPE>(a, W, row0 + vr - W.row_begin, b);
}

template <int TYPE>
__device__ __forceinline__ void wide_load(Regs &rg, const WideTask &t) {
  constexpr int CH = TYPE == kTypeQ4K ? 9 : 13;
#pragma unroll
  for (int c = 0; c < CH; c++) rg.c[c] = t.ch[(size_t)c * t.cs];
  if (TYPE == kTypeQ6K) rg.d6 = *t.d6;
}

// The chunks of half h of a task: Q4_K chunk 0 and nibble chunks 1 + 2p + h;
// Q6_K the scales (chunk 12), low-nibble chunks 2p + h and high-bit chunks
// 8 + 2p + h, and d.
template <int TYPE>
__device__ __forceinline__ void wide_load(HalfRegs &rg, const WideTask &t, int h) {
  constexpr bool Q4 = TYPE == kTypeQ4K;
  rg.c0 = t.ch[(size_t)(Q4 ? 0 : 12) * t.cs];
#pragma unroll
  for (int p = 0; p < 4; p++) rg.d[p] = t.ch[(size_t)(Q4 ? 1 + 2 * p + h : 2 * p + h) * t.cs];
  if (!Q4) {
#pragma unroll
    for (int p = 0; p < 2; p++) rg.e[p] = t.ch[(size_t)(8 + 2 * p + h) * t.cs];
    rg.d6 = *t.d6;
  }
}

}  // namespace

// NORM (1, 2; one column, nb <= 16): the input formed from a residual stream
// in the prologue (NormIn), by the first four waves.  PAIR: weights 0 and 1
// are gate and up with equal rows; the workgroup takes the same rows of both
// and writes fround(gelu(gate) * up) to a.pair_out (layers.ts:435-456).
// TPL (1, 2): tasks per thread whose loads are issued before the prologue
// (the launch's tasks per workgroup fit TPL * blockDim.x; more run after,
// their loads waited for one at a time).  HALF: tasks are half row-blocks,
// task te = h * (rows * nb) + row * nb + b (h the slowest index, so a wave's
// halves agree but for one wave at the boundary).
template <int M, int TYPE, int NORM, bool PAIR, int TPL, bool HALF>
__global__ __launch_bounds__(HALF ? kWideHalfThreads : kWideMaxThreads) void kquant_wide_kernel(const MatvecArgs a) {
  // the argument lines in one round trip where the first loads need most of
  // them: the norm prologue's inputs, the two weights of gate/up (measured:
  // gate/up + GeGLU 11.1 -> 10.7 us); a plain launch's input loads go out
  // after the first few lines and the rest arrive under them (down 9.2 us,
  // 9.8 with the warm-up)
  if constexpr (NORM != 0 || PAIR) kernarg_warm<MatvecArgs>();
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool Q4 = TYPE == kTypeQ4K;
  constexpr int NC = Q4 ? 9 : 8;
  const int nb = a.g.nb;
  const int R = a.wide_rows;
  const int row0 = blockIdx.x * R;
  const int VRh = min(R, (PAIR ? a.w[0].rows : a.total_rows) - row0);  // rows of each weight (PAIR)
  const int VR = PAIR ? 2 * VRh : VRh;
  const WideLayout L = wide_layout(M, nb, TYPE, PAIR ? 2 * R : R);
  uint8_t *xq = smem;  // Q4_K: the image; Q6_K: the lower-half copies
  uint8_t *xhi = smem + L.xhi;
  float *xd = reinterpret_cast<float *>(smem + L.xd);
  float *prod = reinterpret_cast<float *>(smem + L.prod);
  float *fin = reinterpret_cast<float *>(smem + L.fin);

  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int nfull = VR * nb;  // (row, block) tasks
  const int ntask = HALF ? 2 * nfull : nfull;
  using TaskRegs = typename std::conditional<HALF, HalfRegs, Regs>::type;
  // task te's half (0 without HALF) and its (row, block) index
  auto half_of = [&](int te) { return HALF ? (int)(te >= nfull) : 0; };

  // prologue input first (vector loads return in order), then the first
  // task's weights, so the weights stream in while the prologue computes
  const int grp = tid >> 4, i16 = tid & 15, ngrp = nthr >> 4;
  const int nq = M * nb;
  const bool pre = M >= 2 && a.q8img != nullptr;
  auto x_block = [&](int q) { return a.x + (size_t)(q / nb) * a.k + (size_t)(q % nb) * kQK; };
  // the blocks of this group's first two passes, loaded unconditionally (a
  // group past the end re-reads the last block): with no branch around these
  // loads the waits for them count exactly and never wait for the weights
  float xv[16], xv2[16];
  __shared__ double norm_sh[8];  // two workgroup sums
  NormRegs nr;
  if (NORM) {
    // the norm's 16 groups (nb <= 16) are in the first four waves; every
    // wave loads (groups past nb re-read block nb - 1 and wide_norm_finish zeroes
    // them): a branch around these loads lets the compiler wait for them
    // before the weight loads are issued
    norm_load<NORM>(a.norm, nr, grp, nb, i16);
  } else if (!pre) {
    load_x16(xv, x_block(min(grp, nq - 1)), i16);
    if (!HALF) load_x16(xv2, x_block(min(grp + ngrp, nq - 1)), i16);
  }
  // or the first kImgRegs 16-byte pieces per thread of the input image (a
  // thread past the end re-reads the last piece), likewise before the weights
  const int n16 = (int)(q8_image_bytes(M, nb) / 16);
  const uint4 *img = reinterpret_cast<const uint4 *>(a.q8img);
  constexpr int NIMG = kImgRegs<HALF>;
  uint4 iv[NIMG];
  if (pre) {
#pragma unroll
    for (int i = 0; i < NIMG; i++) iv[i] = img[min(tid + i * nthr, n16 - 1)];
  }

  // the first TPL tasks' weights; a thread past the end loads the
  // workgroup's last task: no branch around the loads
  // (every address first: no branch between the loads)
  WideTask tk[TPL];
  int th[TPL];
#pragma unroll
  for (int i = 0; i < TPL; i++) {
    const int te = min(tid + i * nthr, ntask - 1);
    th[i] = half_of(te);
    const int tf = te - th[i] * nfull;
    const int vr = mdiv(tf, a.mg_nb);
    tk[i] = task_at<TYPE, PAIR>(a, row0, VRh, vr, tf - vr * nb);
  }
  TaskRegs rg[TPL];
#pragma unroll
  for (int i = 0; i < TPL; i++) {
    if constexpr (HALF)
      wide_load<TYPE>(rg[i], tk[i], th[i]);
    else
      wide_load<TYPE>(rg[i], tk[i]);
  }
  // keep the loads here: without a memory barrier the compiler may sink them
  // past the prologue to their first use (a machine scheduling barrier does
  // not stop that); the barrier reads none of the loaded registers, so it
  // waits for nothing
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  if (NORM)
    wide_norm_finish<NORM>(a.norm, nr, xv, grp, nb, i16, a.k, norm_sh,
                           4 * __builtin_amdgcn_readfirstlane(tid >> 6) < nb);

  if (pre) {
    // the image into LDS: Q4_K as it is (the same layout), Q6_K as the two
    // masked copies of each block's quants (the first 16 of its 17 pieces;
    // the bsums are not read) and the scales
    auto put = [&](int u, const uint4 v) {
      if (Q4) {
        reinterpret_cast<uint4 *>(smem)[u] = v;
      } else if (u < nq * 17) {
        const int q = u / 17, c = u - q * 17;
        if (c < 16) {
          reinterpret_cast<uint4 *>(xq + (size_t)q * kSplitStride)[c] =
              make_uint4(v.x & 0xFFFFu, v.y & 0xFFFFu, v.z & 0xFFFFu, v.w & 0xFFFFu);
          reinterpret_cast<uint4 *>(xhi + (size_t)q * kSplitStride)[c] =
              make_uint4(v.x & 0xFFFF0000u, v.y & 0xFFFF0000u, v.z & 0xFFFF0000u, v.w & 0xFFFF0000u);
        }
      } else {
        reinterpret_cast<uint4 *>(xd)[u - nq * 17] = v;
      }
    };
#pragma unroll
    for (int i = 0; i < NIMG; i++)
      if (tid + i * nthr < n16) put(tid + i * nthr, iv[i]);
    for (int u = tid + NIMG * nthr; u < n16; u += nthr) put(u, img[u]);
  } else {
    auto put_words = [&](const Q8Words &w, int q) {
      if (Q4)
        q8k_store16(w, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
      else
        q8k_store16_split(w, i16, xq + (size_t)q * kSplitStride, xhi + (size_t)q * kSplitStride, xd + q);
    };
    auto quant = [&](const float (&v)[16], int q) { put_words(q8k_words16(v, i16), q); };
    if (!HALF && !NORM && grp + ngrp < nq) {
      // two blocks: their two dependency chains interleave
      const Q8Words q0 = q8k_words16(xv, i16), q1 = q8k_words16(xv2, i16);
      put_words(q0, grp);
      put_words(q1, grp + ngrp);
    } else if (grp < nq) {
      put_words(q8k_words16(xv, i16), grp);
    }
    // more passes (several columns; with HALF from the second)
    for (int q = grp + (HALF ? 1 : 2) * ngrp; !NORM && q < nq; q += ngrp) {
      load_x16(xv, x_block(q), i16);
      quant(xv, q);
    }
  }
  __syncthreads();

  // phase 1: products
  // a thread past the end computes the clamped task's products and stores
  // none (no branch around the work: branches split the loaded registers'
  // live ranges, and the copies that follow wait for the loads)
  auto products = [&](const TaskRegs &cur, int t_in) {
    const bool live = t_in < ntask;
    const int te = min(t_in, ntask - 1);
    const int h = half_of(te);
    const int t = te - h * nfull;
    const int vr = mdiv(t, a.mg_nb);
    const int b = t - vr * nb;
    constexpr int NL = HALF ? 4 : 8;  // lane classes of a task: 4h + li
    int aux[M][NL];
    int sumi[M];
    float dw, dminw = 0.0f;
    if constexpr (HALF) {
      if (Q4) {
        q4k_ints_half<M>(cur, xq, nb, b, h, aux, sumi);
        dw = h2f(cur.c0.x & 0xFFFFu);
        dminw = h2f(cur.c0.x >> 16);
      } else {
        q6k_ints_half_split<M, kSplitStride>(cur, xq, xhi, nb, b, h, aux);
        dw = h2f(cur.d6);
      }
    } else {
      if (Q4) {
        q4k_ints<M>(cur, xq, nb, b, aux, sumi);
        dw = h2f(cur.c[0].x & 0xFFFFu);
        dminw = h2f(cur.c[0].x >> 16);
      } else {
        q6k_ints_split<M, kSplitStride>(cur, xq, xhi, nb, b, aux);
        dw = h2f(cur.d6);
      }
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const float dx = xd[m * nb + b];
      const float dd = __fmul_rn(dw, dx);
      float *pr = prod + ((size_t)(vr * M + m) * NC + NL * h) * L.nbp + b;
      float p[NL];
#pragma unroll
      for (int l = 0; l < NL; l++) p[l] = __fmul_rn(dd, (float)aux[m][l]);
      // class 8 (Q4_K sumf -= ...) stored negated: s - p == s + (-p) in IEEE;
      // with HALF by the h = 0 half
      const float p8 = Q4 ? -__fmul_rn(__fmul_rn(dminw, dx), (float)sumi[m]) : 0.0f;
      if (live) {
#pragma unroll
        for (int l = 0; l < NL; l++) pr[l * L.nbp] = p[l];
        if (Q4 && h == 0) pr[(8 - NL * h) * L.nbp] = p8;
      }
    }
  };
  // each task's chunks used whole here (no instruction): the register
  // allocator then keeps every loaded tuple intact up to this point instead
  // of copying parts of one right after its load, a copy that would wait for
  // the load during the prologue
  auto keep = [](uint4 &c) {
    u32x4 v = __builtin_bit_cast(u32x4, c);
    asm volatile("" : "+v"(v));
    c = __builtin_bit_cast(uint4, v);
  };
#pragma unroll
  for (int i = 0; i < TPL; i++) {
    if constexpr (HALF) {
      keep(rg[i].c0);
#pragma unroll
      for (int p = 0; p < 4; p++) keep(rg[i].d[p]);
      if (!Q4) {
#pragma unroll
        for (int p = 0; p < 2; p++) keep(rg[i].e[p]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < (Q4 ? 9 : 13); c++) keep(rg[i].c[c]);
    }
  }
#pragma unroll
  for (int i = 0; i < TPL; i++) products(rg[i], tid + i * nthr);
  for (int t = tid + TPL * nthr; t < ntask; t += nthr) {
    const int h = half_of(t);
    const int tf = t - h * nfull;
    const int vr = mdiv(tf, a.mg_nb);
    TaskRegs more;
    if constexpr (HALF)
      wide_load<TYPE>(more, task_at<TYPE, PAIR>(a, row0, VRh, vr, tf - vr * nb), h);
    else
      wide_load<TYPE>(more, task_at<TYPE, PAIR>(a, row0, VRh, vr, tf - vr * nb));
    products(more, t);
  }
  __syncthreads();

  // phase 2: block-order chains, one thread per (row, column, class)
  for (int u = tid; u < VR * M * NC; u += nthr) {
    const float *pr = prod + (size_t)u * L.nbp;
    float s = 0.0f;
    int b = 0;
    for (; b + 4 <= nb; b += 4) {
      const float4 p = *reinterpret_cast<const float4 *>(pr + b);
      s = __fadd_rn(s, p.x);
      s = __fadd_rn(s, p.y);
      s = __fadd_rn(s, p.z);
      s = __fadd_rn(s, p.w);
    }
    for (; b < nb; b++) s = __fadd_rn(s, pr[b]);
    fin[u] = s;
  }
  __syncthreads();

  // phase 3: result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
  auto tail = [&](int vr, int m) {
    const float *f = fin + (size_t)(vr * M + m) * NC;
    float tsum = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) tsum = __fadd_rn(tsum, f[l]);
    return Q4 ? __fadd_rn(f[8], tsum) : tsum;
  };
  for (int u = tid; u < VRh * M; u += nthr) {
    const int vr = u / M, m = u - vr * M;
    if (PAIR) {
      a.pair_out[(size_t)(a.out_col0 + m) * a.w[0].rows + row0 + vr] =
          geglu_lut(tail(vr, m), tail(VRh + vr, m), a.gelu_lut);
    } else {
      const WeightDesc W = weight_of(a, row0 + vr);
      W.out[(size_t)(a.out_col0 + m) * W.rows + (row0 + vr - W.row_begin)] = tail(vr, m);
    }
  }
}

size_t wide_lds_bytes(int cols, int nb, int type, int rows_per_wg) {
  return wide_layout(cols, nb, type, rows_per_wg).total;
}

// Threads per workgroup: enough for one task per thread and for one pass of
// the Q8_K prologue (16 per block), in whole waves, at most
// kWideMaxThreads (kWideHalfThreads with half tasks).
int wide_threads(int cols, int nb, int rows_per_wg, bool half) {
  int n = rows_per_wg * nb * (half ? 2 : 1);
  const int q = 16 * cols * nb;
  if (q > n) n = q;
  n = (n + 63) & ~63;
  const int cap = half ? kWideHalfThreads : kWideMaxThreads;
  return n < cap ? n : cap;
}

template <int M, int NORM, bool PAIR, bool HALF>
static void launch_wide_h(const MatvecArgs &a, int type, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  const int vrows = PAIR ? 2 * a.wide_rows : a.wide_rows;
  const bool two = vrows * a.g.nb * (HALF ? 2 : 1) > (int)block.x;
  if (type == kTypeQ4K) {
    if (two)
      hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ4K, NORM, PAIR, 2, HALF>), grid, block, lds, s, a);
    else
      hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ4K, NORM, PAIR, 1, HALF>), grid, block, lds, s, a);
  } else {
    if (two)
      hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ6K, NORM, PAIR, 2, HALF>), grid, block, lds, s, a);
    else
      hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ6K, NORM, PAIR, 1, HALF>), grid, block, lds, s, a);
  }
}

// Half tasks are built for launches without a norm prologue or GeGLU at one
// or two columns (128 registers hold them; more columns spill).
template <int M, int NORM, bool PAIR>
constexpr bool kWideHalfBuilt = NORM == 0 && !PAIR && M <= 2;

template <int M, int NORM, bool PAIR>
static void launch_wide_t(const MatvecArgs &a, int type, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if constexpr (kWideHalfBuilt<M, NORM, PAIR>) {
    if (a.wide_half) {
      launch_wide_h<M, NORM, PAIR, true>(a, type, grid, block, lds, s);
      return;
    }
  }
  launch_wide_h<M, NORM, PAIR, false>(a, type, grid, block, lds, s);
}

template <int M, bool PAIR>
static void launch_wide_m(const MatvecArgs &a, int type, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (M == 1 && a.norm.mode == 1)
    launch_wide_t<1, 1, PAIR>(a, type, grid, block, lds, s);
  else if (M == 1 && a.norm.mode == 2)
    launch_wide_t<1, 2, PAIR>(a, type, grid, block, lds, s);
  else
    launch_wide_t<M, 0, PAIR>(a, type, grid, block, lds, s);
}

template <bool PAIR>
static hipError_t launch_wide_pair(const MatvecArgs &a, int type, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  switch (a.cols) {
    case 1: launch_wide_m<1, PAIR>(a, type, grid, block, lds, s); break;
    case 2: launch_wide_m<2, PAIR>(a, type, grid, block, lds, s); break;
    case 3: launch_wide_m<3, PAIR>(a, type, grid, block, lds, s); break;
    case 4: launch_wide_m<4, PAIR>(a, type, grid, block, lds, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_matvec_wide(const MatvecArgs &a, hipStream_t s) {
  const bool pair = a.pair_out != nullptr;
  if (a.count < 1 || a.count > kMaxWeights || a.wide_rows < 1 || a.total_rows < 1) return hipErrorInvalidValue;
  if (a.norm.mode < 0 || a.norm.mode > 2 || (a.norm.mode != 0 && (a.cols != 1 || a.g.nb > 16)))
    return hipErrorInvalidValue;
  if (a.q8img && (a.cols < 2 || a.norm.mode != 0)) return hipErrorInvalidValue;
  if (pair && (a.count != 2 || a.w[0].rows != a.w[1].rows)) return hipErrorInvalidValue;
  const int type = a.w[0].type;
  if (type != kTypeQ4K && type != kTypeQ6K) return hipErrorInvalidValue;
  for (int i = 1; i < a.count; i++)
    if (a.w[i].type != type) return hipErrorInvalidValue;
  if (a.wide_half && (a.norm.mode != 0 || pair || a.cols > 2)) return hipErrorInvalidValue;
  const int rows = pair ? a.w[0].rows : a.total_rows;
  const int grid = (rows + a.wide_rows - 1) / a.wide_rows;
  const int vrows = pair ? 2 * a.wide_rows : a.wide_rows;
  // a norm prologue sums over four waves (wg_sum_f64): at least 256 threads
  const int threads = wide_threads(a.cols, a.g.nb, vrows, a.wide_half != 0);
  const dim3 block(a.norm.mode != 0 && threads < 256 ? 256 : threads);
  const size_t lds = wide_lds_bytes(a.cols, a.g.nb, type, vrows);
  return pair ? launch_wide_pair<true>(a, type, dim3(grid), block, lds, s)
              : launch_wide_pair<false>(a, type, dim3(grid), block, lds, s);
}

}  // namespace hp
