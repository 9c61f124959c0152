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
#include "hp_kquant.h"
#include "hp_q8k16.h"
#include "hp_wave.h"

namespace hp {

namespace {

// Threads per workgroup at most: eight waves (two per SIMD leave each wave
// 256 registers, room for a task's raw chunks twice: the next task's loads
// are issued before the current one's work).
constexpr int kWideMaxThreads = 512;

// LDS carve-up of one workgroup (byte offsets).  The input: Q4_K reads the
// Q8_K image (cols * nb blocks of kQ8BlockBytes), Q6_K two masked copies of
// its quants (q8k_store16_split, 256 bytes per block each, at a stride of
// kSplitStride bytes).  Lanes of a wave read the same 16 bytes of
// consecutive blocks; a stride of 68 dwords (4 mod 32 banks) spreads eight
// such lanes over all banks, where 256 bytes would put them in one.
constexpr int kSplitStride = kQ8BlockBytes;

// 16-byte pieces of an input image each thread loads ahead of the weights:
// four columns of 40 blocks over 512 threads need six.
constexpr int kImgRegs = 6;

struct WideLayout {
  int nbp;        // products per (row, col, class) row: nb rounded up to 4, == 4 (mod 8)
  size_t xhi;     // Q6_K: [cols][nb] upper-half copies (the lower ones at 0)
  size_t xd;      // [cols * nb] f32 Q8_K scales (padded to 4 entries)
  size_t prod;    // [rows][cols][NC][nbp] f32 products
  size_t fin;     // [rows][cols][NC] f32 chain results
  size_t total;
};

__host__ __device__ inline WideLayout wide_layout(int cols, int nb, int type, int rows) {
  WideLayout L;
  const int nc = type == kTypeQ4K ? 9 : 8;
  const size_t nq = (size_t)cols * nb;
  L.nbp = ((nb + 3) & ~3) | 4;
  L.xhi = type == kTypeQ6K ? nq * kSplitStride : 0;
  L.xd = type == kTypeQ6K ? 2 * nq * kSplitStride : nq * kQ8BlockBytes;
  L.prod = L.xd + (size_t)((nq + 3) & ~3) * 4;
  L.fin = L.prod + (size_t)rows * cols * nc * L.nbp * 4;
  L.total = L.fin + (size_t)rows * cols * nc * 4;
  return L;
}

__device__ __forceinline__ int mdiv(int x, uint32_t m) { return m ? (int)__umulhi((uint32_t)x, m) : x; }

// One (row, block) task's addresses in the tile layout.
struct WideTask {
  const uint4 *ch;     // chunk 0 of this row-block
  size_t cs;           // uint4 stride between chunks (the tile's lanes)
  const uint16_t *d6;  // Q6_K: f16 d of this row-block
};

template <int TYPE>
__device__ __forceinline__ WideTask wide_task(const MatvecArgs &a, int lrow, int b) {
  constexpr int CH = TYPE == kTypeQ4K ? 9 : 13;
  const int nb = a.g.nb, S = a.g.S, RG = a.g.R;
  WeightDesc W = a.w[0];
  if (a.count > 1) {  // wave-uniform: single-weight launches skip the selects
    if (lrow >= a.w[1].row_begin) W = a.w[1];
    if (a.count > 2 && lrow >= a.w[2].row_begin) W = a.w[2];
    if (a.count > 3 && lrow >= a.w[3].row_begin) W = a.w[3];
  }
  const int row = lrow - W.row_begin;
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

template <int TYPE>
__device__ __forceinline__ void wide_load(Regs &rg, const WideTask &t) {
  constexpr int CH = TYPE == kTypeQ4K ? 9 : 13;
#pragma unroll
  for (int c = 0; c < CH; c++) rg.c[c] = t.ch[(size_t)c * t.cs];
  if (TYPE == kTypeQ6K) rg.d6 = *t.d6;
}

}  // namespace

template <int M, int TYPE>
__global__ __launch_bounds__(kWideMaxThreads) void kquant_wide_kernel(const MatvecArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool Q4 = TYPE == kTypeQ4K;
  constexpr int NC = Q4 ? 9 : 8;
  const int nb = a.g.nb;
  const int R = a.wide_rows;
  const int row0 = blockIdx.x * R;
  const int VR = min(R, a.total_rows - row0);
  const WideLayout L = wide_layout(M, nb, TYPE, R);
  uint8_t *xq = smem;  // Q4_K: the image; Q6_K: the lower-half copies
  uint8_t *xhi = smem + L.xhi;
  float *xd = reinterpret_cast<float *>(smem + L.xd);
  float *prod = reinterpret_cast<float *>(smem + L.prod);
  float *fin = reinterpret_cast<float *>(smem + L.fin);

  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int ntask = VR * nb;

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
  if (!pre) {
    load_x16(xv, x_block(min(grp, nq - 1)), i16);
    load_x16(xv2, x_block(min(grp + ngrp, nq - 1)), i16);
  }
  // or the first kImgRegs 16-byte pieces per thread of the input image (a
  // thread past the end re-reads the last piece), likewise before the weights
  const int n16 = (int)(q8_image_bytes(M, nb) / 16);
  const uint4 *img = reinterpret_cast<const uint4 *>(a.q8img);
  uint4 iv[kImgRegs];
  if (pre) {
#pragma unroll
    for (int i = 0; i < kImgRegs; i++) iv[i] = img[min(tid + i * nthr, n16 - 1)];
  }

  // an idle thread loads the workgroup's last task: no branch around the loads
  int t = tid;
  Regs cur;
  {
    const int te = min(t, ntask - 1);
    const int vr = mdiv(te, a.mg_nb);
    wide_load<TYPE>(cur, wide_task<TYPE>(a, row0 + vr, te - vr * nb));
  }
  __builtin_amdgcn_sched_barrier(0);

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
    for (int i = 0; i < kImgRegs; i++)
      if (tid + i * nthr < n16) put(tid + i * nthr, iv[i]);
    for (int u = tid + kImgRegs * nthr; u < n16; u += nthr) put(u, img[u]);
  } else {
    auto put_words = [&](const Q8Words &w, int q) {
      if (Q4)
        q8k_store16(w, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
      else
        q8k_store16_split(w, i16, xq + (size_t)q * kSplitStride, xhi + (size_t)q * kSplitStride, xd + q);
    };
    auto quant = [&](const float (&v)[16], int q) { put_words(q8k_words16(v, i16), q); };
    if (grp + ngrp < nq) {
      // two blocks: their two dependency chains interleave
      const Q8Words q0 = q8k_words16(xv, i16), q1 = q8k_words16(xv2, i16);
      put_words(q0, grp);
      put_words(q1, grp + ngrp);
    } else if (grp < nq) {
      put_words(q8k_words16(xv, i16), grp);
    }
    for (int q = grp + 2 * ngrp; q < nq; q += ngrp) {  // more than two passes (several columns)
      load_x16(xv, x_block(q), i16);
      quant(xv, q);
    }
  }
  __syncthreads();

  // phase 1: products
  for (; t < ntask; t += nthr) {
    const int vr = mdiv(t, a.mg_nb);
    const int b = t - vr * nb;
    Regs nxt;
    const int tn = t + nthr;
    const bool more = tn < ntask;
    if (more) {
      const int vn = mdiv(tn, a.mg_nb);
      wide_load<TYPE>(nxt, wide_task<TYPE>(a, row0 + vn, tn - vn * nb));
    }
    __builtin_amdgcn_sched_barrier(0);
    int aux[M][8];
    int sumi[M];
    float dw, dminw = 0.0f;
    if (Q4) {
      q4k_ints<M>(cur, xq, nb, b, aux, sumi);
      dw = h2f(cur.c[0].x & 0xFFFFu);
      dminw = h2f(cur.c[0].x >> 16);
    } else {
      q6k_ints_split<M, kSplitStride>(cur, xq, xhi, nb, b, aux);
      dw = h2f(cur.d6);
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const float dx = xd[m * nb + b];
      const float dd = __fmul_rn(dw, dx);
      float *pr = prod + ((size_t)(vr * M + m) * NC) * L.nbp + b;
#pragma unroll
      for (int l = 0; l < 8; l++) pr[l * L.nbp] = __fmul_rn(dd, (float)aux[m][l]);
      // class 8 (Q4_K sumf -= ...) stored negated: s - p == s + (-p) in IEEE
      if (Q4) pr[8 * L.nbp] = -__fmul_rn(__fmul_rn(dminw, dx), (float)sumi[m]);
    }
    if (more) cur = nxt;
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
  for (int u = tid; u < VR * M; u += nthr) {
    const int vr = u / M, m = u - vr * M;
    const float *f = fin + (size_t)u * NC;
    float tsum = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) tsum = __fadd_rn(tsum, f[l]);
    const float res = Q4 ? __fadd_rn(f[8], tsum) : tsum;
    const int lrow = row0 + vr;
    WeightDesc W = a.w[0];
    if (a.count > 1) {
      if (lrow >= a.w[1].row_begin) W = a.w[1];
      if (a.count > 2 && lrow >= a.w[2].row_begin) W = a.w[2];
      if (a.count > 3 && lrow >= a.w[3].row_begin) W = a.w[3];
    }
    W.out[(size_t)(a.out_col0 + m) * W.rows + (lrow - W.row_begin)] = res;
  }
}

size_t wide_lds_bytes(int cols, int nb, int type, int rows_per_wg) {
  return wide_layout(cols, nb, type, rows_per_wg).total;
}

// Threads per workgroup: enough for one task per thread and for one pass of
// the Q8_K prologue (16 per block), in whole waves, at most
// kWideMaxThreads.
int wide_threads(int cols, int nb, int rows_per_wg) {
  int n = rows_per_wg * nb;
  const int q = 16 * cols * nb;
  if (q > n) n = q;
  n = (n + 63) & ~63;
  return n < kWideMaxThreads ? n : kWideMaxThreads;
}

template <int M>
static void launch_wide_m(const MatvecArgs &a, int type, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (type == kTypeQ4K)
    hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ4K>), grid, block, lds, s, a);
  else
    hipLaunchKernelGGL((kquant_wide_kernel<M, kTypeQ6K>), grid, block, lds, s, a);
}

hipError_t launch_matvec_wide(const MatvecArgs &a, hipStream_t s) {
  if (a.count < 1 || a.count > kMaxWeights || a.wide_rows < 1 || a.total_rows < 1 || a.norm.mode != 0)
    return hipErrorInvalidValue;
  if (a.q8img && a.cols < 2) return hipErrorInvalidValue;
  const int type = a.w[0].type;
  if (type != kTypeQ4K && type != kTypeQ6K) return hipErrorInvalidValue;
  for (int i = 1; i < a.count; i++)
    if (a.w[i].type != type) return hipErrorInvalidValue;
  const int grid = (a.total_rows + a.wide_rows - 1) / a.wide_rows;
  const dim3 block(wide_threads(a.cols, a.g.nb, a.wide_rows));
  const size_t lds = wide_lds_bytes(a.cols, a.g.nb, type, a.wide_rows);
  switch (a.cols) {
    case 1: launch_wide_m<1>(a, type, dim3(grid), block, lds, s); break;
    case 2: launch_wide_m<2>(a, type, dim3(grid), block, lds, s); break;
    case 3: launch_wide_m<3>(a, type, dim3(grid), block, lds, s); break;
    case 4: launch_wide_m<4>(a, type, dim3(grid), block, lds, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hp
