// decode_fused.hip -- a whole one-token decode step through every decoder
// layer as one persistent launch (gfx950): one workgroup of eight waves per
// CU, the stage boundaries inside the kernel (hp_fused.h).
//
// Reference: forwardAttentionLayer + forwardFfn (packages/engine/src/runner/
// wasm/layers.ts:161-473), projections as hp_matmul_quantized_prepared_f32
// (packages/engine/wasm-kernels/src/lib.rs:224-298, dots 1923-1968 and
// 2116-2172), attention as hp_gqa_attention_f32 (lib.rs:538-654).
//
// Each stage performs the arithmetic of the launch that hp_hip_decode_layers_
// device runs for it, in the same order, so both paths give the same bits:
//   Q/K/V    the wide kernel's phases (kquant_wide.hip: products in LDS,
//            block-order chains, tails) over this workgroup's rows, after
//            the norm prologue of the half-split launch (norm_load /
//            wide_norm_finish: the same f64 sums);
//   ATT      attn_partial_kernel (decode_layer.hip) for one (32-slot chunk,
//            kv head) item: head norms, RoPE, cache append, chunk softmax;
//   MERGE    attn_reduce_kernel for one (query head, 64 dims) item;
//   O, down  the wide kernel's phases without a prologue;
//   gate/up  the wide kernel's phases with the residual norm prologue and
//            GeGLU;
//   final    norm_residual_kernel: the last post-FFN residual and the output
//            norm.
// Projections are bit-exact with the reference whatever the split of rows
// over workgroups, so every stage's rows are shared out by weight bytes.
//
// Values that cross workgroups are exchanged as tagged words (hp_fused.h).
// Every stage issues its weight (or cache) loads first and then waits for
// its input: the weights stream while the previous stage finishes on other
// CUs.  Loads return in issue order, so the first check of the input also
// waits for the weights; a stale input is re-read until its tag matches.
#include "hp_attn.h"
#include "hp_common.h"
#include "hp_fused.h"
#include "hp_gelu.h"
#include "hp_kquant.h"
#include "hp_q8k16.h"
#include "hp_wave.h"
#include "hp_wide.h"

#include <algorithm>

namespace hp {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kCpolSc1 = 16;           // cache policy sc1: agent-coherent loads, write-through stores
constexpr int kDescBytes = 1024;       // one layer descriptor (device table stride)
static_assert(sizeof(FusedLayer) <= kDescBytes, "layer descriptor exceeds its slot");
constexpr int kRopeMax = kHeadDim / 2;

// ---------------------------------------------------------------------------
// Exchange words.

struct Fx {
  __amdgpu_buffer_rsrc_t rs;  // the exchange arena
  uint32_t *status;
  uint64_t spin;
  uint64_t *trace;  // this workgroup's stamps of the current stage (FusedArgs::trace), or null
};

// Stage timeline stamp k (FusedArgs::trace), by thread 0.
__device__ __forceinline__ void stamp(const Fx &f, int k) {
  if (f.trace && threadIdx.x == 0) f.trace[k] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ u32x4 xld2(const Fx &f, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(f.rs, off, 0, kCpolSc1);
}
__device__ __forceinline__ u32x2 xld1(const Fx &f, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(f.rs, off, 0, kCpolSc1);
}
__device__ __forceinline__ void xst1(const Fx &f, uint32_t off, float v, uint32_t tag) {
  const u32x2 w = {__float_as_uint(v), tag};
  __builtin_amdgcn_raw_buffer_store_b64(w, f.rs, off, 0, kCpolSc1);
}
__device__ __forceinline__ void xst2(const Fx &f, uint32_t off, float v0, float v1, uint32_t tag) {
  const u32x4 w = {__float_as_uint(v0), tag, __float_as_uint(v1), tag};
  __builtin_amdgcn_raw_buffer_store_b128(w, f.rs, off, 0, kCpolSc1);
}
__device__ __forceinline__ uint32_t wofs(uint32_t base, int i) { return base + 8u * (uint32_t)i; }

__device__ __forceinline__ bool tag2(const u32x4 &w, uint32_t t) { return (w.y == t) & (w.w == t); }
__device__ __forceinline__ bool tag1(const u32x2 &w, uint32_t t) { return w.y == t; }

__device__ __forceinline__ uint32_t status_now(const Fx &f) {
  return __hip_atomic_load(f.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Re-reads stale words until every tag is `tag`.  false: the wait outlived
// the launch's limit (the timeout bit is set) or a status bit was set
// elsewhere.  The first reads were issued by the caller.
template <int N, class Off>
__device__ __forceinline__ bool xwait2(const Fx &f, u32x4 (&w)[N], Off off, uint32_t tag) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < N; i++) ok &= tag2(w[i], tag);
  if (ok) return true;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; i++)
      if (!tag2(w[i], tag)) w[i] = xld2(f, off(i));
    const uint32_t st = status_now(f);
    ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok &= tag2(w[i], tag);
    if (ok) return true;
    if (st != 0) return false;
    if (__builtin_amdgcn_s_memrealtime() - t0 > f.spin) {
      __hip_atomic_fetch_or(f.status, kFusedTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

template <int N, class Off>
__device__ __forceinline__ bool xwait1(const Fx &f, u32x2 (&w)[N], Off off, uint32_t tag) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < N; i++) ok &= tag1(w[i], tag);
  if (ok) return true;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; i++)
      if (!tag1(w[i], tag)) w[i] = xld1(f, off(i));
    const uint32_t st = status_now(f);
    ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok &= tag1(w[i], tag);
    if (ok) return true;
    if (st != 0) return false;
    if (__builtin_amdgcn_s_memrealtime() - t0 > f.spin) {
      __hip_atomic_fetch_or(f.status, kFusedTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

// The 16 values of load_x16's lane pattern (hp_q8k16.h) of the block whose
// first element is word e0 of the buffer at `base`: lane i16 = 2j + u reads
// elements 32j + 8c + 4u .. + 3, i.e. two 16-byte pairs per c.
__device__ __forceinline__ uint32_t x16_off(uint32_t base, int e0, int i16, int i) {
  const int j = i16 >> 1, u = i16 & 1;
  return wofs(base, e0 + 32 * j + 8 * (i >> 1) + 4 * u + 2 * (i & 1));
}
__device__ __forceinline__ void x16_issue(const Fx &f, u32x4 (&w)[8], uint32_t base, int e0, int i16) {
#pragma unroll
  for (int i = 0; i < 8; i++) w[i] = xld2(f, x16_off(base, e0, i16, i));
}
__device__ __forceinline__ void x16_values(const u32x4 (&w)[8], float (&v)[16]) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    v[2 * i] = __uint_as_float(w[i].x);
    v[2 * i + 1] = __uint_as_float(w[i].z);
  }
}
// store_x16's pattern as tagged words.
__device__ __forceinline__ void x16_store(const Fx &f, uint32_t base, int e0, int i16, const float (&v)[16],
                                          uint32_t tag) {
#pragma unroll
  for (int i = 0; i < 8; i++) xst2(f, x16_off(base, e0, i16, i), v[2 * i], v[2 * i + 1], tag);
}

// Cooperative wait of the whole workgroup for np pairs of tagged words
// (pair q at byte offset off(q), 16 bytes), all carrying `tag`: thread t takes
// pairs t, t + kFusedThreads, ... (indices past the end re-read the last
// pair; at most kPollPer per thread) and leaves pair q's two values at
// dst[2q], dst[2q + 1] in LDS.  false: the wait failed.
constexpr int kPollPer = 20;  // 10240 values over 256 threads

template <class Off>
__device__ __forceinline__ bool poll_pairs(const Fx &f, int np, Off off_of, uint32_t tag, float *dst) {
  const int tid = threadIdx.x;
  const int ns = (np + kFusedThreads - 1) / kFusedThreads;  // slots in use (wave-uniform)
  auto off = [&](int i) { return off_of(min(tid + i * kFusedThreads, np - 1)); };
  u32x4 w[kPollPer];
#pragma unroll
  for (int i = 0; i < kPollPer; i++)
    if (i < ns) w[i] = xld2(f, off(i));
  bool ok = true;
#pragma unroll
  for (int i = 0; i < kPollPer; i++)
    if (i < ns) ok &= tag2(w[i], tag);
  if (!ok) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int i = 0; i < kPollPer; i++)
        if (i < ns && !tag2(w[i], tag)) w[i] = xld2(f, off(i));
      const uint32_t st = status_now(f);
      ok = true;
#pragma unroll
      for (int i = 0; i < kPollPer; i++)
        if (i < ns) ok &= tag2(w[i], tag);
      if (ok || st != 0) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > f.spin) {
        __hip_atomic_fetch_or(f.status, kFusedTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kPollPer; i++) {
    const int q = tid + i * kFusedThreads;
    if (i < ns && q < np)
      *reinterpret_cast<float2 *>(dst + 2 * q) = make_float2(__uint_as_float(w[i].x), __uint_as_float(w[i].z));
  }
  return ok;
}

// n values (even) of the tagged buffer at `base` into dst.
__device__ __forceinline__ bool poll_lds(const Fx &f, uint32_t base, int n, uint32_t tag, float *dst) {
  return poll_pairs(f, n >> 1, [&](int q) { return base + 16u * (uint32_t)q; }, tag, dst);
}

// load_x16's lane pattern (hp_q8k16.h) from an LDS array.
__device__ __forceinline__ void lds_x16(float (&v)[16], const float *xb, int i16) {
  const int j = i16 >> 1, u = i16 & 1;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const float4 q = *reinterpret_cast<const float4 *>(xb + 32 * j + 8 * c + 4 * u);
    v[4 * c] = q.x;
    v[4 * c + 1] = q.y;
    v[4 * c + 2] = q.z;
    v[4 * c + 3] = q.w;
  }
}
__device__ __forceinline__ void lds_st16(float *xb, const float (&v)[16], int i16) {
  const int j = i16 >> 1, u = i16 & 1;
#pragma unroll
  for (int c = 0; c < 4; c++)
    *reinterpret_cast<float4 *>(xb + 32 * j + 8 * c + 4 * u) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2],
                                                                          v[4 * c + 3]);
}

// ---------------------------------------------------------------------------
// Wave-uniform reads of the layer descriptor (in LDS).

__device__ __forceinline__ int u32v(const int32_t &v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t u32v(const uint32_t &v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ float uf32(const float &v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ double uf64(const double &v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  return __builtin_bit_cast(double, (hi << 32) | lo);
}
template <class T>
__device__ __forceinline__ T *uptr(T *const &p) {
  const uint64_t b = (uint64_t)p;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  return reinterpret_cast<T *>((hi << 32) | lo);
}

// Pointers read from the descriptor carry no address space; a generic
// pointer would compile to flat loads, which also count against the LDS
// counter, so every LDS access would wait for the weight stream.  All of
// them point to device memory.
#define HP_G __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ HP_G T *gptr(T *p) {
  return (HP_G T *)p;
}
template <class T>
__device__ __forceinline__ HP_G T *ugptr(T *const &p) {
  return gptr(uptr(p));
}

// 16- and 8-byte loads from device memory (clang vector types: HIP's vector
// structs take no address-space-qualified copies).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gld16(const HP_G void *p) {
  const u32x4 v = *reinterpret_cast<const HP_G u32x4 *>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gld8(const HP_G void *p) {
  const u32x2 v = *reinterpret_cast<const HP_G u32x2 *>(p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ f32x4 gld16f(const HP_G void *p) { return *reinterpret_cast<const HP_G f32x4 *>(p); }

// load_x16's lane pattern (hp_q8k16.h) from device memory.
__device__ __forceinline__ void load_x16g(float (&v)[16], const HP_G float *xb, int i16) {
  const int j = i16 >> 1, u = i16 & 1;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const f32x4 q = gld16f(xb + 32 * j + 8 * c + 4 * u);
    v[4 * c] = q.x;
    v[4 * c + 1] = q.y;
    v[4 * c + 2] = q.z;
    v[4 * c + 3] = q.w;
  }
}

// One stage's projection, wave-uniform.  A lane's weight is picked by adding
// offsets to the first weight's addresses, each offset selected against a
// constant: a select between two fields would become a load through a
// selected address and keep the whole struct in scratch memory.
struct ProjU {
  const HP_G uint8_t *data0;
  const HP_G uint16_t *dpl0;
  int64_t doff1, doff2, poff1, poff2;  // byte offsets of weights 1, 2 from weight 0
  int rows0, drows1, drows2, rbeg1, rbeg2;
  int count, nb, S, R;
  uint32_t mg_nb, mg_S, mg_R;
};

__device__ __forceinline__ ProjU proj_u(const FusedProj &P) {
  ProjU u;
  u.data0 = ugptr(P.w[0].data);
  u.dpl0 = ugptr(P.w[0].dplane);
  const int64_t d0 = (int64_t)uptr(P.w[0].data), p0 = (int64_t)uptr(P.w[0].dplane);
  u.doff1 = (int64_t)uptr(P.w[1].data) - d0;
  u.doff2 = (int64_t)uptr(P.w[2].data) - d0;
  u.poff1 = (int64_t)uptr(P.w[1].dplane) - p0;
  u.poff2 = (int64_t)uptr(P.w[2].dplane) - p0;
  u.rows0 = u32v(P.w[0].rows);
  u.drows1 = u32v(P.w[1].rows) - u.rows0;
  u.drows2 = u32v(P.w[2].rows) - u.rows0;
  u.rbeg1 = u32v(P.w[1].row_begin);
  u.rbeg2 = u32v(P.w[2].row_begin);
  u.count = u32v(P.count);
  u.nb = u32v(P.nb);
  u.S = u32v(P.S);
  u.R = u32v(P.R);
  u.mg_nb = u32v(P.mg_nb);
  u.mg_S = u32v(P.mg_S);
  u.mg_R = u32v(P.mg_R);
  return u;
}

// This workgroup's rows of a stage: launch rows [row0, row0 + nrows) of
// one type (nrows 0: none).
struct Share {
  int row0, nrows, type;
};

__device__ __forceinline__ Share share_of(const FusedProj &P, int wg) {
  Share s{0, 0, 0};
  const int nseg = u32v(P.nseg);
  for (int i = 0; i < nseg; i++) {
    const int b = u32v(P.seg[i].wg_begin), n = u32v(P.seg[i].wg_count);
    if (wg >= b && wg < b + n) {
      const int rpw = u32v(P.seg[i].rows_per_wg), r0 = u32v(P.seg[i].row_begin), rows = u32v(P.seg[i].rows);
      s.row0 = r0 + (wg - b) * rpw;
      s.nrows = min(rpw, r0 + rows - s.row0);
      s.type = u32v(P.seg[i].type);
    }
  }
  return s;
}

// ---------------------------------------------------------------------------
// Projection stage (M = 1): one code instance for every stage and type (the
// instruction cache holds a layer's stages only if they are few).

struct Task {
  const HP_G uint4 *ch;
  size_t cs;
  const HP_G uint16_t *d6;
};

// The tile-layout address of (weight w, row, block b); CH chunks per lane.
__device__ __forceinline__ Task task_of(const ProjU &u, int CH, int w, int row, int b) {
  const int nb = u.nb, S = u.S, RG = u.R;
  const HP_G uint8_t *data = u.data0 + ((w == 1 ? u.doff1 : 0) + (w == 2 ? u.doff2 : 0));
  const HP_G uint16_t *dpl =
      reinterpret_cast<const HP_G uint16_t *>(reinterpret_cast<const HP_G uint8_t *>(u.dpl0) +
                                              ((w == 1 ? u.poff1 : 0) + (w == 2 ? u.poff2 : 0)));
  const int rows = u.rows0 + (w == 1 ? u.drows1 : 0) + (w == 2 ? u.drows2 : 0);
  const int tile = mdiv(row, u.mg_R);
  const int r = row - tile * RG;
  const int Rt = min(RG, rows - tile * RG);
  const int it = mdiv(b, u.mg_S);
  const int s = b - it * S;
  const int lanes = Rt * S;
  const int k = r * S + s;
  Task t;
  t.ch = reinterpret_cast<const HP_G uint4 *>(data + (size_t)tile * RG * nb * CH * 16) + (size_t)it * CH * lanes + k;
  t.cs = (size_t)lanes;
  t.d6 = dpl + (size_t)tile * RG * nb + (size_t)it * lanes + k;
  return t;
}

// Task te = vr * nb + b of a workgroup whose first launch row is row0 (pair:
// virtual rows vr < nh are gate rows row0 + vr, the others the same rows of
// up; otherwise launch row row0 + vr of the weights end to end).
__device__ __forceinline__ Task task_at(const ProjU &u, bool pair, int CH, int row0, int nh, int te) {
  const int vr = mdiv(te, u.mg_nb);
  const int b = te - vr * u.nb;
  int w, row;
  if (pair) {
    w = vr >= nh ? 1 : 0;
    row = row0 + vr - (w ? nh : 0);
  } else {
    const int lrow = row0 + vr;
    w = (u.count > 1 && lrow >= u.rbeg1 ? 1 : 0) + (u.count > 2 && lrow >= u.rbeg2 ? 1 : 0);
    row = lrow - (w == 1 ? u.rbeg1 : 0) - (w == 2 ? u.rbeg2 : 0);
  }
  return task_of(u, CH, w, row, b);
}

// Where a projection stage reads its input and writes its output.
struct StageIn {
  int mode;             // 0: x as it is; 1: x = rmsnorm(y) * w_next; 2: the residual form (hp_common.h NormIn)
  int pair;             // gate/up + GeGLU
  uint32_t x, x_tag;    // tagged words of x (modes 1, 2: y)
  const HP_G float *y_plain; // mode 1 at the first layer: y in plain memory
  uint32_t r;           // mode 2: x_res, followed by y (x is unused), both with x_tag
  const HP_G float *w_post, *w_next;
  float scale;
  double eps;
  uint32_t xo, xo_tag;  // modes 1, 2: x_out (mode 2: x1; mode 1: a copy of y), by workgroup 0
  int k;                // input size
  uint32_t out, out_tag;  // tagged output words, by launch row
  const uint16_t *lut;    // pair: the gelu table
};

// LDS of a projection stage (byte offsets from the dynamic base):
//   W  [0, w_bytes): the weights, chunk-major: chunk c of task te at
//      (c * nt + te) * 16, nt = tasks rounded up to 64 (direct global->LDS
//      copies, issued before the input wait, hold no registers);
//   S  [w_bytes, + s_bytes): the input as f32 (x; or x_res then y);
//   Q  the Q8_K image (wide_layout's xq / xhi / xd) over S, written once every
//      thread has read its inputs from S;
//   prod / fin (wide_layout's offsets from prod) over W, written once every
//      thread holds its tasks' chunks in registers.
struct ProjLds {
  size_t w_bytes, s_bytes, q_bytes, pf_bytes;
  int nt;
};

__host__ __device__ inline ProjLds proj_lds(int type, int nb, int vrows, bool norm) {
  ProjLds p;
  const int ch = type == kTypeQ4K ? 9 : 13;
  p.nt = (vrows * nb + 63) & ~63;
  p.w_bytes = (size_t)ch * p.nt * 16;
  p.s_bytes = (size_t)(norm ? 2 : 1) * nb * kQK * sizeof(float);
  const WideLayout L = wide_layout(1, nb, type, vrows);
  p.q_bytes = L.prod;              // xq, xhi, xd
  p.pf_bytes = L.total - L.prod;   // prod, fin
  return p;
}

// One projection stage of this workgroup (every thread calls it).  The
// prologue (modes 1, 2) needs nb <= 16; without it the Q8_K prologue takes
// up to four passes (nb <= 64).  A thread takes up to kSlots4 Q4_K tasks or
// kSlots6 Q6_K tasks (checked by the host).  false: a wait failed (the
// workgroup leaves).
constexpr int kSlots4 = kFusedSlotsQ4, kSlots6 = kFusedSlotsQ6, kPasses = 4;

__device__ __forceinline__ bool proj_stage(const Fx &f, const FusedProj &P, const Share sh, const StageIn &in,
                                           uint8_t *smem, double *norm_sh, int *s_abort) {
  const ProjU u = proj_u(P);
  const bool q4 = sh.type == kTypeQ4K;
  const bool pair = in.pair != 0;
  const int mode = in.mode;
  const int nb = u.nb;
  const int VRh = sh.nrows;
  const int VR = pair ? 2 * VRh : VRh;
  const int NC = q4 ? 9 : 8;
  const int CH = q4 ? 9 : 13;
  const WideLayout L = wide_layout(1, nb, sh.type, VR);
  const ProjLds pl = proj_lds(sh.type, nb, VR, mode != 0);
  uint8_t *wl = smem;
  float *sbuf = reinterpret_cast<float *>(smem + pl.w_bytes);
  uint8_t *xq = reinterpret_cast<uint8_t *>(sbuf);
  uint8_t *xhi = xq + L.xhi;
  float *xd = reinterpret_cast<float *>(xq + L.xd);
  float *prod = reinterpret_cast<float *>(smem);
  float *fin = prod + (L.fin - L.prod) / sizeof(float);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  constexpr int nthr = kFusedThreads;
  constexpr int ngrp = nthr / 16;
  const int ntask = VR * nb;
  const int slots = (ntask + nthr - 1) / nthr;
  const int grp = tid >> 4, i16 = tid & 15;
  const int row0 = sh.row0;
  const int gblk = min(grp, nb - 1);

  // 1. this stage's weights straight into LDS (a lane past the end copies the
  // last task again), the Q6_K d of its tasks, the prologue's norm weights
  uint16_t d6[kSlots6] = {};
#pragma unroll 1
  for (int s = 0; s < slots; s++) {
    const int te0 = s * nthr + wave * 64;  // the wave's first task of this slot
    if (te0 < ntask) {
      const Task t = task_at(u, pair, CH, row0, VRh, min(te0 + lane, ntask - 1));
      uint8_t *dst = wl + (size_t)te0 * 16;
#pragma unroll 1
      for (int c = 0; c < CH; c++)
        __builtin_amdgcn_global_load_lds((HP_G void *)(t.ch + (size_t)c * t.cs),
                                         (__attribute__((address_space(3))) void *)(dst + (size_t)c * pl.nt * 16), 16,
                                         0, 0);
    }
  }
  // (after the copies, with a fixed slot per register: a load whose
  // destination depended on a loop counter would wait for every copy before it)
  if (!q4) {
#pragma unroll
    for (int s = 0; s < kSlots6; s++)
      if (s < slots) d6[s] = *task_at(u, pair, CH, row0, VRh, min(tid + s * nthr, ntask - 1)).d6;
  }
  float ny[16], nres[16], nwp[16], nwn[16];  // the prologue's operands (hp_kquant.h NormRegs)
  if (mode != 0) {
    const size_t o = (size_t)gblk * kQK;
    load_x16g(nwn, in.w_next + o, i16);
    load_x16g(nwp, (mode == 2 ? in.w_post : in.w_next) + o, i16);
  }

  stamp(f, 1);
  // 2. the input, polled by the whole workgroup into S: modes 0, 1: x or y;
  // mode 2: x_res then y (adjacent in the arena, one tag).  Waiting for the
  // poll's loads also waits for the copies above (loads complete in order).
  float *rs = sbuf;
  float *xs = mode == 2 ? sbuf + in.k : sbuf;
  bool ok = true;
  if (mode != 0 && in.y_plain) {
    for (int e = 4 * tid; e < in.k; e += 4 * nthr)
    {
      const f32x4 q = gld16f(in.y_plain + e);
      *reinterpret_cast<float4 *>(xs + e) = make_float4(q.x, q.y, q.z, q.w);
    }
    __builtin_amdgcn_s_waitcnt(0);  // (no poll load to wait for the weight copies)
  } else if (mode == 2) {
    ok = poll_lds(f, in.r, 2 * in.k, in.x_tag, rs);
  } else {
    ok = poll_lds(f, in.x, in.k, in.x_tag, xs);
  }
  if (!ok) *s_abort = 1;
  __syncthreads();
  stamp(f, 2);

  // 3. this lane's input blocks in registers (modes 1, 2: normed), then,
  // past a barrier (inside the norm), Q8_K into Q over S
  float xv[kPasses][16];
  if (mode != 0) {
    lds_x16(ny, xs + (size_t)gblk * kQK, i16);
    if (mode == 2) {
      lds_x16(nres, rs + (size_t)gblk * kQK, i16);
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) nres[i] = 0.0f;
    }
    const bool active = 4 * wave < nb;
    NormIn n{};
    n.scale = in.scale;
    n.eps = in.eps;
    const bool st = blockIdx.x == 0;
    if (mode == 2) {
      wide_norm_finish_with<2>(n, ny, nres, nwp, nwn, xv[0], grp, nb, in.k, norm_sh, active, st,
                               [&](int g, const float (&v)[16]) { x16_store(f, in.xo, g * kQK, i16, v, in.xo_tag); });
    } else {
      if (st && grp < nb) x16_store(f, in.xo, grp * kQK, i16, ny, in.xo_tag);
      wide_norm_finish_with<1>(n, ny, nres, nwp, nwn, xv[0], grp, nb, in.k, norm_sh, active, false,
                               [&](int, const float (&)[16]) {});
    }
  } else {
#pragma unroll
    for (int p = 0; p < kPasses; p++) lds_x16(xv[p], xs + (size_t)min(grp + p * ngrp, nb - 1) * kQK, i16);
    __syncthreads();
  }
  auto quant = [&](const float (&v)[16], int q) {
    const Q8Words w = q8k_words16(v, i16);
    if (q4)
      q8k_store16(w, i16, xq + (size_t)q * kQ8BlockBytes, xd + q);
    else
      q8k_store16_split(w, i16, xq + (size_t)q * kSplitStride, xhi + (size_t)q * kSplitStride, xd + q);
  };
#pragma unroll
  for (int p = 0; p < kPasses; p++)
    if (grp + p * ngrp < nb) quant(xv[p], grp + p * ngrp);
  __syncthreads();
  stamp(f, 3);
  if (*s_abort) return false;

  // 4. every task's chunks into registers, then (past a barrier) the products
  // over W (a thread past the end computes the clamped task, stores none)
  if (q4) {
    uint4 w[kSlots4][9];
#pragma unroll
    for (int s = 0; s < kSlots4; s++)
      if (s < slots) {
        const uint4 *src = reinterpret_cast<const uint4 *>(wl) + min(tid + s * nthr, ntask - 1);
#pragma unroll
        for (int c = 0; c < 9; c++) w[s][c] = src[(size_t)c * pl.nt];
      }
    __syncthreads();
    stamp(f, 4);
#pragma unroll 1
    for (int s = 0; s < slots; s++) {
      Regs cur;
#pragma unroll
      for (int c = 0; c < 9; c++) cur.c[c] = w[0][c];
#pragma unroll
      for (int k = 0; k + 1 < kSlots4; k++)
#pragma unroll
        for (int c = 0; c < 9; c++) w[k][c] = w[k + 1][c];
      const int t_in = tid + s * nthr;
      const int te = min(t_in, ntask - 1);
      const int vr = mdiv(te, u.mg_nb);
      const int b = te - vr * nb;
      int aux[1][8], sumi[1];
      q4k_ints<1>(cur, xq, nb, b, aux, sumi);
      const float dx = xd[b];
      const float dd = __fmul_rn(h2f(cur.c[0].x & 0xFFFFu), dx);
      const float p8 = -__fmul_rn(__fmul_rn(h2f(cur.c[0].x >> 16), dx), (float)sumi[0]);
      float *pr = prod + (size_t)vr * 9 * L.nbp + b;
      if (t_in < ntask) {
#pragma unroll
        for (int l = 0; l < 8; l++) pr[l * L.nbp] = __fmul_rn(dd, (float)aux[0][l]);
        pr[8 * L.nbp] = p8;
      }
    }
  } else {
    Regs w6[kSlots6];
#pragma unroll
    for (int s = 0; s < kSlots6; s++)
      if (s < slots) {
        const uint4 *src = reinterpret_cast<const uint4 *>(wl) + min(tid + s * nthr, ntask - 1);
#pragma unroll
        for (int c = 0; c < 13; c++) w6[s].c[c] = src[(size_t)c * pl.nt];
        w6[s].d6 = d6[s];
      }
    __syncthreads();
    stamp(f, 4);
#pragma unroll 1
    for (int s = 0; s < slots; s++) {
      const Regs cur = w6[0];
      w6[0] = w6[1];
      const int t_in = tid + s * nthr;
      const int te = min(t_in, ntask - 1);
      const int vr = mdiv(te, u.mg_nb);
      const int b = te - vr * nb;
      int aux[1][8];
      q6k_ints_split<1, kSplitStride>(cur, xq, xhi, nb, b, aux);
      const float dd = __fmul_rn(h2f(cur.d6), xd[b]);
      float *pr = prod + (size_t)vr * 8 * L.nbp + b;
      if (t_in < ntask) {
#pragma unroll
        for (int l = 0; l < 8; l++) pr[l * L.nbp] = __fmul_rn(dd, (float)aux[0][l]);
      }
    }
  }
  __syncthreads();
  stamp(f, 5);

  // 5. block-order chains, one thread per (row, class)
  for (int v = tid; v < VR * NC; v += nthr) {
    const float *pr = prod + (size_t)v * L.nbp;
    float s = 0.0f;
    int b = 0;
    for (; b + 4 <= nb; b += 4) {
      const float4 q = *reinterpret_cast<const float4 *>(pr + b);
      s = __fadd_rn(s, q.x);
      s = __fadd_rn(s, q.y);
      s = __fadd_rn(s, q.z);
      s = __fadd_rn(s, q.w);
    }
    for (; b < nb; b++) s = __fadd_rn(s, pr[b]);
    fin[v] = s;
  }
  __syncthreads();
  stamp(f, 6);

  // 6. tails: result = [sumf +] ((((-0 + s0) + s1) + ...) + s7)
  auto tail = [&](int vr) {
    const float *fr = fin + (size_t)vr * NC;
    float tsum = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) tsum = __fadd_rn(tsum, fr[l]);
    return q4 ? __fadd_rn(fr[8], tsum) : tsum;
  };
  for (int vr = tid; vr < VRh; vr += nthr) {
    const float res = pair ? geglu_lut(tail(vr), tail(VRh + vr), in.lut) : tail(vr);
    xst1(f, wofs(in.out, row0 + vr), res, in.out_tag);
  }
  return true;
}

// ---------------------------------------------------------------------------
// Attention partials of one item (attn_partial_kernel, decode_layer.hip, one
// token with the prologue): waves 0-3 work, every thread passes the barriers.

struct AttnU {
  const HP_G float *wq, *wk, *ff;
  HP_G _Float16 *kc, *vc;
  double theta_scale, eps;
  int nq, nkv, cap, window, rope_dims, chunks, k_off, v_off, rope_key;
};

__device__ __forceinline__ AttnU attn_u(const FusedLayer &D) {
  AttnU a;
  a.wq = ugptr(D.q_norm);
  a.wk = ugptr(D.k_norm);
  a.ff = ugptr(D.freq_factors);
  a.kc = ugptr(D.k_cache);
  a.vc = ugptr(D.v_cache);
  a.theta_scale = uf64(D.theta_scale);
  a.eps = uf64(D.eps);
  a.nq = u32v(D.nq);
  a.nkv = u32v(D.nkv);
  a.cap = u32v(D.capacity);
  a.window = u32v(D.window);
  a.rope_dims = u32v(D.rope_dims);
  a.chunks = u32v(D.chunks);
  a.k_off = u32v(D.k_off);
  a.v_off = u32v(D.v_off);
  a.rope_key = u32v(D.rope_key);
  return a;
}

template <int G>
struct AttnSmem {
  float xs[G + 2][kHeadDim];
  float sc[G][kAttnChunk];
  float4 red[4][G][kHeadDim / 4];
};

struct AttnXchg {
  uint32_t qkv, qkv_tag, part, part_tag;
  int slots;  // partial slots per array (m, l; o has 256 per slot)
};

template <int G>
__device__ __forceinline__ bool attn_stage(const Fx &f, const AttnU &a, const AttnXchg x, int pos, int item,
                                        uint8_t *smem, double2 *rope_tab, int *rope_key_lds, int *s_abort) {
  AttnSmem<G> &S = *reinterpret_cast<AttnSmem<G> *>(smem);
  const int tid = threadIdx.x;
  constexpr bool act = true;  // every thread of the workgroup
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int c = item % a.chunks, g = item / a.chunks;
  const int cap = a.cap;
  const size_t head_base = (size_t)g * cap * kHeadDim;
  const int half = a.rope_dims >> 1;
  const bool have_tab = *rope_key_lds == a.rope_key;

  constexpr int kRows = (G + 2 + 3) / 4;
  // 1. the chunk's cache rows (streaming while Q/K/V finish elsewhere), the
  // norm weights (a value row has none: its loads re-read wq, unused), the
  // RoPE angles kept from an earlier layer; waves 4-7 load nothing
  const int kj = (tid & 255) >> 3, kp = tid & 7;
  const int kslot = c * kAttnChunk + kj;
  const int vslot0 = c * kAttnChunk + 8 * (wave & 3);
  uint4 kraw[4];
  uint2 vraw[8];
  float pw[kRows][4];
  double2 tab[2] = {make_double2(1.0, 0.0), make_double2(1.0, 0.0)};
  u32x2 px_w[kRows][4];
  auto px_off = [&](int k3, int j) {
    const int r = min(wave + 4 * k3, G + 1);
    const int row = r < G ? (g * G + r) * kHeadDim : (r == G ? a.k_off : a.v_off) + g * kHeadDim;
    return wofs(x.qkv, row + lane + 64 * j);
  };
  bool ok = true;
  if (act) {
    const HP_G _Float16 *kr = a.kc + head_base + (size_t)min(kslot, cap - 1) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 4; i++) kraw[i] = gld16(kr + 8 * (8 * i + kp));
#pragma unroll
    for (int j = 0; j < 8; j++)
      vraw[j] = gld8(a.vc + head_base + (size_t)min(vslot0 + j, cap - 1) * kHeadDim + 4 * lane);
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++) {
      const int r = min(wave + 4 * k3, G + 1);
      const HP_G float *w = r < G ? a.wq : (r == G ? a.wk : a.wq);
#pragma unroll
      for (int j = 0; j < 4; j++) pw[k3][j] = w[lane + 64 * j];
    }
    if (have_tab && half > 0) {
#pragma unroll
      for (int p = 0; p < 2; p++) tab[p] = rope_tab[min(lane + 64 * p, half - 1)];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // 2. the projection rows: queries g*G + r, the key, the value
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++)
#pragma unroll
      for (int j = 0; j < 4; j++) px_w[k3][j] = xld1(f, px_off(k3, j));
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++)
      if (ok) ok = xwait1(f, px_w[k3], [&](int j) { return px_off(k3, j); }, x.qkv_tag);
  }
  if (!ok) *s_abort = 1;
  float px[kRows][4];
#pragma unroll
  for (int k3 = 0; k3 < kRows; k3++)
#pragma unroll
    for (int j = 0; j < 4; j++) px[k3][j] = __uint_as_float(px_w[k3][j].x);

  int start, count;
  window_of(pos, cap, a.window, &start, &count);
  const int s0 = pos < 0 ? 0 : start % cap;
  const int last_w = pos - start;
  auto in_window = [&](int slot) {
    int w = slot - s0;
    w += w < 0 ? cap : 0;
    return pos >= 0 && slot < cap && w < count && w <= last_w;
  };
  const int new_slot = pos < 0 ? -1 : pos % cap;

  // 3. RoPE angles (once per launch and parameter set: kept in LDS)
  if (!have_tab) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int i = lane + 64 * p;
      if (act && i < half) {
        double theta = (double)pos;
        for (int it = 0; it < i; it++) theta = (double)(float)(theta * a.theta_scale);
        const double ang = a.ff ? theta / (double)a.ff[i] : theta;
        double sn, cn;
        sincos(ang, &sn, &cn);
        tab[p] = make_double2(cn, sn);
        if (wave == 0) rope_tab[i] = tab[p];
      }
    }
  }
  // 4. norms, RoPE, f16 rounding (queries as the scorer rounds them, the new
  // key and value as the cache stores them)
  if (act) {
#pragma unroll
    for (int k3 = 0; k3 < kRows; k3++) {
      const int r = wave + 4 * k3;
      if (r < G + 2) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 4; j++) ss += (double)px[k3][j] * (double)px[k3][j];
        const double scl = 1.0 / sqrt(wave_sum_f64(ss) / (double)kHeadDim + a.eps);
        float xr[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
          xr[j] = r <= G ? (float)(((double)px[k3][j] * scl) * (double)pw[k3][j]) : (float)((double)px[k3][j] * scl);
        if (r <= G) {
          const int hj = half >> 6;
#pragma unroll
          for (int j = 0; j < 2; j++) {
            if (j < hj) {
              const double x0 = xr[j], x1 = xr[j + hj];
              const double cc = tab[j].x, sn = tab[j].y;
              xr[j] = (float)(x0 * cc) - (float)(x1 * sn);
              xr[j + hj] = (float)(x0 * sn) + (float)(x1 * cc);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) S.xs[r][lane + 64 * j] = r < G ? rs_f16_round(xr[j]) : (float)(_Float16)xr[j];
      }
    }
  }
  __syncthreads();
  stamp(f, 2);
  if (!have_tab && tid == 0) *rope_key_lds = a.rope_key;  // read again only after later barriers
  if (*s_abort) return false;
  if (act && new_slot >= 0 && new_slot / kAttnChunk == c) {
    const size_t o = head_base + (size_t)new_slot * kHeadDim + tid;
    a.kc[o] = (_Float16)S.xs[G][tid];
    a.vc[o] = (_Float16)S.xs[G + 1][tid];
  }
  // 5. scores (the token's own key from LDS)
  const bool kvalid = act && in_window(kslot);
  if (kslot == new_slot) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 lo = *reinterpret_cast<const float4 *>(&S.xs[G][8 * (8 * i + kp)]);
      const float4 hi = *reinterpret_cast<const float4 *>(&S.xs[G][8 * (8 * i + kp) + 4]);
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
        const float4 qa = *reinterpret_cast<const float4 *>(&S.xs[h][d0]);
        const float4 qb = *reinterpret_cast<const float4 *>(&S.xs[h][d0 + 4]);
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
  if (act) {
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float t = oct_sum_f32(dot[h]);
      if (kp == 0) S.sc[h][kj] = kvalid ? t : -__builtin_inff();
    }
  }
  __syncthreads();
  // 6. softmax within the chunk: half-wave tid / 32 takes query head tid / 32
  {
    const int h = tid >> 5, j = tid & 31;
    if (h < G) {
      const float sv = S.sc[h][j];
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
      S.sc[h][j] = p;
      if (j == 0) {
        const int base = (g * a.chunks + c) * kAttnMaxGroup + h;
        xst1(f, wofs(x.part, base), m, x.part_tag);
        xst1(f, wofs(x.part, x.slots + base), l, x.part_tag);
      }
    }
  }
  __syncthreads();
  // 7. exp-weighted values (the token's own value from LDS)
  if (act && new_slot >= vslot0 && new_slot < vslot0 + 8) {
    const float4 nvv = *reinterpret_cast<const float4 *>(&S.xs[G + 1][4 * lane]);
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (vslot0 + j == new_slot) vraw[j] = make_uint2(pack2_f16(nvv.x, nvv.y), pack2_f16(nvv.z, nvv.w));
  }
  if (act) {
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
          const float p = S.sc[h][8 * wave + j];
          acc[h].x = __builtin_fmaf(p, f0, acc[h].x);
          acc[h].y = __builtin_fmaf(p, f1, acc[h].y);
          acc[h].z = __builtin_fmaf(p, f2, acc[h].z);
          acc[h].w = __builtin_fmaf(p, f3, acc[h].w);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++) S.red[wave][h][lane] = acc[h];
  }
  __syncthreads();
  for (int idx = tid; idx < G * (kHeadDim / 4); idx += kFusedThreads) {
    const int h = idx >> 6, d4 = idx & 63;
    const float4 r0 = S.red[0][h][d4], r1 = S.red[1][h][d4], r2 = S.red[2][h][d4], r3 = S.red[3][h][d4];
    const float4 o = make_float4((r0.x + r1.x) + (r2.x + r3.x), (r0.y + r1.y) + (r2.y + r3.y),
                                 (r0.z + r1.z) + (r2.z + r3.z), (r0.w + r1.w) + (r2.w + r3.w));
    const int base = ((g * a.chunks + c) * kAttnMaxGroup + h) * kHeadDim + 4 * d4;
    const uint32_t ob = wofs(x.part, 2 * x.slots + base);
    xst2(f, ob, o.x, o.y, x.part_tag);
    xst2(f, ob + 16, o.z, o.w, x.part_tag);
  }
  return true;
}

// ---------------------------------------------------------------------------
// Merge of one (query head, 64 dims) item (attn_reduce_kernel, one tile of
// at most 128 chunks): waves 0-3 work.

struct MergeSmem {
  float po[128][64];  // chunk c's 64 dims of this item
  float ml[2][128];   // m, l of each chunk
  float fw[4][128];
  float red[4][64];
};

__device__ __forceinline__ bool merge_stage(const Fx &f, const AttnU &a, const AttnXchg x, uint32_t att, uint32_t att_tag,
                                            int item, uint8_t *smem, int *s_abort) {
  MergeSmem &S = *reinterpret_cast<MergeSmem *>(smem);
  const int tid = threadIdx.x;
  constexpr bool act = true;  // every thread of the workgroup
  const int qh = item >> 2, dg = item & 3;
  const int group = a.nq / a.nkv, g = qh / group, h = qh % group;
  const int n = a.chunks;
  const int row0 = g * n * kAttnMaxGroup + h;  // chunk c at row0 + c * kAttnMaxGroup
  const int lane = tid & 63, cg = (tid >> 6) & 3;
  const int d = dg * 64 + lane;
  // the chunks' outputs (32 pairs of dims per chunk), then m and l
  bool ok = poll_pairs(
      f, n * 32,
      [&](int q) {
        const int c = q >> 5, j = q & 31;
        return wofs(x.part, 2 * x.slots + (row0 + c * kAttnMaxGroup) * kHeadDim + dg * 64 + 2 * j);
      },
      x.part_tag, &S.po[0][0]);
  u32x2 mlw[1];
  auto ml_off = [&](int) { return wofs(x.part, (tid >> 7) * x.slots + row0 + min(tid & 127, n - 1) * kAttnMaxGroup); };
  if (act) {
    mlw[0] = xld1(f, ml_off(0));
    if (ok) ok = xwait1(f, mlw, ml_off, x.part_tag);
    if ((tid & 127) < n) S.ml[tid >> 7][tid & 127] = __uint_as_float(mlw[0].x);
  }
  if (!ok) *s_abort = 1;
  __syncthreads();
  stamp(f, 2);
  float o = 0.0f, l = 0.0f;
  if (act) {
    float mc[2], lc[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      mc[k] = lane + 64 * k < n ? S.ml[0][lane + 64 * k] : -__builtin_inff();
      lc[k] = lane + 64 * k < n ? S.ml[1][lane + 64 * k] : 0.0f;
    }
    const float m = wave_max_f32(fmaxf(mc[0], mc[1]));
    float lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const float fk = mc[k] == -__builtin_inff() ? 0.0f : (float)exp((double)(mc[k] - m));
      S.fw[cg][lane + 64 * k] = fk;
      lsum = __builtin_fmaf(fk, lc[k], lsum);
    }
    l = wave_sum_f32(lsum);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int c = cg + 4 * i;
      o = __builtin_fmaf(S.fw[cg][c], c < n ? S.po[c][lane] : 0.0f, o);
    }
    S.red[cg][lane] = o;
  }
  __syncthreads();
  if (*s_abort) return false;
  if (tid < 64) {
    const float oo = (S.red[0][tid] + S.red[1][tid]) + (S.red[2][tid] + S.red[3][tid]);
    xst1(f, wofs(att, qh * kHeadDim + d), l > 0.0f ? ts_f16_round(oo / l) : 0.0f, att_tag);
  }
  return true;
}

// ---------------------------------------------------------------------------
// The last post-FFN residual and the output norm (norm_residual_kernel, one
// row): x = f32(f32(x1 + rmsnorm(y) * w_post) * scale) -> hidden, then
// out = rmsnorm(x) * w_next.  Threads 0-255 hold elements t + 256 j.

constexpr int kFinPer = 16;

__device__ __forceinline__ double fin_sum(double v, double *sh) {
  const int tid = threadIdx.x;
  if (tid < 256) v = wave_sum_f64(v);
  if ((tid & 63) == 0 && tid < 256) sh[tid >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

__device__ __forceinline__ bool final_stage(const Fx &f, int n, uint32_t y, uint32_t y_tag, uint32_t xr, uint32_t xr_tag,
                                           const HP_G float *w_post, float scale, double eps, HP_G float *x_out,
                                           const HP_G float *w_next, HP_G float *next_out, double *sh, int *s_abort) {
  const int tid = threadIdx.x;
  constexpr bool act = true;
  float v[kFinPer], r[kFinPer], wp[kFinPer], wn[kFinPer];
  u32x2 yw[kFinPer], rw[kFinPer];
#pragma unroll
  for (int j = 0; j < kFinPer; j++) {
    const int ic = min(tid + 256 * j, n - 1);
    wp[j] = w_post[ic];
    wn[j] = w_next ? w_next[ic] : 1.0f;
  }
  auto yo = [&](int j) { return wofs(y, min(tid + 256 * j, n - 1)); };
  auto ro = [&](int j) { return wofs(xr, min(tid + 256 * j, n - 1)); };
  bool ok = true;
  if (act) {
#pragma unroll
    for (int j = 0; j < kFinPer; j++) yw[j] = xld1(f, yo(j));
#pragma unroll
    for (int j = 0; j < kFinPer; j++) rw[j] = xld1(f, ro(j));
    ok = xwait1(f, yw, yo, y_tag);
    if (ok) ok = xwait1(f, rw, ro, xr_tag);
  }
  if (!ok) *s_abort = 1;
#pragma unroll
  for (int j = 0; j < kFinPer; j++) {
    const bool in = tid + 256 * j < n;
    v[j] = in ? __uint_as_float(yw[j].x) : 0.0f;
    r[j] = in ? __uint_as_float(rw[j].x) : 0.0f;
    wp[j] = in ? wp[j] : 1.0f;
    wn[j] = in && w_next ? wn[j] : 1.0f;
  }
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < kFinPer; j++) s += (double)v[j] * (double)v[j];
  const double sc = 1.0 / sqrt(fin_sum(s, sh) / (double)n + eps);
  if (*s_abort) return false;
#pragma unroll
  for (int j = 0; j < kFinPer; j++) {
    const int i = tid + 256 * j;
    const float t = (float)(((double)v[j] * sc) * (double)wp[j]);
    v[j] = i < n ? (r[j] + t) * scale : 0.0f;
    if (act && i < n) x_out[i] = v[j];
  }
  if (next_out) {
    s = 0.0;
#pragma unroll
    for (int j = 0; j < kFinPer; j++) s += (double)v[j] * (double)v[j];
    const double sc2 = 1.0 / sqrt(fin_sum(s, sh + 4) / (double)n + eps);
#pragma unroll
    for (int j = 0; j < kFinPer; j++) {
      const int i = tid + 256 * j;
      const float o = w_next ? (float)(((double)v[j] * sc2) * (double)wn[j]) : (float)((double)v[j] * sc2);
      if (act && i < n) next_out[i] = o;
    }
  }
  return true;
}

// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t tag_of(uint32_t epoch, int layer, int id) {
  return epoch * (uint32_t)kFusedTagStride + (uint32_t)(layer * 8 + id + 1);
}

// Stages of a layer, in order.
enum Stage { kStQkv = 0, kStAtt = 1, kStMerge = 2, kStO = 3, kStGu = 4, kStDown = 5, kStages = 6 };

template <int G>
__global__ __launch_bounds__(kFusedThreads) void decode_fused_kernel(const FusedArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ __align__(16) uint8_t desc[2][kDescBytes];
  __shared__ double2 rope_tab[kRopeMax];
  __shared__ double norm_sh[8];
  __shared__ int s_abort, rope_key;
  __shared__ uint32_t s_epoch;
  __shared__ int s_pos;
  const int tid = threadIdx.x, wg = blockIdx.x, W = gridDim.x;
  const int lane = tid & 63;
  const bool wave0 = tid < 64;

  Fx f;
  f.rs = __builtin_amdgcn_make_buffer_rsrc(a.xchg, 0, (int)a.xchg_bytes, 0x00020000);
  f.status = &a.ctl->status;
  f.spin = a.spin_ticks;
  f.trace = nullptr;

  // layer 0's descriptor, the epoch, the position and the sticky status
  if (wave0) reinterpret_cast<uint4 *>(desc[0])[lane] = reinterpret_cast<const uint4 *>(a.layers)[lane];
  if (tid == 0) {
    s_epoch = __hip_atomic_load(&a.ctl->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_abort = __hip_atomic_load(&a.ctl->status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    s_pos = *a.position;
    rope_key = -1;
  }
  __syncthreads();
  const uint32_t epoch = __builtin_amdgcn_readfirstlane(s_epoch);
  const int pos = __builtin_amdgcn_readfirstlane(s_pos);
  const FusedXchg X = a.x;

  int L = 0;
#pragma unroll 1
  for (; L < a.n_layers && !s_abort; L++) {
    const FusedLayer &D = *reinterpret_cast<const FusedLayer *>(desc[L & 1]);
    const FusedLayer &Pv = *reinterpret_cast<const FusedLayer *>(desc[(L + 1) & 1]);  // layer L - 1
    // the next layer's descriptor, written to the other slot at the layer's end
    uint4 nd = make_uint4(0, 0, 0, 0);
    const bool more = L + 1 < a.n_layers;
    if (wave0 && more)
      nd = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.layers) +
                                           (size_t)(L + 1) * kDescBytes)[lane];
#pragma unroll 1
    for (int st = 0; st < kStages && !s_abort; st++) {
      bool ok = true;
      f.trace = a.trace ? a.trace + ((size_t)(wg * a.n_layers + L) * kStages + st) * 8 : nullptr;
      stamp(f, 0);
      if (st == kStAtt) {
        // attention partials, one (chunk, kv head) item per workgroup
        const AttnU au = attn_u(D);
        const AttnXchg ax{X.qkv, tag_of(epoch, L, kTagQkv), X.part, tag_of(epoch, L, kTagPart), (int)X.part_slots};
        const int items = au.chunks * au.nkv;
        for (int it = wg; ok && it < items; it += W) ok = attn_stage<G>(f, au, ax, pos, it, smem, rope_tab, &rope_key, &s_abort);
      } else if (st == kStMerge) {
        const AttnU au = attn_u(D);
        const AttnXchg ax{X.qkv, 0, X.part, tag_of(epoch, L, kTagPart), (int)X.part_slots};
        const int items = au.nq * 4;
        for (int it = wg; ok && it < items; it += W)
          ok = merge_stage(f, au, ax, X.att, tag_of(epoch, L, kTagAtt), it, smem, &s_abort);
      } else {
        const FusedProj &P = st == kStQkv ? D.qkv : st == kStO ? D.o : st == kStGu ? D.gu : D.down;
        StageIn in{};
        in.k = u32v(P.nb) * kQK;
        if (st == kStQkv) {
          // the previous layer's post-FFN residual and attn_norm; both norms
          // use the previous layer's epsilon (the first layer: attn_norm only)
          in.w_next = ugptr(D.attn_norm);
          in.xo = X.hid;
          in.xo_tag = tag_of(epoch, L, kTagO);  // read with O's output
          in.out = X.qkv;
          in.out_tag = tag_of(epoch, L, kTagQkv);
          if (L == 0) {
            in.mode = 1;
            in.y_plain = gptr(a.hidden);
            in.eps = uf64(D.eps);
          } else {
            in.mode = 2;
            in.r = X.x1;  // x1, then y
            in.x_tag = tag_of(epoch, L - 1, kTagY);
            in.w_post = ugptr(Pv.post_ffw_norm);
            in.scale = uf32(Pv.out_scale);
            in.eps = uf64(Pv.eps);
          }
        } else if (st == kStO) {
          in.x = X.att;
          in.x_tag = tag_of(epoch, L, kTagAtt);
          in.out = X.o;
          in.out_tag = tag_of(epoch, L, kTagO);
        } else if (st == kStGu) {
          // the post-attention residual and ffn_norm, then gate/up + GeGLU
          in.mode = 2;
          in.pair = 1;
          in.r = X.hid;  // the residual entering the layer, then O's output
          in.x_tag = tag_of(epoch, L, kTagO);
          in.w_post = ugptr(D.post_attn_norm);
          in.w_next = ugptr(D.ffn_norm);
          in.scale = 1.0f;
          in.eps = uf64(D.eps);
          in.xo = X.x1;
          in.xo_tag = tag_of(epoch, L, kTagY);  // read with down's output
          in.out = X.h;
          in.out_tag = tag_of(epoch, L, kTagH);
          in.lut = a.gelu_lut;
        } else {
          in.x = X.h;
          in.x_tag = tag_of(epoch, L, kTagH);
          in.out = X.y;
          in.out_tag = tag_of(epoch, L, kTagY);
        }
        const Share sh = share_of(P, wg);
        if (sh.nrows > 0) ok = proj_stage(f, P, sh, in, smem, norm_sh, &s_abort);
      }
      (void)ok;
      stamp(f, 7);
      __syncthreads();
    }
    if (wave0 && more) reinterpret_cast<uint4 *>(desc[(L + 1) & 1])[lane] = nd;
    __syncthreads();
  }
  // the last post-FFN residual and the output norm, by workgroup 0
  if (!s_abort && wg == 0 && L == a.n_layers && L > 0) {
    const FusedLayer &D = *reinterpret_cast<const FusedLayer *>(desc[(L - 1) & 1]);
    final_stage(f, a.hidden_n, X.y, tag_of(epoch, L - 1, kTagY), X.x1, tag_of(epoch, L - 1, kTagY),
                ugptr(D.post_ffw_norm), uf32(D.out_scale), uf64(D.eps), gptr(a.hidden), gptr(a.out_norm),
                a.out_norm ? gptr(a.out) : nullptr, norm_sh, &s_abort);
  }
  // the last workgroup to finish advances the epoch for the next launch
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(&a.ctl->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)W - 1) {
      __hip_atomic_store(&a.ctl->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.ctl->epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

bool fused_group_supported(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }

namespace {
template <int G>
int blocks_per_cu(size_t lds) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_fused_kernel<G>, kFusedThreads, lds) != hipSuccess)
    return 0;
  return n;
}
template <int G>
size_t static_lds() {
  hipFuncAttributes fa{};
  if (hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(decode_fused_kernel<G>)) != hipSuccess) return 0;
  return fa.sharedSizeBytes;
}
}  // namespace

int fused_blocks_per_cu(int G, size_t lds) {
  switch (G) {
    case 1: return blocks_per_cu<1>(lds);
    case 2: return blocks_per_cu<2>(lds);
    case 4: return blocks_per_cu<4>(lds);
    case 8: return blocks_per_cu<8>(lds);
    default: return 0;
  }
}

size_t fused_static_lds(int G) {
  switch (G) {
    case 1: return static_lds<1>();
    case 2: return static_lds<2>();
    case 4: return static_lds<4>();
    case 8: return static_lds<8>();
    default: return 0;
  }
}

size_t fused_lds_bytes(const FusedLayer *layers, int n_layers, int hidden_n) {
  size_t need = 0;
  // W + S of every projection stage (the Q8_K image over S and the products
  // over W must fit; 0 when they do not)
  bool fits = true;
  auto proj = [&](const FusedProj &P, int pair, int norm) {
    for (int i = 0; i < P.nseg; i++) {
      const int vr = (pair ? 2 : 1) * P.seg[i].rows_per_wg;
      const ProjLds p = proj_lds(P.seg[i].type, P.nb, vr, norm != 0);
      if (p.q_bytes > p.s_bytes || p.pf_bytes > p.w_bytes) fits = false;
      const int slots = (vr * P.nb + kFusedThreads - 1) / kFusedThreads;
      if (slots > (P.seg[i].type == kTypeQ4K ? kFusedSlotsQ4 : kFusedSlotsQ6)) fits = false;
      const int kin = (norm ? 2 : 1) * P.nb * kQK;  // polled input values
      if ((norm && P.nb > 16) || P.nb > 16 * kPasses || kin > 2 * kPollPer * kFusedThreads) fits = false;
      need = std::max(need, p.w_bytes + p.s_bytes);
    }
  };
  for (int l = 0; l < n_layers; l++) {
    const FusedLayer &D = layers[l];
    proj(D.qkv, 0, 1);
    proj(D.o, 0, 0);
    proj(D.gu, 1, 1);
    proj(D.down, 0, 0);
    const int G = D.nq / D.nkv;
    need = std::max(need, (size_t)(G + 2) * kHeadDim * 4 + (size_t)G * kAttnChunk * 4 + (size_t)4 * G * kHeadDim * 4);
    if (D.chunks > 128) fits = false;  // one merge tile (MergeSmem)
  }
  need = std::max(need, sizeof(MergeSmem));
  (void)hidden_n;
  return fits ? (need + 255) & ~(size_t)255 : 0;
}

hipError_t launch_decode_fused(const FusedArgs &a, int num_cus, hipStream_t s) {
  if (a.n_layers < 1 || a.n_layers > kFusedMaxLayers || num_cus < 1) return hipErrorInvalidValue;
  const dim3 grid(num_cus), block(kFusedThreads);
  const size_t lds = (size_t)a.lds_bytes;
  switch (a.G) {
    case 1: hipLaunchKernelGGL(decode_fused_kernel<1>, grid, block, lds, s, a); break;
    case 2: hipLaunchKernelGGL(decode_fused_kernel<2>, grid, block, lds, s, a); break;
    case 4: hipLaunchKernelGGL(decode_fused_kernel<4>, grid, block, lds, s, a); break;
    case 8: hipLaunchKernelGGL(decode_fused_kernel<8>, grid, block, lds, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hp
