// hp_common.h -- shared definitions of the gfx950 quantized-projection runner.
//
// Device layouts (all byte counts equal the GGUF tensor's byte count):
//
// Weight tile layout.  A weight of N rows x nb super-blocks is cut into
// tiles of R rows.  Lane k of a wave handles row r = k / S and block slot
// s = k % S; iteration i covers blocks i*S .. i*S+S-1 (S divides nb).  A
// tile stores, per iteration, CH chunks of 16 bytes for each of its Rt*S
// lanes, chunk-major, so one 16-byte load per lane reads Rt*S*16
// contiguous bytes:
//     tile_base(t)      = t * R * nb * CH * 16
//     chunk(t, i, c, k) = tile_base(t) + ((i * CH + c) * Rt * S + k) * 16
// Q4_K (CH = 9): chunk 0 = bytes 0..15 of the GGUF block (d, dmin, 12
//   scale/min bytes).  Chunks 1..8 hold 32 dwords D[p][l] (p = 0..3, l =
//   0..7, dword 8p+l) with byte c of D[p][l] = qs[32p + 8c + l]: the four
//   elements 32j+8c+l (c = 0..3) that share accumulator lane l sit in one
//   dword (low nibbles: sub-block j = 2p, high nibbles: j = 2p+1).
// Q6_K (CH = 13): chunks 0..7 hold Dql[p][l] with byte c = nibble of
//   element (2p, c, l) | nibble of element (2p+1, c, l) << 4; chunks 8..11
//   hold Dqh[q][l] with byte c = qh[32q + 8c + l] ^ 0xAA (each 2-bit field
//   stores hi ^ 2, so (nibble | field << 4) is the 6-bit two's complement of
//   q - 32); chunk 12 = the 16 int8 scales.  The f16 d of every row-block
//   sits in a plane after all tiles, in tile order.
//
// Q8_K activation layout in LDS (per column m, per block b, 272 bytes): 64
// dwords X[j][l] (j = 0..7, l = 0..7, dword 8j+l) with byte c =
// q8[32j + 8c + l], then the 8 int16 sums of 32 (bsums32).  The f32 d of
// each block is kept in a separate [M][nb] array.  Every matvec workgroup
// quantises the f32 input into this layout itself (its prologue).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hp {

constexpr int kQK = 256;
constexpr int kTypeQ4K = 1;
constexpr int kTypeQ6K = 3;
constexpr int kQ8BlockBytes = 272;
constexpr int kMaxWeights = 4;
constexpr int kMaxCols = 8;  // columns per matvec launch

__host__ __device__ constexpr int chunks_for(int type) { return type == kTypeQ4K ? 9 : 13; }
__host__ __device__ constexpr int block_bytes(int type) { return type == kTypeQ4K ? 144 : 210; }

// Tile geometry shared by every weight of one launch (depends on nb only).
struct TileGeom {
  int nb;     // blocks per row
  int S;      // block slots per wave iteration
  int R;      // rows per tile (R * S <= 64)
  int iters;  // nb / S
};

TileGeom choose_geometry(int nb);

// One row's place in the tile layout, for the matrix-core kernels, which
// read a row at a time: chunk c of (row, block b = i * S + s) sits at byte
//     base + i * iter + c * chunk + s * 16
// of the weight's tiles, and the Q6_K d of (row, b) at
//     dplane[dbase + i * diter + s].
// 32-bit offsets: the launches that use it take weights under 4 GiB.
struct TileRow {
  uint32_t base, chunk, iter, dbase, diter;
};
__host__ __device__ inline TileRow tile_row(int row, int rows, int nb, int S, int R, int CH) {
  const int t = row / R, r = row - t * R, row0 = t * R;
  const int rt = rows - row0 < R ? rows - row0 : R;
  TileRow p;
  p.base = (uint32_t)(((size_t)row0 * nb * CH + (size_t)r * S) * 16);
  p.chunk = (uint32_t)(rt * S * 16);
  p.iter = (uint32_t)CH * p.chunk;
  p.dbase = (uint32_t)((size_t)row0 * nb + (size_t)r * S);
  p.diter = (uint32_t)(rt * S);
  return p;
}

// b = i * S + s for a block index the whole wave shares (nb / S steps at
// most, none for one-iteration geometries).
__device__ __forceinline__ void block_split(int b, int S, int &i, int &s) {
  i = 0;
  s = b;
  while (s >= S) {
    s -= S;
    i++;
  }
}

struct WeightDesc {
  const uint8_t *data;    // tiles
  const uint16_t *dplane; // Q6_K: f16 d per row-block in tile order; else null
  float *out;             // [M][N] output (device)
  int type;
  int rows;               // N
  int tiles;              // ceil(N / R)
  int tile_begin;         // first global tile index of this weight
  int row_begin;          // half-split kernel: first row of this weight in the
                          // launch's rows (the weights' rows end to end)
};

// Input of a one-column matvec launch formed in every workgroup's prologue
// from a residual stream (input size <= 16 * 256), in place of a plain x:
//   mode 1: x = rmsnorm(y) * w_next
//   mode 2: x1 = f32(f32(x_res + rmsnorm(y) * w_post) * scale), written to
//           x_out by workgroup 0 (x_out must not alias y or x_res), and
//           x = rmsnorm(x1) * w_next
// with rmsnorm as the norm kernels compute it (f64 sum of squares).
struct NormIn {
  const float *y, *w_post, *x_res, *w_next;
  float *x_out;
  float scale;
  int mode;  // 0: plain x
  double eps;
};

struct MatvecArgs {
  NormIn norm;
  WeightDesc w[kMaxWeights];
  int count;
  int total_tiles;
  TileGeom g;
  const float *x;     // f32 activations of this launch's first column, [cols][k]
  int k;              // input size (nb * 256)
  int cols;           // columns in this launch (<= kMaxCols)
  int out_col0;       // first output column written by this launch
  int total_units;    // half-split kernel: ceil(total_rows / Rh) units of Rh
                      // consecutive launch rows (a unit may span two weights)
  int total_rows;     // half-split kernel: the weights' rows summed
  int Rh;             // half-split kernel: rows per unit (floor(32 / S))
  float *pair_out;    // gate/up + GeGLU launch: [cols][rows] output
  const uint16_t *gelu_lut;  // the gelu table (hp_gelu.h gelu_lut)
  // non-null (launches of 2 or more columns): the input already quantised,
  // as the LDS image of this launch's columns (q8_image_bytes(cols, nb)),
  // copied in place of the Q8_K prologue
  const uint8_t *q8img;
  int wide_rows;      // wide kernel: launch rows per workgroup (with pair_out:
                      // rows of each of gate and up)
  // wide kernel: div_magic of nb, g.S and g.R (x / d as one high multiply)
  uint32_t mg_nb, mg_S, mg_R;
  int wide_half;      // wide kernel: 1 = tasks are half row-blocks (lane
                      // classes 4h .. 4h+3), up to 1024 threads
};

// x / d for 0 <= x < 2^20 as __umulhi(x, div_magic(d)) (0 for d = 1: x);
// exact for 1 <= d <= 256 (checked exhaustively).
__host__ __device__ constexpr uint32_t div_magic(int d) { return d <= 1 ? 0u : 0xFFFFFFFFu / (uint32_t)d + 1u; }

// x / d with m = div_magic(d) (0 <= x < 2^20, 1 <= d <= 256).  No branch (a
// divisor of 1 adds x back): a branch between loads would split the loaded
// registers' live ranges and make the compiler wait for them.
__device__ __forceinline__ int mdiv(int x, uint32_t m) {
  const uint32_t keep = 0u - (uint32_t)(m == 0u);
  return (int)(__umulhi((uint32_t)x, m) + ((uint32_t)x & keep));
}

// The vector-ALU matvec's LDS image of `cols` quantised input columns: the
// cols * nb Q8_K blocks (kQ8BlockBytes each, column-major) and then their
// cols * nb f32 scales, padded to 16 bytes.
__host__ __device__ constexpr size_t q8_image_bytes(int cols, int nb) {
  return (size_t)cols * nb * kQ8BlockBytes + (size_t)((cols * nb + 3) & ~3) * 4;
}

// Kernel entry: one dword of every 64-byte line of the kernel's argument
// segment (an argument struct of sizeof(T) bytes at its start), read as one
// batch of scalar loads followed by one wait, in one asm statement (the
// compiler splits such loads into dependent batches otherwise, each a round
// trip to memory).  The scalar loads of the arguments that follow then hit
// the scalar cache.  The loads complete inside the statement, so no load is
// in flight when its registers are reused.
template <int N>
__device__ __forceinline__ void kernarg_lines(const void *p);
template <>
__device__ __forceinline__ void kernarg_lines<1>(const void *p) {
  uint32_t d[1];
  asm volatile("s_load_dword %0, %1, 0x0\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<2>(const void *p) {
  uint32_t d[2];
  asm volatile("s_load_dword %0, %2, 0x0\n"
               "s_load_dword %1, %2, 0x40\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<3>(const void *p) {
  uint32_t d[3];
  asm volatile("s_load_dword %0, %3, 0x0\n"
               "s_load_dword %1, %3, 0x40\n"
               "s_load_dword %2, %3, 0x80\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<4>(const void *p) {
  uint32_t d[4];
  asm volatile("s_load_dword %0, %4, 0x0\n"
               "s_load_dword %1, %4, 0x40\n"
               "s_load_dword %2, %4, 0x80\n"
               "s_load_dword %3, %4, 0xc0\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<5>(const void *p) {
  uint32_t d[5];
  asm volatile("s_load_dword %0, %5, 0x0\n"
               "s_load_dword %1, %5, 0x40\n"
               "s_load_dword %2, %5, 0x80\n"
               "s_load_dword %3, %5, 0xc0\n"
               "s_load_dword %4, %5, 0x100\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<6>(const void *p) {
  uint32_t d[6];
  asm volatile("s_load_dword %0, %6, 0x0\n"
               "s_load_dword %1, %6, 0x40\n"
               "s_load_dword %2, %6, 0x80\n"
               "s_load_dword %3, %6, 0xc0\n"
               "s_load_dword %4, %6, 0x100\n"
               "s_load_dword %5, %6, 0x140\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<7>(const void *p) {
  uint32_t d[7];
  asm volatile("s_load_dword %0, %7, 0x0\n"
               "s_load_dword %1, %7, 0x40\n"
               "s_load_dword %2, %7, 0x80\n"
               "s_load_dword %3, %7, 0xc0\n"
               "s_load_dword %4, %7, 0x100\n"
               "s_load_dword %5, %7, 0x140\n"
               "s_load_dword %6, %7, 0x180\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<8>(const void *p) {
  uint32_t d[8];
  asm volatile("s_load_dword %0, %8, 0x0\n"
               "s_load_dword %1, %8, 0x40\n"
               "s_load_dword %2, %8, 0x80\n"
               "s_load_dword %3, %8, 0xc0\n"
               "s_load_dword %4, %8, 0x100\n"
               "s_load_dword %5, %8, 0x140\n"
               "s_load_dword %6, %8, 0x180\n"
               "s_load_dword %7, %8, 0x1c0\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<9>(const void *p) {
  uint32_t d[9];
  asm volatile("s_load_dword %0, %9, 0x0\n"
               "s_load_dword %1, %9, 0x40\n"
               "s_load_dword %2, %9, 0x80\n"
               "s_load_dword %3, %9, 0xc0\n"
               "s_load_dword %4, %9, 0x100\n"
               "s_load_dword %5, %9, 0x140\n"
               "s_load_dword %6, %9, 0x180\n"
               "s_load_dword %7, %9, 0x1c0\n"
               "s_load_dword %8, %9, 0x200\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<10>(const void *p) {
  uint32_t d[10];
  asm volatile("s_load_dword %0, %10, 0x0\n"
               "s_load_dword %1, %10, 0x40\n"
               "s_load_dword %2, %10, 0x80\n"
               "s_load_dword %3, %10, 0xc0\n"
               "s_load_dword %4, %10, 0x100\n"
               "s_load_dword %5, %10, 0x140\n"
               "s_load_dword %6, %10, 0x180\n"
               "s_load_dword %7, %10, 0x1c0\n"
               "s_load_dword %8, %10, 0x200\n"
               "s_load_dword %9, %10, 0x240\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<11>(const void *p) {
  uint32_t d[11];
  asm volatile("s_load_dword %0, %11, 0x0\n"
               "s_load_dword %1, %11, 0x40\n"
               "s_load_dword %2, %11, 0x80\n"
               "s_load_dword %3, %11, 0xc0\n"
               "s_load_dword %4, %11, 0x100\n"
               "s_load_dword %5, %11, 0x140\n"
               "s_load_dword %6, %11, 0x180\n"
               "s_load_dword %7, %11, 0x1c0\n"
               "s_load_dword %8, %11, 0x200\n"
               "s_load_dword %9, %11, 0x240\n"
               "s_load_dword %10, %11, 0x280\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10])
               : "s"(p));
}
template <>
__device__ __forceinline__ void kernarg_lines<12>(const void *p) {
  uint32_t d[12];
  asm volatile("s_load_dword %0, %12, 0x0\n"
               "s_load_dword %1, %12, 0x40\n"
               "s_load_dword %2, %12, 0x80\n"
               "s_load_dword %3, %12, 0xc0\n"
               "s_load_dword %4, %12, 0x100\n"
               "s_load_dword %5, %12, 0x140\n"
               "s_load_dword %6, %12, 0x180\n"
               "s_load_dword %7, %12, 0x1c0\n"
               "s_load_dword %8, %12, 0x200\n"
               "s_load_dword %9, %12, 0x240\n"
               "s_load_dword %10, %12, 0x280\n"
               "s_load_dword %11, %12, 0x2c0\n"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(d[0]), "=&s"(d[1]), "=&s"(d[2]), "=&s"(d[3]), "=&s"(d[4]), "=&s"(d[5]), "=&s"(d[6]), "=&s"(d[7]), "=&s"(d[8]), "=&s"(d[9]), "=&s"(d[10]), "=&s"(d[11])
               : "s"(p));
}
template <class T>
__device__ __forceinline__ void kernarg_warm() {
  constexpr int kLines = (int)((sizeof(T) + 63) / 64);
  static_assert(kLines >= 1 && kLines <= 12, "argument struct of at most 768 bytes");
  kernarg_lines<kLines>((const void *)__builtin_amdgcn_kernarg_segment_ptr());
}

// Launchers (return hipError_t of the launch).
hipError_t launch_q8k_natural(const float *x, int k, int cols, int8_t *qs, float *d, int16_t *bsums,
                              hipStream_t s);
hipError_t launch_matvec(const MatvecArgs &a, int num_cus, hipStream_t s);
// Half-split variant (two lanes per row-block, lane classes 0-3 / 4-7):
// needs S <= 32 and cols <= 4; a.w[].row_begin, total_rows, total_units, Rh set.
hipError_t launch_matvec_half(const MatvecArgs &a, int num_cus, hipStream_t s);
// Gate/up + GeGLU in one vector-ALU launch (count == 2, equal rows, cols <= 4):
// a.pair_out[m][r] = fround(gelu(gate) * up).
hipError_t launch_matvec_pair(const MatvecArgs &a, int num_cus, hipStream_t s);
// Wide kernel: one workgroup per a.wide_rows launch rows (every block of
// each row), products in LDS, block-order chains per (row, lane class).
// Uniform Q4_K or Q6_K weights, 1..4 columns; the norm prologue (one column,
// nb <= 16); with a.pair_out, gate/up + GeGLU (a.wide_rows rows of each).
size_t wide_lds_bytes(int cols, int nb, int type, int rows_per_wg);
int wide_threads(int cols, int nb, int rows_per_wg, bool half);
hipError_t launch_matvec_wide(const MatvecArgs &a, hipStream_t s);
// Q6_K also sets *f16_flag (zeroed by the caller) to 1 when some scale makes
// sc * (q - 32) inexact in f16, which the matrix-core kernels need exact.
hipError_t launch_repack(int type, const uint8_t *raw, int rows, const TileGeom &g, uint8_t *tiles,
                         uint16_t *dplane, uint32_t *f16_flag, hipStream_t s);
// Top-k (k <= kTopkMaxK) of each of `rows` (<= kTopkMaxRows) rows of n
// (<= kTopkMaxN) logits, optional softcap (cap > 0).  scratch holds
// topk_scratch_bytes(rows, n, k) bytes, zero when first used; the kernels
// leave their counters at zero again.  Calls sharing one scratch buffer must
// be ordered (one stream).
constexpr int kTopkMaxK = 64;
constexpr int kTopkMaxN = 524288;
constexpr int kTopkMaxRows = 16;
hipError_t launch_topk(const float *logits, int rows, int n, int k, double cap, uint8_t *scratch, uint32_t *ids,
                       float *vals, hipStream_t s);
size_t topk_scratch_bytes(int rows, int n, int k);
// Zeroes the counters a top-k scratch buffer must start with (one small kernel).
hipError_t launch_topk_clear(uint8_t *scratch, hipStream_t s);

// Next-token sampling over [cols][k] sorted candidates (count valid per
// column): one wave; rng points to the 32-bit generator state, advanced once
// per sampled column.  tokens [cols], probs [cols][k] (first kept[c] valid).
struct SampleParams {
  int do_sample;  // 0: greedy
  int top_k;      // >= 1
  double temperature;
  double top_p;
};
hipError_t launch_sample(const uint32_t *ids, const float *vals, int cols, int k, int count, const SampleParams &p,
                         uint32_t *rng, int32_t *tokens, double *probs, int32_t *kept, hipStream_t s);
// Matrix-core matvec (kquant_mfma.hip).  Each weight is read from its
// 16-row tile segments, or, where seg is null (one resident layout), from its
// tiles (geometry S, R of choose_geometry(k / 256)).
struct MfmaLaunch {
  const uint8_t *seg[kMaxWeights];
  const uint8_t *wt[kMaxWeights];
  const uint16_t *dplane[kMaxWeights];
  int S, R;
  float *out[kMaxWeights];
  int type[kMaxWeights];
  int rows[kMaxWeights];
  int count;
  const float *x;  // f32 input of the launch's first column
  int k;
  int cols;        // 1..8 columns in this launch
  int out_col0;
};
size_t mfma_segment_bytes(int type, int rows, int nb);
size_t mfma_lds_bytes(int cols, int nb);
hipError_t launch_repack_mfma(int type, const uint8_t *raw, int rows, int nb, uint8_t *segs, hipStream_t s);
// Some weight of the launch is kept in one layout: the launch reads every
// weight's tiles.
inline bool launch_reads_tiles(const MfmaLaunch &l) {
  for (int i = 0; i < l.count; i++)
    if (!l.seg[i]) return true;
  return false;
}
// The launch's tile geometry is the one choose_geometry gives its weights.
inline bool mfma_geometry_ok(const MfmaLaunch &l) {
  const int nb = l.k / kQK;
  return l.S >= 1 && l.R >= 1 && l.S * l.R <= 64 && nb >= 1 && nb % l.S == 0;
}
hipError_t launch_matvec_mfma(const MfmaLaunch &l, int num_cus, hipStream_t s);

// Prefill (many columns) on the matrix cores: a Q8_K pre-pass writes
// prefill_q8k_bytes(k, cols) of class-major quants, half-block sums and
// scales to `scratch`; launch_prefill runs every weight of `l` (l.x unused,
// l.cols = all columns, l.out_col0 = 0) over them.  Needs prefill_lds_bytes()
// of LDS per workgroup.
size_t prefill_q8k_bytes(int k, int cols);
size_t prefill_lds_bytes();
hipError_t launch_q8k_prefill(const float *x, int k, int cols, uint8_t *scratch, hipStream_t s);
hipError_t launch_prefill(const MfmaLaunch &l, const uint8_t *scratch, int num_cus, hipStream_t s);
// Fast prefill (within the 1e-4 relative tolerance of projections, not
// bit-exact): its own pre-pass of x into scratch (skipped with tiles_ready:
// the norm kernel already wrote the tiles, NormArgs::xt, at the scratch's
// start), then 128-row x 64-column
// tiles with the eight classes in one accumulator.  A launch with fewer
// tiles than two per CU splits each tile's blocks into consecutive ranges
// whose partial sums (in scratch) a reduction adds in range order.
// prefill_fast_bytes: the scratch of a launch of these weights' rows.
size_t prefill_fast_bytes(const MfmaLaunch &l, int num_cus);
int prefill_fast_launches(const MfmaLaunch &l, int num_cus);  // 2, or 3 with the reduction
// Gate/up (l.w 0 and 1, same type and rows) + GeGLU with the fast prefill
// kernel: out[m][r] = fround(gelu(gate) * up), gate and up as the fast
// kernel computes them; prefill_fast_geglu_bytes(l, num_cus) of scratch.
// When fewer than half a round of tiles trail the last full round, those
// tiles run as two block ranges whose sums a second kernel adds before the
// GeGLU (prefill_fast_geglu_launches: 2, or 3 with it).
size_t prefill_fast_geglu_bytes(const MfmaLaunch &l, int num_cus);
int prefill_fast_geglu_launches(const MfmaLaunch &l, int num_cus);
// Those trailing tiles' range sums may instead be left for the pre-pass of
// the next fast prefill launch, whose input is `out` (the down projection):
// with defer non-null and tail_part a buffer of
// prefill_fast_geglu_tail_bytes(l, num_cus) bytes, no tail kernel runs, the
// trailing tiles' outputs are not written, and *defer describes them (part
// null: none trail); the pre-pass forms those inputs from the sums with the
// same GeGLU, so its tiles are the same bits.
struct GegluTail {
  const float *part;
  const uint16_t *gelu_lut;
  int tail_full, col_tiles;
};
size_t prefill_fast_geglu_tail_bytes(const MfmaLaunch &l, int num_cus);
hipError_t launch_prefill_fast_geglu(const MfmaLaunch &l, const float *x, uint8_t *scratch, const uint16_t *gelu_lut,
                                     float *out, int num_cus, hipStream_t s, bool tiles_ready = false,
                                     GegluTail *defer = nullptr, float *tail_part = nullptr);
size_t prefill_fast_lds_bytes();
// A fast prefill launch may leave its block-range partial sums for the
// consumer to add (a norm launch, NormArgs::y_ks; the attention prologue,
// QkvPostArgs::src_ks): the caller sets part to a buffer of
// prefill_fast_part_bytes(l, num_cus) and passes it to launch_prefill_fast,
// which then launches no reduction and sets ks (> 1: range r of element e of
// weight w's [cols][rows] output at part[r * stride + off[w] + e]; 1: the
// outputs were written as usual).
constexpr int kNormParts = 4;
struct PrefillParts {
  float *part;
  size_t stride;
  size_t off[kMaxWeights];
  int ks;
};
size_t prefill_fast_part_bytes(const MfmaLaunch &l, int num_cus);
// tail (non-null part): x is a deferred GeGLU output (GegluTail above); the
// pre-pass (not tiles_ready) completes its trailing tiles' inputs.
hipError_t launch_prefill_fast(const MfmaLaunch &l, const float *x, uint8_t *scratch, int num_cus, hipStream_t s,
                               bool tiles_ready = false, PrefillParts *defer = nullptr,
                               const GegluTail *tail = nullptr);

// The gelu table (65536 f16 entries, hp_gelu.h gelu_lut) for the constant c.
hipError_t launch_gelu_lut(double c, uint16_t *lut, hipStream_t s);
// GeGLU of cols columns of `rows` (a multiple of 256) that also writes the
// result as a matvec input image (q8_image_bytes(cols, rows / 256)).
hipError_t launch_geglu_q8k(const float *gate, const float *up, int rows, int cols, const uint16_t *lut, float *out,
                            uint8_t *q8img, hipStream_t s);
hipError_t launch_geglu(const float *gate, const float *up, size_t n, const uint16_t *lut, float *out, int num_cus,
                        hipStream_t s);

// Decoder-layer steps for one decode token (decode_layer.hip).  Heads are
// kHeadDim wide; `position` points to the token's position in device memory.
constexpr int kHeadDim = 256;
constexpr int kAttnChunk = 32;    // cache slots per attention workgroup
constexpr int kAttnMaxGroup = 8;  // query heads per kv head
constexpr int kMaxTokens = 8;     // tokens of a decode call (a draft to verify) on the decode attention
constexpr int kMaxChunkTokens = 4096;  // tokens of one prefill chunk (the prefill attention beyond 8)
constexpr int kMaxLayerTokens = 65536; // tokens of one decoder-layers call (in chunks of <= kMaxChunkTokens)

// Per row of [rows][n] (n <= 4096): x_res == null: next_out = rmsnorm(y) *
// w_next.  Otherwise x_out = f32(f32(x_res + rmsnorm(y) * w_post) * scale)
// and, if next_out != null, next_out = rmsnorm(x_out) * w_next.  A null
// norm weight means a norm without weight.
struct NormArgs {
  const float *y, *w_post, *x_res, *w_next;
  float *x_out, *next_out;
  uint8_t *q8img;  // non-null: next_out also as a matvec input image (q8_image_bytes(rows, n / 256))
  // non-null: next_out also as the fast prefill kernel's activation tiles
  // (hp_f2tile.h; row r is column r; the grid covers whole 64-column tiles,
  // workgroups past `rows` write their padding columns as zeros)
  uint8_t *xt;
  // x16: 16-lane groups hold whole 256-element blocks (norm_residual_x16_kernel;
  // n a multiple of 256, at most 4096): the norms that feed a projection
  int x16;
  // next_image_only: the launch that follows reads only q8img or xt, so the
  // f32 values of next_out are formed for them but not stored (prefill
  // chunks through all layers 10.86 -> 10.82 ms)
  int next_image_only;
  // y_ks > 1: y holds y_ks block-range partial sums of the projection, range
  // r of element e at y[r * y_stride + e], added in range order (as
  // f2_reduce_kernel adds them); at most kNormParts
  int y_ks;
  size_t y_stride;
  float scale;
  int n, rows;
  double eps;
};
struct QkvPostArgs {
  const float *q, *k, *v;  // projections [heads][kHeadDim]
  const float *wq, *wk;    // head norm weights [kHeadDim]
  const float *freq_factors;  // [rope_dims / 2] or null
  const int *position;
  float *q_out;
  // non-null: the queries leave as the f16 bits of float32_to_float16, the
  // rounding the attention applies, in place of q_out (rows as q_out's)
  uint16_t *q_half;
  _Float16 *k_cache, *v_cache;  // [nkv][capacity][kHeadDim]
  double2 *rope_table;  // [tokens][kHeadDim / 2] cos, sin (rope_table_mode 1: written, 2: read)
  int rope_table_mode;
  int nq, nkv, capacity, rope_dims;
  int tokens;          // token t at position *position + pos_offset + t; rows [t][heads][kHeadDim]
  int pos_offset;
  // src_ks > 1: q, k, v hold src_ks block-range partial sums, range r of
  // element e at [r * src_stride + e], added in range order (at most kNormParts)
  int src_ks;
  size_t src_stride;
  double theta_scale;  // base^(-2 / rope_dims)
  double eps;
};
// prep == 0: q holds the queries after RoPE and the caches already hold the
// token.  prep == 1: q, k, v are the token's projections ([heads][kHeadDim],
// v may equal k); the kernel applies the head norms (wq, wk; v without
// weight) and RoPE and appends the key and value at slot position % capacity.
struct AttnArgs {
  const float *q, *k, *v;
  // prefill attention only: non-null, the queries already rounded to f16
  // (float32_to_float16 bits, rows as q's), read in place of q
  const uint16_t *q_half;
  // prefill attention only: non-null, the slice merge also writes out as
  // the fast prefill kernel's activation tiles (hp_f2tile.h; K = nq * 256,
  // whole 64-column tiles, padding columns as zeros), the next projection's
  // input
  uint8_t *o_tiles;
  const float *wq, *wk, *freq_factors;
  _Float16 *k_cache, *v_cache;
  const int *position;
  float *out;      // [nq][kHeadDim], f16-rounded
  float *part_m, *part_l, *part_o;  // set by launch_attention
  double2 *rope_table;  // [kHeadDim / 2] cos, sin (rope_table_mode 1: written, 2: read)
  int nq, nkv, capacity, window, chunks, rope_dims, prep, rope_table_mode;
  int tokens;  // prep == 0: queries of tokens *position + pos_offset .. + tokens - 1, rows [t][nq][kHeadDim]
  int pos_offset;
  int qsplit;  // set by launch_attention: workgroups per (chunk, kv head), each taking nq / nkv / qsplit query heads
  double theta_scale, eps;
};
hipError_t launch_norm_residual(const NormArgs &a, hipStream_t s);
hipError_t launch_qkv_post(const QkvPostArgs &a, hipStream_t s);
// partials: attn_partial_floats(nkv, capacity) floats of device scratch
// (a.rope_table, when used, lives elsewhere).
size_t attn_partial_floats(int nkv, int capacity, int tokens);
hipError_t launch_attention(AttnArgs a, float *partials, hipStream_t s);
// The merge of attention partials (a.part_m/l/o, a.chunks slices per row)
// into a.out: exp-weighted sum, division by l, castF16Rows.
hipError_t launch_attention_merge(const AttnArgs &a, hipStream_t s);
// Prefill attention (attn_prefill.hip): a chunk of a.tokens (<= capacity,
// <= kMaxChunkTokens) queries after RoPE, causal over the caches, in
// `ranges` window slices merged by launch_attention_merge.
constexpr int kAttnPrefillMaxRanges = 16;
int attn_prefill_ranges(int tokens, int nq, int nkv, int capacity, int num_cus);
size_t attn_prefill_partial_floats(int nkv, int tokens, int ranges);
hipError_t launch_attention_prefill(AttnArgs a, float *partials, int ranges, hipStream_t s);
hipError_t launch_dequantize(int type, const uint8_t *tiles, const uint16_t *dplane, int rows,
                             const TileGeom &g, int row_start, int row_count, float *out, hipStream_t s);

}  // namespace hp
