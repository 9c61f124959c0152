// topk.hip -- per-row top-k over logits on gfx950, candidates only read back.
//
// Semantics: packages/engine/src/runtime.ts:514-527 (topK): the k largest
// values in descending order, equal values in increasing id order (the
// stable sort keeps ids ascending; -0 and +0 compare equal).  Optional
// softcap first, as packages/engine/src/runner/wasm/layers.ts:407-412 applies
// it to every logit: v' = fround(tanh(v / c) * c) in f64.
//
// Key: (ord(v) << 32) | (0xFFFFFFFF - id), where ord is the order-preserving
// map of the f32 bits with -0 folded onto +0; NaN maps to ord 0 (below every
// number).  A larger key is a better candidate, keys of distinct ids never
// tie, and every real key is >= 1 (0 is padding).
//
// Selection by a provable lower bound.  A row is cut into G chunks of 1024
// logits.  If t is the k-th largest of the G chunk maxima, the k chunks whose
// maxima are >= t hold k distinct keys >= t, so the row's k-th largest key
// K* >= t: every top-k key passes the filter key >= t, and only those k
// chunks can contribute, so at most k * 1024 keys pass (G < k: t = 0 and all
// n keys pass).  For i.i.d. logits about 43 of 262144 pass for k = 40.
//
//   topk_max_kernel    (G x rows): chunk maxima.
//   topk_filter_kernel (G x rows): every workgroup selects t from the G
//                      maxima (radix select in LDS) and appends its keys
//                      >= t to the row's candidate list (slots reserved with
//                      one atomic add per workgroup).
//   topk_final_kernel  (rows): the exact top k of the candidates (<= 64: one
//                      bitonic sort in a wave; more: radix select for K*,
//                      then the sort), values gathered by id, (id, value)
//                      written, the candidate count reset to 0.
// Data crosses workgroups only at kernel boundaries and through the atomic
// slot counter, so no workgroup needs a device-wide memory fence.
#include "hp_common.h"
#include "hp_tanh.h"

namespace hp {

constexpr int kTopkChunk = 1024;  // logits per workgroup: 256 threads x 4
constexpr int kTopkThreads = 256;

// Scratch: a fixed header of kTopkMaxRows x 16 bytes holding each row's u32
// candidate count, at the same place for every shape, so the zero the final
// kernel leaves behind serves the next call of any shape; then per row, at
// kTopkHeader + row * stride: u64 maxima[G], u64 candidates.
constexpr size_t kTopkHeader = 16 * kTopkMaxRows;
struct RowScratch {
  uint32_t *ncand;
  uint64_t *maxima, *cand;
};

__host__ __device__ inline size_t topk_candidate_capacity(int n, int k) {
  return (size_t)n < (size_t)k * kTopkChunk ? (size_t)n : (size_t)k * kTopkChunk;
}

__host__ __device__ inline size_t topk_row_stride(int n, int k) {
  const size_t g = (size_t)(n + kTopkChunk - 1) / kTopkChunk;
  return (8 * g + 8 * topk_candidate_capacity(n, k) + 255) & ~(size_t)255;
}

__device__ __forceinline__ RowScratch row_scratch(uint8_t *base, size_t stride, int row, int g) {
  RowScratch r;
  r.ncand = reinterpret_cast<uint32_t *>(base + 16 * (size_t)row);
  r.maxima = reinterpret_cast<uint64_t *>(base + kTopkHeader + (size_t)row * stride);
  r.cand = r.maxima + g;
  return r;
}

__device__ __forceinline__ uint32_t ord_bits(float v) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (v != v) return 0u;                   // NaN: below every number
  if (v == 0.0f) b = 0u;                   // -0 ties with +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float softcap_value(float v, double cap) {
  return cap > 0.0 ? (float)(hp_tanh((double)v / cap) * cap) : v;
}

__device__ __forceinline__ uint64_t make_key(float v, uint32_t id) {
  return ((uint64_t)ord_bits(v) << 32) | (uint64_t)(0xFFFFFFFFu - id);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

template <int CTRL>
__device__ __forceinline__ uint64_t max_step(uint64_t k) {
  const uint32_t hi = dpp_u32<CTRL>((uint32_t)(k >> 32));
  const uint32_t lo = dpp_u32<CTRL>((uint32_t)k);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > k ? o : k;
}

// Maximum of one u64 per lane over the whole wave (wave-uniform result).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  k = max_step<0xB1>(k);   // quad_perm [1,0,3,2]
  k = max_step<0x4E>(k);   // quad_perm [2,3,0,1]
  k = max_step<0x141>(k);  // row_half_mirror
  k = max_step<0x140>(k);  // row_mirror
  uint64_t best = 0;
#pragma unroll
  for (int row = 0; row < 4; row++) {
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), row * 16);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, row * 16);
    const uint64_t v = ((uint64_t)hi << 32) | lo;
    best = v > best ? v : best;
  }
  return best;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const int lo = __shfl_xor((int)(uint32_t)v, mask, 64);
  const int hi = __shfl_xor((int)(uint32_t)(v >> 32), mask, 64);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Descending bitonic sort of one u64 per lane across the 64 lanes.
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t other = shfl_xor_u64(key, stride);
      const bool desc = (lane & size) == 0 || size == 64;
      const bool lower = (lane & stride) == 0;
      const bool take_max = lower == desc;
      const uint64_t hi = key > other ? key : other;
      const uint64_t lo = key > other ? other : key;
      key = take_max ? hi : lo;
    }
  return key;
}

// Radix select over `count` distinct keys at keys[0..count) (global or LDS):
// returns T such that exactly `rank` keys are >= T (1 <= rank <= count).
// All kTopkThreads threads of the workgroup must call it.  8-bit digits from
// the top; stops as soon as the chosen bin holds exactly the keys still
// needed.
__device__ uint64_t radix_select(const uint64_t *keys, uint32_t count, uint32_t rank) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick_bin, pick_above;
  const int tid = threadIdx.x;
  uint64_t prefix = 0, pmask = 0;
  uint32_t rem = rank;
  for (int shift = 56; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < count; i += kTopkThreads) {
      const uint64_t key = keys[i];
      if ((key & pmask) == prefix) atomicAdd(&hist[(uint32_t)(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane L holds bins 4L..4L+3; suffix sums over higher lanes
      const uint32_t h0 = hist[4 * tid], h1 = hist[4 * tid + 1], h2 = hist[4 * tid + 2], h3 = hist[4 * tid + 3];
      const uint32_t own = h0 + h1 + h2 + h3;
      uint32_t incl = own;  // inclusive suffix sum: lanes >= tid
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_down(incl, d, 64);
        if (tid + d < 64) incl += o;
      }
      uint32_t above = incl - own;  // keys in bins of higher lanes
      const uint32_t hb[4] = {h0, h1, h2, h3};
#pragma unroll
      for (int j = 3; j >= 0; j--) {
        if (above < rem && above + hb[j] >= rem) {
          pick_bin = 4 * tid + j;
          pick_above = above;
        }
        above += hb[j];
      }
    }
    __syncthreads();
    const uint32_t b = pick_bin;
    rem -= pick_above;
    prefix |= (uint64_t)b << shift;
    pmask |= (uint64_t)255 << shift;
    const bool exact = hist[b] == rem;
    __syncthreads();  // hist is cleared by the next pass
    if (exact) break;
  }
  return prefix;
}

// Loads this thread's 4 logits of a chunk (ids chunk*1024 + i*256 + tid) as keys.
__device__ __forceinline__ void chunk_keys(const float *__restrict__ src, int n, int chunk, double cap,
                                           uint64_t (&key)[4]) {
  float v[4];
  const int base = chunk * kTopkChunk + threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int id = base + i * kTopkThreads;
    v[i] = id < n ? src[id] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int id = base + i * kTopkThreads;
    key[i] = id < n ? make_key(softcap_value(v[i], cap), (uint32_t)id) : 0;
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_max_kernel(const float *__restrict__ logits, int n, double cap,
                                                                uint8_t *scratch, size_t stride) {
  __shared__ uint64_t wmax[kTopkThreads / 64];
  const int g = gridDim.x, chunk = blockIdx.x, row = blockIdx.y;
  const RowScratch rs = row_scratch(scratch, stride, row, g);
  uint64_t key[4];
  chunk_keys(logits + (size_t)row * n, n, chunk, cap, key);
  uint64_t m = key[0];
#pragma unroll
  for (int i = 1; i < 4; i++) m = key[i] > m ? key[i] : m;
  m = wave_max_u64(m);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) wmax[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wmax[0];
    for (int w = 1; w < kTopkThreads / 64; w++) b = wmax[w] > b ? wmax[w] : b;
    rs.maxima[chunk] = b;
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_filter_kernel(const float *__restrict__ logits, int n, int k,
                                                                   double cap, uint8_t *scratch, size_t stride) {
  __shared__ uint64_t maxima[kTopkMaxN / kTopkChunk];
  __shared__ uint32_t wcount[kTopkThreads / 64];
  __shared__ uint32_t wbase[kTopkThreads / 64];
  const int g = gridDim.x, chunk = blockIdx.x, row = blockIdx.y;
  const RowScratch rs = row_scratch(scratch, stride, row, g);
  const uint32_t cap_cand = (uint32_t)topk_candidate_capacity(n, k);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  uint64_t key[4];
  chunk_keys(logits + (size_t)row * n, n, chunk, cap, key);
  // t = k-th largest chunk maximum (every chunk holds a real key, since
  // G = ceil(n / 1024)); G < k: t = 0 and every key passes
  uint64_t t = 0;
  if (g >= k) {
    for (int i = threadIdx.x; i < g; i += kTopkThreads) maxima[i] = rs.maxima[i];
    __syncthreads();
    t = radix_select(maxima, (uint32_t)g, (uint32_t)k);
  }
  // wave-local positions of passing keys, slot-major
  uint32_t pos[4];
  uint32_t total = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const bool pass = key[i] != 0 && key[i] >= t;
    const uint64_t mask = __ballot(pass);
    pos[i] = pass ? total + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u))
                  : 0xFFFFFFFFu;
    total += (uint32_t)__popcll(mask);
  }
  if (lane == 0) wcount[wave] = total;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t sum = 0;
    for (int w = 0; w < kTopkThreads / 64; w++) {
      wbase[w] = sum;
      sum += wcount[w];
    }
    const uint32_t base = sum ? atomicAdd(rs.ncand, sum) : 0;
    for (int w = 0; w < kTopkThreads / 64; w++) wbase[w] += base;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // at most min(n, k * 1024) keys pass (see the header); the bound check
    // only guards the buffer
    const uint32_t at = wbase[wave] + pos[i];
    if (pos[i] != 0xFFFFFFFFu && at < cap_cand) rs.cand[at] = key[i];
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_final_kernel(const float *__restrict__ logits, int n, int k,
                                                                  double cap, uint8_t *scratch, size_t stride,
                                                                  uint32_t *__restrict__ ids,
                                                                  float *__restrict__ vals) {
  __shared__ uint32_t nsel;
  __shared__ uint64_t sel[kTopkMaxK];
  const int g = (n + kTopkChunk - 1) / kTopkChunk, row = blockIdx.x;
  const RowScratch rs = row_scratch(scratch, stride, row, g);
  const float *src = logits + (size_t)row * n;
  const uint32_t cap_cand = (uint32_t)topk_candidate_capacity(n, k);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t stored = *rs.ncand;
  const uint32_t count = stored < cap_cand ? stored : cap_cand;
  const uint32_t want = count < (uint32_t)k ? count : (uint32_t)k;
  uint64_t mine = 0;  // wave 0: this lane's key of the final sort
  if (count <= 64) {
    if (wave == 0) mine = lane < (int)count ? rs.cand[lane] : 0;
  } else {
    const uint64_t kth = radix_select(rs.cand, count, want);
    if (threadIdx.x == 0) nsel = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < count; i += kTopkThreads) {
      const uint64_t c = rs.cand[i];
      if (c >= kth) {
        const uint32_t slot = atomicAdd(&nsel, 1u);  // exactly `want` (<= 64) keys pass
        if (slot < (uint32_t)kTopkMaxK) sel[slot] = c;
      }
    }
    __syncthreads();
    if (wave == 0) mine = lane < (int)nsel ? sel[lane] : 0;  // nsel == want <= 64
  }
  if (wave == 0) {
    mine = wave_sort_desc(mine, lane);
    if (lane < k) {
      uint32_t id = 0xFFFFFFFFu;
      float v = 0.0f;
      const uint32_t cid = 0xFFFFFFFFu - (uint32_t)mine;
      if (mine != 0 && (uint32_t)lane < want && cid < (uint32_t)n) {
        id = cid;
        v = softcap_value(src[id], cap);
      }
      ids[(size_t)row * k + lane] = id;
      vals[(size_t)row * k + lane] = v;
    }
    if (lane == 0) *rs.ncand = 0;
  }
}

size_t topk_scratch_bytes(int rows, int n, int k) { return kTopkHeader + (size_t)rows * topk_row_stride(n, k); }

// Zeroes the per-row candidate counters at the head of a scratch buffer (a
// kernel rather than a memset, so a captured graph replays it faithfully).
__global__ __launch_bounds__(64) void topk_clear_kernel(uint32_t *header) {
  for (int i = threadIdx.x; i < (int)(kTopkHeader / 4); i += 64) header[i] = 0u;
}

hipError_t launch_topk_clear(uint8_t *scratch, hipStream_t s) {
  hipLaunchKernelGGL(topk_clear_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<uint32_t *>(scratch));
  return hipGetLastError();
}

hipError_t launch_topk(const float *logits, int rows, int n, int k, double cap, uint8_t *scratch, uint32_t *ids,
                       float *vals, hipStream_t s) {
  if (n < 1 || n > kTopkMaxN || k < 1 || k > kTopkMaxK || rows < 1 || rows > kTopkMaxRows)
    return hipErrorInvalidValue;
  const int g = (n + kTopkChunk - 1) / kTopkChunk;
  const size_t stride = topk_row_stride(n, k);
  const dim3 grid(g, rows);
  hipLaunchKernelGGL(topk_max_kernel, grid, dim3(kTopkThreads), 0, s, logits, n, cap, scratch, stride);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(topk_filter_kernel, grid, dim3(kTopkThreads), 0, s, logits, n, k, cap, scratch, stride);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(topk_final_kernel, dim3(rows), dim3(kTopkThreads), 0, s, logits, n, k, cap, scratch, stride,
                     ids, vals);
  return hipGetLastError();
}

}  // namespace hp
