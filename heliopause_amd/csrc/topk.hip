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
// number) and padding to key 0.  A larger key is a better candidate, and
// keys of distinct ids never tie.
//
// Stage 1 (grid [chunks][rows], 4 waves): each lane register-sorts E keys,
// the lanes' sorted lists go to LDS, and each wave extracts its top-k by
// repeated maximum of the 64 list heads (DPP within 16-lane rows, readlane
// across rows).  Wave 0 then merges the 4 wave lists the same way and
// writes the chunk's k candidates.  Stage 2 (one wave per row) merges the
// <= 64 chunk lists, gathers the values by id and writes (id, value).
#include "hp_common.h"
#include "hp_tanh.h"

namespace hp {

constexpr int kTopkMaxK = 64;

__device__ __forceinline__ uint32_t ord_bits(float v) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (v != v) return 0u;                   // NaN: below every number
  if (v == 0.0f) b = 0u;                   // -0 ties with +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float softcap_value(float v, double cap) {
  return cap > 0.0 ? (float)(hp_tanh((double)v / cap) * cap) : v;
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

// Descending bitonic sort of N keys held in registers (N a power of two).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&a)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; i++) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint64_t x = a[i], y = a[j];
          const bool sw = desc ? (x < y) : (x > y);
          a[i] = sw ? y : x;
          a[j] = sw ? x : y;
        }
      }
}

// Top-k (k <= 64) of up to 64 descending lists, one per lane, stored in LDS
// at list + lane * stride with len entries each.  Returns this lane's
// element of the merged result: lane t holds the t-th best key (0 padding).
__device__ __forceinline__ uint64_t wave_merge(const uint64_t *list, int stride, int len, int k, int lane) {
  int ptr = 0;
  uint64_t head = len > 0 ? list[lane * stride] : 0;
  uint64_t nxt = len > 1 ? list[lane * stride + 1] : 0;
  uint64_t mine = 0;
  for (int t = 0; t < k; t++) {
    const uint64_t m = wave_max_u64(head);
    if (lane == t) mine = m;
    if (m == 0) break;  // only padding remains
    if (head == m) {     // keys are unique: exactly one lane advances
      ptr++;
      head = nxt;
      nxt = ptr + 1 < len ? list[lane * stride + ptr + 1] : 0;
    }
  }
  return mine;
}

template <int E>
__global__ __launch_bounds__(256) void topk_stage1(const float *__restrict__ logits, int n, int k, double cap,
                                                   uint64_t *__restrict__ cand) {
  __shared__ uint64_t lists[4][64][E];  // per wave, per lane sorted keys
  __shared__ uint64_t wl[4][kTopkMaxK];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int base = chunk * 256 * E + wave * 64 * E + lane * E;
  const float *src = logits + (size_t)row * n;
  uint64_t key[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int id = base + i;
    key[i] = 0;
    if (id < n) {
      const float v = softcap_value(src[id], cap);
      key[i] = ((uint64_t)ord_bits(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)id);
    }
  }
  sort_desc<E>(key);
#pragma unroll
  for (int i = 0; i < E; i++) lists[wave][lane][i] = key[i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint64_t mine = wave_merge(&lists[wave][0][0], E, E, k, lane);
  if (lane < k) wl[wave][lane] = mine;
  __syncthreads();
  if (wave == 0) {
    const uint64_t best = wave_merge(&wl[0][0], kTopkMaxK, lane < 4 ? k : 0, k, lane);
    if (lane < k) cand[((size_t)row * gridDim.x + chunk) * k + lane] = best;
  }
}

__global__ __launch_bounds__(64) void topk_stage2(const float *__restrict__ logits, int n, int k, double cap,
                                                  const uint64_t *__restrict__ cand, int chunks,
                                                  uint32_t *__restrict__ ids, float *__restrict__ vals) {
  __shared__ uint64_t lists[64 * kTopkMaxK];
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  for (int i = lane; i < chunks * k; i += 64) lists[i] = cand[(size_t)row * chunks * k + i];
  __syncthreads();
  const uint64_t best = wave_merge(lists, k, lane < chunks ? k : 0, k, lane);
  if (lane < k) {
    uint32_t id = 0xFFFFFFFFu;
    float v = 0.0f;
    if (best != 0) {
      id = 0xFFFFFFFFu - (uint32_t)best;
      v = softcap_value(logits[(size_t)row * n + id], cap);
    }
    ids[(size_t)row * k + lane] = id;
    vals[(size_t)row * k + lane] = v;
  }
}

int topk_elements_per_lane(int n) {
  for (int e = 16; e <= 32; e <<= 1)
    if ((long long)64 * 256 * e >= n) return e;
  return 0;
}

hipError_t launch_topk(const float *logits, int rows, int n, int k, double cap, uint64_t *cand, uint32_t *ids,
                       float *vals, hipStream_t s) {
  const int e = topk_elements_per_lane(n);
  if (e == 0 || k < 1 || k > kTopkMaxK) return hipErrorInvalidValue;
  const int chunks = (n + 256 * e - 1) / (256 * e);
  const dim3 g1(chunks, rows);
  if (e == 16)
    hipLaunchKernelGGL(topk_stage1<16>, g1, dim3(256), 0, s, logits, n, k, cap, cand);
  else
    hipLaunchKernelGGL(topk_stage1<32>, g1, dim3(256), 0, s, logits, n, k, cap, cand);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(topk_stage2, dim3(rows), dim3(64), 0, s, logits, n, k, cap, cand, chunks, ids, vals);
  return hipGetLastError();
}

size_t topk_candidate_bytes(int rows, int n, int k) {
  const int e = topk_elements_per_lane(n);
  if (e == 0) return 0;
  const int chunks = (n + 256 * e - 1) / (256 * e);
  return (size_t)rows * chunks * k * sizeof(uint64_t);
}

}  // namespace hp
