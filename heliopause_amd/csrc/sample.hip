// sample.hip -- next-token sampling from top-k candidates, on the device.
//
// Restates tokenSamplingDistribution / sampleNextToken with their softmax,
// applyTopP and createDeterministicRng (packages/engine/src/generation.ts
// 78-165) over the [columns][k] candidates the top-k kernels leave in HBM, so
// a decode loop can pick the next token without a host round trip.  JS
// numbers are IEEE doubles: every step here is a double operation in the
// reference's order (no contraction), Math.exp is hp_exp (the JS engine's
// algorithm), and the sums the reference takes left to right (softmax total,
// top-p and draw cumulatives) are taken left to right by one lane.  Columns
// are sampled in order from one generator state, as the reference draws
// them one after another; greedy columns draw nothing.
#include "hp_common.h"
#include "hp_exp.h"

namespace hp {

namespace {

constexpr int kLanes = 64;

// createDeterministicRng (generation.ts:78-87): the JS operations are 32-bit
// wrapping ones (Math.imul, ToInt32 of a sum of two int32, >>> 0).
__device__ __forceinline__ double rng_next(uint32_t &state) {
  state += 0x6D2B79F5u;
  uint32_t v = state;
  v = (v ^ (v >> 15)) * (v | 1u);
  v ^= v + (v ^ (v >> 7)) * (v | 61u);
  return (double)(v ^ (v >> 14)) / 4294967296.0;
}

// softmax (generation.ts:157-165) of the n values held by lanes 0..n-1;
// returns this lane's probability (0 for lanes >= n).
__device__ double softmax_lane(double x, int n, double *sh, double *total) {
  const int lane = threadIdx.x;
  const bool valid = lane < n;
  // Math.max over the values from -Infinity: NaN if any value is NaN.  The
  // sign of a zero maximum cannot change exp(x - max).
  const bool nan = valid && __builtin_isnan(x);
  double m = valid && !nan ? x : -__builtin_inf();
#pragma unroll
  for (int off = kLanes / 2; off > 0; off >>= 1) {
    const double o = __shfl_xor(m, off);
    m = o > m ? o : m;
  }
  if (__any(nan)) m = __builtin_nan("");
  const double e = valid ? hp_exp(x - m) : 0.0;
  sh[lane] = e;
  __syncthreads();
  if (lane == 0) {
    double s = 0.0;
    for (int i = 0; i < n; i++) s = s + sh[i];
    *total = s;
  }
  __syncthreads();
  const double s = *total;
  double p;
  if (s <= 0.0 || !__builtin_isfinite(s))
    p = lane == 0 ? 1.0 : 0.0;
  else
    p = e / s;
  __syncthreads();  // sh is reused by the caller
  return valid ? p : 0.0;
}

__global__ __launch_bounds__(kLanes) void sample_kernel(const uint32_t *__restrict__ ids,
                                                        const float *__restrict__ vals, int cols, int k, int count,
                                                        SampleParams p, uint32_t *__restrict__ rng,
                                                        int32_t *__restrict__ tokens, double *__restrict__ probs,
                                                        int32_t *__restrict__ kept) {
  __shared__ double sh[kLanes];
  __shared__ uint32_t sh_id[kLanes];
  __shared__ double total;
  __shared__ int sh_n;
  const int lane = threadIdx.x;
  const bool greedy = p.do_sample == 0 || p.temperature == 0.0;
  uint32_t state = rng[0];
  for (int c = 0; c < cols; c++) {
    const uint32_t id = lane < count ? ids[(size_t)c * k + lane] : 0u;
    const double v = lane < count ? (double)vals[(size_t)c * k + lane] : 0.0;
    if (greedy) {  // the best candidate with probability 1; no draw
      if (lane == 0) {
        tokens[c] = (int32_t)id;
        probs[(size_t)c * k] = 1.0;
        kept[c] = 1;
      }
      continue;
    }
    sh_id[lane] = id;
    const int n1 = count < p.top_k ? count : p.top_k;  // topK slice of the sorted candidates
    int n2 = n1;
    if (!(p.top_p >= 1.0) && n1 > 1) {  // applyTopP (generation.ts:135-155)
      const double q = softmax_lane(v, n1, sh, &total);
      sh[lane] = q;
      __syncthreads();
      if (lane == 0) {
        double cum = 0.0;
        int n = n1;
        for (int i = 0; i < n1; i++) {
          cum = cum + sh[i];
          if (cum >= p.top_p) {
            n = i + 1;
            break;
          }
        }
        sh_n = n;
      }
      __syncthreads();
      n2 = sh_n;
      __syncthreads();
    }
    const double q = softmax_lane(v / p.temperature, n2, sh, &total);
    if (lane < n2) probs[(size_t)c * k + lane] = q;
    sh[lane] = q;
    __syncthreads();
    if (lane == 0) {  // sampleNextToken (generation.ts:89-108)
      const double draw = rng_next(state);
      double cum = 0.0;
      int32_t tok = (int32_t)sh_id[n2 - 1];
      for (int i = 0; i < n2; i++) {
        cum = cum + sh[i];
        if (draw < cum) {
          tok = (int32_t)sh_id[i];
          break;
        }
      }
      tokens[c] = tok;
      kept[c] = n2;
    }
    __syncthreads();
  }
  if (lane == 0) rng[0] = state;
}

}  // namespace

hipError_t launch_sample(const uint32_t *ids, const float *vals, int cols, int k, int count, const SampleParams &p,
                         uint32_t *rng, int32_t *tokens, double *probs, int32_t *kept, hipStream_t s) {
  if (cols < 1 || k < 1 || k > kLanes || count < 1 || count > k || p.top_k < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kLanes), 0, s, ids, vals, cols, k, count, p, rng, tokens, probs,
                     kept);
  return hipGetLastError();
}

}  // namespace hp
