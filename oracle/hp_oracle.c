/*
 * hp_oracle.c -- CPU restatement of heliopause's Q4_K/Q6_K projection path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See hp_oracle.h.
 *
 * Reference files followed (paths relative to the heliopause repository):
 *   packages/engine/wasm-kernels/src/lib.rs     -- kernels and numerics
 *   packages/engine/src/quant.ts                -- TS f16 conversions (gelu)
 *   packages/engine/src/runner/wasm/layers.ts   -- gelu / GeGLU / softcap
 *   packages/engine/src/runtime.ts              -- topK
 *   packages/engine/src/runner/wasm/thread-pool.ts -- splitRows sharding
 *
 * Pinning: every function is checked by tests/test_oracle_*.py against the
 * reference's known answers, closed forms, brute force or V8's own outputs.
 * Open item, parity unpinned: bit-level agreement of the vec-dot f32 tail
 * (hpo_vec_dot_*) with the compiled WASM module, which cannot run here; its
 * operation order follows lib.rs:1961-1967 and 2163-2171, and its values are
 * checked against an f64 dot to 2e-6.
 */
#include "hp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <unistd.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256

static size_t sat_mul(size_t a, size_t b) {
  size_t r;
  if (__builtin_mul_overflow(a, b, &r)) return (size_t)-1;
  return r;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---------------------------------------------------------------------- */
/* lib.rs:2507-2532 float16_to_float32 (exact, keeps NaN payload bits).    */
float hpo_f16_to_f32(uint16_t value) {
  uint32_t sign = ((uint32_t)(value & 0x8000u)) << 16;
  int32_t exponent = (value >> 10) & 0x1f;
  uint32_t fraction = value & 0x03ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (fraction == 0) {
      bits = sign;
    } else {
      uint32_t mantissa = fraction;
      int32_t e = -14;
      while ((mantissa & 0x0400u) == 0) {
        mantissa <<= 1;
        e -= 1;
      }
      mantissa &= 0x03ffu;
      bits = sign | ((uint32_t)(e + 127) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (fraction << 13);
  } else {
    bits = sign | ((uint32_t)(exponent + 112) << 23) | (fraction << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Bit pattern of hpo_f16_to_f32 (keeps signalling NaNs intact for tests). */
uint32_t hpo_f16_to_f32_bits(uint16_t value) {
  float f = hpo_f16_to_f32(value);
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* lib.rs:2534-2569 float32_to_float16 (round half up on the mantissa). */
uint16_t hpo_f32_to_f16_rust(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
  uint32_t mantissa = bits & 0x007fffffu;
  if (exponent == 0xff) return mantissa == 0 ? (uint16_t)(sign | 0x7c00u) : (uint16_t)0x7e00u;
  int32_t half_exponent = exponent - 127 + 15;
  if (half_exponent >= 31) return (uint16_t)(sign | 0x7bffu);
  if (half_exponent <= 0) {
    if (half_exponent < -10) return sign;
    uint32_t with_hidden = mantissa | 0x00800000u;
    uint32_t shift = (uint32_t)(14 - half_exponent);
    uint32_t rounded = (with_hidden + (1u << (shift - 1))) >> shift;
    return (uint16_t)(sign | rounded);
  }
  uint32_t rounded_mantissa = mantissa + 0x00001000u;
  if (rounded_mantissa & 0x00800000u) {
    int32_t rounded_exponent = half_exponent + 1;
    if (rounded_exponent >= 31) return (uint16_t)(sign | 0x7bffu);
    return (uint16_t)(sign | (rounded_exponent << 10));
  }
  return (uint16_t)(sign | (half_exponent << 10) | (rounded_mantissa >> 13));
}

/* quant.ts:618-630 float16ToFloat32 (f64 result; exact for every input). */
double hpo_f16_to_f64_ts(uint16_t value) {
  double sign = (value & 0x8000u) ? -1.0 : 1.0;
  int exponent = (value >> 10) & 0x1f;
  int fraction = value & 0x03ff;
  if (exponent == 0) return sign * ldexp(1.0, -14) * (fraction / 1024.0);
  if (exponent == 31) return fraction == 0 ? sign * INFINITY : NAN;
  return sign * ldexp(1.0, exponent - 15) * (1.0 + fraction / 1024.0);
}

/* quant.ts:671-681 roundTiesToEven */
static double ts_round_ties_to_even(double value) {
  double fl = floor(value);
  double fraction = value - fl;
  if (fraction < 0.5) return fl;
  if (fraction > 0.5) return fl + 1.0;
  return fmod(fl, 2.0) == 0.0 ? fl : fl + 1.0;
}

/* quant.ts:632-669 float32ToFloat16: saturates at 65504 and flushes
 * |v| < 2^-24 to signed zero; otherwise rounds to nearest, ties to even. */
uint16_t hpo_f64_to_f16_ts(double value) {
  if (isnan(value)) return 0x7e00u;
  if (value == INFINITY) return 0x7c00u;
  if (value == -INFINITY) return 0xfc00u;
  uint16_t sign = (value < 0 || (value == 0 && signbit(value))) ? 0x8000u : 0;
  double a = fabs(value);
  if (a == 0) return sign;
  if (a >= 65504.0) return (uint16_t)(sign | 0x7bffu);
  if (a < ldexp(1.0, -24)) return sign;
  /* Math.floor(Math.log2(abs)) is exact for the f32 inputs this is used on;
   * ilogb gives the same integer without a transcendental. */
  int exponent = ilogb(a);
  double mantissa = a / ldexp(1.0, exponent) - 1.0;
  if (exponent < -14) {
    double sub = ts_round_ties_to_even(a / ldexp(1.0, -24));
    return (uint16_t)(sign | (uint16_t)sub);
  }
  double half_mantissa = ts_round_ties_to_even(mantissa * 1024.0);
  if (half_mantissa == 1024.0) {
    exponent += 1;
    half_mantissa = 0.0;
  }
  return (uint16_t)(sign | ((exponent + 15) << 10) | (uint16_t)half_mantissa);
}

/* ---------------------------------------------------------------------- */
/* lib.rs:1551-1561 quantized_row_bytes (only the two restated types). */
size_t hpo_row_bytes(int32_t type_id, size_t elements) {
  if (elements % QK_K != 0) return 0;
  if (type_id == HPO_Q4_K) return elements / QK_K * 144;
  if (type_id == HPO_Q6_K) return elements / QK_K * 210;
  return 0;
}

/* lib.rs:2249-2259 get_scale_min_k4 */
void hpo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
  if (j < 4) {
    *sc = q[j] & 63;
    *mn = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
    *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* lib.rs:1630-1664 dequantize_q4_k: y = (d*sc)*q - (dmin*m), f32, no FMA. */
int hpo_dequantize_q4_k(const uint8_t *bytes, size_t elements, float *out) {
  if (elements % QK_K != 0) return 0;
  for (size_t b = 0; b < elements / QK_K; b++) {
    const uint8_t *blk = bytes + 144 * b;
    float d = hpo_f16_to_f32(rd16(blk));
    float dmin = hpo_f16_to_f32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *qs = blk + 16;
    float *o = out + QK_K * b;
    for (int g = 0; g < 4; g++) {
      uint8_t sc1, m1, sc2, m2;
      hpo_get_scale_min_k4(2 * g, scales, &sc1, &m1);
      hpo_get_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
      float d1 = d * (float)sc1, d2 = d * (float)sc2;
      float mm1 = dmin * (float)m1, mm2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) o[64 * g + l] = d1 * (float)(qs[32 * g + l] & 0x0f) - mm1;
      for (int l = 0; l < 32; l++) o[64 * g + 32 + l] = d2 * (float)(qs[32 * g + l] >> 4) - mm2;
    }
  }
  return 1;
}

/* lib.rs:1709-1744 dequantize_q6_k: y = (d*sc)*(q-32), exact in f32. */
int hpo_dequantize_q6_k(const uint8_t *bytes, size_t elements, float *out) {
  if (elements % QK_K != 0) return 0;
  for (size_t b = 0; b < elements / QK_K; b++) {
    const uint8_t *blk = bytes + 210 * b;
    const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
    float d = hpo_f16_to_f32(rd16(blk + 208));
    float *o = out + QK_K * b;
    for (int h = 0; h < 2; h++) {
      for (int lane = 0; lane < 32; lane++) {
        int is = lane / 16;
        uint8_t qhb = qh[32 * h + lane];
        int q1 = (int)((ql[64 * h + lane] & 0x0f) | (((qhb >> 0) & 3) << 4)) - 32;
        int q2 = (int)((ql[64 * h + lane + 32] & 0x0f) | (((qhb >> 2) & 3) << 4)) - 32;
        int q3 = (int)((ql[64 * h + lane] >> 4) | (((qhb >> 4) & 3) << 4)) - 32;
        int q4 = (int)((ql[64 * h + lane + 32] >> 4) | (((qhb >> 6) & 3) << 4)) - 32;
        o[128 * h + lane] = d * (float)(int8_t)scales[8 * h + is] * (float)q1;
        o[128 * h + lane + 32] = d * (float)(int8_t)scales[8 * h + is + 2] * (float)q2;
        o[128 * h + lane + 64] = d * (float)(int8_t)scales[8 * h + is + 4] * (float)q3;
        o[128 * h + lane + 96] = d * (float)(int8_t)scales[8 * h + is + 6] * (float)q4;
      }
    }
  }
  return 1;
}

/* ---------------------------------------------------------------------- */
/* Rust `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float r) {
  if (r != r) return 0;
  if (r >= 127.0f) return 127;
  if (r <= -128.0f) return -128;
  return (int8_t)r;
}

/* lib.rs:1774-1811 quantize_q8_k.  First index of the largest |x| gives
 * `max`; is = -127/max (correctly rounded f32 divide); q = min(127,
 * round(is*x)) with ties away from zero; d = 1/is; bsums32 = sums of 32. */
void hpo_quantize_q8_k(const float *x, size_t n, int8_t *qs, float *d, int16_t *bsums32) {
  size_t nb = n / QK_K;
  for (size_t b = 0; b < nb; b++) {
    const float *xb = x + QK_K * b;
    int8_t *qb = qs + QK_K * b;
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < QK_K; i++) {
      float v = xb[i];
      float a = fabsf(v);
      if (a > amax) {
        amax = a;
        max = v;
      }
    }
    if (amax == 0.0f) {
      memset(qb, 0, QK_K);
      for (int g = 0; g < 8; g++) bsums32[8 * b + g] = 0;
      d[b] = 0.0f;
      continue;
    }
    float inverse_scale = -127.0f / max;
    for (int i = 0; i < QK_K; i++) {
      float p = inverse_scale * xb[i];
      qb[i] = sat_i8(fminf(roundf(p), 127.0f));
    }
    for (int g = 0; g < 8; g++) {
      int16_t sum = 0;
      for (int i = 0; i < 32; i++) sum = (int16_t)(sum + qb[32 * g + i]);
      bsums32[8 * b + g] = sum;
    }
    d[b] = 1.0f / inverse_scale;
  }
}

/* ---------------------------------------------------------------------- */
/* Integer part of one Q4_K block, lib.rs:2121-2160: nibbles unpacked to
 * aux8 (2136-2146), sumi = sum_j bsums32[j]*min[j] (2148-2152),
 * aux32[l] += sc[j] * sum_{c<4} q8[32j+8c+l]*aux8[32j+8c+l] (2154-2160 with
 * accumulate_scaled_i8_i8_32_lanes 2443-2501). */
void hpo_block_ints_q4_k(const uint8_t *blk, const int8_t *q8, const int16_t *bs,
                         int32_t aux32[8], int32_t *sumi) {
  uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; j++) hpo_get_scale_min_k4(j, blk + 4, &sc[j], &mn[j]);
  int8_t aux8[QK_K];
  const uint8_t *qs = blk + 16;
  for (int g = 0; g < 4; g++) {
    for (int l = 0; l < 32; l++) {
      aux8[64 * g + l] = (int8_t)(qs[32 * g + l] & 0x0f);
      aux8[64 * g + 32 + l] = (int8_t)(qs[32 * g + l] >> 4);
    }
  }
  int32_t si = 0;
  for (int j = 0; j < 8; j++) si += (int32_t)bs[j] * (int32_t)mn[j];
  *sumi = si;
  for (int l = 0; l < 8; l++) aux32[l] = 0;
  for (int j = 0; j < 8; j++) {
    int32_t s = sc[j];
    for (int c = 0; c < 4; c++)
      for (int l = 0; l < 8; l++)
        aux32[l] += s * (int32_t)q8[32 * j + 8 * c + l] * (int32_t)aux8[32 * j + 8 * c + l];
  }
}

/* Integer part of one Q6_K block, lib.rs:1928-1959: 6-bit unpack minus 32
 * (1938-1949), then aux32[l] += sc[g] * sum_{c<2} q8[16g+8c+l]*aux8[16g+8c+l]
 * (1951-1959 with accumulate_scaled_i8_i8_16_lanes 2265-2313). */
void hpo_block_ints_q6_k(const uint8_t *blk, const int8_t *q8, int32_t aux32[8]) {
  const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
  int8_t aux8[QK_K];
  for (int h = 0; h < 2; h++) {
    for (int lane = 0; lane < 32; lane++) {
      uint8_t qhb = qh[32 * h + lane];
      aux8[128 * h + lane] = (int8_t)((int16_t)((ql[64 * h + lane] & 0x0f) | (((qhb >> 0) & 3) << 4)) - 32);
      aux8[128 * h + lane + 32] = (int8_t)((int16_t)((ql[64 * h + lane + 32] & 0x0f) | (((qhb >> 2) & 3) << 4)) - 32);
      aux8[128 * h + lane + 64] = (int8_t)((int16_t)((ql[64 * h + lane] >> 4) | (((qhb >> 4) & 3) << 4)) - 32);
      aux8[128 * h + lane + 96] = (int8_t)((int16_t)((ql[64 * h + lane + 32] >> 4) | (((qhb >> 6) & 3) << 4)) - 32);
    }
  }
  for (int l = 0; l < 8; l++) aux32[l] = 0;
  for (int g = 0; g < 16; g++) {
    int32_t s = (int8_t)scales[g];
    for (int c = 0; c < 2; c++)
      for (int l = 0; l < 8; l++)
        aux32[l] += s * (int32_t)q8[16 * g + 8 * c + l] * (int32_t)aux8[16 * g + 8 * c + l];
  }
}

/* lib.rs:2116-2172 vec_dot_q4_k_q8_k_prepared.  The prepared f32 scales
 * (lib.rs:156-222) are float16_to_float32 of the block's d/dmin, so they are
 * read straight from the block here.  Float tail in Rust order, no FMA:
 *   d = dW*dX; sums[l] += d*f32(aux32[l]); dm = dminW*dX; sumf -= dm*f32(sumi)
 *   return sumf + sums.iter().sum()   (f32 Sum folds from -0.0). */
float hpo_vec_dot_q4_k_q8_k(const uint8_t *row, size_t nblocks, const int8_t *qs,
                            const float *d, const int16_t *bsums32) {
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float sumf = 0.0f;
  for (size_t b = 0; b < nblocks; b++) {
    const uint8_t *blk = row + 144 * b;
    int32_t aux32[8], sumi;
    hpo_block_ints_q4_k(blk, qs + QK_K * b, bsums32 + 8 * b, aux32, &sumi);
    float dd = hpo_f16_to_f32(rd16(blk)) * d[b];
    for (int l = 0; l < 8; l++) sums[l] += dd * (float)aux32[l];
    float dm = hpo_f16_to_f32(rd16(blk + 2)) * d[b];
    sumf -= dm * (float)sumi;
  }
  float t = -0.0f;
  for (int l = 0; l < 8; l++) t += sums[l];
  return sumf + t;
}

/* lib.rs:1923-1968 vec_dot_q6_k_q8_k_prepared. */
float hpo_vec_dot_q6_k_q8_k(const uint8_t *row, size_t nblocks, const int8_t *qs, const float *d) {
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (size_t b = 0; b < nblocks; b++) {
    const uint8_t *blk = row + 210 * b;
    int32_t aux32[8];
    hpo_block_ints_q6_k(blk, qs + QK_K * b, aux32);
    float dd = hpo_f16_to_f32(rd16(blk + 208)) * d[b];
    for (int l = 0; l < 8; l++) sums[l] += dd * (float)aux32[l];
  }
  float t = -0.0f;
  for (int l = 0; l < 8; l++) t += sums[l];
  return t;
}

/* ---------------------------------------------------------------------- */
typedef struct {
  int8_t *qs;
  float *d;
  int16_t *bsums;
} q8k_buf;

static int q8k_alloc(q8k_buf *q, size_t k) {
  q->qs = (int8_t *)malloc(k);
  q->d = (float *)malloc(sizeof(float) * (k / QK_K + 1));
  q->bsums = (int16_t *)malloc(sizeof(int16_t) * (k / 32 + 1));
  return q->qs && q->d && q->bsums;
}

static void q8k_free(q8k_buf *q) {
  free(q->qs);
  free(q->d);
  free(q->bsums);
}

static void dot_rows(int32_t type_id, const uint8_t *weight, size_t row_bytes, size_t nb,
                     const q8k_buf *q, size_t row_begin, size_t row_end, float *out) {
  for (size_t row = row_begin; row < row_end; row++) {
    const uint8_t *r = weight + row * row_bytes;
    out[row] = type_id == HPO_Q4_K ? hpo_vec_dot_q4_k_q8_k(r, nb, q->qs, q->d, q->bsums)
                                   : hpo_vec_dot_q6_k_q8_k(r, nb, q->qs, q->d);
  }
}

/* lib.rs:224-298 hp_matmul_quantized_prepared_f32 (checks in the same order). */
int32_t hpo_matmul_quantized(int32_t type_id, const uint8_t *weight, size_t weight_len,
                             const float *input, size_t input_len, size_t input_size,
                             size_t row_count, size_t column_count, float *output,
                             size_t output_len) {
  if (input_len != sat_mul(input_size, column_count) || output_len != sat_mul(row_count, column_count))
    return HPO_ERR_SHAPE;
  size_t row_bytes = hpo_row_bytes(type_id, input_size);
  if (row_bytes == 0) return HPO_ERR_TYPE;
  if (weight_len != sat_mul(row_bytes, row_count)) return HPO_ERR_SHAPE;
  q8k_buf q;
  if (!q8k_alloc(&q, input_size)) {
    q8k_free(&q);
    return HPO_ERR_SHAPE;
  }
  size_t nb = input_size / QK_K;
  for (size_t col = 0; col < column_count; col++) {
    hpo_quantize_q8_k(input + col * input_size, input_size, q.qs, q.d, q.bsums);
    dot_rows(type_id, weight, row_bytes, nb, &q, 0, row_count, output + col * row_count);
  }
  q8k_free(&q);
  return HPO_OK;
}

/* lib.rs:300-426 hp_matmul_quantized_prepared_multi_f32: one Q8_K
 * quantisation per column shared by every weight. */
int32_t hpo_matmul_quantized_multi(size_t count, const float *input, size_t input_len,
                                   size_t input_size, size_t column_count,
                                   const int32_t *type_ids, const uint8_t *const *weights,
                                   const size_t *weight_lens, const size_t *row_counts,
                                   float *const *outputs, const size_t *output_lens) {
  if (count == 0 || count > 4 || input_len != sat_mul(input_size, column_count)) return HPO_ERR_SHAPE;
  for (size_t i = 0; i < count; i++) {
    size_t row_bytes = hpo_row_bytes(type_ids[i], input_size);
    if (row_bytes == 0) return HPO_ERR_TYPE;
    if (weight_lens[i] != sat_mul(row_bytes, row_counts[i]) ||
        output_lens[i] != sat_mul(row_counts[i], column_count))
      return HPO_ERR_SHAPE;
  }
  q8k_buf q;
  if (!q8k_alloc(&q, input_size)) {
    q8k_free(&q);
    return HPO_ERR_SHAPE;
  }
  size_t nb = input_size / QK_K;
  for (size_t col = 0; col < column_count; col++) {
    hpo_quantize_q8_k(input + col * input_size, input_size, q.qs, q.d, q.bsums);
    for (size_t i = 0; i < count; i++) {
      size_t row_bytes = hpo_row_bytes(type_ids[i], input_size);
      dot_rows(type_ids[i], weights[i], row_bytes, nb, &q, 0, row_counts[i],
               outputs[i] + col * row_counts[i]);
    }
  }
  q8k_free(&q);
  return HPO_OK;
}

/* ---------------------------------------------------------------------- */
/* Threaded variants: thread-pool.ts:410-424 splitRows gives each worker a
 * contiguous row shard (the first N mod T shards carry one extra row); each
 * worker quantises every column itself and fills its rows of [M][N]
 * (copyShardOutput, thread-pool.ts:426-443). */
typedef struct {
  size_t count;
  const int32_t *type_ids;
  const uint8_t *const *weights;
  const size_t *row_counts;
  float *const *outputs;
  const float *input;
  size_t input_size, column_count;
  size_t shard[4][2]; /* [weight][begin,end) */
} shard_job;

static void *shard_worker(void *arg) {
  shard_job *job = (shard_job *)arg;
  q8k_buf q;
  if (!q8k_alloc(&q, job->input_size)) {
    q8k_free(&q);
    return NULL;
  }
  size_t nb = job->input_size / QK_K;
  for (size_t col = 0; col < job->column_count; col++) {
    hpo_quantize_q8_k(job->input + col * job->input_size, job->input_size, q.qs, q.d, q.bsums);
    for (size_t i = 0; i < job->count; i++) {
      size_t row_bytes = hpo_row_bytes(job->type_ids[i], job->input_size);
      dot_rows(job->type_ids[i], job->weights[i], row_bytes, nb, &q, job->shard[i][0],
               job->shard[i][1], job->outputs[i] + col * job->row_counts[i]);
    }
  }
  q8k_free(&q);
  return NULL;
}

static void split_rows(size_t rows, size_t shards, size_t index, size_t *begin, size_t *end) {
  size_t base = rows / shards, extra = rows % shards;
  size_t start = index * base + (index < extra ? index : extra);
  *begin = start;
  *end = start + base + (index < extra ? 1 : 0);
}

int32_t hpo_matmul_quantized_multi_threaded(size_t count, const float *input, size_t input_len,
                                            size_t input_size, size_t column_count,
                                            const int32_t *type_ids, const uint8_t *const *weights,
                                            const size_t *weight_lens, const size_t *row_counts,
                                            float *const *outputs, const size_t *output_lens,
                                            int threads) {
  if (count == 0 || count > 4 || input_len != sat_mul(input_size, column_count)) return HPO_ERR_SHAPE;
  for (size_t i = 0; i < count; i++) {
    size_t row_bytes = hpo_row_bytes(type_ids[i], input_size);
    if (row_bytes == 0) return HPO_ERR_TYPE;
    if (weight_lens[i] != sat_mul(row_bytes, row_counts[i]) ||
        output_lens[i] != sat_mul(row_counts[i], column_count))
      return HPO_ERR_SHAPE;
  }
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  shard_job *jobs = (shard_job *)calloc((size_t)threads, sizeof(shard_job));
  pthread_t *tids = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
  if (!jobs || !tids) {
    free(jobs);
    free(tids);
    return HPO_ERR_SHAPE;
  }
  for (int t = 0; t < threads; t++) {
    shard_job *job = &jobs[t];
    job->count = count;
    job->type_ids = type_ids;
    job->weights = weights;
    job->row_counts = row_counts;
    job->outputs = outputs;
    job->input = input;
    job->input_size = input_size;
    job->column_count = column_count;
    for (size_t i = 0; i < count; i++)
      split_rows(row_counts[i], (size_t)threads, (size_t)t, &job->shard[i][0], &job->shard[i][1]);
  }
  for (int t = 1; t < threads; t++) pthread_create(&tids[t], NULL, shard_worker, &jobs[t]);
  shard_worker(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(tids[t], NULL);
  free(jobs);
  free(tids);
  return HPO_OK;
}

int32_t hpo_matmul_quantized_threaded(int32_t type_id, const uint8_t *weight, size_t weight_len,
                                      const float *input, size_t input_len, size_t input_size,
                                      size_t row_count, size_t column_count, float *output,
                                      size_t output_len, int threads) {
  if (input_len != sat_mul(input_size, column_count) || output_len != sat_mul(row_count, column_count))
    return HPO_ERR_SHAPE;
  if (hpo_row_bytes(type_id, input_size) == 0) return HPO_ERR_TYPE;
  return hpo_matmul_quantized_multi_threaded(1, input, input_len, input_size, column_count, &type_id,
                                             &weight, &weight_len, &row_count, &output, &output_len,
                                             threads);
}

/* ---------------------------------------------------------------------- */
/* Math.tanh as V8 evaluates it: fdlibm's s_tanh.c over s_expm1.c (Sun
 * Microsystems 1993; the published algorithm V8 ships as ieee754::tanh).
 * Pinned against Math.tanh outputs in tests/golden/v8_tanh.json. */
static uint32_t hiw(double x) { uint64_t b; memcpy(&b, &x, 8); return (uint32_t)(b >> 32); }
static uint32_t low(double x) { uint64_t b; memcpy(&b, &x, 8); return (uint32_t)b; }
static double words(uint32_t hi, uint32_t lo) { uint64_t b = ((uint64_t)hi << 32) | lo; double d; memcpy(&d, &b, 8); return d; }

/* Math.exp as V8 evaluates it: fdlibm's e_exp.c in FreeBSD msun's form (the
 * published algorithm V8 ships as ieee754::exp), including V8's exact answer
 * for exp(1).  Called by the sampling softmax, generation.ts:157-165.
 * Pinned against Math.exp outputs in tests/golden/v8_exp.json. */
double hpo_exp(double x) {
  const double o_threshold = 7.09782712893383973096e+02, u_threshold = -7.45133219101941108420e+02,
               ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10,
               invln2 = 1.44269504088896338700e+00, P1 = 1.66666666666666019037e-01,
               P2 = -2.77777777770155933842e-03, P3 = 6.61375632143793436117e-05,
               P4 = -1.65339022054652515390e-06, P5 = 4.13813679705723846039e-08,
               E = 2.718281828459045, huge = 1.0e+300, twom1000 = 9.33263618503218878990e-302,
               two1023 = 8.988465674311579539e307;
  uint32_t hx = hiw(x);
  int xsb = (int)(hx >> 31);
  double hi = 0, lo = 0, t, c, y, twopk;
  int k = 0;
  hx &= 0x7fffffffu;
  if (hx >= 0x40862E42u) {
    if (hx >= 0x7ff00000u) return (((hx & 0xfffffu) | low(x)) != 0) ? x + x : (xsb ? 0.0 : x);
    if (x > o_threshold) return huge * huge;
    if (x < u_threshold) return twom1000 * twom1000;
  }
  if (hx > 0x3FD62E42u) {
    if (hx < 0x3FF0A2B2u) {
      if (x == 1.0) return E;
      hi = xsb ? x + ln2hi : x - ln2hi;
      lo = xsb ? -ln2lo : ln2lo;
      k = 1 - 2 * xsb;
    } else {
      k = (int)(invln2 * x + (xsb ? -0.5 : 0.5));
      t = k;
      hi = x - t * ln2hi;
      lo = t * ln2lo;
    }
    x = hi - lo;
  } else if (hx < 0x3E300000u) {
    if (huge + x > 1.0) return 1.0 + x;
  }
  t = x * x;
  twopk = words(0x3FF00000u + ((uint32_t)(k >= -1021 ? k : k + 1000) << 20), 0);
  c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) return k == 1024 ? y * 2.0 * two1023 : y * twopk;
  return y * twopk * twom1000;
}

double hpo_expm1(double x) {
  const double o_threshold = 7.09782712893383973096e+02, ln2_hi = 6.93147180369123816490e-01,
               ln2_lo = 1.90821492927058770002e-10, invln2 = 1.44269504088896338700e+00,
               Q1 = -3.33333333333331316428e-02, Q2 = 1.58730158725481460165e-03,
               Q3 = -7.93650757867487942473e-05, Q4 = 4.00821782732936239552e-06,
               Q5 = -2.01099218183624371326e-07, huge = 1.0e+300, tiny = 1.0e-300;
  double y, hi, lo, c = 0.0, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = hiw(x);
  uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4043687Au) {
    if (hx >= 0x40862E42u) {
      if (hx >= 0x7ff00000u) {
        if (((hx & 0xfffffu) | low(x)) != 0) return x + x;
        return xsb == 0 ? x : -1.0;
      }
      if (x > o_threshold) return huge * huge;
    }
    if (xsb != 0 && x + tiny < 0.0) return tiny - 1.0;
  }
  if (hx > 0x3fd62e42u) {
    if (hx < 0x3FF0A2B2u) {
      if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
      else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
    } else {
      k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5 : -0.5));
      t = k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x3c900000u) {
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5 * x;
  hxs = x * hfx;
  r1 = 1.0 + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0 - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0 - x * t));
  if (k == 0) return x - (x * e - hxs);
  double twopk = words(0x3ff00000u + ((uint32_t)k << 20), 0);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5 * (x - e) - 0.5;
  if (k == 1) {
    if (x < -0.25) return -2.0 * (e - (x + 0.5));
    return 1.0 + 2.0 * (x - e);
  }
  if (k <= -2 || k > 56) {
    y = 1.0 - (e - x);
    y = (k == 1024) ? y * 2.0 * 8.98846567431158e+307 : y * twopk;
    return y - 1.0;
  }
  if (k < 20) {
    t = words(0x3ff00000u - (0x200000u >> k), 0);
    y = t - (e - x);
    y = y * twopk;
  } else {
    t = words((uint32_t)(0x3ff - k) << 20, 0);
    y = x - (e + t);
    y += 1.0;
    y = y * twopk;
  }
  return y;
}

double hpo_tanh(double x) {
  const double tiny = 1.0e-300, huge = 1.0e300;
  double t, z;
  uint32_t jx = hiw(x), ix = jx & 0x7fffffffu;
  int neg = (jx & 0x80000000u) != 0;
  if (ix >= 0x7ff00000u) return neg ? 1.0 / x - 1.0 : 1.0 / x + 1.0;
  if (ix < 0x40360000u) {
    if (ix < 0x3e300000u && huge + x > 1.0) return x;
    if (ix >= 0x3ff00000u) {
      t = hpo_expm1(2.0 * fabs(x));
      z = 1.0 - 2.0 / (t + 2.0);
    } else {
      t = hpo_expm1(-2.0 * fabs(x));
      z = -t / (t + 2.0);
    }
  } else {
    z = 1.0 - tiny;
  }
  return neg ? -z : z;
}

/* ---------------------------------------------------------------------- */
/* layers.ts:1062-1076 gelu.  JS numbers are f64: every Math.fround is a
 * cast to float, every other operation is an f64 operation; Math.tanh is
 * hpo_tanh (V8's algorithm). */
float hpo_gelu(float vf) {
  double value = vf;
  if (value <= -10.0) return 0.0f;
  if (value >= 10.0) return vf;
  double x = hpo_f16_to_f64_ts(hpo_f64_to_f16_ts(value));
  double c = sqrt(2.0 / M_PI);
  double t1 = (float)(c * x);
  double x2 = (float)(x * x);
  double t2 = (float)(0.044715 * x2);
  double t3 = (float)(1.0 + t2);
  double inner = (float)(t1 * t3);
  double half = (float)(0.5 * x);
  double t4 = (float)(1.0 + hpo_tanh(inner));
  double activated = (float)(half * t4);
  return (float)hpo_f16_to_f64_ts(hpo_f64_to_f16_ts(activated));
}

/* layers.ts:450-456: output[i] = Math.fround(gelu(gate[i]) * up[i]). */
void hpo_geglu(const float *gate, const float *up, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = (float)((double)hpo_gelu(gate[i]) * (double)up[i]);
}

/* layers.ts:407-412 softcap: Math.fround(Math.tanh(v / c) * c). */
float hpo_softcap(float v, double cap) { return (float)(hpo_tanh((double)v / cap) * cap); }

/* runtime.ts:514-527 topK: a candidate enters while fewer than k are kept
 * or when it ranks above the current k-th value; the stable descending sort
 * keeps equal values in id order, so ties go to the lower id (-0 and +0
 * tie).  NaN ranks below every number (JS leaves NaN's place to the sort
 * implementation; logits carry no NaN), so NaNs fill the tail in id order. */
static int ranks_above(float a, float b) {
  if (b != b) return a == a;
  if (a != a) return 0;
  return a > b;
}

size_t hpo_topk(const float *values, size_t n, size_t k, uint32_t *ids, float *out_values) {
  size_t len = 0;
  if (k == 0) return 0;
  for (size_t id = 0; id < n; id++) {
    float v = values[id];
    if (len < k || ranks_above(v, out_values[len - 1])) {
      size_t pos = 0;
      while (pos < len && !ranks_above(v, out_values[pos])) pos++;
      size_t last = len < k ? len : k - 1;
      for (size_t i = last; i > pos; i--) {
        ids[i] = ids[i - 1];
        out_values[i] = out_values[i - 1];
      }
      if (pos < k) {
        ids[pos] = (uint32_t)id;
        out_values[pos] = v;
      }
      if (len < k) len++;
    }
  }
  return len;
}

/* ---------------------------------------------------------------------- */
/* Decoder-layer steps (packages/engine/src/runner/wasm/layers.ts).         */

/* rmsNormVector (layers.ts:871-885): sumSquares += value * value in f64, in
 * index order; scale = 1 / sqrt(sumSquares / n + eps); output[i] =
 * f32((x[i] * scale) * w[i]) in f64.  w == NULL: rmsNormRowsNoWeight
 * (layers.ts:834-849), output[i] = f32(x[i] * scale). */
void hpo_rms_norm_vector(const float *x, size_t n, const float *w, double eps, float *out) {
  double sum = 0.0;
  for (size_t i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
  const double scale = 1.0 / sqrt(sum / (double)n + eps);
  for (size_t i = 0; i < n; i++)
    out[i] = w ? (float)(((double)x[i] * scale) * (double)w[i]) : (float)((double)x[i] * scale);
}

/* residualAdd (layers.ts:851-860): f32(a + b). */
void hpo_residual_add(const float *a, const float *b, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = (float)((double)a[i] + (double)b[i]);
}

/* castF16Rows (layers.ts:982-988): float16ToFloat32(float32ToFloat16(v)). */
void hpo_cast_f16_rows(const float *in, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = (float)hpo_f16_to_f64_ts(hpo_f64_to_f16_ts((double)in[i]));
}

/* ropeNeox (layers.ts:990-1033) over [token_count][head_count][head_size].
 * thetaScale = pow(freqBase, -2 / nDims); per head theta starts at the
 * token's position and becomes f32(theta * thetaScale) after each pair;
 * the angle is theta / freq_factors[i] (1 without factors); outputs
 * f32(f32(x0 cos) - f32(x1 sin)) and f32(f32(x0 sin) + f32(x1 cos)).
 * Returns HPO_ERR_SHAPE for an odd or too large nDims. */
int32_t hpo_rope_neox(const float *input, size_t head_size, size_t head_count, size_t token_count,
                      const int32_t *positions, size_t n_dims, double freq_base, const float *freq_factors,
                      float *output) {
  if (n_dims > head_size || n_dims % 2 != 0) return HPO_ERR_SHAPE;
  const size_t total = head_size * head_count * token_count;
  memcpy(output, input, total * sizeof(float));
  const double theta_scale = pow(freq_base, -2.0 / (double)n_dims);
  const size_t half = n_dims / 2;
  for (size_t t = 0; t < token_count; t++) {
    for (size_t h = 0; h < head_count; h++) {
      const size_t row = (t * head_count + h) * head_size;
      double theta = (double)positions[t];
      for (size_t i = 0; i < half; i++) {
        const double x0 = input[row + i], x1 = input[row + half + i];
        const double ang = freq_factors ? theta / (double)freq_factors[i] : theta;
        const double c = cos(ang), s = sin(ang);
        output[row + i] = (float)((double)(float)(x0 * c) - (double)(float)(x1 * s));
        output[row + half + i] = (float)((double)(float)(x0 * s) + (double)(float)(x1 * c));
        theta = (double)(float)(theta * theta_scale);
      }
    }
  }
  return HPO_OK;
}

/* hp_gqa_attention_f32 (packages/engine/wasm-kernels/src/lib.rs:538-654):
 * the same checks and status codes, f32 arithmetic in the same order
 * (dot = dot + q * k per index; score = (dot * scale) + mask; p =
 * f32(exp(f64(score - max))); weighted = weighted + (p / sum) * v).  exp is
 * f64 exp as Rust's std resolves it on wasm32 (compiler-builtins' libm, a
 * port of FreeBSD msun e_exp.c: hpo_exp).  value_layout 1 =
 * "dim-head-token" ((index * kv_heads + kv_head) * capacity + token), else
 * token-major like the key. */
/* One (token, query head) row of hpo_gqa_attention_f32.  Every score and
 * every weighted sum is its own chain in the reference's order; the loops
 * run four independent chains side by side (four keys, then four output
 * dims), which changes no chain's order. */
typedef struct {
  const float *query, *key, *value, *mask;
  size_t mask_len, head_size, query_head_count, key_value_head_count, token_count, key_value_token_count,
      key_value_start, key_value_capacity, group;
  float scale;
  int32_t value_layout, quantize_query_f16;
  float *output;
  size_t row_begin, row_end;  /* rows t * query_head_count + qh */
  int failed;
} GqaJob;

static void gqa_rows(GqaJob *J) {
  const size_t hs = J->head_size, nkv = J->key_value_head_count, cap = J->key_value_capacity;
  const size_t kvn = J->key_value_token_count;
  float *scores = malloc((kvn ? kvn : 1) * sizeof(float));
  float *qv = malloc((hs ? hs : 1) * sizeof(float));
  size_t *phys = malloc((kvn ? kvn : 1) * sizeof(size_t));
  if (!scores || !qv || !phys) {
    free(scores);
    free(qv);
    free(phys);
    J->failed = 1;
    return;
  }
  for (size_t kt = 0; kt < kvn; kt++) phys[kt] = (J->key_value_start + kt) % cap;
  for (size_t row = J->row_begin; row < J->row_end; row++) {
    const size_t t = row / J->query_head_count, qh = row % J->query_head_count;
    const size_t kvh = qh / J->group;
    const size_t qo = row * hs;
    for (size_t i = 0; i < hs; i++)
      qv[i] = J->quantize_query_f16 ? hpo_f16_to_f32(hpo_f32_to_f16_rust(J->query[qo + i])) : J->query[qo + i];
    float max_score = -INFINITY;
    size_t kt = 0;
    for (; kt + 4 <= kvn; kt += 4) {
      const float *k0 = J->key + (phys[kt] * nkv + kvh) * hs, *k1 = J->key + (phys[kt + 1] * nkv + kvh) * hs;
      const float *k2 = J->key + (phys[kt + 2] * nkv + kvh) * hs, *k3 = J->key + (phys[kt + 3] * nkv + kvh) * hs;
      float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
      for (size_t i = 0; i < hs; i++) {
        d0 = d0 + qv[i] * k0[i];
        d1 = d1 + qv[i] * k1[i];
        d2 = d2 + qv[i] * k2[i];
        d3 = d3 + qv[i] * k3[i];
      }
      const float dd[4] = {d0, d1, d2, d3};
      for (int u = 0; u < 4; u++) {
        const float mv = J->mask_len == 0 ? 0.0f : J->mask[t * kvn + kt + u];
        const float score = mv == -INFINITY ? -INFINITY : (dd[u] * J->scale) + mv;
        scores[kt + u] = score;
        if (score > max_score) max_score = score;
      }
    }
    for (; kt < kvn; kt++) {
      const float *kr = J->key + (phys[kt] * nkv + kvh) * hs;
      float dot = 0.0f;
      for (size_t i = 0; i < hs; i++) dot = dot + qv[i] * kr[i];
      const float mv = J->mask_len == 0 ? 0.0f : J->mask[t * kvn + kt];
      const float score = mv == -INFINITY ? -INFINITY : (dot * J->scale) + mv;
      scores[kt] = score;
      if (score > max_score) max_score = score;
    }
    float sum = 0.0f;
    for (kt = 0; kt < kvn; kt++) {
      const float sc = scores[kt];
      const float p = sc == -INFINITY ? 0.0f : (float)hpo_exp((double)(sc - max_score));
      scores[kt] = p;
      sum += p;
    }
    /* the reference forms (p / sum) inside the sum; the same f32 quotient */
    for (kt = 0; kt < kvn; kt++) scores[kt] = scores[kt] / sum;
    size_t i = 0;
    for (; i + 4 <= hs; i += 4) {
      float w0 = 0.0f, w1 = 0.0f, w2 = 0.0f, w3 = 0.0f;
      for (kt = 0; kt < kvn; kt++) {
        const size_t ph = phys[kt];
        const float pw = scores[kt];
        if (J->value_layout == 1) {
          w0 = w0 + pw * J->value[((i + 0) * nkv + kvh) * cap + ph];
          w1 = w1 + pw * J->value[((i + 1) * nkv + kvh) * cap + ph];
          w2 = w2 + pw * J->value[((i + 2) * nkv + kvh) * cap + ph];
          w3 = w3 + pw * J->value[((i + 3) * nkv + kvh) * cap + ph];
        } else {
          const float *vr = J->value + (ph * nkv + kvh) * hs + i;
          w0 = w0 + pw * vr[0];
          w1 = w1 + pw * vr[1];
          w2 = w2 + pw * vr[2];
          w3 = w3 + pw * vr[3];
        }
      }
      J->output[qo + i] = w0;
      J->output[qo + i + 1] = w1;
      J->output[qo + i + 2] = w2;
      J->output[qo + i + 3] = w3;
    }
    for (; i < hs; i++) {
      float weighted = 0.0f;
      for (kt = 0; kt < kvn; kt++) {
        const size_t vo = J->value_layout == 1 ? (i * nkv + kvh) * cap + phys[kt] : (phys[kt] * nkv + kvh) * hs + i;
        weighted = weighted + scores[kt] * J->value[vo];
      }
      J->output[qo + i] = weighted;
    }
  }
  free(scores);
  free(qv);
  free(phys);
}

static void *gqa_worker(void *arg) {
  gqa_rows((GqaJob *)arg);
  return NULL;
}

int32_t hpo_gqa_attention_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                              const float *value, size_t value_len, const float *mask, size_t mask_len,
                              size_t head_size, size_t query_head_count, size_t key_value_head_count,
                              size_t token_count, size_t key_value_token_count, size_t key_value_start,
                              size_t key_value_capacity, float scale, int32_t value_layout,
                              int32_t quantize_query_f16, float *output, size_t output_len) {
  if (query_len != sat_mul(sat_mul(token_count, query_head_count), head_size) ||
      key_len != sat_mul(sat_mul(key_value_capacity, key_value_head_count), head_size) ||
      value_len != sat_mul(sat_mul(key_value_capacity, key_value_head_count), head_size) ||
      output_len != sat_mul(sat_mul(token_count, query_head_count), head_size) ||
      (mask_len != 0 && mask_len != sat_mul(token_count, key_value_token_count)))
    return HPO_ERR_SHAPE;
  if (key_value_head_count == 0 || key_value_capacity == 0 || key_value_token_count > key_value_capacity ||
      query_head_count % key_value_head_count != 0)
    return HPO_ERR_HEADS;
  const size_t rows = token_count * query_head_count;
  /* rows are independent: spread them over up to 16 threads when the work
   * is large enough to pay for them */
  long hw = sysconf(_SC_NPROCESSORS_ONLN);
  size_t threads = hw > 0 ? (size_t)hw : 1;
  if (threads > 16) threads = 16;
  const double work = (double)rows * (double)key_value_token_count * (double)head_size;
  if (work < 4e6) threads = 1;
  if (threads > rows) threads = rows ? rows : 1;
  GqaJob base = {query, key, value, mask, mask_len, head_size, query_head_count, key_value_head_count, token_count,
                 key_value_token_count, key_value_start, key_value_capacity, query_head_count / key_value_head_count,
                 scale, value_layout, quantize_query_f16, output, 0, 0, 0};
  GqaJob *jobs = calloc(threads, sizeof(GqaJob));
  pthread_t *tids = calloc(threads, sizeof(pthread_t));
  if (!jobs || !tids) {
    free(jobs);
    free(tids);
    return HPO_ERR_SHAPE;
  }
  int started[16] = {0};
  for (size_t w = 0; w < threads; w++) {
    jobs[w] = base;
    jobs[w].row_begin = rows * w / threads;
    jobs[w].row_end = rows * (w + 1) / threads;
  }
  for (size_t w = 1; w < threads; w++) started[w] = pthread_create(&tids[w], NULL, gqa_worker, &jobs[w]) == 0;
  gqa_rows(&jobs[0]);
  int failed = jobs[0].failed;
  for (size_t w = 1; w < threads; w++) {
    if (started[w])
      pthread_join(tids[w], NULL);
    else
      gqa_rows(&jobs[w]);  /* no thread: this one runs here */
    failed |= jobs[w].failed;
  }
  free(jobs);
  free(tids);
  return failed ? HPO_ERR_SHAPE : HPO_OK;
}
