/*
 * hp_oracle.h -- CPU restatement of heliopause's quantized-projection path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (libhp_hip.so) never links or calls it.
 *
 * Every function restates one function of the reference (file:line cited
 * beside it) in plain C, keeping the reference's operation order wherever it
 * is observable in f32 results.  Build flags: -O2 -ffp-contract=off
 * -fno-fast-math (see oracle/Makefile); integer loops may be vectorised by
 * the compiler since integer sums are exact in any order.
 */
#ifndef HP_ORACLE_H
#define HP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes and type ids: packages/engine/wasm-kernels/src/lib.rs:7-17 */
enum { HPO_OK = 0, HPO_ERR_SHAPE = 1, HPO_ERR_HEADS = 2, HPO_ERR_TYPE = 3 };
enum { HPO_Q4_K = 1, HPO_Q5_K = 2, HPO_Q6_K = 3, HPO_IQ4_XS = 4, HPO_Q8_0 = 5, HPO_Q4_0 = 6 };

/* ---- scalar conversions ---------------------------------------------- */
float hpo_f16_to_f32(uint16_t h);            /* lib.rs:2507-2532 */
uint32_t hpo_f16_to_f32_bits(uint16_t h);    /* the same, as bits */
uint16_t hpo_f32_to_f16_rust(float v);       /* lib.rs:2534-2569 (round half up) */
double hpo_f16_to_f64_ts(uint16_t h);        /* quant.ts:618-630 */
uint16_t hpo_f64_to_f16_ts(double v);        /* quant.ts:632-669 (ties to even) */

/* ---- block formats ----------------------------------------------------- */
size_t hpo_row_bytes(int32_t type_id, size_t elements);            /* lib.rs:1551-1561 */
void hpo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn); /* lib.rs:2249-2259 */
int hpo_dequantize_q4_k(const uint8_t *bytes, size_t elements, float *out);  /* lib.rs:1630-1664 */
int hpo_dequantize_q6_k(const uint8_t *bytes, size_t elements, float *out);  /* lib.rs:1709-1744 */

/* ---- Q8_K activation quantisation: lib.rs:1774-1811 -------------------- */
/* qs: n int8, d: n/256 f32, bsums32: n/32 int16 */
void hpo_quantize_q8_k(const float *x, size_t n, int8_t *qs, float *d, int16_t *bsums32);

/* ---- vector dots (resident "prepared" variants) ------------------------ */
/* lib.rs:2116-2172 */
float hpo_vec_dot_q4_k_q8_k(const uint8_t *row, size_t nblocks, const int8_t *qs,
                            const float *d, const int16_t *bsums32);
/* lib.rs:1923-1968 */
float hpo_vec_dot_q6_k_q8_k(const uint8_t *row, size_t nblocks, const int8_t *qs, const float *d);
/* Integer part of one block (exposed so tests can pin the f32 tail):
 * aux32[8] as in lib.rs:2148-2160 / 1951-1959; *sumi (Q4_K only) lib.rs:2148-2152. */
void hpo_block_ints_q4_k(const uint8_t *blk, const int8_t *qs, const int16_t *bsums32,
                         int32_t aux32[8], int32_t *sumi);
void hpo_block_ints_q6_k(const uint8_t *blk, const int8_t *qs, int32_t aux32[8]);

/* ---- matmul entry points ------------------------------------------------ */
/* hp_matmul_quantized_prepared_f32, lib.rs:224-298.  input [M][K], output [M][N]. */
int32_t hpo_matmul_quantized(int32_t type_id, const uint8_t *weight, size_t weight_len,
                             const float *input, size_t input_len, size_t input_size,
                             size_t row_count, size_t column_count, float *output,
                             size_t output_len);
/* hp_matmul_quantized_prepared_multi_f32, lib.rs:300-426 (count 1..4). */
int32_t hpo_matmul_quantized_multi(size_t count, const float *input, size_t input_len,
                                   size_t input_size, size_t column_count,
                                   const int32_t *type_ids, const uint8_t *const *weights,
                                   const size_t *weight_lens, const size_t *row_counts,
                                   float *const *outputs, const size_t *output_lens);
/* Row-sharded, threaded variant of hpo_matmul_quantized: the WasmThreadPool
 * semantics (thread-pool.ts:197-232, splitRows 410-424); every shard
 * re-quantises the input as each worker's WASM call does (lib.rs:264-296). */
int32_t hpo_matmul_quantized_threaded(int32_t type_id, const uint8_t *weight, size_t weight_len,
                                      const float *input, size_t input_len, size_t input_size,
                                      size_t row_count, size_t column_count, float *output,
                                      size_t output_len, int threads);
int32_t hpo_matmul_quantized_multi_threaded(size_t count, const float *input, size_t input_len,
                                            size_t input_size, size_t column_count,
                                            const int32_t *type_ids, const uint8_t *const *weights,
                                            const size_t *weight_lens, const size_t *row_counts,
                                            float *const *outputs, const size_t *output_lens,
                                            int threads);

/* ---- epilogues ------------------------------------------------------------ */
/* Math.tanh / expm1 as V8 computes them (fdlibm s_tanh.c, s_expm1.c). */
double hpo_tanh(double x);
double hpo_expm1(double x);
double hpo_exp(double x);
/* gelu: packages/engine/src/runner/wasm/layers.ts:1062-1076 (returns an f32). */
float hpo_gelu(float v);
/* GeGLU: layers.ts:450-456: out[i] = fround(gelu(gate[i]) * up[i]). */
void hpo_geglu(const float *gate, const float *up, size_t n, float *out);
/* topK: packages/engine/src/runtime.ts:514-527 on one row; returns count. */
size_t hpo_topk(const float *values, size_t n, size_t k, uint32_t *ids, float *out_values);
/* softcap: layers.ts:407-412: fround(tanh(v / c) * c) in f64. */
float hpo_softcap(float v, double cap);

/* ---- decoder-layer steps ---------------------------------------------- */
/* rmsNormVector (layers.ts:871-885); w NULL: rmsNormRowsNoWeight (834-849). */
void hpo_rms_norm_vector(const float *x, size_t n, const float *w, double eps, float *out);
/* residualAdd (layers.ts:851-860). */
void hpo_residual_add(const float *a, const float *b, size_t n, float *out);
/* castF16Rows (layers.ts:982-988). */
void hpo_cast_f16_rows(const float *in, size_t n, float *out);
/* ropeNeox (layers.ts:990-1033). */
int32_t hpo_rope_neox(const float *input, size_t head_size, size_t head_count, size_t token_count,
                      const int32_t *positions, size_t n_dims, double freq_base, const float *freq_factors,
                      float *output);
/* hp_gqa_attention_f32 (lib.rs:538-654). */
int32_t hpo_gqa_attention_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                              const float *value, size_t value_len, const float *mask, size_t mask_len,
                              size_t head_size, size_t query_head_count, size_t key_value_head_count,
                              size_t token_count, size_t key_value_token_count, size_t key_value_start,
                              size_t key_value_capacity, float scale, int32_t value_layout,
                              int32_t quantize_query_f16, float *output, size_t output_len);

#ifdef __cplusplus
}
#endif
#endif
