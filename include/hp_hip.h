/*
 * hp_hip.h -- C ABI of the MI355X (gfx950) quantized-projection runner.
 *
 * Drop-in boundary for heliopause's resident-weight matmul path.  The
 * reference exposes the same operations as WASM exports
 * (packages/engine/wasm-kernels/src/lib.rs:23-536) wrapped by the TS runner
 * API in packages/engine/src/runner/wasm/wasm-kernels.ts.  This ABI keeps
 * the reference's type ids, status codes, argument order and layouts:
 *   input  [column_count][input_size] f32   (column m at m * input_size)
 *   output [column_count][row_count]  f32   (out[m * row_count + row])
 *   weight [row_count][row_bytes]     GGUF super-blocks as stored
 * Plain pointers and sizes only.  Host-pointer entry points copy through
 * the library's HIP stream and return when results are in host memory;
 * *_device entry points take device pointers and are asynchronous on the
 * given stream.  Calls are serialised by an internal lock; results written
 * by concurrent calls on one device must not overlap.
 *
 * Intermediate device memory of the *_device entry points (decode
 * activations, attention partials, top-k selection state, prefill images,
 * gate/up sums) belongs to the stream a call is queued on: calls on
 * different streams never share it, and calls queued on one stream run in
 * order.  It only grows, and replaced buffers are kept until
 * hp_hip_shutdown, so a HIP graph captured earlier never points at freed
 * memory.  Growth is refused while the stream captures (HP_ERR_ARG): a
 * captured call must follow an uncaptured call of the same shape on the
 * capturing stream.  Replaying a graph concurrently with other calls on its
 * capture stream races on that stream's scratch.
 *
 * The host-pointer matmul entry points (hp_hip_matmul, _multi, _geglu,
 * _topk, _topk_sample) stay on the bit-exact kernels under the automatic
 * kernel policy; the fast prefill kernel (1e-4 relative) runs automatically
 * only on *_device calls of 64 or more columns.
 */
#ifndef HP_HIP_H
#define HP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  0..3 are lib.rs:7-10 (OK, ERR_SHAPE, ERR_HEADS, ERR_TYPE);
 * the TS wrapper maps them like assertWasmOk (wasm-kernels.ts:1882-1896).
 * Codes >= 16 are this runtime's own. */
#define HP_OK 0
#define HP_ERR_SHAPE 1
#define HP_ERR_HEADS 2
#define HP_ERR_TYPE 3
#define HP_ERR_HIP 16     /* a HIP runtime call failed (see hp_hip_last_error) */
#define HP_ERR_HANDLE 17  /* unknown or released weight handle */
#define HP_ERR_ARG 18     /* null pointer or out-of-range argument */
#define HP_ERR_NODEV 19   /* no usable GPU */
#define HP_ERR_OOM 20     /* device allocation failed */

/* Type ids: lib.rs:12-17 (wasm-kernels.ts:1908-1923).  This runner
 * implements Q4_K and Q6_K; the others return HP_ERR_TYPE so the caller
 * falls back to the WASM runner, as wasm-kernels.ts:424-431 does. */
#define HP_TYPE_Q4_K 1
#define HP_TYPE_Q5_K 2
#define HP_TYPE_Q6_K 3
#define HP_TYPE_IQ4_XS 4
#define HP_TYPE_Q8_0 5
#define HP_TYPE_Q4_0 6

/* Kernel ids for hp_hip_profile_read. */
#define HP_KERNEL_Q8K 0
#define HP_KERNEL_MATVEC 1
#define HP_KERNEL_TOPK 2
#define HP_KERNEL_GEGLU 3
#define HP_KERNEL_ATTENTION 4 /* attention prologue, partials and merge */
#define HP_KERNEL_NORM 5      /* norm / residual launches of the decoder layer */
#define HP_KERNEL_SAMPLE 6
#define HP_KERNEL_COUNT 7

typedef struct hp_hip_stats {
  uint64_t handle_count;   /* live weight handles */
  uint64_t resident_bytes; /* device bytes held by weight handles */
  uint64_t scratch_bytes;  /* device bytes held by activation scratch */
  uint64_t matmul_calls;
  uint64_t kernel_launches;
  int32_t device;
  int32_t compute_units;
} hp_hip_stats_t;

/* Human-readable name of a status code (never NULL). */
const char *hp_hip_status_string(int32_t status);
/* Message describing the last failure on the calling thread ("" if none). */
const char *hp_hip_last_error(void);

/* Select the GPU and create the library stream (idempotent; other entry
 * points call it with device 0 on first use).  Analog of the module
 * instantiation behind prefillWasmExports (wasm-kernels.ts:1678-1741) and
 * of checkWasmSupport (1657-1675): HP_ERR_NODEV when no GPU is usable. */
int32_t hp_hip_init(int32_t device);
/* Release every handle and the scratch buffers (shutdownWasmExecutionProvider,
 * acceleration.ts:93-112). */
int32_t hp_hip_shutdown(void);
int32_t hp_hip_device_count(int32_t *count);

/* Upload GGUF super-blocks once into an HBM-resident handle.  Replaces
 * createWasmQuantizedWeightHandle (wasm-kernels.ts:520-574) and the scale
 * preparation hp_prepare_quantized_scales_f32 (lib.rs:156-222): the GPU keeps
 * no f32 side table.  weight_len must equal row_count * row_bytes. */
int32_t hp_hip_weight_upload(int32_t type_id, const uint8_t *weight, size_t weight_len, size_t input_size,
                             size_t row_count, uint64_t *out_handle);
/* Same from a device buffer already holding the GGUF bytes. */
int32_t hp_hip_weight_upload_device(int32_t type_id, const void *d_weight, size_t weight_len, size_t input_size,
                                    size_t row_count, uint64_t *out_handle);
/* Upload tensors of a parsed GGUF file (hp_gguf.h) straight from the file
 * into HBM-resident handles: readWasmWeightHandle's readTensorBytes +
 * createWasmQuantizedWeightHandle (acceleration.ts:164-201), for a batch of
 * tensors at once.  Shape as matMulKQ8K reads it (wasm/layers.ts:758-759):
 * input size = dims[0], rows = dims[1].  Bytes stream file -> pinned host
 * chunks (parallel pread) -> device staging -> repack; no pageable copy.
 * statuses[i] = HP_OK with handles[i] set, or HP_ERR_TYPE with handles[i] = 0
 * for a block type this runner does not implement (the caller falls back).
 * Any other failure (a tensor that is not a [rows][input] weight of whole
 * blocks, data past the end of the file, a read or HIP error) returns that
 * code and leaves no handle from this call. */
struct hp_gguf;
int32_t hp_hip_weight_upload_gguf(const struct hp_gguf *gguf, size_t count, const uint64_t *tensor_indices,
                                  uint64_t *handles, int32_t *statuses);
/* releaseWasmQuantizedWeightHandle (wasm-kernels.ts:576-584). */
int32_t hp_hip_weight_release(uint64_t handle);
int32_t hp_hip_weight_info(uint64_t handle, int32_t *type_id, size_t *input_size, size_t *row_count,
                           size_t *byte_length);

/* matMulQuantizedWasmResident (wasm-kernels.ts:593-646) ->
 * hp_matmul_quantized_prepared_f32 (lib.rs:224-298).  Q8_K-quantises each
 * input column, then out[m*N+n] = vec_dot(row n, q8_m), bit-exact with the
 * reference.  HP_ERR_SHAPE when the handle's shape differs from
 * (input_size, row_count) or the lengths do not match. */
int32_t hp_hip_matmul(uint64_t handle, const float *input, size_t input_len, size_t input_size, size_t row_count,
                      size_t column_count, float *output, size_t output_len);

/* matMulQuantizedWasmResidentMulti (wasm-kernels.ts:648-749) ->
 * hp_matmul_quantized_prepared_multi_f32 (lib.rs:300-426): 1..4 handles of
 * any supported type share one Q8_K quantisation per column and one launch.
 * outputs[i] receives [column_count][rows_i]. */
int32_t hp_hip_matmul_multi(size_t count, const uint64_t *handles, const float *input, size_t input_len,
                            size_t input_size, size_t column_count, float *const *outputs,
                            const size_t *output_lens);

/* Device-pointer form of hp_hip_matmul_multi for chained on-device work
 * (inputs and outputs stay in HBM).  stream: a hipStream_t, or NULL for the
 * library stream.  Asynchronous. */
int32_t hp_hip_matmul_multi_device(size_t count, const uint64_t *handles, const float *d_input, size_t input_len,
                                   size_t input_size, size_t column_count, float *const *d_outputs,
                                   const size_t *output_lens, void *stream);

/* Output head + sampling candidates: forwardOutput (layers.ts:381-416) ->
 * logits = matmul(handle, input) kept in HBM, optional softcap
 * fround(tanh(v / softcap) * softcap) when softcap > 0 (layers.ts:407-412),
 * then topK (runtime.ts:514-527) per column: k (<= 64) ids and values in
 * descending value order, ties to the lower id.  Only the candidates are
 * copied back: ids / values are [column_count][k] (out_len = column_count*k).
 * Replaces the WebGPU dispatchOutputTopK (segment-runner.ts:3208-3248). */
int32_t hp_hip_matmul_topk(uint64_t handle, const float *input, size_t input_len, size_t input_size,
                           size_t column_count, size_t k, double softcap, uint32_t *ids, float *values,
                           size_t out_len);
/* topK over host logits [rows][n] (n <= 524288, k <= 64); same semantics. */
int32_t hp_hip_topk(const float *logits, size_t rows, size_t n, size_t k, double softcap, uint32_t *ids,
                    float *values, size_t out_len);
/* Device-pointer topK; asynchronous on stream (NULL = library stream). */
int32_t hp_hip_topk_device(const float *d_logits, size_t rows, size_t n, size_t k, double softcap,
                           uint32_t *d_ids, float *d_values, void *stream);
/* hp_hip_topk_device without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture on a stream no earlier call has sized, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results.  Its
 * selection state lives in a static device array of 8.5 MiB per GPU, held
 * until the process ends, which fits one batch of 16 rows at every shape
 * hp_hip_topk_device takes (n <= 524288, k <= 64; larger row counts run in
 * batches of 16); a shape whose state would not fit fails with HP_ERR_SHAPE.
 * The library must be initialised first (hp_hip_init, or any earlier call):
 * HP_ERR_ARG otherwise.  Every call on one GPU shares that array, so calls
 * that overlap on one GPU (two streams at once) race; calls queued on one
 * stream are ordered.  Each call starts by clearing the array's counters
 * with a kernel (no memset), so a captured call replays correctly. */
int32_t hp_hip_topk_device_noalloc(const float *d_logits, size_t rows, size_t n, size_t k, double softcap,
                                   uint32_t *d_ids, float *d_values, void *stream);

/* Next-token sampling options, resolved as resolveGenerationSamplingOptions
 * does (generation.ts:40-76): greedy when do_sample == 0 or temperature ==
 * 0; top_k = floor(topK) >= 1; temperature finite >= 0; top_p in (0, 1]. */
typedef struct hp_hip_sampling {
  int32_t do_sample;
  int32_t top_k;
  double temperature;
  double top_p;
} hp_hip_sampling_t;

/* sampleNextToken / tokenSamplingDistribution (generation.ts:89-165) on the
 * device, over top-k candidates [column_count][k] in the order the top-k
 * entry points produce (value descending, ties to the lower id; count <= k
 * valid per column).  Per column: the top_k slice, top-p nucleus
 * (applyTopP), softmax of value / temperature in double with the JS engine's
 * exp, one draw from the generator (createDeterministicRng, state at
 * *d_rng_state, advanced per sampled column in column order; greedy draws
 * nothing).  Writes d_tokens [column_count], d_kept [column_count] (the
 * nucleus size) and d_probabilities [column_count][k] (first kept valid),
 * bit-exact with the reference.  Asynchronous on stream (NULL = library
 * stream); a decode loop keeps the generator state in HBM across steps. */
int32_t hp_hip_sample_device(const uint32_t *d_ids, const float *d_values, size_t column_count, size_t k,
                             size_t count, const hp_hip_sampling_t *sampling, uint32_t *d_rng_state,
                             int32_t *d_tokens, double *d_probabilities, int32_t *d_kept, void *stream);
/* Output head + top-k + sampling in one call (forwardOutput, then
 * sampleNextToken per column).  *rng_state (host) is read and advanced.
 * ids / values / probabilities are [column_count][k] (out_len =
 * column_count * k); tokens and kept are [column_count]. */
int32_t hp_hip_matmul_topk_sample(uint64_t handle, const float *input, size_t input_len, size_t input_size,
                                  size_t column_count, size_t k, double softcap, const hp_hip_sampling_t *sampling,
                                  uint32_t *rng_state, int32_t *tokens, uint32_t *ids, float *values,
                                  double *probabilities, int32_t *kept, size_t out_len);

/* GeGLU epilogue (layers.ts:450-456 with gelu 1062-1076):
 * out[i] = fround(gelu(gate[i]) * up[i]), bit-exact with the JS engine. */
int32_t hp_hip_geglu(const float *gate, const float *up, size_t n, float *output);
int32_t hp_hip_geglu_device(const float *d_gate, const float *d_up, size_t n, float *d_output, void *stream);

/* FFN gate/up + GeGLU: forwardFfn's matMulWeightBatch([gate, up]) followed
 * by its GeGLU loop (layers.ts:432-456): output[m][r] =
 * fround(gelu(gate_m . x)[r] * (up_m . x)[r]), bit-exact.  gate and up need
 * the same input size and row count.  With one column on large projections
 * it is a single launch: the gate and up sums of a row finish in the same
 * lane, which applies GeGLU and writes only the product; otherwise the two
 * projections run as one launch and GeGLU as a second.  output_len =
 * column_count * rows. */
int32_t hp_hip_matmul_geglu(uint64_t gate, uint64_t up, const float *input, size_t input_len, size_t input_size,
                            size_t column_count, float *output, size_t output_len);
int32_t hp_hip_matmul_geglu_device(uint64_t gate, uint64_t up, const float *d_input, size_t input_len,
                                   size_t input_size, size_t column_count, float *d_output, size_t output_len,
                                   void *stream);

/* Dequantise rows [row_start, row_start + row_count) of a handle into f32
 * [row_count][input_size] (lib.rs:1630-1664, 1709-1744; bit-exact).  Test
 * hook proving the resident layout is lossless. */
int32_t hp_hip_dequantize(uint64_t handle, size_t row_start, size_t row_count, float *output, size_t output_len);

/* Q8_K activation quantisation exactly as the matvec prologue performs it
 * (quantize_q8_k, lib.rs:1774-1811), exposed as a test hook in the
 * reference's QuantizedQ8K layout (lib.rs:1540-1544): qs [column_count]
 * [input_size] int8, d [column_count][input_size/256] f32, bsums32
 * [column_count][input_size/32] int16.  Host pointers. */
int32_t hp_hip_quantize_q8_k(const float *input, size_t input_len, size_t input_size, size_t column_count,
                             int8_t *qs, float *d, int16_t *bsums32);

/* Matvec kernel selection (no counterpart in the reference; a tuning and
 * test hook): 0 = automatic (by column count and tile count: half-split
 * vector ALU for small projections, vector ALU for one column, matrix
 * cores for several columns of large ones, the bit-exact prefill kernel
 * from 32 columns, the fast prefill kernel from 64 on *_device calls), 1 = always the
 * vector-ALU kernel, 2 = the matrix-core kernel whenever its LDS fits the
 * device, 3 = the half-split vector-ALU kernel (two lanes per row-block) for
 * up to four columns, 4 = the bit-exact prefill kernel (64-column tiles) for
 * any column count, 5 = the fast prefill kernel for any column count,
 * 6 = the wide kernel (one workgroup per block of rows) wherever it applies
 * (one weight type, one to four columns), 7 and 8 = the wide kernel with
 * whole or with half row-blocks (lane classes 0-3 / 4-7) per thread (half
 * row-blocks at one or two columns without the norm prologue or GeGLU).
 * Kernels 1-4 and 6-8 are bit-exact with the reference; the fast prefill kernel adds
 * each block's eight lane-class sums before scaling, so its outputs agree
 * within the 1e-4 relative tolerance of projections (M >= 64 prefill). */
int32_t hp_hip_set_matvec_kernel(int32_t which);

/* Pre-quantised input images inside a draft step (no counterpart in the
 * reference; a test hook): with enable != 0 (the default) the norm and GeGLU
 * launches of hp_hip_decode_layers_device at 2..8 tokens also write their
 * output as the next projection's Q8_K input, which the projection copies
 * instead of quantising; with 0 every projection quantises its f32 input
 * itself.  Both give the same bits. */
int32_t hp_hip_set_input_images(int32_t enable);

/* Launch folds of a prefill chunk in hp_hip_decode_layers_device (no
 * counterpart in the reference; a test hook): with enable != 0 (the default)
 * the norm launches write the next projection's activation tiles, the Q/K/V,
 * O and down launches leave their block-range sums for the next launch to
 * add, the attention prologue hands the queries over rounded to f16 and the
 * attention's slice merge writes O's tiles; with 0 every projection quantises
 * its own input and reduces its own ranges, and the queries stay f32.  Both
 * give the same bits. */
int32_t hp_hip_set_prefill_folds(int32_t enable);

/* Resident layouts of the weights uploaded from now on (no counterpart in
 * the reference, whose WASM arena keeps one copy of each tensor).  both != 0
 * (the default): every weight is kept twice, in the vector-ALU tile layout
 * and in the matrix-core segments, so each kernel family streams its own
 * layout at full rate.  both == 0: the tiles only, exactly the tensor's GGUF
 * byte count (hp_hip_stats.resident_bytes); the matrix-core kernels (prefill
 * chunks, drafts of several tokens) then gather their operands from the
 * tiles, slower (a 512-token prefill chunk ~30 %).  Results are the same
 * bits either way. */
int32_t hp_hip_set_weight_layouts(int32_t both);

/* wasmResidentWeightStats (wasm-kernels.ts:586-591) plus call counters. */
int32_t hp_hip_stats(hp_hip_stats_t *out);
/* Wait for all work queued on the library stream. */
int32_t hp_hip_synchronize(void);

/* Kernel timing with HIP events on the stream each kernel is launched on.
 * enable != 0 starts recording (and clears totals); read returns the total
 * device milliseconds and launch count of one kernel id since enabling. */
int32_t hp_hip_profile(int32_t enable);
int32_t hp_hip_profile_read(int32_t kernel, double *total_ms, uint64_t *launches);
/* `count` launches of an empty kernel (one workgroup of 64 lanes) on
 * `stream` (NULL = library stream), 1..65536: the floor of a launch or a
 * graph node, for measurements.  No counterpart in the reference. */
int32_t hp_hip_empty_launches(size_t count, void *stream);

/* ---- Device buffers for host runtimes without a HIP binding ------------
 * What the WebGPU runner does with its arena (device.createBuffer,
 * queue.writeBuffer, copyBufferToBuffer + mapAsync readback;
 * webgpu/segment-runner.ts:1135-1180, 942-960) for the Node runner, whose
 * hidden rows, positions, norm weights and KV rings stay in HBM between
 * calls.  hp_hip_device_alloc returns a zero-filled buffer (refused while
 * the library stream captures); hp_hip_device_free waits for the library
 * stream, then frees (NULL: no-op; any other pointer not from
 * hp_hip_device_alloc: HP_ERR_ARG).  The copies are ordered on `stream`
 * (NULL = library stream) after the work queued there and return once the
 * bytes have arrived; the device range must lie inside one buffer of
 * hp_hip_device_alloc (else HP_ERR_ARG).  hp_hip_shutdown frees what is left. */
int32_t hp_hip_device_alloc(size_t bytes, void **d_out);
int32_t hp_hip_device_free(void *d);
int32_t hp_hip_copy_to_device(void *d_dst, const void *src, size_t bytes, void *stream);
int32_t hp_hip_copy_to_host(void *dst, const void *d_src, size_t bytes, void *stream);
/* Frees the device scratch the asynchronous entry points keep for `stream`
 * (decode activations, attention partials, top-k state, prefill images;
 * one set per stream, grown and never freed while a graph captured on the
 * stream may still use it).  Call once the stream's work is done and no
 * graph captured on it will be replayed; the next call on the stream
 * allocates anew.  Waits for the stream.  NULL (the library stream) or a
 * capturing stream: HP_ERR_ARG.  No counterpart in the reference. */
int32_t hp_hip_release_stream_scratch(void *stream);

/* hp_hip_matmul_topk_sample on a device input ([column_count][input_size]
 * f32, 16-byte aligned, ordered on the library stream): forwardOutput's head,
 * topK and, when `sampling` is not NULL, sampleNextToken per column
 * (layers.ts:381-416, runtime.ts:514-527, generation.ts:40-165), only the
 * candidates (and tokens) read back.  sampling NULL: rng_state, tokens,
 * probabilities and kept are not used (may be NULL). */
int32_t hp_hip_matmul_topk_sample_device(uint64_t handle, const float *d_input, size_t input_len, size_t input_size,
                                         size_t column_count, size_t k, double softcap,
                                         const hp_hip_sampling_t *sampling, uint32_t *rng_state, int32_t *tokens,
                                         uint32_t *ids, float *values, double *probabilities, int32_t *kept,
                                         size_t out_len);

/* ---- Decoder layer for one decode token -------------------------------
 * The non-projection steps of forwardAttentionLayer / forwardFfn
 * (packages/engine/src/runner/wasm/layers.ts:161-473) on the device, for
 * chaining a whole decode step in HBM and capturing it in one HIP graph.
 * The token position is read from device memory (d_position, one int32) when
 * the kernels run, so one captured step serves every position.
 *
 * Numerics follow the reference's operation order per element; its sums (the
 * f64 sum of squares of a norm, the f32 dot products and softmax sums of
 * attention) are tree sums here, so these steps agree with the reference
 * within a tolerance, not bit for bit.  The KV cache holds f16 keys and
 * values (as the WebGPU runner's caches, shaders.ts:1134-1202) laid out
 * [head_count_kv][capacity][head_dim], entries rounded to nearest even; the
 * WASM runner keeps f32 entries.
 *
 * Calls under HIP graph capture must follow an uncaptured call of the same
 * shape on the capturing stream: the stream's scratch is sized outside
 * capture, and a call that would have to grow it while its stream is
 * capturing fails with HP_ERR_ARG. */
typedef struct hp_hip_attention_config {
  int32_t head_count;     /* query heads */
  int32_t head_count_kv;  /* key/value heads: head_count % head_count_kv == 0,
                             head_count / head_count_kv <= 8 */
  int32_t head_dim;       /* 256 (the only width the kernels take) */
  int32_t rope_dims;      /* ropeDimensionCount: even, <= head_dim (0: no RoPE) */
  double rope_freq_base;  /* ropeFreqBase */
  const float *d_rope_freq_factors; /* rope_freqs.weight [rope_dims / 2], or NULL */
  int32_t capacity;       /* KV ring slots; slot = position % capacity */
  int32_t sliding_window; /* 0: none; else the window of attentionRange */
  double epsilon;         /* layer_norm_rms_epsilon */
} hp_hip_attention_config_t;

/* rmsNormRows (layers.ts:825-832, rmsNormVector 871-885) over [rows][n]
 * (n <= 4096): out = f32((x * scale) * w), scale = 1 / sqrt(sum(x^2) / n +
 * eps) in f64.  d_weight NULL: rmsNormRowsNoWeight (834-849). */
int32_t hp_hip_rms_norm_device(const float *d_input, size_t rows, size_t n, const float *d_weight,
                               double epsilon, float *d_output, void *stream);

/* Post-norm residual of a block, fused with the next norm:
 *   d_residual_out = f32(residualAdd(d_residual, rmsNormRows(d_branch,
 *                    d_post_weight)) * scale)
 * (layers.ts:350-355 and 466-472: post_attention_norm / post_ffw_norm then
 * residualAdd 851-860; the layer output scale 360-369 with scale 1 when
 * absent), then, when d_next_out is not NULL, d_next_out =
 * rmsNormRows(d_residual_out, d_next_weight) (the next ffn_norm,
 * attn_norm or output_norm).  d_residual_out may equal d_residual. */
int32_t hp_hip_residual_norm_device(const float *d_branch, size_t rows, size_t n, const float *d_post_weight,
                                    const float *d_residual, float scale, float *d_residual_out,
                                    const float *d_next_weight, float *d_next_out, double epsilon,
                                    void *stream);

/* Attention prologue (layers.ts:205-268, as the WebGPU runner fuses it,
 * shaders.ts:1306-1385) of token_count (1..8) tokens at positions
 * *d_position + t: q = ropeNeox(normHeads(d_q, d_q_norm)) -> d_q_out
 * [token][head_count][256]; k = ropeNeox(normHeads(d_k, d_k_norm)) and v =
 * rmsNormRowsNoWeight(d_v) ([token][head_count_kv][256]) appended to the
 * caches at slot position % capacity (updateFullAttentionCache,
 * layers.ts:887-911).  d_v NULL: the value shares the key projection
 * (layerValueProjectionModes "shared-with-key", layers.ts:231-238). */
int32_t hp_hip_attention_prep_device(const hp_hip_attention_config_t *config, size_t token_count, const float *d_q,
                                     const float *d_k, const float *d_v, const float *d_q_norm,
                                     const float *d_k_norm, const int32_t *d_position, float *d_q_out,
                                     uint16_t *d_key_cache, uint16_t *d_value_cache, void *stream);

/* GQA attention of token_count (1..8) tokens at positions *d_position + t
 * over the caches, as forwardAttentionLayer runs it (layers.ts:270-335): the
 * window is attentionRange of the largest position (972-980), each token
 * sees the keys up to its own position (causalMask, 913-925), scores and
 * softmax as hp_gqa_attention_f32 (packages/engine/wasm-kernels/src/
 * lib.rs:538-654) with scale 1 and an f16-rounded query, then castF16Rows
 * (layers.ts:982-988).  d_q and d_output are [token][head_count][256]. */
int32_t hp_hip_gqa_attention_device(const hp_hip_attention_config_t *config, size_t token_count, const float *d_q,
                                    const uint16_t *d_key_cache, const uint16_t *d_value_cache,
                                    const int32_t *d_position, float *d_output, void *stream);

/* One decoder layer's weights and state.  Handles from hp_hip_weight_upload*;
 * attn_v 0 means the value shares the key projection.  Norm weights are f32
 * device arrays: attn_norm, post_attention_norm, ffn_norm, post_ffw_norm
 * [hidden]; attn_q_norm, attn_k_norm [head_dim]. */
typedef struct hp_hip_decode_layer {
  uint64_t attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down;
  const float *d_attn_norm, *d_attn_q_norm, *d_attn_k_norm, *d_post_attention_norm, *d_ffn_norm,
      *d_post_ffw_norm;
  float layer_output_scale; /* layer_output_scale.weight[0], or 1 */
  int32_t reserved;         /* 0 */
  uint16_t *d_key_cache, *d_value_cache; /* f16 [head_count_kv][capacity][head_dim] */
  hp_hip_attention_config_t attention;
  /* The per-layer input step (applyPerLayerInput, layers.ts:475-521), after
   * the FFN's residual and before the layer output scale:
   *   x = x + rmsNormRows(proj . f32(gelu(inp_gate . x) * input), post_norm).
   * inp_gate [per_layer_length][hidden] and proj [hidden][per_layer_length]
   * handles (both 0: the layer has no such step), post_norm [hidden] f32, and
   * this layer's rows of the prepared per-layer inputs, [token_count]
   * [per_layer_length] f32 (the caller points each layer at its own block
   * of preparePerLayerInputs' [layer][token][per_layer_length] array). */
  uint64_t inp_gate, proj;
  const float *d_post_norm;
  const float *d_per_layer_input;
} hp_hip_decode_layer_t;

/* forwardAttentionLayer (layers.ts:161-379, with forwardFfn 418-473) for
 * token_count (1..8) tokens at positions *d_position + t through
 * layers[0 .. layer_count): d_hidden [token][hidden] is the residual stream,
 * updated in place; every token's row is kept (a draft being verified needs
 * each position's logits, as the WebGPU MTP target runner reads all hidden
 * rows, mtp-target-runner.ts:80-130).  When d_output_norm is not NULL,
 * d_output [token][hidden] = rmsNormRows(hidden, d_output_norm)
 * (forwardOutput's final norm, layers.ts:389-396), ready for the output head.
 * Per layer (one token): Q/K/V in one matvec launch whose prologue forms
 * attn_norm of the residual, attention with the head norms, RoPE and the
 * cache append inside it plus the merge, O, gate/up + GeGLU whose prologue
 * forms the post-attention residual and ffn_norm, down.  Several tokens add a
 * prologue launch (norms, RoPE, every token's cache append) before the
 * attention, and the norms run as their own launches.  A layer with the
 * per-layer input step adds a norm launch (the FFN residual), the inp_gate
 * matvec, the gelu product and the proj matvec. */
int32_t hp_hip_decode_layers_device(const hp_hip_decode_layer_t *layers, size_t layer_count, size_t token_count,
                                    float *d_hidden, const int32_t *d_position, const float *d_output_norm,
                                    float *d_output, void *stream);

/* On request, the one-token step of hp_hip_decode_layers_device runs as one
 * persistent launch (one workgroup per CU, every layer's stages inside it,
 * values handed between stages as round-tagged words) when the layers are
 * within what it covers: hidden size a multiple of 256 up to 4096, at most 511
 * layers, RoPE over 0, 128 or 256 dims, caches of at most 4096 slots, gate
 * and up of one type, and each stage's share of rows within the
 * workgroup's task slots; otherwise, and at 2..65536 tokens, the launch
 * sequence runs.  Both give identical bits.  No counterpart in the
 * reference; these are a switch and test hooks for it:
 *   hp_hip_set_decode_fused: 1 uses the persistent step where it applies,
 *     0 (the default) always the launch sequence, which is the faster of
 *     the two on gfx950;
 *   hp_hip_set_fused_wait_limit: the bound of one stage wait in 10 ns ticks
 *     (0: the default, one second).  A wait past it ends the launch early,
 *     leaves invalid outputs and a status that the next call below reports;
 *     every launch reached after that skips its work until the status is
 *     read;
 *   hp_hip_decode_fused_status: waits for `stream` (NULL = library stream)
 *     and returns HP_ERR_HIP (clearing the status) when a persistent step
 *     queued on it stopped at a wait, else HP_OK. */
int32_t hp_hip_set_decode_fused(int32_t mode);
int32_t hp_hip_set_fused_wait_limit(uint64_t ticks);
int32_t hp_hip_decode_fused_status(void *stream);
/* Stage timeline of later persistent steps (a profiling hook): with a
 * device buffer of at least compute_units * layers * 48 uint64 entries,
 * workgroup w stamps the 100 MHz s_memrealtime clock at eight points of
 * stage s (0..5: Q/K/V, attention, merge, O, gate/up, down) of layer l at
 * d_stamps[((w * layers + l) * 6 + s) * 8 + k]: k = 0 stage start, 1 loads
 * issued, 2 input arrived, 3 prologue done, 4 weights in registers, 5
 * products done, 6 chains done, 7 end (points a stage lacks stay 0).
 * NULL turns it off; a shorter buffer is not written. */
int32_t hp_hip_set_fused_trace(uint64_t *d_stamps, size_t len);

#ifdef __cplusplus
}
#endif
#endif
