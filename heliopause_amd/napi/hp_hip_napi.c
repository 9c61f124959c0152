/*
 * hp_hip_napi.c -- Node N-API binding of the HIP runner's C ABI (hp_hip.h).
 *
 * The binding the engine's TS runner loads (hip-kernels.js / .ts) in place of
 * the WASM module behind packages/engine/src/runner/wasm/wasm-kernels.ts: it
 * turns typed arrays into pointers and lengths and returns status codes
 * unchanged; the JS layer maps them as assertWasmOk does
 * (wasm-kernels.ts:1882-1896).  Projections run as napi_async_work on the
 * libuv pool and resolve Promises (the reference's API is async); the C ABI
 * serialises its calls internally.  Handles cross into JS as BigInt.
 *
 * Exports:
 *   statusString(code), lastError(), deviceCount(), init(device)
 *   upload(typeId, Uint8Array, inputSize, rowCount) -> {status, handle}
 *   release(handle), info(handle) -> {status, typeId, inputSize, rowCount, byteLength}
 *   stats() -> {handleCount, residentBytes, scratchBytes, matmulCalls, kernelLaunches, device, computeUnits}
 *   matmulMulti(handles[], Float32Array, inputSize, columnCount, rowCounts[]) -> Promise<{status, error, outputs[]}>
 *   matmulTopK(handle, Float32Array, inputSize, columnCount, k, softcap) -> Promise<{status, error, ids, values}>
 *   matmulGeglu(gate, up, Float32Array, inputSize, columnCount, rowCount) -> Promise<{status, error, output}>
 *   dequantize(handle, rowStart, rowCount, inputSize) -> {status, output}
 *   geglu(Float32Array gate, Float32Array up) -> {status, output}
 *   matmulTopKSample(handle, Float32Array, inputSize, columnCount, k, softcap,
 *                    {doSample, topK, temperature, topP}, Uint32Array(1) rngState)
 *       -> Promise<{status, error, tokens, ids, values, probabilities, kept}>
 *   ggufOpen(path, maxArraySample, completeArrayKeys[]) -> {status, error, file}
 *   ggufInfo(file) -> parseGguf's GgufMetadata (gguf.ts:30-37) + byteLength per tensor
 *   ggufUpload(file, tensorIndices[]) -> Promise<{status, error, handles[], statuses[]}>
 *   ggufClose(file)
 * device-resident decode (napi/hip/segment-runner.js):
 *   deviceAlloc(bytes) -> {status, ptr}, deviceFree(ptr) -> status
 *   copyToDevice(ptr, typedArray, byteOffset) / copyToHost(ptr, typedArray, byteOffset) -> status
 *   runLayers(layers[], tokenCount, hiddenSize, {hidden, position, outputNorm, output}, Float32Array | null,
 *             position, readOutput, rowStart, rowCount) -> Promise<{status, error, output}>
 *   headTopK(handle, dInput, inputSize, columnCount, k, softcap, sampling | null, Uint32Array | null)
 *       -> Promise<{status, error, ids, values[, tokens, probabilities, kept]}>
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hp_gguf.h"
#include "hp_hip.h"

#define CHECK(env, call)                                             \
  do {                                                               \
    if ((call) != napi_ok) {                                         \
      napi_throw_error((env), NULL, "hp_hip addon: N-API call failed"); \
      return NULL;                                                   \
    }                                                                \
  } while (0)

static napi_value make_i32(napi_env env, int32_t v) {
  napi_value r;
  napi_create_int32(env, v, &r);
  return r;
}

static napi_value make_f64(napi_env env, double v) {
  napi_value r;
  napi_create_double(env, v, &r);
  return r;
}

static void set(napi_env env, napi_value obj, const char *name, napi_value v) {
  napi_set_named_property(env, obj, name, v);
}

static int get_u64(napi_env env, napi_value v, uint64_t *out) {
  bool lossless = false;
  if (napi_get_value_bigint_uint64(env, v, out, &lossless) == napi_ok) return 1;
  double d;
  if (napi_get_value_double(env, v, &d) == napi_ok && d >= 0) {
    *out = (uint64_t)d;
    return 1;
  }
  return 0;
}

static int get_size(napi_env env, napi_value v, size_t *out) {
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok || d < 0 || d != (double)(size_t)d) return 0;
  *out = (size_t)d;
  return 1;
}

/* typed array of the given type: data pointer and element count */
static int get_typed(napi_env env, napi_value v, napi_typedarray_type want, void **data, size_t *len) {
  bool is = false;
  if (napi_is_typedarray(env, v, &is) != napi_ok || !is) return 0;
  napi_typedarray_type t;
  napi_value ab;
  size_t off;
  if (napi_get_typedarray_info(env, v, &t, len, data, &ab, &off) != napi_ok || t != want) return 0;
  return 1;
}

static void free_cb(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  free(data);
}

/* hands a malloc'd buffer of n elements to JS as a typed array */
static napi_value adopt(napi_env env, void *data, size_t n, size_t elem, napi_typedarray_type t) {
  napi_value ab, arr;
  if (n == 0) {
    void *p;
    napi_create_arraybuffer(env, 0, &p, &ab);
    free(data);
  } else if (napi_create_external_arraybuffer(env, data, n * elem, free_cb, NULL, &ab) != napi_ok) {
    free(data);
    return NULL;
  }
  napi_create_typedarray(env, t, n, ab, 0, &arr);
  return arr;
}

static napi_value js_status_string(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1], r;
  int32_t code = 0;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  napi_get_value_int32(env, argv[0], &code);
  napi_create_string_utf8(env, hp_hip_status_string(code), NAPI_AUTO_LENGTH, &r);
  return r;
}

static napi_value js_last_error(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  napi_create_string_utf8(env, hp_hip_last_error(), NAPI_AUTO_LENGTH, &r);
  return r;
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int32_t n = 0;
  const int32_t rc = hp_hip_device_count(&n);
  return make_i32(env, rc == HP_OK ? n : 0);
}

static napi_value js_init(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  int32_t dev = 0;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc > 0) napi_get_value_int32(env, argv[0], &dev);
  return make_i32(env, hp_hip_init(dev));
}

static napi_value js_upload(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value argv[4], r, hv;
  int32_t type_id = 0;
  void *data;
  size_t len, input_size, rows;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 4 || napi_get_value_int32(env, argv[0], &type_id) != napi_ok ||
      !get_typed(env, argv[1], napi_uint8_array, &data, &len) || !get_size(env, argv[2], &input_size) ||
      !get_size(env, argv[3], &rows)) {
    napi_throw_type_error(env, NULL, "upload(typeId, Uint8Array, inputSize, rowCount)");
    return NULL;
  }
  uint64_t h = 0;
  const int32_t rc = hp_hip_weight_upload(type_id, (const uint8_t *)data, len, input_size, rows, &h);
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  napi_create_bigint_uint64(env, h, &hv);
  set(env, r, "handle", hv);
  return r;
}

static napi_value js_release(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  uint64_t h = 0;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 1 || !get_u64(env, argv[0], &h)) {
    napi_throw_type_error(env, NULL, "release(handle)");
    return NULL;
  }
  return make_i32(env, hp_hip_weight_release(h));
}

static napi_value js_info(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1], r;
  uint64_t h = 0;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 1 || !get_u64(env, argv[0], &h)) {
    napi_throw_type_error(env, NULL, "info(handle)");
    return NULL;
  }
  int32_t t = 0;
  size_t in = 0, rows = 0, bytes = 0;
  const int32_t rc = hp_hip_weight_info(h, &t, &in, &rows, &bytes);
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  set(env, r, "typeId", make_i32(env, t));
  set(env, r, "inputSize", make_f64(env, (double)in));
  set(env, r, "rowCount", make_f64(env, (double)rows));
  set(env, r, "byteLength", make_f64(env, (double)bytes));
  return r;
}

static napi_value js_stats(napi_env env, napi_callback_info info) {
  (void)info;
  hp_hip_stats_t st;
  memset(&st, 0, sizeof st);
  const int32_t rc = hp_hip_stats(&st);
  napi_value r;
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  set(env, r, "handleCount", make_f64(env, (double)st.handle_count));
  set(env, r, "residentBytes", make_f64(env, (double)st.resident_bytes));
  set(env, r, "scratchBytes", make_f64(env, (double)st.scratch_bytes));
  set(env, r, "matmulCalls", make_f64(env, (double)st.matmul_calls));
  set(env, r, "kernelLaunches", make_f64(env, (double)st.kernel_launches));
  set(env, r, "device", make_i32(env, st.device));
  set(env, r, "computeUnits", make_i32(env, st.compute_units));
  return r;
}

/* ---- asynchronous projections ------------------------------------------ */

enum { JOB_MULTI, JOB_TOPK, JOB_GEGLU, JOB_SAMPLE };

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref input_ref;
  int kind;
  uint64_t handles[4];
  size_t count;
  const float *input;
  size_t input_len, input_size, columns;
  float *outputs[4];
  size_t output_lens[4];
  size_t k;
  double softcap;
  uint32_t *ids;
  size_t rows[4];
  hp_hip_sampling_t sampling;
  uint32_t rng;           /* generator state in, advanced state out */
  napi_ref rng_ref;       /* the caller's Uint32Array(1), updated on completion */
  uint32_t *rng_out;
  int32_t *tokens, *kept;
  double *probs;
  int32_t status;
  char error[512]; /* hp_hip_last_error of the worker thread */
} Job;

static void job_execute(napi_env env, void *data) {
  (void)env;
  Job *j = (Job *)data;
  if (j->kind == JOB_MULTI) {
    j->status = j->count == 1
                    ? hp_hip_matmul(j->handles[0], j->input, j->input_len, j->input_size, j->rows[0],
                                    j->columns, j->outputs[0], j->output_lens[0])
                    : hp_hip_matmul_multi(j->count, j->handles, j->input, j->input_len, j->input_size, j->columns,
                                          j->outputs, j->output_lens);
  } else if (j->kind == JOB_TOPK) {
    j->status = hp_hip_matmul_topk(j->handles[0], j->input, j->input_len, j->input_size, j->columns, j->k,
                                   j->softcap, j->ids, j->outputs[0], j->output_lens[0]);
  } else if (j->kind == JOB_SAMPLE) {
    j->status = hp_hip_matmul_topk_sample(j->handles[0], j->input, j->input_len, j->input_size, j->columns, j->k,
                                          j->softcap, &j->sampling, &j->rng, j->tokens, j->ids, j->outputs[0],
                                          j->probs, j->kept, j->output_lens[0]);
  } else {
    j->status = hp_hip_matmul_geglu(j->handles[0], j->handles[1], j->input, j->input_len, j->input_size, j->columns,
                                    j->outputs[0], j->output_lens[0]);
  }
  if (j->status != HP_OK) {
    strncpy(j->error, hp_hip_last_error(), sizeof j->error - 1);
    j->error[sizeof j->error - 1] = 0;
  }
}

static void job_complete(napi_env env, napi_status s, void *data) {
  (void)s;
  Job *j = (Job *)data;
  napi_value r;
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, j->status));
  napi_value err;
  napi_create_string_utf8(env, j->error, NAPI_AUTO_LENGTH, &err);
  set(env, r, "error", err);
  if (j->kind == JOB_MULTI) {
    napi_value outs;
    napi_create_array_with_length(env, j->count, &outs);
    for (size_t i = 0; i < j->count; i++) {
      napi_set_element(env, outs, (uint32_t)i, adopt(env, j->outputs[i], j->output_lens[i], 4, napi_float32_array));
      j->outputs[i] = NULL;
    }
    set(env, r, "outputs", outs);
  } else if (j->kind == JOB_TOPK) {
    set(env, r, "ids", adopt(env, j->ids, j->output_lens[0], 4, napi_uint32_array));
    set(env, r, "values", adopt(env, j->outputs[0], j->output_lens[0], 4, napi_float32_array));
    j->ids = NULL;
    j->outputs[0] = NULL;
  } else if (j->kind == JOB_SAMPLE) {
    set(env, r, "ids", adopt(env, j->ids, j->output_lens[0], 4, napi_uint32_array));
    set(env, r, "values", adopt(env, j->outputs[0], j->output_lens[0], 4, napi_float32_array));
    set(env, r, "probabilities", adopt(env, j->probs, j->output_lens[0], 8, napi_float64_array));
    set(env, r, "tokens", adopt(env, j->tokens, j->columns, 4, napi_int32_array));
    set(env, r, "kept", adopt(env, j->kept, j->columns, 4, napi_int32_array));
    j->ids = NULL;
    j->outputs[0] = NULL;
    j->probs = NULL;
    j->tokens = NULL;
    j->kept = NULL;
    if (j->status == HP_OK && j->rng_out) *j->rng_out = j->rng;  /* the caller's state advances */
    napi_delete_reference(env, j->rng_ref);
  } else {
    set(env, r, "output", adopt(env, j->outputs[0], j->output_lens[0], 4, napi_float32_array));
    j->outputs[0] = NULL;
  }
  napi_delete_reference(env, j->input_ref);
  napi_resolve_deferred(env, j->deferred, r);
  napi_delete_async_work(env, j->work);
  for (size_t i = 0; i < 4; i++) free(j->outputs[i]);
  free(j->ids);
  free(j->probs);
  free(j->tokens);
  free(j->kept);
  free(j);
}

static napi_value start_job(napi_env env, Job *j, napi_value input, const char *name) {
  napi_value promise, wname;
  napi_create_reference(env, input, 1, &j->input_ref);  /* keeps the input alive on the worker */
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &wname);
  napi_create_async_work(env, NULL, wname, job_execute, job_complete, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

static int alloc_outputs(Job *j) {
  for (size_t i = 0; i < j->count; i++) {
    j->outputs[i] = (float *)malloc(j->output_lens[i] ? j->output_lens[i] * sizeof(float) : 1);
    if (!j->outputs[i]) return 0;
  }
  return 1;
}

static void free_job(Job *j) {
  for (size_t i = 0; i < 4; i++) free(j->outputs[i]);
  free(j->ids);
  free(j->probs);
  free(j->tokens);
  free(j->kept);
  free(j);
}

static napi_value js_matmul_multi(napi_env env, napi_callback_info info) {
  size_t argc = 5;
  napi_value argv[5];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  Job *j = (Job *)calloc(1, sizeof(Job));
  uint32_t n = 0, nr = 0;
  void *in;
  bool is_arr = false, is_arr2 = false;
  if (!j) return NULL;
  j->kind = JOB_MULTI;
  if (argc < 5 || napi_is_array(env, argv[0], &is_arr) != napi_ok || !is_arr ||
      napi_get_array_length(env, argv[0], &n) != napi_ok || n < 1 || n > 4 ||
      !get_typed(env, argv[1], napi_float32_array, &in, &j->input_len) || !get_size(env, argv[2], &j->input_size) ||
      !get_size(env, argv[3], &j->columns) || napi_is_array(env, argv[4], &is_arr2) != napi_ok || !is_arr2 ||
      napi_get_array_length(env, argv[4], &nr) != napi_ok || nr != n) {
    free_job(j);
    napi_throw_type_error(env, NULL, "matmulMulti(handles[1..4], Float32Array, inputSize, columnCount, rowCounts[])");
    return NULL;
  }
  j->count = n;
  j->input = (const float *)in;
  for (uint32_t i = 0; i < n; i++) {
    napi_value h, rc;
    size_t rows;
    napi_get_element(env, argv[0], i, &h);
    napi_get_element(env, argv[4], i, &rc);
    if (!get_u64(env, h, &j->handles[i]) || !get_size(env, rc, &rows)) {
      free_job(j);
      napi_throw_type_error(env, NULL, "matmulMulti: bad handle or row count");
      return NULL;
    }
    j->rows[i] = rows;
    j->output_lens[i] = rows * j->columns;
  }
  if (!alloc_outputs(j)) {
    free_job(j);
    napi_throw_error(env, NULL, "matmulMulti: out of host memory");
    return NULL;
  }
  return start_job(env, j, argv[1], "hp_hip_matmul_multi");
}

static napi_value js_matmul_topk(napi_env env, napi_callback_info info) {
  size_t argc = 6;
  napi_value argv[6];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  Job *j = (Job *)calloc(1, sizeof(Job));
  void *in;
  if (!j) return NULL;
  j->kind = JOB_TOPK;
  j->count = 1;
  if (argc < 6 || !get_u64(env, argv[0], &j->handles[0]) ||
      !get_typed(env, argv[1], napi_float32_array, &in, &j->input_len) || !get_size(env, argv[2], &j->input_size) ||
      !get_size(env, argv[3], &j->columns) || !get_size(env, argv[4], &j->k) ||
      napi_get_value_double(env, argv[5], &j->softcap) != napi_ok) {
    free_job(j);
    napi_throw_type_error(env, NULL, "matmulTopK(handle, Float32Array, inputSize, columnCount, k, softcap)");
    return NULL;
  }
  j->input = (const float *)in;
  j->output_lens[0] = j->columns * j->k;
  j->ids = (uint32_t *)malloc(j->output_lens[0] ? j->output_lens[0] * 4 : 1);
  if (!j->ids || !alloc_outputs(j)) {
    free_job(j);
    napi_throw_error(env, NULL, "matmulTopK: out of host memory");
    return NULL;
  }
  return start_job(env, j, argv[1], "hp_hip_matmul_topk");
}

static napi_value js_matmul_geglu(napi_env env, napi_callback_info info) {
  size_t argc = 6;
  napi_value argv[6];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  Job *j = (Job *)calloc(1, sizeof(Job));
  void *in;
  size_t rows;
  if (!j) return NULL;
  j->kind = JOB_GEGLU;
  j->count = 1;
  if (argc < 6 || !get_u64(env, argv[0], &j->handles[0]) || !get_u64(env, argv[1], &j->handles[1]) ||
      !get_typed(env, argv[2], napi_float32_array, &in, &j->input_len) || !get_size(env, argv[3], &j->input_size) ||
      !get_size(env, argv[4], &j->columns) || !get_size(env, argv[5], &rows)) {
    free_job(j);
    napi_throw_type_error(env, NULL, "matmulGeglu(gate, up, Float32Array, inputSize, columnCount, rowCount)");
    return NULL;
  }
  j->input = (const float *)in;
  j->output_lens[0] = rows * j->columns;
  if (!alloc_outputs(j)) {
    free_job(j);
    napi_throw_error(env, NULL, "matmulGeglu: out of host memory");
    return NULL;
  }
  return start_job(env, j, argv[2], "hp_hip_matmul_geglu");
}

static int get_prop_f64(napi_env env, napi_value obj, const char *name, double *out) {
  napi_value v;
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return 0;
  if (napi_get_named_property(env, obj, name, &v) != napi_ok) return 0;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_boolean) {
    bool b;
    napi_get_value_bool(env, v, &b);
    *out = b ? 1.0 : 0.0;
    return 1;
  }
  return napi_get_value_double(env, v, out) == napi_ok;
}

static napi_value js_matmul_topk_sample(napi_env env, napi_callback_info info) {
  size_t argc = 8;
  napi_value argv[8];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  Job *j = (Job *)calloc(1, sizeof(Job));
  void *in, *rng;
  size_t rng_len = 0;
  double do_sample = 1, top_k = 0, temperature = 0, top_p = 0;
  if (!j) return NULL;
  j->kind = JOB_SAMPLE;
  j->count = 1;
  if (argc < 8 || !get_u64(env, argv[0], &j->handles[0]) ||
      !get_typed(env, argv[1], napi_float32_array, &in, &j->input_len) || !get_size(env, argv[2], &j->input_size) ||
      !get_size(env, argv[3], &j->columns) || !get_size(env, argv[4], &j->k) ||
      napi_get_value_double(env, argv[5], &j->softcap) != napi_ok || !get_prop_f64(env, argv[6], "topK", &top_k) ||
      !get_prop_f64(env, argv[6], "temperature", &temperature) || !get_prop_f64(env, argv[6], "topP", &top_p) ||
      !get_typed(env, argv[7], napi_uint32_array, &rng, &rng_len) || rng_len < 1) {
    free_job(j);
    napi_throw_type_error(env, NULL,
                          "matmulTopKSample(handle, Float32Array, inputSize, columnCount, k, softcap, "
                          "{doSample, topK, temperature, topP}, Uint32Array rngState)");
    return NULL;
  }
  get_prop_f64(env, argv[6], "doSample", &do_sample);
  j->sampling.do_sample = do_sample != 0;
  j->sampling.top_k = top_k >= 2147483647.0 ? 2147483647 : (int32_t)top_k;
  j->sampling.temperature = temperature;
  j->sampling.top_p = top_p;
  j->input = (const float *)in;
  j->rng_out = (uint32_t *)rng;
  j->rng = j->rng_out[0];
  j->output_lens[0] = j->columns * j->k;
  const size_t n = j->output_lens[0] ? j->output_lens[0] : 1, c = j->columns ? j->columns : 1;
  j->ids = (uint32_t *)malloc(n * 4);
  j->outputs[0] = (float *)malloc(n * 4);
  j->probs = (double *)malloc(n * 8);
  j->tokens = (int32_t *)malloc(c * 4);
  j->kept = (int32_t *)malloc(c * 4);
  if (!j->ids || !j->outputs[0] || !j->probs || !j->tokens || !j->kept) {
    free_job(j);
    napi_throw_error(env, NULL, "matmulTopKSample: out of host memory");
    return NULL;
  }
  napi_create_reference(env, argv[7], 1, &j->rng_ref);  /* the state array outlives the worker */
  return start_job(env, j, argv[1], "hp_hip_matmul_topk_sample");
}

/* ---- synchronous test hooks -------------------------------------------- */

static napi_value js_dequantize(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value argv[4], r;
  uint64_t h;
  size_t row_start, rows, input_size;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 4 || !get_u64(env, argv[0], &h) || !get_size(env, argv[1], &row_start) ||
      !get_size(env, argv[2], &rows) || !get_size(env, argv[3], &input_size)) {
    napi_throw_type_error(env, NULL, "dequantize(handle, rowStart, rowCount, inputSize)");
    return NULL;
  }
  const size_t n = rows * input_size;
  float *out = (float *)malloc(n ? n * 4 : 1);
  if (!out) return NULL;
  const int32_t rc = hp_hip_dequantize(h, row_start, rows, out, n);
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  set(env, r, "output", adopt(env, out, n, 4, napi_float32_array));
  return r;
}

static napi_value js_geglu(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value argv[2], r;
  void *g, *u;
  size_t ng, nu;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 2 || !get_typed(env, argv[0], napi_float32_array, &g, &ng) ||
      !get_typed(env, argv[1], napi_float32_array, &u, &nu) || ng != nu) {
    napi_throw_type_error(env, NULL, "geglu(Float32Array gate, Float32Array up) of equal lengths");
    return NULL;
  }
  float *out = (float *)malloc(ng ? ng * 4 : 1);
  if (!out) return NULL;
  const int32_t rc = hp_hip_geglu((const float *)g, (const float *)u, ng, out);
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  set(env, r, "output", adopt(env, out, ng, 4, napi_float32_array));
  return r;
}

/* ---- GGUF files ----------------------------------------------------------- */

typedef struct {
  hp_gguf_t *g;
  int busy; /* async uploads in flight */
  int close_requested;
} GgufBox;

static void gguf_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  GgufBox *b = (GgufBox *)data;
  if (b->g) hp_gguf_close(b->g);
  free(b);
}

static GgufBox *get_box(napi_env env, napi_value v) {
  void *p = NULL;
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return (GgufBox *)p;
}

static napi_value js_gguf_open(napi_env env, napi_callback_info info) {
  size_t argc = 3;
  napi_value argv[3], r, ext;
  char path[4096];
  size_t plen = 0;
  double max_sample = 16;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  if (argc < 1 || napi_get_value_string_utf8(env, argv[0], path, sizeof path, &plen) != napi_ok ||
      plen >= sizeof path - 1) {
    napi_throw_type_error(env, NULL, "ggufOpen(path, maxArraySample?, completeArrayKeys?)");
    return NULL;
  }
  if (argc > 1) napi_get_value_double(env, argv[1], &max_sample);
  uint32_t nkeys = 0;
  bool is_arr = false;
  if (argc > 2 && napi_is_array(env, argv[2], &is_arr) == napi_ok && is_arr) napi_get_array_length(env, argv[2], &nkeys);
  char **keys = (char **)calloc(nkeys ? nkeys : 1, sizeof(char *));
  for (uint32_t i = 0; keys && i < nkeys; i++) {
    napi_value k;
    size_t len = 0;
    napi_get_element(env, argv[2], i, &k);
    if (napi_get_value_string_utf8(env, k, NULL, 0, &len) != napi_ok) continue;
    keys[i] = (char *)malloc(len + 1);
    if (keys[i]) napi_get_value_string_utf8(env, k, keys[i], len + 1, &len);
  }
  hp_gguf_t *g = NULL;
  const uint64_t ms = max_sample >= 9007199254740991.0 ? 9007199254740991ull
                      : max_sample > 0 ? (uint64_t)max_sample : 0;
  const int32_t rc = hp_gguf_open(path, ms, (const char *const *)keys, nkeys, &g);
  for (uint32_t i = 0; keys && i < nkeys; i++) free(keys[i]);
  free(keys);
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  napi_value err;
  napi_create_string_utf8(env, rc == 0 ? "" : hp_gguf_last_error(), NAPI_AUTO_LENGTH, &err);
  set(env, r, "error", err);
  if (rc == 0) {
    GgufBox *b = (GgufBox *)calloc(1, sizeof(GgufBox));
    if (!b) {
      hp_gguf_close(g);
      napi_throw_error(env, NULL, "out of host memory");
      return NULL;
    }
    b->g = g;
    napi_create_external(env, b, gguf_finalize, NULL, &ext);
    set(env, r, "file", ext);
  }
  return r;
}

static napi_value gguf_value(napi_env env, const hp_gguf_t *g, const hp_gguf_value_t *v) {
  static const char *names[] = {"uint8", "int8", "uint16", "int16", "uint32", "int32", "float32",
                                "bool",  "string", "array", "uint64", "int64", "float64"};
  napi_value r;
  if (v->type == HP_GGUF_STRING) {
    napi_create_string_utf8(env, v->string, (size_t)v->string_length, &r);
  } else if (v->type == HP_GGUF_BOOL) {
    napi_get_boolean(env, v->number != 0, &r);
  } else if (v->type != HP_GGUF_ARRAY) {
    napi_create_double(env, v->number, &r);
  } else {
    napi_value sample, t, b;
    napi_create_object(env, &r);
    napi_create_string_utf8(env, v->element_type >= 0 && v->element_type <= 12 ? names[v->element_type] : "array",
                            NAPI_AUTO_LENGTH, &t);
    set(env, r, "type", t);
    set(env, r, "length", make_f64(env, (double)v->length));
    napi_create_array_with_length(env, (size_t)v->sample_count, &sample);
    for (uint64_t i = 0; i < v->sample_count; i++) {
      hp_gguf_value_t c;
      hp_gguf_array_element(g, v->node, i, &c);
      napi_set_element(env, sample, (uint32_t)i, gguf_value(env, g, &c));
    }
    set(env, r, "sample", sample);
    napi_get_boolean(env, v->truncated != 0, &b);
    set(env, r, "truncated", b);
  }
  return r;
}

static napi_value make_bigint(napi_env env, uint64_t v) {
  napi_value r;
  napi_create_bigint_uint64(env, v, &r);
  return r;
}

static napi_value js_gguf_info(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1], r, md, tensors;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  GgufBox *b = argc > 0 ? get_box(env, argv[0]) : NULL;
  if (!b || !b->g) {
    napi_throw_type_error(env, NULL, "ggufInfo(file): not an open GGUF file");
    return NULL;
  }
  uint32_t version = 0;
  uint64_t tc = 0, mc = 0, ds = 0, al = 0, fs = 0;
  hp_gguf_header(b->g, &version, &tc, &mc, &ds, &al, &fs);
  napi_create_object(env, &r);
  set(env, r, "version", make_f64(env, version));
  set(env, r, "tensorCount", make_f64(env, (double)tc));
  set(env, r, "metadataCount", make_f64(env, (double)mc));
  set(env, r, "dataStart", make_bigint(env, ds));
  set(env, r, "alignment", make_f64(env, (double)al));
  set(env, r, "fileSize", make_f64(env, (double)fs));
  napi_create_object(env, &md);
  const uint64_t n = hp_gguf_metadata_count(b->g);
  for (uint64_t i = 0; i < n; i++) {
    const char *key;
    uint64_t klen;
    hp_gguf_value_t v;
    napi_value kv;
    hp_gguf_metadata_entry(b->g, i, &key, &klen, &v);
    napi_create_string_utf8(env, key, (size_t)klen, &kv);
    napi_set_property(env, md, kv, gguf_value(env, b->g, &v));
  }
  set(env, r, "metadata", md);
  napi_create_array_with_length(env, (size_t)tc, &tensors);
  for (uint64_t i = 0; i < tc; i++) {
    hp_gguf_tensor_t t;
    napi_value o, name, dims, tn;
    hp_gguf_tensor_info(b->g, i, &t);
    napi_create_object(env, &o);
    napi_create_string_utf8(env, t.name, (size_t)t.name_length, &name);
    set(env, o, "name", name);
    napi_create_array_with_length(env, t.n_dims, &dims);
    for (uint32_t d = 0; d < t.n_dims; d++) napi_set_element(env, dims, d, make_f64(env, (double)t.dims[d]));
    set(env, o, "dimensions", dims);
    napi_create_string_utf8(env, hp_gguf_type_name(t.type_id), NAPI_AUTO_LENGTH, &tn);
    set(env, o, "type", tn);
    set(env, o, "typeId", make_f64(env, t.type_id));
    set(env, o, "offset", make_bigint(env, t.offset));
    set(env, o, "dataOffset", make_bigint(env, t.data_offset));
    if (t.storage_known) set(env, o, "byteLength", make_f64(env, (double)t.byte_length));
    napi_set_element(env, tensors, (uint32_t)i, o);
  }
  set(env, r, "tensors", tensors);
  return r;
}

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref file_ref;
  GgufBox *box;
  size_t count;
  uint64_t *indices, *handles;
  int32_t *statuses;
  int32_t status;
  char error[512];
} GgufJob;

static void gguf_execute(napi_env env, void *data) {
  (void)env;
  GgufJob *j = (GgufJob *)data;
  j->status = hp_hip_weight_upload_gguf(j->box->g, j->count, j->indices, j->handles, j->statuses);
  if (j->status != HP_OK) {
    strncpy(j->error, hp_hip_last_error(), sizeof j->error - 1);
    j->error[sizeof j->error - 1] = 0;
  }
}

static void gguf_complete(napi_env env, napi_status s, void *data) {
  (void)s;
  GgufJob *j = (GgufJob *)data;
  napi_value r, hs, st, err;
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, j->status));
  napi_create_string_utf8(env, j->error, NAPI_AUTO_LENGTH, &err);
  set(env, r, "error", err);
  napi_create_array_with_length(env, j->count, &hs);
  napi_create_array_with_length(env, j->count, &st);
  for (size_t i = 0; i < j->count; i++) {
    napi_set_element(env, hs, (uint32_t)i, make_bigint(env, j->handles[i]));
    napi_set_element(env, st, (uint32_t)i, make_i32(env, j->statuses[i]));
  }
  set(env, r, "handles", hs);
  set(env, r, "statuses", st);
  j->box->busy--;
  if (j->box->close_requested && j->box->busy == 0 && j->box->g) {
    hp_gguf_close(j->box->g);
    j->box->g = NULL;
  }
  napi_delete_reference(env, j->file_ref);
  napi_resolve_deferred(env, j->deferred, r);
  napi_delete_async_work(env, j->work);
  free(j->indices);
  free(j->handles);
  free(j->statuses);
  free(j);
}

static napi_value js_gguf_upload(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value argv[2], promise, name;
  uint32_t n = 0;
  bool is_arr = false;
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  GgufBox *b = argc > 0 ? get_box(env, argv[0]) : NULL;
  if (!b || !b->g || b->close_requested || argc < 2 || napi_is_array(env, argv[1], &is_arr) != napi_ok || !is_arr ||
      napi_get_array_length(env, argv[1], &n) != napi_ok) {
    napi_throw_type_error(env, NULL, "ggufUpload(file, tensorIndices[]) on an open GGUF file");
    return NULL;
  }
  GgufJob *j = (GgufJob *)calloc(1, sizeof(GgufJob));
  if (!j) return NULL;
  j->box = b;
  j->count = n;
  j->indices = (uint64_t *)calloc(n ? n : 1, sizeof(uint64_t));
  j->handles = (uint64_t *)calloc(n ? n : 1, sizeof(uint64_t));
  j->statuses = (int32_t *)calloc(n ? n : 1, sizeof(int32_t));
  if (!j->indices || !j->handles || !j->statuses) {
    free(j->indices);
    free(j->handles);
    free(j->statuses);
    free(j);
    napi_throw_error(env, NULL, "out of host memory");
    return NULL;
  }
  for (uint32_t i = 0; i < n; i++) {
    napi_value v;
    size_t idx;
    napi_get_element(env, argv[1], i, &v);
    if (!get_size(env, v, &idx)) {
      free(j->indices);
      free(j->handles);
      free(j->statuses);
      free(j);
      napi_throw_type_error(env, NULL, "ggufUpload: tensor indices must be non-negative integers");
      return NULL;
    }
    j->indices[i] = idx;
  }
  b->busy++;
  napi_create_reference(env, argv[0], 1, &j->file_ref);  /* the file stays open while the worker reads */
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_string_utf8(env, "hp_hip_weight_upload_gguf", NAPI_AUTO_LENGTH, &name);
  napi_create_async_work(env, NULL, name, gguf_execute, gguf_complete, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

static napi_value js_gguf_close(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  GgufBox *b = argc > 0 ? get_box(env, argv[0]) : NULL;
  if (!b) {
    napi_throw_type_error(env, NULL, "ggufClose(file)");
    return NULL;
  }
  if (b->busy > 0) {
    b->close_requested = 1; /* closed when the last upload completes */
  } else if (b->g) {
    hp_gguf_close(b->g);
    b->g = NULL;
  }
  return make_i32(env, 0);
}

/* ---- device-resident decode (the segment runner) ------------------------
 * Buffers cross into JS as BigInt device addresses of hp_hip_device_alloc. */

static napi_value js_device_alloc(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  size_t bytes;
  if (argc < 1 || !get_size(env, argv[0], &bytes)) {
    napi_throw_type_error(env, NULL, "deviceAlloc(bytes)");
    return NULL;
  }
  void *d = NULL;
  const int32_t rc = hp_hip_device_alloc(bytes, &d);
  napi_value r, ptr;
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, rc));
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)d, &ptr);
  set(env, r, "ptr", ptr);
  return r;
}

static napi_value js_device_free(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  uint64_t p;
  if (argc < 1 || !get_u64(env, argv[0], &p)) {
    napi_throw_type_error(env, NULL, "deviceFree(ptr)");
    return NULL;
  }
  return make_i32(env, hp_hip_device_free((void *)(uintptr_t)p));
}

/* any typed array: its bytes */
static int get_bytes(napi_env env, napi_value v, void **data, size_t *bytes) {
  bool is = false;
  if (napi_is_typedarray(env, v, &is) != napi_ok || !is) return 0;
  napi_typedarray_type t;
  napi_value ab;
  size_t off, len;
  if (napi_get_typedarray_info(env, v, &t, &len, data, &ab, &off) != napi_ok) return 0;
  static const size_t elem[] = {1, 1, 1, 2, 2, 4, 4, 4, 8, 8, 8};
  if ((size_t)t >= sizeof elem / sizeof elem[0]) return 0;
  *bytes = len * elem[t];
  return 1;
}

/* copyToDevice(ptr, typedArray, byteOffset = 0) / copyToHost(ptr, typedArray, byteOffset = 0) */
static napi_value device_copy(napi_env env, napi_callback_info info, int to_device) {
  size_t argc = 3;
  napi_value argv[3];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  uint64_t p;
  void *data;
  size_t bytes, off = 0;
  if (argc < 2 || !get_u64(env, argv[0], &p) || !get_bytes(env, argv[1], &data, &bytes) ||
      (argc > 2 && !get_size(env, argv[2], &off))) {
    napi_throw_type_error(env, NULL, to_device ? "copyToDevice(ptr, typedArray, byteOffset)"
                                               : "copyToHost(ptr, typedArray, byteOffset)");
    return NULL;
  }
  void *d = (void *)(uintptr_t)(p + off);
  return make_i32(env, to_device ? hp_hip_copy_to_device(d, data, bytes, NULL) : hp_hip_copy_to_host(data, d, bytes, NULL));
}

static napi_value js_copy_to_device(napi_env env, napi_callback_info info) { return device_copy(env, info, 1); }
static napi_value js_copy_to_host(napi_env env, napi_callback_info info) { return device_copy(env, info, 0); }

static int get_prop(napi_env env, napi_value obj, const char *name, napi_value *out) {
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return 0;
  return napi_get_named_property(env, obj, name, out) == napi_ok;
}

static int get_prop_u64(napi_env env, napi_value obj, const char *name, uint64_t *out) {
  napi_value v;
  if (!get_prop(env, obj, name, &v)) return 0;
  return get_u64(env, v, out);
}

static int get_prop_ptr(napi_env env, napi_value obj, const char *name, void **out) {
  uint64_t u = 0;
  if (!get_prop_u64(env, obj, name, &u)) return 0;
  *out = (void *)(uintptr_t)u;
  return 1;
}

/* one layer object of runLayers -> hp_hip_decode_layer_t */
static int get_layer(napi_env env, napi_value o, hp_hip_decode_layer_t *L) {
  memset(L, 0, sizeof *L);
  napi_value a;
  double d;
  void *p;
  if (!get_prop_u64(env, o, "attnQ", &L->attn_q) || !get_prop_u64(env, o, "attnK", &L->attn_k) ||
      !get_prop_u64(env, o, "attnV", &L->attn_v) || !get_prop_u64(env, o, "attnOutput", &L->attn_output) ||
      !get_prop_u64(env, o, "ffnGate", &L->ffn_gate) || !get_prop_u64(env, o, "ffnUp", &L->ffn_up) ||
      !get_prop_u64(env, o, "ffnDown", &L->ffn_down))
    return 0;
  if (!get_prop_ptr(env, o, "attnNorm", &p)) return 0;
  L->d_attn_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "attnQNorm", &p)) return 0;
  L->d_attn_q_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "attnKNorm", &p)) return 0;
  L->d_attn_k_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "postAttentionNorm", &p)) return 0;
  L->d_post_attention_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "ffnNorm", &p)) return 0;
  L->d_ffn_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "postFfwNorm", &p)) return 0;
  L->d_post_ffw_norm = (const float *)p;
  if (!get_prop_ptr(env, o, "keyCache", &p)) return 0;
  L->d_key_cache = (uint16_t *)p;
  if (!get_prop_ptr(env, o, "valueCache", &p)) return 0;
  L->d_value_cache = (uint16_t *)p;
  if (!get_prop_f64(env, o, "layerOutputScale", &d)) return 0;
  L->layer_output_scale = (float)d;
  if (!get_prop(env, o, "attention", &a)) return 0;
  hp_hip_attention_config_t *c = &L->attention;
  if (!get_prop_f64(env, a, "headCount", &d)) return 0;
  c->head_count = (int32_t)d;
  if (!get_prop_f64(env, a, "headCountKv", &d)) return 0;
  c->head_count_kv = (int32_t)d;
  if (!get_prop_f64(env, a, "headDim", &d)) return 0;
  c->head_dim = (int32_t)d;
  if (!get_prop_f64(env, a, "ropeDims", &d)) return 0;
  c->rope_dims = (int32_t)d;
  if (!get_prop_f64(env, a, "ropeFreqBase", &c->rope_freq_base)) return 0;
  if (!get_prop_ptr(env, a, "ropeFreqFactors", &p)) return 0;
  c->d_rope_freq_factors = (const float *)p;
  if (!get_prop_f64(env, a, "capacity", &d)) return 0;
  c->capacity = (int32_t)d;
  if (!get_prop_f64(env, a, "slidingWindow", &d)) return 0;
  c->sliding_window = (int32_t)d;
  if (!get_prop_f64(env, a, "epsilon", &c->epsilon)) return 0;
  /* the per-layer input step (absent: none) */
  get_prop_u64(env, o, "inpGate", &L->inp_gate);
  get_prop_u64(env, o, "proj", &L->proj);
  if (get_prop_ptr(env, o, "postNorm", &p)) L->d_post_norm = (const float *)p;
  if (get_prop_ptr(env, o, "perLayerInput", &p)) L->d_per_layer_input = (const float *)p;
  return 1;
}

enum { DJOB_LAYERS, DJOB_HEAD };

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref input_ref, rng_ref;
  int kind;
  /* layers */
  hp_hip_decode_layer_t *layers;
  size_t n_layers, tokens, hidden_n;
  void *d_hidden, *d_position, *d_output_norm, *d_output, *d_read;
  const float *input; /* NULL: the rows are already in d_hidden */
  size_t input_len;
  int32_t position;
  size_t row_start, row_count;
  float *out;
  /* head */
  uint64_t handle;
  size_t input_size, columns, k;
  double softcap;
  int sample;
  hp_hip_sampling_t sampling;
  uint32_t rng, *rng_out;
  uint32_t *ids;
  float *values;
  double *probs;
  int32_t *tokens_out, *kept;
  int32_t status;
  char error[512];
} DevJob;

static void free_devjob(DevJob *j) {
  free(j->layers);
  free(j->out);
  free(j->ids);
  free(j->values);
  free(j->probs);
  free(j->tokens_out);
  free(j->kept);
  free(j);
}

static void devjob_execute(napi_env env, void *data) {
  (void)env;
  DevJob *j = (DevJob *)data;
  int32_t rc = HP_OK;
  if (j->kind == DJOB_LAYERS) {
    if (j->input) rc = hp_hip_copy_to_device(j->d_hidden, j->input, j->input_len * sizeof(float), NULL);
    if (rc == HP_OK) rc = hp_hip_copy_to_device(j->d_position, &j->position, sizeof(int32_t), NULL);
    if (rc == HP_OK)
      rc = hp_hip_decode_layers_device(j->layers, j->n_layers, j->tokens, (float *)j->d_hidden,
                                       (const int32_t *)j->d_position, (const float *)j->d_output_norm,
                                       (float *)j->d_output, NULL);
    if (rc == HP_OK && j->row_count)
      rc = hp_hip_copy_to_host(j->out, (const char *)j->d_read + j->row_start * j->hidden_n * sizeof(float),
                               j->row_count * j->hidden_n * sizeof(float), NULL);
  } else {
    rc = hp_hip_matmul_topk_sample_device(j->handle, (const float *)j->d_hidden, j->input_size * j->columns,
                                          j->input_size, j->columns, j->k, j->softcap,
                                          j->sample ? &j->sampling : NULL, j->sample ? &j->rng : NULL,
                                          j->tokens_out, j->ids, j->values, j->probs, j->kept, j->columns * j->k);
  }
  j->status = rc;
  if (rc != HP_OK) {
    strncpy(j->error, hp_hip_last_error(), sizeof j->error - 1);
    j->error[sizeof j->error - 1] = 0;
  }
}

static void devjob_complete(napi_env env, napi_status s, void *data) {
  (void)s;
  DevJob *j = (DevJob *)data;
  napi_value r, err;
  napi_create_object(env, &r);
  set(env, r, "status", make_i32(env, j->status));
  napi_create_string_utf8(env, j->error, NAPI_AUTO_LENGTH, &err);
  set(env, r, "error", err);
  if (j->kind == DJOB_LAYERS) {
    set(env, r, "output", adopt(env, j->out, j->row_count * j->hidden_n, 4, napi_float32_array));
    j->out = NULL;
    if (j->input_ref) napi_delete_reference(env, j->input_ref);
  } else {
    const size_t n = j->columns * j->k;
    set(env, r, "ids", adopt(env, j->ids, n, 4, napi_uint32_array));
    set(env, r, "values", adopt(env, j->values, n, 4, napi_float32_array));
    j->ids = NULL;
    j->values = NULL;
    if (j->sample) {
      set(env, r, "probabilities", adopt(env, j->probs, n, 8, napi_float64_array));
      set(env, r, "tokens", adopt(env, j->tokens_out, j->columns, 4, napi_int32_array));
      set(env, r, "kept", adopt(env, j->kept, j->columns, 4, napi_int32_array));
      j->probs = NULL;
      j->tokens_out = NULL;
      j->kept = NULL;
      if (j->status == HP_OK && j->rng_out) *j->rng_out = j->rng;
      napi_delete_reference(env, j->rng_ref);
    }
  }
  napi_resolve_deferred(env, j->deferred, r);
  napi_delete_async_work(env, j->work);
  free_devjob(j);
}

static napi_value start_devjob(napi_env env, DevJob *j, const char *name) {
  napi_value promise, wname;
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &wname);
  napi_create_async_work(env, NULL, wname, devjob_execute, devjob_complete, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

/* runLayers(layers[], tokenCount, hiddenSize, {hidden, position, outputNorm, output}, input Float32Array | null,
 *           position, readOutput, rowStart, rowCount) -> Promise<{status, error, output}>
 * input rows -> hidden (unless null), *position, hp_hip_decode_layers_device over the layers, then rows
 * [rowStart, rowStart + rowCount) of hidden (readOutput false) or of the output norm back. */
static napi_value js_run_layers(napi_env env, napi_callback_info info) {
  size_t argc = 9;
  napi_value argv[9];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  DevJob *j = (DevJob *)calloc(1, sizeof(DevJob));
  if (!j) return NULL;
  j->kind = DJOB_LAYERS;
  uint32_t n = 0;
  bool is_array = false, read_output = false;
  double pos = 0;
  int ok = argc >= 9 && napi_is_array(env, argv[0], &is_array) == napi_ok && is_array &&
           napi_get_array_length(env, argv[0], &n) == napi_ok && n > 0 && get_size(env, argv[1], &j->tokens) &&
           get_size(env, argv[2], &j->hidden_n) && get_prop_ptr(env, argv[3], "hidden", &j->d_hidden) &&
           get_prop_ptr(env, argv[3], "position", &j->d_position) &&
           napi_get_value_double(env, argv[5], &pos) == napi_ok &&
           napi_get_value_bool(env, argv[6], &read_output) == napi_ok && get_size(env, argv[7], &j->row_start) &&
           get_size(env, argv[8], &j->row_count);
  if (ok) {
    get_prop_ptr(env, argv[3], "outputNorm", &j->d_output_norm);
    get_prop_ptr(env, argv[3], "output", &j->d_output);
    j->layers = (hp_hip_decode_layer_t *)calloc(n, sizeof(hp_hip_decode_layer_t));
    ok = j->layers != NULL;
    for (uint32_t i = 0; ok && i < n; i++) {
      napi_value o;
      ok = napi_get_element(env, argv[0], i, &o) == napi_ok && get_layer(env, o, &j->layers[i]);
    }
    j->n_layers = n;
  }
  if (ok) {
    napi_valuetype t;
    napi_typeof(env, argv[4], &t);
    if (t != napi_null && t != napi_undefined) {
      void *in;
      ok = get_typed(env, argv[4], napi_float32_array, &in, &j->input_len) &&
           j->input_len == j->tokens * j->hidden_n;
      j->input = (const float *)in;
    }
  }
  if (ok) ok = j->row_start + j->row_count <= j->tokens && (!read_output || j->d_output);
  if (!ok) {
    free_devjob(j);
    napi_throw_type_error(env, NULL,
                          "runLayers(layers[], tokenCount, hiddenSize, {hidden, position, outputNorm, output}, "
                          "Float32Array | null, position, readOutput, rowStart, rowCount)");
    return NULL;
  }
  j->position = (int32_t)pos;
  j->d_read = read_output ? j->d_output : j->d_hidden;
  j->out = (float *)malloc(j->row_count * j->hidden_n * sizeof(float) + 4);
  if (!j->out) {
    free_devjob(j);
    napi_throw_error(env, NULL, "runLayers: out of host memory");
    return NULL;
  }
  if (j->input) napi_create_reference(env, argv[4], 1, &j->input_ref);
  return start_devjob(env, j, "hp_hip_decode_layers_device");
}

/* headTopK(handle, dInputPtr, inputSize, columnCount, k, softcap, sampling | null, Uint32Array rngState | null)
 *   -> Promise<{status, error, ids, values[, tokens, probabilities, kept]}> */
static napi_value js_head_topk(napi_env env, napi_callback_info info) {
  size_t argc = 8;
  napi_value argv[8];
  CHECK(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
  DevJob *j = (DevJob *)calloc(1, sizeof(DevJob));
  if (!j) return NULL;
  j->kind = DJOB_HEAD;
  uint64_t din = 0;
  int ok = argc >= 8 && get_u64(env, argv[0], &j->handle) && get_u64(env, argv[1], &din) &&
           get_size(env, argv[2], &j->input_size) && get_size(env, argv[3], &j->columns) &&
           get_size(env, argv[4], &j->k) && napi_get_value_double(env, argv[5], &j->softcap) == napi_ok;
  j->d_hidden = (void *)(uintptr_t)din;
  napi_valuetype t = napi_null;
  if (ok) napi_typeof(env, argv[6], &t);
  if (ok && t != napi_null && t != napi_undefined) {
    double do_sample = 1, top_k = 0, temperature = 0, top_p = 0;
    void *rng;
    size_t rng_len = 0;
    ok = get_prop_f64(env, argv[6], "topK", &top_k) && get_prop_f64(env, argv[6], "temperature", &temperature) &&
         get_prop_f64(env, argv[6], "topP", &top_p) &&
         get_typed(env, argv[7], napi_uint32_array, &rng, &rng_len) && rng_len >= 1;
    if (ok) {
      get_prop_f64(env, argv[6], "doSample", &do_sample);
      j->sample = 1;
      j->sampling.do_sample = do_sample != 0;
      j->sampling.top_k = top_k >= 2147483647.0 ? 2147483647 : (int32_t)top_k;
      j->sampling.temperature = temperature;
      j->sampling.top_p = top_p;
      j->rng_out = (uint32_t *)rng;
      j->rng = j->rng_out[0];
    }
  }
  if (!ok) {
    free_devjob(j);
    napi_throw_type_error(env, NULL,
                          "headTopK(handle, dInput, inputSize, columnCount, k, softcap, sampling | null, "
                          "Uint32Array | null)");
    return NULL;
  }
  const size_t n = (j->columns * j->k) != 0 ? j->columns * j->k : 1, c = j->columns ? j->columns : 1;
  j->ids = (uint32_t *)malloc(n * 4);
  j->values = (float *)malloc(n * 4);
  if (j->sample) {
    j->probs = (double *)malloc(n * 8);
    j->tokens_out = (int32_t *)malloc(c * 4);
    j->kept = (int32_t *)malloc(c * 4);
  }
  if (!j->ids || !j->values || (j->sample && (!j->probs || !j->tokens_out || !j->kept))) {
    free_devjob(j);
    napi_throw_error(env, NULL, "headTopK: out of host memory");
    return NULL;
  }
  if (j->sample) napi_create_reference(env, argv[7], 1, &j->rng_ref);
  return start_devjob(env, j, "hp_hip_matmul_topk_sample_device");
}

static napi_value init_module(napi_env env, napi_value exports) {
  napi_property_descriptor d[] = {
      {"statusString", NULL, js_status_string, NULL, NULL, NULL, napi_enumerable, NULL},
      {"lastError", NULL, js_last_error, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, napi_enumerable, NULL},
      {"init", NULL, js_init, NULL, NULL, NULL, napi_enumerable, NULL},
      {"upload", NULL, js_upload, NULL, NULL, NULL, napi_enumerable, NULL},
      {"release", NULL, js_release, NULL, NULL, NULL, napi_enumerable, NULL},
      {"info", NULL, js_info, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stats", NULL, js_stats, NULL, NULL, NULL, napi_enumerable, NULL},
      {"matmulMulti", NULL, js_matmul_multi, NULL, NULL, NULL, napi_enumerable, NULL},
      {"matmulTopK", NULL, js_matmul_topk, NULL, NULL, NULL, napi_enumerable, NULL},
      {"matmulGeglu", NULL, js_matmul_geglu, NULL, NULL, NULL, napi_enumerable, NULL},
      {"matmulTopKSample", NULL, js_matmul_topk_sample, NULL, NULL, NULL, napi_enumerable, NULL},
      {"dequantize", NULL, js_dequantize, NULL, NULL, NULL, napi_enumerable, NULL},
      {"geglu", NULL, js_geglu, NULL, NULL, NULL, napi_enumerable, NULL},
      {"ggufOpen", NULL, js_gguf_open, NULL, NULL, NULL, napi_enumerable, NULL},
      {"ggufInfo", NULL, js_gguf_info, NULL, NULL, NULL, napi_enumerable, NULL},
      {"ggufUpload", NULL, js_gguf_upload, NULL, NULL, NULL, napi_enumerable, NULL},
      {"ggufClose", NULL, js_gguf_close, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceAlloc", NULL, js_device_alloc, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceFree", NULL, js_device_free, NULL, NULL, NULL, napi_enumerable, NULL},
      {"copyToDevice", NULL, js_copy_to_device, NULL, NULL, NULL, napi_enumerable, NULL},
      {"copyToHost", NULL, js_copy_to_host, NULL, NULL, NULL, napi_enumerable, NULL},
      {"runLayers", NULL, js_run_layers, NULL, NULL, NULL, napi_enumerable, NULL},
      {"headTopK", NULL, js_head_topk, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  napi_define_properties(env, exports, sizeof d / sizeof d[0], d);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init_module)
