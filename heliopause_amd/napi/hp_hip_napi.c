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
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

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

enum { JOB_MULTI, JOB_TOPK, JOB_GEGLU };

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
  } else {
    set(env, r, "output", adopt(env, j->outputs[0], j->output_lens[0], 4, napi_float32_array));
    j->outputs[0] = NULL;
  }
  napi_delete_reference(env, j->input_ref);
  napi_resolve_deferred(env, j->deferred, r);
  napi_delete_async_work(env, j->work);
  for (size_t i = 0; i < 4; i++) free(j->outputs[i]);
  free(j->ids);
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
      {"dequantize", NULL, js_dequantize, NULL, NULL, NULL, napi_enumerable, NULL},
      {"geglu", NULL, js_geglu, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  napi_define_properties(env, exports, sizeof d / sizeof d[0], d);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init_module)
