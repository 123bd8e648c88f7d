/* Node.js N-API (version 8) binding of the C ABI in include/tg.h.
 *
 * This is the native half of the drop-in for the reference's worker
 * (src/worker.ts:86-334 behind src/worker-proxy.ts:49-73): worker_shim.js keeps the
 * WorkerProxy surface (request / send / terminate with the Req kinds of
 * src/worker-protocol.ts:54-63) and calls these functions. Typed arrays cross as
 * pointers into their backing stores; results come back in fresh typed arrays.
 * Errors are thrown as JS Errors carrying tg_last_error(); TG_ABORTED becomes an Error
 * named "AbortError" (the reference's abort contract, src/compile.ts:1201-1208).
 *
 * Built by __graft_entry__.build() with gcc against /usr/include/node, linked to
 * ../libtg.so (rpath $ORIGIN/..).
 */
#define NAPI_VERSION 8
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/tg.h"

#define CHECK_NAPI(env, call)                                          \
  do {                                                                 \
    if ((call) != napi_ok) {                                           \
      napi_throw_error((env), NULL, "tg_napi: N-API call failed: " #call); \
      return NULL;                                                     \
    }                                                                  \
  } while (0)

static napi_value throw_status(napi_env env, tg_status st) {
  napi_value msg, err, name, code;
  const char* m = tg_last_error();
  napi_create_string_utf8(env, m && *m ? m : "tensorgrad: native call failed", NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  if (st == TG_ABORTED) {
    napi_create_string_utf8(env, "AbortError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, err, "name", name);
  }
  napi_create_int32(env, (int32_t)st, &code);
  napi_set_named_property(env, err, "tgStatus", code);
  napi_throw(env, err);
  return NULL;
}

#define CHECK_TG(env, call)                     \
  do {                                          \
    tg_status st_ = (call);                     \
    if (st_ != TG_OK) return throw_status(env, st_); \
  } while (0)

/* ---- argument helpers --------------------------------------------------------------- */

static char* get_string(napi_env env, napi_value v) {
  size_t n = 0;
  if (napi_get_value_string_utf8(env, v, NULL, 0, &n) != napi_ok) {
    napi_throw_type_error(env, NULL, "tg_napi: expected a string");
    return NULL;
  }
  char* s = (char*)malloc(n + 1);
  napi_get_value_string_utf8(env, v, s, n + 1, &n);
  return s;
}

static tg_runtime* get_handle(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) {
    napi_throw_type_error(env, NULL, "tg_napi: expected a runtime handle");
    return NULL;
  }
  return (tg_runtime*)p;
}

/* Pointer and byte length of a TypedArray / ArrayBuffer / DataView argument. */
static int get_bytes(napi_env env, napi_value v, void** data, size_t* len) {
  bool is;
  napi_is_typedarray(env, v, &is);
  if (is) {
    napi_typedarray_type t;
    size_t n, off;
    napi_value ab;
    void* base;
    napi_get_typedarray_info(env, v, &t, &n, &base, &ab, &off);
    size_t es = (t == napi_int8_array || t == napi_uint8_array || t == napi_uint8_clamped_array) ? 1
                : (t == napi_int16_array || t == napi_uint16_array)                           ? 2
                : (t == napi_float64_array || t == napi_bigint64_array || t == napi_biguint64_array) ? 8
                                                                                                      : 4;
    *data = base;
    *len = n * es;
    return 1;
  }
  napi_is_arraybuffer(env, v, &is);
  if (is) {
    napi_get_arraybuffer_info(env, v, data, len);
    return 1;
  }
  napi_throw_type_error(env, NULL, "tg_napi: expected a TypedArray or ArrayBuffer");
  return 0;
}

/* A {name: TypedArray} record as parallel C arrays. */
typedef struct {
  int n;
  char** names;
  void** data;
  int64_t* nbytes;
} record_t;

static void record_free(record_t* r) {
  for (int i = 0; i < r->n; ++i) free(r->names[i]);
  free(r->names);
  free(r->data);
  free(r->nbytes);
  memset(r, 0, sizeof *r);
}

static int get_record(napi_env env, napi_value obj, record_t* r) {
  napi_value keys;
  uint32_t n = 0;
  memset(r, 0, sizeof *r);
  if (napi_get_property_names(env, obj, &keys) != napi_ok || napi_get_array_length(env, keys, &n) != napi_ok) {
    napi_throw_type_error(env, NULL, "tg_napi: expected a record of typed arrays");
    return 0;
  }
  r->names = (char**)calloc(n ? n : 1, sizeof(char*));
  r->data = (void**)calloc(n ? n : 1, sizeof(void*));
  r->nbytes = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  for (uint32_t i = 0; i < n; ++i) {
    napi_value k, v;
    napi_get_element(env, keys, i, &k);
    napi_get_property(env, obj, k, &v);
    char* name = get_string(env, k);
    if (!name) { r->n = (int)i; record_free(r); return 0; }
    size_t len = 0;
    r->names[i] = name;
    r->n = (int)i + 1;
    if (!get_bytes(env, v, &r->data[i], &len)) { record_free(r); return 0; }
    r->nbytes[i] = (int64_t)len;
  }
  return 1;
}

static napi_value make_typed(napi_env env, int is_int, size_t count, void** data) {
  napi_value ab, arr;
  if (napi_create_arraybuffer(env, count * 4, data, &ab) != napi_ok) return NULL;
  if (napi_create_typedarray(env, is_int ? napi_int32_array : napi_float32_array, count, ab, 0, &arr) != napi_ok)
    return NULL;
  return arr;
}

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

#define ARGS(nargs)                                   \
  size_t argc = (nargs);                              \
  napi_value argv[(nargs) > 0 ? (nargs) : 1];         \
  CHECK_NAPI(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL)); \
  if (argc < (size_t)(nargs)) {                       \
    napi_throw_type_error(env, NULL, "tg_napi: missing arguments"); \
    return NULL;                                      \
  }

/* ---- exported functions ---------------------------------------------------------------- */

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  napi_value r;
  (void)info;
  napi_create_int32(env, tg_device_count(), &r);
  return r;
}

/* Host-only lowering: the launch schedule JSON for an IR document (no device). */
static napi_value js_plan(napi_env env, napi_callback_info info) {
  ARGS(1);
  char* ir = get_string(env, argv[0]);
  if (!ir) return NULL;
  size_t cap = 1u << 24;
  char* buf = (char*)malloc(cap);
  tg_status st = tg_plan(ir, buf, (int64_t)cap);
  free(ir);
  if (st != TG_OK) { free(buf); return throw_status(env, st); }
  napi_value r;
  napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &r);
  free(buf);
  return r;
}

static napi_value js_safetensors_index(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* data;
  size_t len;
  if (!get_bytes(env, argv[0], &data, &len)) return NULL;
  uint64_t hlen = 0;
  if (len >= 8)
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | ((const uint8_t*)data)[i];
  size_t cap = 4096 + 8 * (size_t)(hlen < len ? hlen : len);
  char* out = (char*)malloc(cap);
  tg_status st = tg_safetensors_index(data, (int64_t)len, out, (int64_t)cap);
  if (st != TG_OK) { free(out); return throw_status(env, st); }
  napi_value r;
  napi_create_string_utf8(env, out, NAPI_AUTO_LENGTH, &r);
  free(out);
  return r;
}

static napi_value js_create(napi_env env, napi_callback_info info) {
  ARGS(1);
  char* ir = get_string(env, argv[0]);
  if (!ir) return NULL;
  tg_runtime* h = NULL;
  tg_status st = tg_runtime_create(ir, &h);
  free(ir);
  if (st != TG_OK) return throw_status(env, st);
  napi_value r;
  CHECK_NAPI(env, napi_create_external(env, h, NULL, NULL, &r));
  return r;
}

static napi_value js_create_sibling(napi_env env, napi_callback_info info) {
  ARGS(2);
  tg_runtime* p = get_handle(env, argv[0]);
  if (!p) return NULL;
  char* ir = get_string(env, argv[1]);
  if (!ir) return NULL;
  tg_runtime* h = NULL;
  tg_status st = tg_runtime_create_sibling(p, ir, &h);
  free(ir);
  if (st != TG_OK) return throw_status(env, st);
  napi_value r;
  CHECK_NAPI(env, napi_create_external(env, h, NULL, NULL, &r));
  return r;
}

static napi_value js_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  tg_destroy(h);
  return undefined(env);
}

static napi_value string_list(napi_env env, int n, const char* (*get)(tg_runtime*, int), tg_runtime* h) {
  napi_value arr;
  napi_create_array_with_length(env, (size_t)n, &arr);
  for (int i = 0; i < n; ++i) {
    napi_value s;
    napi_create_string_utf8(env, get(h, i), NAPI_AUTO_LENGTH, &s);
    napi_set_element(env, arr, (uint32_t)i, s);
  }
  return arr;
}

static const char* param_name_(tg_runtime* h, int i) { return tg_param_name(h, i); }
static const char* capture_name_(tg_runtime* h, int i) { return tg_capture_name(h, i); }

static napi_value js_param_names(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  return string_list(env, tg_param_count(h), param_name_, h);
}

static napi_value js_capture_names(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  return string_list(env, tg_capture_count(h), capture_name_, h);
}

static napi_value js_state_names(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  return string_list(env, tg_state_count(h), tg_state_name, h);
}

static napi_value js_upload_params(napi_env env, napi_callback_info info) {
  ARGS(2);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  record_t r;
  if (!get_record(env, argv[1], &r)) return NULL;
  int64_t* numel = (int64_t*)calloc(r.n ? r.n : 1, sizeof(int64_t));
  for (int i = 0; i < r.n; ++i) numel[i] = r.nbytes[i] / 4;
  tg_status st = tg_upload_params(h, r.n, (const char* const*)r.names, (const float* const*)r.data, numel);
  free(numel);
  record_free(&r);
  CHECK_TG(env, st);
  return undefined(env);
}

static napi_value js_download_params(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  int n = tg_param_count(h);
  napi_value obj;
  napi_create_object(env, &obj);
  const char** names = (const char**)calloc(n ? n : 1, sizeof(char*));
  float** ptrs = (float**)calloc(n ? n : 1, sizeof(float*));
  int64_t* numel = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  for (int i = 0; i < n; ++i) {
    void* d;
    names[i] = tg_param_name(h, i);
    numel[i] = tg_param_numel(h, i);
    napi_value arr = make_typed(env, 0, (size_t)numel[i], &d);
    ptrs[i] = (float*)d;
    napi_set_named_property(env, obj, names[i], arr);
  }
  tg_status st = tg_download_params(h, n, names, ptrs, numel);
  free(names);
  free(ptrs);
  free(numel);
  CHECK_TG(env, st);
  return obj;
}

static napi_value js_step(napi_env env, napi_callback_info info) {
  ARGS(2);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  record_t r;
  if (!get_record(env, argv[1], &r)) return NULL;
  float loss = 0;
  tg_status st = tg_step(h, r.n, (const char* const*)r.names, (const void* const*)r.data, r.nbytes, &loss);
  record_free(&r);
  CHECK_TG(env, st);
  napi_value v;
  napi_create_double(env, (double)loss, &v);
  return v;
}

/* run(h, inputs, outCount, outIsInt) -> Float32Array | Int32Array */
static napi_value js_run(napi_env env, napi_callback_info info) {
  ARGS(4);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  int64_t count;
  bool is_int;
  napi_get_value_int64(env, argv[2], &count);
  napi_get_value_bool(env, argv[3], &is_int);
  record_t r;
  if (!get_record(env, argv[1], &r)) return NULL;
  void* out;
  napi_value arr = make_typed(env, is_int, (size_t)count, &out);
  tg_status st = tg_run(h, r.n, (const char* const*)r.names, (const void* const*)r.data, r.nbytes, out, count * 4);
  record_free(&r);
  CHECK_TG(env, st);
  return arr;
}

/* getCapture(h, name, count, isInt) -> typed array */
static napi_value js_get_capture(napi_env env, napi_callback_info info) {
  ARGS(4);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  char* name = get_string(env, argv[1]);
  if (!name) return NULL;
  int64_t count;
  bool is_int;
  napi_get_value_int64(env, argv[2], &count);
  napi_get_value_bool(env, argv[3], &is_int);
  void* out;
  napi_value arr = make_typed(env, is_int, (size_t)count, &out);
  tg_status st = tg_get_capture(h, name, out, count * 4);
  free(name);
  CHECK_TG(env, st);
  return arr;
}

static napi_value js_reset_optimizer(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  CHECK_TG(env, tg_reset_optimizer(h));
  return undefined(env);
}

static napi_value js_string_call(napi_env env, napi_callback_info info, tg_status (*f)(tg_runtime*, const char*)) {
  ARGS(2);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  char* s = get_string(env, argv[1]);
  if (!s) return NULL;
  tg_status st = f(h, s);
  free(s);
  CHECK_TG(env, st);
  return undefined(env);
}

static napi_value js_set_lr(napi_env env, napi_callback_info info) { return js_string_call(env, info, tg_set_lr); }
static napi_value js_save_checkpoint(napi_env env, napi_callback_info info) {
  return js_string_call(env, info, tg_save_checkpoint);
}
static napi_value js_load_checkpoint(napi_env env, napi_callback_info info) {
  return js_string_call(env, info, tg_load_checkpoint);
}

static napi_value js_describe(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  size_t cap = 1u << 24;
  char* buf = (char*)malloc(cap);
  tg_status st = tg_describe(h, buf, (int64_t)cap);
  if (st != TG_OK) { free(buf); return throw_status(env, st); }
  napi_value r;
  napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &r);
  free(buf);
  return r;
}

/* downloadState(h) -> {state: {name: Float32Array}, t, prngCounter} */
static napi_value js_download_state(napi_env env, napi_callback_info info) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  int n = tg_state_count(h);
  napi_value obj, state, v;
  napi_create_object(env, &obj);
  napi_create_object(env, &state);
  const char** names = (const char**)calloc(n ? n : 1, sizeof(char*));
  float** ptrs = (float**)calloc(n ? n : 1, sizeof(float*));
  int64_t* numel = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  for (int i = 0; i < n; ++i) {
    void* d;
    names[i] = tg_state_name(h, i);
    numel[i] = tg_state_numel(h, i);
    napi_value arr = make_typed(env, 0, (size_t)numel[i], &d);
    ptrs[i] = (float*)d;
    napi_set_named_property(env, state, names[i], arr);
  }
  int64_t t = 0, c = 0;
  tg_status st = tg_download_state(h, n, names, ptrs, numel, &t, &c);
  free(names);
  free(ptrs);
  free(numel);
  CHECK_TG(env, st);
  napi_set_named_property(env, obj, "state", state);
  napi_create_int64(env, t, &v);
  napi_set_named_property(env, obj, "t", v);
  napi_create_int64(env, c, &v);
  napi_set_named_property(env, obj, "prngCounter", v);
  return obj;
}

/* uploadState(h, {name: Float32Array}, t, prngCounter) */
static napi_value js_upload_state(napi_env env, napi_callback_info info) {
  ARGS(4);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  int64_t t, c;
  napi_get_value_int64(env, argv[2], &t);
  napi_get_value_int64(env, argv[3], &c);
  record_t r;
  if (!get_record(env, argv[1], &r)) return NULL;
  int64_t* numel = (int64_t*)calloc(r.n ? r.n : 1, sizeof(int64_t));
  for (int i = 0; i < r.n; ++i) numel[i] = r.nbytes[i] / 4;
  tg_status st = tg_upload_state(h, r.n, (const char* const*)r.names, (const float* const*)r.data, numel, t, c);
  free(numel);
  record_free(&r);
  CHECK_TG(env, st);
  return undefined(env);
}

static napi_value init(napi_env env, napi_value exports) {
  napi_property_descriptor props[] = {
      {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"plan", NULL, js_plan, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"safetensorsIndex", NULL, js_safetensors_index, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"create", NULL, js_create, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"createSibling", NULL, js_create_sibling, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"destroy", NULL, js_destroy, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"paramNames", NULL, js_param_names, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"captureNames", NULL, js_capture_names, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"stateNames", NULL, js_state_names, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"uploadParams", NULL, js_upload_params, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"downloadParams", NULL, js_download_params, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"step", NULL, js_step, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"run", NULL, js_run, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"getCapture", NULL, js_get_capture, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"resetOptimizer", NULL, js_reset_optimizer, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"setLR", NULL, js_set_lr, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"describe", NULL, js_describe, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"saveCheckpoint", NULL, js_save_checkpoint, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"loadCheckpoint", NULL, js_load_checkpoint, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"downloadState", NULL, js_download_state, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
      {"uploadState", NULL, js_upload_state, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL},
  };
  CHECK_NAPI(env, napi_define_properties(env, exports, sizeof props / sizeof props[0], props));
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
