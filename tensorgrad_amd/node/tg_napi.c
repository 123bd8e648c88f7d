/* Node.js N-API (version 8) binding of the C ABI in include/tg.h.
 *
 * This is the native half of the drop-in for the reference's worker
 * (src/worker.ts:86-334 behind src/worker-proxy.ts:49-73): worker_shim.js keeps the
 * WorkerProxy surface (request / send / terminate with the Req kinds of
 * src/worker-protocol.ts:54-63) and calls these functions.
 *
 * Off the JS thread, as the reference's Web Worker is: every call that touches the device
 * (create, createSibling, destroy, uploadParams, downloadParams, step, run,
 * resetOptimizer, setLR, checkpoints, optimizer state) returns a Promise and runs as
 * napi_async_work on a libuv worker thread. Input arrays are copied on the JS thread when
 * the call is made (the reference transfers them, so the caller cannot change them
 * afterwards either); results come back in fresh typed arrays. Calls on one runtime
 * family must not overlap: worker_shim.js queues them one family at a time, as the
 * reference's runtime chains its dispatches (src/runtime.ts:303-313). Host-only calls
 * (plan, describe, names, safetensorsIndex) stay synchronous.
 *
 * Errors reject with JS Errors carrying tg_last_error() (read on the worker thread that
 * made the call: the message is thread-local); TG_ABORTED becomes an Error named
 * "AbortError" (the reference's abort contract, src/compile.ts:1201-1208).
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

/* Largest element count of one typed array crossing the binding (its bytes fit int32). */
#define MAX_ELEMS ((int64_t)1 << 29)

static napi_value make_error(napi_env env, tg_status st, const char* m) {
  napi_value msg, err, name, code;
  napi_create_string_utf8(env, m && *m ? m : "tensorgrad: native call failed", NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  if (st == TG_ABORTED) {
    napi_create_string_utf8(env, "AbortError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, err, "name", name);
  }
  napi_create_int32(env, (int32_t)st, &code);
  napi_set_named_property(env, err, "tgStatus", code);
  return err;
}

static napi_value throw_status(napi_env env, tg_status st) {
  napi_throw(env, make_error(env, st, tg_last_error()));
  return NULL;
}

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
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "tg_napi: expected a runtime handle");
    return NULL;
  }
  return (tg_runtime*)p;
}

/* An element count from JS: an integer in [0, MAX_ELEMS]. */
static int get_count(napi_env env, napi_value v, int64_t* out) {
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok || !(d >= 0) || d > (double)MAX_ELEMS || d != (double)(int64_t)d) {
    napi_throw_range_error(env, NULL, "tg_napi: element count must be an integer in [0, 2^29]");
    return 0;
  }
  *out = (int64_t)d;
  return 1;
}

/* Pointer and byte length of a TypedArray / DataView / ArrayBuffer argument. */
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
  napi_is_dataview(env, v, &is);
  if (is) {
    napi_value ab;
    size_t off;
    napi_get_dataview_info(env, v, len, data, &ab, &off);
    return 1;
  }
  napi_is_arraybuffer(env, v, &is);
  if (is) {
    napi_get_arraybuffer_info(env, v, data, len);
    return 1;
  }
  napi_throw_type_error(env, NULL, "tg_napi: expected a TypedArray, DataView or ArrayBuffer");
  return 0;
}

/* A {name: TypedArray} record as parallel C arrays. With `own`, the bytes are copied into
 * buffers the record owns (for work that runs after the call returns). */
typedef struct {
  int n, own;
  char** names;
  void** data;
  int64_t* nbytes;
} record_t;

static void record_free(record_t* r) {
  for (int i = 0; i < r->n; ++i) {
    free(r->names[i]);
    if (r->own) free(r->data[i]);
  }
  free(r->names);
  free(r->data);
  free(r->nbytes);
  memset(r, 0, sizeof *r);
}

static int get_record(napi_env env, napi_value obj, record_t* r, int own) {
  napi_value keys;
  uint32_t n = 0;
  memset(r, 0, sizeof *r);
  r->own = own;
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
    void* src = NULL;
    size_t len = 0;
    r->names[i] = name;
    r->n = (int)i + 1;
    if (!get_bytes(env, v, &src, &len)) { record_free(r); return 0; }
    if (own) {
      r->data[i] = malloc(len ? len : 1);
      if (len) memcpy(r->data[i], src, len);
    } else {
      r->data[i] = src;
    }
    r->nbytes[i] = (int64_t)len;
  }
  return 1;
}

static void free_cb(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  free(data);
}

/* A typed array over a malloc'ed buffer of `count` 4-byte elements (ownership passes to JS). */
static napi_value adopt_typed(napi_env env, int is_int, size_t count, void* data) {
  napi_value ab, arr;
  if (napi_create_external_arraybuffer(env, data, count * 4, free_cb, NULL, &ab) != napi_ok) {
    free(data);
    return NULL;
  }
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

/* ---- asynchronous jobs ----------------------------------------------------------------- */

enum {
  J_CREATE, J_SIBLING, J_DESTROY, J_UPLOAD, J_DOWNLOAD, J_STEP, J_RUN, J_RESET, J_SETLR, J_SAVE, J_LOAD,
  J_DL_STATE, J_UL_STATE
};

typedef struct {
  char* name;
  int64_t count;
  int is_int;
  void* out;
} capture_t;

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  int kind;
  tg_runtime* h;
  tg_runtime* created;
  char* str;                 /* IR JSON, LR JSON or checkpoint path */
  record_t in;               /* owned copies of the input arrays */
  int ncap;
  capture_t* caps;           /* captures read back after a step / run */
  int64_t count;             /* run: output elements */
  int is_int;
  void* out;
  int n;                     /* downloads: tensors */
  char** names;
  void** bufs;
  int64_t* numel;
  int64_t t, c;              /* optimizer state counters */
  float loss;
  tg_status st;
  char* err;
} job_t;

static void job_free(job_t* j) {
  record_free(&j->in);
  for (int i = 0; i < j->ncap; ++i) {
    free(j->caps[i].name);
    free(j->caps[i].out);
  }
  free(j->caps);
  for (int i = 0; i < j->n; ++i) {
    free(j->names[i]);
    if (j->bufs) free(j->bufs[i]);
  }
  free(j->names);
  free(j->bufs);
  free(j->numel);
  free(j->out);
  free(j->str);
  free(j->err);
  free(j);
}

static char* dup_str(const char* s) {
  size_t n = s ? strlen(s) : 0;
  char* d = (char*)malloc(n + 1);
  if (n) memcpy(d, s, n);
  d[n] = 0;
  return d;
}

/* Allocate `n` named download buffers of the given element counts. */
static void alloc_downloads(job_t* j, int n) {
  j->n = n > 0 ? n : 0;
  j->names = (char**)calloc(j->n ? j->n : 1, sizeof(char*));
  j->bufs = (void**)calloc(j->n ? j->n : 1, sizeof(void*));
  j->numel = (int64_t*)calloc(j->n ? j->n : 1, sizeof(int64_t));
}

static tg_status read_captures(job_t* j) {
  for (int i = 0; i < j->ncap; ++i) {
    capture_t* c = &j->caps[i];
    c->out = malloc(c->count ? (size_t)c->count * 4 : 4);
    tg_status st = tg_get_capture(j->h, c->name, c->out, c->count * 4);
    if (st != TG_OK) return st;
  }
  return TG_OK;
}

/* Runs on a libuv worker thread: C ABI calls only, no N-API. */
static void execute(napi_env env, void* data) {
  (void)env;
  job_t* j = (job_t*)data;
  tg_status st = TG_OK;
  switch (j->kind) {
    case J_CREATE: st = tg_runtime_create(j->str, &j->created); break;
    case J_SIBLING: st = tg_runtime_create_sibling(j->h, j->str, &j->created); break;
    case J_DESTROY: tg_destroy(j->h); break;
    case J_UPLOAD: {
      int64_t* numel = (int64_t*)calloc(j->in.n ? j->in.n : 1, sizeof(int64_t));
      for (int i = 0; i < j->in.n; ++i) numel[i] = j->in.nbytes[i] / 4;
      st = tg_upload_params(j->h, j->in.n, (const char* const*)j->in.names, (const float* const*)j->in.data, numel);
      free(numel);
      break;
    }
    case J_DOWNLOAD:
    case J_DL_STATE: {
      const int state = j->kind == J_DL_STATE;
      const int n = state ? tg_state_count(j->h) : tg_param_count(j->h);
      alloc_downloads(j, n);
      for (int i = 0; i < j->n; ++i) {
        const char* nm = state ? tg_state_name(j->h, i) : tg_param_name(j->h, i);
        j->names[i] = dup_str(nm);
        j->numel[i] = state ? tg_state_numel(j->h, i) : tg_param_numel(j->h, i);
        if (!nm || j->numel[i] < 0 || j->numel[i] > MAX_ELEMS) {
          st = TG_ABORTED;
          break;
        }
        j->bufs[i] = malloc(j->numel[i] ? (size_t)j->numel[i] * 4 : 4);
      }
      if (st != TG_OK) break;
      if (state)
        st = tg_download_state(j->h, j->n, (const char* const*)j->names, (float* const*)j->bufs, j->numel, &j->t, &j->c);
      else
        st = tg_download_params(j->h, j->n, (const char* const*)j->names, (float* const*)j->bufs, j->numel);
      break;
    }
    case J_STEP:
      st = tg_step(j->h, j->in.n, (const char* const*)j->in.names, (const void* const*)j->in.data, j->in.nbytes, &j->loss);
      if (st == TG_OK) st = read_captures(j);
      break;
    case J_RUN:
      j->out = malloc(j->count ? (size_t)j->count * 4 : 4);
      st = tg_run(j->h, j->in.n, (const char* const*)j->in.names, (const void* const*)j->in.data, j->in.nbytes, j->out,
                  j->count * 4);
      if (st == TG_OK) st = read_captures(j);
      break;
    case J_RESET: st = tg_reset_optimizer(j->h); break;
    case J_SETLR: st = tg_set_lr(j->h, j->str); break;
    case J_SAVE: st = tg_save_checkpoint(j->h, j->str); break;
    case J_LOAD: st = tg_load_checkpoint(j->h, j->str); break;
    case J_UL_STATE: {
      int64_t* numel = (int64_t*)calloc(j->in.n ? j->in.n : 1, sizeof(int64_t));
      for (int i = 0; i < j->in.n; ++i) numel[i] = j->in.nbytes[i] / 4;
      st = tg_upload_state(j->h, j->in.n, (const char* const*)j->in.names, (const float* const*)j->in.data, numel, j->t,
                           j->c);
      free(numel);
      break;
    }
    default: st = TG_INTERNAL;
  }
  j->st = st;
  if (st != TG_OK) {
    const char* m = tg_last_error();
    j->err = dup_str(m && *m ? m : (st == TG_ABORTED ? "graph destroyed" : "tensorgrad: native call failed"));
  }
}

static napi_value capture_record(napi_env env, job_t* j) {
  if (j->ncap == 0) {
    napi_value nul;
    napi_get_null(env, &nul);
    return nul;
  }
  napi_value obj;
  napi_create_object(env, &obj);
  for (int i = 0; i < j->ncap; ++i) {
    capture_t* c = &j->caps[i];
    napi_value arr = adopt_typed(env, c->is_int, (size_t)c->count, c->out);
    c->out = NULL;
    if (arr) napi_set_named_property(env, obj, c->name, arr);
  }
  return obj;
}

static napi_value download_record(napi_env env, job_t* j) {
  napi_value obj;
  napi_create_object(env, &obj);
  for (int i = 0; i < j->n; ++i) {
    napi_value arr = adopt_typed(env, 0, (size_t)j->numel[i], j->bufs[i]);
    j->bufs[i] = NULL;
    if (arr) napi_set_named_property(env, obj, j->names[i], arr);
  }
  return obj;
}

/* Back on the JS thread: settle the Promise, free the job. */
static void complete(napi_env env, napi_status status, void* data) {
  job_t* j = (job_t*)data;
  if (status != napi_ok) {
    napi_value e = make_error(env, TG_INTERNAL, "tg_napi: asynchronous work was cancelled");
    napi_reject_deferred(env, j->deferred, e);
  } else if (j->st != TG_OK) {
    napi_reject_deferred(env, j->deferred, make_error(env, j->st, j->err));
  } else {
    napi_value r = NULL, v;
    switch (j->kind) {
      case J_CREATE:
      case J_SIBLING:
        if (napi_create_external(env, j->created, NULL, NULL, &r) != napi_ok) r = NULL;
        break;
      case J_DOWNLOAD: r = download_record(env, j); break;
      case J_DL_STATE:
        napi_create_object(env, &r);
        napi_set_named_property(env, r, "state", download_record(env, j));
        napi_create_int64(env, j->t, &v);
        napi_set_named_property(env, r, "t", v);
        napi_create_int64(env, j->c, &v);
        napi_set_named_property(env, r, "prngCounter", v);
        break;
      case J_STEP:
        napi_create_object(env, &r);
        napi_create_double(env, (double)j->loss, &v);
        napi_set_named_property(env, r, "loss", v);
        napi_set_named_property(env, r, "captures", capture_record(env, j));
        break;
      case J_RUN:
        napi_create_object(env, &r);
        v = adopt_typed(env, j->is_int, (size_t)j->count, j->out);
        j->out = NULL;
        if (v) napi_set_named_property(env, r, "output", v);
        napi_set_named_property(env, r, "captures", capture_record(env, j));
        break;
      default: r = undefined(env);
    }
    if (r) napi_resolve_deferred(env, j->deferred, r);
    else napi_reject_deferred(env, j->deferred, make_error(env, TG_INTERNAL, "tg_napi: building the result failed"));
  }
  napi_delete_async_work(env, j->work);
  job_free(j);
}

static job_t* new_job(int kind) {
  job_t* j = (job_t*)calloc(1, sizeof(job_t));
  j->kind = kind;
  return j;
}

static napi_value start(napi_env env, job_t* j, const char* what) {
  napi_value promise, name;
  if (napi_create_promise(env, &j->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, what, NAPI_AUTO_LENGTH, &name) != napi_ok ||
      napi_create_async_work(env, NULL, name, execute, complete, j, &j->work) != napi_ok ||
      napi_queue_async_work(env, j->work) != napi_ok) {
    job_free(j);
    napi_throw_error(env, NULL, "tg_napi: could not queue asynchronous work");
    return NULL;
  }
  return promise;
}

/* [[name, count, isInt], ...] -> capture list of a job (null / undefined: none). */
static int get_captures(napi_env env, napi_value v, job_t* j) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined || t == napi_null) return 1;
  uint32_t n = 0;
  if (napi_get_array_length(env, v, &n) != napi_ok) {
    napi_throw_type_error(env, NULL, "tg_napi: captures must be an array of [name, count, isInt]");
    return 0;
  }
  j->caps = (capture_t*)calloc(n ? n : 1, sizeof(capture_t));
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e, x;
    bool b = false;
    napi_get_element(env, v, i, &e);
    napi_get_element(env, e, 0, &x);
    char* name = get_string(env, x);
    if (!name) return 0;
    j->caps[i].name = name;
    j->ncap = (int)i + 1;
    napi_get_element(env, e, 1, &x);
    if (!get_count(env, x, &j->caps[i].count)) return 0;
    napi_get_element(env, e, 2, &x);
    napi_get_value_bool(env, x, &b);
    j->caps[i].is_int = b;
  }
  return 1;
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

/* create(irJson) -> Promise<handle> */
static napi_value js_create(napi_env env, napi_callback_info info) {
  ARGS(1);
  char* ir = get_string(env, argv[0]);
  if (!ir) return NULL;
  job_t* j = new_job(J_CREATE);
  j->str = ir;
  return start(env, j, "tg_create");
}

/* createSibling(parent, irJson) -> Promise<handle> */
static napi_value js_create_sibling(napi_env env, napi_callback_info info) {
  ARGS(2);
  tg_runtime* p = get_handle(env, argv[0]);
  if (!p) return NULL;
  char* ir = get_string(env, argv[1]);
  if (!ir) return NULL;
  job_t* j = new_job(J_SIBLING);
  j->h = p;
  j->str = ir;
  return start(env, j, "tg_create_sibling");
}

/* A job on one handle with no further arguments. */
static napi_value handle_job(napi_env env, napi_callback_info info, int kind, const char* what) {
  ARGS(1);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = new_job(kind);
  j->h = h;
  return start(env, j, what);
}

static napi_value js_destroy(napi_env env, napi_callback_info info) { return handle_job(env, info, J_DESTROY, "tg_destroy"); }
static napi_value js_download_params(napi_env env, napi_callback_info info) {
  return handle_job(env, info, J_DOWNLOAD, "tg_download_params");
}
static napi_value js_reset_optimizer(napi_env env, napi_callback_info info) {
  return handle_job(env, info, J_RESET, "tg_reset_optimizer");
}
/* downloadState(h) -> Promise<{state: {name: Float32Array}, t, prngCounter}> */
static napi_value js_download_state(napi_env env, napi_callback_info info) {
  return handle_job(env, info, J_DL_STATE, "tg_download_state");
}

/* A job on one handle with one string argument. */
static napi_value string_job(napi_env env, napi_callback_info info, int kind, const char* what) {
  ARGS(2);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  char* s = get_string(env, argv[1]);
  if (!s) return NULL;
  job_t* j = new_job(kind);
  j->h = h;
  j->str = s;
  return start(env, j, what);
}

static napi_value js_set_lr(napi_env env, napi_callback_info info) { return string_job(env, info, J_SETLR, "tg_set_lr"); }
static napi_value js_save_checkpoint(napi_env env, napi_callback_info info) {
  return string_job(env, info, J_SAVE, "tg_save_checkpoint");
}
static napi_value js_load_checkpoint(napi_env env, napi_callback_info info) {
  return string_job(env, info, J_LOAD, "tg_load_checkpoint");
}

/* uploadParams(h, {name: Float32Array}) -> Promise<undefined> */
static napi_value js_upload_params(napi_env env, napi_callback_info info) {
  ARGS(2);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = new_job(J_UPLOAD);
  j->h = h;
  if (!get_record(env, argv[1], &j->in, 1)) { job_free(j); return NULL; }
  return start(env, j, "tg_upload_params");
}

/* step(h, inputs, captures) -> Promise<{loss, captures}>; captures: [[name, count, isInt]] */
static napi_value js_step(napi_env env, napi_callback_info info) {
  ARGS(3);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = new_job(J_STEP);
  j->h = h;
  if (!get_record(env, argv[1], &j->in, 1) || !get_captures(env, argv[2], j)) { job_free(j); return NULL; }
  return start(env, j, "tg_step");
}

/* run(h, inputs, outCount, outIsInt, captures) -> Promise<{output, captures}> */
static napi_value js_run(napi_env env, napi_callback_info info) {
  ARGS(5);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = new_job(J_RUN);
  j->h = h;
  bool is_int = false;
  if (!get_count(env, argv[2], &j->count)) { job_free(j); return NULL; }
  napi_get_value_bool(env, argv[3], &is_int);
  j->is_int = is_int;
  if (!get_record(env, argv[1], &j->in, 1) || !get_captures(env, argv[4], j)) { job_free(j); return NULL; }
  return start(env, j, "tg_run");
}

/* uploadState(h, {name: Float32Array}, t, prngCounter) -> Promise<undefined> */
static napi_value js_upload_state(napi_env env, napi_callback_info info) {
  ARGS(4);
  tg_runtime* h = get_handle(env, argv[0]);
  if (!h) return NULL;
  job_t* j = new_job(J_UL_STATE);
  j->h = h;
  napi_get_value_int64(env, argv[2], &j->t);
  napi_get_value_int64(env, argv[3], &j->c);
  if (!get_record(env, argv[1], &j->in, 1)) { job_free(j); return NULL; }
  return start(env, j, "tg_upload_state");
}

/* Names of a live handle (the library answers 0 / NULL for a destroyed one). */
static napi_value string_list(napi_env env, int n, const char* (*get)(tg_runtime*, int), tg_runtime* h) {
  napi_value arr;
  napi_create_array_with_length(env, (size_t)(n > 0 ? n : 0), &arr);
  for (int i = 0; i < n; ++i) {
    napi_value s;
    const char* nm = get(h, i);
    napi_create_string_utf8(env, nm ? nm : "", NAPI_AUTO_LENGTH, &s);
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

#define FN(name, fn) {name, NULL, fn, NULL, NULL, NULL, (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), NULL}

static napi_value init(napi_env env, napi_value exports) {
  napi_property_descriptor props[] = {
      FN("deviceCount", js_device_count),     FN("plan", js_plan),
      FN("safetensorsIndex", js_safetensors_index), FN("create", js_create),
      FN("createSibling", js_create_sibling), FN("destroy", js_destroy),
      FN("paramNames", js_param_names),       FN("captureNames", js_capture_names),
      FN("stateNames", js_state_names),       FN("uploadParams", js_upload_params),
      FN("downloadParams", js_download_params), FN("step", js_step),
      FN("run", js_run),                      FN("resetOptimizer", js_reset_optimizer),
      FN("setLR", js_set_lr),                 FN("describe", js_describe),
      FN("saveCheckpoint", js_save_checkpoint), FN("loadCheckpoint", js_load_checkpoint),
      FN("downloadState", js_download_state), FN("uploadState", js_upload_state),
  };
  CHECK_NAPI(env, napi_define_properties(env, exports, sizeof props / sizeof props[0], props));
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
