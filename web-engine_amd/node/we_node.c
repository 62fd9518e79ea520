/*
 * Node N-API (v8) addon over the C ABI of include/we.h: the binding a TypeScript host of the engine uses in
 * place of its WebGPU Graph (src/gpu/graph.ts) to reach the MI355X kernels.
 *
 * Conventions of the JS side:
 *   - a context and every device / pinned-host buffer are passed as BigInt addresses;
 *   - null or undefined stands for a NULL pointer;
 *   - matmul Params travel as the reference's 13 x u32 image (a Uint32Array, src/kernels/matmul.ts:120-126);
 *   - a non-zero status throws an Error whose message is we_last_error() (for shape errors the reference's
 *     own text, e.g. "K must be a multiple of 4, got 6").
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "we.h"

#define MAXARGS 20

typedef struct {
  napi_env env;
  size_t argc;
  napi_value argv[MAXARGS];
  int bad;
} args_t;

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static int get_args(napi_env env, napi_callback_info info, args_t* a, size_t need) {
  a->env = env;
  a->argc = MAXARGS;
  a->bad = 0;
  napi_get_cb_info(env, info, &a->argc, a->argv, NULL, NULL);
  if (a->argc < need) {
    napi_throw_type_error(env, NULL, "too few arguments");
    a->bad = 1;
    return 0;
  }
  return 1;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_null || t == napi_undefined;
}

static void* ptr_arg(args_t* a, size_t i) {
  if (i >= a->argc || is_nullish(a->env, a->argv[i])) return NULL;
  uint64_t v = 0;
  bool lossless = true;
  if (napi_get_value_bigint_uint64(a->env, a->argv[i], &v, &lossless) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a BigInt address");
    a->bad = 1;
  }
  return (void*)(uintptr_t)v;
}

static uint32_t u32_arg(args_t* a, size_t i) {
  uint32_t v = 0;
  if (napi_get_value_uint32(a->env, a->argv[i], &v) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a number");
    a->bad = 1;
  }
  return v;
}

static int32_t i32_arg(args_t* a, size_t i) {
  int32_t v = 0;
  if (napi_get_value_int32(a->env, a->argv[i], &v) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a number");
    a->bad = 1;
  }
  return v;
}

static int64_t i64_arg(args_t* a, size_t i) { /* undefined / null -> -1: the reference's default */
  if (i >= a->argc || is_nullish(a->env, a->argv[i])) return -1;
  int64_t v = 0;
  if (napi_get_value_int64(a->env, a->argv[i], &v) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a number");
    a->bad = 1;
  }
  return v;
}

static double f64_arg(args_t* a, size_t i) {
  double v = 0;
  if (napi_get_value_double(a->env, a->argv[i], &v) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a number");
    a->bad = 1;
  }
  return v;
}

static napi_value status(napi_env env, we_ctx* ctx, int rc) {
  if (rc != WE_OK) napi_throw_error(env, NULL, we_last_error(ctx));
  return undefined(env);
}

static napi_value big(napi_env env, const void* p) {
  napi_value v;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &v);
  return v;
}

static napi_value num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

/* ---- context ---- */
static napi_value Create(napi_env env, napi_callback_info info) {
  args_t a;
  get_args(env, info, &a, 0);
  int device = a.argc > 0 ? i32_arg(&a, 0) : 0;
  if (a.bad) return NULL;
  we_ctx* ctx = NULL;
  int rc = we_ctx_create(device, &ctx);
  if (rc != WE_OK) return status(env, NULL, rc);
  return big(env, ctx);
}

static napi_value Destroy(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_ctx_destroy(ctx));
}

static napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  char name[128] = {0};
  int cus = 0, lds = 0;
  int rc = we_device_info(ctx, name, sizeof name, &cus, &lds);
  if (rc != WE_OK) return status(env, ctx, rc);
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "arch", s);
  napi_set_named_property(env, o, "computeUnits", num(env, cus));
  napi_set_named_property(env, o, "ldsBytes", num(env, lds));
  return o;
}

static napi_value Sync(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_sync(ctx));
}

static napi_value StreamSelect(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  int which = (int)f64_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_stream_select(ctx, which));
}

static napi_value StreamFork(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_stream_fork(ctx));
}

static napi_value StreamJoin(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_stream_join(ctx));
}

/* ---- buffers ---- */
static napi_value BufAlloc(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double bytes = f64_arg(&a, 1);
  if (a.bad) return NULL;
  void* p = NULL;
  int rc = we_buf_alloc(ctx, (size_t)bytes, &p);
  if (rc != WE_OK) return status(env, ctx, rc);
  return big(env, p);
}

static napi_value BufFree(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* p = ptr_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_buf_free(ctx, p));
}

/* bytes of a TypedArray / DataView / ArrayBuffer / Buffer argument */
static int bytes_of(args_t* a, size_t i, void** data, size_t* len) {
  napi_value v = a->argv[i];
  bool is;
  if (napi_is_typedarray(a->env, v, &is) == napi_ok && is) {
    napi_typedarray_type t;
    size_t n, off;
    napi_value ab;
    napi_get_typedarray_info(a->env, v, &t, &n, data, &ab, &off);
    size_t el = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
      default: el = 1;
    }
    *len = n * el;
    return 1;
  }
  if (napi_is_arraybuffer(a->env, v, &is) == napi_ok && is) {
    napi_get_arraybuffer_info(a->env, v, data, len);
    return 1;
  }
  if (napi_is_dataview(a->env, v, &is) == napi_ok && is) {
    napi_value ab;
    size_t off;
    napi_get_dataview_info(a->env, v, len, data, &ab, &off);
    return 1;
  }
  napi_throw_type_error(a->env, NULL, "expected a TypedArray, DataView or ArrayBuffer");
  a->bad = 1;
  return 0;
}

static napi_value Upload(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 4)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* dst = ptr_arg(&a, 1);
  double off = f64_arg(&a, 2);
  void* data = NULL;
  size_t len = 0;
  bytes_of(&a, 3, &data, &len);
  if (a.bad) return NULL;
  return status(env, ctx, we_buf_upload(ctx, dst, (size_t)off, data, len));
}

static napi_value Download(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 4)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* src = ptr_arg(&a, 1);
  double off = f64_arg(&a, 2), bytes = f64_arg(&a, 3);
  if (a.bad) return NULL;
  void* data = NULL;
  napi_value ab;
  napi_create_arraybuffer(env, (size_t)bytes, &data, &ab);
  int rc = we_buf_download(ctx, src, (size_t)off, data, (size_t)bytes);
  if (rc != WE_OK) return status(env, ctx, rc);
  return ab;
}

static napi_value Copy(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 6)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* src = ptr_arg(&a, 1);
  double so = f64_arg(&a, 2);
  void* dst = ptr_arg(&a, 3);
  double doff = f64_arg(&a, 4), bytes = f64_arg(&a, 5);
  if (a.bad) return NULL;
  return status(env, ctx, we_buf_copy(ctx, src, (size_t)so, dst, (size_t)doff, (size_t)bytes));
}

static napi_value Mark(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  size_t m = 0;
  int rc = we_mark(ctx, &m);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)m);
}

static napi_value Release(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double mark = f64_arg(&a, 1);
  if (a.bad) return NULL;
  void* keep[64];
  uint32_t nkeep = 0;
  if (a.argc > 2 && !is_nullish(env, a.argv[2])) {
    napi_get_array_length(env, a.argv[2], &nkeep);
    if (nkeep > 64) {
      napi_throw_range_error(env, NULL, "at most 64 buffers can be kept");
      return NULL;
    }
    for (uint32_t i = 0; i < nkeep; i++) {
      napi_value e;
      uint64_t v = 0;
      bool lossless;
      napi_get_element(env, a.argv[2], i, &e);
      napi_get_value_bigint_uint64(env, e, &v, &lossless);
      keep[i] = (void*)(uintptr_t)v;
    }
  }
  return status(env, ctx, we_release(ctx, (size_t)mark, keep, nkeep));
}

static napi_value Stats(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  uint64_t created = 0, reused = 0, bytes = 0;
  int rc = we_stats(ctx, &created, &reused, &bytes);
  if (rc != WE_OK) return status(env, ctx, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "created", num(env, (double)created));
  napi_set_named_property(env, o, "reused", num(env, (double)reused));
  napi_set_named_property(env, o, "createdBytes", num(env, (double)bytes));
  return o;
}

/* ---- pinned host memory and streaming ---- */
/* setAllocCap(ctx, bytes) -> bytes held now; setPoison(ctx, on) */
static napi_value SetAllocCap(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double bytes = f64_arg(&a, 1);
  if (a.bad) return NULL;
  uint64_t held = 0;
  int rc = we_set_alloc_cap(ctx, (uint64_t)bytes, &held);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)held);
}

static napi_value SetPoison(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  int32_t on = i32_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_set_poison(ctx, on));
}

/* timerMark(ctx, slot); timerBetween(ctx, from, to) -> ms */
static napi_value TimerMark(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t slot = u32_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_timer_mark(ctx, slot));
}

static napi_value TimerBetween(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 3)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t from = u32_arg(&a, 1), to = u32_arg(&a, 2);
  if (a.bad) return NULL;
  float ms = 0.0f;
  int rc = we_timer_between(ctx, from, to, &ms);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)ms);
}

/* setTuning(ctx, key, value) -> previous value (WE_TUNE_* keys) */
static napi_value SetTuning(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 3)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  int32_t key = i32_arg(&a, 1);
  int32_t value = i32_arg(&a, 2);
  if (a.bad) return NULL;
  int prev = 0;
  int rc = we_set_tuning(ctx, key, value, &prev);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)prev);
}

static napi_value HostAlloc(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double bytes = f64_arg(&a, 1);
  if (a.bad) return NULL;
  void* p = NULL;
  int rc = we_host_alloc(ctx, (size_t)bytes, &p);
  if (rc != WE_OK) return status(env, ctx, rc);
  return big(env, p);
}

static napi_value HostFree(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* p = ptr_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_host_free(ctx, p));
}

/* hostWrite(ctx, pinned, offset, bytes): fill pinned host memory from JS */
static napi_value HostWrite(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 4)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* p = ptr_arg(&a, 1);
  double off = f64_arg(&a, 2);
  void* data = NULL;
  size_t len = 0;
  bytes_of(&a, 3, &data, &len);
  if (a.bad) return NULL;
  if (!p) {
    napi_throw_error(env, NULL, "pinned buffer is null");
    return NULL;
  }
  if (!(off >= 0 && off <= 9007199254740991.0 && off == (double)(uint64_t)off)) {
    napi_throw_range_error(env, NULL, "offset must be a non-negative integer");
    return NULL;
  }
  /* the whole destination must lie in one live pinned block of this context */
  int rc = we_host_span(ctx, (char*)p + (size_t)off, len);
  if (rc != WE_OK) return status(env, ctx, rc);
  memcpy((char*)p + (size_t)off, data, len);
  return undefined(env);
}

/* hostSpan(ctx, ptr, bytes): throws unless [ptr, ptr + bytes) is inside live pinned memory of ctx */
static napi_value HostSpan(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 3)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* p = ptr_arg(&a, 1);
  double bytes = f64_arg(&a, 2);
  if (a.bad) return NULL;
  return status(env, ctx, we_host_span(ctx, p, (size_t)bytes));
}

/* hostRead(ctx, ptr, bytes) -> ArrayBuffer: a copy of pinned memory of ctx (e.g. what downloadAsync wrote) */
static napi_value HostRead(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 3)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* p = ptr_arg(&a, 1);
  double bytes = f64_arg(&a, 2);
  if (a.bad) return NULL;
  if (!(bytes >= 0 && bytes <= 9007199254740991.0 && bytes == (double)(uint64_t)bytes)) {
    napi_throw_range_error(env, NULL, "bytes must be a non-negative integer");
    return NULL;
  }
  int rc = we_host_span(ctx, p, (size_t)bytes);
  if (rc != WE_OK) return status(env, ctx, rc);
  void* data = NULL;
  napi_value ab;
  if (napi_create_arraybuffer(env, (size_t)bytes, &data, &ab) != napi_ok) return NULL;
  if (bytes) memcpy(data, p, (size_t)bytes);
  return ab;
}

static napi_value StreamCopy(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* dst = ptr_arg(&a, 1);
  void* src = ptr_arg(&a, 2);
  double bytes = f64_arg(&a, 3);
  double after = f64_arg(&a, 4);
  if (a.bad) return NULL;
  uint64_t ticket = 0;
  int rc = we_stream_copy(ctx, dst, src, (size_t)bytes, (uint64_t)after, &ticket);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)ticket);
}

static napi_value WaitTicket(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double t = f64_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_wait_ticket(ctx, (uint64_t)t));
}

/* downloadAsync(ctx, buf, offset, pinnedDst, bytes) -> ticket: the copy into pinned memory is queued, not done */
static napi_value DownloadAsync(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* src = ptr_arg(&a, 1);
  double off = f64_arg(&a, 2);
  void* dst = ptr_arg(&a, 3);
  double bytes = f64_arg(&a, 4);
  if (a.bad) return NULL;
  uint64_t t = 0;
  int rc = we_buf_download_async(ctx, src, (size_t)off, dst, (size_t)bytes, &t);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)t);
}

/* waitTicketAsync(ctx, ticket) -> Promise<void>: we_ticket_wait runs on a libuv worker thread, so the event loop
 * keeps running while the GPU works (the mapAsync / onSubmittedWorkDone promises of src/gpu/graph.ts:117 and
 * src/model/weights.ts:128). */
typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  we_ctx* ctx;
  uint64_t ticket;
  int rc;
  char msg[512];
} ticket_wait_t;

static void ticket_wait_exec(napi_env env, void* data) {
  (void)env;
  ticket_wait_t* w = (ticket_wait_t*)data;
  w->rc = we_ticket_wait(w->ctx, w->ticket);
  if (w->rc != WE_OK) snprintf(w->msg, sizeof w->msg, "%s", we_last_error(NULL));
}

static void ticket_wait_done(napi_env env, napi_status st, void* data) {
  ticket_wait_t* w = (ticket_wait_t*)data;
  if (st == napi_ok && w->rc == WE_OK) {
    napi_resolve_deferred(env, w->deferred, undefined(env));
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, st == napi_ok ? w->msg : "ticket wait cancelled", NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, NULL, msg, &err);
    napi_reject_deferred(env, w->deferred, err);
  }
  napi_delete_async_work(env, w->work);
  free(w);
}

static napi_value WaitTicketAsync(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double t = f64_arg(&a, 1);
  if (a.bad) return NULL;
  if (!ctx) {
    napi_throw_error(env, NULL, "context is null");
    return NULL;
  }
  ticket_wait_t* w = (ticket_wait_t*)calloc(1, sizeof *w);
  if (!w) {
    napi_throw_error(env, NULL, "out of host memory");
    return NULL;
  }
  w->ctx = ctx;
  w->ticket = (uint64_t)t;
  napi_value promise, name;
  napi_create_promise(env, &w->deferred, &promise);
  napi_create_string_utf8(env, "we.waitTicketAsync", NAPI_AUTO_LENGTH, &name);
  if (napi_create_async_work(env, NULL, name, ticket_wait_exec, ticket_wait_done, w, &w->work) != napi_ok) {
    free(w);
    napi_throw_error(env, NULL, "could not create the ticket wait");
    return NULL;
  }
  if (napi_queue_async_work(env, w->work) != napi_ok) {
    napi_delete_async_work(env, w->work);
    free(w);
    napi_throw_error(env, NULL, "could not queue the ticket wait");
    return NULL;
  }
  return promise;
}

/* recordAll(ctx) -> [t0, t1, tCopy]: tickets for the work queued so far on both compute streams and the copy stream */
static napi_value RecordAll(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  uint64_t t[3] = {0, 0, 0};
  int rc = we_record_all(ctx, t);
  if (rc != WE_OK) return status(env, ctx, rc);
  napi_value arr;
  napi_create_array_with_length(env, 3, &arr);
  for (uint32_t i = 0; i < 3; i++) napi_set_element(env, arr, i, num(env, (double)t[i]));
  return arr;
}

static napi_value RecordCompute(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  uint64_t t = 0;
  int rc = we_record_compute(ctx, &t);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, (double)t);
}

/* ---- matmul ---- */
static napi_value MatmulParams(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t m = u32_arg(&a, 1), n = u32_arg(&a, 2), k = u32_arg(&a, 3);
  double scale = f64_arg(&a, 4);
  int64_t xs = i64_arg(&a, 5), ws = i64_arg(&a, 6), ys = i64_arg(&a, 7), xo = i64_arg(&a, 8), wo = i64_arg(&a, 9),
          yo = i64_arg(&a, 10), ks = i64_arg(&a, 11);
  if (a.bad) return NULL;
  we_matmul_params p;
  int rc = we_matmul_params_make(ctx, m, n, k, (float)scale, xs, ws, ys, xo, wo, yo, ks, &p);
  if (rc != WE_OK) return status(env, ctx, rc);
  void* data;
  napi_value ab, arr;
  napi_create_arraybuffer(env, sizeof p, &data, &ab);
  memcpy(data, &p, sizeof p);
  napi_create_typedarray(env, napi_uint32_array, sizeof p / 4, ab, 0, &arr);
  return arr;
}

/* conv3x3Params(ctx, height, width, cin, cout) -> the 13 x u32 Params image (src/kernels/matmul.ts:268-272) */
static napi_value Conv3x3Params(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t h = u32_arg(&a, 1), w = u32_arg(&a, 2), cin = u32_arg(&a, 3), cout = u32_arg(&a, 4);
  if (a.bad) return NULL;
  we_matmul_params p;
  int rc = we_conv3x3_params(ctx, h, w, cin, cout, &p);
  if (rc != WE_OK) return status(env, ctx, rc);
  void* data;
  napi_value ab, arr;
  napi_create_arraybuffer(env, sizeof p, &data, &ab);
  memcpy(data, &p, sizeof p);
  napi_create_typedarray(env, napi_uint32_array, sizeof p / 4, ab, 0, &arr);
  return arr;
}

static napi_value KSplitFor(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 3)) return NULL;
  uint32_t m = u32_arg(&a, 0), n = u32_arg(&a, 1), k = u32_arg(&a, 2);
  if (a.bad) return NULL;
  return num(env, we_ksplit_for(m, n, k));
}

/* matmul(ctx, params, xDtype, x, wDtype, w, scales, group, yDtype, y, bias, flags) */
static napi_value matmul_call(napi_env env, napi_callback_info info, int noalloc) {
  args_t a;
  if (!get_args(env, info, &a, 12)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* pdata = NULL;
  size_t plen = 0;
  bytes_of(&a, 1, &pdata, &plen);
  int32_t xdt = i32_arg(&a, 2);
  void* x = ptr_arg(&a, 3);
  int32_t wdt = i32_arg(&a, 4);
  void* w = ptr_arg(&a, 5);
  void* scales = ptr_arg(&a, 6);
  uint32_t group = u32_arg(&a, 7);
  int32_t ydt = i32_arg(&a, 8);
  void* y = ptr_arg(&a, 9);
  void* bias = ptr_arg(&a, 10);
  uint32_t flags = u32_arg(&a, 11);
  if (a.bad) return NULL;
  if (plen != sizeof(we_matmul_params)) {
    napi_throw_type_error(env, NULL, "params must be the 13 x u32 image from matmulParams");
    return NULL;
  }
  const we_matmul_params* p = (const we_matmul_params*)pdata;
  return status(env, ctx, noalloc ? we_matmul_noalloc(ctx, p, xdt, x, wdt, w, scales, group, ydt, y, (const float*)bias, flags)
                                  : we_matmul(ctx, p, xdt, x, wdt, w, scales, group, ydt, y, (const float*)bias, flags));
}

static napi_value Matmul(napi_env env, napi_callback_info info) { return matmul_call(env, info, 0); }

/* matmulNoalloc(...): the arguments of matmul; allocates nothing (split-K scratch in a fixed per-GPU array) */
static napi_value MatmulNoalloc(napi_env env, napi_callback_info info) { return matmul_call(env, info, 1); }

/* matmulGated(ctx, params, xDtype, x, wDtype, w, scales, group, yDtype, y, bias, flags, gate, residual):
 * y = residual + gate * v, the reference's gatedAdd after the GEMM fused into its epilogue */
static napi_value MatmulGated(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 14)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* pdata = NULL;
  size_t plen = 0;
  bytes_of(&a, 1, &pdata, &plen);
  int32_t xdt = i32_arg(&a, 2);
  void* x = ptr_arg(&a, 3);
  int32_t wdt = i32_arg(&a, 4);
  void* w = ptr_arg(&a, 5);
  void* scales = ptr_arg(&a, 6);
  uint32_t group = u32_arg(&a, 7);
  int32_t ydt = i32_arg(&a, 8);
  void* y = ptr_arg(&a, 9);
  void* bias = ptr_arg(&a, 10);
  uint32_t flags = u32_arg(&a, 11);
  void* gate = ptr_arg(&a, 12);
  void* res = ptr_arg(&a, 13);
  if (a.bad) return NULL;
  if (plen != sizeof(we_matmul_params)) {
    napi_throw_type_error(env, NULL, "params must be the 13 x u32 image from matmulParams");
    return NULL;
  }
  return status(env, ctx, we_matmul_gated(ctx, (const we_matmul_params*)pdata, xdt, x, wdt, w, scales, group, ydt, y,
                                          (const float*)bias, flags, (const float*)gate, res));
}

/* matmulGroup(ctx, count, xDtype, wDtype, yDtype, flags, then per item params, x, w, y, bias, gate, residual):
 * we_matmul_group, one or two GEMMs of one N, K, dtypes and flags as one launch */
static napi_value MatmulGroup(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 6)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t count = u32_arg(&a, 1);
  int32_t xdt = i32_arg(&a, 2), wdt = i32_arg(&a, 3), ydt = i32_arg(&a, 4);
  uint32_t flags = u32_arg(&a, 5);
  if (a.bad) return NULL;
  if (count < 1 || count > 2 || a.argc < 6 + 7 * (size_t)count) {
    napi_throw_type_error(env, NULL, "matmulGroup takes 1 or 2 items of 7 arguments each");
    return NULL;
  }
  we_matmul_item items[2];
  memset(items, 0, sizeof(items));
  for (uint32_t i = 0; i < count; i++) {
    const size_t b = 6 + 7 * (size_t)i;
    void* pdata = NULL;
    size_t plen = 0;
    bytes_of(&a, b, &pdata, &plen);
    items[i].x = ptr_arg(&a, b + 1);
    items[i].w = ptr_arg(&a, b + 2);
    items[i].y = ptr_arg(&a, b + 3);
    items[i].bias = (const float*)ptr_arg(&a, b + 4);
    items[i].gate = (const float*)ptr_arg(&a, b + 5);
    items[i].residual = ptr_arg(&a, b + 6);
    if (a.bad) return NULL;
    if (plen != sizeof(we_matmul_params)) {
      napi_throw_type_error(env, NULL, "params must be the 13 x u32 image from matmulParams");
      return NULL;
    }
    items[i].p = (const we_matmul_params*)pdata;
  }
  return status(env, ctx, we_matmul_group(ctx, count, items, xdt, wdt, ydt, flags));
}

/* matmulMul(ctx, params, xDtype, x, wDtype, w, scales, group, yDtype, y, bias, flags, mul, aux): we_matmul_mul */
static napi_value MatmulMul(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 14)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* pdata = NULL;
  size_t plen = 0;
  bytes_of(&a, 1, &pdata, &plen);
  int32_t xdt = i32_arg(&a, 2);
  void* x = ptr_arg(&a, 3);
  int32_t wdt = i32_arg(&a, 4);
  void* w = ptr_arg(&a, 5);
  void* scales = ptr_arg(&a, 6);
  uint32_t group = u32_arg(&a, 7);
  int32_t ydt = i32_arg(&a, 8);
  void* y = ptr_arg(&a, 9);
  void* bias = ptr_arg(&a, 10);
  uint32_t flags = u32_arg(&a, 11);
  int32_t mul = i32_arg(&a, 12);
  void* aux = ptr_arg(&a, 13);
  if (a.bad) return NULL;
  if (plen != sizeof(we_matmul_params)) {
    napi_throw_type_error(env, NULL, "params must be the 13 x u32 image from matmulParams");
    return NULL;
  }
  return status(env, ctx, we_matmul_mul(ctx, (const we_matmul_params*)pdata, xdt, x, wdt, w, scales, group, ydt, y,
                                        (const float*)bias, flags, mul, aux));
}

/* matmulQkNormRope(ctx, params, xDtype, x, wDtype, w, yDtype, y, bias, flags, qHeads, kHeads, eps, offset, normQ,
 * normK, ropeFrom, cos, sin): we_matmul_qk_norm_rope */
static napi_value MatmulQkNormRope(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 19)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* pdata = NULL;
  size_t plen = 0;
  bytes_of(&a, 1, &pdata, &plen);
  int32_t xdt = i32_arg(&a, 2);
  void* x = ptr_arg(&a, 3);
  int32_t wdt = i32_arg(&a, 4);
  void* w = ptr_arg(&a, 5);
  int32_t ydt = i32_arg(&a, 6);
  void* y = ptr_arg(&a, 7);
  void* bias = ptr_arg(&a, 8);
  uint32_t flags = u32_arg(&a, 9), qh = u32_arg(&a, 10), kh = u32_arg(&a, 11);
  double eps = f64_arg(&a, 12), offset = f64_arg(&a, 13);
  void *nq = ptr_arg(&a, 14), *nk = ptr_arg(&a, 15);
  uint32_t rope_from = u32_arg(&a, 16);
  void *c = ptr_arg(&a, 17), *sn = ptr_arg(&a, 18);
  if (a.bad) return NULL;
  if (plen != sizeof(we_matmul_params)) {
    napi_throw_type_error(env, NULL, "params must be the 13 x u32 image from matmulParams");
    return NULL;
  }
  return status(env, ctx, we_matmul_qk_norm_rope(ctx, (const we_matmul_params*)pdata, xdt, x, wdt, w, ydt, y,
                                                 (const float*)bias, flags, qh, kh, (float)eps, (float)offset,
                                                 (const float*)nq, (const float*)nk, rope_from, (const float*)c,
                                                 (const float*)sn));
}

/* ---- norms, rotary, elementwise ---- */
static napi_value RmsNorm(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 11)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t rows = u32_arg(&a, 1), d = u32_arg(&a, 2);
  double eps = f64_arg(&a, 3), offset = f64_arg(&a, 4);
  int32_t dt = i32_arg(&a, 5);
  void *x = ptr_arg(&a, 6), *wt = ptr_arg(&a, 7), *sc = ptr_arg(&a, 8), *sh = ptr_arg(&a, 9), *out = ptr_arg(&a, 10);
  if (a.bad) return NULL;
  return status(env, ctx, we_rmsnorm(ctx, rows, d, (float)eps, (float)offset, dt, x, (const float*)wt,
                                     (const float*)sc, (const float*)sh, out));
}

/* rmsnormMod(ctx, rows, d, eps, offset, dtype, x, weight, tvec, table, modN, mod, out): we_rmsnorm_mod */
static napi_value RmsNormMod(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 13)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t rows = u32_arg(&a, 1), d = u32_arg(&a, 2);
  double eps = f64_arg(&a, 3), offset = f64_arg(&a, 4);
  int32_t dt = i32_arg(&a, 5);
  void *x = ptr_arg(&a, 6), *wt = ptr_arg(&a, 7), *tv = ptr_arg(&a, 8), *tb = ptr_arg(&a, 9);
  uint32_t mod_n = u32_arg(&a, 10);
  void *mod = ptr_arg(&a, 11), *out = ptr_arg(&a, 12);
  if (a.bad) return NULL;
  return status(env, ctx, we_rmsnorm_mod(ctx, rows, d, (float)eps, (float)offset, dt, x, (const float*)wt,
                                         (const float*)tv, (const float*)tb, mod_n, (float*)mod, out));
}

static napi_value Rope(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 10)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t tokens = u32_arg(&a, 1), heads = u32_arg(&a, 2), pairs = u32_arg(&a, 3);
  int32_t half = i32_arg(&a, 4), dt = i32_arg(&a, 5);
  void *x = ptr_arg(&a, 6), *c = ptr_arg(&a, 7), *s = ptr_arg(&a, 8), *out = ptr_arg(&a, 9);
  if (a.bad) return NULL;
  return status(env, ctx, we_rope(ctx, tokens, heads, pairs, half, dt, x, (const float*)c, (const float*)s, out));
}

static napi_value Elementwise(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 9)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  int32_t op = i32_arg(&a, 1);
  double n = f64_arg(&a, 2), d = f64_arg(&a, 3);
  int32_t dt = i32_arg(&a, 4);
  void *x = ptr_arg(&a, 5), *b = ptr_arg(&a, 6), *c = ptr_arg(&a, 7), *out = ptr_arg(&a, 8);
  if (a.bad) return NULL;
  return status(env, ctx, we_elementwise(ctx, op, (size_t)n, (size_t)d, dt, x, b, c, out));
}

static napi_value LayerSum(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 7)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t tokens = u32_arg(&a, 1), layers = u32_arg(&a, 2), dim = u32_arg(&a, 3);
  void *x = ptr_arg(&a, 4), *w = ptr_arg(&a, 5), *out = ptr_arg(&a, 6);
  if (a.bad) return NULL;
  return status(env, ctx, we_layer_sum(ctx, tokens, layers, dim, (const float*)x, (const float*)w, (float*)out));
}

static napi_value QkNormRope(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 16)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t tokens = u32_arg(&a, 1), heads = u32_arg(&a, 2), hd = u32_arg(&a, 3);
  double eps = f64_arg(&a, 4), offset = f64_arg(&a, 5);
  void* wt = ptr_arg(&a, 6);
  uint32_t rope_from = u32_arg(&a, 7);
  int32_t half = i32_arg(&a, 8);
  void *c = ptr_arg(&a, 9), *s = ptr_arg(&a, 10);
  int32_t dt = i32_arg(&a, 11);
  void* x = ptr_arg(&a, 12);
  uint32_t xs = u32_arg(&a, 13);
  void* out = ptr_arg(&a, 14);
  uint32_t os = u32_arg(&a, 15);
  if (a.bad) return NULL;
  return status(env, ctx, we_qk_norm_rope(ctx, tokens, heads, hd, (float)eps, (float)offset, (const float*)wt,
                                          rope_from, half, (const float*)c, (const float*)s, dt, x, xs, out, os));
}

/* attention(ctx, tokens, heads, kvHeads, dim, causal, dtype, q, qStride, k, kStride, v, vStride, out, outStride) */
static napi_value Attention(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 15)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  uint32_t tokens = u32_arg(&a, 1), heads = u32_arg(&a, 2), kvh = u32_arg(&a, 3), dim = u32_arg(&a, 4);
  int32_t causal = i32_arg(&a, 5), dt = i32_arg(&a, 6);
  void* q = ptr_arg(&a, 7);
  uint32_t qs = u32_arg(&a, 8);
  void* k = ptr_arg(&a, 9);
  uint32_t ks = u32_arg(&a, 10);
  void* v = ptr_arg(&a, 11);
  uint32_t vs = u32_arg(&a, 12);
  void* out = ptr_arg(&a, 13);
  uint32_t os = u32_arg(&a, 14);
  if (a.bad) return NULL;
  return status(env, ctx, we_attention(ctx, tokens, heads, kvh, dim, causal, dt, q, qs, k, ks, v, vs, out, os));
}

static napi_value UnpackFp8(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* packed = ptr_arg(&a, 1);
  double n = f64_arg(&a, 2);
  void *sc = ptr_arg(&a, 3), *out = ptr_arg(&a, 4);
  if (a.bad) return NULL;
  return status(env, ctx, we_unpack_fp8(ctx, packed, (size_t)n, (const float*)sc, (float*)out));
}

static napi_value DequantInt4(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 7)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void *words = ptr_arg(&a, 1), *scales = ptr_arg(&a, 2);
  uint32_t rows = u32_arg(&a, 3), k = u32_arg(&a, 4), group = u32_arg(&a, 5);
  void* out = ptr_arg(&a, 6);
  if (a.bad) return NULL;
  return status(env, ctx, we_dequant_int4(ctx, (const uint32_t*)words, (const uint16_t*)scales, rows, k, group,
                                          (float*)out));
}

static napi_value TicketDone(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  double t = f64_arg(&a, 1);
  if (a.bad) return NULL;
  int done = 0;
  int rc = we_ticket_done(ctx, (uint64_t)t, &done);
  if (rc != WE_OK) return status(env, ctx, rc);
  napi_value v;
  napi_get_boolean(env, done != 0, &v);
  return v;
}

static napi_value TimerStart(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_timer_start(ctx));
}

static napi_value TimerStop(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  float ms = 0;
  int rc = we_timer_stop(ctx, &ms);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, ms);
}

static napi_value GraphBegin(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return status(env, ctx, we_graph_begin(ctx));
}

static napi_value GraphEnd(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  we_graph* g = NULL;
  int rc = we_graph_end(ctx, &g);
  if (rc != WE_OK) return status(env, ctx, rc);
  return big(env, g);
}

static napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  we_graph* g = ptr_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_graph_launch(ctx, g));
}

static napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  we_graph* g = ptr_arg(&a, 1);
  if (a.bad) return NULL;
  return status(env, ctx, we_graph_destroy(ctx, g));
}

/* ---- peak probes: timePeak (src/bench/peak.ts:69-109) ---- */
/* peak(ctx, kind, workgroups, iters, out) -> operation count of the dispatch */
static napi_value Peak(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  int32_t kind = i32_arg(&a, 1);
  uint32_t wg = u32_arg(&a, 2), iters = u32_arg(&a, 3);
  void* out = ptr_arg(&a, 4);
  if (a.bad) return NULL;
  double ops = 0;
  int rc = we_peak(ctx, kind, wg, iters, (uint32_t*)out, &ops);
  if (rc != WE_OK) return status(env, ctx, rc);
  return num(env, ops);
}

static napi_value ReadPeak(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 4)) return NULL;
  we_ctx* ctx = ptr_arg(&a, 0);
  void* buf = ptr_arg(&a, 1);
  double bytes = f64_arg(&a, 2);
  void* out = ptr_arg(&a, 3);
  if (a.bad) return NULL;
  return status(env, ctx, we_read_peak(ctx, buf, (size_t)bytes, (uint32_t*)out));
}

/* ---- .safetensors files: readHeader / readTensor (src/weights/safetensors.ts:28-70) ---- */

/* throws Error(we_last_error(NULL)); a malformed file's error is named SafetensorsError, as the reference's */
static napi_value st_status(napi_env env, int rc) {
  if (rc == WE_OK) return undefined(env);
  napi_value msg, err;
  napi_create_string_utf8(env, we_last_error(NULL), NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  if (rc == WE_EFORMAT) {
    napi_value name;
    napi_create_string_utf8(env, "SafetensorsError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, err, "name", name);
  }
  napi_throw(env, err);
  return NULL;
}

static int str_arg(args_t* a, size_t i, char* buf, size_t cap) {
  size_t len = 0;
  if (napi_get_value_string_utf8(a->env, a->argv[i], buf, cap, &len) != napi_ok) {
    napi_throw_type_error(a->env, NULL, "expected a string");
    a->bad = 1;
    return 0;
  }
  if (len + 1 >= cap) {
    napi_throw_range_error(a->env, NULL, "string argument too long");
    a->bad = 1;
    return 0;
  }
  return 1;
}

static napi_value str(napi_env env, const char* s) {
  napi_value v;
  napi_create_string_utf8(env, s, NAPI_AUTO_LENGTH, &v);
  return v;
}

static napi_value StOpen(napi_env env, napi_callback_info info) {
  args_t a;
  char path[4096];
  if (!get_args(env, info, &a, 1) || !str_arg(&a, 0, path, sizeof path)) return NULL;
  we_safetensors* st = NULL;
  int rc = we_st_open(path, &st);
  if (rc != WE_OK) return st_status(env, rc);
  return big(env, st);
}

static napi_value StClose(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  return st_status(env, we_st_close(st));
}

static napi_value StCount(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  uint32_t n = 0;
  int rc = we_st_count(st, &n);
  if (rc != WE_OK) return st_status(env, rc);
  return num(env, n);
}

/* {name, dtype, shape: number[], offset, size} (TensorInfo, src/weights/safetensors.ts:15) */
static napi_value StInfo(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  uint32_t i = u32_arg(&a, 1);
  if (a.bad) return NULL;
  we_tensor_info t;
  int rc = we_st_info(st, i, &t);
  if (rc != WE_OK) return st_status(env, rc);
  napi_value o, shape;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "name", str(env, t.name));
  napi_set_named_property(env, o, "dtype", str(env, t.dtype));
  napi_create_array_with_length(env, t.ndim, &shape);
  for (uint32_t d = 0; d < t.ndim; d++) napi_set_element(env, shape, d, num(env, (double)t.shape[d]));
  napi_set_named_property(env, o, "shape", shape);
  napi_set_named_property(env, o, "offset", num(env, (double)t.offset));
  napi_set_named_property(env, o, "size", num(env, (double)t.size));
  return o;
}

static napi_value StFind(napi_env env, napi_callback_info info) {
  args_t a;
  char name[4096];
  if (!get_args(env, info, &a, 2)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  if (a.bad || !str_arg(&a, 1, name, sizeof name)) return NULL;
  uint32_t i = 0;
  int rc = we_st_find(st, name, &i);
  if (rc != WE_OK) return st_status(env, rc);
  return num(env, i);
}

static napi_value StMetadataCount(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 1)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  if (a.bad) return NULL;
  uint32_t n = 0;
  int rc = we_st_metadata_count(st, &n);
  if (rc != WE_OK) return st_status(env, rc);
  return num(env, n);
}

static napi_value StMetadataAt(napi_env env, napi_callback_info info) { /* [key, value] */
  args_t a;
  if (!get_args(env, info, &a, 2)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  uint32_t i = u32_arg(&a, 1);
  if (a.bad) return NULL;
  const char *k = NULL, *v = NULL;
  int rc = we_st_metadata_at(st, i, &k, &v);
  if (rc != WE_OK) return st_status(env, rc);
  napi_value pair;
  napi_create_array_with_length(env, 2, &pair);
  napi_set_element(env, pair, 0, str(env, k));
  napi_set_element(env, pair, 1, str(env, v));
  return pair;
}

/* stRead(handle, index, begin, bytes, dst, threads, ctx): dst = a TypedArray / Buffer of at least `bytes` bytes,
 * or a BigInt address of pinned memory from hostAlloc of the context ctx, which must then hold all `bytes` */
static napi_value StRead(napi_env env, napi_callback_info info) {
  args_t a;
  if (!get_args(env, info, &a, 5)) return NULL;
  we_safetensors* st = ptr_arg(&a, 0);
  uint32_t idx = u32_arg(&a, 1);
  double begin = f64_arg(&a, 2), bytes = f64_arg(&a, 3);
  uint32_t threads = a.argc > 5 && !is_nullish(env, a.argv[5]) ? u32_arg(&a, 5) : 0;
  if (a.bad) return NULL;
  if (!(begin >= 0 && bytes >= 0 && begin <= 9007199254740991.0 && bytes <= 9007199254740991.0)) {
    napi_throw_range_error(env, NULL, "begin and bytes must be non-negative integers");
    return NULL;
  }
  void* dst = NULL;
  bool is_ta = false;
  napi_is_typedarray(env, a.argv[4], &is_ta);
  if (is_ta) {
    napi_typedarray_type type;
    size_t length = 0, offset = 0;
    napi_value ab;
    void* data = NULL;
    napi_get_typedarray_info(env, a.argv[4], &type, &length, &data, &ab, &offset);
    size_t elem = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: elem = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
      default: elem = 1;
    }
    if ((double)(length * elem) < bytes) {
      napi_throw_range_error(env, NULL, "destination is smaller than the bytes to read");
      return NULL;
    }
    dst = data;
  } else {
    dst = ptr_arg(&a, 4);
    we_ctx* ctx = a.argc > 6 && !is_nullish(env, a.argv[6]) ? ptr_arg(&a, 6) : NULL;
    if (a.bad) return NULL;
    if (!ctx) {
      napi_throw_type_error(env, NULL, "a raw destination address needs the context that owns its pinned memory");
      return NULL;
    }
    int rc = we_host_span(ctx, dst, (size_t)bytes);
    if (rc != WE_OK) return status(env, ctx, rc);
  }
  return st_status(env, we_st_read(st, idx, (uint64_t)begin, (uint64_t)bytes, dst, threads));
}

static napi_value LastError(napi_env env, napi_callback_info info) {
  args_t a;
  get_args(env, info, &a, 0);
  we_ctx* ctx = a.argc > 0 ? ptr_arg(&a, 0) : NULL;
  if (a.bad) return NULL;
  napi_value s;
  napi_create_string_utf8(env, we_last_error(ctx), NAPI_AUTO_LENGTH, &s);
  return s;
}

static napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback fn;
  } fns[] = {
      {"create", Create},         {"destroy", Destroy},       {"deviceInfo", DeviceInfo},
      {"sync", Sync},             {"streamSelect", StreamSelect}, {"streamFork", StreamFork}, {"streamJoin", StreamJoin},             {"bufAlloc", BufAlloc},     {"bufFree", BufFree},
      {"upload", Upload},         {"download", Download},     {"copy", Copy},
      {"mark", Mark},             {"release", Release},       {"stats", Stats},
      {"setAllocCap", SetAllocCap}, {"setPoison", SetPoison}, {"setTuning", SetTuning}, {"timerMark", TimerMark}, {"timerBetween", TimerBetween},
      {"hostAlloc", HostAlloc},   {"hostFree", HostFree},     {"hostWrite", HostWrite}, {"hostSpan", HostSpan}, {"hostRead", HostRead},
      {"streamCopy", StreamCopy}, {"waitTicket", WaitTicket}, {"recordCompute", RecordCompute},
      {"downloadAsync", DownloadAsync}, {"waitTicketAsync", WaitTicketAsync}, {"recordAll", RecordAll},
      {"matmulParams", MatmulParams}, {"conv3x3Params", Conv3x3Params}, {"kSplitFor", KSplitFor}, {"matmul", Matmul}, {"matmulNoalloc", MatmulNoalloc}, {"matmulGated", MatmulGated}, {"matmulGroup", MatmulGroup}, {"matmulMul", MatmulMul}, {"matmulQkNormRope", MatmulQkNormRope},
      {"rmsnorm", RmsNorm},       {"rmsnormMod", RmsNormMod},       {"rope", Rope},             {"elementwise", Elementwise},
      {"layerSum", LayerSum},     {"lastError", LastError},   {"qkNormRope", QkNormRope}, {"attention", Attention},
      {"unpackFp8", UnpackFp8},   {"dequantInt4", DequantInt4}, {"ticketDone", TicketDone},
      {"timerStart", TimerStart}, {"timerStop", TimerStop},
      {"graphBegin", GraphBegin}, {"graphEnd", GraphEnd}, {"graphLaunch", GraphLaunch}, {"graphDestroy", GraphDestroy},
      {"peak", Peak},             {"readPeak", ReadPeak},
      {"stOpen", StOpen},         {"stClose", StClose},       {"stCount", StCount},
      {"stInfo", StInfo},         {"stFind", StFind},         {"stMetadataCount", StMetadataCount},
      {"stMetadataAt", StMetadataAt}, {"stRead", StRead},
  };
  for (size_t i = 0; i < sizeof fns / sizeof fns[0]; i++) {
    napi_value f;
    napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f);
    napi_set_named_property(env, exports, fns[i].name, f);
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
