/*
 * Node-API addon: the binding torch.js's TypeScript host uses to reach
 * libtorchjs_hip.so (include/torchjs_hip.h).
 *
 * Device pointers cross into JavaScript as BigInt (so views can add byte
 * offsets); an allocation is owned by an External whose finalizer returns
 * it to the library's stream-ordered cache, which is safe whenever the GC
 * runs because every later use is ordered on the library stream.  An
 * explicit free(allocation) returns the block at once and marks the
 * External, so its finalizer does nothing later (the block may by then
 * belong to another allocation).
 * Every failing call throws an Error carrying tjh_last_error().
 * Host data moves through TypedArrays.  d2hAsync enqueues its copy on the
 * library stream when it is called (tjh_d2h_start: submission order is
 * execution order, as on torch.js's single WebGPU queue), and a libuv
 * worker (napi_async_work) waits for it and resolves the Promise
 * (tjh_d2h_finish), so readbacks do not block the event loop: the
 * analogue of torch.js's mapAsync readback (buffer.ts:150-206).
 *
 * Every entry point of include/torchjs_hip.h is bound (tjh_last_error's
 * message rides on the thrown Error; tjh_version is the `version`
 * property): the runtime (init, device info and count, malloc / free,
 * copies, sync, memory stats, launch timing, timers) and every kernel
 * entry of the autograd hot path.
 */
#ifndef NAPI_VERSION
#define NAPI_VERSION 8
#endif
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "torchjs_hip.h"

#define MAXA 24

static napi_value throw_last(napi_env env, int rc) {
  char msg[1200];
  snprintf(msg, sizeof(msg), "torchjs_hip error %d: %s", rc, tjh_last_error());
  napi_throw_error(env, NULL, msg);
  return NULL;
}

#define CHECK_RC(call)                      \
  do {                                      \
    int _rc = (call);                       \
    if (_rc != 0) return throw_last(env, _rc); \
  } while (0)

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = MAXA;
  napi_value tmp[MAXA];
  if (napi_get_cb_info(env, info, &argc, tmp, NULL, NULL) != napi_ok) return 0;
  if (argc < want) {
    napi_throw_type_error(env, NULL, "too few arguments");
    return 0;
  }
  for (size_t i = 0; i < want; ++i) argv[i] = tmp[i];
  return 1;
}

static int64_t i64(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint) {
    int64_t r = 0;
    bool lossless;
    napi_get_value_bigint_int64(env, v, &r, &lossless);
    return r;
  }
  double d = 0;
  napi_get_value_double(env, v, &d);
  return (int64_t)d;
}

static double f64(napi_env env, napi_value v) {
  double d = 0;
  napi_get_value_double(env, v, &d);
  return d;
}

/* device pointer: BigInt (or 0 / null / undefined -> NULL) */
static void* ptr(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint) {
    uint64_t r = 0;
    bool lossless;
    napi_get_value_bigint_uint64(env, v, &r, &lossless);
    return (void*)(uintptr_t)r;
  }
  return NULL;
}

/* JS array of numbers -> int64 array (<= 8) */
static int i64arr(napi_env env, napi_value v, int64_t* out, int maxn) {
  uint32_t n = 0;
  napi_get_array_length(env, v, &n);
  if ((int)n > maxn) n = (uint32_t)maxn;
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, v, i, &e);
    out[i] = i64(env, e);
  }
  return (int)n;
}

static napi_value undef(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static napi_value bigint(napi_env env, void* p) {
  napi_value r;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &r);
  return r;
}

static napi_value num(napi_env env, double d) {
  napi_value r;
  napi_create_double(env, d, &r);
  return r;
}

/* ---------------------------------------------------------------- runtime */

static napi_value js_init(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_init((int)i64(env, a[0])));
  return undef(env);
}

static napi_value js_device_info(napi_env env, napi_callback_info info) {
  (void)info;
  tjh_device_info d;
  CHECK_RC(tjh_get_device_info(&d));
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, d.name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "name", s);
  napi_create_string_utf8(env, d.arch, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "arch", s);
  napi_set_named_property(env, o, "computeUnits", num(env, d.compute_units));
  napi_set_named_property(env, o, "totalMem", num(env, (double)d.total_mem));
  napi_set_named_property(env, o, "warpSize", num(env, d.warp_size));
  return o;
}

/* What an allocation's External holds: the block, and whether free() has
 * already returned it (then the GC finalizer must not). */
typedef struct {
  void* p;
  int freed;
} Block;

static void free_ext(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  Block* b = (Block*)data;
  if (!b->freed) tjh_free(b->p);
  free(b);
}

/* malloc(bytes) -> { ptr: BigInt, handle: External (frees on GC) } */
static napi_value js_malloc(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  void* p = NULL;
  CHECK_RC(tjh_malloc((size_t)i64(env, a[0]), &p));
  Block* b = (Block*)malloc(sizeof(Block));
  if (!b) {
    tjh_free(p);
    napi_throw_error(env, NULL, "malloc: out of host memory");
    return NULL;
  }
  b->p = p;
  b->freed = 0;
  napi_value o, ext;
  napi_create_object(env, &o);
  if (napi_create_external(env, b, free_ext, NULL, &ext) != napi_ok) {
    tjh_free(p);
    free(b);
    napi_throw_error(env, NULL, "malloc: napi_create_external failed");
    return NULL;
  }
  napi_set_named_property(env, o, "ptr", bigint(env, p));
  napi_set_named_property(env, o, "handle", ext);
  return o;
}

/* The Block behind an allocation object { ptr, handle } or its handle. */
static Block* block_of(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_object) {
    napi_value h;
    if (napi_get_named_property(env, v, "handle", &h) != napi_ok) return NULL;
    v = h;
    napi_typeof(env, v, &t);
  }
  if (t != napi_external) return NULL;
  void* data = NULL;
  if (napi_get_value_external(env, v, &data) != napi_ok) return NULL;
  return (Block*)data;
}

static int typed(napi_env env, napi_value v, void** data, size_t* bytes) {
  napi_typedarray_type t;
  size_t len, off;
  napi_value buf;
  if (napi_get_typedarray_info(env, v, &t, &len, data, &buf, &off) != napi_ok) return 0;
  size_t es = 1;
  switch (t) {
    case napi_int8_array: case napi_uint8_array: case napi_uint8_clamped_array: es = 1; break;
    case napi_int16_array: case napi_uint16_array: es = 2; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
    default: es = 4;
  }
  *bytes = len * es;
  return 1;
}

static napi_value js_h2d(napi_env env, napi_callback_info info) {
  napi_value a[2];
  if (!get_args(env, info, 2, a)) return NULL;
  void* src;
  size_t bytes;
  if (!typed(env, a[1], &src, &bytes)) {
    napi_throw_type_error(env, NULL, "h2d: expected a TypedArray");
    return NULL;
  }
  CHECK_RC(tjh_h2d(ptr(env, a[0]), src, bytes));
  return undef(env);
}

static napi_value js_d2h(napi_env env, napi_callback_info info) {
  napi_value a[2];
  if (!get_args(env, info, 2, a)) return NULL;
  void* dst;
  size_t bytes;
  if (!typed(env, a[1], &dst, &bytes)) {
    napi_throw_type_error(env, NULL, "d2h: expected a TypedArray");
    return NULL;
  }
  CHECK_RC(tjh_d2h(dst, ptr(env, a[0]), bytes));
  return undef(env);
}

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref keep;      /* the destination TypedArray */
  napi_ref keep_src;  /* the source allocation, when given (or NULL) */
  void* dst;
  uint64_t ticket;
  int rc;
  char msg[1024];
} D2HJob;

static void d2h_exec(napi_env env, void* data) {
  (void)env;
  D2HJob* j = (D2HJob*)data;
  j->rc = tjh_d2h_finish(j->ticket, j->dst);
  if (j->rc) snprintf(j->msg, sizeof(j->msg), "%s", tjh_last_error());
}

static void d2h_done(napi_env env, napi_status status, void* data) {
  (void)status;
  D2HJob* j = (D2HJob*)data;
  napi_value arr;
  napi_get_reference_value(env, j->keep, &arr);
  if (j->rc == 0) {
    napi_resolve_deferred(env, j->deferred, arr);
  } else {
    napi_value m, e;
    napi_create_string_utf8(env, j->msg, NAPI_AUTO_LENGTH, &m);
    napi_create_error(env, NULL, m, &e);
    napi_reject_deferred(env, j->deferred, e);
  }
  napi_delete_reference(env, j->keep);
  if (j->keep_src) napi_delete_reference(env, j->keep_src);
  napi_delete_async_work(env, j->work);
  free(j);
}

/* d2hAsync(ptr, typedArray[, allocation]) -> Promise<typedArray>.  The copy
 * is enqueued now, in submission order: kernels launched after this call,
 * or a free of the source, cannot change the bytes it reads.  The optional
 * allocation object is kept alive until the Promise settles. */
static napi_value js_d2h_async(napi_env env, napi_callback_info info) {
  size_t argc = 3;
  napi_value a[3];
  if (napi_get_cb_info(env, info, &argc, a, NULL, NULL) != napi_ok) return NULL;
  if (argc < 2) {
    napi_throw_type_error(env, NULL, "d2hAsync(ptr, typedArray[, allocation])");
    return NULL;
  }
  D2HJob* j = (D2HJob*)calloc(1, sizeof(D2HJob));
  if (!j) {
    napi_throw_error(env, NULL, "d2hAsync: out of host memory");
    return NULL;
  }
  size_t bytes = 0;
  if (!typed(env, a[1], &j->dst, &bytes)) {
    free(j);
    napi_throw_type_error(env, NULL, "d2hAsync: expected a TypedArray");
    return NULL;
  }
  int rc = tjh_d2h_start(ptr(env, a[0]), bytes, &j->ticket);
  if (rc != 0) {
    free(j);
    return throw_last(env, rc);
  }
  napi_value promise, name;
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_reference(env, a[1], 1, &j->keep);
  if (argc >= 3) {
    napi_valuetype t;
    napi_typeof(env, a[2], &t);
    if (t == napi_object || t == napi_external) napi_create_reference(env, a[2], 1, &j->keep_src);
  }
  napi_create_string_utf8(env, "tjh_d2h", NAPI_AUTO_LENGTH, &name);
  napi_create_async_work(env, NULL, name, d2h_exec, d2h_done, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

static napi_value js_sync(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_synchronize());
  return undef(env);
}

static napi_value js_memory_stats(napi_env env, napi_callback_info info) {
  (void)info;
  tjh_mem_stats s;
  CHECK_RC(tjh_memory_stats(&s));
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "activeBytes", num(env, (double)s.active_bytes));
  napi_set_named_property(env, o, "pooledBytes", num(env, (double)s.pooled_bytes));
  napi_set_named_property(env, o, "peakBytes", num(env, (double)s.peak_bytes));
  /* bufferPool.getStats() (src/backend/webgpu/buffer.ts:10-15, 98-105):
   * allocationCount counts the blocks created on a cache miss, as the
   * reference's totalAllocations does; allocationRequests (every request
   * served) is this allocator's own */
  napi_set_named_property(env, o, "allocationCount", num(env, (double)s.device_mallocs));
  napi_set_named_property(env, o, "allocationRequests", num(env, (double)s.allocations));
  return o;
}

static napi_value js_empty_cache(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_empty_cache());
  return undef(env);
}

/* ---------------------------------------------------------------- kernels */

static napi_value js_fill(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_fill_f32((float*)ptr(env, a[0]), i64(env, a[1]), (float)f64(env, a[2])));
  return undef(env);
}

static napi_value js_random(napi_env env, napi_callback_info info) {
  napi_value a[4];
  if (!get_args(env, info, 4, a)) return NULL;
  CHECK_RC(tjh_random((float*)ptr(env, a[0]), i64(env, a[1]), (uint32_t)i64(env, a[2]),
                      (int)i64(env, a[3])));
  return undef(env);
}

static napi_value js_copy_strided(napi_env env, napi_callback_info info) {
  napi_value a[5];
  if (!get_args(env, info, 5, a)) return NULL;
  int64_t shape[TJH_MAX_DIMS], ss[TJH_MAX_DIMS], ds[TJH_MAX_DIMS];
  int nd = i64arr(env, a[0], shape, TJH_MAX_DIMS);
  i64arr(env, a[2], ss, TJH_MAX_DIMS);
  i64arr(env, a[4], ds, TJH_MAX_DIMS);
  CHECK_RC(tjh_copy_strided(nd, shape, (const float*)ptr(env, a[1]), ss, (float*)ptr(env, a[3]), ds));
  return undef(env);
}

static napi_value js_unary(napi_env env, napi_callback_info info) {
  napi_value a[5];
  if (!get_args(env, info, 5, a)) return NULL;
  CHECK_RC(tjh_unary((int)i64(env, a[0]), (const float*)ptr(env, a[1]), (float*)ptr(env, a[2]),
                     i64(env, a[3]), (float)f64(env, a[4])));
  return undef(env);
}

static napi_value js_unary_backward(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_unary_backward((int)i64(env, a[0]), (const float*)ptr(env, a[1]),
                              (const float*)ptr(env, a[2]), (const float*)ptr(env, a[3]),
                              (float*)ptr(env, a[4]), i64(env, a[5]), (float)f64(env, a[6])));
  return undef(env);
}

/* binary(op, shape[], a, aStrides[], b, bStrides[], out) */
static napi_value js_binary(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  int64_t shape[TJH_MAX_DIMS], as[TJH_MAX_DIMS], bs[TJH_MAX_DIMS];
  int nd = i64arr(env, a[1], shape, TJH_MAX_DIMS);
  i64arr(env, a[3], as, TJH_MAX_DIMS);
  i64arr(env, a[5], bs, TJH_MAX_DIMS);
  CHECK_RC(tjh_binary((int)i64(env, a[0]), nd, shape, (const float*)ptr(env, a[2]), as,
                      (const float*)ptr(env, a[4]), bs, (float*)ptr(env, a[6])));
  return undef(env);
}

static napi_value js_scalar(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  CHECK_RC(tjh_scalar((int)i64(env, a[0]), (const float*)ptr(env, a[1]), (float)f64(env, a[2]),
                      (int)i64(env, a[3]), (float*)ptr(env, a[4]), i64(env, a[5])));
  return undef(env);
}

static napi_value js_reduce(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  CHECK_RC(tjh_reduce((int)i64(env, a[0]), (const float*)ptr(env, a[1]), i64(env, a[2]),
                      i64(env, a[3]), i64(env, a[4]), (float*)ptr(env, a[5])));
  return undef(env);
}

/* Fused expression program from a JS object
 *   { ins: [[op, code, dst, a, b, c, f], ...],
 *     leaves: [[devicePtr (BigInt), kind, period], ...], result }
 * (tjh_expr; a / b / c of an absent operand are 255).  Returns 0 and throws
 * on a malformed object. */
static int get_expr(napi_env env, napi_value obj, tjh_expr* P) {
  memset(P, 0, sizeof(*P));
  napi_value ins, leaves, res;
  uint32_t n = 0, nl = 0;
  if (napi_get_named_property(env, obj, "ins", &ins) != napi_ok ||
      napi_get_named_property(env, obj, "leaves", &leaves) != napi_ok ||
      napi_get_named_property(env, obj, "result", &res) != napi_ok ||
      napi_get_array_length(env, ins, &n) != napi_ok ||
      napi_get_array_length(env, leaves, &nl) != napi_ok || n > TJH_EXPR_MAX_INS ||
      nl > TJH_EXPR_MAX_LEAVES) {
    napi_throw_error(env, NULL, "expression: {ins, leaves, result} within the program limits");
    return 0;
  }
  P->n_ins = (int32_t)n;
  P->n_leaves = (int32_t)nl;
  P->result = (int32_t)i64(env, res);
  /* optional: the second (written) and third (column-summed) values,
   * register + 1, 0 for none */
  bool has = false;
  napi_value v;
  if (napi_has_named_property(env, obj, "result2", &has) == napi_ok && has &&
      napi_get_named_property(env, obj, "result2", &v) == napi_ok)
    P->result2 = (int32_t)i64(env, v);
  has = false;
  if (napi_has_named_property(env, obj, "result3", &has) == napi_ok && has &&
      napi_get_named_property(env, obj, "result3", &v) == napi_ok)
    P->result3 = (int32_t)i64(env, v);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value row, e[7];
    napi_get_element(env, ins, i, &row);
    for (uint32_t k = 0; k < 7; ++k) napi_get_element(env, row, k, &e[k]);
    tjh_expr_ins* in = &P->ins[i];
    in->op = (uint8_t)i64(env, e[0]);
    in->code = (uint8_t)i64(env, e[1]);
    in->dst = (uint8_t)i64(env, e[2]);
    in->a = (uint8_t)i64(env, e[3]);
    in->b = (uint8_t)i64(env, e[4]);
    in->c = (uint8_t)i64(env, e[5]);
    in->f = (float)f64(env, e[6]);
  }
  for (uint32_t k = 0; k < nl; ++k) {
    napi_value row, e[3];
    napi_get_element(env, leaves, k, &row);
    for (uint32_t j = 0; j < 3; ++j) napi_get_element(env, row, j, &e[j]);
    P->leaf[k] = (const float*)ptr(env, e[0]);
    P->kind[k] = (int32_t)i64(env, e[1]);
    P->period[k] = i64(env, e[2]);
  }
  return 1;
}

/* exprEval(program, n, out) */
static napi_value js_expr_eval(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  tjh_expr P;
  if (!get_expr(env, a[0], &P)) return NULL;
  CHECK_RC(tjh_expr_eval(&P, i64(env, a[1]), (float*)ptr(env, a[2])));
  return undef(env);
}

/* graphBegin() -> id; graphEnd(id); graphReplay(id); graphDestroy(id) */
static napi_value js_graph_begin(napi_env env, napi_callback_info info) {
  (void)info;
  int id = 0;
  CHECK_RC(tjh_graph_begin(&id));
  return num(env, id);
}

static napi_value js_graph_end(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_graph_end((int)i64(env, a[0])));
  return undef(env);
}

static napi_value js_graph_replay(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_graph_replay((int)i64(env, a[0])));
  return undef(env);
}

static napi_value js_graph_destroy(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_graph_destroy((int)i64(env, a[0])));
  return undef(env);
}

/* exprCompile(program, n, colsum) */
static napi_value js_expr_compile(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  tjh_expr P;
  if (!get_expr(env, a[0], &P)) return NULL;
  CHECK_RC(tjh_expr_compile(&P, i64(env, a[1]), (int)i64(env, a[2])));
  return undef(env);
}

/* exprColsum(program, outer, r, inner, out, values | null) */
static napi_value js_expr_colsum(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  tjh_expr P;
  if (!get_expr(env, a[0], &P)) return NULL;
  CHECK_RC(tjh_expr_colsum(&P, i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                           (float*)ptr(env, a[4]), (float*)ptr(env, a[5])));
  return undef(env);
}

/* exprColsum2(program, outer, r, inner, out, values, values2) */
static napi_value js_expr_colsum2(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  tjh_expr P;
  if (!get_expr(env, a[0], &P)) return NULL;
  CHECK_RC(tjh_expr_colsum2(&P, i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                            (float*)ptr(env, a[4]), (float*)ptr(env, a[5]), (float*)ptr(env, a[6])));
  return undef(env);
}

/* exprColsum3(program, outer, r, inner, out, values, values2, out3) */
static napi_value js_expr_colsum3(napi_env env, napi_callback_info info) {
  napi_value a[8];
  if (!get_args(env, info, 8, a)) return NULL;
  tjh_expr P;
  if (!get_expr(env, a[0], &P)) return NULL;
  CHECK_RC(tjh_expr_colsum3(&P, i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                            (float*)ptr(env, a[4]), (float*)ptr(env, a[5]), (float*)ptr(env, a[6]),
                            (float*)ptr(env, a[7])));
  return undef(env);
}

static napi_value js_softmax_forward(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_softmax_forward((const float*)ptr(env, a[0]), i64(env, a[1]), (float*)ptr(env, a[2]),
                               i64(env, a[3]), i64(env, a[4]), i64(env, a[5]), (int)i64(env, a[6])));
  return undef(env);
}

static napi_value js_softmax_backward(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  CHECK_RC(tjh_softmax_backward((const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]),
                                (float*)ptr(env, a[2]), i64(env, a[3]), i64(env, a[4]),
                                (int)i64(env, a[5])));
  return undef(env);
}

/* crossEntropyForward(logits, ld, targets, rows, cols, ignore, weight, labelSmoothing, lse,
 *                     lossRows, reduction, out); weight may be null */
static napi_value js_ce_forward(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  CHECK_RC(tjh_cross_entropy_forward((const float*)ptr(env, a[0]), i64(env, a[1]),
                                     (const int32_t*)ptr(env, a[2]), i64(env, a[3]), i64(env, a[4]),
                                     (int32_t)i64(env, a[5]), (const float*)ptr(env, a[6]),
                                     (float)f64(env, a[7]), (float*)ptr(env, a[8]),
                                     (float*)ptr(env, a[9]), (int)i64(env, a[10]),
                                     (float*)ptr(env, a[11])));
  return undef(env);
}

/* crossEntropyBackward(logits, ld, targets, weight, labelSmoothing, lse, gradOut, rows, cols,
 *                      ignore, reduction, d, ldd, acc) */
static napi_value js_ce_backward(napi_env env, napi_callback_info info) {
  napi_value a[14];
  if (!get_args(env, info, 14, a)) return NULL;
  CHECK_RC(tjh_cross_entropy_backward(
      (const float*)ptr(env, a[0]), i64(env, a[1]), (const int32_t*)ptr(env, a[2]),
      (const float*)ptr(env, a[3]), (float)f64(env, a[4]), (const float*)ptr(env, a[5]),
      (const float*)ptr(env, a[6]), i64(env, a[7]), i64(env, a[8]), (int32_t)i64(env, a[9]),
      (int)i64(env, a[10]), (float*)ptr(env, a[11]), i64(env, a[12]), (int)i64(env, a[13])));
  return undef(env);
}

/* crossEntropyForwardGrad(logits, ld, targets, rows, cols, ignore, lse, lossRows, reduction,
 *                         out, d, ldd): the scalar loss and its logits' gradient for a unit
 * seed, one pass over the logits */
static napi_value js_ce_forward_grad(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  CHECK_RC(tjh_cross_entropy_forward_grad(
      (const float*)ptr(env, a[0]), i64(env, a[1]), (const int32_t*)ptr(env, a[2]),
      i64(env, a[3]), i64(env, a[4]), (int32_t)i64(env, a[5]), (float*)ptr(env, a[6]),
      (float*)ptr(env, a[7]), (int)i64(env, a[8]), (float*)ptr(env, a[9]),
      (float*)ptr(env, a[10]), i64(env, a[11])));
  return undef(env);
}

static napi_value js_ln_forward(napi_env env, napi_callback_info info) {
  napi_value a[9];
  if (!get_args(env, info, 9, a)) return NULL;
  CHECK_RC(tjh_layer_norm_forward((const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]),
                                  (const float*)ptr(env, a[2]), (float*)ptr(env, a[3]),
                                  (float*)ptr(env, a[4]), (float*)ptr(env, a[5]), i64(env, a[6]),
                                  i64(env, a[7]), (float)f64(env, a[8])));
  return undef(env);
}

static napi_value js_ln_backward(napi_env env, napi_callback_info info) {
  napi_value a[11];
  if (!get_args(env, info, 11, a)) return NULL;
  CHECK_RC(tjh_layer_norm_backward(
      (const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]),
      (const float*)ptr(env, a[3]), (const float*)ptr(env, a[4]), (float*)ptr(env, a[5]),
      (float*)ptr(env, a[6]), (float*)ptr(env, a[7]), i64(env, a[8]), i64(env, a[9]),
      (int)i64(env, a[10])));
  return undef(env);
}

/* layerNormBackwardRes(dy, x, gamma, mean, rstd, res, dx, dgamma, dbeta, rows, cols, accumulate) */
static napi_value js_ln_backward_res(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  CHECK_RC(tjh_layer_norm_backward_res(
      (const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]),
      (const float*)ptr(env, a[3]), (const float*)ptr(env, a[4]), (const float*)ptr(env, a[5]),
      (float*)ptr(env, a[6]), (float*)ptr(env, a[7]), (float*)ptr(env, a[8]), i64(env, a[9]),
      i64(env, a[10]), (int)i64(env, a[11])));
  return undef(env);
}

/* layerNormBackwardNoalloc(dy, x, gamma, mean, rstd, res, dx, dgamma, dbeta, rows, cols, acc):
 * the allocation-free variant (partials in the library's static scratch) */
static napi_value js_ln_backward_noalloc(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  CHECK_RC(tjh_layer_norm_backward_noalloc(
      (const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]),
      (const float*)ptr(env, a[3]), (const float*)ptr(env, a[4]), (const float*)ptr(env, a[5]),
      (float*)ptr(env, a[6]), (float*)ptr(env, a[7]), (float*)ptr(env, a[8]), i64(env, a[9]),
      i64(env, a[10]), (int)i64(env, a[11])));
  return undef(env);
}

/* flushDeferred() */
static napi_value js_flush_deferred(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_flush_deferred());
  return undef(env);
}

static napi_value js_emb_forward(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  CHECK_RC(tjh_embedding_forward((const float*)ptr(env, a[0]), i64(env, a[1]), i64(env, a[2]),
                                 (const int32_t*)ptr(env, a[3]), i64(env, a[4]),
                                 (float*)ptr(env, a[5])));
  return undef(env);
}

static napi_value js_emb_backward(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_embedding_backward((const float*)ptr(env, a[0]), (const int32_t*)ptr(env, a[1]),
                                  i64(env, a[2]), i64(env, a[3]), (float*)ptr(env, a[4]),
                                  i64(env, a[5]), (int)i64(env, a[6])));
  return undef(env);
}

/* embeddingPosForward(weight, num, dim, ids, batch, T, posWeight, numPos, pos0, out) */
static napi_value js_emb_pos_forward(napi_env env, napi_callback_info info) {
  napi_value a[10];
  if (!get_args(env, info, 10, a)) return NULL;
  CHECK_RC(tjh_embedding_pos_forward((const float*)ptr(env, a[0]), i64(env, a[1]),
                                     i64(env, a[2]), (const int32_t*)ptr(env, a[3]),
                                     i64(env, a[4]), i64(env, a[5]), (const float*)ptr(env, a[6]),
                                     i64(env, a[7]), i64(env, a[8]), (float*)ptr(env, a[9])));
  return undef(env);
}

/* embeddingPosBackward(dout, ids, batch, T, dim, dweight, num, accumulate, dpos, numPos, pos0,
 * accPos); a table passed as null gets no gradient */
static napi_value js_emb_pos_backward(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  CHECK_RC(tjh_embedding_pos_backward((const float*)ptr(env, a[0]),
                                      (const int32_t*)ptr(env, a[1]), i64(env, a[2]),
                                      i64(env, a[3]), i64(env, a[4]), (float*)ptr(env, a[5]),
                                      i64(env, a[6]), (int)i64(env, a[7]),
                                      (float*)ptr(env, a[8]), i64(env, a[9]), i64(env, a[10]),
                                      (int)i64(env, a[11])));
  return undef(env);
}

/* gemm(transA, transB, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, batch, bias, biasMode) */
static napi_value js_gemm(napi_env env, napi_callback_info info) {
  napi_value a[19];
  if (!get_args(env, info, 19, a)) return NULL;
  CHECK_RC(tjh_gemm((int)i64(env, a[0]), (int)i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                    i64(env, a[4]), (float)f64(env, a[5]), (const float*)ptr(env, a[6]),
                    i64(env, a[7]), i64(env, a[8]), (const float*)ptr(env, a[9]), i64(env, a[10]),
                    i64(env, a[11]), (float)f64(env, a[12]), (float*)ptr(env, a[13]),
                    i64(env, a[14]), i64(env, a[15]), i64(env, a[16]),
                    (const float*)ptr(env, a[17]), (int)i64(env, a[18])));
  return undef(env);
}

/* gemmAct(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, biasMode, aux, ldaux, act) */
static napi_value js_gemm_act(napi_env env, napi_callback_info info) {
  napi_value a[18];
  if (!get_args(env, info, 18, a)) return NULL;
  CHECK_RC(tjh_gemm_act((int)i64(env, a[0]), (int)i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                        i64(env, a[4]), (float)f64(env, a[5]), (const float*)ptr(env, a[6]),
                        i64(env, a[7]), (const float*)ptr(env, a[8]), i64(env, a[9]),
                        (float)f64(env, a[10]), (float*)ptr(env, a[11]), i64(env, a[12]),
                        (const float*)ptr(env, a[13]), (int)i64(env, a[14]), (float*)ptr(env, a[15]),
                        i64(env, a[16]), (int)i64(env, a[17])));
  return undef(env);
}

/* crossEntropyRowScale(targets, gradOut, rows, cols, ignoreIndex, reduction, rowScale) */
static napi_value js_ce_row_scale(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_cross_entropy_row_scale((const int32_t*)ptr(env, a[0]), (const float*)ptr(env, a[1]),
                                       i64(env, a[2]), i64(env, a[3]), (int32_t)i64(env, a[4]),
                                       (int)i64(env, a[5]), (float*)ptr(env, a[6])));
  return undef(env);
}

/* gemmCe(transA, M, N, K, logits, ld, lse, targets, rowScale, B, ldb, C, ldc) */
static napi_value js_gemm_ce(napi_env env, napi_callback_info info) {
  napi_value a[13];
  if (!get_args(env, info, 13, a)) return NULL;
  CHECK_RC(tjh_gemm_ce((int)i64(env, a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                       (const float*)ptr(env, a[4]), i64(env, a[5]), (const float*)ptr(env, a[6]),
                       (const int32_t*)ptr(env, a[7]), (const float*)ptr(env, a[8]),
                       (const float*)ptr(env, a[9]), i64(env, a[10]), (float*)ptr(env, a[11]),
                       i64(env, a[12])));
  return undef(env);
}

/* sdpaForward(q, k, v, o, lse, B, H, Tq, Tk, D, qs[3], ks[3], vs[3], os[3], scale, causal) */
static napi_value js_sdpa_forward(napi_env env, napi_callback_info info) {
  napi_value a[16];
  if (!get_args(env, info, 16, a)) return NULL;
  int64_t qs[3], ks[3], vs[3], os[3];
  i64arr(env, a[10], qs, 3);
  i64arr(env, a[11], ks, 3);
  i64arr(env, a[12], vs, 3);
  i64arr(env, a[13], os, 3);
  CHECK_RC(tjh_sdpa_forward((const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]),
                            (const float*)ptr(env, a[2]), (float*)ptr(env, a[3]),
                            (float*)ptr(env, a[4]), i64(env, a[5]), i64(env, a[6]), i64(env, a[7]),
                            i64(env, a[8]), i64(env, a[9]), qs, ks, vs, os, (float)f64(env, a[14]),
                            (int)i64(env, a[15])));
  return undef(env);
}

/* sdpaBackward(q,k,v,o,dO,lse,dq,dk,dv, B,H,Tq,Tk,D, strides[8][3], scale, causal) */
static napi_value js_sdpa_backward(napi_env env, napi_callback_info info) {
  napi_value a[17];
  if (!get_args(env, info, 17, a)) return NULL;
  int64_t st[8][3];
  const int64_t* sp[8];
  for (uint32_t i = 0; i < 8; ++i) {
    napi_value e;
    napi_get_element(env, a[14], i, &e);
    i64arr(env, e, st[i], 3);
    sp[i] = st[i];
  }
  CHECK_RC(tjh_sdpa_backward(
      (const float*)ptr(env, a[0]), (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]),
      (const float*)ptr(env, a[3]), (const float*)ptr(env, a[4]), (const float*)ptr(env, a[5]),
      (float*)ptr(env, a[6]), (float*)ptr(env, a[7]), (float*)ptr(env, a[8]), i64(env, a[9]),
      i64(env, a[10]), i64(env, a[11]), i64(env, a[12]), i64(env, a[13]), sp,
      (float)f64(env, a[15]), (int)i64(env, a[16])));
  return undef(env);
}

/* adamStep(params[], grads[], m[], v[], numels[], steps[], lr, b1, b2, eps, wd, decoupled) */
static napi_value js_adam_step(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  uint32_t n = 0;
  napi_get_array_length(env, a[0], &n);
  float** p = (float**)calloc(n ? n : 1, sizeof(float*));
  const float** g = (const float**)calloc(n ? n : 1, sizeof(float*));
  float** m = (float**)calloc(n ? n : 1, sizeof(float*));
  float** v = (float**)calloc(n ? n : 1, sizeof(float*));
  int64_t* ne = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  int64_t* st = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, a[0], i, &e); p[i] = (float*)ptr(env, e);
    napi_get_element(env, a[1], i, &e); g[i] = (const float*)ptr(env, e);
    napi_get_element(env, a[2], i, &e); m[i] = (float*)ptr(env, e);
    napi_get_element(env, a[3], i, &e); v[i] = (float*)ptr(env, e);
    napi_get_element(env, a[4], i, &e); ne[i] = i64(env, e);
    napi_get_element(env, a[5], i, &e); st[i] = i64(env, e);
  }
  int rc = tjh_adam_step((int)n, p, g, m, v, ne, st, f64(env, a[6]), f64(env, a[7]),
                         f64(env, a[8]), f64(env, a[9]), f64(env, a[10]), (int)i64(env, a[11]));
  free(p); free(g); free(m); free(v); free(ne); free(st);
  if (rc) return throw_last(env, rc);
  return undef(env);
}

/* adamStepDev(params, grads, expAvg, expAvgSq, numels, stepCounters (device
 * pointers to int64), lr, beta1, beta2, eps, weightDecay, decoupled) */
static napi_value js_adam_step_dev(napi_env env, napi_callback_info info) {
  napi_value a[12];
  if (!get_args(env, info, 12, a)) return NULL;
  uint32_t n = 0;
  napi_get_array_length(env, a[0], &n);
  float** p = (float**)calloc(n ? n : 1, sizeof(float*));
  const float** g = (const float**)calloc(n ? n : 1, sizeof(float*));
  float** m = (float**)calloc(n ? n : 1, sizeof(float*));
  float** v = (float**)calloc(n ? n : 1, sizeof(float*));
  int64_t* ne = (int64_t*)calloc(n ? n : 1, sizeof(int64_t));
  int64_t** st = (int64_t**)calloc(n ? n : 1, sizeof(int64_t*));
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, a[0], i, &e); p[i] = (float*)ptr(env, e);
    napi_get_element(env, a[1], i, &e); g[i] = (const float*)ptr(env, e);
    napi_get_element(env, a[2], i, &e); m[i] = (float*)ptr(env, e);
    napi_get_element(env, a[3], i, &e); v[i] = (float*)ptr(env, e);
    napi_get_element(env, a[4], i, &e); ne[i] = i64(env, e);
    napi_get_element(env, a[5], i, &e); st[i] = (int64_t*)ptr(env, e);
  }
  int rc = tjh_adam_step_dev((int)n, p, g, m, v, ne, st, f64(env, a[6]), f64(env, a[7]),
                             f64(env, a[8]), f64(env, a[9]), f64(env, a[10]), (int)i64(env, a[11]));
  free(p); free(g); free(m); free(v); free(ne); free(st);
  if (rc) return throw_last(env, rc);
  return undef(env);
}

/* ------------------------------------------------- remaining entry points */

#define F32(v) ((float*)ptr(env, (v)))
#define CF32(v) ((const float*)ptr(env, (v)))
#define I32(v) ((int32_t*)ptr(env, (v)))
#define CI32(v) ((const int32_t*)ptr(env, (v)))

static napi_value js_is_initialized(napi_env env, napi_callback_info info) {
  (void)info;
  return num(env, tjh_is_initialized());
}
static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int n = 0;
  CHECK_RC(tjh_device_count(&n));
  return num(env, n);
}
/* free(allocation): returns the block of an allocation object from malloc
 * (or its handle) to the cache now, in stream order; the handle's GC
 * finalizer then does nothing.  Freeing an allocation twice throws. */
static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  Block* b = block_of(env, a[0]);
  if (!b) {
    napi_throw_type_error(env, NULL, "free: expected the allocation returned by malloc");
    return NULL;
  }
  if (b->freed) {
    napi_throw_error(env, NULL, "free: allocation already freed");
    return NULL;
  }
  CHECK_RC(tjh_free(b->p));
  b->freed = 1;
  return undef(env);
}
static napi_value js_reset_peak(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_reset_peak());
  return undef(env);
}
static napi_value js_d2d(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_d2d(ptr(env, a[0]), ptr(env, a[1]), (size_t)i64(env, a[2])));
  return undef(env);
}
static napi_value js_kprof_enable(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_kprof_enable((int)i64(env, a[0])));
  return undef(env);
}
static napi_value js_kprof_filter(napi_env env, napi_callback_info info) {
  napi_value a[1];
  char buf[256];
  size_t len = 0;
  if (!get_args(env, info, 1, a)) return NULL;
  napi_get_value_string_utf8(env, a[0], buf, sizeof(buf), &len);
  CHECK_RC(tjh_kprof_filter(buf));
  return undef(env);
}
static napi_value js_kprof_reset(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_kprof_reset());
  return undef(env);
}
/* kprofQuery(family) -> { launches, ms } */
static napi_value js_kprof_query(napi_env env, napi_callback_info info) {
  napi_value a[1], o;
  char buf[256];
  size_t len = 0;
  int64_t n = 0;
  double ms = 0.0;
  if (!get_args(env, info, 1, a)) return NULL;
  napi_get_value_string_utf8(env, a[0], buf, sizeof(buf), &len);
  CHECK_RC(tjh_kprof_query(buf, &n, &ms));
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "launches", num(env, (double)n));
  napi_set_named_property(env, o, "ms", num(env, ms));
  return o;
}
static napi_value js_kprof_names(napi_env env, napi_callback_info info) {
  (void)info;
  static char buf[65536];
  napi_value s;
  CHECK_RC(tjh_kprof_names(buf, sizeof(buf)));
  napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &s);
  return s;
}
static napi_value js_timer_start(napi_env env, napi_callback_info info) {
  (void)info;
  int id = 0;
  CHECK_RC(tjh_timer_start(&id));
  return num(env, id);
}
static napi_value js_timer_stop(napi_env env, napi_callback_info info) {
  napi_value a[1];
  double ms = 0.0;
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_timer_stop((int)i64(env, a[0]), &ms));
  return num(env, ms);
}
static napi_value js_timer_end(napi_env env, napi_callback_info info) {
  napi_value a[1];
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_timer_end((int)i64(env, a[0])));
  return undef(env);
}
static napi_value js_timer_read(napi_env env, napi_callback_info info) {
  napi_value a[1];
  double ms = 0.0;
  if (!get_args(env, info, 1, a)) return NULL;
  CHECK_RC(tjh_timer_read((int)i64(env, a[0]), &ms));
  return num(env, ms);
}
/* rangePush(name) / rangePop() / mark(name): roctx ranges for record_function */
static napi_value js_range_push(napi_env env, napi_callback_info info) {
  napi_value a[1];
  char buf[512];
  size_t len = 0;
  if (!get_args(env, info, 1, a)) return NULL;
  napi_get_value_string_utf8(env, a[0], buf, sizeof(buf), &len);
  CHECK_RC(tjh_range_push(buf));
  return undef(env);
}
static napi_value js_range_pop(napi_env env, napi_callback_info info) {
  (void)info;
  CHECK_RC(tjh_range_pop());
  return undef(env);
}
static napi_value js_mark(napi_env env, napi_callback_info info) {
  napi_value a[1];
  char buf[512];
  size_t len = 0;
  if (!get_args(env, info, 1, a)) return NULL;
  napi_get_value_string_utf8(env, a[0], buf, sizeof(buf), &len);
  CHECK_RC(tjh_mark(buf));
  return undef(env);
}
static napi_value js_fill_i32(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_fill_i32(I32(a[0]), i64(env, a[1]), (int32_t)i64(env, a[2])));
  return undef(env);
}
static napi_value js_copy_strided_i32(napi_env env, napi_callback_info info) {
  napi_value a[5];
  int64_t shape[TJH_MAX_DIMS], ss[TJH_MAX_DIMS], ds[TJH_MAX_DIMS];
  if (!get_args(env, info, 5, a)) return NULL;
  int nd = i64arr(env, a[0], shape, TJH_MAX_DIMS);
  i64arr(env, a[2], ss, TJH_MAX_DIMS);
  i64arr(env, a[4], ds, TJH_MAX_DIMS);
  CHECK_RC(tjh_copy_strided_i32(nd, shape, CI32(a[1]), ss, I32(a[3]), ds));
  return undef(env);
}
static napi_value js_cast_f32_i32(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_cast_f32_i32(CF32(a[0]), I32(a[1]), i64(env, a[2])));
  return undef(env);
}
static napi_value js_cast_i32_f32(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_cast_i32_f32(CI32(a[0]), F32(a[1]), i64(env, a[2])));
  return undef(env);
}
/* ternary(op, shape, g, gStrides, a, aStrides, b, bStrides, out) */
static napi_value js_ternary(napi_env env, napi_callback_info info) {
  napi_value a[9];
  int64_t shape[TJH_MAX_DIMS], gs[TJH_MAX_DIMS], as[TJH_MAX_DIMS], bs[TJH_MAX_DIMS];
  if (!get_args(env, info, 9, a)) return NULL;
  int nd = i64arr(env, a[1], shape, TJH_MAX_DIMS);
  i64arr(env, a[3], gs, TJH_MAX_DIMS);
  i64arr(env, a[5], as, TJH_MAX_DIMS);
  i64arr(env, a[7], bs, TJH_MAX_DIMS);
  CHECK_RC(tjh_ternary((int)i64(env, a[0]), nd, shape, CF32(a[2]), gs, CF32(a[4]), as, CF32(a[6]),
                       bs, F32(a[8])));
  return undef(env);
}
static napi_value js_pow_scalar_backward(napi_env env, napi_callback_info info) {
  napi_value a[5];
  if (!get_args(env, info, 5, a)) return NULL;
  CHECK_RC(tjh_pow_scalar_backward(CF32(a[0]), CF32(a[1]), (float)f64(env, a[2]), F32(a[3]),
                                   i64(env, a[4])));
  return undef(env);
}
static napi_value js_axpy(napi_env env, napi_callback_info info) {
  napi_value a[5];
  if (!get_args(env, info, 5, a)) return NULL;
  CHECK_RC(tjh_axpy((float)f64(env, a[0]), CF32(a[1]), CF32(a[2]), F32(a[3]), i64(env, a[4])));
  return undef(env);
}
/* maskedFill(shape, x, xStrides, mask(uint8), maskStrides, value, out) */
static napi_value js_masked_fill(napi_env env, napi_callback_info info) {
  napi_value a[7];
  int64_t shape[TJH_MAX_DIMS], xs[TJH_MAX_DIMS], ms[TJH_MAX_DIMS];
  if (!get_args(env, info, 7, a)) return NULL;
  int nd = i64arr(env, a[0], shape, TJH_MAX_DIMS);
  i64arr(env, a[2], xs, TJH_MAX_DIMS);
  i64arr(env, a[4], ms, TJH_MAX_DIMS);
  CHECK_RC(tjh_masked_fill(nd, shape, CF32(a[1]), xs, (const uint8_t*)ptr(env, a[3]), ms,
                           (float)f64(env, a[5]), F32(a[6])));
  return undef(env);
}
/* compare(op, shape, a, aStrides, b, bStrides, out) */
static napi_value js_compare(napi_env env, napi_callback_info info) {
  napi_value a[7];
  int64_t shape[TJH_MAX_DIMS], as[TJH_MAX_DIMS], bs[TJH_MAX_DIMS];
  if (!get_args(env, info, 7, a)) return NULL;
  int nd = i64arr(env, a[1], shape, TJH_MAX_DIMS);
  i64arr(env, a[3], as, TJH_MAX_DIMS);
  i64arr(env, a[5], bs, TJH_MAX_DIMS);
  CHECK_RC(tjh_compare((int)i64(env, a[0]), nd, shape, CF32(a[2]), as, CF32(a[4]), bs, F32(a[6])));
  return undef(env);
}
/* argmax(x, outer, r, inner, isMin, out(int32)) */
static napi_value js_argmax(napi_env env, napi_callback_info info) {
  napi_value a[6];
  if (!get_args(env, info, 6, a)) return NULL;
  CHECK_RC(tjh_argmax(CF32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                      (int)i64(env, a[4]), I32(a[5])));
  return undef(env);
}
/* nllLossForward(logp, ld, targets, rows, cols, ignore, weight, lossRows, reduction, out) */
static napi_value js_nll_forward(napi_env env, napi_callback_info info) {
  napi_value a[10];
  if (!get_args(env, info, 10, a)) return NULL;
  CHECK_RC(tjh_nll_loss_forward(CF32(a[0]), i64(env, a[1]), CI32(a[2]), i64(env, a[3]),
                                i64(env, a[4]), (int32_t)i64(env, a[5]), CF32(a[6]), F32(a[7]),
                                (int)i64(env, a[8]), F32(a[9])));
  return undef(env);
}
/* nllLossBackward(targets, weight, gradOut, rows, cols, ignore, reduction, dlogp) */
static napi_value js_nll_backward(napi_env env, napi_callback_info info) {
  napi_value a[8];
  if (!get_args(env, info, 8, a)) return NULL;
  CHECK_RC(tjh_nll_loss_backward(CI32(a[0]), CF32(a[1]), CF32(a[2]), i64(env, a[3]),
                                 i64(env, a[4]), (int32_t)i64(env, a[5]), (int)i64(env, a[6]),
                                 F32(a[7])));
  return undef(env);
}
/* cast(srcDtype, dstDtype, src, dst, n): dtypes 0 f32, 1 i32, 2 u8, 3 bool */
static napi_value js_cast(napi_env env, napi_callback_info info) {
  napi_value a[5];
  if (!get_args(env, info, 5, a)) return NULL;
  CHECK_RC(tjh_cast((int)i64(env, a[0]), (int)i64(env, a[1]), ptr(env, a[2]), ptr(env, a[3]),
                    i64(env, a[4])));
  return undef(env);
}
/* fillU8(ptr, n, value) */
static napi_value js_fill_u8(napi_env env, napi_callback_info info) {
  napi_value a[3];
  if (!get_args(env, info, 3, a)) return NULL;
  CHECK_RC(tjh_fill_u8((uint8_t*)ptr(env, a[0]), i64(env, a[1]), (uint8_t)i64(env, a[2])));
  return undef(env);
}
/* copyStridedU8(shape, src, srcStrides, dst, dstStrides) */
static napi_value js_copy_strided_u8(napi_env env, napi_callback_info info) {
  napi_value a[5];
  int64_t shape[TJH_MAX_DIMS], ss[TJH_MAX_DIMS], ds[TJH_MAX_DIMS];
  if (!get_args(env, info, 5, a)) return NULL;
  int nd = i64arr(env, a[0], shape, TJH_MAX_DIMS);
  i64arr(env, a[2], ss, TJH_MAX_DIMS);
  i64arr(env, a[4], ds, TJH_MAX_DIMS);
  CHECK_RC(tjh_copy_strided_u8(nd, shape, (const uint8_t*)ptr(env, a[1]), ss,
                               (uint8_t*)ptr(env, a[3]), ds));
  return undef(env);
}
/* triangle(x, out, batch, rows, cols, diagonal, upper) */
static napi_value js_triangle(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_triangle(CF32(a[0]), F32(a[1]), i64(env, a[2]), i64(env, a[3]), i64(env, a[4]),
                        i64(env, a[5]), (int)i64(env, a[6])));
  return undef(env);
}
/* multinomial(probs, rows, cols, numSamples, replacement, seed, out) */
static napi_value js_multinomial(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_multinomial(CF32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]),
                           (int)i64(env, a[4]), (uint32_t)i64(env, a[5]), I32(a[6])));
  return undef(env);
}
/* indexSelect(x, outer, srcLen, inner, idx, nIdx, out) */
static napi_value js_index_select(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_index_select(CF32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]), CI32(a[4]),
                            i64(env, a[5]), F32(a[6])));
  return undef(env);
}
/* indexAdd(dx, outer, srcLen, inner, idx, nIdx, dout) */
static napi_value js_index_add(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_index_add(F32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]), CI32(a[4]),
                         i64(env, a[5]), CF32(a[6])));
  return undef(env);
}
/* gather(x, outer, srcLen, inner, idx, idxLen, out) */
static napi_value js_gather(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_gather(CF32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]), CI32(a[4]),
                      i64(env, a[5]), F32(a[6])));
  return undef(env);
}
/* scatterAdd(dx, outer, dstLen, inner, idx, idxLen, src) */
static napi_value js_scatter_add(napi_env env, napi_callback_info info) {
  napi_value a[7];
  if (!get_args(env, info, 7, a)) return NULL;
  CHECK_RC(tjh_scatter_add(F32(a[0]), i64(env, a[1]), i64(env, a[2]), i64(env, a[3]), CI32(a[4]),
                           i64(env, a[5]), CF32(a[6])));
  return undef(env);
}
/* oneHot(x(float), n, classes, out) and oneHotI32(x(int32), n, classes, out) */
static napi_value js_one_hot(napi_env env, napi_callback_info info) {
  napi_value a[4];
  if (!get_args(env, info, 4, a)) return NULL;
  CHECK_RC(tjh_one_hot(CF32(a[0]), i64(env, a[1]), i64(env, a[2]), F32(a[3])));
  return undef(env);
}
static napi_value js_one_hot_i32(napi_env env, napi_callback_info info) {
  napi_value a[4];
  if (!get_args(env, info, 4, a)) return NULL;
  CHECK_RC(tjh_one_hot_i32(CI32(a[0]), i64(env, a[1]), i64(env, a[2]), F32(a[3])));
  return undef(env);
}
/* nonzero(x, shape, out(int32 [maxOut, ndim]), maxOut) -> count */
static napi_value js_nonzero(napi_env env, napi_callback_info info) {
  napi_value a[4];
  int64_t shape[TJH_MAX_DIMS], count = 0;
  if (!get_args(env, info, 4, a)) return NULL;
  int nd = i64arr(env, a[1], shape, TJH_MAX_DIMS);
  CHECK_RC(tjh_nonzero(CF32(a[0]), nd, shape, I32(a[2]), i64(env, a[3]), &count));
  return num(env, (double)count);
}
/* conv descriptor: [n, c, h, w, oc, kh, kw, strideH, strideW, padH, padW,
 * dilH, dilW, groups, oh, ow] */
static int conv_desc(napi_env env, napi_value v, tjh_conv2d_desc* d) {
  int64_t f[16];
  if (i64arr(env, v, f, 16) != 16) {
    napi_throw_type_error(env, NULL, "conv2d: descriptor must have 16 numbers");
    return 0;
  }
  d->n = f[0]; d->c = f[1]; d->h = f[2]; d->w = f[3]; d->oc = f[4]; d->kh = f[5]; d->kw = f[6];
  d->stride_h = f[7]; d->stride_w = f[8]; d->pad_h = f[9]; d->pad_w = f[10]; d->dil_h = f[11];
  d->dil_w = f[12]; d->groups = f[13]; d->oh = f[14]; d->ow = f[15];
  return 1;
}
static napi_value js_conv_forward(napi_env env, napi_callback_info info) {
  napi_value a[5];
  tjh_conv2d_desc d;
  if (!get_args(env, info, 5, a) || !conv_desc(env, a[0], &d)) return NULL;
  CHECK_RC(tjh_conv2d_forward(&d, CF32(a[1]), CF32(a[2]), CF32(a[3]), F32(a[4])));
  return undef(env);
}
/* conv2dForwardAct(desc, x, w, bias, y, act) */
static napi_value js_conv_forward_act(napi_env env, napi_callback_info info) {
  napi_value a[6];
  tjh_conv2d_desc d;
  if (!get_args(env, info, 6, a) || !conv_desc(env, a[0], &d)) return NULL;
  CHECK_RC(tjh_conv2d_forward_act(&d, CF32(a[1]), CF32(a[2]), CF32(a[3]), F32(a[4]),
                                  (int)i64(env, a[5])));
  return undef(env);
}
static napi_value js_conv_backward_input(napi_env env, napi_callback_info info) {
  napi_value a[4];
  tjh_conv2d_desc d;
  if (!get_args(env, info, 4, a) || !conv_desc(env, a[0], &d)) return NULL;
  CHECK_RC(tjh_conv2d_backward_input(&d, CF32(a[1]), CF32(a[2]), F32(a[3])));
  return undef(env);
}
static napi_value js_conv_backward_weight(napi_env env, napi_callback_info info) {
  napi_value a[5];
  tjh_conv2d_desc d;
  if (!get_args(env, info, 5, a) || !conv_desc(env, a[0], &d)) return NULL;
  CHECK_RC(tjh_conv2d_backward_weight(&d, CF32(a[1]), CF32(a[2]), F32(a[3]), (int)i64(env, a[4])));
  return undef(env);
}
/* conv2dBackwardWeightBias(desc, dy, x, dw, db|null, accumulate) */
static napi_value js_conv_backward_weight_bias(napi_env env, napi_callback_info info) {
  napi_value a[6];
  tjh_conv2d_desc d;
  if (!get_args(env, info, 6, a) || !conv_desc(env, a[0], &d)) return NULL;
  CHECK_RC(tjh_conv2d_backward_weight_bias(&d, CF32(a[1]), CF32(a[2]), F32(a[3]), F32(a[4]),
                                           (int)i64(env, a[5])));
  return undef(env);
}

/* ---------------------------------------------------------------- module */

#define FN(name, fn)                                                              \
  {name, NULL, fn, NULL, NULL, NULL,                                               \
   (napi_property_attributes)(napi_writable | napi_enumerable | napi_configurable), \
   NULL}

static napi_value init_module(napi_env env, napi_value exports) {
  napi_property_descriptor desc[] = {
      FN("init", js_init), FN("deviceInfo", js_device_info), FN("malloc", js_malloc),
      FN("h2d", js_h2d), FN("d2h", js_d2h), FN("d2hAsync", js_d2h_async),
      FN("synchronize", js_sync), FN("memoryStats", js_memory_stats),
      FN("emptyCache", js_empty_cache), FN("fill", js_fill), FN("random", js_random),
      FN("copyStrided", js_copy_strided), FN("unary", js_unary),
      FN("unaryBackward", js_unary_backward), FN("binary", js_binary), FN("scalar", js_scalar),
      FN("reduce", js_reduce), FN("exprEval", js_expr_eval), FN("exprColsum", js_expr_colsum),
      FN("exprColsum2", js_expr_colsum2), FN("exprColsum3", js_expr_colsum3),
      FN("exprCompile", js_expr_compile),
      FN("graphBegin", js_graph_begin), FN("graphEnd", js_graph_end),
      FN("graphReplay", js_graph_replay), FN("graphDestroy", js_graph_destroy),
      FN("softmaxForward", js_softmax_forward),
      FN("softmaxBackward", js_softmax_backward), FN("crossEntropyForward", js_ce_forward),
      FN("crossEntropyBackward", js_ce_backward),
      FN("crossEntropyForwardGrad", js_ce_forward_grad), FN("layerNormForward", js_ln_forward),
      FN("layerNormBackward", js_ln_backward),
      FN("layerNormBackwardRes", js_ln_backward_res),
      FN("layerNormBackwardNoalloc", js_ln_backward_noalloc),
      FN("flushDeferred", js_flush_deferred), FN("embeddingForward", js_emb_forward),
      FN("embeddingBackward", js_emb_backward), FN("embeddingPosForward", js_emb_pos_forward),
      FN("embeddingPosBackward", js_emb_pos_backward), FN("gemm", js_gemm), FN("gemmAct", js_gemm_act),
      FN("gemmCe", js_gemm_ce), FN("crossEntropyRowScale", js_ce_row_scale),
      FN("sdpaForward", js_sdpa_forward), FN("sdpaBackward", js_sdpa_backward),
      FN("adamStep", js_adam_step), FN("adamStepDev", js_adam_step_dev), FN("isInitialized", js_is_initialized),
      FN("deviceCount", js_device_count), FN("free", js_free), FN("resetPeak", js_reset_peak),
      FN("d2d", js_d2d), FN("kprofEnable", js_kprof_enable), FN("kprofFilter", js_kprof_filter),
      FN("kprofReset", js_kprof_reset), FN("kprofQuery", js_kprof_query),
      FN("kprofNames", js_kprof_names), FN("timerStart", js_timer_start),
      FN("timerStop", js_timer_stop), FN("fillI32", js_fill_i32),
      FN("copyStridedI32", js_copy_strided_i32), FN("castF32I32", js_cast_f32_i32),
      FN("castI32F32", js_cast_i32_f32), FN("ternary", js_ternary),
      FN("powScalarBackward", js_pow_scalar_backward), FN("axpy", js_axpy),
      FN("maskedFill", js_masked_fill), FN("compare", js_compare), FN("argmax", js_argmax),
      FN("nllLossForward", js_nll_forward), FN("nllLossBackward", js_nll_backward),
      FN("indexSelect", js_index_select), FN("indexAdd", js_index_add), FN("gather", js_gather),
      FN("scatterAdd", js_scatter_add), FN("oneHot", js_one_hot), FN("oneHotI32", js_one_hot_i32),
      FN("nonzero", js_nonzero), FN("conv2dForward", js_conv_forward),
      FN("conv2dForwardAct", js_conv_forward_act),
      FN("conv2dBackwardInput", js_conv_backward_input),
      FN("conv2dBackwardWeight", js_conv_backward_weight),
      FN("conv2dBackwardWeightBias", js_conv_backward_weight_bias),
      FN("cast", js_cast), FN("fillU8", js_fill_u8), FN("copyStridedU8", js_copy_strided_u8),
      FN("triangle", js_triangle), FN("multinomial", js_multinomial),
      FN("timerEnd", js_timer_end), FN("timerRead", js_timer_read),
      FN("rangePush", js_range_push), FN("rangePop", js_range_pop), FN("mark", js_mark),
  };
  napi_define_properties(env, exports, sizeof(desc) / sizeof(desc[0]), desc);
  napi_value v;
  napi_create_string_utf8(env, tjh_version(), NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, exports, "version", v);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init_module)
