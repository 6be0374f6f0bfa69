/*
 * N-API addon over the C ABI of libanima.so (include/anima.h).
 *
 * The JS side (gpu.mjs / ops.mjs) keeps the op interface of the reference's app/gpu/ops.js and
 * app/gpu/device.js; this file only marshals arguments.  Device pointers cross the boundary as
 * JS Numbers (user-space virtual addresses are below 2^53), the context as an external.
 * Every negative status becomes a thrown Error carrying anima_last_error().
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/anima.h"

#define NAPI_CALL(env, call)                                    \
  do {                                                          \
    if ((call) != napi_ok) {                                    \
      napi_throw_error((env), NULL, "N-API call failed: " #call); \
      return NULL;                                              \
    }                                                           \
  } while (0)

static int g_bad_arg = 0; /* a RangeError is pending from num() */

static napi_value throw_status(napi_env env, anima_ctx* c, int rc) {
  char msg[1200];
  snprintf(msg, sizeof msg, "anima error %d: %s", rc, anima_last_error(c));
  napi_throw_error(env, NULL, msg);
  return NULL;
}

/* Runs an ABI call; a RangeError raised while converting its arguments (or earlier in the same
 * binding: descriptor fields) stops the binding before the call. */
#define CHECK_RC(env, c, expr)                   \
  do {                                           \
    if (g_bad_arg) { g_bad_arg = 0; return NULL; } \
    int rc_ = (expr);                            \
    if (bad_arg()) return NULL;                  \
    if (rc_ != ANIMA_OK) return throw_status(env, c, rc_); \
  } while (0)

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return -1;
  for (size_t i = argc; i < want; i++) napi_get_undefined(env, &argv[i]);
  return (int)argc;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 1;
  return t == napi_undefined || t == napi_null;
}

/* Numbers crossing into the C ABI: undefined / null read as 0; anything else must be a finite
 * Number (a NaN or an infinity cast to an integer type is undefined behaviour in C), otherwise a
 * RangeError is raised and 0 returned; CHECK_RC then skips the call. */
static double num(napi_env env, napi_value v) {
  double d = 0;
  if (is_nullish(env, v)) return 0;
  if (napi_get_value_double(env, v, &d) != napi_ok || !(d == d) || d > 9.3e18 || d < -9.3e18) {
    if (!g_bad_arg) napi_throw_range_error(env, NULL, "expected a finite Number argument");
    g_bad_arg = 1;
    return 0;
  }
  return d;
}

/* Pending RangeError from num(): clears the flag and reports whether the call must stop. */
static int bad_arg(void) {
  int b = g_bad_arg;
  g_bad_arg = 0;
  return b;
}

static int64_t i64(napi_env env, napi_value v) { return (int64_t)num(env, v); }
static void* ptr(napi_env env, napi_value v) { return (void*)(uintptr_t)num(env, v); }

static napi_value prop(napi_env env, napi_value obj, const char* name) {
  napi_value v;
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) {
    napi_get_undefined(env, &v);
    return v;
  }
  napi_get_named_property(env, obj, name, &v);
  return v;
}

static double pnum(napi_env env, napi_value obj, const char* name) { return num(env, prop(env, obj, name)); }
static void* pptr(napi_env env, napi_value obj, const char* name) { return ptr(env, prop(env, obj, name)); }

static anima_ctx* ctx_of(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return (anima_ctx*)p;
}

static napi_value make_num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

/* typed array -> (data, byte length) */
static int typed(napi_env env, napi_value v, void** data, size_t* bytes) {
  napi_typedarray_type type;
  size_t len, off;
  napi_value ab;
  void* d;
  if (napi_get_typedarray_info(env, v, &type, &len, &d, &ab, &off) != napi_ok) return -1;
  size_t es = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: es = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
    default: es = 1;
  }
  *data = d;
  *bytes = len * es;
  return 0;
}

/* ------------------------------------------------------------------ runtime */

/* Contexts created by init() and not yet destroyed: a growable registry, so release() and the
 * finalizers can tell whether a buffer's context still exists. */
static anima_ctx** g_ctx = NULL;
static size_t g_nctx = 0, g_capctx = 0;
static double g_finalized = 0; /* buffers reclaimed by finalizers (leak guard, for tests) */

static int ctx_live(anima_ctx* c) {
  for (size_t i = 0; i < g_nctx; i++)
    if (c && g_ctx[i] == c) return 1;
  return 0;
}

static int ctx_register(anima_ctx* c) {
  if (g_nctx == g_capctx) {
    size_t cap = g_capctx ? 2 * g_capctx : 16;
    anima_ctx** n = (anima_ctx**)realloc(g_ctx, cap * sizeof *n);
    if (!n) return -1;
    g_ctx = n;
    g_capctx = cap;
  }
  g_ctx[g_nctx++] = c;
  return 0;
}

static void ctx_unregister(anima_ctx* c) {
  for (size_t i = 0; i < g_nctx; i++)
    if (g_ctx[i] == c) {
      g_ctx[i] = g_ctx[--g_nctx];
      return;
    }
}

/* The context travels as an external without a finalizer: a context is destroyed by destroy(),
 * and one still open at exit goes with the process.  (A finalizer here would be queued by Node's
 * environment teardown and run after the N-API environment is gone.) */
static napi_value js_init(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = NULL;
  int dev = (int)num(env, argv[0]);
  CHECK_RC(env, NULL, anima_init(dev, &c));
  if (ctx_register(c)) {
    anima_destroy(c);
    napi_throw_error(env, NULL, "init: out of host memory for the context registry");
    return NULL;
  }
  napi_value ext;
  if (napi_create_external(env, c, NULL, NULL, &ext) != napi_ok) {
    ctx_unregister(c);
    anima_destroy(c);
    napi_throw_error(env, NULL, "init: napi_create_external failed");
    return NULL;
  }
  return ext;
}

static napi_value js_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  ctx_unregister(c);
  anima_destroy(c);
  return NULL;
}

static napi_value js_sync(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_sync(c));
  return NULL;
}

static napi_value js_alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  void* p = NULL;
  size_t bytes = (size_t)num(env, argv[1]);
  CHECK_RC(env, c, anima_alloc(c, bytes, &p));
  return make_num(env, (double)(uintptr_t)p);
}

static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_free(c, ptr(env, argv[1])));
  return NULL;
}

/* Device buffers owned by JS Tensors.  A handle is a plain JS object wrapping a dev_buf; the
 * wrap's finalizer returns the buffer to the pool when the Tensor is garbage-collected without
 * release() (the reference's buffers are reclaimed by WebGPU the same way,
 * app/gpu/device.js:10-24).  release() frees the buffer at once and leaves the finalizer only the
 * host record to drop.  Contexts destroyed in between are skipped (their memory is already gone).
 *
 * Every dev_buf sits on a list together with the reference its wrap returned.  At environment
 * teardown the cleanup hook below deletes those references before Node finalizes what is left:
 * a finalizer queued by the teardown itself would run after the N-API environment has been freed
 * (a crash at exit in Node 12), while a deleted reference is never finalized. */
typedef struct dev_buf {
  anima_ctx* c;
  void* p;
  int live;
  napi_ref ref;
  struct dev_buf *prev, *next;
} dev_buf;

static dev_buf* g_bufs = NULL; /* every handle not yet finalized */

static void buf_unlink(dev_buf* b) {
  if (b->prev) b->prev->next = b->next;
  else g_bufs = b->next;
  if (b->next) b->next->prev = b->prev;
  b->prev = b->next = NULL;
}

static void buf_finalize(napi_env env, void* data, void* hint) {
  (void)hint;
  dev_buf* b = (dev_buf*)data;
  if (b->live && ctx_live(b->c) && anima_free(b->c, b->p) == ANIMA_OK) g_finalized += 1;
  buf_unlink(b);
  if (b->ref) napi_delete_reference(env, b->ref);
  free(b);
}

/* Environment cleanup: runs before N-API tears its environment down (hooks run newest first and
 * this one is added after the environment exists). */
static void bufs_cleanup(void* arg) {
  napi_env env = (napi_env)arg;
  while (g_bufs) {
    dev_buf* b = g_bufs;
    buf_unlink(b);
    if (b->live && ctx_live(b->c)) anima_free(b->c, b->p);
    if (b->ref) napi_delete_reference(env, b->ref);
    free(b);
  }
}

/* allocHandle(ctx, bytes) -> handle object (the buffer's owner) */
static napi_value js_alloc_handle(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  size_t bytes = (size_t)num(env, argv[1]);
  void* p = NULL;
  CHECK_RC(env, c, anima_alloc(c, bytes, &p));
  dev_buf* b = (dev_buf*)calloc(1, sizeof *b);
  if (!b) {
    anima_free(c, p);
    napi_throw_error(env, NULL, "allocHandle: out of host memory");
    return NULL;
  }
  b->c = c;
  b->p = p;
  b->live = 1;
  napi_value obj;
  if (napi_create_object(env, &obj) != napi_ok || napi_wrap(env, obj, b, buf_finalize, NULL, &b->ref) != napi_ok) {
    anima_free(c, p);
    free(b);
    napi_throw_error(env, NULL, "allocHandle: napi_wrap failed");
    return NULL;
  }
  b->next = g_bufs;
  if (g_bufs) g_bufs->prev = b;
  g_bufs = b;
  return obj;
}

static dev_buf* buf_of(napi_env env, napi_value v) {
  void* p = NULL;
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_object) return NULL;
  if (napi_unwrap(env, v, &p) != napi_ok) return NULL;
  return (dev_buf*)p;
}

/* handleAddr(handle) -> the device address as a Number (0 once released) */
static napi_value js_handle_addr(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  dev_buf* b = buf_of(env, argv[0]);
  if (!b) {
    napi_throw_type_error(env, NULL, "handleAddr: not a buffer handle");
    return NULL;
  }
  return make_num(env, b->live ? (double)(uintptr_t)b->p : 0);
}

/* release(handle): back to the pool now (stream-ordered); a second release is a no-op */
static napi_value js_release(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  dev_buf* b = buf_of(env, argv[0]);
  if (!b) {
    napi_throw_type_error(env, NULL, "release: not a buffer handle");
    return NULL;
  }
  if (!b->live) return NULL;
  b->live = 0;
  if (!ctx_live(b->c)) return NULL;
  CHECK_RC(env, b->c, anima_free(b->c, b->p));
  return NULL;
}

static napi_value js_finalized(napi_env env, napi_callback_info info) {
  (void)info;
  return make_num(env, g_finalized);
}

/* anima_mark / anima_wait_mark: tickets travel as JS numbers (exact below 2^53) */
static napi_value js_mark(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  uint64_t t = 0;
  CHECK_RC(env, c, anima_mark(c, &t));
  return make_num(env, (double)t);
}

static napi_value js_wait_mark(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_wait_mark(c, (uint64_t)i64(env, argv[1])));
  return NULL;
}

static napi_value js_trim(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_pool_trim(c));
  return NULL;
}

/* setW4Path(ctx, path): ANIMA_W4_GRID_SCRATCH (0) or ANIMA_W4_IN_GEMM (1), anima_set_w4_path */
static napi_value js_set_w4_path(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  int32_t path = 0;
  NAPI_CALL(env, napi_get_value_int32(env, argv[1], &path));
  CHECK_RC(env, c, anima_set_w4_path(c, path));
  return NULL;
}

/* deviceLimits(ctx) -> the adapter limits in WebGPU's names (app/gpu/device.js:63-88) */
static napi_value js_device_limits(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  anima_limits L;
  CHECK_RC(env, c, anima_device_limits(c, &L));
  napi_value o, s;
  NAPI_CALL(env, napi_create_object(env, &o));
  napi_set_named_property(env, o, "maxBufferSize", make_num(env, (double)L.max_buffer_size));
  napi_set_named_property(env, o, "maxStorageBufferBindingSize", make_num(env, (double)L.max_binding_size));
  napi_set_named_property(env, o, "maxComputeWorkgroupStorageSize", make_num(env, (double)L.workgroup_storage_size));
  napi_set_named_property(env, o, "maxComputeInvocationsPerWorkgroup", make_num(env, (double)L.max_workgroup_size));
  napi_set_named_property(env, o, "maxComputeWorkgroupsPerDimension", make_num(env, (double)L.max_workgroups_per_dimension));
  napi_set_named_property(env, o, "totalMemory", make_num(env, (double)L.total_memory));
  napi_set_named_property(env, o, "freeMemory", make_num(env, (double)L.free_memory));
  napi_set_named_property(env, o, "computeUnits", make_num(env, (double)L.compute_units));
  napi_set_named_property(env, o, "subgroupSize", make_num(env, (double)L.wavefront_size));
  napi_set_named_property(env, o, "clockKHz", make_num(env, (double)L.clock_khz));
  NAPI_CALL(env, napi_create_string_utf8(env, L.arch, NAPI_AUTO_LENGTH, &s));
  napi_set_named_property(env, o, "architecture", s);
  return o;
}

static napi_value js_mem_stats(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  uint64_t a = 0, p = 0, q = 0;
  CHECK_RC(env, c, anima_mem_stats(c, &a, &p, &q));
  napi_value o;
  NAPI_CALL(env, napi_create_object(env, &o));
  napi_set_named_property(env, o, "allocated", make_num(env, (double)a));
  napi_set_named_property(env, o, "peak", make_num(env, (double)p));
  napi_set_named_property(env, o, "pooled", make_num(env, (double)q));
  return o;
}

/* h2d(ctx, dst, typedArray) */
static napi_value js_h2d(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  get_args(env, info, 3, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  void* data;
  size_t bytes;
  if (typed(env, argv[2], &data, &bytes)) {
    napi_throw_type_error(env, NULL, "h2d: expected a typed array");
    return NULL;
  }
  CHECK_RC(env, c, anima_h2d(c, ptr(env, argv[1]), data, bytes));
  return NULL;
}

/* d2h(ctx, src, typedArray) fills the typed array */
static napi_value js_d2h(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  get_args(env, info, 3, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  void* data;
  size_t bytes;
  if (typed(env, argv[2], &data, &bytes)) {
    napi_throw_type_error(env, NULL, "d2h: expected a typed array");
    return NULL;
  }
  CHECK_RC(env, c, anima_d2h(c, data, ptr(env, argv[1]), bytes));
  return NULL;
}

static napi_value js_d2d(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  get_args(env, info, 4, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_d2d(c, ptr(env, argv[1]), ptr(env, argv[2]), (size_t)num(env, argv[3])));
  return NULL;
}

static napi_value js_profile_enable(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  bool on = false;
  napi_get_value_bool(env, argv[1], &on);
  CHECK_RC(env, c, anima_profile_enable(c, on ? 1 : 0));
  return NULL;
}

static napi_value js_profile_reset(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_profile_reset(c));
  return NULL;
}

static napi_value js_profile_report(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  static char buf[1 << 17];
  CHECK_RC(env, c, anima_profile_report(c, buf, sizeof buf));
  napi_value s;
  NAPI_CALL(env, napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &s));
  return s;
}

static napi_value js_timer_start(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_timer_start(c));
  return NULL;
}

static napi_value js_timer_stop(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  float ms = 0;
  CHECK_RC(env, c, anima_timer_stop(c, &ms));
  return make_num(env, ms);
}

/* ------------------------------------------------------------------ ops */

/* attention(ctx, desc) -- desc mirrors anima_attn_desc (pointers as Numbers, kvLen array) */
static napi_value js_attention(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  napi_value o = argv[1];
  anima_attn_desc d;
  memset(&d, 0, sizeof d);
  d.B = (int)pnum(env, o, "B");
  d.Lq = (int)pnum(env, o, "Lq");
  d.Lk = (int)pnum(env, o, "Lk");
  d.H = (int)pnum(env, o, "H");
  d.D = (int)pnum(env, o, "D");
  d.group = (int)pnum(env, o, "group");
  d.q = (const float*)pptr(env, o, "q");
  d.k = (const float*)pptr(env, o, "k");
  d.v = (const float*)pptr(env, o, "v");
  d.o = (float*)pptr(env, o, "o");
  d.ldq = (int64_t)pnum(env, o, "ldq");
  d.ldk = (int64_t)pnum(env, o, "ldk");
  d.ldv = (int64_t)pnum(env, o, "ldv");
  d.ldo = (int64_t)pnum(env, o, "ldo");
  d.q_off = (int64_t)pnum(env, o, "qOff");
  d.k_off = (int64_t)pnum(env, o, "kOff");
  d.v_off = (int64_t)pnum(env, o, "vOff");
  d.o_off = (int64_t)pnum(env, o, "oOff");
  d.q_bstride = (int64_t)pnum(env, o, "qBatch");
  d.k_bstride = (int64_t)pnum(env, o, "kBatch");
  d.v_bstride = (int64_t)pnum(env, o, "vBatch");
  d.o_bstride = (int64_t)pnum(env, o, "oBatch");
  d.scale = (float)pnum(env, o, "scale");
  d.precision = (int)pnum(env, o, "precision");
  d.q_norm = (const float*)pptr(env, o, "qNorm");
  d.k_norm = (const float*)pptr(env, o, "kNorm");
  d.rope_cs = (const float*)pptr(env, o, "cs");
  d.rope_sin_off = (int64_t)pnum(env, o, "sinOff");
  d.eps = (float)pnum(env, o, "eps");
  d.causal = (int)pnum(env, o, "causal");
  d.kv_prep = pptr(env, o, "kvPrep");
  d.kv_prep_bytes = (int64_t)pnum(env, o, "kvPrepBytes");
  d.q_prep = pptr(env, o, "qPrep");
  d.o_bf16 = (int)pnum(env, o, "oBf16");
  void* prepare_into = pptr(env, o, "prepareInto"); /* run anima_attention_prepare_kv into it */
  int kv[64];
  napi_value kvl = prop(env, o, "kvLen");
  if (!is_nullish(env, kvl)) {
    uint32_t n = 0;
    napi_get_array_length(env, kvl, &n);
    if (n > 64 || (int)n < d.B) {
      if (!bad_arg()) napi_throw_range_error(env, NULL, "attention: kvLen must hold B (<= 64) entries");
      return NULL;
    }
    for (uint32_t i = 0; i < n; i++) {
      napi_value e;
      napi_get_element(env, kvl, i, &e);
      kv[i] = (int)num(env, e);
    }
    d.kv_len = kv;
  }
  if (prepare_into) CHECK_RC(env, c, anima_attention_prepare_kv(c, &d, prepare_into));
  else CHECK_RC(env, c, anima_attention(c, &d));
  return NULL;
}

/* attentionKvBytes(B, Hkv, Lk, precision) */
static napi_value js_attention_kv_bytes(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  int B = (int)num(env, a[0]), Hkv = (int)num(env, a[1]), Lk = (int)num(env, a[2]), prec = (int)num(env, a[3]);
  if (bad_arg()) return NULL;
  return make_num(env, (double)anima_attention_kv_bytes(B, Hkv, Lk, prec));
}

/* qkNormRope(ctx, qkv, L, H, D, ld, qn, kn, cs, sinOff, eps) */
static napi_value js_qk_norm_rope(napi_env env, napi_callback_info info) {
  napi_value a[11];
  get_args(env, info, 11, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_qk_norm_rope(c, (float*)ptr(env, a[1]), i64(env, a[2]), (int)num(env, a[3]), (int)num(env, a[4]),
                                      i64(env, a[5]), (const float*)ptr(env, a[6]), (const float*)ptr(env, a[7]),
                                      (const float*)ptr(env, a[8]), i64(env, a[9]), (float)num(env, a[10])));
  return NULL;
}

/* rmsnorm(ctx, x, w, y, rows, cols, eps) */
static napi_value js_rmsnorm(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_rmsnorm(c, (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]), (float*)ptr(env, a[3]),
                                 i64(env, a[4]), (int)num(env, a[5]), (float)num(env, a[6])));
  return NULL;
}

/* rope(ctx, x, cs, L, H, D, sinOff, rowStride, colOff) */
static napi_value js_rope(napi_env env, napi_callback_info info) {
  napi_value a[9];
  get_args(env, info, 9, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_rope(c, (float*)ptr(env, a[1]), (const float*)ptr(env, a[2]), i64(env, a[3]), (int)num(env, a[4]),
                              (int)num(env, a[5]), i64(env, a[6]), i64(env, a[7]), i64(env, a[8])));
  return NULL;
}

/* hadamard(ctx, x, y, n) */
static napi_value js_hadamard(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_hadamard(c, (const float*)ptr(env, a[1]), (float*)ptr(env, a[2]), i64(env, a[3])));
  return NULL;
}

/* quantRows(ctx, x, M, K, rotate, q, s[, act]) */
static napi_value js_quant_rows(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  anima_ctx* c = ctx_of(env, a[0]);
  const int act = (int)num(env, a[7]); /* optional: the activation applied first (anima_quant_rows_act) */
  if (act)
    CHECK_RC(env, c, anima_quant_rows_act(c, (const float*)ptr(env, a[1]), i64(env, a[2]), (int)num(env, a[3]), act,
                                          (int)num(env, a[4]), (int8_t*)ptr(env, a[5]), (float*)ptr(env, a[6])));
  else
    CHECK_RC(env, c, anima_quant_rows(c, (const float*)ptr(env, a[1]), i64(env, a[2]), (int)num(env, a[3]),
                                      (int)num(env, a[4]), (int8_t*)ptr(env, a[5]), (float*)ptr(env, a[6])));
  return NULL;
}

/* quantRowsBf16(ctx, x, M, K, rotate, q, s): anima_quant_rows_bf16 */
static napi_value js_quant_rows_bf16(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_quant_rows_bf16(c, (const uint16_t*)ptr(env, a[1]), i64(env, a[2]), (int)num(env, a[3]),
                                         (int)num(env, a[4]), (int8_t*)ptr(env, a[5]), (float*)ptr(env, a[6])));
  return NULL;
}

/* layernormMod(ctx, x, mod, shiftOff, scaleOff, rows, cols, eps, rotate, y, q, s) */
static napi_value js_layernorm_mod(napi_env env, napi_callback_info info) {
  napi_value a[12];
  get_args(env, info, 12, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_layernorm_mod(c, (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]), i64(env, a[3]),
                                       i64(env, a[4]), i64(env, a[5]), (int)num(env, a[6]), (float)num(env, a[7]),
                                       (int)num(env, a[8]), (float*)ptr(env, a[9]), (int8_t*)ptr(env, a[10]),
                                       (float*)ptr(env, a[11])));
  return NULL;
}

/* elementwise(ctx, op, a, b, y, n) */
static napi_value js_elementwise(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_elementwise(c, (int)num(env, a[1]), (const float*)ptr(env, a[2]), (const float*)ptr(env, a[3]),
                                     (float*)ptr(env, a[4]), i64(env, a[5])));
  return NULL;
}

/* gemvGroupedF32(ctx, G, N, K, x, xStride, w, wStride, y, yStride, alpha, accumulate) */
static napi_value js_gemv_grouped_f32(napi_env env, napi_callback_info info) {
  napi_value a[12];
  get_args(env, info, 12, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_gemv_grouped_f32(c, (int)num(env, a[1]), (int)num(env, a[2]), (int)num(env, a[3]),
                                          (const float*)ptr(env, a[4]), i64(env, a[5]), (const float*)ptr(env, a[6]),
                                          i64(env, a[7]), (float*)ptr(env, a[8]), i64(env, a[9]), (float)num(env, a[10]),
                                          (int)num(env, a[11])));
  return NULL;
}

/* linearGroupedBf16(ctx, G, M, N, K, x, ldx, xStride, w, wStride, bias, biasStride, out, ldc, outStride) */
static napi_value js_linear_grouped_bf16(napi_env env, napi_callback_info info) {
  napi_value a[15];
  get_args(env, info, 15, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_linear_grouped_bf16(c, (int)num(env, a[1]), i64(env, a[2]), (int)num(env, a[3]),
                                             (int)num(env, a[4]), (const float*)ptr(env, a[5]), i64(env, a[6]),
                                             i64(env, a[7]), (const uint16_t*)ptr(env, a[8]), i64(env, a[9]),
                                             (const float*)ptr(env, a[10]), i64(env, a[11]), (float*)ptr(env, a[12]),
                                             i64(env, a[13]), i64(env, a[14])));
  return NULL;
}

/* patchify(ctx, latents, B, h, w, patches) */
static napi_value js_patchify(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_patchify(c, (const float*)ptr(env, a[1]), (int)num(env, a[2]), (int)num(env, a[3]),
                                  (int)num(env, a[4]), (float*)ptr(env, a[5])));
  return NULL;
}

/* unpatchify(ctx, o, B, h, w, latents) */
static napi_value js_unpatchify(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_unpatchify(c, (const float*)ptr(env, a[1]), (int)num(env, a[2]), (int)num(env, a[3]),
                                    (int)num(env, a[4]), (float*)ptr(env, a[5])));
  return NULL;
}

/* zero(ctx, y, n) */
static napi_value js_zero(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_zero(c, (float*)ptr(env, a[1]), i64(env, a[2])));
  return NULL;
}

/* fillRandom(ctx, dst, n, kind, seed, lo, hi) -- seed < 2^53 */
static napi_value js_fill_random(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_fill_random(c, ptr(env, a[1]), i64(env, a[2]), (int)num(env, a[3]), (uint64_t)num(env, a[4]),
                                     (float)num(env, a[5]), (float)num(env, a[6])));
  return NULL;
}

/* linear(ctx, W, desc): W = {kind, N, K, w, scale, srel, codebook, bias}, desc mirrors
 * anima_linear_desc (x, ldx, xRotated, xq, xs, out, ldc, alpha, act, epilogue, gate, gOff, accOut) */
/* the weight object {kindId, N, K, buf, scale, srel, codebook, bias} of ops.mjs weightArg */
static void read_weight(napi_env env, napi_value wo, anima_weight* w) {
  memset(w, 0, sizeof *w);
  w->kind = (int)pnum(env, wo, "kindId");
  w->N = (int)pnum(env, wo, "N");
  w->K = (int)pnum(env, wo, "K");
  w->w = pptr(env, wo, "buf");
  w->scale = (const float*)pptr(env, wo, "scale");
  w->srel = (const uint8_t*)pptr(env, wo, "srel");
  w->codebook = (const float*)pptr(env, wo, "codebook");
  w->bias = (const float*)pptr(env, wo, "bias");
}

/* weightUnpackW4(ctx, weight, grid) */
static napi_value js_weight_unpack_w4(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  anima_ctx* c = ctx_of(env, a[0]);
  anima_weight w;
  read_weight(env, a[1], &w);
  CHECK_RC(env, c, anima_weight_unpack_w4(c, &w, (int8_t*)ptr(env, a[2])));
  return NULL;
}

static napi_value js_linear(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  anima_ctx* c = ctx_of(env, a[0]);
  napi_value wo = a[1], o = a[2];
  anima_weight w;
  read_weight(env, wo, &w);
  anima_linear_desc d;
  memset(&d, 0, sizeof d);
  d.M = (int64_t)pnum(env, o, "M");
  d.W = &w;
  d.x = (const float*)pptr(env, o, "x");
  d.ldx = (int64_t)pnum(env, o, "ldx");
  d.x_rotated = (int)pnum(env, o, "xRotated");
  d.xq = (const int8_t*)pptr(env, o, "xq");
  d.xs = (const float*)pptr(env, o, "xs");
  d.out = (float*)pptr(env, o, "out");
  d.ldc = (int64_t)pnum(env, o, "ldc");
  d.alpha = (float)pnum(env, o, "alpha");
  d.act = (int)pnum(env, o, "act");
  d.epilogue = (int)pnum(env, o, "epilogue");
  d.gate = (const float*)pptr(env, o, "gate");
  d.gate_off = (int64_t)pnum(env, o, "gOff");
  d.acc_out = (int32_t*)pptr(env, o, "accOut");
  d.add = (const float*)pptr(env, o, "add");
  d.ld_add = (int64_t)pnum(env, o, "ldAdd");
  d.lora_xa = (const float*)pptr(env, o, "loraXa");
  d.ld_lora_xa = (int64_t)pnum(env, o, "ldLoraXa");
  d.lora_b = (const uint16_t*)pptr(env, o, "loraB");
  d.lora_r = (int)pnum(env, o, "loraR");
  d.lora_cols = (int)pnum(env, o, "loraCols");
  CHECK_RC(env, c, anima_linear(c, &d));
  return NULL;
}

/* linearQkv(ctx, weight, desc, qkv) -- desc as for linear(); qkv mirrors anima_qkv_desc */
static napi_value js_linear_qkv(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  anima_ctx* c = ctx_of(env, a[0]);
  napi_value wo = a[1], o = a[2], k = a[3];
  anima_weight w;
  read_weight(env, wo, &w);
  anima_linear_desc d;
  memset(&d, 0, sizeof d);
  d.M = (int64_t)pnum(env, o, "M");
  d.W = &w;
  d.x = (const float*)pptr(env, o, "x");
  d.x_rotated = (int)pnum(env, o, "xRotated");
  d.xq = (const int8_t*)pptr(env, o, "xq");
  d.xs = (const float*)pptr(env, o, "xs");
  d.out = (float*)pptr(env, o, "out");
  d.ldc = (int64_t)pnum(env, o, "ldc");
  d.alpha = (float)pnum(env, o, "alpha");
  d.lora_xa = (const float*)pptr(env, o, "loraXa");
  d.ld_lora_xa = (int64_t)pnum(env, o, "ldLoraXa");
  d.lora_b = (const uint16_t*)pptr(env, o, "loraB");
  d.lora_r = (int)pnum(env, o, "loraR");
  d.lora_cols = (int)pnum(env, o, "loraCols");
  anima_qkv_desc q;
  memset(&q, 0, sizeof q);
  q.B = (int)pnum(env, k, "B");
  q.L = (int)pnum(env, k, "L");
  q.H = (int)pnum(env, k, "H");
  q.k_norm = (const float*)pptr(env, k, "kNorm");
  q.rope_cs = (const float*)pptr(env, k, "cs");
  q.rope_sin_off = (int64_t)pnum(env, k, "sinOff");
  q.eps = (float)pnum(env, k, "eps");
  q.kv_prep = pptr(env, k, "kvPrep");
  q.kv_prep_bytes = (int64_t)pnum(env, k, "kvPrepBytes");
  q.q_norm = (const float*)pptr(env, k, "qNorm");
  q.q_prep = pptr(env, k, "qPrep");
  q.q_scale = (float)pnum(env, k, "qScale");
  CHECK_RC(env, c, anima_linear_qkv(c, &d, &q));
  return NULL;
}

/* split3(ctx, src, dst, n) */
static napi_value js_split3(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_split3_bf16(c, (const float*)ptr(env, a[1]), (uint16_t*)ptr(env, a[2]), i64(env, a[3])));
  return NULL;
}

/* samplerStep(ctx, {kind, n, x, v, vUncond, cfg, sigma, final, stage, den, old, oldD, eps, c: [10]}) */
static napi_value js_sampler_step(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  anima_ctx* c = ctx_of(env, a[0]);
  napi_value o = a[1];
  anima_sampler_desc d;
  memset(&d, 0, sizeof d);
  d.kind = (int)pnum(env, o, "kind");
  d.n = (int64_t)pnum(env, o, "n");
  d.x = (float*)pptr(env, o, "x");
  d.v = (const float*)pptr(env, o, "v");
  d.v_uncond = (const float*)pptr(env, o, "vUncond");
  d.cfg = pnum(env, o, "cfg");
  d.sigma = pnum(env, o, "sigma");
  bool fin = false;
  napi_value fv = prop(env, o, "final");
  if (!is_nullish(env, fv)) napi_get_value_bool(env, fv, &fin);
  d.final_step = fin ? 1 : 0;
  d.stage = (int)pnum(env, o, "stage");
  d.den_out = (float*)pptr(env, o, "den");
  d.old = (float*)pptr(env, o, "old");
  d.old_d = (float*)pptr(env, o, "oldD");
  d.eps = (const float*)pptr(env, o, "eps");
  napi_value cv = prop(env, o, "c");
  if (!is_nullish(env, cv)) {
    uint32_t len = 0;
    napi_get_array_length(env, cv, &len);
    for (uint32_t i = 0; i < len && i < 10; i++) {
      napi_value e;
      napi_get_element(env, cv, i, &e);
      d.c[i] = num(env, e);
    }
  }
  CHECK_RC(env, c, anima_sampler_step(c, &d));
  return NULL;
}

/* conv3x3(ctx, desc) -- desc mirrors anima_conv_desc */
static napi_value js_conv3x3(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  napi_value o = argv[1];
  anima_conv_desc d;
  memset(&d, 0, sizeof d);
  d.B = (int)pnum(env, o, "B");
  d.H = (int)pnum(env, o, "H");
  d.W = (int)pnum(env, o, "W");
  d.cin = (int)pnum(env, o, "cin");
  d.cout = (int)pnum(env, o, "cout");
  d.up = (int)pnum(env, o, "up");
  d.x = (const float*)pptr(env, o, "x");
  d.w = (const uint16_t*)pptr(env, o, "w");
  d.bias = (const float*)pptr(env, o, "bias");
  d.out = (float*)pptr(env, o, "out");
  d.resid = (int)pnum(env, o, "resid");
  d.precision = (int)pnum(env, o, "precision");
  CHECK_RC(env, c, anima_conv3x3(c, &d));
  return NULL;
}

/* channelNorm(ctx, x, gamma, y, rows, cols, silu) */
static napi_value js_channel_norm(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_channel_norm(c, (const float*)ptr(env, a[1]), (const float*)ptr(env, a[2]), (float*)ptr(env, a[3]),
                                      i64(env, a[4]), (int)num(env, a[5]), (int)num(env, a[6])));
  return NULL;
}

/* toRgba(ctx, x, n, out) */
static napi_value js_to_rgba(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  anima_ctx* c = ctx_of(env, a[0]);
  CHECK_RC(env, c, anima_to_rgba(c, (const float*)ptr(env, a[1]), i64(env, a[2]), (uint8_t*)ptr(env, a[3])));
  return NULL;
}

/* lastError(ctx | null) */
static napi_value js_last_error(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  anima_ctx* c = is_nullish(env, a[0]) ? NULL : ctx_of(env, a[0]);
  napi_value s;
  NAPI_CALL(env, napi_create_string_utf8(env, anima_last_error(c), NAPI_AUTO_LENGTH, &s));
  return s;
}

/* recorded submission: graph handles are host addresses passed as Numbers (< 2^53) */
static napi_value js_graph_begin(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_graph_begin(c));
  return NULL;
}

static napi_value js_graph_end(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  anima_graph* g = NULL;
  CHECK_RC(env, c, anima_graph_end(c, &g));
  return make_num(env, (double)(uintptr_t)g);
}

static napi_value js_graph_launch(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_graph_launch(c, (anima_graph*)ptr(env, argv[1])));
  return NULL;
}

static napi_value js_graph_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  anima_ctx* c = ctx_of(env, argv[0]);
  CHECK_RC(env, c, anima_graph_destroy(c, (anima_graph*)ptr(env, argv[1])));
  return NULL;
}

static napi_value Init(napi_env env, napi_value exports) {
#define FN(name, f) {name, NULL, f, NULL, NULL, NULL, napi_enumerable, NULL}
  napi_property_descriptor desc[] = {
      FN("init", js_init), FN("destroy", js_destroy), FN("sync", js_sync), FN("mark", js_mark), FN("waitMark", js_wait_mark), FN("alloc", js_alloc),
      FN("free", js_free), FN("allocHandle", js_alloc_handle), FN("handleAddr", js_handle_addr),
      FN("release", js_release), FN("finalized", js_finalized), FN("trim", js_trim), FN("memStats", js_mem_stats), FN("deviceLimits", js_device_limits), FN("setW4Path", js_set_w4_path), FN("h2d", js_h2d),
      FN("d2h", js_d2h), FN("d2d", js_d2d), FN("profileEnable", js_profile_enable),
      FN("profileReset", js_profile_reset), FN("profileReport", js_profile_report),
      FN("timerStart", js_timer_start), FN("timerStop", js_timer_stop), FN("attention", js_attention),
      FN("qkNormRope", js_qk_norm_rope), FN("rmsnorm", js_rmsnorm), FN("rope", js_rope),
      FN("hadamard", js_hadamard), FN("quantRows", js_quant_rows), FN("quantRowsBf16", js_quant_rows_bf16), FN("layernormMod", js_layernorm_mod),
      FN("elementwise", js_elementwise), FN("zero", js_zero), FN("patchify", js_patchify), FN("linearGroupedBf16", js_linear_grouped_bf16), FN("gemvGroupedF32", js_gemv_grouped_f32), FN("unpatchify", js_unpatchify), FN("fillRandom", js_fill_random),
      FN("linear", js_linear), FN("linearQkv", js_linear_qkv), FN("samplerStep", js_sampler_step), FN("attentionKvBytes", js_attention_kv_bytes), FN("split3", js_split3), FN("lastError", js_last_error),
      FN("graphBegin", js_graph_begin), FN("graphEnd", js_graph_end), FN("graphLaunch", js_graph_launch),
      FN("graphDestroy", js_graph_destroy), FN("conv3x3", js_conv3x3), FN("channelNorm", js_channel_norm), FN("toRgba", js_to_rgba),
      FN("weightUnpackW4", js_weight_unpack_w4),
  };
#undef FN
  if (napi_define_properties(env, exports, sizeof desc / sizeof desc[0], desc) != napi_ok) return NULL;
  if (napi_add_env_cleanup_hook(env, bufs_cleanup, env) != napi_ok) return NULL;
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
